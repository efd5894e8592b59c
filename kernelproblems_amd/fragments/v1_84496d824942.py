"""RMSNorm forward with the weight taken from an FSDP flat buffer, y as
three views: v1/84496d824942/problem.py:8-36 (inputs :39-42).  The ops of
v7/215dd2e6a519 with a no-op view.dtype(bf16) on the weight and reshape in
place of view; the same drop-in."""
from .v7_215dd2e6a519 import get_inputs, kernel_function  # noqa: F401
