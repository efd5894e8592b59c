"""SwiGLU gate forward, silu -> mul, with the operands named mm_221 / mm_222:
v5/c68dae22972b/problem.py:10-29 (inputs :32-35).  The ops of
v4/65b4b565ed67 with _unsafe_view in place of reshape; the same drop-in."""
from .v4_65b4b565ed67 import get_inputs, kernel_function  # noqa: F401
