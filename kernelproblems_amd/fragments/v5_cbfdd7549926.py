"""Residual add + attention-norm forward -> backward with a 2-term gradient
and residual epilogue, FSDP weight view: v5/cbfdd7549926/problem.py:10-72
(inputs :75-82).  The ops of v4/9c745ea697a7 with view in place of reshape;
the same drop-in."""
from .v4_9c745ea697a7 import get_inputs, kernel_function  # noqa: F401
