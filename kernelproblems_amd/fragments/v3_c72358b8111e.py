"""v3/c72358b8111e/problem.py:10-48 (inputs :51-55) is the op sequence of
v4/c72358b8111e (same signature, outputs and input shapes); its drop-in serves both."""
from .v4_c72358b8111e import get_inputs, kernel_function  # noqa: F401
