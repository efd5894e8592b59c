"""v2/075cb40f3d5d/problem.py:10-29 (inputs :32-37) is the op sequence of
v1/075cb40f3d5d (same signature, outputs and input shapes); its drop-in serves both."""
from .v1_075cb40f3d5d import get_inputs, kernel_function  # noqa: F401
