"""v6/97032595d968/problem.py:10-67 (inputs :70-75) is the op sequence of
v8/97032595d968 (same signature, outputs and input shapes); its drop-in serves both."""
from .v8_97032595d968 import get_inputs, kernel_function  # noqa: F401
