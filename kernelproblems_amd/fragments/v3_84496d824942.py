"""v3/84496d824942/problem.py:10-38 (inputs :41-44) is the op sequence of
v1/84496d824942 (same signature, outputs and input shapes); its drop-in serves both."""
from .v1_84496d824942 import get_inputs, kernel_function  # noqa: F401
