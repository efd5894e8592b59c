"""v2/d7efc428b2f5/problem.py:10-509 (inputs :512-581) is the op sequence of
v1/d7efc428b2f5 (same signature, outputs and input shapes); its drop-in serves both."""
from .v1_d7efc428b2f5 import get_inputs, kernel_function  # noqa: F401
