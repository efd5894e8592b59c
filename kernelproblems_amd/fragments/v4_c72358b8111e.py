"""As v5/441b7bf23822 (reshape in place of view): v4/c72358b8111e/problem.py:10-48
(inputs :51-55)."""
from .v5_441b7bf23822 import forward_backward_t, get_inputs  # noqa: F401


def kernel_function(mm_4, mm_5, mm_662):
    return forward_backward_t(mm_4, mm_5, mm_662)
