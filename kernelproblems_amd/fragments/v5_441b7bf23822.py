"""As v6/182d2dcd0652, with the two gradients returned as the transposed
[14336, 8192] views the weight-gradient matmuls read:
v5/441b7bf23822/problem.py:10-48 (inputs :51-55)."""
from .. import fused as F
from ._common import randn

M, N = 8192, 14336


def get_inputs(device="cuda", generator=None):
    return [randn([M, N], device=device, generator=generator) for _ in range(3)]


def forward_backward_t(mm_4, mm_5, mm_662):
    h, db, da = F.swiglu_forward_backward(mm_4, mm_5, mm_662)
    return h, db.t(), da.t()


def kernel_function(mm_4, mm_5, mm_662):
    return forward_backward_t(mm_4, mm_5, mm_662)
