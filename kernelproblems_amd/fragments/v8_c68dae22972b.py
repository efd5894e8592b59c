"""SwiGLU gate forward, silu -> mul: v8/c68dae22972b/problem.py:10-28
(inputs :31-34).

The w1 and w3 projection outputs mm_4, mm_5 (bf16 [8192, 14336]) give
view(mul(silu(mm_4), mm_5)) as a fresh [8192, 14336] tensor, in one
streaming launch (2 reads + 1 write)."""
from .. import fused as F
from ._common import randn

M, N = 8192, 14336


def get_inputs(device="cuda", generator=None):
    return [randn([M, N], device=device, generator=generator),
            randn([M, N], device=device, generator=generator)]


def kernel_function(mm_4, mm_5):
    return F.swiglu(mm_4, mm_5).view(mm_4.shape[0], -1)
