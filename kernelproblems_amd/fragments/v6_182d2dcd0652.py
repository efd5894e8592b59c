"""SwiGLU gate forward recomputed with its backward: v6/182d2dcd0652/problem.py:10-46
(inputs :49-53).  s = bf16(silu(mm_4)) stays in registers; one launch reads
mm_4, mm_5, mm_662 and writes h = s * mm_5 (the w2 input), db = mm_662 * s
(the w3 branch gradient) and da = silu_backward(mm_662 * mm_5, mm_4) (the
w1 branch gradient), each a fresh [8192, 14336] tensor."""
from .. import fused as F
from ._common import randn

M, N = 8192, 14336


def get_inputs(device="cuda", generator=None):
    return [randn([M, N], device=device, generator=generator) for _ in range(3)]


def kernel_function(mm_4, mm_5, mm_662):
    return F.swiglu_forward_backward(mm_4, mm_5, mm_662)
