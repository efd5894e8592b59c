"""SwiGLU gate backward, mul / mul -> silu_backward:
v8/385e1beb9bb9/problem.py:10-33 (inputs :36-41).

mm_662 is the gradient of the gate product (bf16 [8192, 14336]); the
recomputed silu(w1 out), w3 output and w1 output arrive as [1, 8192, 14336].
Returns (grad of the w3 branch, grad of the w1 branch), each a fresh
[8192, 14336] tensor, from one launch (4 reads + 2 writes)."""
from .. import fused as F
from ._common import randn

M, N = 8192, 14336


def get_inputs(device="cuda", generator=None):
    return [randn([M, N], device=device, generator=generator),
            randn([1, M, N], device=device, generator=generator),
            randn([1, M, N], device=device, generator=generator),
            randn([1, M, N], device=device, generator=generator)]


def kernel_function(mm_662, silu_recomputed, _unsafe_view_5_recomputed, _unsafe_view_4_recomputed):
    db, da = F.swiglu_backward(mm_662, silu_recomputed, _unsafe_view_5_recomputed, _unsafe_view_4_recomputed)
    return db.view(mm_662.shape[0], -1), da.view(mm_662.shape[0], -1)
