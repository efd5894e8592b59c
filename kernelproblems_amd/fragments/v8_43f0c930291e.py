"""Attention-norm backward of a middle layer with a three-term gradient and a
residual epilogue, the saved forward passed as a tuple:
v8/43f0c930291e/problem.py:10-52 (31 instances per step, v8/README.md:10).

rstd = _fused_rms_norm_2_recomputed[1] (the saved (y, rstd) tuple; only rstd
is read); dy = bf16(bf16(mm_656 + mm_658) + mm_660); out = bf16(add_215 + dx)
as an [8192, 4096] view; dw is the bf16 weight gradient widened to fp32.  One
row kernel and the weight-gradient finalize.  The reference's own get_inputs
hands a 0-dim tensor where the graph passes the tuple (its benchmark records
an index error); get_inputs here builds the tuple."""
from .. import fused as F
from ._common import EPS, norm_saved, randn, rows2d


def get_inputs(device="cuda", generator=None):
    mm = [randn([8192, 4096], device=device, generator=generator) for _ in range(3)]
    add_1 = randn([1, 8192, 4096], device=device, generator=generator)
    w = randn([4096], device=device, generator=generator)
    add_215 = randn([1, 8192, 4096], device=device, generator=generator)
    return [norm_saved(add_1, w), *mm, add_1, w, add_215]


def kernel_function(_fused_rms_norm_2_recomputed, mm_656, mm_658, mm_660, add_1, _unsafe_view_450, add_215):
    n = add_1.shape[-1]
    out, dw = F.rms_norm_backward([mm_656, mm_658, mm_660], [add_1], _fused_rms_norm_2_recomputed[1],
                                  _unsafe_view_450, EPS, n, dx_residual=add_215, dw="f32_bf16")
    return rows2d(out), dw
