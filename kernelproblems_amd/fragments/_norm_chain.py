"""The RMSNorm forward -> backward chain shared by the layer-boundary
fragments of the reference (e.g. v6/822931829090/problem.py,
v6/408ac0979ac5/problem.py, v6/28b45679fca1/problem.py).

h = bf16 running sum of x_terms (eager add.Tensor rounding), y = rms(h)
returned as ``n_views`` views of one [M, N] tensor; dy = bf16 running sum of
dy_terms; the backward gives out = bf16(residual + dx) (or dx) and dw widened
from its bf16 rounding to fp32.  With y wanted, the forward and the backward
are one row pass (rstd computed once, the x terms read once) plus the
weight-gradient finalize; without it (the fragments that only recompute the
norm for its backward) the backward recomputes rstd itself."""
from __future__ import annotations

from .. import fused as F
from ._common import EPS, rows2d


def norm_fwd_bwd(x_terms, w, dy_terms, residual=None, n_views=0):
    n = x_terms[0].shape[-1]
    if n_views:
        y, out, dw, _, _ = F.rms_norm_forward_backward(dy_terms, x_terms, w, EPS, n, dx_residual=residual,
                                                       dw="f32_bf16")
        v = rows2d(y)
        views = (v,) + tuple(v.view(v.shape) for _ in range(n_views - 1))
        return (*views, out, dw.view(-1))
    out, dw = F.rms_norm_backward(dy_terms, x_terms, None, w, EPS, n, dx_residual=residual, dw="f32_bf16")
    return out, dw.view(-1)
