"""RMSNorm forward returning (y, rstd): v7/59f786beb25f/problem.py:10-21
(inputs :24-27).  _fused_rms_norm(embedding, [4096], w, 1e-05)."""
from .. import fused as F
from ._common import EPS, randn, rstd_view


def get_inputs(device="cuda", generator=None):
    return [randn([1, 8192, 4096], device=device, generator=generator),
            randn([4096], device=device, generator=generator)]


def kernel_function(embedding, _unsafe_view_432):
    _, y, rstd = F.rms_norm([embedding], _unsafe_view_432, EPS, embedding.shape[-1])
    return y, rstd_view(rstd, embedding)
