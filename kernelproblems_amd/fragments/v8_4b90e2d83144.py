"""RMSNorm forward, y returned as three [8192, 4096] views:
v8/4b90e2d83144/problem.py:10-29 (inputs :32-35).  rstd is not an output,
so the kernel does not write it."""
from .. import fused as F
from ._common import EPS, randn, rows2d


def get_inputs(device="cuda", generator=None):
    return [randn([1, 8192, 4096], device=device, generator=generator),
            randn([4096], device=device, generator=generator)]


def kernel_function(embedding, _unsafe_view_432):
    _, y, _ = F.rms_norm([embedding], _unsafe_view_432, EPS, embedding.shape[-1], return_rstd=False)
    v = rows2d(y)
    return v, v.view(v.shape), v.view(v.shape)
