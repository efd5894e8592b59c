"""RMSNorm forward with the weight taken from an FSDP flat buffer:
v7/215dd2e6a519/problem.py:10-38 (inputs :41-44).  The [8, 512] view with
row stride 27264000 is read in place by the kernel (the reference clones it
to a contiguous [4096] first, :16-18)."""
from .. import fused as F
from ._common import EPS, randn, rows2d, strided_randn


def get_inputs(device="cuda", generator=None):
    return [strided_randn(190848512, [8, 512], [27264000, 1], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator)]


def kernel_function(getitem_1614, add_61):
    _, y, _ = F.rms_norm([add_61], getitem_1614, EPS, add_61.shape[-1], return_rstd=False)
    v = rows2d(y)
    return v, v.view(v.shape), v.view(v.shape)
