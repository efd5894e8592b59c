"""v6/e9198b707240 with the norm weight an [8, 512] FSDP view read in place:
v5/401b52261ef5/problem.py:10-65 (inputs :69-73)."""
from ._common import randn, strided_randn  # noqa: F401
from ._norm_chain import norm_fwd_bwd

_X = [1, 8192, 4096]
_MM = [8192, 4096]


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [strided_randn(190848512, [8, 512], [27264000, 1], **kw), randn(_X, **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_X, **kw)]


def kernel_function(getitem_1624, add_62_recomputed, mm_230, mm_232, getitem_420):
    return norm_fwd_bwd([add_62_recomputed], getitem_1624, [mm_230, mm_232], getitem_420, n_views=2)
