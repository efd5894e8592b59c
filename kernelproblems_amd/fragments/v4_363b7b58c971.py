"""v5/92ce4a0c7b2c as traced with reshape instead of view (same outputs):
v4/363b7b58c971/problem.py:10-75 (inputs :79-84)."""
from ._common import randn, strided_randn  # noqa: F401
from ._norm_chain import norm_fwd_bwd

_X = [1, 8192, 4096]
_MM = [8192, 4096]


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [strided_randn(190848512, [8, 512], [27264000, 1], **kw), randn(_X, **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_X, **kw)]


def kernel_function(getitem_818, add_1, mm_656, mm_658, mm_660, add_215):
    return norm_fwd_bwd([add_1], getitem_818, [mm_656, mm_658, mm_660], add_215, n_views=3)
