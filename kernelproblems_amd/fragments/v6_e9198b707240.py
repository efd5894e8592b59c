"""FFN-norm forward (y as 2 views) and its backward with a 2-term gradient
and residual epilogue: v6/e9198b707240/problem.py:10-56 (inputs :60-64)."""
from ._common import randn, strided_randn  # noqa: F401
from ._norm_chain import norm_fwd_bwd

_X = [1, 8192, 4096]
_MM = [8192, 4096]


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randn(_X, **kw), randn([4096], **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_X, **kw)]


def kernel_function(add_62_recomputed, _unsafe_view_986, mm_230, mm_232, getitem_420):
    return norm_fwd_bwd([add_62_recomputed], _unsafe_view_986, [mm_230, mm_232], getitem_420, n_views=2)
