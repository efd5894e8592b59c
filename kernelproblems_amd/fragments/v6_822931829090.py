"""Attention-norm forward (y as 3 views) and its backward with a 3-term
gradient and residual epilogue: v6/822931829090/problem.py:10-66 (inputs :70-75)."""
from ._common import randn, strided_randn  # noqa: F401
from ._norm_chain import norm_fwd_bwd

_X = [1, 8192, 4096]
_MM = [8192, 4096]


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randn(_X, **kw), randn([4096], **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_X, **kw)]


def kernel_function(add_1, _unsafe_view_450, mm_656, mm_658, mm_660, add_215):
    return norm_fwd_bwd([add_1], _unsafe_view_450, [mm_656, mm_658, mm_660], add_215, n_views=3)
