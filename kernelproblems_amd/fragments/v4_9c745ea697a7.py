"""v6/408ac0979ac5 with the norm weight an [8, 512] FSDP view read in place
(traced with reshape): v4/9c745ea697a7/problem.py:10-72 (inputs :76-81)."""
from ._common import randn, strided_randn  # noqa: F401
from ._norm_chain import norm_fwd_bwd

_X = [1, 8192, 4096]
_MM = [8192, 4096]


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randn(_MM, **kw), randn(_X, **kw), strided_randn(190848512, [8, 512], [27264000, 1], **kw), randn(_MM, **kw), randn(_MM, **kw), randn(_X, **kw)]


def kernel_function(mm_3, embedding, getitem_787, mm_664, mm_666, add_218):
    return norm_fwd_bwd([embedding, mm_3], getitem_787, [mm_664, mm_666], add_218, n_views=2)
