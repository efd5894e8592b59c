"""Attention-norm forward with the FSDP weight view, y as two views, plus the
unshard of the layer's three feed-forward weights (w1, w3 as [4096, 14336]
and w2 as [14336, 4096] transposed views): v1/2a844503364a/problem.py:8-72
(inputs :75-81).  Each weight shard row [8, 7340032] (row stride 27264000)
is copied to a contiguous tensor by the unshard kernel; the norm reads its
weight in place."""
from .. import fused as F
from ._common import EPS, SHARDS, randn, rows2d, strided_randn

_W = 198188032  # 7 x 27264000 + 7340032: the buffer behind each [8, 7340032] view


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [strided_randn(190848512, [8, 512], [27264000, 1], **kw), randn([1, 8192, 4096], **kw),
            strided_randn(_W, [8, 7340032], [27264000, 1], **kw),
            strided_randn(_W, [8, 7340032], [27264000, 1], **kw),
            strided_randn(_W, [8, 7340032], [27264000, 1], **kw)]


def _contiguous_shards(view):
    (c,) = F.unshard(view, SHARDS, (view.shape[1],), [0])
    return c


def kernel_function(getitem_1619, add_62, getitem_1620, getitem_1621, getitem_1622):
    _, y, _ = F.rms_norm([add_62], getitem_1619, EPS, add_62.shape[-1], return_rstd=False)
    v = rows2d(y)
    w1 = _contiguous_shards(getitem_1620).view(14336, 4096)
    w3 = _contiguous_shards(getitem_1621).view(14336, 4096)
    w2 = _contiguous_shards(getitem_1622).view(4096, 14336)
    return v, v.view(v.shape), w1.t(), w3.t(), w2.t()
