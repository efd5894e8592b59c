"""RoPE backward of q (table _conj_63) and k (table _conj_62) plus the v
gradient, each returned as the transposed [H*D, S] view the wq / wk / wv
weight-gradient matmuls read: v5/a1bb72d946b0/problem.py:10-85 (inputs
:88-94).  The gradients arrive as [1, H, S, D] views with [S, H, D] memory
order; v's is only re-viewed (an alias of getitem_643, no copy).  q and k
take their own tables, so they are two launches."""
import torch

from ._common import randn, strided_randn
from ._rope import rotate, table_rows


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randn([1, 8192, 1, 64], dtype=torch.complex64, **kw),
            randn([1, 8192, 1, 64], dtype=torch.complex64, **kw),
            strided_randn(33554432, [1, 32, 8192, 128], [33554432, 128, 4096, 1], **kw),
            strided_randn(8388608, [1, 8, 8192, 128], [8388608, 128, 1024, 1], **kw),
            strided_randn(8388608, [1, 8, 8192, 128], [8388608, 128, 1024, 1], **kw)]


def qkv_backward(conj_k, conj_q, gq, gk, gv):
    q, _ = rotate(gq.transpose(1, 2), freqs=table_rows(conj_q))
    k, _ = rotate(gk.transpose(1, 2), freqs=table_rows(conj_k))
    v = gv.transpose(1, 2)
    return q.view(q.shape[1], -1).t(), k.view(k.shape[1], -1).t(), v.view(v.shape[1], -1).t()


def kernel_function(_conj_62, _conj_63, getitem_641, getitem_642, getitem_643):
    return qkv_backward(_conj_62, _conj_63, getitem_641, getitem_642, getitem_643)
