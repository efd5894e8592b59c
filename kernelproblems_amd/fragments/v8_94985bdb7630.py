"""Residual add + RMSNorm forward with one layer's FSDP parameter unshard:
v8/94985bdb7630/problem.py:10-106 (inputs :109-113).

The attention-norm weight (segment 0) is read in place; segments 1-7 (wq,
wk, wv, wo, ffn_norm, w1, w2) are copied out in one launch.  Segment 8 is
not an output of this fragment."""
from .. import fused as F
from ._common import EPS, LAYER_SHAPES, LAYER_SPLITS, SHARDS, layer_norm_weight, randn, rows2d

_KEEP = (1, 2, 3, 4, 5, 6, 7)


def get_inputs(device="cuda", generator=None):
    return [randn([8192, 4096], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator),
            randn([218112000], device=device, generator=generator)]


def kernel_function(mm_216, add_60, wait_tensor_966):
    w = layer_norm_weight(wait_tensor_966, 0)
    _, y, _ = F.rms_norm([add_60, mm_216], w, EPS, add_60.shape[-1], return_rstd=False)
    params = F.unshard(wait_tensor_966, SHARDS, LAYER_SPLITS, _KEEP)
    v = rows2d(y)
    return (v, v.view(v.shape), v.view(v.shape),
            *(p.view(LAYER_SHAPES[i]) for p, i in zip(params, _KEEP)))
