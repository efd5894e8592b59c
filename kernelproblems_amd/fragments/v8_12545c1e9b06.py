"""Token embedding, first-layer attention RMSNorm and that layer's FSDP
parameter unshard: v8/12545c1e9b06/problem.py:10-102 (inputs :105-109).

The embedding rows are not an output of the fragment: the gather is fused
into the norm kernel, so they go from the table straight into registers.
The norm weight is read in place from segment 0 of the layer buffer, and
segments 1-6 are copied out in one launch."""
from .. import fused as F
from ._common import EPS, LAYER_SHAPES, LAYER_SPLITS, SHARDS, layer_norm_weight, randint, randn, rows2d

_KEEP = (1, 2, 3, 4, 5, 6)


def get_inputs(device="cuda", generator=None):
    return [randn([525336576], device=device, generator=generator),
            randint(100, [1, 8192], device=device, generator=generator),
            randn([218112000], device=device, generator=generator)]


def kernel_function(wait_tensor_871, arg583_1, wait_tensor_873):
    table = wait_tensor_871.view(128256, 4096)
    w = layer_norm_weight(wait_tensor_873, 0)
    _, y, _ = F.embedding_rms_norm(table, arg583_1, w, EPS, return_rstd=False)
    params = F.unshard(wait_tensor_873, SHARDS, LAYER_SPLITS, _KEEP)
    v = rows2d(y)
    return (v, v.view(v.shape), v.view(v.shape), *(p.view(LAYER_SHAPES[i]) for p, i in zip(params, _KEEP)))
