"""Token cross-entropy forward with the targets second and already flat:
v7/e59c6b1b5156/problem.py:10-36 (inputs :39-42).  As v8/71f1d2c9f38b:
returns (loss / 8192, total_weight), one pass over the bf16 logits."""
from .. import fused as F
from ._common import randint, randn

M, V = 8192, 128256


def get_inputs(device="cuda", generator=None):
    return [randn([M, V], device=device, generator=generator),
            randint(100, [M], device=device, generator=generator)]


def kernel_function(mm_224, view_805):
    return F.cross_entropy_loss(mm_224, view_805, ignore_index=-100, scale=1.0 / 8192.0)
