"""Embedding forward from an FSDP flat buffer: v7/1e49beb8a123/problem.py:10-24
(inputs :27-30).  A single split covering each whole shard row makes the
[128256, 4096] table a plain view of the flat buffer (:16-20); the gather is
a bit copy.  The single output is returned bare."""
from .. import fused as F
from ._common import randint, randn


def get_inputs(device="cuda", generator=None):
    return [randn([525336576], device=device, generator=generator),
            randint(100, [1, 8192], device=device, generator=generator)]


def kernel_function(wait_tensor_871, arg583_1):
    table = wait_tensor_871.view(128256, 4096)
    return F.embedding(table, arg583_1)
