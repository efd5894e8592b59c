"""The chain of v6/0b493aad68f0 with the norm weight taken from an FSDP flat
buffer: v5/118d525f44e0/problem.py:10-59 (inputs :62-70).  The [8, 512] view
(row stride 27264000) is read in place by the norm's row pass; the reference
clones it to a contiguous [4096] first (:17-19)."""
from ._common import randint, randn, strided_randn
from .v6_0b493aad68f0 import chain


def get_inputs(device="cuda", generator=None):
    return [strided_randn(190848512, [8, 512], [27264000, 1], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator),
            randn([8192, 4096], device=device, generator=generator),
            randn([8192, 4096], device=device, generator=generator),
            randn([8192, 4096], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator),
            randint(100, [1, 8192], device=device, generator=generator)]


def kernel_function(getitem_791, embedding, mm_670, mm_672, mm_674, add_220, arg583_1):
    return chain(embedding, getitem_791, [mm_670, mm_672, mm_674], add_220, arg583_1)
