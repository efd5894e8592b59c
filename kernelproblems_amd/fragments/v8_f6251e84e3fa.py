"""First-layer attention-norm backward with a three-term gradient and a
residual epilogue, then the token-embedding backward of the result, the saved
forward passed as a tuple: v8/f6251e84e3fa/problem.py:10-57.

rstd = _fused_rms_norm_recomputed[1]; dy = bf16(bf16(mm_670 + mm_672) +
mm_674); g = bf16(add_220 + dx) is made in the norm's row pass, which walks the
tokens in (id, token) order and sums each id's g rows into its table row in
registers (fp32 accumulation, one bf16 rounding as the eager bf16 table, stored
fp32), so g never reaches HBM; dw is the bf16 weight gradient widened to
fp32.  The reference's own get_inputs hands a 0-dim tensor where
the graph passes the tuple (v8/f6251e84e3fa/benchmark.json records the index
error); get_inputs here builds the tuple."""
import torch

from .. import fused as F
from ._common import EPS, norm_saved, randint, randn

NUM_WEIGHTS = 128256


def get_inputs(device="cuda", generator=None):
    mm = [randn([8192, 4096], device=device, generator=generator) for _ in range(3)]
    emb = randn([1, 8192, 4096], device=device, generator=generator)
    w = randn([4096], device=device, generator=generator)
    add_220 = randn([1, 8192, 4096], device=device, generator=generator)
    ids = randint(100, [1, 8192], device=device, generator=generator)
    return [norm_saved(emb, w), *mm, emb, w, add_220, ids]


def kernel_function(_fused_rms_norm_recomputed, mm_670, mm_672, mm_674, embedding, _unsafe_view_432, add_220,
                    arg583_1):
    n = embedding.shape[-1]
    _, dw, table = F.rms_norm_embedding_backward([mm_670, mm_672, mm_674], embedding, _fused_rms_norm_recomputed[1],
                                                 _unsafe_view_432, EPS, n, add_220, arg583_1, NUM_WEIGHTS, -1,
                                                 dw="f32_bf16", out_dtype=torch.float32, round_to_bf16=True)
    return dw, table
