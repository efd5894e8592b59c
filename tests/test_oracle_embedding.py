"""Pins the oracle's embedding forward / dense backward against torch's
library ops on the CPU (index_select, fp64 index_add_, fp64
embedding_dense_backward) and the invariants of a scatter-sum."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import bf16_round_exact, gen, randn_bf16, to_u16, zipf_ids

aten = torch.ops.aten


def test_fwd_bit_exact_vs_index_select():
    g = gen(1)
    V, D, T = 500, 96, 700
    table = randn_bf16((V, D), g, std=0.02)
    ids = torch.cat([torch.randint(0, V, (T - 3,), generator=g), torch.tensor([0, V - 1, 0])])
    out, bad = oracle.embedding_fwd(to_u16(table), ids.numpy())
    assert bad == 0
    assert np.array_equal(out, to_u16(table.index_select(0, ids)))


def test_fwd_out_of_range_rows_are_zero():
    table = randn_bf16((10, 8), gen(2))
    out, bad = oracle.embedding_fwd(to_u16(table), np.array([3, -1, 10, 9]))
    assert bad == 2
    assert not out[1].any() and not out[2].any()
    assert np.array_equal(out[0], to_u16(table[3])) and np.array_equal(out[3], to_u16(table[9]))


@pytest.mark.parametrize("padding_idx", [-1, 0, 7])
def test_bwd_rows_match_fp64_index_add(padding_idx):
    g = gen(3)
    V, D, T = 300, 64, 2000
    grad = randn_bf16((T, D), g)
    ids = zipf_ids(T, V, 1.1, g)
    rid, rows, absrows, counts, bad = oracle.embedding_bwd_rows(to_u16(grad), ids.numpy(), V, padding_idx)
    assert bad == 0
    keep = ids != padding_idx
    exp = torch.zeros(V, D, dtype=torch.float64).index_add_(0, ids[keep], grad[keep].double())
    touched = torch.unique(ids[keep]).numpy()
    assert np.array_equal(rid, touched)
    np.testing.assert_allclose(rows, exp[touched].numpy(), rtol=1e-12, atol=1e-12)
    assert np.all(absrows >= np.abs(rows))
    np.testing.assert_array_equal(counts, torch.bincount(ids[keep], minlength=V)[touched].numpy())


def test_bwd_dense_vs_torch_embedding_dense_backward_fp64():
    g = gen(4)
    V, D, T = 257, 40, 900
    grad = randn_bf16((T, D), g)
    ids = torch.randint(0, V, (T,), generator=g)
    for scale in (False, True):
        dense = oracle.embedding_bwd_dense(to_u16(grad), ids.numpy(), V, -1, scale)
        # torch scales in the computation dtype; the oracle divides in fp32 then sums in fp64
        exp = aten.embedding_dense_backward.default(grad.double(), ids, V, -1, scale).numpy()
        np.testing.assert_allclose(dense, exp, rtol=2.0**-22, atol=1e-6)


def test_bwd_dense_invariants():
    g = gen(5)
    V, D, T, pad = 1000, 32, 3000, 2
    grad = randn_bf16((T, D), g)
    ids = zipf_ids(T, V, 1.1, g)
    dense = oracle.embedding_bwd_dense(to_u16(grad), ids.numpy(), V, pad)
    untouched = np.setdiff1d(np.arange(V), ids.numpy())
    assert not dense[untouched].any()
    assert not dense[pad].any()
    keep = (ids != pad).numpy()
    np.testing.assert_allclose(dense.astype(np.float64).sum(0), grad.double().numpy()[keep].sum(0),
                               rtol=1e-5, atol=1e-3)


def test_bwd_dense_bf16_rounding_is_single():
    """round_bf16: the fp64 row sums rounded once to bf16 (the reference's
    bf16 dense gradient widened by _to_copy)."""
    g = gen(6)
    V, D, T = 50, 16, 400
    grad = randn_bf16((T, D), g)
    ids = torch.randint(0, V, (T,), generator=g)
    dense = oracle.embedding_bwd_dense(to_u16(grad), ids.numpy(), V, -1, False, round_bf16=True)
    exact = torch.zeros(V, D, dtype=torch.float64).index_add_(0, ids, grad.double()).numpy()
    exp = bf16_round_exact(exact).reshape(V, D)
    assert np.array_equal(to_u16(torch.from_numpy(dense).bfloat16()), exp)
    assert np.array_equal(torch.from_numpy(dense).bfloat16().float().numpy(), dense)
