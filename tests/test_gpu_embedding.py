"""GPU parity: embedding gather (bit-exact) and dense deterministic backward vs the C oracle."""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
import oracle
from tests._util import bf, gen, randn_bf16, to_u16, ulp_bf16, zipf_ids

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("V,D,T", [(1000, 4096, 777), (50, 64, 300), (128256, 4096, 2048), (300, 100, 129),
                                   (300, 4608, 257), (70, 8192, 65)])
@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_embedding_fwd_bit_exact(gpu, oracle_lib, V, D, T, idx_dtype):
    g = gen(V + D + T)
    table = randn_bf16((V, D), g, 0.0, 0.02)
    ids = zipf_ids(T, V, 1.1, g)
    ids[0], ids[-1] = 0, V - 1  # first and last rows
    out = kp.embedding(table.to(gpu), ids.to(idx_dtype).to(gpu))
    exp, bad = oracle_lib.embedding_fwd(to_u16(table), ids.numpy())
    assert bad == 0
    assert out.shape == (T, D)
    assert np.array_equal(to_u16(out).reshape(T, D), exp)


def test_embedding_fwd_flat_buffer_view(gpu, oracle_lib):
    """Table = [V, D] view of a flat FSDP buffer (v7/1e49beb8a123/problem.py:16-20), ids [1, T]."""
    g = gen(9)
    V, D = 4096, 1024
    flat = randn_bf16(V * D, g, 0.0, 0.02)
    ids = torch.randint(0, 100, (1, 512), generator=g)
    out = kp.aten.embedding(flat.to(gpu).view(8, -1).view(V, D), ids.to(gpu))
    exp, _ = oracle_lib.embedding_fwd(to_u16(flat).reshape(V, D), ids.numpy())
    assert out.shape == (1, 512, D)
    assert np.array_equal(to_u16(out).reshape(512, D), exp)


def test_embedding_fwd_out_of_range_flagged(gpu):
    table = torch.ones((10, 64), dtype=torch.bfloat16, device=gpu)
    ids = torch.tensor([1, 10, 3], device=gpu)
    with pytest.raises(IndexError):
        kp.embedding(table, ids)


@pytest.mark.parametrize("D", [4096, 4608])
@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_embedding_fwd_out_of_range_rows_zero_vector_path(gpu, oracle_lib, D, idx_dtype):
    """Out-of-range ids (negative, V, far above V) in the 16-byte path: those
    rows come out zero, every other row bit-exact, and the id is recorded."""
    g = gen(D + 5)
    V, T = 500, 300
    table = randn_bf16((V, D), g, 0.0, 0.02)
    ids = zipf_ids(T, V, 1.1, g)
    bad_pos = [0, 7, 150, T - 1]
    ids[bad_pos[0]], ids[bad_pos[1]], ids[bad_pos[2]], ids[bad_pos[3]] = -1, V, V + 100000, -(2 ** 30)
    kp.set_index_checking(False)
    try:
        kp.check_indices()
        out = kp.embedding(table.to(gpu), ids.to(idx_dtype).to(gpu))
        with pytest.raises(IndexError):
            kp.check_indices()
    finally:
        kp.set_index_checking(True)
    got = to_u16(out).reshape(T, D)
    assert not got[bad_pos].any()
    good = np.setdiff1d(np.arange(T), bad_pos)
    exp, _ = oracle_lib.embedding_fwd(to_u16(table), ids.clamp(0, V - 1).numpy())
    assert np.array_equal(got[good], exp[good])


def test_out_of_range_recorded_without_checking_mode(gpu):
    """With per-call checking off (the default outside the tests), an
    out-of-range id gives zero rows without a host synchronisation and is
    reported by the next kp.check_indices(); the record is then cleared."""
    table = torch.ones((10, 64), dtype=torch.bfloat16, device=gpu)
    kp.set_index_checking(False)
    try:
        kp.check_indices()  # nothing recorded yet (or cleared)
        out = kp.embedding(table, torch.tensor([1, 10, 3], device=gpu))
        assert torch.count_nonzero(out[1]) == 0 and torch.count_nonzero(out[0]) == 64
        grad = torch.ones((3, 64), dtype=torch.bfloat16, device=gpu)
        kp.embedding_dense_backward(grad, torch.tensor([1, -5, 3], device=gpu), 10)
        with pytest.raises(IndexError):
            kp.check_indices()
        kp.check_indices()  # cleared by the report
        kp.embedding(table, torch.tensor([1, 2, 3], device=gpu))
        kp.check_indices()
    finally:
        kp.set_index_checking(True)


def _check_bwd(gpu, O, V, D, ids, grad, padding_idx=-1, scale=False):
    T = ids.numel()
    out = kp.embedding_dense_backward(grad.to(gpu), ids.to(gpu), V, padding_idx, scale)
    torch.cuda.synchronize()
    rid, rows, absrows, counts, bad = O.embedding_bwd_rows(to_u16(grad), ids.numpy(), V, padding_idx, scale)
    assert bad == 0
    o = out.cpu().numpy().astype(np.float64)
    touched = np.zeros(V, bool)
    touched[rid] = True
    # untouched rows (incl. padding) are exactly zero
    assert not np.any(o[~touched]), "rows without contributions must be exactly 0"
    # touched rows: fp32 summation error bound gamma_{n-1} * sum|x| plus the final fp32 rounding
    got = o[rid]
    u = 2.0 ** -24
    n = counts[:, None].astype(np.float64)
    bound = (n * u / (1 - n * u)) * absrows + u * np.abs(rows) + 1e-30
    err = np.abs(got - rows)
    assert np.all(err <= bound), f"max err/bound {np.max(err / bound):.3f}"
    # column sums of the dense gradient equal the column sums of the contributing rows
    return out


_SLAB = (1 << 21) - 1  # ids per pass of the backward's sort (21 id bits in its keys)


@pytest.mark.parametrize("V,scale,pad", [(_SLAB + 1000, False, -1), (_SLAB + 1000, True, _SLAB + 7),
                                         (2 * _SLAB + 3, False, _SLAB + 7)])
def test_embedding_bwd_vocabulary_slabs(gpu, oracle_lib, V, scale, pad):
    """A vocabulary past the sort key's 21 id bits runs the pipeline once per
    slab of 2^21 - 1 rows: ids on both sides of every slab boundary, the last
    row, a hot id at the first row of the second slab (a run spanning
    windows), padding inside the second slab -- every touched row against the
    oracle's fp64 rows within the fp32 summation bound, every other row 0."""
    print(f"[emb bwd slabs] V={V} scale={scale} pad={pad}", flush=True)
    D, T = 64, 6000
    g = gen(V % 1000 + int(scale))
    ids = torch.randint(0, V, (T,), generator=g)
    special = [0, _SLAB - 1, _SLAB, _SLAB + 1, V - 1] + ([2 * _SLAB - 1, 2 * _SLAB] if V > 2 * _SLAB else [])
    ids[:len(special)] = torch.tensor(special)
    ids[100:180] = _SLAB
    if pad >= 0:
        ids[200:210] = pad
    grad = randn_bf16((T, D), g)
    out = _check_bwd(gpu, oracle_lib, V, D, ids, grad, padding_idx=pad, scale=scale)
    if pad >= 0:
        assert not out[pad].any()
    again = kp.embedding_dense_backward(grad.to(gpu), ids.to(gpu), V, pad, scale)
    assert torch.equal(out, again)  # bitwise repeatable


def test_embedding_bwd_vocabulary_slabs_bad_ids(gpu):
    """Out-of-range ids (negative, V, far above V) under the slab passes are
    skipped and recorded; the in-range rows of both slabs are unchanged."""
    V, D = _SLAB + 50, 32
    ids = torch.tensor([3, _SLAB + 2, -1, V, V + (1 << 22), _SLAB + 2, 3])
    grad = torch.ones((ids.numel(), D), dtype=torch.bfloat16)
    kp.set_index_checking(False)
    try:
        kp.check_indices()
        out = kp.embedding_dense_backward(grad.to(gpu), ids.to(gpu), V)
        with pytest.raises(IndexError):
            kp.check_indices()
    finally:
        kp.set_index_checking(True)
    assert torch.equal(out[3], torch.full((D,), 2.0, device=gpu))
    assert torch.equal(out[_SLAB + 2], torch.full((D,), 2.0, device=gpu))
    assert float(out.abs().sum()) == 4.0 * D


@pytest.mark.parametrize("V,D,T", [(1000, 4096, 777), (64, 128, 4000), (5000, 512, 2048), (37, 100, 250)])
def test_embedding_bwd_matches_oracle(gpu, oracle_lib, V, D, T):
    g = gen(V * 3 + T)
    ids = zipf_ids(T, V, 1.1, g)
    grad = randn_bf16((T, D), g)
    _check_bwd(gpu, oracle_lib, V, D, ids, grad)


@pytest.mark.parametrize("V,D,T,dist", [(128256, 256, 65536, "zipf"), (50000, 64, 40000, "uniform"),
                                        (20000, 128, 100000, "zipf")])
def test_embedding_bwd_many_tokens(gpu, oracle_lib, V, D, T, dist):
    """Token counts past one 2048-key chunk batch of the rank search (32 and
    49 chunks): [8, 8192] tokens of a 128256-id vocabulary, and uniform ids
    whose touched rows also fall in the unconditionally zeroed shares of the
    sort and rank launches (those rows must still end with their sums)."""
    print(f"[emb_bwd] V={V} D={D} T={T} {dist}", flush=True)
    g = gen(V + T)
    ids = zipf_ids(T, V, 1.1, g) if dist == "zipf" else torch.randint(0, V, (T,), generator=g)
    ids[-1] = V - 1  # the top row, inside the first unconditional share
    grad = randn_bf16((T, D), g)
    _check_bwd(gpu, oracle_lib, V, D, ids, grad)


def test_embedding_bwd_aten_full_batch_vs_eager(gpu):
    """aten.embedding_dense_backward at [8, 8192] tokens (65536) over the
    128256-id vocabulary, D = 4096 (bf16 out, the reference op's dtype):
    within the north-star tolerance of torch-ROCm eager, same untouched rows."""
    print("[emb_bwd] aten [8, 8192] x 4096 vs eager", flush=True)
    g = gen(31)
    V, D = 128256, 4096
    ids = zipf_ids(8 * 8192, V, 1.1, g).view(8, 8192).to(gpu)
    grad = randn_bf16((8, 8192, D), g).to(gpu)
    ours = kp.aten.embedding_dense_backward(grad, ids, V, -1, False)
    ref = torch.ops.aten.embedding_dense_backward.default(grad, ids, V, -1, False)
    assert ours.dtype == ref.dtype == torch.bfloat16 and ours.shape == ref.shape
    assert torch.equal(ours.abs().sum(1) == 0, ref.abs().sum(1) == 0)
    diff = (ours.float() - ref.float()).abs()
    assert bool((diff <= 1e-2 + 1.6e-2 * ref.float().abs()).all()), f"worst |diff| {float(diff.max()):.4g}"


def test_embedding_bwd_hot_row_and_padding(gpu, oracle_lib):
    g = gen(21)
    V, D, T = 300, 256, 3000
    ids = torch.randint(0, V, (T,), generator=g)
    ids[::3] = 7  # one id with ~1000 contributions (many parts)
    ids[1::5] = 5  # padding id
    grad = randn_bf16((T, D), g)
    out = _check_bwd(gpu, oracle_lib, V, D, ids, grad, padding_idx=5)
    assert torch.count_nonzero(out[5]) == 0


def test_embedding_bwd_scale_grad_by_freq(gpu, oracle_lib):
    g = gen(22)
    V, D, T = 200, 64, 1500
    ids = zipf_ids(T, V, 1.1, g)
    grad = randn_bf16((T, D), g)
    _check_bwd(gpu, oracle_lib, V, D, ids, grad, scale=True)


def test_embedding_bwd_all_same_id(gpu, oracle_lib):
    g = gen(23)
    V, D, T = 16, 512, 4096
    ids = torch.full((T,), 3, dtype=torch.int64)
    grad = randn_bf16((T, D), g)
    _check_bwd(gpu, oracle_lib, V, D, ids, grad)


def test_embedding_bwd_deterministic_and_dtypes(gpu):
    g = gen(24)
    V, D, T = 4000, 1024, 4096
    ids = zipf_ids(T, V, 1.1, g).to(gpu)
    grad = randn_bf16((T, D), g).to(gpu)
    a = kp.embedding_dense_backward(grad, ids, V)
    b = kp.embedding_dense_backward(grad, ids, V)
    assert torch.equal(a, b)
    r = kp.embedding_dense_backward(grad, ids, V, round_to_bf16=True)
    assert torch.equal(r, a.to(torch.bfloat16).float())
    h = kp.aten.embedding_dense_backward(grad, ids, V, -1, False)
    assert h.dtype == torch.bfloat16 and torch.equal(h, a.to(torch.bfloat16))


def test_embedding_bwd_vs_torch_eager(gpu, oracle_lib):
    """torch-ROCm eager embedding_dense_backward (the reference op, bf16 output)
    on the reference's own id distribution (randint(0, 100), v7/a12a160cb11b).
    Eager rounds to bf16 between index batches, so it is the less accurate of
    the two: ours must be at least as close to the exact sums everywhere, and
    both must agree on which rows are untouched."""
    g = gen(25)
    V, D, T = 1000, 512, 2048
    ids = torch.randint(0, 100, (1, T), generator=g)
    grad = randn_bf16((1, T, D), g)
    ref = torch.ops.aten.embedding_dense_backward.default(grad.to(gpu), ids.to(gpu), V, -1, False)
    out = kp.embedding_dense_backward(grad.to(gpu), ids.to(gpu), V, -1, False)
    exact = np.zeros((V, D))
    rid, rows, _, _, _ = oracle_lib.embedding_bwd_rows(to_u16(grad), ids.numpy(), V)
    exact[rid] = rows
    o = out.cpu().numpy().astype(np.float64)
    r = ref.float().cpu().numpy().astype(np.float64)
    untouched = np.ones(V, bool)
    untouched[rid] = False
    assert not np.any(r[untouched]) and not np.any(o[untouched])
    assert np.all(np.abs(o - exact) <= np.abs(r - exact) + 2.0 ** -20 * np.abs(exact) + 1e-6)


def test_embedding_bwd_empty(gpu):
    out = kp.embedding_dense_backward(torch.empty((0, 64), dtype=torch.bfloat16, device=gpu),
                                      torch.empty(0, dtype=torch.int64, device=gpu), 10)
    assert out.shape == (10, 64) and torch.count_nonzero(out) == 0


def test_embedding_bwd_on_side_stream_repeated(gpu, oracle_lib):
    """Calls issued on a non-default torch stream, back to back, must give the
    oracle's rows and identical bits each time: the window tickets that let
    the last window block of a spanning run finish it are cleared by every
    call, and all of a call's work stays ordered on the caller's stream."""
    g = gen(26)
    V, D, T = 3000, 2048, 8192
    ids = zipf_ids(T, V, 1.1, g)
    grad = randn_bf16((T, D), g)
    exact = oracle_lib.embedding_bwd_dense(to_u16(grad), ids.numpy(), V)
    side = torch.cuda.Stream(device=gpu)
    gd, idd = grad.to(gpu), ids.to(gpu)
    torch.cuda.synchronize()
    outs = []
    with torch.cuda.stream(side):
        for _ in range(3):
            o = kp.embedding_dense_backward(gd, idd, V)
            outs.append(o.clone())  # enqueued on `side` after the join
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    np.testing.assert_allclose(outs[0].cpu().numpy(), exact, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("V,D,T,idx_dtype", [(1000, 4096, 777, torch.int64), (5000, 8192, 300, torch.int32),
                                              (300, 2048, 64, torch.int64), (50, 100, 33, torch.int64)])
def test_embedding_rms_norm_equals_the_two_launch_composition(gpu, V, D, T, idx_dtype):
    """The fused gather + norm (D = 100: the two-launch fallback) against
    embedding() then rms_norm(): h, y and rstd bit for bit, and y within the
    oracle's tolerance."""
    print(f"[emb+rms] V={V} D={D} T={T} {idx_dtype}", flush=True)
    g = torch.Generator().manual_seed(V + D + T)
    table = (torch.randn(V, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    w = (1 + 0.02 * torch.randn(D, generator=g)).to(torch.bfloat16).to(gpu)
    ids = torch.randint(0, V, (T,), generator=g).to(idx_dtype).to(gpu)
    h, y, r = kp.embedding_rms_norm(table, ids, w, 1e-5, return_h=True)
    emb = kp.embedding(table, ids)
    _, y2, r2 = kp.rms_norm([emb], w, 1e-5, D)
    assert torch.equal(h, emb) and torch.equal(y, y2) and torch.equal(r, r2.view(r.shape))
    _, yo, _ = oracle.rmsnorm_fwd([to_u16(emb)], to_u16(w), 1e-5, D)
    assert (ulp_bf16(to_u16(y), yo) <= 1).all()


def test_embedding_rms_norm_long_block_walk(gpu):
    """1.2M tokens of width 512: each block walks ~150 row steps, so the
    ids it holds in lanes (64 steps at a time) are fetched again twice;
    h, y and rstd bit for bit those of embedding() then rms_norm()."""
    V, D, T = 1000, 512, 1_200_000
    print(f"[emb+rms long] V={V} D={D} T={T}", flush=True)
    g = torch.Generator().manual_seed(12)
    table = (torch.randn(V, D, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    w = (1 + 0.02 * torch.randn(D, generator=g)).to(torch.bfloat16).to(gpu)
    ids = torch.randint(0, V, (T,), generator=g, dtype=torch.int32).to(gpu)
    h, y, r = kp.embedding_rms_norm(table, ids, w, 1e-5, return_h=True)
    emb = kp.embedding(table, ids)
    assert torch.equal(h, emb)
    del h
    _, y2, r2 = kp.rms_norm([emb], w, 1e-5, D)
    assert torch.equal(y, y2) and torch.equal(r, r2.view(r.shape))


def test_embedding_rms_norm_fsdp_weight_and_bad_ids(gpu):
    """Weight as an [8, 512] row-strided view of a flat buffer; ids outside
    [0, V) give zero h / y rows and raise with index checking on."""
    V, D = 64, 4096
    g = torch.Generator().manual_seed(11)
    table = torch.randn(V, D, generator=g).to(torch.bfloat16).to(gpu)
    flat = torch.randn(8 * 27264, generator=g).to(torch.bfloat16).to(gpu)
    wv = flat.as_strided((8, 512), (27264, 1))
    ids = torch.tensor([[3, 63, 0, 17]], device=gpu)
    h, y, _ = kp.embedding_rms_norm(table, ids, wv, 1e-5, return_h=True)
    _, y2, _ = kp.rms_norm([kp.embedding(table, ids)], wv.contiguous().view(-1), 1e-5, D)
    assert y.shape == (1, 4, D) and torch.equal(y, y2)
    bad = torch.tensor([1, 64, -1, 5], device=gpu)
    with pytest.raises(IndexError):
        kp.embedding_rms_norm(table, bad, wv, 1e-5)
    kp.set_index_checking(False)
    try:
        h, y, r = kp.embedding_rms_norm(table, bad, wv, 1e-5, return_h=True)
    finally:
        kp.set_index_checking(True)
    assert not h[1:3].any() and not y[1:3].any()
    assert torch.equal(h[[0, 3]], table[[1, 5]])
