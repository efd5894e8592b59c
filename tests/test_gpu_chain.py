"""GPU parity of the RMSNorm forward -> backward -> embedding backward chain
(v6/0b493aad68f0, v5/118d525f44e0; and v8/f6251e84e3fa, whose forward arrives
saved) link by link against torch-ROCm eager:
the norm output and weight gradient within the bf16 tolerance, the summed
gradient rows g = add_220 + dx within the bf16 tolerance, the table gradient
against eager's embedding_dense_backward of our own g (accumulation order
only), and against eager's whole chain within the bound that the summands'
differences allow: |table - table_eager| <= sum over the id's tokens of
|g - g_eager| + one bf16 rounding of each side."""
import pytest
import torch

from kernelproblems_amd import fragments as fr
from kernelproblems_amd import fused as F
from tests._util import BF16_ATOL, BF16_RTOL

pytestmark = pytest.mark.gpu
aten = torch.ops.aten
V = 128256
EPS = 1e-05


def _close(a, e, what, rtol=BF16_RTOL, atol=BF16_ATOL):
    bad = (a.double() - e.double()).abs() > atol + rtol * e.double().abs()
    assert int(bad.sum()) == 0, f"{what}: {int(bad.sum())} of {a.numel()} outside rtol={rtol} atol={atol}"


@pytest.mark.parametrize("fid", ["v6/0b493aad68f0", "v5/118d525f44e0", "v8/f6251e84e3fa"])
def test_chain_link_by_link(gpu, fid):
    print(f"[chain] {fid}", flush=True)
    mod = fr.load(fid)
    gen = torch.Generator(device=gpu).manual_seed(7)
    inputs = mod.get_inputs(device=gpu, generator=gen)
    saved = None
    if fid == "v6/0b493aad68f0":
        x, w, a, b, c, res, ids = inputs
        w_eager = w
    elif fid == "v5/118d525f44e0":
        wv, x, a, b, c, res, ids = inputs
        w = wv
        w_eager = aten._unsafe_view.default(aten.clone.default(wv, memory_format=torch.contiguous_format), [-1])
    else:  # the saved forward arrives as a tuple; only its rstd is read
        saved, a, b, c, x, w, res, ids = inputs
        w_eager = w
    outs = mod.kernel_function(*inputs)
    dw, table = outs[-2], outs[-1]

    # eager chain, link by link
    if saved is None:
        ye, re = aten._fused_rms_norm.default(x, [x.shape[-1]], w_eager, EPS)
    else:
        ye, re = None, saved[1]
    dy = aten.add.Tensor(aten.add.Tensor(a.view(x.shape), b.view(x.shape)), c.view(x.shape))
    dxe, dwe = aten._fused_rms_norm_backward.default(dy, x, [x.shape[-1]], re, w_eager, [True, True])
    ge = aten.add.Tensor(res, dxe)
    if ye is not None:
        y0, y1, y2 = outs[:3]
        _close(y0, ye.view(y0.shape), "y")
        assert y1.data_ptr() == y0.data_ptr() == y2.data_ptr()
    _close(dw, dwe.float(), "dw")

    # our g, the chain's middle link, made the way the chain makes it: one row
    # pass for the forward and backward (rstd computed once from x), or the
    # backward from the saved rstd
    if saved is None:
        _, g, _, _, _ = F.rms_norm_forward_backward([a, b, c], [x], w, EPS, x.shape[-1], dx_residual=res, dw=None)
    else:
        g, _ = F.rms_norm_backward([a, b, c], [x], saved[1], w, EPS, x.shape[-1], dx_residual=res, dw=None)
    _close(g, ge, "g = add_220 + dx")

    # the table from our g: eager's bf16 embedding backward of the same rows
    t_same = aten.embedding_dense_backward.default(g, ids, V, -1, False).float()
    _close(table, t_same, "table vs eager(our g)")

    # against eager's whole chain: bounded by the summands' differences
    te = aten.embedding_dense_backward.default(ge, ids, V, -1, False).float()
    dsum = aten.embedding_dense_backward.default((g.float() - ge.float()).abs(), ids, V, -1, False)
    bound = dsum + 2.0**-8 * (table.abs() + te.abs()) + 1e-6
    excess = (table - te).abs() - bound
    assert float(excess.max()) <= 0, f"table vs eager chain: max excess over the bound {float(excess.max()):.4g}"


def _compose(dy_terms, x, rstd, w, res, ids, v, pad, want_y, out_dtype):
    """The unfused form of the fused chain: the norm entry point writes g,
    then the embedding backward reads it back (same y, g and table bits)."""
    n = x.shape[-1]
    if rstd is None:
        y, g, dw, _, _ = F.rms_norm_forward_backward(dy_terms, [x], w, EPS, n, dx_residual=res, dw="f32")
    else:
        y = None
        g, dw = F.rms_norm_backward(dy_terms, [x], rstd, w, EPS, n, dx_residual=res, dw="f32")
    table = F.embedding_dense_backward(g, ids, v, pad, False, out_dtype=out_dtype, round_to_bf16=True)
    return (y if want_y else None), dw, table


# (name, M, N, dy terms, vocabulary, ids, padding_idx, saved rstd, y, table dtype)
FUSED_CASES = [
    ("fragment_fwd", 8192, 4096, 3, 128256, "randint100", -1, False, True, torch.float32),
    ("fragment_saved_rstd", 8192, 4096, 3, 128256, "randint100", -1, True, False, torch.float32),
    ("short_runs_no_y", 1000, 4096, 1, 5000, "uniform", -1, False, False, torch.float32),
    ("padding_and_out_of_range", 777, 2048, 2, 3000, "padded", 3, False, True, torch.float32),
    ("one_run_all_windows", 300, 8192, 1, 1000, "constant", -1, True, False, torch.float32),
    ("bf16_table", 513, 4096, 2, 4000, "uniform", -1, False, True, torch.bfloat16),
    ("unsupported_width_falls_back", 96, 1000, 2, 700, "uniform", -1, False, True, torch.float32),
]


def _ids(kind, m, v, g, gpu):
    if kind == "randint100":
        ids = torch.randint(0, 100, (1, m), generator=g)
    elif kind == "uniform":
        ids = torch.randint(0, v, (1, m), generator=g)
    elif kind == "constant":
        ids = torch.full((1, m), 42, dtype=torch.int64)
    else:  # padding index 3 on ~10% of the tokens, a few ids out of range (-1, v, v + 5)
        ids = torch.randint(0, 40, (1, m), generator=g)
        ids[torch.rand((1, m), generator=g) < 0.1] = 3
        ids[0, 5], ids[0, 200], ids[0, 600] = -1, v, v + 5
    return ids.to(gpu)


@pytest.mark.parametrize("case", FUSED_CASES, ids=[c[0] for c in FUSED_CASES])
def test_fused_chain_matches_composition(gpu, case):
    """rms_norm_embedding_backward (one row pass that sums g = res + dx into
    the table in registers) against the norm entry point followed by the
    embedding backward of the stored g: y and the table bit for bit (the same
    per-row results, summed in the same ascending token order per id), the
    weight gradient within fp32 summation-order differences (its rows are
    grouped differently) and bitwise equal over two calls."""
    name, m, n, n_dy, v, kind, pad, saved, want_y, out_dtype = case
    print(f"[chain] fused vs composition: {name}", flush=True)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(m, n, generator=g).to(torch.bfloat16).to(gpu)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16).to(gpu)
    dys = [torch.randn(m, n, generator=g).to(torch.bfloat16).to(gpu) for _ in range(n_dy)]
    w = (1 + 0.02 * torch.randn(n, generator=g)).to(torch.bfloat16).to(gpu)
    ids = _ids(kind, m, v, g, gpu)
    rstd = None
    if saved:
        _, _, rstd = F.rms_norm([x], w, EPS, n, return_rstd=True)

    def fused():
        return F.rms_norm_embedding_backward(dys, x, rstd, w, EPS, n, res, ids, v, pad, want_y=want_y, dw="f32",
                                             out_dtype=out_dtype, round_to_bf16=True)

    bad_ids = kind == "padded"
    if bad_ids:  # out-of-range ids raise in checking mode, and are recorded (and skipped) without it
        with pytest.raises(IndexError):
            fused()
        F.set_index_checking(False)
    try:
        yc, dwc, tc = _compose(dys, x, rstd, w, res, ids, v, pad, want_y, out_dtype)
        if bad_ids:
            with pytest.raises(IndexError):
                F.check_indices()  # the composition's record (reported, then cleared)
        runs = [fused() for _ in range(2)]
        torch.cuda.synchronize()
        if bad_ids:
            with pytest.raises(IndexError):
                F.check_indices()
    finally:
        F.set_index_checking(True)
    (y, dw, table), (y2, dw2, table2) = runs
    assert table.dtype == out_dtype and table.shape == (v, n)
    assert torch.equal(table.view(torch.int16) if out_dtype == torch.bfloat16 else table.view(torch.int32),
                       tc.view(torch.int16) if out_dtype == torch.bfloat16 else tc.view(torch.int32)), \
        "table differs from the embedding backward of the stored g"
    if want_y:
        assert torch.equal(y.view(torch.int16), yc.view(torch.int16))
    else:
        assert y is None
    assert torch.equal(dw.view(torch.int32), dw2.view(torch.int32)) and torch.equal(table, table2)
    scale = float(dwc.abs().max()) + 1e-30
    assert float((dw - dwc).abs().max()) <= 1e-5 * scale, "weight gradient beyond summation-order differences"
