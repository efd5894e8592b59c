"""The oracle (CPU) and the HIP kernels (GPU) against the committed golden
vectors of tests/golden/golden.npz (made by tests/golden/make_golden.py with
torch library ops in float64)."""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests._util import bf, from_u16, ulp_bf16

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")


def _check_rms_fwd(y, rstd, tag, exact_ulps=1):
    u = ulp_bf16(y, G[f"{tag}_y"])
    assert u.max() <= exact_ulps, u.max()
    np.testing.assert_allclose(rstd, G[f"{tag}_rstd"], rtol=4 * 2.0**-24)


def _check_dx(dx, exact):
    assert np.all(np.abs(bf(dx) - exact) <= 2.0**-8 * np.abs(exact) + 1e-5 * np.abs(exact).max())


def _dw_bound(rstd):
    x = bf(G["rms_x"])
    return 2.0**-22 * (np.abs(bf(G["rms_dy"]) * x) * np.abs(rstd)[:, None]).sum(0) + 1e-9


def _check_emb_bwd(dense):
    exact, absd = G["emb_bwd"], G["emb_bwd_abs"]
    counts = np.bincount(G["emb_ids"][G["emb_ids"] != G["emb_pad"]], minlength=exact.shape[0])[:, None]
    # fp32 accumulation: within (count + 1) * 2^-24 * sum|g| of the fp64 sum
    assert np.all(np.abs(dense.astype(np.float64) - exact) <= (counts + 1) * 2.0**-24 * absd)
    assert not dense[int(G["emb_pad"])].any()


def _check_rope(out_u16, exact):
    ov = bf(out_u16)
    # one bf16 rounding; the angle reduction and fp32 evaluation add < 1e-5 absolute
    assert np.all(np.abs(ov - exact) <= 2.0**-8 * np.abs(exact) + 1e-5)


# ---------------------------------------------------------------- CPU: oracle
def test_oracle_rms_fwd_golden():
    eps = float(G["rms_eps"])
    _, y, r = oracle.rmsnorm_fwd([G["rms_x"]], G["rms_w"], eps, G["rms_x"].shape[1])
    _check_rms_fwd(y, r, "rms", exact_ulps=0)
    h, y, r = oracle.rmsnorm_fwd([G["rms_res"], G["rms_x"]], G["rms_w"], eps, G["rms_x"].shape[1])
    assert np.array_equal(h, G["rms_h"])
    _check_rms_fwd(y, r, "addrms", exact_ulps=0)


def test_oracle_rms_bwd_golden():
    eps, N = float(G["rms_eps"]), G["rms_x"].shape[1]
    dx, dw, r = oracle.rmsnorm_bwd([G["rms_dy"]], [G["rms_x"]], None, G["rms_w"], eps, N)
    _check_dx(dx, G["rmsbwd_dx"])
    assert np.all(np.abs(dw - G["rmsbwd_dw"]) <= _dw_bound(r))
    dx, dw, _ = oracle.rmsnorm_bwd([G["rms_dy"]], [G["rms_x"]], G["rmsbwd_given_rstd"], G["rms_w"], eps, N)
    _check_dx(dx, G["rmsbwd_given_dx"])
    np.testing.assert_allclose(dw, G["rmsbwd_given_dw"], rtol=1e-12, atol=1e-12)


def test_oracle_embedding_golden():
    out, bad = oracle.embedding_fwd(G["emb_table"], G["emb_ids"])
    assert bad == 0 and np.array_equal(out, G["emb_fwd"])
    dense = oracle.embedding_bwd_dense(G["emb_grad"], G["emb_ids"], G["emb_table"].shape[0], int(G["emb_pad"]))
    _check_emb_bwd(dense)


def test_oracle_rope_golden():
    out = oracle.rope(G["rope_x"], G["rope_pos"], pairing="half", theta=float(G["rope_theta"]))
    _check_rope(out, G["rope_half"])
    out = oracle.rope(G["rope_x"], G["rope_tpos"], pairing="interleaved", freqs=G["rope_table"])
    _check_rope(out, G["rope_inter"])


def _check_swiglu(out, db, da, exact=True):
    if exact:
        assert np.array_equal(out, G["swiglu_out"])
    else:
        # fp32 evaluation: e^-a overflows for a < -88.7, so silu(a) is -0 there
        # where the exact value is a tiny negative number; NaN may carry a sign
        ov, ev = bf(out), bf(G["swiglu_out"])
        nan = np.isnan(ev)
        assert np.array_equal(np.isnan(ov), nan)
        fin = np.isfinite(ev)
        assert np.array_equal(ov[~fin & ~nan], ev[~fin & ~nan])
        assert ulp_bf16(out, G["swiglu_out"])[fin & (np.abs(ev) > 1e-30)].max() <= 1
        assert np.all(np.abs(ov[fin] - ev[fin]) <= 1e-30 + 2.0**-8 * np.abs(ev[fin]))
    assert np.array_equal(db, G["swiglu_db"])
    ex = G["swiglu_da_exact"]
    v = bf(da)
    nan = np.isnan(ex)
    assert np.array_equal(np.isnan(v), nan)
    # one bf16 rounding of the exact value (signed zeros compare equal); in
    # fp32, sig underflows to 0 for a < -88.7 where the exact da is ~1e-37
    slack = 0.0 if exact else 1e-30
    assert np.all(np.abs(v[~nan] - ex[~nan]) <= 2.0**-8 * np.abs(ex[~nan]) + slack)


def test_oracle_swiglu_golden():
    out = oracle.swiglu_fwd(G["swiglu_a"], G["swiglu_b"])
    db, da = oracle.swiglu_bwd(G["swiglu_g"], G["swiglu_s"], G["swiglu_b"], G["swiglu_a"])
    _check_swiglu(out, db, da)


def test_oracle_loss_golden():
    loss, tw, lse, bad = oracle.cross_entropy_fwd(G["xent_x"], G["xent_t"], scale=float(G["xent_scale"]))
    assert bad == 0 and tw == float(G["xent_tw"])
    assert loss == pytest.approx(float(G["xent_loss"]), rel=1e-13)
    np.testing.assert_allclose(lse, G["xent_lse"], rtol=1e-13)
    out, _ = oracle.cross_entropy_bwd(G["xent_L"], G["xent_t"], float(G["xent_scale"]))
    assert np.array_equal(out, G["xent_grad"])


# ---------------------------------------------------------------- GPU: kernels
@pytest.mark.gpu
def test_kernels_rms_golden(gpu):
    import kernelproblems_amd as kp

    eps, N = float(G["rms_eps"]), G["rms_x"].shape[1]
    x, res, dy, w = (from_u16(G[k], gpu) for k in ("rms_x", "rms_res", "rms_dy", "rms_w"))
    _, y, r = kp.rms_norm([x], w, eps, N)
    _check_rms_fwd(y.cpu().view(torch.int16).numpy().view(np.uint16), r.cpu().numpy(), "rms")
    h, y, r = kp.rms_norm([res, x], w, eps, N, return_h=True)
    assert np.array_equal(h.cpu().view(torch.int16).numpy().view(np.uint16), G["rms_h"])
    _check_rms_fwd(y.cpu().view(torch.int16).numpy().view(np.uint16), r.cpu().numpy(), "addrms")
    dx, dw = kp.rms_norm_backward([dy], [x], None, w, eps, N)
    _check_dx(dx.cpu().view(torch.int16).numpy().view(np.uint16), G["rmsbwd_dx"])
    _, _, r = kp.rms_norm([x], w, eps, N)
    assert np.all(np.abs(dw.cpu().double().numpy() - G["rmsbwd_dw"]) <= _dw_bound(r.cpu().numpy()))
    rs = torch.from_numpy(G["rmsbwd_given_rstd"]).to(gpu)
    dx, dw = kp.rms_norm_backward([dy], [x], rs, w, eps, N)
    _check_dx(dx.cpu().view(torch.int16).numpy().view(np.uint16), G["rmsbwd_given_dx"])
    ex = G["rmsbwd_given_dw"]
    mag = (np.abs(bf(G["rms_dy"]) * bf(G["rms_x"])) * np.abs(G["rmsbwd_given_rstd"])[:, None]).sum(0)
    assert np.all(np.abs(dw.cpu().double().numpy() - ex) <= 2.0**-20 * mag)


@pytest.mark.gpu
def test_kernels_embedding_golden(gpu):
    import kernelproblems_amd as kp

    table, grad = from_u16(G["emb_table"], gpu), from_u16(G["emb_grad"], gpu)
    ids = torch.from_numpy(G["emb_ids"]).to(gpu)
    out = kp.embedding(table, ids)
    assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), G["emb_fwd"])
    dense = kp.embedding_dense_backward(grad, ids, table.shape[0], int(G["emb_pad"]))
    _check_emb_bwd(dense.cpu().numpy())


@pytest.mark.gpu
def test_kernels_rope_golden(gpu):
    import kernelproblems_amd as kp

    x = from_u16(G["rope_x"], gpu)
    out, _ = kp.rope(x, positions=torch.from_numpy(G["rope_pos"]).to(gpu), theta=float(G["rope_theta"]))
    _check_rope(out.cpu().view(torch.int16).numpy().view(np.uint16), G["rope_half"])
    tab = torch.from_numpy(G["rope_table"]).to(gpu)
    out, _ = kp.rope(x, positions=torch.from_numpy(G["rope_tpos"]).to(gpu), freqs_cis=tab, pairing="interleaved")
    _check_rope(out.cpu().view(torch.int16).numpy().view(np.uint16), G["rope_inter"])


@pytest.mark.gpu
def test_kernels_swiglu_golden(gpu):
    import kernelproblems_amd as kp

    a, b, g, s = (from_u16(G[f"swiglu_{k}"], gpu) for k in "abgs")
    out = kp.swiglu(a, b)
    db, da = kp.swiglu_backward(g, s, b, a)
    u16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    _check_swiglu(u16(out), u16(db), u16(da), exact=False)


@pytest.mark.gpu
def test_kernels_loss_golden(gpu):
    import kernelproblems_amd as kp

    x = from_u16(G["xent_x"], gpu)
    t = torch.from_numpy(G["xent_t"]).to(gpu)
    loss, tw, lse = kp.cross_entropy_loss(x, t, scale=float(G["xent_scale"]), return_lse=True)
    assert float(tw) == float(G["xent_tw"])
    # fp32 exponentials and sums over 333 terms: well inside 1e-6 relative
    assert float(loss) == pytest.approx(float(G["xent_loss"]), rel=1e-6)
    np.testing.assert_allclose(lse.cpu().double().numpy(), G["xent_lse"], rtol=1e-6)
    out = kp.cross_entropy_backward(torch.from_numpy(G["xent_L"]).to(gpu), t, float(G["xent_scale"]))
    u = ulp_bf16(out.cpu().view(torch.int16).numpy().view(np.uint16), G["xent_grad"])
    assert u.max() <= 1 and (u == 0).mean() > 0.99
