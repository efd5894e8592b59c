"""GPU parity of the cross-entropy kernels (v8/71f1d2c9f38b forward,
v8/622c35f5d1c6 backward) with the fp64 CPU oracle on seeded inputs --
16-byte path (full and tail steps, row-strided views) and scalar path
(ragged V, unaligned views), ignored and out-of-range targets, -inf and
large logits that move the running max -- and with torch-ROCm eager at the
fragments' full shape (backward bit for bit)."""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
import oracle
from tests._util import from_u16, to_u16, ulp_bf16

pytestmark = pytest.mark.gpu

# fp32 exponentials and per-lane sums of a few thousand terms, fp64 row sums:
# the loss within 2e-6 relative of the exact value; each lse within 2e-6
# absolute (whatever the logits' magnitude) plus its fp32 output rounding
LOSS_RTOL = 2e-6


def _check_lse(lse, exact):
    np.testing.assert_allclose(lse.cpu().double().numpy(), exact, rtol=2.0**-24, atol=2e-6)


def _logits(M, V, gen, gpu, kind="contig", std=2.0):
    x = (torch.randn(M, V + 24, generator=gen) * std).to(torch.bfloat16)
    if kind == "contig":
        return x[:, :V].contiguous().to(gpu)
    if kind == "rows":       # row stride V + 24 (16-byte granular)
        return x.to(gpu)[:, 8:8 + V]
    if kind == "unaligned":  # 3 elements into each row: scalar path
        return x.to(gpu)[:, 3:3 + V]
    raise ValueError(kind)


def _targets(M, V, gen, gpu, dtype=torch.int64):
    t = torch.randint(0, V, (M,), generator=gen)
    t[::4] = -100
    return t.to(dtype).to(gpu)


FWD_CASES = [("contig", 1, 8), ("contig", 5, 1000), ("contig", 16, 128256), ("contig", 7, 1003),
             ("rows", 6, 4096), ("unaligned", 5, 2000), ("contig", 64, 2048 + 8)]


@pytest.mark.parametrize("kind,M,V", FWD_CASES)
@pytest.mark.parametrize("tdtype", [torch.int64, torch.int32])
def test_fwd_matches_oracle(gpu, kind, M, V, tdtype):
    print(f"[xent fwd] {kind} [{M},{V}] {tdtype}", flush=True)
    g = torch.Generator().manual_seed(M * 13 + V)
    x, t = _logits(M, V, g, gpu, kind), _targets(M, V, g, gpu, tdtype)
    loss, tw, lse = kp.cross_entropy_loss(x, t, scale=1 / 8192, return_lse=True)
    eloss, etw, else_, bad = oracle.cross_entropy_fwd(to_u16(x), t.cpu().numpy(), scale=1 / 8192)
    assert bad == 0 and float(tw) == etw
    assert float(loss) == pytest.approx(eloss, rel=LOSS_RTOL)
    _check_lse(lse, else_)


def test_fwd_special_rows(gpu):
    """-inf logits (masked vocabulary), a row that is -inf but for its target,
    logits of 1e3 and 3e4 (exponentials against a stale running max would
    overflow), a ramp whose max only arrives at the end, and constant rows."""
    V = 4096
    x = torch.randn(8, V, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    x[0, 100:3000] = float("-inf")
    x[1, :] = float("-inf")
    x[1, 7] = 0.5
    x[2, 2047] = 1000.0
    x[3, ::97] = 30000.0
    x[4] = torch.linspace(-60, 60, V).to(torch.bfloat16)
    x[5] = 3.0
    x[6, :8] = 80.0
    x[7] = -1e4
    t = torch.tensor([5, 7, 2047, 0, V - 1, 11, -100, 3])
    xd, td = x.to(gpu), t.to(gpu)
    loss, tw, lse = kp.cross_entropy_loss(xd, td, return_lse=True)
    eloss, etw, else_, _ = oracle.cross_entropy_fwd(to_u16(x), t.numpy())
    assert float(tw) == etw == 7
    _check_lse(lse, else_)
    assert float(loss) == pytest.approx(eloss, rel=LOSS_RTOL)


def test_fwd_out_of_range_targets(gpu):
    x = torch.randn(4, 64, device=gpu).to(torch.bfloat16)
    t = torch.tensor([1, 64, -100, -5], device=gpu)
    with pytest.raises(IndexError):
        kp.cross_entropy_loss(x, t)  # index checking is on for the GPU tests
    kp.set_index_checking(False)
    try:
        loss, tw = kp.cross_entropy_loss(x, t)
    finally:
        kp.set_index_checking(True)
    eloss, etw, _, bad = oracle.cross_entropy_fwd(to_u16(x), t.cpu().numpy())
    assert bad == 2 and float(tw) == etw == 1
    assert float(loss) == pytest.approx(eloss, rel=LOSS_RTOL)


def test_fwd_deterministic_and_empty(gpu):
    g = torch.Generator().manual_seed(4)
    x, t = _logits(300, 32000, g, gpu), _targets(300, 32000, g, gpu)
    a = kp.cross_entropy_loss(x, t)
    b = kp.cross_entropy_loss(x, t)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    e = torch.empty((0, 128), dtype=torch.bfloat16, device=gpu)
    loss, tw = kp.cross_entropy_loss(e, torch.empty(0, dtype=torch.int64, device=gpu))
    assert float(loss) == 0.0 and float(tw) == 0.0


BWD_CASES = [("contig", 1, 8), ("contig", 5, 1000), ("contig", 9, 128256), ("contig", 7, 1003), ("contig", 3, 1004),
             ("rows", 6, 4096), ("unaligned", 4, 2000)]


@pytest.mark.parametrize("kind,M,V", BWD_CASES)
@pytest.mark.parametrize("true_lsm", [False, True])
def test_bwd_matches_oracle(gpu, kind, M, V, true_lsm):
    print(f"[xent bwd] {kind} [{M},{V}] true_lsm={true_lsm}", flush=True)
    g = torch.Generator().manual_seed(M * 17 + V + true_lsm)
    x = torch.randn(M, V + 24, generator=g) * 2
    if true_lsm:
        x = torch.log_softmax(x, 1)
    base = x.to(gpu)
    L = {"contig": base[:, :V].contiguous(), "rows": base[:, 8:8 + V], "unaligned": base[:, 3:3 + V]}[kind]
    t = _targets(M, V, g, gpu)
    out = kp.cross_entropy_backward(L, t, 1 / 8192)
    eo, bad = oracle.cross_entropy_bwd(L.cpu().numpy(), t.cpu().numpy(), 1 / 8192)
    assert bad == 0
    u = ulp_bf16(to_u16(out), eo)
    assert u.max() <= 1 and (u == 0).mean() > 0.999


def test_bwd_ignored_and_out_of_range_rows(gpu):
    L = torch.randn(4, 4096, device=gpu)
    t = torch.tensor([-100, 4096, 5, -3], device=gpu)
    with pytest.raises(IndexError):
        kp.cross_entropy_backward(L, t, 0.5)
    kp.set_index_checking(False)
    try:
        out = kp.cross_entropy_backward(L, t, 0.5)
    finally:
        kp.set_index_checking(True)
    assert not out[[0, 1, 3]].any()
    eo, bad = oracle.cross_entropy_bwd(L.cpu().numpy(), t.cpu().numpy(), 0.5)
    assert bad == 2 and (ulp_bf16(to_u16(out), eo) <= 1).all()


@pytest.mark.parametrize("M,V", [(8192, 128256), (37, 1003)])
def test_against_torch_eager(gpu, M, V):
    """Backward: the same fp32 operations as torch's nll_loss_backward ->
    _log_softmax_backward_data kernels (expf, one product, one subtraction),
    bit for bit.  Forward: a different summation order, within LOSS_RTOL
    of eager's fp32 result (and the total weight exact)."""
    print(f"[xent eager] [{M},{V}]", flush=True)
    g = torch.Generator(device=gpu).manual_seed(8)
    aten = torch.ops.aten
    t = torch.randint(0, V, (M,), device=gpu, generator=g)
    t[::7] = -100
    L = torch.randn(M, V, device=gpu, generator=g)
    gl = torch.ones((), device=gpu) / 8192.0
    ref = aten._log_softmax_backward_data(
        aten.nll_loss_backward(gl, L, t, None, 2, -100, (t != -100).sum().float()), L, 1, torch.float32
    ).to(torch.bfloat16)
    out = kp.cross_entropy_backward(L, t, 1 / 8192)
    assert torch.equal(out, ref)
    del L, ref, out
    x = (torch.randn(M, V, device=gpu, generator=g) * 2).to(torch.bfloat16)
    eloss, etw = aten.nll_loss_forward(aten._log_softmax(x.float(), 1, False), t, None, 2, -100)
    loss, tw = kp.cross_entropy_loss(x, t, scale=1 / 8192)
    assert float(tw) == float(etw)
    assert float(loss) == pytest.approx(float(eloss) / 8192, rel=1e-5)


# ---------------------------------------------------------------- forward + backward from the logits
FB_CASES = [("contig", 1, 8), ("contig", 5, 1000), ("contig", 4, 16384), ("contig", 3, 40000),
            ("contig", 6, 128256), ("rows", 6, 4096), ("contig", 7, 1003), ("unaligned", 5, 2000),
            ("contig", 2, 140000)]


@pytest.mark.parametrize("kind,M,V", FB_CASES)
def test_fwd_bwd_matches_oracle(gpu, kind, M, V):
    """kp.cross_entropy_forward_backward (v5/fb5b36393cbd): the register-row
    kernel (V % 8 == 0, V <= 131072, every chunk count 1..16) and the
    two-pass fallback (ragged V, unaligned views, V > 131072) against the
    fp64 oracle: at most 1 bf16 ulp (fp32 exponentials), >= 99.9% exact;
    and the forward outputs as cross_entropy_loss gives them."""
    print(f"[xent fwd+bwd] {kind} [{M},{V}]", flush=True)
    g = torch.Generator().manual_seed(M * 19 + V)
    x, t = _logits(M, V, g, gpu, kind), _targets(M, V, g, gpu)
    gl = 1 / 8192
    out, loss, tw = kp.cross_entropy_forward_backward(x, t, gl, scale=gl, return_loss=True)
    eo, bad = oracle.cross_entropy_fwd_bwd(to_u16(x), t.cpu().numpy(), gl)
    assert bad == 0 and out.shape == x.shape and out.is_contiguous()
    u = ulp_bf16(to_u16(out), eo)
    assert u.max() <= 1 and (u == 0).mean() > 0.999
    eloss, etw, _, _ = oracle.cross_entropy_fwd(to_u16(x), t.cpu().numpy(), scale=gl)
    assert float(tw) == etw
    assert float(loss) == pytest.approx(eloss, rel=LOSS_RTOL)
    assert torch.equal(kp.cross_entropy_forward_backward(x, t, gl), out)  # without the forward outputs


@pytest.mark.parametrize("M,V", [(5, 128256), (9, 16384), (1, 8)])
def test_fwd_bwd_int32_targets(gpu, M, V):
    """int32 targets in the register-row kernel: the last row's id is the
    array's last 4 bytes (its would-be high word lies past the end), ignored
    rows carry -100 as int32.  Same bits as with the same ids as int64."""
    print(f"[xent fwd+bwd int32] [{M},{V}]", flush=True)
    g = torch.Generator().manual_seed(M * 23 + V)
    x = _logits(M, V, g, gpu, "contig")
    t64 = _targets(M, V, g, gpu)
    gl = 1 / 8192
    o64, l64, w64 = kp.cross_entropy_forward_backward(x, t64, gl, scale=gl, return_loss=True)
    o32, l32, w32 = kp.cross_entropy_forward_backward(x, t64.to(torch.int32), gl, scale=gl, return_loss=True)
    assert torch.equal(o32, o64) and float(l32) == float(l64) and float(w32) == float(w64)
    eo, bad = oracle.cross_entropy_fwd_bwd(to_u16(x), t64.cpu().numpy(), gl)
    assert bad == 0 and ulp_bf16(to_u16(o32), eo).max() <= 1


def test_fwd_bwd_special_rows(gpu):
    """Confident rows (a dominant target logit: the target gradient g (p - 1)
    cancels), masked vocabulary, large logits, ramps; out-of-range targets
    zero their row and raise with index checking on."""
    V = 4096
    x = torch.randn(8, V, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    x[0, 100:3000] = float("-inf")
    x[1, :] = float("-inf")
    x[1, 7] = 0.5
    x[2, 2047] = 1000.0
    x[3, ::97] = 30000.0
    x[4] = torch.linspace(-60, 60, V).to(torch.bfloat16)
    x[5, 11] = 40.0
    x[7] = -1e4
    t = torch.tensor([5, 7, 2047, 0, V - 1, 11, -100, 3])
    xd, td = x.to(gpu), t.to(gpu)
    gl = 0.25
    out = kp.cross_entropy_forward_backward(xd, td, gl)
    eo, _ = oracle.cross_entropy_fwd_bwd(to_u16(x), t.numpy(), gl)
    # exact rounding of the fp64 gradient; near-cancellation at confident
    # targets leaves an fp32 absolute error of a few 2^-24 g
    d = np.abs(from_u16(to_u16(out)).double().numpy() - from_u16(eo).double().numpy())
    ulp = ulp_bf16(to_u16(out), eo)
    assert ((ulp <= 1) | (d <= 8 * 2.0**-24 * gl)).all()
    assert not out[6].any()
    with pytest.raises(IndexError):
        kp.cross_entropy_forward_backward(xd, torch.tensor([1, V, -100, 0, 0, 0, 0, 0], device=gpu), gl)


def test_fwd_bwd_in_place_and_eager(gpu):
    """At the fragment's full shape: within 1 ulp of torch-ROCm eager's fp32
    region for >= 99.9% of entries and the stated tolerance for all; in
    place (gradient over the logits) gives the same bits."""
    M, V = 8192, 128256
    print(f"[xent fwd+bwd eager] [{M},{V}]", flush=True)
    g = torch.Generator(device=gpu).manual_seed(9)
    x = torch.randn(M, V, device=gpu, generator=g).to(torch.bfloat16)
    t = torch.randint(0, V, (M,), device=gpu, generator=g)
    t[::7] = -100
    gl = 1 / 8192
    from oracle import torch_ref
    ref = torch_ref.cross_entropy_fwd_bwd(x, t, gl)
    out = kp.cross_entropy_forward_backward(x, t, gl)
    close = (out.float() - ref.float()).abs() <= 1e-2 + 1.6e-2 * ref.float().abs()
    assert bool(close.all())
    same = (out.view(torch.int16) == ref.view(torch.int16)).float().mean()
    assert float(same) > 0.999
    del ref
    xi = x.clone()
    r = kp.cross_entropy_forward_backward(xi, t, gl, in_place=True)
    assert r.data_ptr() == xi.data_ptr() and torch.equal(xi, out)
