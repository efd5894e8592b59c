"""Pins the oracle's cross-entropy (v8/71f1d2c9f38b forward, v8/622c35f5d1c6
backward): against torch's log_softmax / nll_loss and their backward ops in
fp64 (library routines), against the autograd of the forward, and against
closed forms (uniform rows, a dominant logit, shift invariance, ignored rows,
rows of a true log-softmax summing to zero).  A wrong sign, a dropped
max-shift, counting ignored rows or forgetting the target term fails one."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import bf, bf16_round_exact, gen, randn_bf16, to_u16, ulp_bf16

aten = torch.ops.aten


def _targets(M, V, g, ignore_every=5):
    t = torch.randint(0, V, (M,), generator=g)
    t[::ignore_every] = -100
    return t


@pytest.mark.parametrize("M,V,std", [(7, 1000, 1.0), (16, 4099, 4.0), (3, 128256, 2.0)])
def test_fwd_matches_torch_fp64(M, V, std):
    g = gen(M + V)
    x, t = randn_bf16((M, V), g, std=std), _targets(M, V, g)
    loss, tw, lse, bad = oracle.cross_entropy_fwd(to_u16(x), t.numpy(), scale=1 / 8192)
    lsm = aten._log_softmax(x.double(), 1, False)
    ref, ref_tw = aten.nll_loss_forward(lsm, t, None, 2, -100)
    assert bad == 0
    assert tw == float(ref_tw) == float((t != -100).sum())
    assert loss == pytest.approx(float(ref) / 8192, rel=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(x.double(), 1).numpy(), rtol=1e-13)


def test_fwd_closed_forms():
    V = 4096
    # uniform row: lse = c + log V, loss = log V per counted row
    x = torch.full((3, V), 1.5).to(torch.bfloat16)
    t = torch.tensor([0, -100, V - 1])
    loss, tw, lse, _ = oracle.cross_entropy_fwd(to_u16(x), t.numpy())
    assert tw == 2 and loss == pytest.approx(2 * np.log(V), rel=1e-14)
    np.testing.assert_allclose(lse, 1.5 + np.log(V), rtol=1e-14)
    # a dominant target logit: loss 0 (e^-10000 underflows to exactly 0)
    y = torch.full((1, V), -1e4).to(torch.bfloat16)
    y[0, 17] = 0
    loss, _, lse, _ = oracle.cross_entropy_fwd(to_u16(y), np.array([17]))
    assert loss == 0.0 and lse[0] == 0.0
    # ... and the same row with another target: loss = x_17 - x_t = 1e4 (bf16 of it)
    loss, _, _, _ = oracle.cross_entropy_fwd(to_u16(y), np.array([3]))
    assert loss == -float(bf(to_u16(y))[0, 3])


def test_fwd_shift_invariance_and_ignored_rows():
    g = gen(3)
    V = 2000
    # values k/8 in [-8, 8): +16 stays exact in bf16 (8 significant bits)
    k = torch.randint(-64, 64, (5, V), generator=g).double() / 8
    x, xs = k.to(torch.bfloat16), (k + 16).to(torch.bfloat16)
    assert torch.equal(xs.double(), k + 16)
    t = torch.tensor([3, -100, 1999, 0, -100])
    a = oracle.cross_entropy_fwd(to_u16(x), t.numpy())
    b = oracle.cross_entropy_fwd(to_u16(xs), t.numpy())
    assert a[0] == pytest.approx(b[0], rel=1e-13) and a[1] == b[1] == 3
    # an ignored row's logits do not matter
    x2 = x.clone()
    x2[1] = 100
    assert oracle.cross_entropy_fwd(to_u16(x2), t.numpy())[0] == a[0]
    # out-of-range targets are reported and not counted
    _, tw, _, bad = oracle.cross_entropy_fwd(to_u16(x), np.array([3, -100, V, -1, 0]))
    assert bad == 2 and tw == 2


@pytest.mark.parametrize("true_lsm", [True, False])
def test_bwd_matches_torch_fp64(true_lsm):
    g = gen(5 + true_lsm)
    M, V, gl = 9, 3001, 1.0 / 8192
    x = torch.randn(M, V, generator=g) * 3
    L = torch.log_softmax(x, 1) if true_lsm else torch.randn(M, V, generator=g)  # the fragment's inputs are randn
    t = _targets(M, V, g, ignore_every=4)
    out, bad = oracle.cross_entropy_bwd(L.numpy(), t.numpy(), gl)
    gi = aten.nll_loss_backward(torch.tensor(gl, dtype=torch.float64), L.double(), t, None, 2, -100,
                                torch.tensor(float((t != -100).sum()), dtype=torch.float64))
    ref = aten._log_softmax_backward_data(gi, L.double(), 1, torch.float64)
    assert bad == 0
    assert np.array_equal(out, bf16_round_exact(ref.numpy()).reshape(M, V))
    assert not bf(out)[(t == -100).numpy()].any()  # ignored rows are zero


def test_bwd_is_the_gradient_of_the_forward():
    """With L = log_softmax(x) and g = scale, the backward equals the fp64
    autograd gradient of the forward loss (scale * sum of nll)."""
    g = gen(7)
    M, V, scale = 6, 513, 0.25
    x = randn_bf16((M, V), g, std=2.0).double().requires_grad_(True)
    t = _targets(M, V, g, ignore_every=3)
    loss = torch.nn.functional.nll_loss(torch.log_softmax(x, 1), t, reduction="sum", ignore_index=-100) * scale
    loss.backward()
    L = torch.log_softmax(x.detach(), 1).float()
    out, _ = oracle.cross_entropy_bwd(L.numpy(), t.numpy(), scale)
    # L is rounded to fp32 first: exp(L) carries a relative error <= 2^-24 |L|
    diff = np.abs(bf(out) - x.grad.numpy())
    assert np.all(diff <= 2.0**-8 * np.abs(x.grad.numpy()) + 2.0**-22 * scale)
    # rows of a true log-softmax sum to ~0; the target column is scale * (p_t - 1) < 0
    rows = bf(out).sum(1)
    assert np.all(np.abs(rows) <= 2.0**-8 * scale * 2)
    valid = (t != -100).numpy()
    assert np.all(bf(out)[np.arange(M)[valid], t.numpy()[valid]] < 0)


def test_bwd_out_of_range_rows():
    L = np.zeros((3, 10), np.float32)
    out, bad = oracle.cross_entropy_bwd(L, np.array([10, -100, 2]), 0.5)
    assert bad == 1
    assert not bf(out)[:2].any()
    # exp(0) = 1: row 2 is 0.5 everywhere except 0.5 - 0.5 = 0 at the target
    assert np.array_equal(bf(out)[2], np.where(np.arange(10) == 2, 0.0, 0.5))


@pytest.mark.parametrize("M,V,std", [(6, 513, 2.0), (4, 4099, 5.0)])
def test_fwd_bwd_is_the_fp64_autograd_gradient(M, V, std):
    """cross_entropy_fwd_bwd (v5/fb5b36393cbd) is the fp64 autograd gradient
    of scale * sum(nll(log_softmax(x))) with one bf16 rounding: bit-equal."""
    g = gen(M * 31 + V)
    x = randn_bf16((M, V), g, std=std)
    t = _targets(M, V, g, ignore_every=3)
    scale = 1.0 / 8192
    xd = x.double().requires_grad_(True)
    loss = torch.nn.functional.nll_loss(torch.log_softmax(xd, 1), t, reduction="sum", ignore_index=-100) * scale
    loss.backward()
    out, bad = oracle.cross_entropy_fwd_bwd(to_u16(x), t.numpy(), scale)
    assert bad == 0
    assert np.array_equal(out, bf16_round_exact(xd.grad.numpy()).reshape(M, V))
    assert not bf(out)[(t == -100).numpy()].any()


def test_fwd_bwd_agrees_with_the_two_step_path():
    """The same gradient as cross_entropy_bwd fed the log-softmax (rounded to
    fp32, as the two-step graph stores it): within one bf16 ulp; and an
    out-of-range target is counted and its row zeroed."""
    g = gen(9)
    M, V = 5, 3000
    x = randn_bf16((M, V), g, std=3.0)
    t = torch.tensor([7, -100, V, 2999, 0])
    out, bad = oracle.cross_entropy_fwd_bwd(to_u16(x), t.numpy(), 0.5)
    L = torch.log_softmax(x.double(), 1).float().numpy()
    ref, bad2 = oracle.cross_entropy_bwd(L, t.numpy(), 0.5)
    assert bad == bad2 == 1
    assert (ulp_bf16(out, ref) <= 1).all()
    assert not bf(out)[[1, 2]].any()
