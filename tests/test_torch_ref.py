"""The torch eager restatements (oracle/torch_ref.py: the CPU baseline that
bench.py times, and the on-GPU eager comparison) agree with the C oracle on
the CPU."""
import numpy as np
import torch

import oracle
from oracle import torch_ref
from tests._util import bf, gen, randn_bf16, to_u16, ulp_bf16


def _close_ulp(a, b, max_ulp=1, min_exact=0.98):
    u = ulp_bf16(a, b)
    assert u.max() <= max_ulp and (u == 0).mean() >= min_exact, (u.max(), (u == 0).mean())


def test_rms_norm_fwd_and_bwd():
    g = gen(1)
    M, N = 32, 512
    x, dy = randn_bf16((M, N), g), randn_bf16((M, N), g)
    w = randn_bf16((N,), g, mean=1.0, std=0.02)
    y, r = torch_ref.rms_norm_fwd(x, w, 1e-6)
    _, yo, ro = oracle.rmsnorm_fwd([to_u16(x)], to_u16(w), 1e-6, N)
    _close_ulp(to_u16(y), yo)
    dx, dw = torch_ref.rms_norm_bwd(x, dy, w, 1e-6)
    dxo, dwo, _ = oracle.rmsnorm_bwd([to_u16(dy)], [to_u16(x)], None, to_u16(w), 1e-6, N)
    _close_ulp(to_u16(dx), dxo, max_ulp=2, min_exact=0.9)
    assert dw.dtype == torch.float32
    # the eager dw is rounded to bf16 (then widened): within one bf16 ulp of the fp64 sum
    assert np.all(np.abs(dw.double().numpy() - dwo) <= 2.0**-8 * np.abs(dwo) + 1e-6)


def test_add_rms_norm_fwd_and_bwd():
    g = gen(2)
    M, N = 16, 256
    x, res, dy = (randn_bf16((M, N), g) for _ in range(3))
    w = randn_bf16((N,), g, mean=1.0, std=0.02)
    h, y = torch_ref.add_rms_norm_fwd(x, res, w, 1e-5)
    ho, yo, _ = oracle.rmsnorm_fwd([to_u16(res), to_u16(x)], to_u16(w), 1e-5, N)
    assert np.array_equal(to_u16(h), ho)
    _close_ulp(to_u16(y), yo)
    dx, dw = torch_ref.add_rms_norm_bwd(x, res, dy, w, 1e-5)
    dxo, dwo, _ = oracle.rmsnorm_bwd([to_u16(dy)], [to_u16(res), to_u16(x)], None, to_u16(w), 1e-5, N)
    _close_ulp(to_u16(dx), dxo, max_ulp=2, min_exact=0.9)
    assert np.all(np.abs(dw.double().numpy() - dwo) <= 2.0**-8 * np.abs(dwo) + 1e-6)


def test_embedding_fwd_and_bwd():
    g = gen(3)
    V, D, T = 200, 32, 500
    table, grad = randn_bf16((V, D), g), randn_bf16((T, D), g)
    ids = torch.randint(0, V, (T,), generator=g)
    out = torch_ref.embedding_fwd(table, ids)
    assert np.array_equal(to_u16(out), oracle.embedding_fwd(to_u16(table), ids.numpy())[0])
    gw = torch_ref.embedding_bwd(grad, ids, V)
    rid, rows, absrows, counts, _ = oracle.embedding_bwd_rows(to_u16(grad), ids.numpy(), V)
    assert gw.dtype == torch.float32
    got = gw.double().numpy()
    assert not np.delete(got, rid, axis=0).any()
    # CPU eager accumulates in bf16: each of the count - 1 adds rounds once,
    # so the error is at most count * 2^-8 * sum |g| over the row's tokens
    assert np.all(np.abs(got[rid] - rows) <= counts[:, None] * 2.0**-8 * absrows + 1e-6)


def test_rope_half_and_complex():
    g = gen(4)
    B, S, Hq, Hk, D = 2, 64, 4, 2, 128
    q, k = randn_bf16((B, S, Hq, D), g), randn_bf16((B, S, Hk, D), g)
    pos = torch.arange(S).expand(B, S).contiguous()
    qo, ko = torch_ref.rope_half(q, k, pos, 500000.0)
    for t, o in ((q, qo), (k, ko)):
        e = oracle.rope(to_u16(t), pos.numpy(), pairing="half", theta=500000.0)
        u = ulp_bf16(to_u16(o), e)
        far = (u > 1) & (np.abs(bf(to_u16(o)) - bf(e)) > 1e-5)
        assert not far.any()
    freqs = torch.polar(torch.ones(S, D // 2), torch.rand(S, D // 2, generator=g) * 6.28)
    xo = torch_ref.rope_complex(q[:1], freqs[None, :, None, :])
    e = oracle.rope(to_u16(q[:1]), None, pairing="interleaved", freqs=freqs.numpy())
    u = ulp_bf16(to_u16(xo), e)
    assert not ((u > 1) & (np.abs(bf(to_u16(xo)) - bf(e)) > 4e-6)).any()


def test_swiglu_fwd_and_bwd():
    g = gen(9)
    a, b, gr, s = (randn_bf16((16, 700), g, std=3.0) for _ in range(4))
    _close_ulp(to_u16(torch_ref.swiglu_fwd(a, b)), oracle.swiglu_fwd(to_u16(a), to_u16(b)), min_exact=0.99)
    db, da = torch_ref.swiglu_bwd(gr, s, b, a)
    edb, eda = oracle.swiglu_bwd(to_u16(gr), to_u16(s), to_u16(b), to_u16(a))
    assert np.array_equal(to_u16(db), edb)
    u = ulp_bf16(to_u16(da), eda)
    assert (u == 0).mean() > 0.99


def test_cross_entropy_fwd_and_bwd():
    g = gen(10)
    M, V = 12, 5000
    x = randn_bf16((M, V), g, std=2.0)
    t = torch.randint(0, V, (M,), generator=g)
    t[3] = -100
    loss, tw = torch_ref.cross_entropy_fwd(x, t, 1 / 8192)
    lo, two, _, _ = oracle.cross_entropy_fwd(to_u16(x), t.numpy(), scale=1 / 8192)
    assert float(tw) == two and abs(float(loss) - lo) <= 1e-5 * abs(lo)
    L = torch.log_softmax(x.float(), 1)
    out = torch_ref.cross_entropy_bwd(L, t, 1 / 8192)
    eo, _ = oracle.cross_entropy_bwd(L.numpy(), t.numpy(), 1 / 8192)
    _close_ulp(to_u16(out), eo, min_exact=0.99)
    # the whole region from the logits (v5/fb5b36393cbd)
    fb = torch_ref.cross_entropy_fwd_bwd(x, t, 1 / 8192)
    efb, _ = oracle.cross_entropy_fwd_bwd(to_u16(x), t.numpy(), 1 / 8192)
    _close_ulp(to_u16(fb), efb, min_exact=0.99)
