"""GPU parity: RoPE (rotate-half and interleaved; theta and table angles) vs the C oracle."""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
from tests._util import assert_bf16_close, gen, randn_bf16, to_u16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pairing", ["half", "interleaved"])
@pytest.mark.parametrize("B,S,Hq,Hk,D", [(2, 64, 32, 8, 128), (1, 33, 4, 2, 64), (1, 16, 3, 1, 96)])
@pytest.mark.parametrize("conj", [False, True])
def test_rope_theta_matches_oracle(gpu, oracle_lib, pairing, B, S, Hq, Hk, D, conj):
    g = gen(B * S + Hq + D)
    q = randn_bf16((B, S, Hq, D), g)
    k = randn_bf16((B, S, Hk, D), g)
    pos = (torch.arange(S) * 61 % 4096).repeat(B, 1)  # large angles
    qo, ko = kp.rope(q.to(gpu), k.to(gpu), positions=pos.to(gpu), theta=500000.0, pairing=pairing, conj=conj)
    torch.cuda.synchronize()
    eq = oracle_lib.rope(to_u16(q), pos.numpy(), pairing=pairing, theta=500000.0, conj=conj)
    ek = oracle_lib.rope(to_u16(k), pos.numpy(), pairing=pairing, theta=500000.0, conj=conj)
    # |x| <= ~5: fp32 evaluation error of x_a*c - x_b*s is below 4e-6 absolute
    assert_bf16_close(to_u16(qo), eq, what="q", max_ulp=1, min_exact=0.99, ulp_abs_slack=4e-6)
    assert_bf16_close(to_u16(ko), ek, what="k", max_ulp=1, min_exact=0.99, ulp_abs_slack=4e-6)


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64, None])
def test_rope_table_interleaved(gpu, oracle_lib, idx_dtype):
    """freqs_cis table gathered by position ids (v8/c8c60d8f7015) or by s (v7/e29b92927600)."""
    g = gen(31)
    S, Hq, Hk, D, P = 96, 8, 2, 128, 200
    q = randn_bf16((1, S, Hq, D), g)
    k = randn_bf16((1, S, Hk, D), g)
    freqs = torch.complex(torch.randn(P, D // 2, generator=g), torch.randn(P, D // 2, generator=g))
    pos = torch.randint(0, P, (1, S), generator=g)
    posa = None if idx_dtype is None else pos.to(idx_dtype).to(gpu)
    qo, ko = kp.rope(q.to(gpu), k.to(gpu), positions=posa, freqs_cis=freqs.to(gpu), pairing="interleaved")
    torch.cuda.synchronize()
    pn = None if idx_dtype is None else pos.numpy()
    eq = oracle_lib.rope(to_u16(q), pn, pairing="interleaved", freqs=freqs.numpy())
    ek = oracle_lib.rope(to_u16(k), pn, pairing="interleaved", freqs=freqs.numpy())
    assert_bf16_close(to_u16(qo), eq, what="q", max_ulp=1, min_exact=0.99, ulp_abs_slack=4e-6)
    assert_bf16_close(to_u16(ko), ek, what="k", max_ulp=1, min_exact=0.99, ulp_abs_slack=4e-6)


def test_rope_strided_transposed_input(gpu, oracle_lib):
    """Input given as a transposed view ([B, H, S, D] memory read as [B, S, H, D])."""
    g = gen(32)
    B, S, H, D = 1, 40, 8, 128
    base = randn_bf16((B, H, S, D), g)
    x = base.to(gpu).transpose(1, 2)  # [B, S, H, D] view, strides (H*S*D, D, S*D, 1)
    out, _ = kp.rope(x, theta=10000.0, pairing="half")
    exp = oracle_lib.rope(to_u16(base.transpose(1, 2).contiguous()), None, pairing="half", theta=10000.0)
    assert_bf16_close(to_u16(out), exp, what="transposed", max_ulp=1, min_exact=0.99, ulp_abs_slack=4e-6)


def test_rope_table_vs_torch_complex(gpu):
    """The reference op chain on this GPU: view_as_complex(x.float()) * freqs -> bf16."""
    g = gen(33)
    S, H, D = 128, 8, 128
    x = randn_bf16((1, S, H, D), g).to(gpu)
    freqs = torch.polar(torch.ones(S, D // 2), torch.rand(S, D // 2, generator=g) * 6.28).to(gpu)
    xc = torch.view_as_complex(x.float().view(1, S, H, D // 2, 2))
    ref = torch.view_as_real(xc * freqs.view(1, S, 1, D // 2)).reshape(1, S, H, D).to(torch.bfloat16)
    out, _ = kp.rope(x, freqs_cis=freqs, pairing="interleaved")
    assert_bf16_close(to_u16(out), to_u16(ref), what="vs torch complex", max_ulp=1, ulp_abs_slack=4e-6)


def test_rope_out_of_table_position_flagged(gpu):
    x = torch.ones((1, 4, 1, 8), dtype=torch.bfloat16, device=gpu)
    freqs = torch.ones((3, 4), dtype=torch.complex64, device=gpu)
    with pytest.raises(IndexError):
        kp.rope(x, positions=torch.tensor([0, 1, 2, 3], device=gpu), freqs_cis=freqs, pairing="interleaved")


@pytest.mark.parametrize("vec", [True, False])
def test_rope_fp32_output(gpu, vec):
    """fp32 outputs (v7/0f38bc55457c returns its q rotation unrounded): within
    fp32 evaluation error of the fp64 rotation, and rounding them to bf16
    gives exactly the bf16-output kernel's result."""
    g = gen(77)
    S, Hq, Hk, D, P = 48, 4, 2, 128 if vec else 6, 64
    q = randn_bf16((1, S, Hq, D), g)
    k = randn_bf16((1, S, Hk, D), g)
    freqs = torch.complex(torch.randn(P, D // 2, generator=g), torch.randn(P, D // 2, generator=g))
    pos = torch.randint(0, P, (1, S), generator=g)
    qd, kd, fd, pd = q.to(gpu), k.to(gpu), freqs.to(gpu), pos.to(gpu)
    q32, kb = kp.rope(qd, kd, positions=pd, freqs_cis=fd, pairing="interleaved", q_dtype=torch.float32)
    qb, k32 = kp.rope(qd, kd, positions=pd, freqs_cis=fd, pairing="interleaved", k_dtype=torch.float32)
    torch.cuda.synchronize()
    assert q32.dtype == torch.float32 and kb.dtype == torch.bfloat16
    assert torch.equal(q32.to(torch.bfloat16), qb) and torch.equal(k32.to(torch.bfloat16), kb)
    for x, out in ((q, q32), (k, k32)):
        xc = torch.view_as_complex(x.double().reshape(*x.shape[:-1], D // 2, 2))
        f = freqs.to(torch.complex128)[pos[0]][None, :, None, :]
        exact = torch.view_as_real(xc * f).reshape(x.shape)
        # fp32 a*c - b*d: two rounded products and a rounded difference, each
        # within 2^-24 relative, bounded by 2^-23 (|ac| + |bd|) <= 2^-23 |x||f|
        pair = (2.0**-22 * xc.abs() * f.abs()).unsqueeze(-1).expand(*xc.shape, 2)
        bound = pair.reshape(x.shape)
        assert ((out.cpu().double() - exact).abs() <= bound).all()


@pytest.mark.parametrize("pairing", ["half", "interleaved"])
@pytest.mark.parametrize("table", [False, True])
@pytest.mark.parametrize("conj", [False, True])
@pytest.mark.parametrize("B,S,Hq,Hk", [(1, 33, 4, 8), (3, 19, 12, 20)])
def test_rope_tile_path_matches_position_path(gpu, oracle_lib, pairing, table, conj, B, S, Hq, Hk):
    """Contiguous [B, S, H, 128] tensors with H % 4 == 0 take the tile kernel
    (512-chunk blocks; both tensors end in a partial tile, e.g. 33 * 4 * 16 =
    2112 and 33 * 8 * 16 = 4224 chunks; the second shape has 3 and 5 head
    groups per position and 3 batch rows, so a block's positions and their
    batch rows come from divisions by 3, 5 and 19).  The same data read
    through a view with a wider head stride takes the one-wave-per-position
    kernel: both must give identical bits, and meet the oracle's bar."""
    print(f"[rope tile] {pairing} table={table} conj={conj} B={B} S={S} H={Hq},{Hk}", flush=True)
    g = gen(900 + 4 * table + 2 * conj + (pairing == "half") + 8 * B)
    D, P = 128, 64
    q = randn_bf16((B, S, Hq, D), g)
    k = randn_bf16((B, S, Hk, D), g)
    pos = torch.randint(0, P, (B, S), generator=g) if table else (torch.arange(S) * 97 % 4096).repeat(B, 1)
    kw = dict(positions=pos.to(gpu), pairing=pairing, conj=conj)
    freqs = None
    if table:
        freqs = torch.complex(torch.randn(P, D // 2, generator=g), torch.randn(P, D // 2, generator=g))
        kw["freqs_cis"] = freqs.to(gpu)
    else:
        kw["theta"] = 500000.0
    qo, ko = kp.rope(q.to(gpu), k.to(gpu), **kw)
    # head stride 2 * D: not the tile layout
    qw = torch.zeros((B, S, Hq, 2 * D), dtype=torch.bfloat16, device=gpu)
    kw_ = torch.zeros((B, S, Hk, 2 * D), dtype=torch.bfloat16, device=gpu)
    qw[..., :D] = q.to(gpu)
    kw_[..., :D] = k.to(gpu)
    qf, kf = kp.rope(qw[..., :D], kw_[..., :D], **kw)
    torch.cuda.synchronize()
    assert torch.equal(qo, qf) and torch.equal(ko, kf)
    pn = pos.numpy()
    for x, out in ((q, qo), (k, ko)):
        if table:
            exp = oracle_lib.rope(to_u16(x), pn, pairing=pairing, freqs=freqs.numpy(), conj=conj)
        else:
            exp = oracle_lib.rope(to_u16(x), pn, pairing=pairing, theta=500000.0, conj=conj)
        assert_bf16_close(to_u16(out), exp, what="tile", max_ulp=1, min_exact=0.99, ulp_abs_slack=4e-6)


@pytest.mark.parametrize("table", [False, True])
def test_rope_tile_fp32_output(gpu, table):
    """fp32 outputs (the un-rounded rotation of v7/0f38bc55457c) through the
    tile kernel: identical to the one-wave-per-position kernel's fp32 output
    on a head-strided view of the same data, and rounding it gives the bf16
    result bit for bit."""
    print(f"[rope tile fp32] table={table}", flush=True)
    g = gen(950 + table)
    B, S, Hq, Hk, D, P = 2, 21, 12, 4, 128, 64
    q = randn_bf16((B, S, Hq, D), g).to(gpu)
    k = randn_bf16((B, S, Hk, D), g).to(gpu)
    pos = (torch.randint(0, P, (B, S), generator=g) if table else (torch.arange(S) * 31 % 4096).repeat(B, 1)).to(gpu)
    kw = dict(positions=pos, pairing="half")
    if table:
        kw["freqs_cis"] = torch.complex(torch.randn(P, D // 2, generator=g), torch.randn(P, D // 2, generator=g)).to(gpu)
    else:
        kw["theta"] = 500000.0
    q32, k32 = kp.rope(q, k, q_dtype=torch.float32, k_dtype=torch.float32, **kw)
    qb, kb = kp.rope(q, k, **kw)
    qw = torch.zeros((B, S, Hq, 2 * D), dtype=torch.bfloat16, device=gpu)
    qw[..., :D] = q
    kw_ = torch.zeros((B, S, Hk, 2 * D), dtype=torch.bfloat16, device=gpu)
    kw_[..., :D] = k
    qf, kf = kp.rope(qw[..., :D], kw_[..., :D], q_dtype=torch.float32, k_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    assert torch.equal(q32, qf) and torch.equal(k32, kf)
    assert torch.equal(q32.to(torch.bfloat16), qb) and torch.equal(k32.to(torch.bfloat16), kb)


@pytest.mark.parametrize("pairing", ["interleaved", "half"])
def test_rope_tile_path_out_of_table_position(gpu, pairing):
    """An id outside the table in the tile kernel (rotate-half stages the
    rows through LDS, interleaved reads them per chunk): the flag is raised,
    and with checking off that position's rows are zero while the others
    equal the in-range result."""
    x = torch.ones((1, 6, 4, 128), dtype=torch.bfloat16, device=gpu)
    freqs = torch.complex(torch.rand(3, 64), torch.rand(3, 64)).to(gpu)
    pos = torch.tensor([0, 1, 2, 3, 1, 0], device=gpu)
    with pytest.raises(IndexError):
        kp.rope(x, positions=pos, freqs_cis=freqs, pairing=pairing)
    kp.set_index_checking(False)
    try:
        out, _ = kp.rope(x, positions=pos, freqs_cis=freqs, pairing=pairing)
        ref, _ = kp.rope(x, positions=torch.tensor([0, 1, 2, 0, 1, 0], device=gpu), freqs_cis=freqs, pairing=pairing)
        torch.cuda.synchronize()
        assert torch.count_nonzero(out[0, 3]) == 0
        keep = [0, 1, 2, 4, 5]
        assert torch.equal(out[0, keep], ref[0, keep])
    finally:
        with pytest.raises(IndexError):
            kp.check_indices()
        kp.set_index_checking(True)


@pytest.mark.parametrize("tile", [True, False])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_rope_copies_equal_single_outputs(gpu, tile, out_dtype):
    """kp_rope_bf16_twice (v5/ca76bd89ec38: the pair returned twice): both
    copies hold exactly the bits of one kp_rope_bf16 call, for the tile
    kernel (contiguous [B, S, H, 128]) and for the per-position kernel (a
    head-strided view, one launch per copy); the copies are distinct
    tensors."""
    print(f"[rope copies] tile={tile} dtype={out_dtype}", flush=True)
    g = gen(970 + tile + 2 * (out_dtype == torch.float32))
    B, S, Hq, Hk, D, P = 1, 37, 8, 4, 128, 64
    q = randn_bf16((B, S, Hq, D), g).to(gpu)
    k = randn_bf16((B, S, Hk, D), g).to(gpu)
    if not tile:
        qw = torch.zeros((B, S, Hq, 2 * D), dtype=torch.bfloat16, device=gpu)
        kw_ = torch.zeros((B, S, Hk, 2 * D), dtype=torch.bfloat16, device=gpu)
        qw[..., :D] = q
        kw_[..., :D] = k
        q, k = qw[..., :D], kw_[..., :D]
    pos = torch.randint(0, P, (B, S), generator=g).to(gpu)
    freqs = torch.complex(torch.randn(P, D // 2, generator=g), torch.randn(P, D // 2, generator=g)).to(gpu)
    kw = dict(positions=pos, freqs_cis=freqs, pairing="interleaved", q_dtype=out_dtype, k_dtype=out_dtype)
    qo, ko = kp.rope(q, k, **kw)
    q1, k1, q2, k2 = kp.rope(q, k, copies=True, **kw)
    torch.cuda.synchronize()
    for a in (q1, q2):
        assert torch.equal(a, qo)
    for a in (k1, k2):
        assert torch.equal(a, ko)
    assert q1.data_ptr() != q2.data_ptr() and k1.data_ptr() != k2.data_ptr()
    qs, _, qs2, ks2 = kp.rope(q, None, copies=True, **kw)
    torch.cuda.synchronize()
    assert ks2 is None and torch.equal(qs, qo) and torch.equal(qs2, qo)


def test_native_wrapper_raises_kperror_with_the_library_message(gpu):
    """A status from the C ABI surfaces through the native wrappers as
    KPError carrying the library's message (odd head dim: KP_EINVAL), and
    the tensor checks raise RuntimeError before any launch."""
    print("[native errors]", flush=True)
    x = torch.zeros((1, 4, 2, 7), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(kp.KPError, match="kp_rope_bf16"):
        kp.rope(x, theta=1e4)
    with pytest.raises(RuntimeError, match="q and k must agree"):
        kp.rope(torch.zeros((1, 4, 2, 8), dtype=torch.bfloat16, device=gpu),
                torch.zeros((1, 5, 2, 8), dtype=torch.bfloat16, device=gpu), theta=1e4)
    with pytest.raises(RuntimeError, match="freqs_cis last dim"):
        kp.rope(torch.zeros((1, 4, 2, 8), dtype=torch.bfloat16, device=gpu),
                freqs_cis=torch.zeros((4, 3), dtype=torch.complex64, device=gpu))
    with pytest.raises(RuntimeError, match="rstd has 3 values, expected 4"):
        kp.rms_norm_backward([x.view(4, 14)], [x.view(4, 14)], torch.zeros(3, device=gpu), None, 1e-5, 14, dw=None)
