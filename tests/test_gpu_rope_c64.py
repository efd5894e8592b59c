"""GPU parity of the complex64 RoPE kernel (kp_rope_c64: the v1 captures
v1/075cb40f3d5d, v1/9cd8f72e74ce, v1/d7efc428b2f5) with the complex128 CPU
oracle -- 16-byte path (contiguous and head-strided views) and 8-byte path
(odd P, views starting one complex value in), gathered and per-position
tables, the conjugate table, out-of-range positions -- and with torch-ROCm's
complex multiply at the fragments' full shape."""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
import oracle

pytestmark = pytest.mark.gpu


def _check(out, exact, x, t_rows):
    """Each fp32 component within 2^-22 (|ac| + |bd|) of the complex128 product."""
    o = out.cpu().numpy().astype(np.complex128)
    bound = 2.0**-22 * (np.abs(x.real * t_rows.real) + np.abs(x.imag * t_rows.imag) +
                        np.abs(x.real * t_rows.imag) + np.abs(x.imag * t_rows.real)) + 1e-30
    assert np.all(np.abs(o.real - exact.real) <= bound) and np.all(np.abs(o.imag - exact.imag) <= bound)


def _c64(shape, g):
    return torch.randn(shape, dtype=torch.complex64, generator=g)


@pytest.mark.parametrize("kind", ["contig", "heads_strided", "odd_p", "offset"])
@pytest.mark.parametrize("gather", [False, True])
@pytest.mark.parametrize("conj", [False, True])
def test_matches_oracle(gpu, kind, gather, conj):
    print(f"[rope c64] {kind} gather={gather} conj={conj}", flush=True)
    g = torch.Generator().manual_seed(7)
    B, S, Hq, Hk = 2, 37, 5, 3
    P = 63 if kind == "odd_p" else 64
    rows = 50
    if kind == "heads_strided":       # [B, S, H, P] views of [B, S, H + 2, P]
        q = _c64((B, S, Hq + 2, P), g).to(gpu)[:, :, 1:1 + Hq]
        k = _c64((B, S, Hk + 2, P), g).to(gpu)[:, :, :Hk]
    elif kind == "offset":            # starts one complex value in: the 8-byte path
        q = _c64((B, S, Hq, P + 1), g).to(gpu)[..., 1:]
        k = _c64((B, S, Hk, P + 1), g).to(gpu)[..., 1:]
    else:
        q, k = _c64((B, S, Hq, P), g).to(gpu), _c64((B, S, Hk, P), g).to(gpu)
    table = _c64((rows, P), g).to(gpu)
    pos = torch.randint(0, rows, (B, S), generator=g) if gather else None
    qo, ko = kp.rope_complex(q, k, freqs_cis=table, positions=None if pos is None else pos.to(gpu), conj=conj)
    tn = table.cpu().numpy()
    pn = None if pos is None else pos.numpy()
    for x, o in ((q, qo), (k, ko)):
        xn = x.cpu().numpy()
        exact = oracle.rope_c64(xn, tn, pn, conj=conj)
        p_ = np.broadcast_to(np.arange(S), (B, S)) if pn is None else pn
        rows_ = tn[p_][:, :, None, :]
        _check(o, exact, xn.astype(np.complex128), (np.conj(rows_) if conj else rows_).astype(np.complex128))


def test_out_of_range_positions_and_empty(gpu):
    q = torch.randn(1, 4, 2, 8, dtype=torch.complex64, device=gpu)
    t = torch.randn(3, 8, dtype=torch.complex64, device=gpu)
    pos = torch.tensor([[0, 3, 1, -1]], device=gpu)
    with pytest.raises(IndexError):
        kp.rope_complex(q, freqs_cis=t, positions=pos)
    kp.set_index_checking(False)
    try:
        qo, _ = kp.rope_complex(q, freqs_cis=t, positions=pos)
    finally:
        kp.set_index_checking(True)
    assert not qo[0, 1].any() and not qo[0, 3].any()
    exact = oracle.rope_c64(q[:, [0, 2]].cpu().numpy(), t.cpu().numpy(), np.array([[0, 1]]))
    assert np.allclose(qo[:, [0, 2]].cpu().numpy(), exact, rtol=1e-6, atol=1e-6)
    e = torch.empty((0, 4, 2, 8), dtype=torch.complex64, device=gpu)
    assert kp.rope_complex(e, freqs_cis=t)[0].shape == e.shape


def test_full_shape_against_torch(gpu):
    """v1/075cb40f3d5d at its shape: q [1, 8192, 32, 64], k [1, 8192, 8, 64]
    against torch-ROCm's complex64 multiply of the gathered rows."""
    print("[rope c64 eager] full shape", flush=True)
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randn(1, 8192, 32, 64, dtype=torch.complex64, device=gpu, generator=g)
    k = torch.randn(1, 8192, 8, 64, dtype=torch.complex64, device=gpu, generator=g)
    t = torch.randn(8192, 64, dtype=torch.complex64, device=gpu, generator=g)
    pos = torch.randint(0, 100, (1, 8192), dtype=torch.int32, device=gpu, generator=g)
    qo, ko = kp.rope_complex(q, k, freqs_cis=t, positions=pos)
    rows = t[pos[0].long()].view(1, 8192, 1, 64)
    for o, ref in ((qo, q * rows), (ko, k * rows)):
        d = torch.view_as_real(o) - torch.view_as_real(ref)
        assert float(d.abs().max()) <= 1e-5 * float(torch.view_as_real(ref).abs().max())


@pytest.mark.parametrize("gather", [False, True])
@pytest.mark.parametrize("conj", [False, True])
@pytest.mark.parametrize("B,S,Hq,Hk,P", [(2, 37, 4, 2, 64), (3, 11, 8, 16, 48)])
def test_tile_path_matches_position_path(gpu, gather, conj, B, S, Hq, Hk, P):
    """Contiguous tensors with H * P / 2 a multiple of 64 take the tile
    kernel (e.g. 2 * 37 * 128 and 2 * 37 * 64 chunks: both end in a partial
    512-chunk tile; with P = 48 a head is 24 chunks, so a wave's 64 chunks
    straddle heads and a chunk's place in its head is a division by 24); the
    same values read through a head-strided view take the one-wave-per-
    position kernel.  Identical bits, and the oracle's bound."""
    print(f"[rope c64 tile] gather={gather} conj={conj} B={B} S={S} H={Hq},{Hk} P={P}", flush=True)
    g = torch.Generator().manual_seed(11 + P)
    rows = 50
    q, k = _c64((B, S, Hq, P), g).to(gpu), _c64((B, S, Hk, P), g).to(gpu)
    table = _c64((rows, P), g).to(gpu)
    pos = (torch.randint(0, rows, (B, S), generator=g) if gather else None)
    kw = dict(freqs_cis=table, positions=None if pos is None else pos.to(gpu), conj=conj)
    qo, ko = kp.rope_complex(q, k, **kw)
    qw = torch.zeros((B, S, Hq + 1, P), dtype=torch.complex64, device=gpu)
    kw_ = torch.zeros((B, S, Hk + 1, P), dtype=torch.complex64, device=gpu)
    qw[:, :, :Hq] = q
    kw_[:, :, :Hk] = k
    qf, kf = kp.rope_complex(qw[:, :, :Hq], kw_[:, :, :Hk], **kw)
    torch.cuda.synchronize()
    assert torch.equal(qo.view(torch.float32), qf.view(torch.float32))
    assert torch.equal(ko.view(torch.float32), kf.view(torch.float32))
    tn = table.cpu().numpy()
    pn = None if pos is None else pos.numpy()
    for x, o in ((q, qo), (k, ko)):
        xn = x.cpu().numpy()
        exact = oracle.rope_c64(xn, tn, pn, conj=conj)
        p_ = np.broadcast_to(np.arange(S), (B, S)) if pn is None else pn
        rows_ = tn[p_][:, :, None, :]
        _check(o, exact, xn.astype(np.complex128), (np.conj(rows_) if conj else rows_).astype(np.complex128))


def test_tile_path_out_of_range_positions(gpu):
    """The tile kernel (H * P / 2 = 64) on ids outside the table: flagged,
    their rows zero, the others right."""
    q = torch.randn(1, 4, 2, 64, dtype=torch.complex64, device=gpu)
    t = torch.randn(3, 64, dtype=torch.complex64, device=gpu)
    pos = torch.tensor([[0, 3, 1, -1]], device=gpu)
    with pytest.raises(IndexError):
        kp.rope_complex(q, freqs_cis=t, positions=pos)
    kp.set_index_checking(False)
    try:
        qo, _ = kp.rope_complex(q, freqs_cis=t, positions=pos)
    finally:
        kp.set_index_checking(True)
    assert not qo[0, 1].any() and not qo[0, 3].any()
    exact = oracle.rope_c64(q[:, [0, 2]].cpu().numpy(), t.cpu().numpy(), np.array([[0, 1]]))
    assert np.allclose(qo[:, [0, 2]].cpu().numpy(), exact, rtol=1e-6, atol=1e-6)
