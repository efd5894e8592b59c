"""GPU parity of the SwiGLU gate kernels (v8/c68dae22972b forward,
v8/385e1beb9bb9 backward) with the CPU oracle on seeded inputs -- the
16-byte streaming path (flat and row-strided, partial tiles) and the scalar
path (ragged rows, unaligned views) -- and bitwise with torch-ROCm eager:
exhaustively over every bf16 gate value for the forward's silu, and at the
fragment's full shape for both directions."""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
import oracle
from kernelproblems_amd import _lib as L
from tests._util import BF16_ATOL, BF16_RTOL, assert_bf16_close, to_u16

pytestmark = pytest.mark.gpu


def _rand(shape, gen, gpu, std=3.0):
    return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16).to(gpu)


def _views(kind, M, N, gen, gpu, count):
    """count bf16 [M, N] operands laid out as `kind`."""
    if kind == "contig":
        return [_rand((M, N), gen, gpu) for _ in range(count)]
    if kind == "rows":      # row stride N + 24 (16-byte granular): vector path, one block row per row
        return [_rand((M, N + 24), gen, gpu)[:, 8:8 + N] for _ in range(count)]
    if kind == "unaligned":  # starts 3 elements into a row: scalar path
        return [_rand((M, N + 5), gen, gpu)[:, 3:3 + N] for _ in range(count)]
    raise ValueError(kind)


CASES = [
    ("contig", 1, 8), ("contig", 3, 40), ("contig", 64, 4096), ("contig", 7, 8200),
    ("contig", 5, 43), ("contig", 1, 100003),
    ("rows", 9, 12000), ("rows", 33, 1024 * 8), ("unaligned", 6, 1000),
]


@pytest.mark.parametrize("kind,M,N", CASES)
def test_fwd_matches_oracle(gpu, kind, M, N):
    print(f"[swiglu fwd] {kind} [{M},{N}]", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N)
    a, b = _views(kind, M, N, g, gpu, 2)
    out = kp.swiglu(a, b)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and out.is_contiguous()
    exp = oracle.swiglu_fwd(to_u16(a), to_u16(b))
    # the oracle rounds the exact silu once; fp32 expf/divide can sit on the
    # other side of a bf16 rounding boundary (1 ulp, rare)
    assert_bf16_close(to_u16(out), exp, what="swiglu fwd", max_ulp=1, min_exact=0.999)


@pytest.mark.parametrize("kind,M,N", CASES)
def test_bwd_matches_oracle(gpu, kind, M, N):
    print(f"[swiglu bwd] {kind} [{M},{N}]", flush=True)
    g = torch.Generator().manual_seed(M * 11 + N)
    gr, s, b, a = _views(kind, M, N, g, gpu, 4)
    db, da = kp.swiglu_backward(gr, s, b, a)
    torch.cuda.synchronize()
    edb, eda = oracle.swiglu_bwd(to_u16(gr), to_u16(s), to_u16(b), to_u16(a))
    assert np.array_equal(to_u16(db), edb)  # one exact product, one rounding
    # near silu's stationary point the fp32 cancellation in 1 + a (1 - sig)
    # leaves ~|t| 2^-23 absolute error on a tiny result
    t = np.abs((gr.float() * b.float()).cpu().numpy())
    assert_bf16_close(to_u16(da), eda, what="swiglu bwd da", max_ulp=1, min_exact=0.999,
                      ulp_abs_slack=float(t.max()) * 2.0**-21)


@pytest.mark.parametrize("path", ["vector", "scalar"])
def test_fwd_every_bf16_gate_value_bitwise(gpu, path):
    """The forward's silu is a function of one bf16 value, so comparing all
    65536 bit patterns with torch's eager silu proves the fast evaluation
    plus rounding test bit-identical for every input (b = 1 leaves
    bf16(silu(a)) itself; a random b then checks the product)."""
    a = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).to(gpu).view(64, 1024)
    if path == "scalar":  # a view 2 elements into each row: not 16-byte granular
        base = torch.empty((64, 1026), dtype=torch.bfloat16, device=gpu)
        base[:, 2:] = a
        a = base[:, 2:]
    ref = torch.nn.functional.silu(a)
    for b in (torch.ones_like(a), torch.randn(a.shape, device=gpu, generator=torch.Generator(device=gpu).manual_seed(4)
                                               ).to(torch.bfloat16)):
        out = kp.swiglu(a, b)
        exp = ref * b
        same = (out.view(torch.int16) == exp.contiguous().view(torch.int16)) | (torch.isnan(out) & torch.isnan(exp))
        bad = (~same).flatten().nonzero().flatten().tolist()
        assert not bad, f"{len(bad)} gate values differ, e.g. a={a.flatten()[bad[:5]].tolist()}"


def test_empty_and_shapes(gpu):
    e = torch.empty((0, 64), dtype=torch.bfloat16, device=gpu)
    assert kp.swiglu(e, e).shape == (0, 64)
    db, da = kp.swiglu_backward(e, e, e, e)
    assert db.shape == da.shape == (0, 64)
    a = torch.randn(2, 3, 16, dtype=torch.bfloat16, device=gpu)
    assert kp.swiglu(a, a).shape == (2, 3, 16)
    with pytest.raises(RuntimeError):
        kp.swiglu(a, a[..., :8])
    with pytest.raises(RuntimeError):
        kp.swiglu(a.float(), a.float())


def test_fwd_in_place_through_the_abi(gpu):
    """out may be the a operand itself (each element is read before it is written)."""
    g = torch.Generator().manual_seed(3)
    a, b = _rand((64, 4096), g, gpu), _rand((64, 4096), g, gpu)
    ref = kp.swiglu(a, b)
    L.call("kp_swiglu_fwd_bf16", a.data_ptr(), 4096, b.data_ptr(), 4096, a.data_ptr(), 4096, 64, 4096,
           torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(a, ref)


@pytest.mark.parametrize("shape", [(8192, 14336), (3, 1000, 77)])
def test_bitwise_with_torch_eager(gpu, shape):
    """The backward evaluates torch-ROCm's silu_backward formula in the same
    fp32 operations (expf, IEEE division, operation order, bf16 rounding
    points); the forward's silu is bit-identical by the exhaustive test
    above.  So both agree with eager bit for bit."""
    print(f"[swiglu eager] {shape}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(21)
    a, b, gr, s = (torch.randn(shape, dtype=torch.bfloat16, device=gpu, generator=g) * 3 for _ in range(4))
    out = kp.swiglu(a, b)
    assert torch.equal(out, torch.nn.functional.silu(a) * b)
    db, da = kp.swiglu_backward(gr, s, b, a)
    assert torch.equal(db, gr * s)
    assert torch.equal(da, torch.ops.aten.silu_backward(gr * b, a))
    del out, db, da
    # and within the stated tolerance of the fp64 oracle on a slice
    sl = (slice(0, 2),) + (slice(None),) * (len(shape) - 1)
    exp = oracle.swiglu_fwd(to_u16(a[sl]), to_u16(b[sl]))
    assert_bf16_close(to_u16(kp.swiglu(a[sl], b[sl])), exp, rtol=BF16_RTOL, atol=BF16_ATOL, what="slice")


@pytest.mark.parametrize("path", ["vector", "scalar"])
def test_silu_every_bf16_value_bitwise(gpu, path):
    """kp.silu (v7/58e7a4d6cde3) over all 65536 bf16 patterns against torch's
    eager silu, bit for bit (NaN payloads aside)."""
    a = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).to(gpu).view(64, 1024)
    if path == "scalar":
        base = torch.empty((64, 1026), dtype=torch.bfloat16, device=gpu)
        base[:, 2:] = a
        a = base[:, 2:]
    out = kp.silu(a)
    ref = torch.nn.functional.silu(a).contiguous()
    same = (out.view(torch.int16) == ref.view(torch.int16)) | (torch.isnan(out) & torch.isnan(ref))
    bad = (~same).flatten().nonzero().flatten().tolist()
    assert not bad, f"{len(bad)} values differ, e.g. a={a.flatten()[bad[:5]].tolist()}"


@pytest.mark.parametrize("kind,M,N", CASES)
def test_fwd_bwd_matches_oracle(gpu, kind, M, N):
    """kp.swiglu_forward_backward (v6/182d2dcd0652) against the oracle's
    composition of the restated forward and backward."""
    print(f"[swiglu fwd+bwd] {kind} [{M},{N}]", flush=True)
    g = torch.Generator().manual_seed(M * 13 + N)
    a, b, gr = _views(kind, M, N, g, gpu, 3)
    h, db, da = kp.swiglu_forward_backward(a, b, gr)
    torch.cuda.synchronize()
    eh, edb, eda = oracle.swiglu_fwd_bwd(to_u16(a), to_u16(b), to_u16(gr))
    assert_bf16_close(to_u16(h), eh, what="h", max_ulp=1, min_exact=0.999)
    # db = bf16(g * s): s is one rounding of silu, within 1 ulp of the oracle's
    assert_bf16_close(to_u16(db), edb, what="db", max_ulp=1, min_exact=0.999)
    t = np.abs((gr.float() * b.float()).cpu().numpy())
    assert_bf16_close(to_u16(da), eda, what="da", max_ulp=1, min_exact=0.999,
                      ulp_abs_slack=float(t.max()) * 2.0**-21)


@pytest.mark.parametrize("shape", [(8192, 14336), (3, 1000, 77)])
def test_fwd_bwd_bitwise_with_torch_eager(gpu, shape):
    """silu is bit-identical to eager's (exhaustive test), and the products
    and silu_backward use eager's fp32 operations: all three outputs equal
    eager's bit for bit; silu alone too."""
    print(f"[swiglu fwd+bwd eager] {shape}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(22)
    a, b, gr = (torch.randn(shape, dtype=torch.bfloat16, device=gpu, generator=g) * 3 for _ in range(3))
    s = torch.nn.functional.silu(a)
    h, db, da = kp.swiglu_forward_backward(a, b, gr)
    assert torch.equal(h, s * b)
    assert torch.equal(db, gr * s)
    assert torch.equal(da, torch.ops.aten.silu_backward(gr * b, a))
    del h, db, da
    assert torch.equal(kp.silu(a), s)


def test_fwd_bwd_empty_and_errors(gpu):
    e = torch.empty((0, 64), dtype=torch.bfloat16, device=gpu)
    assert all(t.shape == (0, 64) for t in kp.swiglu_forward_backward(e, e, e))
    assert kp.silu(e).shape == (0, 64)
    a = torch.randn(4, 16, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError):
        kp.swiglu_forward_backward(a, a, a[:, :8])


@pytest.mark.parametrize("op", ["backward", "forward_backward"])
def test_silu_backward_every_bf16_input_bitwise(gpu, op):
    """da = silu_backward(t, a) over all 65536 bf16 patterns of a, with t
    spanning random magnitudes and signs, against torch's eager
    silu_backward bit for bit: the sigmoid's division replaced by rcp and a
    Newton step for |a| < 16 must give eager's value for every input."""
    a = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).to(gpu).view(64, 1024)
    gen = torch.Generator(device=gpu).manual_seed(11)
    g = (torch.randn(a.shape, device=gpu, generator=gen) * 4).to(torch.bfloat16)
    b = torch.randn(a.shape, device=gpu, generator=gen).to(torch.bfloat16)
    ref = torch.ops.aten.silu_backward(g * b, a)
    if op == "backward":
        s = torch.nn.functional.silu(a)
        _, da = kp.swiglu_backward(g, s, b, a)
    else:
        _, _, da = kp.swiglu_forward_backward(a, b, g)
    same = (da.view(torch.int16) == ref.view(torch.int16)) | (torch.isnan(da) & torch.isnan(ref))
    bad = (~same).flatten().nonzero().flatten().tolist()
    assert not bad, f"{len(bad)} inputs differ, e.g. a={a.flatten()[bad[:5]].tolist()}"


def test_fast_sigmoid_and_silu_arithmetic_every_bf16_input(gpu):
    """The identities the kernels rely on, checked on the device over all
    65536 bf16 bit patterns, fp32 bit for bit: the rcp + Newton sigmoid of the
    backward equals the IEEE quotient 1 / (1 + expf(-x)) for every x with
    |x| < 16 (the range it is used in), and the forward's fast bf16 silu
    equals the bf16 rounding of x / (1 + expf(-x)) for every input (NaN as
    NaN)."""
    from kernelproblems_amd import _lib as L

    outs = [torch.empty(65536, dtype=torch.int32, device=gpu) for _ in range(4)]
    L.call("kp_swiglu_math_selftest", *[o.data_ptr() for o in outs], torch.cuda.current_stream().cuda_stream)
    sf, si, lf, lr = (o.cpu().numpy().view(np.uint32) for o in outs)
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    used = np.abs(x) < 16  # False for NaN
    assert int(used.sum()) == 33536
    assert np.array_equal(sf[used], si[used]), f"{int((sf[used] != si[used]).sum())} sigmoid values differ"
    nan = np.isnan(lr.view(np.float32))
    assert np.array_equal(np.isnan(lf.view(np.float32)), nan)
    assert np.array_equal(lf[~nan], lr[~nan]), f"{int((lf[~nan] != lr[~nan]).sum())} silu values differ"
