"""GPU parity: RMSNorm forward / backward kernels vs the C oracle (and torch-ROCm eager)."""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
from tests._util import (BF16_ATOL, BF16_RTOL, DW_RTOL, assert_bf16_close, bf, from_u16, gen, randn_bf16,
                         to_u16)

pytestmark = pytest.mark.gpu

FWD_SHAPES = [
    (64, 4096),   # vector path, 2 waves per row
    (33, 512),    # vector path, 1 chunk per lane, ragged row count
    (17, 8192),   # vector path, 4 waves per row
    (40, 2048),
    (9, 5120),    # vector path with 5 chunks per lane x 2 waves
    (7, 1000),    # generic path (N not a multiple of 512)
    (1, 64),
]


def _weight(n, g, kind, device):
    if kind == "none":
        return None, None, None
    w = randn_bf16(n, g, 1.0, 0.02)
    if kind == "contig":
        return w.to(device), to_u16(w), None
    # FSDP-style [8, n/8] slice of a flat buffer with a large row stride
    rows, cols = 8, n // 8
    stride = cols + 24
    buf = torch.zeros(rows * stride, dtype=torch.bfloat16)
    view = buf.as_strided((rows, cols), (stride, 1))
    view.copy_(w.view(rows, cols))
    dbuf = buf.to(device)
    dview = dbuf.as_strided((rows, cols), (stride, 1))
    return dview, to_u16(buf), (cols, stride)


@pytest.mark.parametrize("M,N", FWD_SHAPES)
@pytest.mark.parametrize("n_terms", [1, 2, 3])
def test_rmsnorm_fwd_matches_oracle(gpu, oracle_lib, M, N, n_terms):
    O = oracle_lib
    g = gen(1000 + M * 7 + N + n_terms)
    xs = [randn_bf16((M, N), g) for _ in range(n_terms)]
    for kind in ("contig", "none") + (("strided",) if N % 8 == 0 and N >= 64 else ()):
        w_dev, w_u16, seg = _weight(N, g, kind, gpu)
        eps = 1e-6
        h, y, rstd = kp.rms_norm([x.to(gpu) for x in xs], w_dev, eps, N, return_h=True, return_rstd=True)
        torch.cuda.synchronize()
        h_o, y_o, r_o = O.rmsnorm_fwd([to_u16(x) for x in xs], w_u16, eps, N, w_seg=seg)
        if n_terms > 1:
            assert np.array_equal(to_u16(h), h_o), "h (bf16 running sum) must be bit-exact"
        np.testing.assert_allclose(rstd.cpu().numpy(), r_o, rtol=1e-5, atol=0)
        assert_bf16_close(to_u16(y), y_o, what=f"y[{kind}]", max_ulp=1, min_exact=0.99)


@pytest.mark.parametrize("n_terms", [1, 2])
def test_rmsnorm_fwd_block_per_row_from_8192_rows(gpu, oracle_lib, n_terms):
    """From 8192 rows of 4096 the forward runs one block of 4 waves per row
    (the row's sum of squares split four ways): every rstd against fp64, h
    bit-exact, and y of 64 sampled rows against the oracle."""
    M, N = 8192, 4096
    print(f"[rms fwd block-per-row] [{M},{N}] terms={n_terms}", flush=True)
    g = gen(8192 + n_terms)
    xs = [randn_bf16((M, N), g) for _ in range(n_terms)]
    w = randn_bf16(N, g, 1.0, 0.02)
    h, y, rstd = kp.rms_norm([x.to(gpu) for x in xs], w.to(gpu), 1e-6, N, return_h=True, return_rstd=True)
    hh = xs[0].to(gpu) if n_terms == 1 else h
    if n_terms > 1:
        assert torch.equal(h, xs[0].to(gpu) + xs[1].to(gpu))
    r64 = torch.rsqrt(hh.double().pow(2).mean(-1) + 1e-6)
    assert float(((rstd.view(-1).double() - r64).abs() / r64).max()) < 1e-6
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(3))[:64].sort().values
    _, y_o, _ = oracle_lib.rmsnorm_fwd([to_u16(x[rows]) for x in xs], to_u16(w), 1e-6, N)
    assert_bf16_close(to_u16(y[rows.to(gpu)]), y_o, what="y", max_ulp=1, min_exact=0.99)


def test_rmsnorm_fwd_vs_torch_eager(gpu):
    """The reference fragment's own op on this GPU (torch-ROCm eager _fused_rms_norm)."""
    g = gen(7)
    x = randn_bf16((1, 512, 4096), g).to(gpu)
    w = randn_bf16(4096, g, 1.0, 0.02).to(gpu)
    y_ref, r_ref = torch.ops.aten._fused_rms_norm.default(x, [4096], w, 1e-5)
    y, r = kp.aten._fused_rms_norm(x, [4096], w, 1e-5)
    assert y.shape == y_ref.shape and r.shape == r_ref.shape and r.dtype == torch.float32
    assert_bf16_close(to_u16(y), to_u16(y_ref), what="y vs eager", max_ulp=1)
    torch.testing.assert_close(r, r_ref, rtol=1e-5, atol=0)


BWD_SHAPES = [(64, 4096), (33, 512), (17, 8192), (9, 5120), (7, 1000), (300, 1024)]


@pytest.mark.parametrize("M,N", BWD_SHAPES)
@pytest.mark.parametrize("variant", ["plain", "rstd_given", "epilogues"])
def test_rmsnorm_bwd_matches_oracle(gpu, oracle_lib, M, N, variant):
    O = oracle_lib
    g = gen(2000 + M + N)
    n_dy = 2 if variant == "epilogues" else 1
    n_x = 2 if variant == "epilogues" else 1
    dys = [randn_bf16((M, N), g) for _ in range(n_dy)]
    xs = [randn_bf16((M, N), g) for _ in range(n_x)]
    w = randn_bf16(N, g, 1.0, 0.02)
    res = randn_bf16((M, N), g) if variant == "epilogues" else None
    eps = 1e-6
    rstd = None
    if variant == "rstd_given":
        _, _, r_np = O.rmsnorm_fwd([to_u16(x) for x in xs], to_u16(w), eps, N)
        rstd = torch.from_numpy(r_np)
    dx, dw = kp.rms_norm_backward(
        [d.to(gpu) for d in dys], [x.to(gpu) for x in xs], None if rstd is None else rstd.to(gpu), w.to(gpu), eps,
        N, dx_residual=None if res is None else res.to(gpu), dw="f32")
    torch.cuda.synchronize()
    dx_o, dw_o, _ = O.rmsnorm_bwd([to_u16(d) for d in dys], [to_u16(x) for x in xs],
                                  None if rstd is None else rstd.numpy(), to_u16(w), eps, N,
                                  dx_residual=None if res is None else to_u16(res))
    assert_bf16_close(to_u16(dx), dx_o, what="dx", min_exact=0.97)
    dwv = dw.cpu().numpy().astype(np.float64)
    scale = np.sqrt(M) * 1.0  # |dw| ~ sqrt(M): compare relative to the column magnitude
    np.testing.assert_allclose(dwv, dw_o, rtol=DW_RTOL, atol=DW_RTOL * scale)


def test_rmsnorm_bwd_deterministic(gpu):
    g = gen(3)
    M, N = 1024, 4096
    x = randn_bf16((M, N), g).to(gpu)
    dy = randn_bf16((M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    a = kp.rms_norm_backward([dy], [x], None, w, 1e-6, N)
    b = kp.rms_norm_backward([dy], [x], None, w, 1e-6, N)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_rmsnorm_bwd_vs_torch_eager(gpu):
    """aten._fused_rms_norm_backward on this GPU: dx within bf16 tolerance, dw
    (bf16 in eager) within its bf16 rounding of our fp32 result."""
    g = gen(11)
    x = randn_bf16((1, 256, 4096), g).to(gpu)
    dy = randn_bf16((1, 256, 4096), g).to(gpu)
    w = randn_bf16(4096, g, 1.0, 0.02).to(gpu)
    _, rstd = torch.ops.aten._fused_rms_norm.default(x, [4096], w, 1e-5)
    dx_ref, dw_ref = torch.ops.aten._fused_rms_norm_backward.default(dy, x, [4096], rstd, w, [True, True])
    dx, dw = kp.aten._fused_rms_norm_backward(dy, x, [4096], rstd, w, [True, True])
    assert dx.dtype == dx_ref.dtype and dw.dtype == dw_ref.dtype == torch.bfloat16
    assert_bf16_close(to_u16(dx), to_u16(dx_ref), what="dx vs eager")
    assert_bf16_close(to_u16(dw), to_u16(dw_ref), rtol=2 ** -7, atol=1e-2, what="dw vs eager")


def test_rmsnorm_bwd_dw_modes(gpu):
    g = gen(5)
    M, N = 96, 4096
    x = randn_bf16((M, N), g).to(gpu)
    dy = randn_bf16((M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    _, dw32 = kp.rms_norm_backward([dy], [x], None, w, 1e-6, N, dw="f32")
    _, dwr = kp.rms_norm_backward([dy], [x], None, w, 1e-6, N, dw="f32_bf16")
    _, dwb = kp.rms_norm_backward([dy], [x], None, w, 1e-6, N, dw="bf16")
    assert dwr.dtype == torch.float32 and dwb.dtype == torch.bfloat16
    assert torch.equal(dwr, dw32.to(torch.bfloat16).float())
    assert torch.equal(dwb, dw32.to(torch.bfloat16))


def test_rmsnorm_empty_rows(gpu):
    x = torch.empty((0, 4096), dtype=torch.bfloat16, device=gpu)
    w = torch.ones(4096, dtype=torch.bfloat16, device=gpu)
    _, y, r = kp.rms_norm([x], w, 1e-6, 4096)
    assert y.shape == (0, 4096) and r.shape == (0,)
    dx, dw = kp.rms_norm_backward([x], [x], None, w, 1e-6, 4096)
    assert dx.shape == (0, 4096) and torch.count_nonzero(dw) == 0


def test_row_layouts_give_the_contiguous_bits(gpu):
    """The wrappers' row-layout rules (kp_torch.cpp as_rows): a padded row
    stride and a 3-D view whose rows share one stride are read in place; a
    transposed tensor (no [M, N] view with unit inner stride) is copied
    first.  Every layout gives exactly the contiguous input's y, rstd, dx
    and dw bits."""
    print("[rms layouts]", flush=True)
    g = gen(4242)
    M, N = 64, 1024
    x = randn_bf16((M, N), g).to(gpu)
    dy = randn_bf16((M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    _, y0, r0 = kp.rms_norm([x], w, 1e-6, N)
    dx0, dw0 = kp.rms_norm_backward([dy], [x], None, w, 1e-6, N)

    def padded(t):
        buf = torch.zeros((M, N + 64), dtype=t.dtype, device=gpu)
        buf[:, :N] = t
        return buf[:, :N]

    def batched(t):  # [2, M/2, N] view of a [2, M/2, N + 128] buffer: one uniform row stride
        buf = torch.zeros((2, M // 2, N + 128), dtype=t.dtype, device=gpu)
        buf[:, :, :N] = t.view(2, M // 2, N)
        return buf[:, :, :N]

    def transposed(t):  # the same values, stored column-major
        return t.t().contiguous().t()

    for name, f in (("padded", padded), ("batched", batched), ("transposed", transposed)):
        xv, dyv = f(x), f(dy)
        _, y, r = kp.rms_norm([xv], w, 1e-6, N)
        dx, dw = kp.rms_norm_backward([dyv], [xv], None, w, 1e-6, N)
        torch.cuda.synchronize()
        assert y.shape == xv.shape and dx.shape == xv.shape, name
        assert torch.equal(y.reshape(M, N), y0) and torch.equal(r, r0), name
        assert torch.equal(dx.reshape(M, N), dx0) and torch.equal(dw, dw0), name


@pytest.mark.parametrize("M, N, residual", [(8192, 4096, False), (4096, 8192, True), (1000, 4096, False)])
def test_block_trace_hook_records_every_block_and_changes_nothing(gpu, M, N, residual):
    """kp_debug_block_trace: with the hook set, every row block of the
    backward's row kernel writes (start <= rows done <= partial stored, XCC id
    < 8) and nothing past its records; dx and dw are bitwise those of an
    untraced call."""
    from kernelproblems_amd import _lib as L
    print(f"[rmsnorm] block trace hook M={M} N={N} residual={residual}", flush=True)
    g = gen(21)
    x = randn_bf16((M, N), g).to(gpu)
    dy = randn_bf16((M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    res = randn_bf16((M, N), g).to(gpu) if residual else None
    dx0, dw0 = kp.rms_norm_backward([dy], [x], None, w, 1e-5, N, dx_residual=res)
    cap = 4096
    buf = torch.zeros(cap * 4 + 64, dtype=torch.int64, device=gpu)
    lib = L.lib()
    lib.kp_debug_block_trace(buf.data_ptr(), cap * 32)
    try:
        dx1, dw1 = kp.rms_norm_backward([dy], [x], None, w, 1e-5, N, dx_residual=res)
    finally:
        lib.kp_debug_block_trace(None, 0)
    torch.cuda.synchronize()
    assert torch.equal(dx0.view(torch.int16), dx1.view(torch.int16))
    assert torch.equal(dw0.view(torch.int32), dw1.view(torch.int32))
    rec = buf[: cap * 4].view(cap, 4).cpu()
    n = int((rec[:, 0] != 0).sum())
    assert n > 0 and bool((rec[:n, 0] != 0).all()) and bool((rec[n:] == 0).all()), "records must be the first n"
    r = rec[:n]
    assert bool((r[:, 0] <= r[:, 1]).all()) and bool((r[:, 1] <= r[:, 2]).all())
    assert bool((r[:, 3] >= 0).all()) and bool((r[:, 3] < 8).all())
    assert bool((buf[cap * 4:] == 0).all()), "nothing may be written past the records"


@pytest.mark.parametrize("M,N", [(8191, 4096), (8192, 4096), (1001, 1024), (3, 512), (16383, 8192), (37, 1000)])
@pytest.mark.parametrize("alias", ["dx_residual", "dy"])
def test_rmsnorm_bwd_in_place(gpu, M, N, alias):
    """dx may be the residual-gradient input (out = res + dx accumulated in
    place) or the dy input: every row is read by the waves that write it, so
    the in-place call gives the bits of the out-of-place one -- also at row
    counts that leave a block's last row group ragged, and on the generic
    kernel (N = 1000)."""
    import ctypes as C
    from kernelproblems_amd import _lib as L
    print(f"[rms bwd in place] [{M},{N}] dx = {alias}", flush=True)
    lib = L.lib()
    g = gen(M + N)
    x, dy, res = (randn_bf16((M, N), g).to(gpu) for _ in range(3))
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    ws = torch.empty(int(lib.kp_rmsnorm_bwd_workspace_size(M, N)), dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream

    def call(dy_t, res_t, dx_t, dw_t):
        st = lib.kp_rmsnorm_bwd_bf16(L.ptr_array([dy_t.data_ptr()]), L.i64_array([N]), 1,
                                     L.ptr_array([x.data_ptr()]), L.i64_array([N]), 1, None, w.data_ptr(), N, N,
                                     res_t.data_ptr(), N, dx_t.data_ptr(), N, dw_t.data_ptr(), None, 0, M, N, 1e-5,
                                     ws.data_ptr(), ws.numel(), stream)
        assert st == 0, lib.kp_last_error_message().decode()

    dx_ref = torch.empty_like(x)
    dw_ref = torch.empty(N, dtype=torch.float32, device=gpu)
    call(dy, res, dx_ref, dw_ref)
    dw = torch.empty_like(dw_ref)
    if alias == "dx_residual":
        buf = res.clone()
        call(dy, buf, buf, dw)
    else:
        buf = dy.clone()
        call(buf, res, buf, dw)
    torch.cuda.synchronize()
    assert torch.equal(buf, dx_ref)
    assert torch.equal(dw, dw_ref)
