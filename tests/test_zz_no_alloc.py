"""The allocation-free RMSNorm backward (kp_rmsnorm_bwd_bf16_noalloc) through
the C ABI against kp_rmsnorm_bwd_bf16 with a caller workspace: bitwise the
same dx and weight gradient (the same row kernel, block count and
fixed-order finalize), on two calls in a row whose second is smaller (the
static scratch keeps the first call's partial rows, which must not leak into
the second), and a clean rejection of a shape whose partial rows exceed the
scratch, before anything is launched; a call on a second stream while the
previous call is pending is refused with KP_EBUSY."""
import ctypes as C

import pytest
import torch

from kernelproblems_amd import _lib as L
from tests._util import gen, randn_bf16

pytestmark = pytest.mark.gpu


def _call(lib, entry, dy, x, res, w, dx, dw, M, N, ws=None):
    stream = torch.cuda.current_stream().cuda_stream
    common = (L.ptr_array([dy.data_ptr()]), L.i64_array([N]), 1, L.ptr_array([x.data_ptr()]), L.i64_array([N]), 1,
              None, w.data_ptr(), N, N, None if res is None else res.data_ptr(), N, dx.data_ptr(), N, dw.data_ptr(),
              None, 0, M, N, 1e-5)
    if entry == "kp_rmsnorm_bwd_bf16":
        return lib.kp_rmsnorm_bwd_bf16(*common, ws.data_ptr(), ws.numel(), stream)
    return lib.kp_rmsnorm_bwd_bf16_noalloc(*common, stream)


def _pair(gpu, M, N, residual, seed):
    lib = L.lib()
    g = gen(seed)
    x, dy = randn_bf16((M, N), g).to(gpu), randn_bf16((M, N), g).to(gpu)
    res = randn_bf16((M, N), g).to(gpu) if residual else None
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    out = []
    for entry in ("kp_rmsnorm_bwd_bf16", "kp_rmsnorm_bwd_bf16_noalloc"):
        dx = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        dw = torch.full((N,), float("nan"), dtype=torch.float32, device=gpu)
        ws = torch.empty(int(lib.kp_rmsnorm_bwd_workspace_size(M, N)), dtype=torch.uint8, device=gpu)
        st = _call(lib, entry, dy, x, res, w, dx, dw, M, N, ws)
        assert st == 0, f"{entry}: {lib.kp_last_error_message().decode()}"
        out.append((dx, dw))
    torch.cuda.synchronize()
    (dx_a, dw_a), (dx_b, dw_b) = out
    assert torch.equal(dx_a, dx_b), f"dx differs at M={M} N={N}"
    assert torch.equal(dw_a, dw_b), f"dw differs at M={M} N={N}"


def test_noalloc_matches_workspace_entry_two_calls(gpu):
    print("[no_alloc] C2 shape then a smaller one", flush=True)
    assert L.lib().kp_rmsnorm_bwd_noalloc_max_bytes() == 8 << 20
    _pair(gpu, 8192, 4096, False, 11)   # the C2 configuration: 256 partial rows of 4096
    _pair(gpu, 96, 1024, False, 12)     # fewer row blocks and a narrower row after it


def test_noalloc_residual_and_generic_shapes(gpu):
    print("[no_alloc] C5-width residual, then a generic-kernel shape", flush=True)
    _pair(gpu, 2048, 8192, True, 13)    # 8192 columns: the largest row the scratch holds at 256 blocks
    _pair(gpu, 33, 1000, True, 14)      # generic kernel (N not a multiple of 512)


def test_noalloc_rejects_oversized_before_launch(gpu):
    print("[no_alloc] oversized shape is rejected", flush=True)
    lib = L.lib()
    M, N = 4096, 16384  # generic kernel, 2 blocks per CU: 512 x 16384 fp32 partial rows = 32 MiB
    g = gen(15)
    x, dy = randn_bf16((M, N), g).to(gpu), randn_bf16((M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    # had anything run, dx and dw (finite inputs) would no longer be all NaN
    dx = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
    dw = torch.full((N,), float("nan"), dtype=torch.float32, device=gpu)
    st = _call(lib, "kp_rmsnorm_bwd_bf16_noalloc", dy, x, None, w, dx, dw, M, N)
    assert st == L.KP_EUNSUPPORTED
    assert b"static scratch" in lib.kp_last_error_message()
    torch.cuda.synchronize()
    assert bool(torch.isnan(dx).all()), "nothing may be launched for a rejected shape"
    assert bool(torch.isnan(dw).all()), "nothing may be launched for a rejected shape"


def test_noalloc_busy_on_another_stream(gpu):
    """A call on a second stream while the previous call (first stream) is
    still pending returns KP_EBUSY and launches nothing; once that call has
    finished, the second stream's call runs and matches the workspace entry.
    Pending is established, not assumed: a torch event recorded on the first
    stream ahead of its call must still be incomplete after the second call
    has returned (the library's event comes later on that stream)."""
    print("[no_alloc] overlap guard across two streams", flush=True)
    lib = L.lib()
    M, N = 8192, 4096
    g = gen(16)
    x, dy = randn_bf16((M, N), g).to(gpu), randn_bf16((M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    big_src = torch.empty(1 << 31, dtype=torch.bfloat16, device=gpu)  # 4 GiB
    big_dst = torch.empty_like(big_src)
    sa, sb = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    dx_a = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
    dw_a = torch.full((N,), float("nan"), dtype=torch.float32, device=gpu)
    dx_b, dw_b = torch.full_like(dx_a, float("nan")), torch.full_like(dw_a, float("nan"))
    before = torch.cuda.Event()
    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        for _ in range(8):  # ~15 ms of copies queued ahead of the call on stream a
            big_dst.copy_(big_src)
        before.record(sa)
        assert _call(lib, "kp_rmsnorm_bwd_bf16_noalloc", dy, x, None, w, dx_a, dw_a, M, N) == 0
    with torch.cuda.stream(sb):
        st = _call(lib, "kp_rmsnorm_bwd_bf16_noalloc", dy, x, None, w, dx_b, dw_b, M, N)
    pending = not before.query()
    assert pending, "stream a's queued copies finished before the second call: the guard was not exercised"
    assert st == L.KP_EBUSY, f"expected KP_EBUSY, got {st}: {lib.kp_last_error_message().decode()}"
    assert b"has not finished" in lib.kp_last_error_message()
    sa.synchronize()
    torch.cuda.synchronize()
    del big_src, big_dst
    assert bool(torch.isnan(dx_b).all()) and bool(torch.isnan(dw_b).all()), "the refused call launched work"
    with torch.cuda.stream(sb):
        assert _call(lib, "kp_rmsnorm_bwd_bf16_noalloc", dy, x, None, w, dx_b, dw_b, M, N) == 0
    torch.cuda.synchronize()
    ws = torch.empty(int(lib.kp_rmsnorm_bwd_workspace_size(M, N)), dtype=torch.uint8, device=gpu)
    dx_r, dw_r = torch.empty_like(dx_a), torch.empty_like(dw_a)
    assert _call(lib, "kp_rmsnorm_bwd_bf16", dy, x, None, w, dx_r, dw_r, M, N, ws) == 0
    torch.cuda.synchronize()
    for dx, dw in ((dx_a, dw_a), (dx_b, dw_b)):
        assert torch.equal(dx, dx_r) and torch.equal(dw, dw_r)
