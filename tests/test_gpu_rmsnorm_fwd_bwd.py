"""GPU parity of the one-pass RMSNorm forward + backward
(kp_rmsnorm_fwd_bwd_bf16, the _fused_rms_norm -> _fused_rms_norm_backward
regions of v6/0b493aad68f0/problem.py:16-47 and v6/822931829090/problem.py:10-66).

* dx and dw are bitwise those of the backward that recomputes rstd itself
  (the same row kernel, the same blocks, the same fixed-order finalize);
* y is bitwise bf16((x * rstd) * w) evaluated on the host in fp32 from the
  rstd the pass returns (two IEEE multiplies, one rounding);
* against the C oracle: y within 1 bf16 ulp and >= 99% identical, rstd within
  1e-5 relative, h bit-exact, dx / dw to the backward's bars;
* shapes and term combinations without a fused kernel take the two-launch
  path and meet the same bars.
"""
import numpy as np
import pytest
import torch

import kernelproblems_amd as kp
from tests._util import DW_RTOL, assert_bf16_close, bf, gen, randn_bf16, to_u16

pytestmark = pytest.mark.gpu

# (M, N, x terms, dy terms, residual): the chain fragments' combinations at
# their row width, other widths, and combinations only the fallback covers.
CASES = [
    (64, 4096, 1, 3, True),    # v6/0b493aad68f0, v6/822931829090
    (64, 4096, 2, 2, True),    # v6/408ac0979ac5
    (64, 4096, 1, 2, True),    # v6/e9198b707240
    (33, 4096, 1, 1, False),   # plain norm, ragged row count
    (17, 8192, 1, 3, True),    # 8 waves per row, 8-wave blocks
    (40, 512, 1, 1, True),     # 1 chunk per lane
    (9, 5120, 3, 1, False),    # no fused kernel for 3 x terms: forward then backward
    (7, 1000, 1, 2, True),     # generic shape: forward then backward
]


def _host_y(x_u16, r, w_u16):
    """bf16((x * r) * w) in fp32 on the host, round to nearest even."""
    xf = (x_u16.astype(np.uint32) << 16).view(np.float32)
    wf = (w_u16.astype(np.uint32) << 16).view(np.float32)
    v = (xf * r[:, None].astype(np.float32)) * wf[None, :]
    u = v.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


@pytest.mark.parametrize("M,N,nx,ndy,res", CASES)
def test_fwd_bwd_one_pass(gpu, oracle_lib, M, N, nx, ndy, res):
    print(f"[fwd_bwd] M={M} N={N} nx={nx} ndy={ndy} res={res}", flush=True)
    O = oracle_lib
    g = gen(4000 + M * 3 + N + nx * 10 + ndy)
    xs = [randn_bf16((M, N), g) for _ in range(nx)]
    dys = [randn_bf16((M, N), g) for _ in range(ndy)]
    w = randn_bf16(N, g, 1.0, 0.02)
    r_in = randn_bf16((M, N), g) if res else None
    eps = 1e-5
    xd, dyd, wd = [x.to(gpu) for x in xs], [d.to(gpu) for d in dys], w.to(gpu)
    rd = None if r_in is None else r_in.to(gpu)
    y, dx, dw, h, rstd = kp.rms_norm_forward_backward(dyd, xd, wd, eps, N, dx_residual=rd, dw="f32",
                                                      return_h=True, return_rstd=True)
    dx_b, dw_b = kp.rms_norm_backward(dyd, xd, None, wd, eps, N, dx_residual=rd, dw="f32")
    torch.cuda.synchronize()

    # against the oracle
    h_o, y_o, r_o = O.rmsnorm_fwd([to_u16(x) for x in xs], to_u16(w), eps, N)
    if nx > 1:
        assert np.array_equal(to_u16(h), h_o), "h must be the bit-exact bf16 running sum"
    r = rstd.cpu().numpy()
    np.testing.assert_allclose(r, r_o, rtol=1e-5, atol=0)
    assert_bf16_close(to_u16(y), y_o, what="y", max_ulp=1, min_exact=0.99)
    dx_o, dw_o, _ = O.rmsnorm_bwd([to_u16(d) for d in dys], [to_u16(x) for x in xs], None, to_u16(w), eps, N,
                                  dx_residual=None if r_in is None else to_u16(r_in))
    assert_bf16_close(to_u16(dx), dx_o, what="dx", min_exact=0.97)
    np.testing.assert_allclose(dw.cpu().numpy().astype(np.float64), dw_o, rtol=DW_RTOL, atol=DW_RTOL * np.sqrt(M))

    # y from the returned rstd, exactly
    hx = h_o if nx > 1 else to_u16(xs[0])
    assert np.array_equal(to_u16(y), _host_y(hx, r, to_u16(w))), "y != bf16((x * rstd) * w)"
    # the backward half is the rstd-recomputing backward, bit for bit
    assert torch.equal(dx, dx_b), "dx differs from the backward that recomputes rstd"
    assert torch.equal(dw, dw_b), "dw differs from the backward that recomputes rstd"


def test_fwd_bwd_deterministic_and_dw_modes(gpu):
    g = gen(77)
    M, N = 512, 4096
    x = randn_bf16((M, N), g).to(gpu)
    dys = [randn_bf16((M, N), g).to(gpu) for _ in range(3)]
    w = randn_bf16(N, g, 1.0, 0.02).to(gpu)
    res = randn_bf16((M, N), g).to(gpu)
    a = kp.rms_norm_forward_backward(dys, [x], w, 1e-5, N, dx_residual=res, dw="f32")
    b = kp.rms_norm_forward_backward(dys, [x], w, 1e-5, N, dx_residual=res, dw="f32_bf16")
    c = kp.rms_norm_forward_backward(dys, [x], w, 1e-5, N, dx_residual=res, dw=None)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[0], c[0])
    assert torch.equal(b[2], a[2].to(torch.bfloat16).float()) and c[2] is None


def test_fwd_bwd_strided_weight_and_views(gpu):
    """The [8, 512] row-strided FSDP weight view of v5/118d525f44e0 read in
    place, inputs given as [1, M, N] views: equal to a contiguous weight."""
    g = gen(78)
    M, N = 128, 4096
    x = randn_bf16((1, M, N), g).to(gpu)
    dys = [randn_bf16((M, N), g).to(gpu) for _ in range(3)]
    res = randn_bf16((1, M, N), g).to(gpu)
    w = randn_bf16(N, g, 1.0, 0.02)
    buf = torch.zeros(8 * 27264000 // 1000, dtype=torch.bfloat16)
    stride = 27264000 // 1000
    view = buf.as_strided((8, 512), (stride, 1))
    view.copy_(w.view(8, 512))
    wv = buf.to(gpu).as_strided((8, 512), (stride, 1))
    a = kp.rms_norm_forward_backward(dys, [x], wv, 1e-5, N, dx_residual=res, dw="f32_bf16")
    b = kp.rms_norm_forward_backward(dys, [x], w.to(gpu), 1e-5, N, dx_residual=res, dw="f32_bf16")
    assert a[0].shape == x.shape and a[1].shape == x.shape and a[2].shape == (8, 512)
    for u, v in zip(a[:2], b[:2]):
        assert torch.equal(u, v)
    assert torch.equal(a[2].view(-1), b[2])


def test_fwd_bwd_empty_rows(gpu):
    x = torch.empty((0, 4096), dtype=torch.bfloat16, device=gpu)
    w = torch.ones(4096, dtype=torch.bfloat16, device=gpu)
    y, dx, dw, _, _ = kp.rms_norm_forward_backward([x], [x], w, 1e-6, 4096)
    assert y.shape == (0, 4096) and dx.shape == (0, 4096) and torch.count_nonzero(dw) == 0
