"""GPU: the streaming-ceiling probe writes the lane-wise 32-bit sum of its inputs."""
import pytest
import torch

from kernelproblems_amd import _lib as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_thread", [1, 2, 4, 8])
@pytest.mark.parametrize("policy", [L.KP_STORE_NONTEMPORAL, L.KP_STORE_WRITE_THROUGH])
@pytest.mark.parametrize("n_in,n_out,in_b,out_b", [(2, 1, 1 << 16, 1 << 16), (3, 2, 48, 48), (4, 2, 1 << 15, 1 << 15), (1, 1, 4096, 65536),
                                                   (3, 3, 1 << 16, 1 << 16),
                                                   (0, 2, 0, 20000 * 16)])
def test_stream_probe_outputs(gpu, n_in, n_out, in_b, out_b, per_thread, policy):
    g = torch.Generator().manual_seed(n_in * 10 + n_out)
    ins = [torch.randint(0, 1 << 30, (in_b // 4,), generator=g, dtype=torch.int64).to(torch.int32).to(gpu)
           for _ in range(n_in)]
    outs = [torch.full((out_b // 4,), -1, dtype=torch.int32, device=gpu) for _ in range(n_out)]
    L.call("kp_stream_probe", L.ptr_array([t.data_ptr() for t in ins]), n_in, in_b,
           L.ptr_array([t.data_ptr() for t in outs]), n_out, out_b, per_thread, policy,
           torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    n = out_b // 4
    idx = torch.arange(n, device=gpu)
    if n_in:
        s = torch.zeros(n, dtype=torch.int64, device=gpu)
        for t in ins:
            s[: t.numel()] += t.to(torch.int64)
        base = (s & 0xFFFFFFFF)
    else:
        base = torch.where(idx % 4 == 0, idx // 4, torch.zeros_like(idx))
    for w, o in enumerate(outs):
        exp = base + torch.where(idx % 4 == 0, torch.full_like(idx, w), torch.zeros_like(idx))
        exp = ((exp & 0xFFFFFFFF) ^ 0x80000000) - 0x80000000  # to signed 32-bit
        assert torch.equal(o.to(torch.int64), exp), f"output {w} differs"
