#!/usr/bin/env python3
"""Throughput of the fused fragment kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2] [--solo] [--all] [--no-cpu]

The default run measures every BASELINE configuration (c1, c2, c3f, c3b, c4,
c5f, c5b) and prints one JSON line: the headline workload (c2, configs[1])
in the top-level fields and one block per configuration under "configs",
each with its whole-call rate, roofline (dominant kernel), traffic, CPU
baseline and the tensor-level drop-in's time per call.  When --steps is
below 100, each block also carries a "steady" pass of 100 calls: the timed
loop's fixed cost (first launch, closing synchronisation) spread over few
steps inflates the per-call time of the small configurations.  The default run also times the canonical
drop-in of each fragment family (CORE_FRAGMENTS: RMSNorm, embedding, RoPE and
the norm -> embedding-backward chain) through its kernel_function at the
reference's own shape, under "fragment_drop_ins", each beside the reference's
record of that fragment on its H100 (--fragments: every distinct drop-in).

A step is one call of the fragment (one pass of the hot path over one batch
of synthetic input, already resident in HBM).  Workloads are the
BASELINE.json configurations:

  c1   RMSNorm forward        x [4096, 4096]              -> y bf16, rstd fp32
  c2   RMSNorm backward       x, dy [8192, 4096]          -> dx bf16, dw fp32   (default: configs[1])
  c3f  embedding forward      table [128256, 4096], ids [8, 2048] Zipf(1.1) -> [8, 2048, 4096]
  c3b  embedding backward     grad [8, 2048, 4096]        -> dense fp32 [128256, 4096]
  c4   RoPE rotate-half       q [4, 4096, 32, 128], k [4, 4096, 8, 128], pos 0..4095, theta 5e5
  c64r RoPE on complex64      q [1, 8192, 32, 64], k [1, 8192, 8, 64] c64, gathered table rows (v1/075cb40f3d5d)
  c5f  add + RMSNorm forward  x, res [16384, 8192]        -> h, y bf16
  c5b  add + RMSNorm backward x, res, dy [16384, 8192]    -> dx bf16, dw fp32
  swf  SwiGLU gate forward    a, b [8192, 14336]          -> bf16(silu(a)) * b        (v8/c68dae22972b)
  swb  SwiGLU gate backward   g, s, b, a [8192, 14336]    -> db, da bf16              (v8/385e1beb9bb9)
  silu SiLU alone            a [8192, 14336]             -> bf16(silu(a))            (v7/58e7a4d6cde3)
  swfb SwiGLU fwd recomputed with bwd  a, b, g [8192, 14336] -> h, db, da bf16      (v6/182d2dcd0652)
  c3n  embedding -> RMSNorm  table [128256, 4096], ids [8, 2048] Zipf(1.1) -> y [8, 2048, 4096] in one launch (v8/12545c1e9b06)
  cef  cross-entropy forward  logits [8192, 128256] bf16, targets -> loss, total_weight (v8/71f1d2c9f38b)
  ceb  cross-entropy backward log-softmax [8192, 128256] fp32, targets -> bf16 grad   (v8/622c35f5d1c6)
  cefb cross-entropy fwd+bwd  logits [8192, 128256] bf16, targets -> bf16 grad, one pass (v5/fb5b36393cbd)
  nfb  RMSNorm fwd + bwd      x, 3 dy, res [8192, 4096] -> y, g, dw in one row pass (v6/0b493aad68f0)
  nfb2 the same as the forward kernel then the backward kernel (the composition nfb replaces)
  nec  RMSNorm fwd + bwd -> embedding bwd  x, 3 dy, res [8192, 4096], ids [8192] -> y, dw, table fp32 [128256, 4096],
       g summed into the table in registers (v6/0b493aad68f0)
  nec2 the same as the norm's row pass writing g, then the embedding backward reading it (what nec replaces)

Each step uses one of R rotating copies of its inputs/outputs (R * bytes >=
~1 GiB, several times the 256 MiB Infinity Cache) so that a call does not
find its operands in cache from the previous call.  The timed loop calls the
C ABI directly through pre-bound ctypes arguments, after ~5 ms of plain
device copies (no part of the workload) and the W warmup steps.  value =
algorithmic bytes per call * steps / wall time of the timed loop
(synchronised on both sides, no instrumentation inside; the GPU time per
step comes from a separate pass with HIP events).  roofline.achieved = the
dominant kernel's algorithmic bytes / its mean duration, from a third pass
over K steps with HIP events that the library has the runtime stamp at that
kernel's own start and completion (kp_profile_dominant_kernel ->
hipExtLaunchKernel), on the stream the kernel runs on; the events are
timing-only (hipEventDisableSystemFence), so the stamp adds no L2 write-back
that back-to-back launches do not pay.  roofline.ceiling is
the same measurement for kp_stream_probe -- plain one-shot streaming of the
workload's byte mix (same number and sizes of arrays read and written, random
bf16 values, 16-byte accesses, 1, 2, 4 or 8 chunks per thread, non-temporal or
write-through stores, the fastest of the eight) -- so kernel_frac_of_ceiling
says how close the kernel comes to what
this GPU streams for those bytes.  The
cpu_baseline is the torch CPU eager restatement of the
fragment (oracle/torch_ref.py) on the same seeded inputs.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBS = 8000.0  # MI355X HBM3E
STEADY_STEPS = 100  # calls in the steady-state pass reported beside a shorter timed loop
MIN_ROTATION_BYTES = 1 << 30


def _u16():
    import torch
    return torch.bfloat16


class Workload:
    """Inputs, pre-bound ABI calls and byte counts of one configuration."""

    name = ""
    description = ""
    bytes_per_call = 0       # algorithmic bytes of the whole fragment call
    dominant_bytes = 0       # algorithmic bytes moved by the dominant kernel
    dominant_kernel = ""
    cpu_sample = ""
    # streaming-ceiling probe of the same byte mix: (inputs, outputs, bytes per
    # input array, bytes per output array, description)
    probe_mix = None

    dropin_entry = ""        # the tensor-level drop-in timed beside the C call
    cpu_bytes = None         # bytes of the CPU sample when it is a part of the call

    def __init__(self, dev):
        self.dev = dev
        self.sets = []     # per rotation set: (fn, args, keepalive)
        self.dropins = []  # per rotation set: (callable, args) of the tensor-level drop-in

    def rotations(self, per_set_bytes):
        return max(2, math.ceil(MIN_ROTATION_BYTES / max(per_set_bytes, 1)))

    def step(self, i):
        fn, args, _ = self.sets[i % len(self.sets)]
        st = fn(*args)
        if st != 0:
            from kernelproblems_amd import _lib as L
            raise L.KPError(fn.__name__, st, L.lib().kp_last_error_message().decode())

    def dropin(self, i):
        fn, args = self.dropins[i % len(self.dropins)]
        return fn(*args)

    def cpu_run(self):
        raise NotImplementedError


def _gen(seed=0):
    import torch
    return torch.Generator().manual_seed(seed)


def _randn(shape, g, mean=0.0, std=1.0):
    import torch
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def _zipf(n, vocab, s, g):
    import torch
    r = torch.arange(1, vocab + 1, dtype=torch.float64)
    p = r.pow(-s)
    p /= p.sum()
    return torch.multinomial(p, n, replacement=True, generator=g).to(torch.int64)


# ------------------------------------------------------------------ RMSNorm
class RmsFwd(Workload):
    def __init__(self, dev, M=4096, N=4096, eps=1e-6, name="c1", residual=False, rstd=True, cpu_rows=None):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        from kernelproblems_amd import fused as F
        self.name = name
        g = _gen(0)
        self.x = _randn((M, N), g)
        self.res = _randn((M, N), g) if residual else None
        self.w = _randn(N, g, 1.0, 0.02)
        self.eps, self.M, self.N = eps, M, N
        n_in = 2 if residual else 1
        n_out = 2 if residual else 1
        self.bytes_per_call = (n_in + n_out) * M * N * 2 + N * 2 + (M * 4 if rstd else 0)
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = "rms_fwd_vec"
        if residual:
            self.description = f"C5 residual add + RMSNorm forward: x, res [{M},{N}] bf16 -> h, y bf16 (eps={eps})"
        else:
            self.description = f"C1 RMSNorm forward: x [{M},{N}] bf16 -> y bf16, rstd fp32 (eps={eps})"
        self.probe_mix = (n_in, n_out, M * N * 2, M * N * 2, f"{n_in} read(s) + {n_out} write(s) of {M * N * 2 / 1e6:.1f} MB")
        per_set = self.bytes_per_call
        R = self.rotations(per_set)
        xd, wd = self.x.to(dev), self.w.to(dev)
        rd = self.res.to(dev) if residual else None
        fn = L.lib().kp_rmsnorm_fwd_bf16
        stream = torch.cuda.current_stream(dev).cuda_stream
        for r in range(R):
            xs = xd.clone()
            rs = rd.clone() if residual else None
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            h = torch.empty((M, N), dtype=torch.bfloat16, device=dev) if residual else None
            rstd_t = torch.empty(M, dtype=torch.float32, device=dev) if rstd else None
            terms = [xs] + ([rs] if residual else [])
            pa, sa = L.ptr_array([t.data_ptr() for t in terms]), L.i64_array([N] * len(terms))
            args = (pa, sa, len(terms), wd.data_ptr(), N, N, None if h is None else h.data_ptr(), N, y.data_ptr(),
                    N, None if rstd_t is None else rstd_t.data_ptr(), M, N, eps, stream)
            self.sets.append((fn, args, (xs, rs, y, h, rstd_t, pa, sa, wd)))
            self.dropins.append((F.rms_norm, (terms, wd, eps, N)) if not residual else
                                (lambda t, w: F.rms_norm(t, w, eps, N, return_h=True, return_rstd=False), (terms, wd)))
        self.dropin_entry = ("fused.rms_norm([x, res], w, eps, N, return_h=True, return_rstd=False)" if residual
                             else "fused.rms_norm([x], w, eps, N)")
        self.cpu_rows = min(cpu_rows or M, M)
        if self.cpu_rows < M:
            self.cpu_bytes = self.bytes_per_call * self.cpu_rows // M
            self.cpu_sample = f"{self.cpu_rows} of the {M} rows (rate scaled by the sample's own bytes)"
        else:
            self.cpu_sample = f"full [{M},{N}] call"

    def cpu_run(self):
        from oracle import torch_ref
        k = self.cpu_rows
        if self.res is not None:
            torch_ref.add_rms_norm_fwd(self.x[:k], self.res[:k], self.w, self.eps)
        else:
            torch_ref.rms_norm_fwd(self.x[:k], self.w, self.eps)


class RmsBwd(Workload):
    def __init__(self, dev, M=8192, N=4096, eps=1e-6, name="c2", residual=False, cpu_rows=None):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        from kernelproblems_amd import fused as F
        self.name = name
        g = _gen(0)
        self.x = _randn((M, N), g)
        self.res = _randn((M, N), g) if residual else None
        self.w = _randn(N, g, 1.0, 0.02)
        self.dy = _randn((M, N), g)
        self.eps, self.M, self.N = eps, M, N
        n_in = 3 if residual else 2
        self.dominant_bytes = (n_in + 1) * M * N * 2 + N * 2
        self.bytes_per_call = self.dominant_bytes + N * 4
        self.dominant_kernel = "rms_bwd_vec"
        self.probe_mix = (n_in, 1, M * N * 2, M * N * 2, f"{n_in} reads + 1 write of {M * N * 2 / 1e6:.1f} MB")
        self.timeline = True  # the row kernel records a block timeline (kp_debug_block_trace)
        if residual:
            self.description = (f"C5 residual add + RMSNorm backward: x, res, dy [{M},{N}] bf16 -> dx bf16, dw fp32 "
                                f"(h, rstd recomputed; eps={eps})")
        else:
            self.description = (f"C2 RMSNorm backward: x, dy [{M},{N}] bf16 -> dx bf16, dw fp32 "
                                f"(rstd recomputed; eps={eps})")
        R = self.rotations(self.bytes_per_call)
        xd, wd, dyd = self.x.to(dev), self.w.to(dev), self.dy.to(dev)
        rd = self.res.to(dev) if residual else None
        fn = L.lib().kp_rmsnorm_bwd_bf16
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws_bytes = int(L.lib().kp_rmsnorm_bwd_workspace_size(M, N))
        for r in range(R):
            xs, dys = xd.clone(), dyd.clone()
            rs = rd.clone() if residual else None
            dx = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            dw = torch.empty(N, dtype=torch.float32, device=dev)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            xterms = [xs] + ([rs] if residual else [])
            dpa, dsa = L.ptr_array([dys.data_ptr()]), L.i64_array([N])
            xpa, xsa = L.ptr_array([t.data_ptr() for t in xterms]), L.i64_array([N] * len(xterms))
            args = (dpa, dsa, 1, xpa, xsa, len(xterms), None, wd.data_ptr(), N, N, None, N, dx.data_ptr(), N,
                    dw.data_ptr(), None, 0, M, N, eps, ws.data_ptr(), ws_bytes, stream)
            self.sets.append((fn, args, (xs, dys, rs, dx, dw, ws, dpa, dsa, xpa, xsa, wd)))
            self.dropins.append((lambda d, xt, w: F.rms_norm_backward([d], xt, None, w, eps, N, dw="f32"),
                                 (dys, xterms, wd)))
        self.dropin_entry = (f"fused.rms_norm_backward([dy], [x{', res' if residual else ''}], None, w, eps, N, "
                             f"dw='f32')")
        self.cpu_rows = min(cpu_rows or M, M)
        if self.cpu_rows < M:
            self.cpu_bytes = self.bytes_per_call * self.cpu_rows // M
            self.cpu_sample = f"{self.cpu_rows} of the {M} rows (rate scaled by the sample's own bytes)"
        else:
            self.cpu_sample = f"full [{M},{N}] call"

    def cpu_run(self):
        from oracle import torch_ref
        k = self.cpu_rows
        if self.res is not None:
            torch_ref.add_rms_norm_bwd(self.x[:k], self.res[:k], self.dy[:k], self.w, self.eps)
        else:
            torch_ref.rms_norm_bwd(self.x[:k], self.dy[:k], self.w, self.eps)


# ---------------------------------------------------------------- embedding
class EmbFwd(Workload):
    def __init__(self, dev, V=128256, D=4096, B=8, S=2048, name="c3f"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        from kernelproblems_amd import fused as F
        self.name = name
        self.ids = _zipf(B * S, V, 1.1, _gen(0)).view(B, S)
        self.table = _randn((V, D), _gen(1), 0.0, 0.02)
        T = B * S
        self.bytes_per_call = 2 * T * D * 2 + T * 8
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = "emb_fwd_vec"
        self.probe_mix = (1, 1, T * D * 2, T * D * 2, f"copy of {T * D * 2 / 1e6:.1f} MB (the gather's bytes)")
        uniq = int(torch.unique(self.ids).numel())
        # The roofline counts the textbook gather (every gathered row read);
        # Zipf repeats are served by L2 / MALL, so the least HBM traffic is
        # each distinct row read once + the output + the ids, reported beside it.
        self.unique_row_bytes = uniq * D * 2 + T * D * 2 + T * 8
        self.description = (f"C3 embedding forward: table [{V},{D}] bf16, ids [{B},{S}] int64 Zipf(1.1) "
                            f"({uniq} distinct) -> [{B},{S},{D}] bf16, bit-exact gather")
        # per call: the distinct rows read + the output written; rotate whole tables
        R = max(2, math.ceil(MIN_ROTATION_BYTES / (uniq * D * 2 + T * D * 2)))
        tab_d, ids_d = self.table.to(dev), self.ids.to(dev)
        fn = L.lib().kp_embedding_fwd_bf16
        stream = torch.cuda.current_stream(dev).cuda_stream
        for r in range(R):
            tab = tab_d if r == 0 else tab_d.clone()
            out = torch.empty((B, S, D), dtype=torch.bfloat16, device=dev)
            args = (tab.data_ptr(), V, D, D, ids_d.data_ptr(), 8, T, out.data_ptr(), D, None, stream)
            self.sets.append((fn, args, (tab, out)))
            self.dropins.append((F.embedding, (tab, ids_d)))
        self.dropin_entry = "fused.embedding(table, ids)"
        self.cpu_sample = f"full [{B},{S}] gather"

    def cpu_run(self):
        from oracle import torch_ref
        torch_ref.embedding_fwd(self.table, self.ids)


class EmbNorm(Workload):
    """The token embedding fused into the first RMSNorm (the gathered rows
    never reach HBM), at the C3 embedding configuration."""

    def __init__(self, dev, V=128256, D=4096, B=8, S=2048, name="c3n"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name = name
        self.ids = _zipf(B * S, V, 1.1, _gen(0)).view(B, S)
        self.table = _randn((V, D), _gen(1), 0.0, 0.02)
        self.w = _randn(D, _gen(2), 1.0, 0.02)
        T = B * S
        self.bytes_per_call = 2 * T * D * 2 + T * 8 + D * 2
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = "rms_fwd_vec"
        self.probe_mix = (1, 1, T * D * 2, T * D * 2, f"copy of {T * D * 2 / 1e6:.1f} MB (gathered rows in, y out)")
        self.description = (f"embedding -> RMSNorm fused (v8/12545c1e9b06 region): table [{V},{D}] bf16, ids "
                            f"[{B},{S}] int64 Zipf(1.1) -> y [{B},{S},{D}] bf16 (eps=1e-5), no HBM intermediate")
        uniq = int(torch.unique(self.ids).numel())
        self.unique_row_bytes = uniq * D * 2 + T * D * 2 + T * 8 + D * 2  # distinct rows read once (as c3f)
        R = max(2, math.ceil(MIN_ROTATION_BYTES / (uniq * D * 2 + T * D * 2)))
        tab_d, ids_d, w_d = self.table.to(dev), self.ids.to(dev), self.w.to(dev)
        fn = L.lib().kp_embedding_rmsnorm_fwd_bf16
        stream = torch.cuda.current_stream(dev).cuda_stream
        for r in range(R):
            tab = tab_d if r == 0 else tab_d.clone()
            y = torch.empty((B, S, D), dtype=torch.bfloat16, device=dev)
            args = (tab.data_ptr(), V, D, ids_d.data_ptr(), 8, T, w_d.data_ptr(), D, D, None, D, y.data_ptr(), D,
                    None, D, 1e-5, None, stream)
            self.sets.append((fn, args, (tab, y, w_d, ids_d)))
        self.cpu_sample = f"full [{B},{S}] gather + norm"

    def cpu_run(self):
        from oracle import torch_ref
        torch_ref.embedding_rms_norm_fwd(self.table, self.ids, self.w, 1e-5)


class EmbBwd(Workload):
    def __init__(self, dev, V=128256, D=4096, B=8, S=2048, name="c3b"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        from kernelproblems_amd import fused as F
        self.name = name
        self.ids = _zipf(B * S, V, 1.1, _gen(0)).view(B, S)  # the same ids as the forward
        self.grad = _randn((B, S, D), _gen(2))
        self.V = V
        T = B * S
        self.bytes_per_call = T * D * 2 + T * 8 + V * D * 4
        # the zero fill is spread over the sort, rank, window and combine
        # launches: the timed span is the whole pipeline (first kernel's start
        # to last kernel's end) and carries every byte of the call
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = "emb_sort_chunks .. emb_combine (4-launch pipeline span)"
        self.probe_mix = (1, 1, T * D * 2, V * D * 4,
                          f"read {T * D * 2 / 1e6:.1f} MB + write {V * D * 4 / 1e6:.1f} MB")
        uniq = int(torch.unique(self.ids).numel())
        self.description = (f"C3 embedding backward: grad [{B},{S},{D}] bf16, ids Zipf(1.1) ({uniq} distinct) -> "
                            f"dense fp32 [{V},{D}], sort-and-segment, every row written (touched rows of the "
                            f"top zero shares twice)")
        R = self.rotations(self.bytes_per_call)
        gd, idd = self.grad.to(dev), self.ids.to(dev)
        fn = L.lib().kp_embedding_bwd_bf16
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws_bytes = int(L.lib().kp_embedding_bwd_workspace_size(T, V, D))
        for r in range(R):
            gs = gd.clone()
            out = torch.empty((V, D), dtype=torch.float32, device=dev)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            args = (gs.data_ptr(), D, idd.data_ptr(), 8, T, V, D, -1, 0, out.data_ptr(), 0, 0, ws.data_ptr(),
                    ws_bytes, None, stream)
            self.sets.append((fn, args, (gs, out, ws)))
            self.dropins.append((F.embedding_dense_backward, (gs, idd, V)))
        self.dropin_entry = "fused.embedding_dense_backward(grad, ids, V)"
        self.cpu_sample = f"full [{B},{S}] x {D} scatter into [{V},{D}]"

    def cpu_run(self):
        from oracle import torch_ref
        torch_ref.embedding_bwd(self.grad, self.ids, self.V)


# --------------------------------------------------------------------- RoPE
class Rope(Workload):
    def __init__(self, dev, B=4, S=4096, Hq=32, Hk=8, D=128, theta=500000.0, name="c4"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        from kernelproblems_amd import fused as F
        self.name = name
        g = _gen(0)
        self.q = _randn((B, S, Hq, D), g)
        self.k = _randn((B, S, Hk, D), g)
        self.pos = torch.arange(S, dtype=torch.int64).expand(B, S).contiguous()
        self.theta = theta
        nq, nk = B * S * Hq * D, B * S * Hk * D
        self.bytes_per_call = 2 * (nq + nk) * 2 + B * S * 8
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = "rope_tile"
        self.probe_mix = (1, 1, (nq + nk) * 2, (nq + nk) * 2, f"copy of {(nq + nk) * 2 / 1e6:.1f} MB (q and k)")
        self.description = (f"C4 RoPE rotate-half: q [{B},{S},{Hq},{D}], k [{B},{S},{Hk},{D}] bf16, positions "
                            f"[{B},{S}] int64 0..{S - 1}, theta={theta:g}, cos/sin in fp32 in-kernel")
        R = self.rotations(self.bytes_per_call)
        qd, kd, pd = self.q.to(dev), self.k.to(dev), self.pos.to(dev)
        fn = L.lib().kp_rope_bf16
        stream = torch.cuda.current_stream(dev).cuda_stream
        for r in range(R):
            qs, ks = qd.clone(), kd.clone()
            qo, ko = torch.empty_like(qs), torch.empty_like(ks)
            sq = L.i64_array(list(qs.stride()[:3]))
            sk = L.i64_array(list(ks.stride()[:3]))
            args = (qs.data_ptr(), qo.data_ptr(), Hq, sq, sq, ks.data_ptr(), ko.data_ptr(), Hk, sk, sk, B, S, D,
                    pd.data_ptr(), 8, S, 1, 0, theta, None, 0, 0, 0, 0, None, stream)
            self.sets.append((fn, args, (qs, ks, qo, ko, sq, sk, pd)))
            self.dropins.append((lambda q, k, p: F.rope(q, k, positions=p, theta=theta, pairing="half"), (qs, ks, pd)))
        self.dropin_entry = "fused.rope(q, k, positions=pos, theta=theta, pairing='half')"
        self.cpu_sample = f"full [{B},{S}] q and k"

    def cpu_run(self):
        from oracle import torch_ref
        torch_ref.rope_half(self.q, self.k, self.pos, self.theta)


class RopeComplex(Workload):
    """The complex64 RoPE of the v1 captures (v1/075cb40f3d5d): q and k
    already viewed as complex, times the table rows gathered by position ids,
    complex64 out."""

    def __init__(self, dev, S=8192, Hq=32, Hk=8, P=64, name="c64r"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name = name
        g = _gen(0)
        self.q = torch.randn((1, S, Hq, P), dtype=torch.complex64, generator=g)
        self.k = torch.randn((1, S, Hk, P), dtype=torch.complex64, generator=g)
        self.table = torch.randn((S, P), dtype=torch.complex64, generator=g)
        self.pos = torch.randint(0, 100, (1, S), dtype=torch.int32, generator=g)
        nq, nk = S * Hq * P, S * Hk * P
        # q and k read and written (8 B per complex), the gathered table row once per position, the id
        self.bytes_per_call = 2 * (nq + nk) * 8 + S * P * 8 + S * 4
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = "rope_c64_tile"
        self.probe_mix = (1, 1, (nq + nk) * 8, (nq + nk) * 8, f"copy of {(nq + nk) * 8 / 1e6:.1f} MB (q and k)")
        self.description = (f"RoPE on complex64 q [1,{S},{Hq},{P}], k [1,{S},{Hk},{P}] (v1/075cb40f3d5d): times "
                            f"table rows gathered by int32 positions, complex64 out")
        R = self.rotations(self.bytes_per_call)
        qd, kd, td, pd = self.q.to(dev), self.k.to(dev), self.table.to(dev), self.pos.to(dev)
        fn = L.lib().kp_rope_c64
        stream = torch.cuda.current_stream(dev).cuda_stream
        for r in range(R):
            qs, ks = qd.clone(), kd.clone()
            qo, ko = torch.empty_like(qs), torch.empty_like(ks)
            sq = L.i64_array(list(qs.stride()[:3]))
            sk = L.i64_array(list(ks.stride()[:3]))
            args = (qs.data_ptr(), qo.data_ptr(), Hq, sq, sq, ks.data_ptr(), ko.data_ptr(), Hk, sk, sk, 1, S, P,
                    pd.data_ptr(), 4, S, 1, torch.view_as_real(td).data_ptr(), S, P, 0, None, stream)
            self.sets.append((fn, args, (qs, ks, qo, ko, sq, sk, pd, td)))
        self.cpu_sample = f"full [1,{S}] q and k"

    def cpu_run(self):
        rows = self.table[self.pos[0].long()].view(1, -1, 1, self.table.shape[-1])
        _ = self.q * rows, self.k * rows  # torch CPU complex multiply: the fragment's eager ops


# ------------------------------------------------------------------ SwiGLU
class SwiGlu(Workload):
    """The feed-forward gate region at its reference shape: forward reads the
    w1 / w3 outputs and writes the gate product; backward reads the product's
    gradient, silu(w1 out), w3 out, w1 out and writes both branch gradients;
    silu alone reads w1 out and writes its silu; the recomputing backward
    reads w1 out, w3 out and the gradient and writes the product and both
    branch gradients."""

    # mode -> (inputs, outputs, entry point, dominant kernel, description)
    MODES = {
        "fwd": (2, 1, "kp_swiglu_fwd_bf16", "swiglu_fwd_vec",
                "SwiGLU gate forward (v8/c68dae22972b): a, b [{M},{N}] bf16 -> bf16(silu(a)) * b bf16"),
        "bwd": (4, 2, "kp_swiglu_bwd_bf16", "swiglu_bwd_vec",
                "SwiGLU gate backward (v8/385e1beb9bb9): g, silu(a), b, a [{M},{N}] bf16 -> "
                "db = g*silu(a), da = silu_backward(g*b, a) bf16"),
        "silu": (1, 1, "kp_silu_bf16", "silu_vec", "SiLU (v7/58e7a4d6cde3): a [{M},{N}] bf16 -> silu(a) bf16"),
        "fwdbwd": (3, 3, "kp_swiglu_fwd_bwd_bf16", "swiglu_fwd_bwd_vec",
                   "SwiGLU gate forward recomputed with its backward (v6/182d2dcd0652): a, b, g [{M},{N}] bf16 -> "
                   "h = silu(a)*b, db = g*silu(a), da = silu_backward(g*b, a) bf16"),
    }

    def __init__(self, dev, M=8192, N=14336, mode="fwd", name="swf"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name = name
        self.mode = mode
        g = _gen(0)
        n_in, n_out, entry, kernel, desc = self.MODES[mode]
        self.ops = [_randn((M, N), g) for _ in range(n_in)]
        self.bytes_per_call = (n_in + n_out) * M * N * 2
        self.dominant_bytes = self.bytes_per_call
        self.dominant_kernel = kernel
        self.probe_mix = (n_in, n_out, M * N * 2, M * N * 2,
                          f"{n_in} read(s) + {n_out} write(s) of {M * N * 2 / 1e6:.1f} MB")
        self.description = desc.format(M=M, N=N)
        R = self.rotations(self.bytes_per_call)
        dev_ops = [t.to(dev) for t in self.ops]
        fn = getattr(L.lib(), entry)
        stream = torch.cuda.current_stream(dev).cuda_stream
        for r in range(R):
            ins = [t if r == 0 else t.clone() for t in dev_ops]
            outs = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _ in range(n_out)]
            ptrs = []
            for t in ins + outs:
                ptrs += [t.data_ptr(), N]
            args = (*ptrs, M, N, stream)
            self.sets.append((fn, args, (ins, outs)))
        self.cpu_sample = f"full [{M},{N}] call"

    def cpu_run(self):
        from oracle import torch_ref
        {"fwd": torch_ref.swiglu_fwd, "bwd": torch_ref.swiglu_bwd, "silu": torch_ref.silu,
         "fwdbwd": torch_ref.swiglu_fwd_bwd}[self.mode](*self.ops)


# ------------------------------------------------------------------ cross-entropy
class CrossEntropy(Workload):
    """Token cross-entropy at the reference's shape (8192 tokens, V = 128256,
    targets uniform over the vocabulary, every 16th ignored).  Forward reads
    the bf16 logits once; backward reads the fp32 log-softmax and writes the
    bf16 logits gradient."""

    def __init__(self, dev, M=8192, V=128256, backward=False, name="cef"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name, self.backward = name, backward
        g = _gen(0)
        self.targets = torch.randint(0, V, (M,), generator=g)
        self.targets[::16] = -100
        td = self.targets.to(dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        if backward:
            x = torch.randn(M, V, generator=g) * 2
            self.lsm = torch.log_softmax(x, 1)
            del x
            self.bytes_per_call = M * V * (4 + 2)
            self.dominant_kernel = "xent_bwd_vec"
            # 4 bytes read per 2 written, interleaved through the whole stream:
            # two read arrays and one write array of equal size
            self.probe_mix = (2, 1, M * V * 2, M * V * 2,
                              f"2 reads + 1 write of {M * V * 2 / 1e9:.2f} GB (4.20 GB read, 2.10 GB written)")
            self.description = (f"cross-entropy backward (v8/622c35f5d1c6): log-softmax [{M},{V}] fp32, targets "
                                f"int64 -> grad bf16 [{M},{V}]")
            fn = L.lib().kp_cross_entropy_bwd_bf16
            src = self.lsm.to(dev)
            for r in range(self.rotations(self.bytes_per_call)):
                Ld = src if r == 0 else src.clone()
                out = torch.empty((M, V), dtype=torch.bfloat16, device=dev)
                args = (Ld.data_ptr(), V, td.data_ptr(), 8, -100, 1.0 / 8192.0, out.data_ptr(), V, M, V, None, stream)
                self.sets.append((fn, args, (Ld, out)))
        else:
            self.logits = _randn((M, V), g, 0.0, 2.0)
            self.bytes_per_call = M * V * 2 + M * 8
            self.dominant_kernel = "xent_fwd_vec"
            # read-only mix: the probe's one output array is a single 16-byte chunk
            self.probe_mix = (1, 1, M * V * 2, 16, f"read of {M * V * 2 / 1e9:.2f} GB")
            self.description = (f"cross-entropy forward (v8/71f1d2c9f38b): logits [{M},{V}] bf16, targets int64 "
                                f"-> loss, total_weight fp32 (log-softmax not materialised)")
            fn = L.lib().kp_cross_entropy_fwd_bf16
            ws_bytes = int(L.lib().kp_cross_entropy_fwd_workspace_size(M))
            src = self.logits.to(dev)
            for r in range(self.rotations(self.bytes_per_call)):
                xd = src if r == 0 else src.clone()
                loss = torch.empty((), dtype=torch.float32, device=dev)
                tw = torch.empty((), dtype=torch.float32, device=dev)
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
                args = (xd.data_ptr(), V, M, V, td.data_ptr(), 8, -100, 1.0 / 8192.0, loss.data_ptr(), tw.data_ptr(),
                        None, None, ws.data_ptr(), ws_bytes, stream)
                self.sets.append((fn, args, (xd, loss, tw, ws)))
        self.dominant_bytes = M * V * (6 if backward else 2)
        self.keep = td
        self.cpu_sample = f"full [{M},{V}] call"

    def cpu_run(self):
        from oracle import torch_ref
        if self.backward:
            torch_ref.cross_entropy_bwd(self.lsm, self.targets, 1.0 / 8192.0)
        else:
            torch_ref.cross_entropy_fwd(self.logits, self.targets, 1.0 / 8192.0)


class CrossEntropyFwdBwd(Workload):
    """The whole loss region from the bf16 logits to their bf16 gradient
    (v5/fb5b36393cbd) at the reference's shape: each logit read once, each
    gradient entry written once (the fp32 log-softmax never stored)."""

    def __init__(self, dev, M=8192, V=128256, name="cefb", cpu_rows=1024):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name = name
        g = _gen(0)
        self.targets = torch.randint(0, V, (M,), generator=g)
        self.targets[::16] = -100
        td = self.targets.to(dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        self.logits = _randn((M, V), g, 0.0, 2.0)
        self.bytes_per_call = M * V * 4 + M * 8
        self.dominant_bytes = M * V * 4 + M * 8
        self.dominant_kernel = "xent_fwd_bwd_vec"
        self.probe_mix = (1, 1, M * V * 2, M * V * 2, f"copy of {M * V * 2 / 1e9:.2f} GB (logits in, gradient out)")
        self.description = (f"cross-entropy forward + backward from the logits (v5/fb5b36393cbd): logits [{M},{V}] "
                            f"bf16, targets int64 -> grad bf16 [{M},{V}] (log-softmax not materialised)")
        fn = L.lib().kp_cross_entropy_fwd_bwd_bf16
        src = self.logits.to(dev)
        for r in range(self.rotations(self.bytes_per_call)):
            xd = src if r == 0 else src.clone()
            out = torch.empty((M, V), dtype=torch.bfloat16, device=dev)
            args = (xd.data_ptr(), V, M, V, td.data_ptr(), 8, -100, 1.0 / 8192.0, out.data_ptr(), V, 1.0 / 8192.0,
                    None, None, None, None, 0, stream)
            self.sets.append((fn, args, (xd, out)))
        self.keep = td
        # the CPU restatement materialises three fp32 [rows, V] arrays: time a row sample
        self.cpu_rows = min(cpu_rows, M)
        self.cpu_bytes = self.cpu_rows * (V * 4 + 8)
        self.cpu_sample = f"{self.cpu_rows} of the {M} rows (rate scaled by the sample's own bytes)"

    def cpu_run(self):
        from oracle import torch_ref
        torch_ref.cross_entropy_fwd_bwd(self.logits[:self.cpu_rows], self.targets[:self.cpu_rows], 1.0 / 8192.0)


# ------------------------------------------------------------ norm fwd + bwd
class NormFwdBwd(Workload):
    """The RMSNorm forward -> backward region of the chain fragments
    (v6/0b493aad68f0/problem.py:16-47) at their shape: x [8192, 4096], dy =
    three gradient terms, g = add_220 + dx.  one_pass=True: one row pass
    (kp_rmsnorm_fwd_bwd_bf16, x read once: 5 arrays read, y and g written);
    one_pass=False: the forward kernel then the backward kernel with its rstd
    (x read twice, rstd written and read) -- the composition it replaces."""

    def __init__(self, dev, M=8192, N=4096, one_pass=True, name="nfb"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name = name
        g = _gen(0)
        self.x = _randn((M, N), g)
        self.dys = [_randn((M, N), g) for _ in range(3)]
        self.res = _randn((M, N), g)
        self.w = _randn(N, g, 1.0, 0.02)
        eps = 1e-5
        nb = M * N * 2
        self.bytes_per_call = 7 * nb + N * 2 + N * 4 if one_pass else 9 * nb + N * 2 + N * 4 + 2 * M * 4
        self.dominant_bytes = 7 * nb + N * 2 if one_pass else 6 * nb + N * 2 + M * 4
        self.dominant_kernel = "rms_bwd_vec<.., FWD>" if one_pass else "rms_bwd_vec (after rms_fwd_vec)"
        self.probe_mix = None  # 5 reads + 2 writes: past what kp_stream_probe streams (<= 4 reads)
        self.description = (f"RMSNorm forward + backward of the chain fragments (v6/0b493aad68f0): x, 3 dy terms, "
                            f"residual [{M},{N}] bf16 -> y, g = res + dx bf16, dw fp32; "
                            + ("one row pass" if one_pass else "forward kernel then backward kernel"))
        lib = L.lib()
        stream = torch.cuda.current_stream(dev).cuda_stream
        R = self.rotations(self.bytes_per_call)
        xd, wd, rd = self.x.to(dev), self.w.to(dev), self.res.to(dev)
        dyd = [d.to(dev) for d in self.dys]
        ws_bytes = int(lib.kp_rmsnorm_fwd_bwd_workspace_size(M, N))
        for r in range(R):
            xs, rs = xd.clone(), rd.clone()
            dys = [d.clone() for d in dyd]
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            gout = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            dw = torch.empty(N, dtype=torch.float32, device=dev)
            rstd = torch.empty(M, dtype=torch.float32, device=dev)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            dpa, dsa = L.ptr_array([d.data_ptr() for d in dys]), L.i64_array([N] * 3)
            xpa, xsa = L.ptr_array([xs.data_ptr()]), L.i64_array([N])
            keep = (xs, rs, dys, y, gout, dw, rstd, ws, dpa, dsa, xpa, xsa, wd)
            if one_pass:
                args = (dpa, dsa, 3, xpa, xsa, 1, wd.data_ptr(), N, N, None, N, y.data_ptr(), N, None,
                        rs.data_ptr(), N, gout.data_ptr(), N, dw.data_ptr(), None, 1, M, N, eps, ws.data_ptr(),
                        ws_bytes, stream)
                self.sets.append((lib.kp_rmsnorm_fwd_bwd_bf16, args, keep))
            else:
                fa = (xpa, xsa, 1, wd.data_ptr(), N, N, None, N, y.data_ptr(), N, rstd.data_ptr(), M, N, eps, stream)
                ba = (dpa, dsa, 3, xpa, xsa, 1, rstd.data_ptr(), wd.data_ptr(), N, N, rs.data_ptr(), N,
                      gout.data_ptr(), N, dw.data_ptr(), None, 1, M, N, eps, ws.data_ptr(), ws_bytes, stream)

                def both(fa=fa, ba=ba):
                    st = lib.kp_rmsnorm_fwd_bf16(*fa)
                    return st if st != 0 else lib.kp_rmsnorm_bwd_bf16(*ba)
                both.__name__ = "kp_rmsnorm_fwd_bf16 + kp_rmsnorm_bwd_bf16"
                self.sets.append((both, (), keep))
        self.cpu_sample = f"full [{M},{N}] call"

    def cpu_run(self):
        from oracle import torch_ref
        torch_ref.rms_norm_fwd(self.x, self.w, 1e-5)
        dy = self.dys[0] + self.dys[1] + self.dys[2]
        torch_ref.rms_norm_bwd(self.x, dy, self.w, 1e-5)


class NormEmbChain(Workload):
    """The whole chain of v6/0b493aad68f0 (problem.py:16-71) at its shape: the
    RMSNorm forward + backward of x [8192, 4096] with three gradient terms and
    the residual, and the dense embedding backward of g = add_220 + dx over
    ids [8192] drawn from 100 values (the fragment's get_inputs) into an fp32
    [128256, 4096] table.  fused=True: kp_rmsnorm_embedding_bwd_bf16 (the ids
    sorted first, the norm's row pass summing g into the table in registers:
    g never stored); fused=False: kp_rmsnorm_fwd_bwd_bf16 writing g, then
    kp_embedding_bwd_bf16 reading it back.  bytes_per_call is the fragment's
    algorithmic bytes for both (2 x 67 MB less than the composition moves)."""

    def __init__(self, dev, M=8192, N=4096, V=128256, fused=True, name="nec"):
        super().__init__(dev)
        import torch
        from kernelproblems_amd import _lib as L
        self.name = name
        g = _gen(0)
        self.x = _randn((M, N), g)
        self.dys = [_randn((M, N), g) for _ in range(3)]
        self.res = _randn((M, N), g)
        self.w = _randn(N, g, 1.0, 0.02)
        self.ids = torch.randint(0, 100, (M,), generator=g)
        eps = 1e-5
        nb = M * N * 2
        self.bytes_per_call = 6 * nb + V * N * 4 + M * 8 + N * 2 + N * 4
        # the timing hook spans the embedding pipeline's first to last launch (the fused
        # row pass included for nec); for nec2 the norm pass runs ahead of that span
        self.dominant_bytes = self.bytes_per_call - N * 4 if fused else V * N * 4 + nb + M * 8
        self.dominant_kernel = ("sort .. row pass .. combine (span)" if fused
                                else "embedding backward of the stored g (span)")
        self.probe_mix = None
        self.description = (f"RMSNorm fwd + bwd -> embedding bwd chain of v6/0b493aad68f0: x, 3 dy terms, residual "
                            f"[{M},{N}] bf16, ids [{M}] in [0, 100) -> y bf16, dw fp32, table fp32 [{V},{N}]; "
                            + ("one row pass over sorted-id windows, g kept in registers" if fused
                               else "norm row pass writing g, then the embedding backward reading it"))
        lib = L.lib()
        stream = torch.cuda.current_stream(dev).cuda_stream
        R = max(2, math.ceil(MIN_ROTATION_BYTES / (6 * nb)))  # rotate the row inputs; the tables are 2.1 GB each
        xd, wd, rd, idd = self.x.to(dev), self.w.to(dev), self.res.to(dev), self.ids.to(dev)
        dyd = [d.to(dev) for d in self.dys]
        tables = [torch.empty((V, N), dtype=torch.float32, device=dev) for _ in range(2)]
        if fused:
            ws_bytes = int(lib.kp_rmsnorm_embedding_bwd_workspace_size(M, N, V))
        else:
            ws_bytes = int(lib.kp_rmsnorm_fwd_bwd_workspace_size(M, N))
            ews_bytes = int(lib.kp_embedding_bwd_workspace_size(M, V, N))
        for r in range(R):
            xs, rs, ids = xd.clone(), rd.clone(), idd.clone()
            dys = [d.clone() for d in dyd]
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            dw = torch.empty(N, dtype=torch.float32, device=dev)
            table = tables[r % 2]
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            dpa, dsa = L.ptr_array([d.data_ptr() for d in dys]), L.i64_array([N] * 3)
            keep = (xs, rs, ids, dys, y, dw, table, ws, dpa, dsa, wd)
            if fused:
                args = (dpa, dsa, 3, xs.data_ptr(), N, None, wd.data_ptr(), N, N, rs.data_ptr(), N, y.data_ptr(), N,
                        None, dw.data_ptr(), None, 1, M, N, eps, ids.data_ptr(), 8, V, -1, table.data_ptr(),
                        L.KP_DTYPE_F32, 1, ws.data_ptr(), ws_bytes, None, stream)
                self.sets.append((lib.kp_rmsnorm_embedding_bwd_bf16, args, keep))
            else:
                gout = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
                ews = torch.empty(ews_bytes, dtype=torch.uint8, device=dev)
                xpa, xsa = L.ptr_array([xs.data_ptr()]), L.i64_array([N])
                na = (dpa, dsa, 3, xpa, xsa, 1, wd.data_ptr(), N, N, None, N, y.data_ptr(), N, None,
                      rs.data_ptr(), N, gout.data_ptr(), N, dw.data_ptr(), None, 1, M, N, eps, ws.data_ptr(),
                      ws_bytes, stream)
                ea = (gout.data_ptr(), N, ids.data_ptr(), 8, M, V, N, -1, 0, table.data_ptr(), L.KP_DTYPE_F32, 1,
                      ews.data_ptr(), ews_bytes, None, stream)

                def both(na=na, ea=ea):
                    st = lib.kp_rmsnorm_fwd_bwd_bf16(*na)
                    return st if st != 0 else lib.kp_embedding_bwd_bf16(*ea)
                both.__name__ = "kp_rmsnorm_fwd_bwd_bf16 + kp_embedding_bwd_bf16"
                self.sets.append((both, (), keep + (gout, ews, xpa, xsa)))
        self.cpu_rows = 256
        self.cpu_bytes = self.cpu_rows * 6 * N * 2
        self.cpu_sample = (f"the norm forward + backward of {self.cpu_rows} of the {M} rows and their table "
                           f"rows' segment sums (rate from the sample's own row bytes)")

    def cpu_run(self):
        import torch
        from oracle import torch_ref
        k = self.cpu_rows
        torch_ref.rms_norm_fwd(self.x[:k], self.w, 1e-5)
        dy = self.dys[0][:k] + self.dys[1][:k] + self.dys[2][:k]
        dx, _ = torch_ref.rms_norm_bwd(self.x[:k], dy, self.w, 1e-5)
        g = (self.res[:k].float() + dx.float()).to(torch.bfloat16)
        torch.zeros(100, g.shape[1]).index_add_(0, self.ids[:k], g.float())


def make_workload(name, dev):
    if name == "nec":
        return NormEmbChain(dev, fused=True, name="nec")
    if name == "nec2":
        return NormEmbChain(dev, fused=False, name="nec2")
    if name == "nfb":
        return NormFwdBwd(dev, one_pass=True, name="nfb")
    if name == "nfb2":
        return NormFwdBwd(dev, one_pass=False, name="nfb2")
    if name == "c1":
        return RmsFwd(dev, 4096, 4096, 1e-6, "c1")
    if name == "c2":
        return RmsBwd(dev, 8192, 4096, 1e-6, "c2")
    if name == "c3f":
        return EmbFwd(dev)
    if name == "c3b":
        return EmbBwd(dev)
    if name == "c3n":
        return EmbNorm(dev)
    if name == "c4":
        return Rope(dev)
    if name == "c64r":
        return RopeComplex(dev)
    if name == "c5f":
        return RmsFwd(dev, 16384, 8192, 1e-5, "c5f", residual=True, rstd=False, cpu_rows=4096)
    if name == "c5b":
        return RmsBwd(dev, 16384, 8192, 1e-5, "c5b", residual=True, cpu_rows=4096)
    if name == "swf":
        return SwiGlu(dev, name="swf")
    if name == "swb":
        return SwiGlu(dev, mode="bwd", name="swb")
    if name == "silu":
        return SwiGlu(dev, mode="silu", name="silu")
    if name == "swfb":
        return SwiGlu(dev, mode="fwdbwd", name="swfb")
    if name == "cef":
        return CrossEntropy(dev, name="cef")
    if name == "ceb":
        return CrossEntropy(dev, backward=True, name="ceb")
    if name == "cefb":
        return CrossEntropyFwdBwd(dev)
    raise SystemExit(f"unknown workload {name!r}")


ALL = ["c1", "c2", "c3f", "c3b", "c3n", "c4", "c64r", "c5f", "c5b", "swf", "swb", "silu", "swfb", "cef", "ceb",
       "cefb", "nfb", "nfb2", "nec", "nec2"]
# The BASELINE.json configurations: every default run measures each of them.
CONFIGS = ["c1", "c2", "c3f", "c3b", "c4", "c5f", "c5b"]


# ------------------------------------------------------------------ measure
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h
_HIP = None


def _hip():
    import ctypes
    global _HIP
    if _HIP is None:
        h = ctypes.CDLL("libamdhip64.so")  # already mapped by torch
        h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _HIP = h
    return _HIP


class StampEvents:
    """n (start, stop) pairs of timing-only HIP events, created with
    hipEventDisableSystemFence.  A default event's stop marker carries a
    system-scope release -- a write-back of L2 -- that back-to-back launches
    on one stream do not pay: stamped by default events, the RMSNorm backward
    row kernel at [8192, 4096] read 36.2 us, stamped by these 34.8 us, and
    the rocprofv3 kernel trace of the same calls 35.2 us (one box; kernels
    that leave little dirty data in L2 read the same either way).  The pairs
    are handed to kp_profile_dominant_kernel (the runtime then stamps the
    launch itself) or recorded around torch ops on a stream."""

    def __init__(self, n):
        import ctypes
        h = _hip()
        self.ev = []
        for _ in range(2 * n):
            e = ctypes.c_void_p()
            st = h.hipEventCreateWithFlags(ctypes.byref(e), HIP_EVENT_DISABLE_SYSTEM_FENCE)
            if st != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({st})")
            self.ev.append(e)

    def start(self, i):
        return self.ev[2 * i]

    def stop(self, i):
        return self.ev[2 * i + 1]

    def record(self, e, stream):
        import ctypes
        st = _hip().hipEventRecord(e, ctypes.c_void_p(stream))
        if st != 0:
            raise RuntimeError(f"hipEventRecord failed ({st})")

    def ms(self, i):
        """Elapsed ms of pair i (after a synchronisation)."""
        import ctypes
        f = ctypes.c_float()
        st = _hip().hipEventElapsedTime(ctypes.byref(f), self.start(i), self.stop(i))
        if st != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({st})")
        return f.value

    def close(self):
        h = _hip()
        for e in self.ev:
            h.hipEventDestroy(e)
        self.ev = []


def warm_device(dev):
    """~5 ms of plain device copies (16 x 1 GiB) before a workload's warmup
    steps.  After an idle stretch (workload set-up, a CPU baseline) the
    memory system needs a few ms of sustained traffic before it runs at full
    rate; five warmup steps of a short call do not supply it, and the first
    timed pass then runs slow (c3b: ~367 against ~355 us per call at K = 20,
    the later passes ~355 either way).  Nothing of the workload runs here."""
    import torch
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(16):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def measure_gpu(wl, steps, warmup):
    """Three passes over K steps: the timed pass (wall clock between two
    synchronisations, nothing else inside: recording even two HIP events in
    it cost ~1-2 us per call at K = 20) gives value and ms_per_step; a
    second pass with HIP events around the loop gives the GPU time per step;
    a third with the timing hook set gives the dominant kernel's per-launch
    durations (events stamped at its own start / end)."""
    import torch
    from kernelproblems_amd import _lib as L
    lib = L.lib()
    warm_device(wl.dev)
    for i in range(warmup):
        wl.step(i)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for i in range(steps):
        wl.step(warmup + i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0

    t0e, t1e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0e.record()
    for i in range(steps):
        wl.step(warmup + i)
    t1e.record()
    torch.cuda.synchronize()
    gpu_ms = t0e.elapsed_time(t1e)

    ev = StampEvents(steps)
    torch.cuda.synchronize()
    for i in range(steps):
        lib.kp_profile_dominant_kernel(ev.start(i), ev.stop(i))
        wl.step(warmup + steps + i)
    lib.kp_profile_dominant_kernel(None, None)
    torch.cuda.synchronize()
    dom = [ev.ms(i) for i in range(steps)]
    ev.close()
    dom_ms = sum(dom) / len(dom)
    ms_per_step = wall * 1e3 / steps
    value = wl.bytes_per_call * steps / wall / 1e9
    achieved = wl.dominant_bytes / (dom_ms * 1e-3) / 1e9
    return {
        "ms_per_step": ms_per_step,
        "gpu_ms_per_step": gpu_ms / steps,
        "value": value,
        "dominant_ms": dom_ms,
        "dominant_ms_min": min(dom),
        "achieved": achieved,
    }


def measure_timeline(wl, calls=5, warmup=10):
    """Where the RMSNorm backward's row kernel spends its time, from the block
    timeline hook (kp_debug_block_trace): each of `calls` calls, amid
    untraced back-to-back calls, records every row block's start, the end of
    its rows and the store of its weight-gradient partial row (constant 100
    MHz clock), and the kernel's own start and end (HIP events stamped by the
    launch, the hook of measure_gpu).  Per call: rows_done_us (median / max
    over blocks, from the first block's start), tail_us = max - median,
    partial_us (the last partial row stored), launch_drain_us = kernel time
    minus the blocks' span (dispatch before the first block, completion after
    the last).  Each field is the median over the calls."""
    import statistics
    import torch
    from kernelproblems_amd import _lib as L
    lib = L.lib()
    if not getattr(wl, "timeline", False):
        return None
    nb = 4096
    bufs = [torch.zeros(nb * 4, dtype=torch.int64, device=wl.dev) for _ in range(calls)]
    ev = StampEvents(calls)
    warm_device(wl.dev)
    i = 0
    for c in range(calls):
        for _ in range(warmup):
            wl.step(i)
            i += 1
        lib.kp_debug_block_trace(bufs[c].data_ptr(), nb * 32)
        lib.kp_profile_dominant_kernel(ev.start(c), ev.stop(c))
        wl.step(i)
        i += 1
        lib.kp_profile_dominant_kernel(None, None)
        lib.kp_debug_block_trace(None, 0)
    torch.cuda.synchronize()
    per = []
    for c in range(calls):
        rec = bufs[c].view(nb, 4).cpu().tolist()
        rec = [r for r in rec if r[0] != 0]
        t0 = min(r[0] for r in rec)
        rows = sorted((r[1] - t0) / 100.0 for r in rec)
        ends = [(r[2] - t0) / 100.0 for r in rec]
        kernel_us = ev.ms(c) * 1e3
        xcc = {}
        for r in rec:
            xcc.setdefault(int(r[3]), []).append((r[1] - t0) / 100.0)
        med = statistics.median(rows)
        per.append({
            "blocks": len(rec),
            "start_spread_us": (max(r[0] for r in rec) - t0) / 100.0,
            "rows_done_median_us": med,
            "rows_done_max_us": rows[-1],
            "tail_us": rows[-1] - med,
            "partial_stored_max_us": max(ends),
            "kernel_us": kernel_us,
            "launch_drain_us": kernel_us - max(ends),
            "rows_done_mean_by_xcc_us": {str(k): statistics.mean(v) for k, v in sorted(xcc.items())},
        })
    out = {k: round(statistics.median(p[k] for p in per), 2) for k in per[0] if k != "rows_done_mean_by_xcc_us"}
    out["rows_done_mean_by_xcc_us"] = {k: round(statistics.median(p["rows_done_mean_by_xcc_us"][k] for p in per), 2)
                                       for k in per[0]["rows_done_mean_by_xcc_us"]}
    out["calls"] = calls
    ev.close()
    return out


def measure_dropin(wl, steps, warmup):
    """The tensor-level drop-in (fused.*) on the same rotating inputs: what a
    caller of the reference's boundary pays per call, with outputs and
    workspace allocated by torch's caching allocator on every call, shape
    checks and the ctypes marshalling included.  us_per_call is the sustained
    wall time over K calls (synchronised on both sides); host_us_per_call is
    the Python time until each call returns (no synchronisation: launches are
    asynchronous), i.e. the host cost the GPU hides while it is longer than
    the kernels."""
    import torch
    if not wl.dropins:
        return None
    for i in range(warmup):
        wl.dropin(i)
    torch.cuda.synchronize()
    host = 0.0
    w0 = time.perf_counter()
    for i in range(steps):
        t = time.perf_counter()
        wl.dropin(warmup + i)
        host += time.perf_counter() - t
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    return {"entry": wl.dropin_entry, "us_per_call": round(wall * 1e6 / steps, 3),
            "host_us_per_call": round(host * 1e6 / steps, 3)}


# Probe schedules: chunks per thread x store policy (kp_stream_probe); the
# fastest for a workload's byte mix is its streaming ceiling.
PROBE_TILES = (1, 2, 4, 8)
PROBE_POLICIES = (0, 1)  # KP_STORE_NONTEMPORAL, KP_STORE_WRITE_THROUGH
PROBE_POLICY_NAMES = {0: "nt", 1: "write-through"}


def measure_probe(wl, steps, warmup):
    """The streaming ceiling of the workload's byte mix: kp_stream_probe over
    fresh arrays of the same sizes holding random bf16 values (rotated past
    the Infinity Cache like the workload's own), timed per launch like the
    dominant kernel, under every schedule of PROBE_TILES x PROBE_POLICIES;
    the fastest is the ceiling."""
    import torch
    from kernelproblems_amd import _lib as L
    if wl.probe_mix is None:
        return None
    n_in, n_out, in_b, out_b, text = wl.probe_mix
    lib = L.lib()
    stream = torch.cuda.current_stream(wl.dev).cuda_stream
    per_set = n_in * in_b + n_out * out_b
    R = max(2, math.ceil(MIN_ROTATION_BYTES / per_set))
    sets = []
    for _ in range(R):
        ins = [torch.empty(in_b, dtype=torch.uint8, device=wl.dev) for _ in range(n_in)]
        outs = [torch.empty(out_b, dtype=torch.uint8, device=wl.dev) for _ in range(n_out)]
        for t in ins:  # random bf16 values like the workloads' N(0, 1) data (bit toggling costs HBM time)
            t.view(torch.bfloat16).normal_()
        sets.append((L.ptr_array([t.data_ptr() for t in ins]), L.ptr_array([t.data_ptr() for t in outs]), ins, outs))

    def launch(i, schedule):
        per_thread, policy = schedule
        ip, op, _, _ = sets[i % R]
        st = lib.kp_stream_probe(ip, n_in, in_b, op, n_out, out_b, per_thread, policy, stream)
        if st != 0:
            raise L.KPError("kp_stream_probe", st, lib.kp_last_error_message().decode())

    per_tile = {}
    for per_thread in PROBE_TILES:
      for policy in PROBE_POLICIES:
        sched = (per_thread, policy)
        for i in range(warmup):
            launch(i, sched)
        ev = StampEvents(steps)
        torch.cuda.synchronize()
        for i in range(steps):
            lib.kp_profile_dominant_kernel(ev.start(i), ev.stop(i))
            launch(warmup + i, sched)
        lib.kp_profile_dominant_kernel(None, None)
        torch.cuda.synchronize()
        per_tile[sched] = sum(ev.ms(i) for i in range(steps)) / steps
        ev.close()
    del sets
    torch.cuda.empty_cache()
    best = min(per_tile, key=per_tile.get)
    ms = per_tile[best]
    return {"GBps": per_set / (ms * 1e-3) / 1e9, "us": ms * 1e3, "mix": text, "bytes": per_set,
            "chunks_per_thread": best[0], "stores": PROBE_POLICY_NAMES[best[1]],
            "us_by_schedule": {f"{k[0]}/{PROBE_POLICY_NAMES[k[1]]}": round(v * 1e3, 3) for k, v in per_tile.items()}}


def measure_vendor(wl, steps, warmup):
    """torch-ROCm's own elementwise kernels on the workload's byte mix, as a
    ceiling written by someone else: 1 read + 1 write of equal size ->
    copy_, 2 reads + 1 write -> add(out=), 3 reads + 1 write ->
    addcmul(out=), a pure write (an fp32 table) -> zero_(); random bf16
    inputs rotated past the Infinity Cache, each op timed by events on the
    stream it runs on.  None for mixes with no single torch op."""
    import torch
    if wl.probe_mix is None:
        return None
    n_in, n_out, in_b, out_b, _ = wl.probe_mix
    if n_out != 1:
        return None
    if in_b == out_b and n_in in (1, 2, 3):
        op = {1: "copy_", 2: "add(out=)", 3: "addcmul(out=)"}[n_in]
        per_set, numel = (n_in + 1) * in_b, in_b // 2
    elif n_in == 1 and out_b > 8 * in_b:  # the embedding backward: the dense fp32 table dominates
        op, per_set, numel = "zero_() of the fp32 output", out_b, out_b // 4
    else:
        return None
    R = max(2, math.ceil(MIN_ROTATION_BYTES / per_set))
    sets = []
    for _ in range(R):
        if op.startswith("zero_"):
            sets.append((torch.empty(numel, dtype=torch.float32, device=wl.dev),))
            continue
        ins = [torch.empty(numel, dtype=torch.bfloat16, device=wl.dev).normal_() for _ in range(n_in)]
        sets.append((torch.empty(numel, dtype=torch.bfloat16, device=wl.dev), *ins))

    def launch(i):
        t = sets[i % R]
        if op.startswith("zero_"):
            t[0].zero_()
        elif n_in == 1:
            t[0].copy_(t[1])
        elif n_in == 2:
            torch.add(t[1], t[2], out=t[0])
        else:
            torch.addcmul(t[1], t[2], t[3], out=t[0])

    for i in range(warmup):
        launch(i)
    ev = StampEvents(steps)
    stream = torch.cuda.current_stream(wl.dev).cuda_stream
    torch.cuda.synchronize()
    for i in range(steps):
        ev.record(ev.start(i), stream)
        launch(warmup + i)
        ev.record(ev.stop(i), stream)
    torch.cuda.synchronize()
    ms = sum(ev.ms(i) for i in range(steps)) / steps
    ev.close()
    del sets
    torch.cuda.empty_cache()
    return {"op": f"torch {op}", "us": round(ms * 1e3, 3), "bytes": per_set,
            "GBps": round(per_set / (ms * 1e-3) / 1e9, 1), "frac_of_peak": round(per_set / (ms * 1e-3) / 1e9 / PEAK_GBS, 4)}


def _tensors(x):
    return [t for y in x for t in _tensors(y)] if isinstance(x, (tuple, list)) else [x]


def _view_bytes(ts):
    """Bytes of each distinct tensor view (a view is counted once even when
    passed twice; an output returned as several views of one storage counts
    once)."""
    seen, total = set(), 0
    for t in ts:
        key = (t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), tuple(t.stride()))
        if key not in seen:
            seen.add(key)
            total += t.numel() * t.element_size()
    return total


# The canonical drop-in of each hot-path fragment family, timed at its
# reference shape in every default run (--fragments times all of them).
CORE_FRAGMENTS = (
    "v7/59f786beb25f",  # RMSNorm forward, y + rstd
    "v7/215dd2e6a519",  # RMSNorm forward, strided FSDP weight view
    "v8/7884328a5557",  # residual add + RMSNorm forward
    "v7/45990c83cfd6",  # RMSNorm backward, dw to fp32
    "v8/d8f596b3df34",  # gradient adds -> RMSNorm backward -> residual add
    "v8/3c6c589cdf81",  # residual add recomputed + RMSNorm backward
    "v7/1e49beb8a123",  # embedding forward from a flat-buffer table
    "v7/a12a160cb11b",  # embedding dense backward -> fp32
    "v7/e29b92927600",  # RoPE forward (interleaved, table)
    "v8/c8c60d8f7015",  # RoPE q + k forward with the position gather
    "v7/5c65f62b0422",  # RoPE backward (conjugate table)
    "v6/0b493aad68f0",  # chain: RMSNorm forward + backward -> embedding backward
)


def measure_fragments(dev, steps, warmup, ids=None):
    """Fragment drop-ins (kernelproblems_amd.fragments) at their reference
    shapes -- `ids`, or every distinct one: kernel_function on rotating
    get_inputs sets (>= 1 GiB of inputs or 2 sets), K calls timed with
    synchronisation on both sides.  moved_bytes = every input view and every
    distinct output once (an upper bound where a fragment reads part of an
    input, e.g. the y of a saved (y, rstd) tuple).  ref = the reference's own
    record of the fragment (its eager time and fastest passing candidate on
    its H100), where it has one."""
    import torch
    from kernelproblems_amd import fragments as fr
    try:
        ref = json.loads((ROOT / "tests" / "golden" / "reference_times.json").read_text())
    except (OSError, ValueError):
        ref = {}
    out = {}
    if ids is None:
        ids = [f for f in fr.FRAGMENTS if f not in fr.SAME_AS and f not in fr.EQUIVALENT]
    for fid in ids:
        mod = fr.load(fid)
        first = mod.get_inputs(device=dev, generator=torch.Generator(device=dev).manual_seed(1))
        in_b = _view_bytes(_tensors(first))
        R = max(2, min(8, math.ceil(MIN_ROTATION_BYTES / max(in_b, 1))))
        sets = [first] + [mod.get_inputs(device=dev, generator=torch.Generator(device=dev).manual_seed(i + 2))
                          for i in range(R - 1)]
        res = mod.kernel_function(*sets[0])
        out_b = _view_bytes(_tensors(res))
        del res
        for i in range(warmup):
            mod.kernel_function(*sets[i % R])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            mod.kernel_function(*sets[i % R])
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) * 1e6 / steps
        gbs = (in_b + out_b) / us / 1e3
        rec = {"us_per_call": round(us, 2), "moved_bytes": in_b + out_b,
               # a gather reads only some rows of the table / flat buffer it is
               # given: there moved_bytes overstates the traffic, and no rate
               "GBps": round(gbs, 1) if gbs <= PEAK_GBS else None}
        r = ref.get(fid)
        if r:
            rec["ref"] = r
        out[fid] = rec
        print(f"[bench] fragment {fid}: {us:.1f} us/call, {(in_b + out_b) / 1e6:.1f} MB moved"
              + (f"; reference best {r['best_ms'] * 1e3:.1f} us ({r['best_backend']}), eager "
                 f"{r.get('eager_ms', float('nan')) * 1e3:.1f} us on its H100" if r and "best_ms" in r else ""),
              file=sys.stderr, flush=True)
        del sets, first
        torch.cuda.empty_cache()
    return out


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def measure_cpu(wl, seconds):
    import torch
    wl.cpu_run()  # warm-up
    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        wl.cpu_run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all >= seconds or len(times) >= 500:
            break
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": (wl.cpu_bytes or wl.bytes_per_call) / med / 1e9,
        "unit": "GB/s",
        "ms_per_call": med * 1e3,
        "cores": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": (f"torch CPU eager restatement of the fragment (oracle/torch_ref.py), {wl.cpu_sample}, "
                   f"median of {len(times)} timed calls after 1 warm-up"),
    }


def _ceiling_json(r):
    c = r.get("ceiling")
    if not c:
        return None
    return {"GBps": round(c["GBps"], 1), "frac_of_peak": round(c["GBps"] / PEAK_GBS, 4), "probe_us": round(c["us"], 3),
            "probe_schedule": f"{c['chunks_per_thread']} chunk(s) per thread, {c['stores']} stores",
            "probe_us_by_schedule": c["us_by_schedule"], "mix": c["mix"],
            "kernel_frac_of_ceiling": round(r["achieved"] / c["GBps"], 4), "vendor": c.get("vendor")}


def load_traffic(name):
    p = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(p.read_text()).get(name)
    except (OSError, ValueError):
        return None


def measure_probe_sizes(dev, steps, warmup):
    """Streaming time against size: kp_stream_probe (the fastest of its eight
    schedules) for a copy, 2 reads + 1 write and 2 reads + 2 writes of 4 MiB
    to 256 MiB arrays of random bf16 values, rotated past the Infinity Cache,
    timed as K back-to-back launches; a least-squares fit of
    t = fixed + bytes / rate over the sizes from 16 MiB says how much of a
    small launch is ramp and drain rather than bandwidth."""
    import torch
    from kernelproblems_amd import _lib as L
    lib = L.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def best(n_in, n_out, nbytes):
        R = max(2, math.ceil(MIN_ROTATION_BYTES / ((n_in + n_out) * nbytes)))
        sets = []
        for _ in range(R):
            ins = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_in)]
            outs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_out)]
            for t in ins:
                t.view(torch.bfloat16).normal_()
            sets.append((L.ptr_array([t.data_ptr() for t in ins]), L.ptr_array([t.data_ptr() for t in outs]), ins, outs))
        times = {}
        for per_thread in PROBE_TILES:
            for policy in PROBE_POLICIES:
                def launch(i):
                    ip, op, _, _ = sets[i % R]
                    st = lib.kp_stream_probe(ip, n_in, nbytes, op, n_out, nbytes, per_thread, policy, stream)
                    if st != 0:
                        raise L.KPError("kp_stream_probe", st, lib.kp_last_error_message().decode())
                for i in range(warmup):
                    launch(i)
                torch.cuda.synchronize()
                e0.record()
                for i in range(steps):
                    launch(i)
                e1.record()
                torch.cuda.synchronize()
                times[(per_thread, policy)] = e0.elapsed_time(e1) * 1e3 / steps
        del sets
        torch.cuda.empty_cache()
        k = min(times, key=times.get)
        return times[k], k

    out = {}
    for n_in, n_out, name in ((1, 1, "copy"), (2, 1, "2 reads + 1 write"), (2, 2, "2 reads + 2 writes")):
        pts = []
        for mib in (4, 8, 16, 32, 64, 128, 256):
            us, k = best(n_in, n_out, mib << 20)
            total = (n_in + n_out) * (mib << 20)
            pts.append({"MiB_per_array": mib, "bytes": total, "us": round(us, 3), "GBps": round(total / us / 1e3, 1),
                        "schedule": f"{k[0]}/{PROBE_POLICY_NAMES[k[1]]}"})
            print(f"[bench] probe {name}, {mib} MiB per array: {us:.2f} us", file=sys.stderr, flush=True)
        xs = [p["bytes"] for p in pts if p["MiB_per_array"] >= 16]
        ys = [p["us"] for p in pts if p["MiB_per_array"] >= 16]
        mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
        slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        out[name] = {"points": pts, "fit_fixed_us": round(my - slope * mx, 3), "fit_GBps": round(1e-3 / slope, 1)}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c2", choices=ALL, help="the headline workload (top-level fields)")
    ap.add_argument("--solo", action="store_true",
                    help="measure the headline workload only (profiling runs); by default every BASELINE "
                         "configuration (c1, c2, c3f, c3b, c4, c5f, c5b) gets a block under 'configs'")
    ap.add_argument("--all", action="store_true", help="also measure every other workload (no CPU baseline)")
    ap.add_argument("--fragments", action="store_true",
                    help="time every distinct fragment drop-in at its reference shape (by default only the "
                         "canonical drop-in of each family, CORE_FRAGMENTS)")
    ap.add_argument("--no-fragments", action="store_true", help="time no fragment drop-ins")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-probe", action="store_true", help="skip the streaming-ceiling probe")
    ap.add_argument("--no-dropin", action="store_true", help="skip timing the tensor-level drop-ins")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU baseline budget per configuration")
    ap.add_argument("--probe-sizes", action="store_true",
                    help="instead of the workloads: streaming time against array size (fixed cost + rate fit)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after the workload, run 5 plain device copies of this many MiB (a known-size "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every kernel runs on one GPU's rows; sharding would split tokens across ranks with the "
              "weight-gradient sum as the only collective)", file=sys.stderr)
        return 2

    import torch
    import kernelproblems_amd as kp  # noqa: F401  (loads libkp_hip.so; raises if it is missing)

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.probe_sizes:
        print(json.dumps({"probe_sizes": measure_probe_sizes(dev, args.steps, args.warmup)}), flush=True)
        return 0

    def run(name, with_cpu):
        print(f"[bench] preparing {name}", file=sys.stderr, flush=True)
        wl = make_workload(name, dev)
        r = measure_gpu(wl, args.steps, args.warmup)
        print(f"[bench] {name}: {r['ms_per_step'] * 1e3:.1f} us/call, {r['value']:.0f} GB/s, dominant kernel "
              f"{r['dominant_ms'] * 1e3:.1f} us -> {r['achieved']:.0f} GB/s", file=sys.stderr, flush=True)
        # With few steps the timed loop's fixed cost (the first launch's latency and the closing
        # synchronisation, ~20 us) is spread over few calls; a second, longer pass gives the
        # steady per-call time beside it.
        r["steady"] = None
        if args.steps < STEADY_STEPS:
            st = measure_gpu(wl, STEADY_STEPS, args.warmup)
            r["steady"] = {"steps": STEADY_STEPS, "us_per_call": round(st["ms_per_step"] * 1e3, 3),
                           "GBps": round(st["value"], 1), "kernel_us": round(st["dominant_ms"] * 1e3, 3)}
        r["timeline"] = measure_timeline(wl)
        if r["timeline"]:
            t = r["timeline"]
            print(f"[bench] {name}: block timeline (median of {t['calls']} calls): rows done median "
                  f"{t['rows_done_median_us']:.1f} us, max {t['rows_done_max_us']:.1f} us (tail {t['tail_us']:.1f}), "
                  f"partial rows stored {t['partial_stored_max_us']:.1f} us, kernel {t['kernel_us']:.1f} us "
                  f"(launch + drain {t['launch_drain_us']:.1f})", file=sys.stderr, flush=True)
        r["dropin"] = None if args.no_dropin else measure_dropin(wl, args.steps, args.warmup)
        if r["dropin"]:
            d = r["dropin"]
            print(f"[bench] {name}: drop-in {d['us_per_call']:.1f} us/call (host {d['host_us_per_call']:.1f} us)",
                  file=sys.stderr, flush=True)
        r["ceiling"] = None if args.no_probe else measure_probe(wl, args.steps, args.warmup)
        if r["ceiling"]:
            c = r["ceiling"]
            print(f"[bench] {name}: streaming ceiling of its mix ({c['mix']}): {c['us']:.1f} us at "
                  f"{c['chunks_per_thread']} chunk(s)/thread -> {c['GBps']:.0f} GB/s; "
                  f"dominant kernel at {r['achieved'] / c['GBps']:.1%} of it", file=sys.stderr, flush=True)
            c["vendor"] = measure_vendor(wl, args.steps, args.warmup)
            if c["vendor"]:
                v = c["vendor"]
                print(f"[bench] {name}: {v['op']} on the same mix: {v['us']:.1f} us -> {v['GBps']:.0f} GB/s",
                      file=sys.stderr, flush=True)
        cpu = None
        if with_cpu:
            print(f"[bench] cpu baseline {name}", file=sys.stderr, flush=True)
            cpu = measure_cpu(wl, args.cpu_seconds)
            print(f"[bench] {name}: cpu {cpu['ms_per_call']:.1f} ms/call ({cpu['cores']} threads)",
                  file=sys.stderr, flush=True)
        wl.sets.clear()
        wl.dropins.clear()
        torch.cuda.empty_cache()
        return wl, r, cpu

    def roofline(name, wl, r):
        out = {
            "bound": "hbm",
            "achieved": round(r["achieved"], 2),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["achieved"] / PEAK_GBS, 4),
            "traffic": load_traffic(name),
            "kernel": wl.dominant_kernel,
            "kernel_us": round(r["dominant_ms"] * 1e3, 3),
            "kernel_bytes": wl.dominant_bytes,
            "ceiling": _ceiling_json(r),
        }
        ub = getattr(wl, "unique_row_bytes", None)
        if ub:
            # a gather: the least HBM traffic (distinct rows once), its rate and fraction of peak
            gbs = ub / r["dominant_ms"] / 1e6
            out["unique_rows"] = {"bytes": ub, "GBps": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        return out

    def block(name, wl, r, cpu):
        return {
            "workload": wl.description,
            "us_per_call": round(r["ms_per_step"] * 1e3, 3),
            "GBps": round(r["value"], 1),
            "pct_of_peak": round(100 * r["value"] / PEAK_GBS, 2),
            "bytes_per_call": wl.bytes_per_call,
            "roofline": roofline(name, wl, r),
            "steady": r["steady"],
            "timeline": r["timeline"],
            "dropin": r["dropin"],
            "cpu_baseline": cpu,
        }

    names = [args.workload] if args.solo else [args.workload] + [c for c in CONFIGS if c != args.workload]
    configs = {}
    head = None
    for name in names:
        wl, r, cpu = run(name, not args.no_cpu)
        configs[name] = block(name, wl, r, cpu)
        if head is None:
            head = (wl, r, cpu)
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty(n, dtype=torch.uint8, device=dev)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copy calibration: 5 x {args.copy_calibration_mib} MiB device copies", file=sys.stderr, flush=True)
    wl, r, cpu = head
    line = {
        "metric": "achieved HBM GB/s and % of 8 TB/s peak per fragment; us/call vs CPU eager",
        "value": round(r["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": wl.description,
            "io_dtype": "bf16",
            "accumulate": "fp32",
            "algorithmic_bytes_per_call": wl.bytes_per_call,
            "gpu_ms_per_step": round(r["gpu_ms_per_step"], 6),
            "pct_of_hbm_peak": round(100 * r["value"] / PEAK_GBS, 2),
            "device": torch.cuda.get_device_name(dev),
        },
        "roofline": roofline(args.workload, wl, r),
        "cpu_baseline": cpu,
        "dropin": r["dropin"],
        "configs": configs,
    }
    if args.all:
        frags = {}
        for name in ALL:
            if name in configs:
                continue
            w2, r2, _ = run(name, False)
            frags[name] = {
                "workload": w2.description,
                "us_per_call": round(r2["ms_per_step"] * 1e3, 3),
                "GBps": round(r2["value"], 1),
                "pct_of_peak": round(100 * r2["value"] / PEAK_GBS, 2),
                "kernel": w2.dominant_kernel,
                "kernel_us": round(r2["dominant_ms"] * 1e3, 3),
                "kernel_GBps": round(r2["achieved"], 1),
                "kernel_bytes": w2.dominant_bytes,
                "ceiling": _ceiling_json(r2),
                "bytes_per_call": w2.bytes_per_call,
            }
            ub = getattr(w2, "unique_row_bytes", None)
            if ub:
                frags[name]["unique_rows"] = {"bytes": ub, "GBps": round(ub / r2["dominant_ms"] / 1e6, 1)}
        line["fragments"] = frags
    if args.fragments:
        line["fragment_drop_ins"] = measure_fragments(dev, args.steps, args.warmup)
    elif not args.no_fragments and not args.solo:
        line["fragment_drop_ins"] = measure_fragments(dev, args.steps, args.warmup, CORE_FRAGMENTS)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
