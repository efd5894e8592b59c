"""CPU oracle for the fused fragment kernels -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check or time against it.
The product path (``kernelproblems_amd``) never imports it.

Two independent restatements live here:

* ``kp_oracle.c`` (bound below with ctypes): scalar C, fp64 accumulation,
  the reference's rounding points (see the file header for the per-function
  citations of the reference and of torch's decompositions).
* ``torch_ref.py``: the reference fragments' aten op sequences restated as
  torch eager calls (CPU, or torch-ROCm on the GPU box).

Parity status of each function (how it is pinned; tests/test_oracle_*.py):

=====================  =====================================================
rmsnorm_fwd            torch CPU ``aten._fused_rms_norm`` (bit-equal y, rstd
                       within fp32 rounding), closed forms (constant row,
                       one-hot row), fp64 brute force.
rmsnorm_bwd            fp64 ``torch.autograd`` of ``F.rms_norm``, central
                       finite differences, the decomposition run by torch in
                       fp64, invariant sum_j xhat_j dx_j = 0 (w = 1).
bf16 add               torch CPU eager bf16 ``add`` (bit-equal).
embedding_fwd          ``torch.index_select`` (bit-equal).
embedding_bwd          fp64 ``index_add_``, column-sum invariant, padding
                       rows zero, ``scale_grad_by_freq`` closed form.
rope (table)           torch complex64 multiply (``view_as_complex``) as in
                       v8/c8c60d8f7015/problem.py:18-71.
rope (theta)           ``torch.polar`` angles in fp64 (pos = 0 identity, norm
                       preservation, conj inverse), rotate-half ==
                       interleaved up to the (2i, 2i+1) <-> (i, i + D/2)
                       permutation.
rope_c64               torch complex128 multiply (library), position 0 with
                       a unit table is the identity, unit-modulus rows keep
                       |x|, conj undoes the rotation.
swiglu_fwd             torch CPU eager ``silu`` * b, fp64 ``x * expit(x)``
                       (scipy), closed forms (silu(0) = 0, silu(x) -
                       silu(-x) = x, saturation), every bf16 input value.
swiglu_bwd             torch CPU eager ``mul`` / ``silu_backward``, central
                       finite differences of fp64 silu, closed forms
                       (silu'(0) = 1/2, the zero of silu' near -1.2785).
silu, swiglu_fwd_bwd   compositions of swiglu_fwd / swiglu_bwd; silu also
                       against torch CPU eager ``silu`` over every bf16 value.
cross_entropy_fwd      torch fp64 ``log_softmax`` + ``nll_loss`` (sum,
                       ignore_index), closed forms (uniform row: log V,
                       dominant logit: 0), shift invariance, ignored rows.
cross_entropy_fwd_bwd  fp64 autograd of the forward loss (one bf16 rounding,
                       bit-equal), cross_entropy_bwd of the fp64 log-softmax.
cross_entropy_bwd      torch fp64 ``nll_loss_backward`` +
                       ``_log_softmax_backward_data`` (bit-exact after one
                       rounding), the autograd of the forward, rows summing
                       to zero for a true log-softmax, ignored rows zero.
=====================  =====================================================

bf16 tensors are handled as numpy ``uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libkp_oracle.so"

_lib = None

vp, i64, i32, f32, f64 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_double
pvp, pi64 = C.POINTER(C.c_void_p), C.POINTER(C.c_int64)

_SIGS = {
    "kpo_bf16_from_f32": (None, [vp, vp, i64]),
    "kpo_bf16_from_f64": (None, [vp, vp, i64]),
    "kpo_bf16_add": (None, [vp, vp, vp, i64]),
    "kpo_rmsnorm_fwd": (i32, [pvp, pi64, i32, vp, i64, i64, vp, vp, vp, i64, i64, f32]),
    "kpo_rmsnorm_bwd": (i32, [pvp, pi64, i32, pvp, pi64, i32, vp, vp, i64, i64, vp, vp, vp, vp, i64, i64, f32]),
    "kpo_embedding_fwd": (i64, [vp, i64, i64, i64, vp, i64, vp]),
    "kpo_embedding_bwd_rows": (i64, [vp, i64, vp, i64, i64, i64, i64, i32, vp, vp, vp, vp, vp]),
    "kpo_embedding_bwd_dense": (i64, [vp, i64, vp, i64, i64, i64, i64, i32, i32, vp]),
    "kpo_rope": (i64, [vp, pi64, vp, pi64, i64, i64, i64, i64, vp, i64, i64, i32, f64, vp, i64, i64, i32]),
    "kpo_swiglu_fwd": (None, [vp, vp, vp, i64]),
    "kpo_swiglu_bwd": (None, [vp, vp, vp, vp, vp, vp, i64]),
    "kpo_cross_entropy_fwd": (i64, [vp, i64, i64, vp, i64, f64, vp, vp, vp]),
    "kpo_cross_entropy_bwd": (i64, [vp, i64, i64, vp, i64, f64, vp]),
    "kpo_cross_entropy_fwd_bwd": (i64, [vp, i64, i64, vp, i64, f64, vp]),
}


def build() -> Path:
    """Compiles kp_oracle.c with the committed Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- bf16
def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    src = _c(a, np.float32)
    out = np.empty(src.shape, dtype=np.uint16)
    lib().kpo_bf16_from_f32(_p(src), _p(out), src.size)
    return out


def f64_to_bf16(a: np.ndarray) -> np.ndarray:
    src = _c(a, np.float64)
    out = np.empty(src.shape, dtype=np.uint16)
    lib().kpo_bf16_from_f64(_p(src), _p(out), src.size)
    return out


def bf16_add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _c(a, np.uint16), _c(b, np.uint16)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().kpo_bf16_add(_p(a), _p(b), _p(out), a.size)
    return out


# ---------------------------------------------------------------- RMSNorm
def _terms(terms: Sequence[np.ndarray], n: int):
    arrs = [_c(t, np.uint16).reshape(-1, n) for t in terms]
    ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    strides = (C.c_int64 * len(arrs))(*([n] * len(arrs)))
    return arrs, ptrs, strides


def _wseg(w: Optional[np.ndarray], n: int, seg):
    if w is None:
        return None, n, n
    w = _c(w, np.uint16)
    if seg is None:
        return w.reshape(-1), n, n
    return w.reshape(-1), int(seg[0]), int(seg[1])


def rmsnorm_fwd(x_terms: Sequence[np.ndarray], w: Optional[np.ndarray], eps: float, n: int, w_seg=None):
    """-> (h uint16 [M, n], y uint16 [M, n], rstd float32 [M]); h is the bf16
    running sum of the terms.  w_seg=(seg_len, seg_stride) addresses a
    segmented weight buffer (element i at (i // len) * stride + i % len)."""
    arrs, ptrs, strides = _terms(x_terms, n)
    m = arrs[0].shape[0]
    wa, sl, ss = _wseg(w, n, w_seg)
    h = np.empty((m, n), np.uint16)
    y = np.empty((m, n), np.uint16)
    rstd = np.empty(m, np.float32)
    st = lib().kpo_rmsnorm_fwd(ptrs, strides, len(arrs), _p(wa), sl, ss, _p(h), _p(y), _p(rstd), m, n, eps)
    if st != 0:
        raise RuntimeError(f"kpo_rmsnorm_fwd failed ({st})")
    return h, y, rstd


def rmsnorm_bwd(dy_terms, x_terms, rstd: Optional[np.ndarray], w: Optional[np.ndarray], eps: float, n: int,
                dx_residual: Optional[np.ndarray] = None, w_seg=None):
    """-> (dx uint16 [M, n], dw float64 [n], rstd float32 [M] used)."""
    dya, dyp, dys = _terms(dy_terms, n)
    xa, xp, xs = _terms(x_terms, n)
    m = xa[0].shape[0]
    wa, sl, ss = _wseg(w, n, w_seg)
    r_in = None if rstd is None else _c(rstd, np.float32).reshape(-1)
    res = None if dx_residual is None else _c(dx_residual, np.uint16).reshape(m, n)
    dx = np.empty((m, n), np.uint16)
    dw = np.empty(n, np.float64)
    r_out = np.empty(m, np.float32)
    st = lib().kpo_rmsnorm_bwd(dyp, dys, len(dya), xp, xs, len(xa), _p(r_in), _p(wa), sl, ss, _p(res), _p(dx),
                               _p(dw), _p(r_out), m, n, eps)
    if st != 0:
        raise RuntimeError(f"kpo_rmsnorm_bwd failed ({st})")
    return dx, dw, r_out


# ---------------------------------------------------------------- embedding
def embedding_fwd(table: np.ndarray, idx: np.ndarray):
    """-> (out uint16 [T, D], number of out-of-range ids)."""
    table = _c(table, np.uint16)
    V, D = table.shape
    ids = _c(idx, np.int64).reshape(-1)
    out = np.empty((ids.size, D), np.uint16)
    bad = lib().kpo_embedding_fwd(_p(table), V, D, D, _p(ids), ids.size, _p(out))
    return out, int(bad)


def embedding_bwd_rows(grad: np.ndarray, idx: np.ndarray, V: int, padding_idx: int = -1, scale: bool = False):
    """-> (ids int64 [U], rows float64 [U, D], absrows float64 [U, D],
    counts int64 [U], number of out-of-range ids).  Rows not listed are 0."""
    ids_in = _c(idx, np.int64).reshape(-1)
    T = ids_in.size
    g = _c(grad, np.uint16).reshape(T, -1) if T else _c(grad, np.uint16).reshape(0, grad.shape[-1])
    D = g.shape[1]
    cap = max(T, 1)
    ids = np.empty(cap, np.int64)
    rows = np.empty((cap, D), np.float64)
    absrows = np.empty((cap, D), np.float64)
    counts = np.empty(cap, np.int64)
    nr = C.c_int64(0)
    bad = lib().kpo_embedding_bwd_rows(_p(g), D, _p(ids_in), T, V, D, -1 if padding_idx is None else padding_idx,
                                       int(scale), _p(ids), _p(rows), _p(absrows), _p(counts), C.addressof(nr))
    if bad < 0:
        raise MemoryError("kpo_embedding_bwd_rows")
    k = nr.value
    return ids[:k], rows[:k], absrows[:k], counts[:k], int(bad)


def embedding_bwd_dense(grad: np.ndarray, idx: np.ndarray, V: int, padding_idx: int = -1, scale: bool = False,
                        round_bf16: bool = False) -> np.ndarray:
    ids_in = _c(idx, np.int64).reshape(-1)
    T = ids_in.size
    g = _c(grad, np.uint16).reshape(T, -1)
    D = g.shape[1]
    out = np.empty((V, D), np.float32)
    bad = lib().kpo_embedding_bwd_dense(_p(g), D, _p(ids_in), T, V, D, -1 if padding_idx is None else padding_idx,
                                        int(scale), int(round_bf16), _p(out))
    if bad < 0:
        raise MemoryError("kpo_embedding_bwd_dense")
    return out


# ---------------------------------------------------------------- RoPE
def rope(x: np.ndarray, pos: Optional[np.ndarray] = None, *, pairing: str = "half", theta: float = 10000.0,
         freqs: Optional[np.ndarray] = None, conj: bool = False) -> np.ndarray:
    """x uint16 [B, S, H, D] contiguous; pos int64 [B, S] or [S] (default s);
    freqs complex64 [P, D/2] (table mode) or None (theta mode)."""
    x = _c(x, np.uint16)
    B, S, H, D = x.shape
    xs = (C.c_int64 * 3)(S * H * D, H * D, D)
    out = np.empty_like(x)
    pp, psb, pss = None, 0, 0
    if pos is not None:
        pa = _c(pos, np.int64)
        if pa.ndim == 1:
            psb, pss = 0, 1
        else:
            psb, pss = (pa.shape[1] if pa.shape[0] == B else 0), 1
        pp = pa
    fa, frows, frs = None, 0, 0
    if freqs is not None:
        fc = np.ascontiguousarray(freqs, dtype=np.complex64).reshape(-1, D // 2)
        fa = fc.view(np.float32)
        frows, frs = fc.shape[0], D // 2
    mode = 0 if pairing == "half" else 1
    bad = lib().kpo_rope(_p(x), xs, _p(out), xs, B, S, H, D, _p(pp), psb, pss, mode, float(theta), _p(fa), frows,
                         frs, int(conj))
    if bad < 0:
        raise MemoryError("kpo_rope")
    return out


def rope_c64(x: np.ndarray, table: np.ndarray, positions=None, conj: bool = False) -> np.ndarray:
    """Complex RoPE of the v1 captures (v1/075cb40f3d5d/problem.py:14-23):
    x complex [B, S, H, P] times table[p] (p = positions[b, s], default s),
    conjugated on request, in complex128 (exact products of the complex64
    inputs, one rounding per component)."""
    x = np.asarray(x).astype(np.complex128)
    t = np.asarray(table).astype(np.complex128).reshape(-1, x.shape[-1])
    B, S = x.shape[:2]
    p = np.broadcast_to(np.arange(S), (B, S)) if positions is None else np.broadcast_to(np.asarray(positions), (B, S))
    rows = t[p]  # [B, S, P]
    if conj:
        rows = np.conj(rows)
    return x * rows[:, :, None, :]


# ---------------------------------------------------------------- SwiGLU
def swiglu_fwd(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """bf16(bf16(silu(a)) * b) elementwise; uint16 arrays of one shape."""
    a, b = _c(a, np.uint16), _c(b, np.uint16)
    if a.shape != b.shape:
        raise ValueError("swiglu_fwd: a and b differ in shape")
    out = np.empty_like(a)
    lib().kpo_swiglu_fwd(_p(a), _p(b), _p(out), a.size)
    return out


def swiglu_bwd(g: np.ndarray, s: np.ndarray, b: np.ndarray, a: np.ndarray):
    """(db, da) = (bf16(g * s), bf16(silu_backward(bf16(g * b), a))); uint16 arrays of one shape."""
    arrs = [_c(t, np.uint16) for t in (g, s, b, a)]
    if any(t.shape != arrs[0].shape for t in arrs):
        raise ValueError("swiglu_bwd: operands differ in shape")
    db, da = np.empty_like(arrs[0]), np.empty_like(arrs[0])
    lib().kpo_swiglu_bwd(*(_p(t) for t in arrs), _p(db), _p(da), arrs[0].size)
    return db, da


def silu(a: np.ndarray) -> np.ndarray:
    """bf16(silu(a)) (v7/58e7a4d6cde3/problem.py:10-19): swiglu_fwd with b = 1,
    since bf16(s * 1) = s for a bf16 s."""
    a = _c(a, np.uint16)
    return swiglu_fwd(a, np.full_like(a, 0x3F80))


def swiglu_fwd_bwd(a: np.ndarray, b: np.ndarray, g: np.ndarray):
    """(h, db, da) of v6/182d2dcd0652/problem.py:10-46: h = swiglu_fwd(a, b) and
    swiglu_bwd(g, silu(a), b, a), the two restated ops composed."""
    h = swiglu_fwd(a, b)
    db, da = swiglu_bwd(g, silu(a), b, a)
    return h, db, da


# ---------------------------------------------------------------- cross-entropy
def cross_entropy_fwd(logits: np.ndarray, targets: np.ndarray, ignore_index: int = -100, scale: float = 1.0):
    """logits uint16 bf16 [M, V]; targets int [M].  Returns (loss, total_weight,
    lse [M], n_out_of_range) in float64: loss = scale * sum over non-ignored
    rows of (lse_i - x_{i, t_i})."""
    x = _c(logits, np.uint16)
    M, V = x.shape
    t = _c(targets, np.int64).reshape(M)
    loss, tw = C.c_double(), C.c_double()
    lse = np.empty(M, dtype=np.float64)
    bad = lib().kpo_cross_entropy_fwd(_p(x), M, V, _p(t), int(ignore_index), float(scale), C.byref(loss), C.byref(tw),
                                      _p(lse))
    return loss.value, tw.value, lse, int(bad)


def cross_entropy_bwd(log_softmax: np.ndarray, targets: np.ndarray, grad_loss: float, ignore_index: int = -100):
    """bf16 (uint16) [M, V] = grad - exp(L) * sum(grad) for the nll (sum) gradient
    grad = -grad_loss at each row's target; returns (out, n_out_of_range)."""
    L = _c(log_softmax, np.float32)
    M, V = L.shape
    t = _c(targets, np.int64).reshape(M)
    out = np.empty((M, V), dtype=np.uint16)
    bad = lib().kpo_cross_entropy_bwd(_p(L), M, V, _p(t), int(ignore_index), float(grad_loss), _p(out))
    return out, int(bad)


def cross_entropy_fwd_bwd(logits: np.ndarray, targets: np.ndarray, grad_loss: float, ignore_index: int = -100):
    """The logits gradient of grad_loss * (sum over non-ignored rows of
    lse_i - x_{i, t_i}) straight from the bf16 logits (uint16 [M, V]):
    bf16 of grad - exp(x - lse) * sum(grad), in double.  Returns
    (out, n_out_of_range)."""
    x = _c(logits, np.uint16)
    M, V = x.shape
    t = _c(targets, np.int64).reshape(M)
    out = np.empty((M, V), dtype=np.uint16)
    bad = lib().kpo_cross_entropy_fwd_bwd(_p(x), M, V, _p(t), int(ignore_index), float(grad_loss), _p(out))
    return out, int(bad)
