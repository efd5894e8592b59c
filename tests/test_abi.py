"""The C ABI without a GPU: include/kp.h, the ctypes table in
kernelproblems_amd/_lib.py and the exports of libkp_hip.so agree one for
one, and argument validation returns its error codes (with a message)
before anything touches a device."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from kernelproblems_amd import _lib as L

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kp.h"
_DECL = re.compile(r"^(?:int|size_t|const char\*|void)\s+(kp_\w+)\(([^;]*?)\);", re.M | re.S)


def _declarations():
    text = HEADER.read_text()
    out = {}
    for name, params in _DECL.findall(text):
        params = " ".join(params.split())
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    if not L.LIB_PATH.exists():
        from kernelproblems_amd import build
        build.build()
    return L.lib()


def test_header_matches_ctypes_table():
    decl = _declarations()
    assert decl, "no declarations parsed"
    assert set(decl) == set(L.SIGNATURES), set(decl) ^ set(L.SIGNATURES)
    for name, n in decl.items():
        assert len(L.SIGNATURES[name][1]) == n, f"{name}: header has {n} parameters"


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(L.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    missing = set(_declarations()) - exported
    assert not missing, missing
    for name in _declarations():
        assert getattr(lib, name) is not None


def test_version(lib):
    assert "gfx950" in L.version()


def _expect(lib, status, fn, *args):
    st = getattr(lib, fn)(*args)
    assert st == status, (fn, st, lib.kp_last_error_message())
    assert fn.encode() in lib.kp_last_error_message()


def test_rmsnorm_validation(lib):
    one = L.i64_array([8])
    _expect(lib, L.KP_EINVAL, "kp_rmsnorm_fwd_bf16", None, one, 0, None, 8, 8, None, 8, None, 8, None, 4, 8,
            1e-5, None)  # no input terms
    _expect(lib, L.KP_EINVAL, "kp_rmsnorm_fwd_bf16", L.ptr_array([None]), one, 1, None, 8, 8, None, 8, None, 8,
            None, 4, 8, 1e-5, None)  # NULL term with rows to do
    ptr = L.ptr_array([16])
    _expect(lib, L.KP_EWORKSPACE, "kp_rmsnorm_bwd_bf16", ptr, one, 1, ptr, one, 1, None, 16, 8, 8, None, 8, 16, 8,
            32, None, 0, 4, 8, 1e-5, 32, 1, None)  # dw requested, 1-byte workspace
    assert lib.kp_rmsnorm_bwd_workspace_size(8192, 4096) >= 4096 * 4


def test_embedding_validation(lib):
    _expect(lib, L.KP_EINVAL, "kp_embedding_fwd_bf16", 16, 10, 8, 8, 32, 3, 4, 48, 8, None, None)  # 3-byte ids
    # any vocabulary: past the sort key's 21 id bits the pipeline runs once per
    # slab of 2^21 - 1 rows, so the workspace holds one slab's bitmap
    slab = (1 << 21) - 1
    assert lib.kp_embedding_bwd_workspace_size(100, 1 << 30, 64) == lib.kp_embedding_bwd_workspace_size(100, slab, 64)
    assert lib.kp_embedding_bwd_workspace_size(100, slab, 64) > lib.kp_embedding_bwd_workspace_size(100, slab - 4096, 64)
    _expect(lib, L.KP_EUNSUPPORTED, "kp_embedding_bwd_bf16", 16, 64, 32, 8, 1 << 31, 1 << 22, 64, -1, 0, 48,
            L.KP_DTYPE_F32, 0, 64, 1 << 20, None, None)  # 2^31 tokens: past the sort's token count
    ws = lib.kp_embedding_bwd_workspace_size(65536, 128256, 64)
    _expect(lib, L.KP_EWORKSPACE, "kp_embedding_bwd_bf16", 16, 64, 32, 8, 65536, 128256, 64, -1, 0, 48,
            L.KP_DTYPE_F32, 0, 64, ws - 1, None, None)  # any token count: only the workspace bounds it
    _expect(lib, L.KP_EINVAL, "kp_embedding_bwd_bf16", 16, 64, 32, 8, 100, 1000, 64, -1, 0, 48, 7, 0, 64,
            1 << 20, None, None)  # unknown output dtype


def test_rope_validation(lib):
    st = L.i64_array([0, 0, 0])
    common = (1, 1)  # B, S
    _expect(lib, L.KP_EINVAL, "kp_rope_bf16", 16, 32, 1, st, st, None, None, 0, None, None, *common, 7, None, 0, 0,
            0, 0, 1e4, None, 0, 0, 0, 0, None, None)  # odd head dim
    _expect(lib, L.KP_EINVAL, "kp_rope_bf16", 16, 32, 1, st, st, None, None, 0, None, None, *common, 8, None, 0, 0,
            0, 0, -1.0, None, 0, 0, 0, 0, None, None)  # theta <= 0 without a table
    _expect(lib, L.KP_EINVAL, "kp_rope_bf16", 16, 32, 1, st, st, None, None, 0, None, None, *common, 8, None, 0, 0,
            0, 5, 1e4, None, 0, 0, 0, 0, None, None)  # unknown pairing
    _expect(lib, L.KP_EINVAL, "kp_rope_bf16_twice", 16, 32, 1, st, st, None, None, 0, None, None, *common, 8, None,
            0, 0, 0, 0, 1e4, None, 0, 0, 0, 0, None, None, None, None)  # no copy
    _expect(lib, L.KP_EINVAL, "kp_rope_bf16_twice", 16, 32, 1, st, st, None, None, 0, None, None, *common, 8, None,
            0, 0, 0, 0, 1e4, None, 0, 0, 0, 0, 32, None, None, None)  # the copy is the output itself
    _expect(lib, L.KP_EINVAL, "kp_rope_bf16_twice", 16, 32, 1, st, st, 48, 64, 1, st, st, *common, 8, None,
            0, 0, 0, 0, 1e4, None, 0, 0, 0, 0, 96, None, None, None)  # k without its copy


def test_unshard_validation(lib):
    off, ln = L.i64_array([0] * 17), L.i64_array([8] * 17)
    _expect(lib, L.KP_EINVAL, "kp_unshard_bf16", 16, 8, 64, off, ln, L.ptr_array([32] * 17), 17, None)
    off2, ln2 = L.i64_array([60]), L.i64_array([8])
    _expect(lib, L.KP_EINVAL, "kp_unshard_bf16", 16, 8, 64, off2, ln2, L.ptr_array([32]), 1, None)  # past the row


def test_empty_work_is_ok_without_device(lib):
    """Zero rows / positions / segments return KP_OK without a launch."""
    one = L.i64_array([8])
    assert lib.kp_rmsnorm_fwd_bf16(L.ptr_array([None]), one, 1, None, 8, 8, None, 8, None, 8, None, 0, 8, 1e-5,
                                   None) == L.KP_OK
    assert lib.kp_unshard_bf16(None, 8, 64, None, None, None, 0, None) == L.KP_OK
    assert lib.kp_swiglu_fwd_bf16(None, 8, None, 8, None, 8, 0, 8, None) == L.KP_OK
    assert lib.kp_swiglu_bwd_bf16(None, 8, None, 8, None, 8, None, 8, None, 8, None, 8, 4, 0, None) == L.KP_OK
    assert lib.kp_cross_entropy_bwd_bf16(None, 8, None, 8, -100, 1.0, None, 8, 0, 8, None, None) == L.KP_OK
    assert lib.kp_cross_entropy_fwd_workspace_size(0) == 0


def test_swiglu_validation(lib):
    _expect(lib, L.KP_EINVAL, "kp_swiglu_fwd_bf16", 16, 8, 32, 8, 48, 8, -1, 8, None)  # negative M
    _expect(lib, L.KP_EINVAL, "kp_swiglu_fwd_bf16", 16, 8, None, 8, 48, 8, 2, 8, None)  # NULL b
    _expect(lib, L.KP_EINVAL, "kp_swiglu_fwd_bf16", 16, 8, 32, 4, 48, 8, 2, 8, None)  # b rows overlap
    _expect(lib, L.KP_EINVAL, "kp_swiglu_bwd_bf16", 16, 8, 32, 8, 48, 8, 64, 8, 80, 8, None, 8, 2, 8, None)  # NULL da
    _expect(lib, L.KP_EINVAL, "kp_swiglu_bwd_bf16", 16, 8, 32, 8, 48, 8, 64, 7, 80, 8, 96, 8, 2, 8, None)


def test_silu_and_fwd_bwd_validation(lib):
    _expect(lib, L.KP_EINVAL, "kp_silu_bf16", None, 8, 32, 8, 2, 8, None)  # NULL a
    _expect(lib, L.KP_EINVAL, "kp_silu_bf16", 16, 8, 32, 7, 2, 8, None)    # out rows overlap
    assert lib.kp_silu_bf16(None, 8, None, 8, 0, 8, None) == L.KP_OK
    fb = "kp_swiglu_fwd_bwd_bf16"
    _expect(lib, L.KP_EINVAL, fb, 16, 8, 32, 8, 48, 8, 64, 8, None, 8, 96, 8, 2, 8, None)  # NULL db
    _expect(lib, L.KP_EINVAL, fb, 16, 8, 32, 8, None, 8, 64, 8, 80, 8, 96, 8, 2, 8, None)  # NULL g
    _expect(lib, L.KP_EINVAL, fb, 16, 8, 32, 8, 48, 8, 64, 8, 80, 8, 96, 8, -2, 8, None)  # negative M
    assert lib.kp_swiglu_fwd_bwd_bf16(None, 8, None, 8, None, 8, None, 8, None, 8, None, 8, 0, 8, None) == L.KP_OK


def test_cross_entropy_validation(lib):
    ws = int(lib.kp_cross_entropy_fwd_workspace_size(4))
    assert ws >= 4 * 12
    fwd = "kp_cross_entropy_fwd_bf16"
    _expect(lib, L.KP_EINVAL, fwd, 16, 8, 4, 8, 32, 2, -100, 1.0, 48, 64, None, None, 128, ws, None)  # 2-byte ids
    _expect(lib, L.KP_EINVAL, fwd, 16, 8, 4, 8, 32, 8, -100, 1.0, None, 64, None, None, 128, ws, None)  # no loss
    _expect(lib, L.KP_EWORKSPACE, fwd, 16, 8, 4, 8, 32, 8, -100, 1.0, 48, 64, None, None, 128, ws - 1, None)
    _expect(lib, L.KP_EINVAL, fwd, 16, 4, 4, 8, 32, 8, -100, 1.0, 48, 64, None, None, 128, ws, None)  # stride < V
    _expect(lib, L.KP_EINVAL, fwd, 16, 8, 4, 8, 32, 8, -100, 1.0, 48, 64, None, None, 132, ws, None)  # misaligned ws
    bwd = "kp_cross_entropy_bwd_bf16"
    _expect(lib, L.KP_EINVAL, bwd, 16, 8, 32, 8, -100, 1.0, None, 8, 4, 8, None, None)  # no output
    _expect(lib, L.KP_EINVAL, bwd, 16, 8, 32, 3, -100, 1.0, 64, 8, 4, 8, None, None)    # 3-byte ids
    _expect(lib, L.KP_EINVAL, bwd, 16, 8, 32, 8, -100, 1.0, 64, 8, 4, 0, None, None)    # V = 0


def test_cross_entropy_fwd_bwd_validation(lib):
    fn = "kp_cross_entropy_fwd_bwd_bf16"
    ws = int(lib.kp_cross_entropy_fwd_workspace_size(4))
    _expect(lib, L.KP_EINVAL, fn, 16, 8, 4, 8, 32, 8, -100, 1.0, 48, 8, 1.0, 64, None, None, 128, ws, None)  # loss only
    _expect(lib, L.KP_EWORKSPACE, fn, 16, 8, 4, 8, 32, 8, -100, 1.0, 48, 8, 1.0, 64, 72, None, 128, ws - 8, None)
    _expect(lib, L.KP_EINVAL, fn, 16, 8, 4, 8, 32, 2, -100, 1.0, 48, 8, 1.0, None, None, None, None, 0, None)  # 2-byte ids
    _expect(lib, L.KP_EINVAL, fn, 16, 8, 4, 8, 32, 8, -100, 1.0, None, 8, 1.0, None, None, None, None, 0, None)  # no out
    _expect(lib, L.KP_EINVAL, fn, 16, 8, 4, 8, 32, 8, -100, 1.0, 48, 4, 1.0, None, None, None, None, 0, None)  # stride
    assert lib.kp_cross_entropy_fwd_bwd_bf16(None, 8, 0, 8, None, 8, -100, 1.0, None, 8, 1.0, None, None, None, None,
                                             0, None) == L.KP_OK


def test_rmsnorm_embedding_bwd_validation(lib):
    fn = "kp_rmsnorm_embedding_bwd_bf16"
    dy, st = L.ptr_array([16]), L.i64_array([4096])
    M, N, V = 8192, 4096, 128256

    def call(status, n_dy=1, x_stride=N, rstd=None, y=None, n=N, ib=8, out_dtype=L.KP_DTYPE_F32, ws=None, wsb=0):
        _expect(lib, status, fn, dy, st, n_dy, 32, x_stride, rstd, 48, n, n, 64, n, y, n, None, 80, None, 1, M, n,
                1e-5, 96, ib, V, -1, 112, out_dtype, 1, ws, wsb, None, None)

    call(L.KP_EINVAL, n_dy=0)                      # no dy terms
    call(L.KP_EINVAL, ib=3)                        # 3-byte ids
    call(L.KP_EINVAL, out_dtype=7)                 # unknown table dtype
    call(L.KP_EINVAL, rstd=128, y=144)             # y is the forward's: not with a saved rstd
    call(L.KP_EUNSUPPORTED, n=1000)                # no fused row pass for N = 1000
    call(L.KP_EUNSUPPORTED, x_stride=N + 4)        # rows not 16-byte aligned
    need = lib.kp_rmsnorm_embedding_bwd_workspace_size(M, N, V)
    assert need > lib.kp_embedding_bwd_workspace_size(M, V, N)  # + the weight-gradient partial rows
    call(L.KP_EWORKSPACE, ws=256, wsb=need - 1)    # one byte short


def test_embedding_rmsnorm_validation(lib):
    fn = "kp_embedding_rmsnorm_fwd_bf16"
    _expect(lib, L.KP_EINVAL, fn, 16, 100, 64, 32, 3, 8, None, 64, 64, None, 64, 48, 64, None, 64, 1e-5, None, None)
    _expect(lib, L.KP_EINVAL, fn, 16, 100, 32, 32, 8, 8, None, 64, 64, None, 64, 48, 64, None, 64, 1e-5, None, None)
    _expect(lib, L.KP_EINVAL, fn, 16, 100, 64, 32, 8, 8, None, 64, 64, None, 64, None, 64, None, 64, 1e-5, None, None)
    _expect(lib, L.KP_EUNSUPPORTED, fn, 16, 100, 64, 32, 8, 8, None, 64, 64, None, 64, 48, 64, None, 60, 1e-5, None,
            None)  # no fast-path row shape for N = 60
    assert lib.kp_embedding_rmsnorm_fwd_bf16(None, 100, 64, None, 8, 0, None, 64, 64, None, 64, None, 64, None, 64,
                                             1e-5, None, None) == L.KP_OK


def test_stream_probe_validation(lib):
    nt = L.KP_STORE_NONTEMPORAL
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([16]), 5, 64, L.ptr_array([32]), 1, 64, 4, nt, None)
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([16]), 1, 64, L.ptr_array([32]), 0, 64, 4, nt, None)
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([16, 16]), 2, 64, L.ptr_array([32, 32, 32]), 3, 64, 4, nt, None)
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([16]), 1, 60, L.ptr_array([32]), 1, 64, 4, nt, None)
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([24]), 1, 64, L.ptr_array([32]), 1, 64, 4, nt, None)
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([16]), 1, 64, L.ptr_array([32]), 1, 64, 3, nt, None)
    _expect(lib, L.KP_EINVAL, "kp_stream_probe", L.ptr_array([16]), 1, 64, L.ptr_array([32]), 1, 64, 4, 7, None)
    _expect(lib, L.KP_EUNSUPPORTED, "kp_stream_probe", L.ptr_array([16]), 1, 1 << 32, L.ptr_array([32]), 1, 64, 1, nt,
            None)
    assert lib.kp_stream_probe(None, 0, 0, L.ptr_array([32]), 1, 0, 1, nt, None) == L.KP_OK  # nothing to stream


def test_rope_c64_validation(lib):
    st = L.i64_array([0, 0, 0])
    fn = "kp_rope_c64"
    _expect(lib, L.KP_EINVAL, fn, 16, 32, 1, st, st, None, None, 0, None, None, 1, 1, 8, None, 0, 0, 0, None, 4, 8, 0,
            None, None)  # no table
    _expect(lib, L.KP_EINVAL, fn, 16, 32, 1, st, st, None, None, 0, None, None, 1, 1, 8, None, 0, 0, 0, 64, 4, 4, 0,
            None, None)  # table row stride < P
    _expect(lib, L.KP_EINVAL, fn, 16, 32, 1, st, st, None, None, 0, None, None, 1, 1, 8, 48, 2, 0, 0, 64, 4, 8, 0,
            None, None)  # 2-byte positions
    _expect(lib, L.KP_EINVAL, fn, None, 32, 1, st, st, None, None, 0, None, None, 1, 1, 8, None, 0, 0, 0, 64, 4, 8, 0,
            None, None)  # no x
    assert lib.kp_rope_c64(16, 32, 1, st, st, None, None, 0, None, None, 0, 1, 8, None, 0, 0, 0, 64, 4, 8, 0, None,
                           None) == L.KP_OK  # B = 0
