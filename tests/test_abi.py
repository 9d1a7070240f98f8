"""The C-ABI library loads and exports every entry point include/mica_amd.h declares, and its
argument validation (which runs before any HIP call) rejects bad inputs with the documented codes.
No kernel is launched here: every call below returns before touching a device."""
import ctypes
import re
from pathlib import Path

import pytest

from mica_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mica_amd.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mica_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared()
    for n in ("mica_act_quant", "mica_rmsnorm_quant", "mica_mm_i8", "mica_gather_logits", "mica_swiglu",
              "mica_version", "mica_status_name", "mica_device_info"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), f"{name} declared in mica_amd.h but not exported"
    # and the ctypes signatures cover them all
    assert set(declared()) == set(_lib.SIGNATURES)


def test_version_and_status_names():
    lib = _lib.load()
    assert lib.mica_version() == (0 << 16) | 1
    assert _lib.status_name(1) == "shape" and _lib.status_name(3) == "align"
    assert lib.mica_status_name(0) == b"ok"
    assert lib.mica_status_name(5) == b"i32_range"


A16 = 1 << 20  # a 16-byte aligned fake address: never dereferenced, every call below is rejected first


@pytest.mark.parametrize("args,code", [
    # (A, lda, B, ldb, sa, sb, bias, res, ldr, C, ldc, out_dtype, M, N, K, epi)
    ((None, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 6),      # NULL A
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 9, 8, 64, 64, 0), 2),       # bad out dtype
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 40, 0), 1),       # K % 16
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 96, 64, 1), 1),       # SILU: N % 128
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 2, 8, 128, 64, 1), 6),      # SILU: not bf16
    ((A16, 48, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 4),       # lda < K
    ((A16, 72, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 4),       # lda % 16
    ((A16 + 8, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 3),   # misaligned A
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 1 << 30, 64, 64, 0), 5),  # M * lda >= 2^31
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 4, 8, 64, 64, 1), 6),       # int32 + SILU
])
def test_mm_i8_rejects(args, code):
    lib = _lib.load()
    assert lib.mica_mm_i8(*args, None, 0, None) == code


def test_mm_i8_rejects_bad_workspace():
    lib = _lib.load()
    ok = (A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0)
    assert lib.mica_mm_i8(*ok, A16 + 4, 1 << 20, None) == 3    # misaligned workspace
    assert lib.mica_mm_i8(*ok, A16, -1, None) == 6             # negative size


@pytest.mark.parametrize("args,code", [
    ((None, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 6),      # NULL A
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 40, 0), 1),       # K % 16
    ((A16, 72, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 4),       # lda % 16
    ((A16 + 8, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 8, 64, 64, 0), 3),   # misaligned A
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 1 << 30, 64, 64, 0), 5),  # M * lda >= 2^31
    ((A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 0, 64, 64, 0), 0),       # M = 0: nothing to do
])
def test_mm_i8_noalloc_checks_arguments_before_any_device_call(args, code):
    """The no-allocation GEMM validates its arguments as mica_mm_i8 does, before it looks up its scratch."""
    lib = _lib.load()
    assert lib.mica_mm_i8_noalloc(*args, None) == code
    assert lib.mica_mm_i8_noalloc_scratch_bytes() == 4096 + 64 * 2 * 256 * 1024


def test_mm_i8_empty_is_a_no_op():
    lib = _lib.load()
    assert lib.mica_mm_i8(A16, 64, A16, 64, A16, A16, None, None, 0, A16, 64, 0, 0, 64, 64, 0, None, 0, None) == 0


@pytest.mark.parametrize("args,code", [
    # (x, x_dtype, ldx, inv, q, ldq, s, M, K, rounding)
    ((None, 0, 64, None, A16, 64, A16, 4, 64, 0), 6),
    ((A16, 3, 64, None, A16, 64, A16, 4, 64, 0), 2),      # int8 input
    ((A16, 0, 64, None, A16, 64, A16, 4, 60, 0), 1),      # K % 8
    ((A16, 0, 64, None, A16, 64, A16, 4, 32768, 0), 1),   # K > 16384
    ((A16, 0, 60, None, A16, 64, A16, 4, 56, 0), 4),      # ldx % 8
    ((A16, 0, 64, None, A16, 64, A16, 4, 64, 7), 6),      # rounding mode
    ((A16, 0, 64, A16 + 4, A16, 64, A16, 4, 64, 0), 3),   # misaligned inv
])
def test_act_quant_rejects(args, code):
    lib = _lib.load()
    assert lib.mica_act_quant(*args, None) == code


def test_rmsnorm_quant_rejects():
    lib = _lib.load()
    base = dict(x=A16, xd=0, ldx=64, r=None, ldr=0, w=A16, wd=0, off=1.0, eps=1e-6, inv=None, q=A16, ldq=64,
                s=A16, y=None, ldy=0, sm=None, lds=0, M=4, K=64, rnd=0)

    def call(**kw):
        a = dict(base, **kw)
        return lib.mica_rmsnorm_quant(*a.values(), None)

    assert call(q=None, y=None) == 6          # nothing to write
    assert call(s=None) == 6                  # q without s
    assert call(sm=A16, lds=64) == 6          # sum without residual
    assert call(xd=2) == 2                    # fp32 activations are not normed
    assert call(wd=3) == 2
    assert call(K=100) == 1
    assert call(r=A16, ldr=32) == 4
    assert call(M=0) == 0


def test_rmsnorm_quant_multi_rejects():
    import ctypes
    lib = _lib.load()
    P = ctypes.c_void_p

    def call(n, q=A16, ldq=64, inv=None, arrays=True, M=4):
        invs, qs, ss = (P * 5)(*([inv] * 5)), (P * 5)(*([q] * 5)), (P * 5)(*([A16] * 5))
        lds = (ctypes.c_int * 5)(*([ldq] * 5))
        if not arrays:
            invs = None
        return lib.mica_rmsnorm_quant_multi(A16, 0, 64, None, 0, A16, 0, 1.0, 1e-6, n, invs, qs, lds, ss, None, 0,
                                            None, 0, M, 64, 0, None)

    assert call(0) == 6                    # no consumer
    assert call(5) == 6                    # more than 4
    assert call(2, arrays=False) == 6      # missing pointer array
    assert call(2, q=None) == 6            # a consumer without int8 output
    assert call(2, ldq=32) == 4            # a consumer's row stride < K
    assert call(2, inv=A16 + 4) == 3       # misaligned smoothing factors
    assert call(4, M=0) == 0


def test_gather_logits_rejects():
    lib = _lib.load()
    # (h, ldh, n_rows, rows, B, norm_w, norm_dtype, offset, eps, W, w_dtype, ldw, w_rows, ids, L, K, logits,
    #  lo, cnt, probs, ldp)
    ok = [A16, 64, 100, A16, 2, None, 0, 1.0, 1e-6, A16, 2, 64, 8, None, 8, 64, A16, None, None, None, 0]

    def with_(**kw):
        a = list(ok)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lib.mica_gather_logits(*a, None)

    assert with_(a10=1) == 2          # fp16 label rows
    assert with_(a17=A16) == 6        # lo without cnt
    assert with_(a14=9000) == 1       # L > 8192
    assert with_(a12=4) == 1          # fewer label rows than L without ids
    assert with_(a2=0) == 1           # no hidden rows
    assert with_(a4=0) == 0           # no requests


def test_swiglu_rejects():
    lib = _lib.load()
    assert lib.mica_swiglu(A16, A16, A16, 16, 2, None) == 2
    assert lib.mica_swiglu(A16, A16 + 2, A16, 16, 0, None) == 3
    assert lib.mica_swiglu(A16, A16, A16, 0, 0, None) == 0


def test_ctypes_signature_arity_matches_header():
    """Each ctypes prototype has as many arguments as the header declaration (stream included)."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), name
    assert ctypes.sizeof(ctypes.c_void_p) == 8


def test_causal_conv1d_rejects():
    lib = _lib.load()
    # (x, sbx, ldx, w, bias, w_dtype, width, init, final, y, sby, ldy, B, T, C, silu, n_norm, eps)
    ok = [A16, 64 * 8, 64, A16, None, 0, 4, None, None, A16, 64 * 8, 64, 2, 8, 64, 1, 0, 1e-6]

    def with_(**kw):
        a = list(ok)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lib.mica_causal_conv1d(*a, None)

    assert with_(a0=None) == 6            # NULL x
    assert with_(a5=1) == 2               # fp16 weights
    assert with_(a6=5) == 1               # width > 4
    assert with_(a14=60) == 1             # C % 8
    assert with_(a16=1) == 1              # a norm head wider than C
    assert with_(a2=56) == 4              # token stride < C
    assert with_(a1=100) == 4             # batch stride < T * ldx
    assert with_(a9=A16 + 2) == 3         # misaligned y
    assert with_(a13=0) == 0              # T = 0: nothing to do


def test_gdn_chunk_rejects():
    lib = _lib.load()
    D = 128
    # (q, sbq, ldq, k, sbk, ldk, v, sbv, ldv, g, beta, beta_dtype, h0, hT, o, scale, B, T, HK, HV, ws, ws_bytes)
    ok = [A16, 8 * 2 * D, 2 * D, A16, 8 * 2 * D, 2 * D, A16, 8 * 4 * D, 4 * D, A16, A16, 0, None, None, A16, 0.1,
          1, 8, 2, 4, A16, 1 << 30]

    def with_(**kw):
        a = list(ok)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lib.mica_gdn_chunk(*a, None)

    assert with_(a11=1) == 2              # fp16 beta
    assert with_(a19=3) == 1              # HV not a multiple of HK
    assert with_(a2=D) == 4               # q token stride < HK * 128
    assert with_(a0=None) == 6            # NULL q with tokens to scan
    assert with_(a14=A16 + 8) == 3        # misaligned o
    assert with_(a20=None) == 6           # no workspace
    assert with_(a21=16) == 6             # workspace too small
    assert with_(a16=0) == 0              # no sequences
    assert lib.mica_gdn_workspace_bytes(8, 2048, 32) == 8 * 32 * 32 * (2 * 64 * 128 * 2 + 64 * 4)


def test_gated_rmsnorm_quant_rejects():
    lib = _lib.load()
    # (x, ldx, z, ldz, w, eps, y, ldy, q, ldq, s, M, N)
    ok = [A16, 4096, A16, 4096, A16, 1e-6, None, 0, A16, 4096, A16, 4, 4096]

    def with_(**kw):
        a = list(ok)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lib.mica_gated_rmsnorm_quant(*a, None)

    assert with_(a8=None) == 6            # no int8 output
    assert with_(a12=1536) == 1           # N / 512 not a power of two
    assert with_(a12=16384) == 1          # N > 8192
    assert with_(a1=2048) == 4            # ldx < N
    assert with_(a2=A16 + 4) == 3         # misaligned z
    assert with_(a11=0) == 0              # M = 0


def test_gdn_gate_rejects():
    lib = _lib.load()
    # (a, lda, b, ldb, A_log, dt_bias, g, beta, M, HV)
    ok = [A16, 32, A16, 32, A16, A16, A16, A16, 4, 32]

    def with_(**kw):
        a = list(ok)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lib.mica_gdn_gate(*a, None)

    assert with_(a6=None) == 6            # no g output
    assert with_(a9=0) == 1               # no heads
    assert with_(a1=16) == 4              # lda < HV
    assert with_(a8=0) == 0               # no tokens


def test_head_norm_rope_rejects():
    lib = _lib.load()
    base = dict(x=A16, ldx=6144, T=4, qo=0, nq=16, ko=4096, nk=4, d=256, wq=A16, wk=A16, off=1.0, eps=1e-6, rd=64,
                cs=A16, sn=A16, npos=100, pos=None, period=4)

    def call(**kw):
        a = dict(base, **kw)
        return lib.mica_head_norm_rope(*a.values(), None)

    assert call(x=None) == 6               # no rows
    assert call(d=192) == 1                # head_dim not a power of two
    assert call(rd=512) == 1               # rotary dims beyond the head
    assert call(rd=48) == 1                # rotary dims not a power of two
    assert call(cs=None) == 6              # rotation without tables
    assert call(period=0) == 6             # rotation without positions
    assert call(ldx=5000) == 4             # k heads past the row
    assert call(ko=4100) == 4              # unaligned segment
    assert call(wq=A16 + 4) == 3           # misaligned weight
    assert call(T=0) == 0


def test_gate_quant_rejects():
    lib = _lib.load()
    base = dict(a=A16, lda=4096, g=A16, ldg=10240, q=A16, ldq=4096, s=A16, y=None, ldy=0, M=4, K=4096, rnd=0)

    def call(**kw):
        a = dict(base, **kw)
        return lib.mica_gate_quant(*a.values(), None)

    assert call(g=None) == 6
    assert call(rnd=1) == 6                # half away is not served
    assert call(K=1000) == 1               # not a multiple of 512
    assert call(ldg=2048) == 4             # gate rows shorter than K
    assert call(s=A16 + 4) == 3
    assert call(M=0) == 0
