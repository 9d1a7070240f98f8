"""Drop-in replacement of the reference's kernel launcher module ``int8_kernels``
(akivet/Mica v0.5/serving/lib/int8_kernels.py), backed by the gfx950 HIP kernels of libmica_amd.so.

Same contract as the reference:
  * ``act_quant(x, inv_smooth=None) -> (q, s) | None`` (int8_kernels.py:325-353)
  * ``mm_i8(qx, sx, qw, sw, bias=None, out_dtype=torch.bfloat16) -> Tensor | None`` (:359-406)
  * ``available(device=None) -> (bool, str)`` (:146-159), ``preload(device=None) -> int`` (:217-224),
    ``kernel_dir()`` (:83-84; MICA_W8A8_AOT_DIR when set, where the reference keeps ``s.pt``),
    ``STATS`` (:19), ``ATTN`` / ``attn_keys`` / ``attn_fwd`` (:409-481)
  * an unsupported input returns ``None`` and counts the reason in ``STATS['fallback']`` (:22-24);
    every launch adds 1 to ``STATS['launch']`` (:310); a device error raises RuntimeError (:60-64).
  * outputs are allocated with torch on the input's device; kernels run on torch's current stream
    (:261-265); nothing synchronises, so the calls can be captured in a HIP graph.

Extensions used by the fused hot path: ``rounding='away'`` (the Triton kernel's rounding,
kernel_src/kernels.py:35), ``mm_i8(..., residual=, epilogue='silu_mul')``, ``mm_i8_int32`` (raw
accumulators), and ``STRICT`` (env ``MICA_AMD_STRICT=1``) which turns a miss into an exception.

Attention: ``ATTN`` / ``attn_keys()`` / ``attn_fwd(q, k, v, scale)`` (:409-481) run the gfx950 flash-attention
kernel for head dim 256 with 4 query heads per key/value head (key ``attn|bf16|hd256|hq16|r4|s0.0625|m64``);
any other shape misses, as the reference does for a shape its container has no kernel for.
"""
from __future__ import annotations

import os
import threading
from pathlib import Path

import torch

from . import _lib

DT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16, torch.float32: _lib.FP32}
I32 = 2 ** 31
STATS = {"launch": 0, "fallback": {}}
STRICT = os.environ.get("MICA_AMD_STRICT", "") not in ("", "0")
ROUNDING = {"even": _lib.ROUND_EVEN, "away": _lib.ROUND_AWAY}
EPILOGUE = {"none": _lib.EPI_SCALE, "silu_mul": _lib.EPI_SILU_MUL}
_STATS_LOCK = threading.Lock()


class KernelMiss(RuntimeError):
    """Raised instead of returning None when STRICT is set."""


def _miss(reason):
    with _STATS_LOCK:
        STATS["fallback"][reason] = STATS["fallback"].get(reason, 0) + 1
    if STRICT:
        raise KernelMiss(f"mica_amd kernel miss: {reason}")
    return None


def _launched():
    with _STATS_LOCK:
        STATS["launch"] += 1


ENV_DIR = "MICA_W8A8_AOT_DIR"   # int8_kernels.py:10


def kernel_dir() -> Path:
    """The directory the reference's callers read their kernel-side files from, the SmoothQuant
    statistics ``s.pt`` among them (``decide`` and ``apply``, int8_runtime.py:227, 265): the directory
    named by MICA_W8A8_AOT_DIR when it is set, as in the reference (int8_kernels.py:83-84), else that of
    libmica_amd.so (lib_dir())."""
    env = os.environ.get(ENV_DIR)
    return Path(env) if env else lib_dir()


def lib_dir() -> Path:
    """Directory holding libmica_amd.so (env MICA_AMD_LIB_DIR overrides)."""
    return _lib.lib_path().parent


_ARCH = {}


def _dev(device):
    dev = torch.device(device) if device is not None else torch.device("cuda")
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _gfx(dev) -> int:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _ARCH:
        _ARCH[idx] = _lib.device_info(idx)["gfx_arch"]
    return _ARCH[idx]


def available(device=None):
    """(True, description) when the kernels can run on ``device`` (a gfx950 GPU)."""
    if not torch.cuda.is_available():
        return (False, "no ROCm GPU available")
    dev = _dev(device)
    if dev.type != "cuda":
        return (False, f"{dev} is not a GPU device")
    try:
        _lib.load()
    except (OSError, RuntimeError) as exc:
        return (False, f"library: {exc!r}"[:200])
    arch = _gfx(dev)
    if arch != 950:
        return (False, f"gfx{arch} is not gfx950")
    return (True, f"gfx950 kernels from {lib_dir()}")


def preload(device=None) -> int:
    """Load the library (its code objects register with the HIP runtime at load); returns the number
    of launchers it exports, or 0 when the device cannot run them."""
    ok, _ = available(device)
    if not ok:
        return 0
    return sum(1 for name in _lib.SIGNATURES if name not in ("mica_version", "mica_status_name",
                                                            "mica_device_info"))


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _aligned(*ts):
    return all(t.data_ptr() % 16 == 0 for t in ts)


def _on(dev, call):
    if dev.index is None or torch.cuda.current_device() == dev.index:
        return call()
    with torch.cuda.device(dev):
        return call()


def _run(dev, name, fn, *args, stream=None):
    """Launch through the C ABI on the current stream (``stream``: its handle, when the caller has it
    already); returns True, or None on a miss."""
    rc = _lib.check(_on(dev, lambda: fn(*args, _stream(dev) if stream is None else stream)), name)
    if rc > 0:
        return _miss(_lib.status_name(rc))
    _launched()
    return True


def _gpu_ok(dev):
    return dev.type == "cuda" and _gfx(dev) == 950


_WORKSPACE = {}
_WS_PTR = {}     # (device index, stream handle) -> (pointer, bytes) of _WORKSPACE's tensor
_WS_LOCK = threading.Lock()


def gemm_workspace(dev, stream=None):
    """The GEMM's split-tile workspace for torch's current stream on ``dev`` (``stream``: its handle,
    when the caller has it already): allocated (zeroed) once per (device, stream) and kept for the
    life of the process, so a HIP graph that captured it stays valid; every launch leaves its counters
    zero again.  Returns (pointer, bytes).  It cannot be first allocated inside a HIP-graph capture
    (RuntimeError): allocate it on the stream before."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream if stream is None else stream)
    got = _WS_PTR.get(key)
    if got is not None:
        return got
    ws = _WORKSPACE.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            # a buffer made during capture comes from the graph's pool and its zero fill is only
            # recorded, not run: its arrival counters would hold garbage for other users of the key
            raise RuntimeError("the GEMM split workspace must be allocated before HIP-graph capture: call "
                               "int8_kernels.gemm_workspace(device) on the capturing stream first, or use "
                               "split=False")
        with _WS_LOCK:
            ws = _WORKSPACE.get(key)
            if ws is None:
                nbytes = int(_lib.load().mica_mm_i8_workspace_bytes(dev.index))
                if nbytes <= 0:
                    raise RuntimeError(f"mica_mm_i8_workspace_bytes({dev.index}) failed: {nbytes}")
                ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
                _WORKSPACE[key] = ws
                _WS_PTR[key] = (ws.data_ptr(), ws.numel())
    return ws.data_ptr(), ws.numel()


# QLinear's GEMMs pass mm_i8(..., split="auto"): the split workspace when this allows it.
SPLIT = {"auto": True}


def _auto_workspace(dev, stream):
    """mm_i8's split="auto": the workspace of (dev, stream) -- made by the first such call on an eager
    stream; under HIP-graph capture only one the capturing stream already has (a workspace cannot be
    made inside a capture; capture on a stream that ran the same work eagerly first, as
    engine.PrefillEngine does) -- else none.  SPLIT["auto"] = False turns the split schedules off."""
    if not SPLIT["auto"]:
        return None, 0
    got = _WS_PTR.get((dev.index, stream))
    if got is not None:
        return got
    if torch.cuda.is_current_stream_capturing():
        return None, 0
    return gemm_workspace(dev, stream)


def auto_split(dev):
    """Whether mm_i8(..., split="auto") gives a GEMM on torch's current stream a workspace (making it
    now on an eager stream that has none)."""
    return _auto_workspace(_dev(dev), _stream(_dev(dev)))[0] is not None


def act_quant(x, inv_smooth=None, rounding="even"):
    """Per-token INT8 quantization of a 2-D activation (int8_kernels.py:325-353)."""
    if x.dim() != 2 or x.device.type != "cuda" or x.dtype not in DT:
        return _miss("act_input")
    m, k = x.shape
    if x.stride(1) != 1 or (m > 1 and x.stride(0) != k):  # a size-1 dim's stride is immaterial
        return _miss("act_contiguous")
    if not _gpu_ok(x.device):
        return _miss("no_container")
    if inv_smooth is not None and (inv_smooth.dtype != torch.float32 or not inv_smooth.is_contiguous()
                                   or inv_smooth.numel() != k or inv_smooth.device != x.device):
        return _miss("act_inv")
    if m * k >= I32:
        return _miss("i32_range")
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    if not _aligned(x, q, s, *(() if inv_smooth is None else (inv_smooth,))):
        return _miss("align")
    L = _lib.load()
    ok = _run(x.device, "mica_act_quant", L.mica_act_quant, x.data_ptr(), DT[x.dtype], k,
              None if inv_smooth is None else inv_smooth.data_ptr(), q.data_ptr(), k, s.data_ptr(), m, k,
              ROUNDING[rounding])
    return (q, s) if ok else None


def mm_i8(qx, sx, qw, sw, bias=None, out_dtype=torch.bfloat16, residual=None, epilogue="none", split=False,
          requant=False):
    """C = (qx . qw^T)_i32 * sx[m] * sw[n] (+ bias[n]) -> out_dtype (int8_kernels.py:359-406).

    Extensions: ``residual`` ([M, N] of out_dtype) is added after the output rounding;
    ``epilogue='silu_mul'`` treats qw as gate/up rows interleaved in groups of 64
    (int8_runtime.pack_gate_up) and returns bf16(bf16(silu(gate)) * up) of shape [M, N / 2];
    ``split=True`` gives the kernel a per-stream workspace (``gemm_workspace``; ``split="auto"``: the one
    ``_auto_workspace`` allows, the choice of QLinear's GEMMs) for schedules that split
    tiles along K, with exact int32 partial sums and so the same bits as without it: for 16-bit outputs
    with K >= 8192 whose output fits at most CUs / 3 tiles of 128 x 160 (128 x 256 for 'silu_mul') -- a
    short request's down projection -- every tile in K / 2560 parts; for int32 / fp32 outputs a partial
    last round of at most CUs / 4 tiles of 256 x 256 over four workgroups each when K >= 8192 and
    M <= 256 (the default schedule runs such a round as 128 x 128 quarter tiles).  ``requant=True``
    returns the per-token int8 quantization (q, s) of the
    output instead of the output (the next QLinear's input, e.g. h of the MLP for the down projection):
    a second launch, because each row's scale needs the absmax of the whole row, which spans every
    column tile of the GEMM.
    """
    if qx.dim() != 2 or qw.dim() != 2 or qx.dtype != torch.int8 or qw.dtype != torch.int8 or out_dtype not in DT:
        return _miss("mm_input")
    m, k = qx.shape
    n = qw.shape[0]
    if (qw.shape[1] != k or qx.stride(1) != 1 or qw.stride(1) != 1 or (m > 1 and qx.stride(0) != k)
            or (n > 1 and qw.stride(0) != k)):
        return _miss("mm_contiguous")
    for t, size in ((sx, m), (sw, n)) + (((bias, n),) if bias is not None else ()):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != size or t.device != qx.device:
            return _miss("mm_scales")
    if qw.device != qx.device:
        return _miss("mm_device")
    if qx.device.type != "cuda" or not _gpu_ok(qx.device):
        return _miss("no_container")
    if epilogue not in EPILOGUE:
        return _miss("mm_epilogue")
    n_out = n // 2 if epilogue == "silu_mul" else n
    if epilogue == "silu_mul" and (n % 128 or out_dtype != torch.bfloat16 or bias is not None
                                   or residual is not None):
        return _miss("mm_epilogue")
    if residual is not None and (residual.shape != (m, n_out) or residual.dtype != out_dtype
                                 or not residual.is_contiguous() or residual.device != qx.device):
        return _miss("mm_residual")
    if m * max(k, n) >= I32:
        return _miss("i32_range")
    if k % 16:
        return _miss("div16:K")
    out = torch.empty((m, n_out), dtype=out_dtype, device=qx.device)
    extra = tuple(t for t in (bias, residual) if t is not None)
    if not _aligned(qx, qw, sx, sw, out, *extra):
        return _miss("align")
    L = _lib.load()
    dev = _dev(qx.device)
    st = _stream(dev)
    if split == "auto":
        ws, ws_bytes = _auto_workspace(dev, st)
    else:
        ws, ws_bytes = gemm_workspace(dev, st) if split else (None, 0)
    ok = _run(qx.device, "mica_mm_i8", L.mica_mm_i8, qx.data_ptr(), k, qw.data_ptr(), k, sx.data_ptr(),
              sw.data_ptr(), None if bias is None else bias.data_ptr(),
              None if residual is None else residual.data_ptr(), n_out, out.data_ptr(), n_out, DT[out_dtype],
              m, n, k, EPILOGUE[epilogue], ws, ws_bytes, stream=st)
    if not ok:
        return None
    return act_quant(out) if requant else out


def mm_i8_int32(qx, qw, split=False):
    """Raw int32 accumulators qx . qw^T on the matrix cores (the int32 result of
    int8_quant.torch_int_mm, int8_quant.py:92-96), or None on a miss."""
    if qx.dim() != 2 or qw.dim() != 2 or qx.dtype != torch.int8 or qw.dtype != torch.int8:
        return _miss("mm_input")
    m, k = qx.shape
    n = qw.shape[0]
    if qw.shape[1] != k or not qx.is_contiguous() or not qw.is_contiguous() or qw.device != qx.device:
        return _miss("mm_contiguous")
    if qx.device.type != "cuda" or not _gpu_ok(qx.device):
        return _miss("no_container")
    if k % 16:
        return _miss("div16:K")
    if m * max(k, n) >= I32:
        return _miss("i32_range")
    out = torch.empty((m, n), dtype=torch.int32, device=qx.device)
    dummy = torch.empty((max(m, n, 1),), dtype=torch.float32, device=qx.device)
    if not _aligned(qx, qw, out):
        return _miss("align")
    L = _lib.load()
    ws, ws_bytes = gemm_workspace(_dev(qx.device)) if split else (None, 0)
    ok = _run(qx.device, "mica_mm_i8", L.mica_mm_i8, qx.data_ptr(), k, qw.data_ptr(), k, dummy.data_ptr(),
              dummy.data_ptr(), None, None, n, out.data_ptr(), n, _lib.INT32, m, n, k, _lib.EPI_SCALE, ws, ws_bytes)
    return out if ok else None


ATTN = {"enabled": True}


def attn_keys(device=None):
    """The attention configuration the gfx950 kernel serves, in the reference's key format
    (int8_kernels.py:420-427): bf16, head dim 256, 16 query heads, 4 per key/value head, scale 1/16 (the
    4B model's full-attention layers).  The kernel itself takes any scale and HQ = 4 HK."""
    try:
        dev = _dev(device)
    except Exception:
        return []
    if dev.type != "cuda" or not _gpu_ok(dev):
        return []
    return ["attn|bf16|hd256|hq16|r4|s0.0625|m64"]


def attn_fwd(q, k, v, scale):
    """Causal GQA attention forward (int8_kernels.py:430-481): q [b, hq, n, d], k / v [b, hk, keys, d]
    (keys >= n; the queries are the last n positions), bf16, unit feature stride.  Returns o [b, hq, n, d]
    (a view of a [b, n, hq, d] tensor, as the reference returns), or None on a miss."""
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape or q.device.type != "cuda" or \
            not q.dtype == k.dtype == v.dtype == torch.bfloat16:
        return _miss("attn_input")
    b, hq, n, d = q.shape
    hk, keys = k.shape[1], k.shape[2]
    if k.shape[0] != b or k.shape[3] != d or hq % hk or n < 1 or keys < n or k.device != q.device:
        return _miss("attn_shape")
    if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1:
        return _miss("attn_stride")
    if not _gpu_ok(q.device):
        return _miss("no_container")
    if d != 256 or hq != 4 * hk:
        return _miss("attn_config")
    if not _aligned(q, k, v) or any(s % 8 for t in (q, k, v) for s in t.stride()[:3]):
        return _miss("align")
    from .attention import attention_fwd
    try:
        return attention_fwd(q, k, v, "bhsd", float(scale))
    except ValueError:
        return _miss("attn_unsupported")
