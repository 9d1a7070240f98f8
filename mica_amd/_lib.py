"""ctypes binding of libmica_amd.so, the C ABI declared in include/mica_amd.h.

The library is loaded after torch, so it binds to the HIP runtime torch already loaded (same soname)
and the stream handles torch hands out are valid in it.  A missing library is an error, never a
silent fallback: build it with ``python -m mica_amd.build``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libmica_amd.so"
ENV_DIR = "MICA_AMD_LIB_DIR"

# dtype codes (mica_amd.h)
BF16, FP16, FP32, INT8, INT32 = 0, 1, 2, 3, 4
ROUND_EVEN, ROUND_AWAY = 0, 1
EPI_SCALE, EPI_SILU_MUL = 0, 1

MISS_NAMES = {1: "shape", 2: "dtype", 3: "align", 4: "stride", 5: "i32_range", 6: "arg", 7: "device"}

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_LL = ctypes.c_longlong

# name -> (restype, argtypes); the order of arguments is that of include/mica_amd.h
SIGNATURES = {
    "mica_version": (_I, []),
    "mica_status_name": (ctypes.c_char_p, [_I]),
    "mica_device_info": (_I, [_I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "mica_act_quant": (_I, [_P, _I, _I, _P, _P, _I, _P, _I, _I, _I, _P]),
    "mica_rmsnorm_quant": (_I, [_P, _I, _I, _P, _I, _P, _I, _F, _F, _P, _P, _I, _P, _P, _I, _P, _I, _I, _I, _I,
                                _P]),
    "mica_rmsnorm_quant_multi": (_I, [_P, _I, _I, _P, _I, _P, _I, _F, _F, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I,
                                      _I, _P]),
    "mica_mm_i8": (_I, [_P, _I, _P, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P, _LL, _P]),
    "mica_mm_i8_workspace_bytes": (_LL, [_I]),
    "mica_mm_i8_noalloc": (_I, [_P, _I, _P, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P]),
    "mica_mm_i8_noalloc_scratch_bytes": (_LL, []),
    "mica_swiglu": (_I, [_P, _P, _P, _LL, _I, _P]),
    "mica_gather_logits": (_I, [_P, _I, _I, _P, _I, _P, _I, _F, _F, _P, _I, _I, _I, _P, _I, _I, _P, _P, _P, _P, _I,
                                _P]),
    "mica_rope_inplace": (_I, [_P, _LL, _I, _I, _P, _P, _I, _P, _I, _I, _P]),
    "mica_head_norm_rope": (_I, [_P, _LL, _I, _I, _I, _I, _I, _I, _P, _P, _F, _F, _I, _P, _P, _I, _P, _I, _P]),
    "mica_gate_quant": (_I, [_P, _LL, _P, _LL, _P, _LL, _P, _P, _LL, _I, _I, _I, _P]),
    "mica_attention_fwd": (_I, [_P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _I, _I,
                                _I, _I, _I, _I, _F, _I, _P, _LL, _P]),
    "mica_attention_workspace_bytes": (_LL, [_I, _I, _I]),
    "mica_attention_fwd_split": (_I, [_P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _I,
                                      _I, _I, _I, _I, _I, _F, _I, _I, _P, _LL, _P]),
    "mica_attention_split_workspace_bytes": (_LL, [_I, _I, _I, _I, _I, _I]),
    "mica_attention_fwd_kvlen": (_I, [_P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _I,
                                      _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _LL, _P]),
    "mica_attention_fwd_prefix": (_I, [_P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _P, _LL,
                                       _LL, _I, _P, _LL, _LL, _LL, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _LL,
                                       _P]),
    "mica_attention_prefix_workspace_bytes": (_LL, [_I, _I, _I, _I, _I, _I, _I]),
    "mica_attention_fwd_rope": (_I, [_P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _LL, _P, _LL, _LL, _P, _LL,
                                     _LL, _I, _P, _LL, _LL, _LL, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _F, _F,
                                     _I, _P, _P, _I, _P, _P, _LL, _P]),
    "mica_causal_conv1d": (_I, [_P, _LL, _I, _P, _P, _I, _I, _P, _P, _P, _LL, _I, _I, _I, _I, _I, _I, _F, _P]),
    "mica_gdn_chunk": (_I, [_P, _LL, _I, _P, _LL, _I, _P, _LL, _I, _P, _P, _I, _P, _P, _P, _F, _I, _I, _I, _I, _P,
                            _LL, _P]),
    "mica_gdn_workspace_bytes": (_LL, [_I, _I, _I]),
    "mica_gated_rmsnorm_quant": (_I, [_P, _I, _P, _I, _P, _F, _P, _I, _P, _I, _P, _I, _I, _P]),
    "mica_gdn_gate": (_I, [_P, _I, _P, _I, _P, _P, _P, _P, _I, _I, _P]),
}

_LIB = None
_LOCK = threading.Lock()


def lib_path() -> Path:
    d = os.environ.get(ENV_DIR)
    return (Path(d) if d else Path(__file__).resolve().parent) / LIB_NAME


def load():
    """Load (once) and return the ctypes library; raises RuntimeError if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            import torch  # noqa: F401  -- bind to torch's HIP runtime (see module docstring)

            path = lib_path()
            if not path.is_file():
                raise RuntimeError(f"{path} is not built; run `python -m mica_amd.build`")
            lib = ctypes.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _LIB = lib
    return _LIB


def status_name(rc: int) -> str:
    if rc > 0:
        return MISS_NAMES.get(rc, f"miss{rc}")
    return load().mica_status_name(rc).decode()


def check(rc: int, what: str) -> int:
    """Raise on a HIP error (rc < 0); return rc (0 = launched, > 0 = miss code)."""
    if rc < 0:
        raise RuntimeError(f"{what} failed: HIP error {-rc} {status_name(rc)}")
    return rc


def device_info(index: int = 0) -> dict:
    cu, clk, lds, arch = _I(), _I(), _I(), _I()
    check(load().mica_device_info(index, ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(lds),
                                  ctypes.byref(arch)), "mica_device_info")
    return {"cu_count": cu.value, "clock_khz": clk.value, "lds_per_block": lds.value, "gfx_arch": arch.value}
