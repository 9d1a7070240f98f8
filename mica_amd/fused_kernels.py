"""Drop-in replacement of the reference's ``fused_kernels`` (akivet/Mica v0.5/serving/lib/fused_kernels.py)
plus the fused RMSNorm + INT8 quantizer of the W8A8 hot path, on the gfx950 HIP kernels.

  rms_norm(x, weight, eps, residual=None)            fused_kernels.py:50-82
  swi_glu(gate, up)                                  fused_kernels.py:85-96
  rms_norm_quant(x, weight, eps, ...)                new: the norm and QLinear's act_quant in one pass
  rms_norm_quant_multi(x, weight, eps, inv_smooths)  new: one norm, quantized for up to 4 consumers
  rope_inplace(rows, n_heads, head_dim, cos, sin, period)  new: bf16 RoPE on QKV output rows, in place

The reference runs Triton here on a GPU and torch formulas on the CPU; mica_amd has no CPU compute
path: a CPU tensor raises ValueError (the reference raises ValueError for unsupported layouts, :57-58).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .int8_kernels import DT, ROUNDING, _aligned, _gpu_ok, _launched, _miss, _on, _stream

NORM_DT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16}


def _check_row_input(x, weight, residual):
    if not x.is_cuda:
        raise ValueError(
            f"mica_amd RMSNorm runs on the GPU only (got a tensor on {x.device}): this module has no CPU "
            "compute path; move x to a gfx950 GPU, or norm CPU rows with torch "
            "(v * rsqrt(mean(v^2) + eps) * (offset + w)) as the reference's rms_norm does there")
    if x.stride(-1) != 1:
        raise ValueError("fused RMSNorm requires unit feature stride")
    if x.dtype not in NORM_DT:
        raise ValueError(f"fused RMSNorm supports bf16/fp16 activations, got {x.dtype}")
    if weight.dtype not in DT or weight.numel() != x.shape[-1] or not weight.is_contiguous():
        raise ValueError("RMSNorm weight must be a contiguous [K] bf16/fp16/fp32 tensor")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype):
        raise ValueError("residual must match x in shape and dtype")


def _launch_norm(x, weight, eps, residual, offset, inv_smooth, want_q, want_y, rounding):
    K = x.shape[-1]
    flat = x.reshape(-1, K)
    if flat.stride(0) != K:
        flat = flat.contiguous()
    M = flat.shape[0]
    res = None
    if residual is not None:
        res = residual.reshape(-1, K)
        if not res.is_contiguous():
            res = res.contiguous()
    dev = x.device
    q = torch.empty((M, K), dtype=torch.int8, device=dev) if want_q else None
    s = torch.empty((M,), dtype=torch.float32, device=dev) if want_q else None
    y = torch.empty((M, K), dtype=x.dtype, device=dev) if want_y else None
    summed = torch.empty((M, K), dtype=x.dtype, device=dev) if res is not None else None
    tensors = [t for t in (flat, weight, res, q, s, y, summed, inv_smooth) if t is not None]
    if not _aligned(*tensors):
        raise ValueError("fused RMSNorm requires 16-byte aligned rows")
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    L = _lib.load()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = _lib.check(_on(dev, lambda: L.mica_rmsnorm_quant(
        ptr(flat), NORM_DT[x.dtype], K, ptr(res), K, ptr(weight), DT[weight.dtype], float(offset), float(eps),
        ptr(inv_smooth), ptr(q), K, ptr(s), ptr(y), K, ptr(summed), K, M, K, ROUNDING[rounding],
        _stream(dev))), "mica_rmsnorm_quant")
    if rc > 0:
        reason = _lib.status_name(rc)
        _miss("norm_" + reason)
        raise ValueError(f"fused RMSNorm does not support this input ({reason})")
    _launched()
    shape = x.shape
    return (q, s, None if y is None else y.view(shape), None if summed is None else summed.view(shape))


def rms_norm_quant_multi(x, weight, eps, inv_smooths, residual=None, offset=1.0, rounding="even"):
    """One RMSNorm of x, quantized per token for each of ``len(inv_smooths)`` (1 to 4) consumers,
    consumer i with its own SmoothQuant factors ``inv_smooths[i]`` (fp32 [K], or None): one read of x.

    Returns a list of (q_i, s_i), each equal to ``rms_norm_quant(x, weight, eps, inv_smooths[i], ...)``,
    plus the summed input v when ``residual`` is given: ([(q, s), ...], v).
    """
    _check_row_input(x, weight, residual)
    K = x.shape[-1]
    n = len(inv_smooths)
    if not 1 <= n <= 4:
        raise ValueError("rms_norm_quant_multi takes 1 to 4 consumers")
    for inv in inv_smooths:
        if inv is not None and (inv.dtype != torch.float32 or inv.numel() != K or not inv.is_contiguous()
                                or inv.device != x.device):
            raise ValueError("each inv_smooth must be None or a contiguous fp32 [K] tensor on x's device")
    flat = x.reshape(-1, K)
    if flat.stride(0) != K:
        flat = flat.contiguous()
    M = flat.shape[0]
    res = None
    if residual is not None:
        res = residual.reshape(-1, K)
        if not res.is_contiguous():
            res = res.contiguous()
    dev = x.device
    qs = [torch.empty((M, K), dtype=torch.int8, device=dev) for _ in range(n)]
    ss = [torch.empty((M,), dtype=torch.float32, device=dev) for _ in range(n)]
    summed = torch.empty((M, K), dtype=x.dtype, device=dev) if res is not None else None
    tensors = [t for t in [flat, weight, res, summed, *qs, *ss, *inv_smooths] if t is not None]
    if not _aligned(*tensors):
        raise ValueError("fused RMSNorm requires 16-byte aligned rows")
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    L = _lib.load()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    P = ctypes.c_void_p
    invs = (P * n)(*[ptr(t) for t in inv_smooths])
    qp = (P * n)(*[t.data_ptr() for t in qs])
    sp = (P * n)(*[t.data_ptr() for t in ss])
    ldq = (ctypes.c_int * n)(*([K] * n))
    rc = _lib.check(_on(dev, lambda: L.mica_rmsnorm_quant_multi(
        ptr(flat), NORM_DT[x.dtype], K, ptr(res), K, ptr(weight), DT[weight.dtype], float(offset), float(eps), n,
        invs, qp, ldq, sp, None, K, ptr(summed), K, M, K, ROUNDING[rounding], _stream(dev))),
        "mica_rmsnorm_quant_multi")
    if rc > 0:
        reason = _lib.status_name(rc)
        _miss("norm_" + reason)
        raise ValueError(f"fused RMSNorm does not support this input ({reason})")
    _launched()
    out = list(zip(qs, ss))
    return out if residual is None else (out, summed.view(x.shape))


def rms_norm(x, weight, eps, residual=None, offset=1.0):
    """y = bf16((v * rsqrt(mean(v^2) + eps)) * (offset + w)), v = x (+ residual rounded to x's dtype).

    Returns y, or (y, v) with a residual (fused_kernels.py:50-82).  offset=1.0 is the reference's
    Qwen3.5 ``(1 + weight)``.

    GPU tensors only: where the reference computes its torch formula for a CPU tensor
    (fused_kernels.py:51-56), this raises ValueError naming the device, so a CPU caller has to norm
    its rows itself.
    """
    _check_row_input(x, weight, residual)
    _, _, y, summed = _launch_norm(x, weight, eps, residual, offset, None, False, True, "even")
    return y if residual is None else (y, summed)


def rms_norm_quant(x, weight, eps, inv_smooth=None, residual=None, offset=1.0, rounding="even",
                   return_normed=False):
    """RMSNorm + per-token INT8 quantization in one read of x.

    Equals ``int8_kernels.act_quant(rms_norm(x, weight, eps, residual), inv_smooth)``: q int8 [M, K]
    and s fp32 [M] over the flattened rows.  Returns (q, s), plus the bf16 normed rows when
    ``return_normed``, plus the summed input v when ``residual`` is given: (q, s[, y][, v]).
    """
    _check_row_input(x, weight, residual)
    K = x.shape[-1]
    if inv_smooth is not None and (inv_smooth.dtype != torch.float32 or inv_smooth.numel() != K
                                   or not inv_smooth.is_contiguous() or inv_smooth.device != x.device):
        raise ValueError("inv_smooth must be a contiguous fp32 [K] tensor on x's device")
    q, s, y, summed = _launch_norm(x, weight, eps, residual, offset, inv_smooth, True, return_normed, rounding)
    out = (q, s)
    if return_normed:
        out += (y,)
    if residual is not None:
        out += (summed,)
    return out


def swi_glu(gate, up):
    """y = bf16(bf16(silu(gate)) * up), elementwise on bf16 (fused_kernels.py:85-96)."""
    if not gate.is_cuda:
        raise ValueError("mica_amd swi_glu runs on the GPU only (got a CPU tensor)")
    if not gate.is_contiguous() or not up.is_contiguous():
        raise ValueError("fused gate-up kernel requires dense projections")
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16 or gate.shape != up.shape:
        raise ValueError("swi_glu takes two bf16 tensors of one shape")
    y = torch.empty_like(gate)
    if not _aligned(gate, up, y):
        raise ValueError("swi_glu requires 16-byte aligned tensors")
    L = _lib.load()
    dev = gate.device
    rc = _lib.check(_on(dev, lambda: L.mica_swiglu(gate.data_ptr(), up.data_ptr(), y.data_ptr(), gate.numel(),
                                                   _lib.BF16, _stream(dev))), "mica_swiglu")
    if rc > 0:
        raise ValueError(f"swi_glu does not support this input ({_lib.status_name(rc)})")
    _launched()
    return y


def rope_inplace(rows, n_heads: int, head_dim: int, cos_tab, sin_tab, period: int | None = None, pos=None):
    """Rotate the first n_heads heads of every row of ``rows`` ([T, >= n_heads * head_dim] bf16, unit
    feature stride) in place: bf16(bf16(x cos) + bf16(rotate_half(x) sin)) as transformers'
    apply_rotary_pos_emb computes it in bf16.  cos_tab / sin_tab: bf16 [n_pos, head_dim / 2].
    Row t has position pos[t] (int32 tensor) or t % period."""
    if not rows.is_cuda:
        raise ValueError("mica_amd RoPE runs on the GPU only (got a CPU tensor)")
    if rows.dim() != 2 or rows.dtype != torch.bfloat16 or rows.stride(1) != 1:
        raise ValueError("rope_inplace expects bf16 [T, C] rows with unit feature stride")
    if cos_tab.dtype != torch.bfloat16 or sin_tab.dtype != torch.bfloat16 or cos_tab.shape != sin_tab.shape or \
            cos_tab.shape[1] != head_dim // 2 or not cos_tab.is_contiguous() or not sin_tab.is_contiguous():
        raise ValueError("cos / sin tables must be contiguous bf16 [n_pos, head_dim / 2]")
    if pos is not None and (pos.dtype != torch.int32 or not pos.is_contiguous() or pos.numel() != rows.shape[0]):
        raise ValueError("pos must be a contiguous int32 [T] tensor")
    if pos is None and not period:
        raise ValueError("give pos or period")
    dev = rows.device
    if not _aligned(rows, cos_tab, sin_tab):
        raise ValueError("rope_inplace requires 16-byte aligned rows and tables")
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    L = _lib.load()
    rc = _lib.check(_on(dev, lambda: L.mica_rope_inplace(
        rows.data_ptr(), rows.stride(0), n_heads, head_dim, cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
        None if pos is None else pos.data_ptr(), int(period or 0), rows.shape[0], _stream(dev))), "mica_rope_inplace")
    if rc:
        raise ValueError(f"rope_inplace: unsupported input ({_lib.status_name(rc)})")
    _launched()
    return rows


def head_norm_rope(rows, head_dim: int, q_heads, k_heads, q_norm_w=None, k_norm_w=None, eps: float = 1e-6,
                   offset: float = 1.0, rot_dim: int = 0, cos_tab=None, sin_tab=None, period: int | None = None,
                   pos=None):
    """In place on bf16 rows [T, C] (unit feature stride): the q / k head RMSNorm and partial RoPE of the
    reference model's full-attention layers (fast_runtime.py:229-236; rope_one, prefill_engine.py:83-89).
    q_heads = (column offset, head count) of the query heads, k_heads likewise; each head of head_dim
    values is normed when its segment's weight (bf16 [head_dim]) is given,
    y = bf16((x * rstd) * (offset + w)) (offset 1: the zero-centred Qwen3.5 RMSNorm), then its first
    rot_dim dims are rotated (cos_tab / sin_tab bf16 [n_pos, rot_dim / 2]; row t at position pos[t] or
    t % period).  One launch (mica_head_norm_rope)."""
    if not rows.is_cuda:
        raise ValueError("mica_amd head norm + RoPE runs on the GPU only (got a CPU tensor)")
    if rows.dim() != 2 or rows.dtype != torch.bfloat16 or rows.stride(1) != 1:
        raise ValueError("head_norm_rope expects bf16 [T, C] rows with unit feature stride")
    for w in (q_norm_w, k_norm_w):
        if w is not None and (w.dtype != torch.bfloat16 or w.numel() != head_dim or not w.is_contiguous()
                              or w.device != rows.device):
            raise ValueError("norm weights must be contiguous bf16 [head_dim] tensors on the rows' device")
    if rot_dim:
        if cos_tab is None or sin_tab is None or cos_tab.dtype != torch.bfloat16 or cos_tab.shape != sin_tab.shape \
                or cos_tab.shape[1] != rot_dim // 2 or not cos_tab.is_contiguous() or not sin_tab.is_contiguous():
            raise ValueError("cos / sin tables must be contiguous bf16 [n_pos, rot_dim / 2]")
        if pos is not None and (pos.dtype != torch.int32 or not pos.is_contiguous() or pos.numel() != rows.shape[0]):
            raise ValueError("pos must be a contiguous int32 [T] tensor")
        if pos is None and not period:
            raise ValueError("give pos or period")
    dev = rows.device
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    L = _lib.load()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = _lib.check(_on(dev, lambda: L.mica_head_norm_rope(
        rows.data_ptr(), rows.stride(0), rows.shape[0], int(q_heads[0]), int(q_heads[1]), int(k_heads[0]),
        int(k_heads[1]), head_dim, ptr(q_norm_w), ptr(k_norm_w), float(offset), float(eps), int(rot_dim),
        ptr(cos_tab), ptr(sin_tab), 0 if cos_tab is None else cos_tab.shape[0], ptr(pos), int(period or 0),
        _stream(dev))), "mica_head_norm_rope")
    if rc:
        raise ValueError(f"head_norm_rope: unsupported input ({_lib.status_name(rc)})")
    _launched()
    return rows


def gate_quant(a, gate, return_gated: bool = False):
    """o_proj's input from the attention output: y = bf16(a * bf16(sigmoid(gate))) (the output gate of
    the full-attention layers, fast_runtime.py:240), quantized per token (int8_quant.quant_act, half even)
    in the same pass.  a, gate: bf16 [M, K] with unit feature stride (gate may be a strided view of the
    QKV projection output), K a multiple of 512.  Returns (q int8 [M, K], s fp32 [M]) and, with
    return_gated, the bf16 gated rows y."""
    for t in (a, gate):
        if not t.is_cuda:
            raise ValueError("mica_amd gate + quant runs on the GPU only (got a CPU tensor)")
        if t.dim() != 2 or t.dtype != torch.bfloat16 or t.stride(1) != 1:
            raise ValueError("gate_quant expects bf16 [M, K] tensors with unit feature stride")
    if a.shape != gate.shape or gate.device != a.device:
        raise ValueError("a and gate must have one shape and device")
    M, K = a.shape
    dev = a.device
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, K), dtype=torch.bfloat16, device=dev) if return_gated else None
    if not _aligned(a, gate, q, s, *(() if y is None else (y,))):
        raise ValueError("gate_quant requires 16-byte aligned rows")
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    L = _lib.load()
    rc = _lib.check(_on(dev, lambda: L.mica_gate_quant(
        a.data_ptr(), a.stride(0), gate.data_ptr(), gate.stride(0), q.data_ptr(), K, s.data_ptr(),
        None if y is None else y.data_ptr(), K, M, K, ROUNDING["even"], _stream(dev))), "mica_gate_quant")
    if rc:
        raise ValueError(f"gate_quant: unsupported input ({_lib.status_name(rc)})")
    _launched()
    return (q, s, y) if return_gated else (q, s)
