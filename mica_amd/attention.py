"""Causal grouped-query attention forward on the gfx950 HIP kernel (head dim 256).

Replaces the attention of the reference's full-attention layers: its Triton kernel
(v0.5/serving/kernel_src/kernels.py:71-124, launched by int8_kernels.attn_fwd, int8_kernels.py:409-481)
and the torch SDPA path taken without it.  ``causal_gqa_attention(q, k, v)`` takes [B, S, heads, 256]
views -- typically of the fused QKV projection output, no copies -- with 4 query heads per key/value
head, and returns o [B, S, HQ, 256] bf16 (the O projection's [B * S, HQ * 256] rows).
GPU only; no fallback.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .int8_kernels import _aligned, _gpu_ok, _launched, _on, _stream

HEAD_DIM = 256
GROUP = 4


def _view(t, name):
    if t.dim() != 4 or t.dtype != torch.bfloat16 or t.shape[-1] != HEAD_DIM or t.stride(3) != 1 or \
            t.stride(2) != HEAD_DIM:
        raise ValueError(f"{name} must be bf16 [B, S, heads, 256] with contiguous heads")
    return t.stride(0), t.stride(1)


def causal_gqa_attention(q, k, v, scale: float | None = None, out=None):
    """softmax(scale q k^T, causal) v per sequence and head; query head h reads key/value head h // 4."""
    for t in (q, k, v):
        if not t.is_cuda:
            raise ValueError("mica_amd attention runs on the GPU only (got a CPU tensor)")
    dev = q.device
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    sbq, ldq = _view(q, "q")
    sbk, ldk = _view(k, "k")
    sbv, ldv = _view(v, "v")
    B, S, HQ, _ = q.shape
    HK = k.shape[2]
    if k.shape[:2] != (B, S) or v.shape[:3] != (B, S, HK) or HQ != GROUP * HK:
        raise ValueError("q / k / v shapes do not match (4 query heads per key/value head)")
    o = out if out is not None else torch.empty((B, S, HQ, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    if o.shape != (B, S, HQ, HEAD_DIM) or not o.is_contiguous():
        raise ValueError("out must be a contiguous bf16 [B, S, HQ, 256] tensor")
    L = _lib.load()
    nbytes = int(L.mica_attention_workspace_bytes(B, S, HK))
    ws = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=dev)
    if not _aligned(q, k, v, o, ws):
        raise ValueError("attention operands must be 16-byte aligned")
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else float(scale)
    sbo, ldo = o.stride(0), o.stride(1)
    rc = _lib.check(_on(dev, lambda: L.mica_attention_fwd(
        q.data_ptr(), sbq, ldq, k.data_ptr(), sbk, ldk, v.data_ptr(), sbv, ldv, o.data_ptr(), sbo, ldo,
        B, S, HQ, HK, HEAD_DIM, scale, 1, ws.data_ptr(), nbytes, _stream(dev))), "mica_attention_fwd")
    if rc:
        raise ValueError(f"causal_gqa_attention: unsupported input ({_lib.status_name(rc)})")
    _launched()
    return o
