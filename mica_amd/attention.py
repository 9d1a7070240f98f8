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


MAX_KEY_SPLITS = 64


def key_splits_for(B: int, Sq: int, Sk: int, HK: int, cus: int = 256, per_cu: int = 2, min_tiles: int = 8) -> int:
    """A split count for few query blocks over many keys: enough workgroups for per_cu per CU, each
    split keeping at least min_tiles key tiles of 32; 1 (no split) when the query blocks already fill
    the GPU."""
    blocks = HK * B * ((Sq + 31) // 32)
    want = -(-per_cu * cus // max(blocks, 1))
    most = max(1, ((Sk + 31) // 32) // min_tiles)
    return int(max(1, min(want, most, MAX_KEY_SPLITS)))


def attention_fwd(q, k, v, q_layout: str, scale: float | None = None, key_splits: int = 1, kv_len=None,
                  prefix=None, rope=None, head_norm=None):
    """Launch the kernel on q [B, Sq, HQ, 256] / k, v [B, Sk, HK, 256] ('bshd') or q [B, HQ, Sq, 256] /
    k, v [B, HK, Sk, 256] ('bhsd') views with unit feature stride.  Returns o in q's layout
    (contiguous [B, Sq, HQ, 256] memory), or raises ValueError on an unsupported input.

    key_splits > 1 divides each query block's keys over that many workgroups and merges their partial
    softmax states (mica_attention_fwd_split): faster for few query blocks over many keys, equal to the
    unsplit result within bf16 rounding but not bit for bit.

    kv_len (int32 [B] on the device, optional): sequence b's key count, clamped to Sq .. Sk; its queries
    are then the last Sq positions of its first kv_len[b] keys (mica_attention_fwd_kvlen), e.g. the last
    real position of each request of a batch padded to a common width.

    prefix ((kp, vp), optional, 'bshd' only): P keys shared by every sequence, [P, HK, 256] or
    [1, P, HK, 256] views, P a multiple of 32; k / v then hold each sequence's keys after them and the
    attention runs over the P + Sk keys as if concatenated (mica_attention_fwd_prefix, bit-identical to
    the concatenated call) without expanding the prefix to the batch.

    rope ((cos, sin, pos), optional, 'bshd' only, no kv_len): the rotary embedding of the new rows folded
    in (mica_attention_fwd_rope) over their first 2 * cos.shape[1] dims (64, 128 or 256).  cos / sin: bf16
    [n_pos, rot_dim / 2] tables; pos: int32 [B * Sq] positions on the device, or None for P + r (row r
    after a prefix of P keys).  Needs Sk = Sq (the new rows are the keys past the prefix).  head_norm
    ((q_norm_w, k_norm_w, offset, eps), optional, same conditions): each q / k head normed first,
    bf16((x rstd) (offset + w)), a weight of None skipping that side.  k is treated in place, exactly as
    ``fused_kernels.rope_inplace`` / ``head_norm_rope`` treat it; q as the kernel loads it, unchanged in
    memory.  The result equals those passes over q and k followed by the plain call, bit for bit."""
    for t in (q, k, v):
        if not t.is_cuda:
            raise ValueError("mica_amd attention runs on the GPU only (got a CPU tensor)")
        if t.dim() != 4 or t.dtype != torch.bfloat16 or t.shape[-1] != HEAD_DIM or t.stride(3) != 1:
            raise ValueError("q / k / v must be bf16 4-D tensors with head dim 256 and unit feature stride")
    dev = q.device
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    if q_layout == "bshd":
        (B, Sq, HQ, _), (_, Sk, HK, _) = q.shape, k.shape
        st = lambda t: (t.stride(0), t.stride(2), t.stride(1))  # noqa: E731  (batch, head, row)
    else:
        (B, HQ, Sq, _), (_, HK, Sk, _) = q.shape, k.shape
        st = lambda t: (t.stride(0), t.stride(1), t.stride(2))  # noqa: E731
    if k.shape != v.shape or k.shape[0] != B or HQ != GROUP * HK or Sk < Sq:
        raise ValueError("q / k / v shapes do not match (4 query heads per key/value head, Sk >= Sq)")
    P = 0
    if prefix is not None:
        kp, vp = (t[0] if t.dim() == 4 else t for t in prefix)
        if q_layout != "bshd":
            raise ValueError("a key prefix needs the 'bshd' layout")
        for t in (kp, vp):
            if (not t.is_cuda or t.device != dev or t.dim() != 3 or t.dtype != torch.bfloat16
                    or t.shape[1:] != (HK, HEAD_DIM) or t.stride(2) != 1):
                raise ValueError("prefix keys / values must be bf16 [P, HK, 256] views on q's device")
        P = kp.shape[0]
        if vp.shape != kp.shape or P % 32:
            raise ValueError("the prefix's keys and values must have one length, a multiple of 32")
        Sk += P
    fold = rope is not None or head_norm is not None
    cos = sin = rpos = None
    rot_dim, qnw, knw, noff, neps = 0, None, None, 0.0, 0.0
    if fold and (q_layout != "bshd" or kv_len is not None or Sk - P != Sq):
        raise ValueError("rope / head_norm need the 'bshd' layout, no kv_len, and one key per query row past "
                         "the prefix")
    if rope is not None:
        cos, sin, rpos = rope
        rot_dim = 2 * cos.shape[-1] if cos.dim() == 2 else 0
        for t in (cos, sin):
            if (not t.is_cuda or t.device != dev or t.dtype != torch.bfloat16 or t.dim() != 2
                    or rot_dim not in (64, 128, 256) or not t.is_contiguous()):
                raise ValueError("rope tables must be contiguous bf16 [n_pos, 32 | 64 | 128] tensors on q's device")
        if cos.shape != sin.shape:
            raise ValueError("rope cos / sin tables differ in shape")
        if rpos is not None and (rpos.dtype != torch.int32 or rpos.device != dev or rpos.numel() != B * Sq
                                 or not rpos.is_contiguous()):
            raise ValueError("rope positions must be a contiguous int32 [B * Sq] tensor on q's device")
    if head_norm is not None:
        qnw, knw, noff, neps = head_norm
        for t in (qnw, knw):
            if t is not None and (not t.is_cuda or t.device != dev or t.dtype != torch.bfloat16
                                  or t.numel() != HEAD_DIM or not t.is_contiguous()):
                raise ValueError("head norm weights must be contiguous bf16 [256] tensors on q's device")
    key_splits = int(key_splits)
    if not 1 <= key_splits <= MAX_KEY_SPLITS:
        raise ValueError(f"key_splits must be 1 .. {MAX_KEY_SPLITS}")
    o = torch.empty((B, Sq, HQ, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    L = _lib.load()
    nbytes = int(L.mica_attention_prefix_workspace_bytes(B, Sq, Sk, P, HQ, HK, key_splits))
    if nbytes < 0:
        raise ValueError("attention: invalid sizes")
    ws = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=dev)
    extra = [t for t in (cos, sin, qnw, knw) if t is not None]
    if not _aligned(q, k, v, o, ws, *((kp, vp) if P else ()), *extra):
        raise ValueError("attention operands must be 16-byte aligned")
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else float(scale)
    o_st = (o.stride(0), o.stride(2), o.stride(1))
    if kv_len is not None:
        if kv_len.dtype != torch.int32 or kv_len.device != dev or kv_len.numel() != B or not kv_len.is_contiguous():
            raise ValueError("kv_len must be a contiguous int32 [B] tensor on q's device")
    if fold:
        pk = (kp.data_ptr(), kp.stride(1), kp.stride(0), vp.data_ptr(), vp.stride(1), vp.stride(0)) if P else \
            (None, 0, 0, None, 0, 0)
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        rc = _lib.check(_on(dev, lambda: L.mica_attention_fwd_rope(
            q.data_ptr(), *st(q), k.data_ptr(), *st(k), v.data_ptr(), *st(v), *pk, P,
            o.data_ptr(), *o_st, B, Sq, Sk, HQ, HK, HEAD_DIM, scale, 1, key_splits,
            ptr(qnw), ptr(knw), float(noff), float(neps), rot_dim, ptr(cos), ptr(sin),
            0 if cos is None else cos.shape[0], ptr(rpos), ws.data_ptr(), nbytes, _stream(dev))),
            "mica_attention_fwd_rope")
    elif P:
        rc = _lib.check(_on(dev, lambda: L.mica_attention_fwd_prefix(
            q.data_ptr(), *st(q), k.data_ptr(), *st(k), v.data_ptr(), *st(v),
            kp.data_ptr(), kp.stride(1), kp.stride(0), vp.data_ptr(), vp.stride(1), vp.stride(0), P,
            o.data_ptr(), *o_st, B, Sq, Sk, HQ, HK, HEAD_DIM, scale, 1, key_splits,
            None if kv_len is None else kv_len.data_ptr(), ws.data_ptr(), nbytes, _stream(dev))),
            "mica_attention_fwd_prefix")
    elif kv_len is not None:
        rc = _lib.check(_on(dev, lambda: L.mica_attention_fwd_kvlen(
            q.data_ptr(), *st(q), k.data_ptr(), *st(k), v.data_ptr(), *st(v), o.data_ptr(), *o_st,
            B, Sq, Sk, HQ, HK, HEAD_DIM, scale, 1, key_splits, kv_len.data_ptr(), ws.data_ptr(), nbytes,
            _stream(dev))), "mica_attention_fwd_kvlen")
    elif key_splits == 1:
        rc = _lib.check(_on(dev, lambda: L.mica_attention_fwd(
            q.data_ptr(), *st(q), k.data_ptr(), *st(k), v.data_ptr(), *st(v), o.data_ptr(), *o_st,
            B, Sq, Sk, HQ, HK, HEAD_DIM, scale, 1, ws.data_ptr(), nbytes, _stream(dev))), "mica_attention_fwd")
    else:
        rc = _lib.check(_on(dev, lambda: L.mica_attention_fwd_split(
            q.data_ptr(), *st(q), k.data_ptr(), *st(k), v.data_ptr(), *st(v), o.data_ptr(), *o_st,
            B, Sq, Sk, HQ, HK, HEAD_DIM, scale, 1, key_splits, ws.data_ptr(), nbytes, _stream(dev))),
            "mica_attention_fwd_split")
    if rc:
        raise ValueError(f"attention: unsupported input ({_lib.status_name(rc)})")
    _launched()
    return o if q_layout == "bshd" else o.transpose(1, 2)


def causal_gqa_attention(q, k, v, scale: float | None = None, key_splits: int = 1, kv_len=None, prefix=None,
                         rope=None, head_norm=None):
    """softmax(scale q k^T, causal) v per sequence and head on [B, S, heads, 256] views (e.g. of the
    fused QKV output); query head h reads key/value head h // 4.  Returns o [B, S, HQ, 256] bf16.
    With Sk > Sq the queries are the last Sq positions; key_splits, kv_len, prefix, rope and head_norm as
    in attention_fwd."""
    return attention_fwd(q, k, v, "bshd", scale, key_splits, kv_len, prefix, rope, head_norm)
