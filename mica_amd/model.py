"""A 4B-shaped decoder stack whose linear layers run on the W8A8 hot path, for prefill-only scoring.

Shape (the benchmark's synthetic 4B configuration): 36 layers, hidden 2560, MLP intermediate 9728,
16 query heads and 4 K/V heads of dim 256 (QKV projection N = 4096 + 2 x 1024 = 6144), vocabulary
151936.  Weights are random int8 with per-output-channel fp32 scales; norms are gamma-style RMSNorm
weights.  With ``full_attention_interval = k > 0`` the stack is the hybrid layout of the reference's
model instead (Qwen3.5: three gated-delta-net layers, then one full-attention layer, repeated).

Weights are random.  By default the full-attention layers are the benchmark's plain shape (QKV
N = 6144, RoPE over the whole head).  StackConfig.reference_model() (or the flags attn_output_gate,
qk_norm, rotary_dim) gives them the reference model's computation (fast_runtime.py:229-241): q_proj also
produces an output gate per head (QKV rows [q | gate | k | v], N = 10240), the q and k heads are
RMSNormed per head (zero-centred weight) and rotated on their first 64 dims (one head_norm_rope launch
in place of the RoPE), and the attention output is gated, o * sigmoid(gate), in the kernel that quantizes
it for the O projection (gate_quant, in place of act_quant).  Per full-attention layer (the call pattern
of the reference's fork.layer_step, v0.5/serving/lib/fork.py:394-422):
  q, s   = rms_norm_quant(h, input_norm)                     1 launch
  qkv    = QKV W8A8 GEMM                                     1 launch
  a      = causal GQA attention per request: RoPE in place on the q / k heads, then the
           flash-attention kernel (head dim 256, 4 query heads per K/V head)   3 launches
  h      = h + O W8A8(a)          (residual in the epilogue)  2 launches (act_quant + GEMM)
  q, s   = rms_norm_quant(h, post_attention_norm)            1 launch
  g      = fused gate+up GEMM, SiLU(gate) * up epilogue      1 launch
  h      = h + down W8A8(act_quant(g))                       2 launches
A gated-delta-net layer replaces the first four steps with mica_amd.gdn.GDNLayer (fork.gdn_step,
fork.py:20-149: one norm + quant for the four input projections, conv, gate, chunked scan, gated
norm fused with out_proj's quantisation, out_proj with the residual).
The last layer runs last-only, as the reference's PrefillEngine does by default (last_only=True,
prefill_engine.py:181, 283-339): its input norm + quant, K / V projection and RoPE of the keys cover
every row (the picked queries attend to all of them), while the query projection, attention, O
projection, post-attention norm and MLP run on the B picked rows only; a GDN last layer runs its mixer
over every row and the MLP on the picked rows.  Each picked row's values are bit-identical to those of
the full layer (rows of a GEMM are independent and the attention kernel's per-query arithmetic is the
same; W8A8Stack(last_only=False) runs the full layer).
Then, as PrefillEngine.final + the readout do (prefill_engine.py:280-304, release_runtime.py:298-306,
:509-517), only each request's last position is normed and dotted with the allowed label rows, and
the option slice is softmaxed.  Requests are packed back to back, all of the same length.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import int8_kernels as aot
from .attention import GROUP as _FA_GROUP, HEAD_DIM as _FA_DIM, causal_gqa_attention, key_splits_for
from .fused_kernels import gate_quant, head_norm_rope, rms_norm_quant, rope_inplace
from .gdn import HEAD_DIM as _GDN_DIM, GDNLayer
from .int8_runtime import GateUpQLinear, QLinear
from .readout import LabelReadout


@dataclass
class StackConfig:
    layers: int = 36
    hidden: int = 2560
    intermediate: int = 9728
    heads: int = 16       # the reference's full-attention layers: 16 query / 4 K/V heads of 256
    kv_heads: int = 4     # (kernel_src/kernels.py:5, 71-124); QKV 6144 = (16 + 2 * 4) * 256
    head_dim: int = 256
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    n_options: int = 255   # option labels after the No / Yes pair (mica/codebook.py:19)
    # 0: every layer is full attention.  k > 0: layer i is full attention when (i + 1) % k == 0 and a
    # gated-delta-net layer otherwise (the reference's model: k = 4, 16 key / 32 value heads of 128)
    full_attention_interval: int = 0
    linear_k_heads: int = 16
    linear_v_heads: int = 32
    conv_width: int = 4
    # the reference model's full-attention extras (fast_runtime.py:229-241): q_proj's per-head output gate
    # o * sigmoid(gate), the per-head q / k RMSNorm (zero-centred weights), RoPE on the first rotary_dim
    # dims of each head (0: all of them)
    attn_output_gate: bool = False
    qk_norm: bool = False
    rotary_dim: int = 0

    def is_gdn(self, i: int) -> bool:
        return self.full_attention_interval > 0 and (i + 1) % self.full_attention_interval != 0

    @property
    def rot_dim(self) -> int:
        return self.rotary_dim or self.head_dim

    @classmethod
    def reference_model(cls, **overrides) -> "StackConfig":
        """The reference model's layer layout and attention (Qwen3.5, as served): 32 layers, every fourth
        full attention (16 / 4 heads of 256 with the output gate, q / k norm, RoPE on 64 dims, theta 1e7),
        the others gated-delta-net layers (16 key / 32 value heads of 128), hidden 2560, MLP 9728."""
        base = dict(layers=32, full_attention_interval=4, attn_output_gate=True, qk_norm=True, rotary_dim=64,
                    rope_theta=10_000_000.0)
        base.update(overrides)
        return cls(**base)


_CUS = {}


def _cu_count(device) -> int:
    """Compute units of a CUDA device (cached per device index)."""
    i = torch.device(device).index or 0
    if i not in _CUS:
        _CUS[i] = torch.cuda.get_device_properties(i).multi_processor_count
    return _CUS[i]


def _rand_qlinear(n, k, g, device):
    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8, device=device)
    sw = torch.empty(n, device=device).uniform_(1e-3, 1e-2, generator=g)
    return QLinear.from_quantized(qw, sw)


def _rand_norm(n, g, device):
    return (torch.randn(n, generator=g, device=device) * 0.1 + 1.0).to(torch.bfloat16)


class Layer:
    """A full-attention decoder layer's weights."""

    def __init__(self, cfg: StackConfig, g, device):
        H = cfg.hidden
        self.cfg = cfg
        self.input_norm = _rand_norm(H, g, device)
        self.post_norm = _rand_norm(H, g, device)
        # fused projection rows: [q | gate | k | v] (the gate rows only with attn_output_gate)
        nq = cfg.heads * cfg.head_dim * (2 if cfg.attn_output_gate else 1)
        self.qkv = _rand_qlinear(nq + 2 * cfg.kv_heads * cfg.head_dim, H, g, device)
        self.o = _rand_qlinear(H, cfg.heads * cfg.head_dim, g, device)
        _mlp_weights(self, cfg, g, device)
        # the per-head norms' zero-centred weights (the norm multiplies by 1 + w)
        self.q_norm = self.k_norm = None
        if cfg.qk_norm:
            self.q_norm = (torch.randn(cfg.head_dim, generator=g, device=device) * 0.1).to(torch.bfloat16)
            self.k_norm = (torch.randn(cfg.head_dim, generator=g, device=device) * 0.1).to(torch.bfloat16)
        # the last-only pass's two projections: views of the fused weight's query (+ gate) rows and K / V rows
        self.q_rows = QLinear.from_quantized(self.qkv.qweight[:nq], self.qkv.wscale[:nq])
        self.kv_rows = QLinear.from_quantized(self.qkv.qweight[nq:], self.qkv.wscale[nq:])


def _mlp_weights(layer, cfg, g, device):
    gate = _rand_qlinear(cfg.intermediate, cfg.hidden, g, device)
    up = _rand_qlinear(cfg.intermediate, cfg.hidden, g, device)
    layer.gate_up = GateUpQLinear(gate, up)
    layer.down = _rand_qlinear(cfg.hidden, cfg.intermediate, g, device)


class GDNBlock:
    """A gated-delta-net decoder layer's weights: the token mixer (a GDNLayer with random int8
    projections, conv taps, decay parameters and gated-norm weight) and the same MLP."""

    def __init__(self, cfg: StackConfig, g, device):
        H, D = cfg.hidden, _GDN_DIM
        hk, hv = cfg.linear_k_heads, cfg.linear_v_heads
        C = (2 * hk + hv) * D
        self.cfg = cfg
        self.mixer = GDNLayer(
            norm_weight=_rand_norm(H, g, device), eps=cfg.eps,
            in_qkv=_rand_qlinear(C, H, g, device), in_z=_rand_qlinear(hv * D, H, g, device),
            in_b=_rand_qlinear(hv, H, g, device), in_a=_rand_qlinear(hv, H, g, device),
            conv_weight=(torch.randn(C, cfg.conv_width, generator=g, device=device) * 0.5).to(torch.bfloat16),
            A_log=torch.rand(hv, generator=g, device=device) * 2 - 1,
            dt_bias=torch.randn(hv, generator=g, device=device) * 0.5,
            norm_z_weight=_rand_norm(D, g, device), out_proj=_rand_qlinear(H, hv * D, g, device),
            num_k_heads=hk, num_v_heads=hv, norm_offset=0.0, z_eps=cfg.eps)
        self.post_norm = _rand_norm(H, g, device)
        _mlp_weights(self, cfg, g, device)


def _norm_quant(h, w, eps, keep_normed):
    """The layer's fused RMSNorm (zero-centred weight: offset 0 on the stored 1 + w) + int8 quant:
    (q, s, None), or (q, s, y) with the bf16 normed rows kept for a trace."""
    if keep_normed:
        return rms_norm_quant(h, w, eps, offset=0.0, return_normed=True)
    q, s = rms_norm_quant(h, w, eps, offset=0.0)
    return q, s, None


def _rope(S, head_dim, theta, device):
    """RoPE tables (fp32 angles, then bf16 as the model's dtype): cos, sin as bf16 [S, head_dim / 2]."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    ang = torch.arange(S, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang).to(torch.bfloat16).contiguous(), torch.sin(ang).to(torch.bfloat16).contiguous()


def _apply_rope(x, cos, sin):
    """The same rotation as torch bf16 ops (a test reference for ``rope_inplace``): x [B, S, heads, d],
    x * (cos, cos) + rotate_half(x) * (-sin, sin), each op rounded to bf16."""
    h = x.shape[-1] // 2
    cs = torch.cat((cos, cos), -1)[None, :, None, :]
    sn = torch.cat((-sin, sin), -1)[None, :, None, :]
    return x * cs + torch.cat((x[..., h:], x[..., :h]), -1) * sn


# A prompt prefix whose length is a multiple of this continues bit-identically: the GDN scan's chunks
# (64 tokens) and the attention kernel's key tiles (32) fall on the same boundaries as in a full run.
PREFIX_ALIGN = 64


class PrefixState:
    """What a prompt prefix of `length` tokens leaves in every layer, for the rest of the prompt to
    continue from (the reference engine's header state, prefill_engine.py:218-226): an attention layer's
    rotated keys and values [1, length, kv_heads, head_dim], a GDN layer's (conv state [1, C, W - 1],
    recurrent state [1, HV, 128, 128] fp32).  Shared by any number of continuations."""

    def __init__(self, length: int, layers: list):
        self.length, self.layers = int(length), layers
        self.positions = {}   # (batch, S) -> int32 [batch * S] RoPE positions of a captured continuation

    def positions_for(self, batch: int, S: int, device):
        """RoPE positions length + (t % S) of a packed continuation batch.  Made during a HIP-graph
        capture, they are kept with the prefix (the graph reads them on every replay), so the kept set
        is bounded by the captured shapes; an eager run makes them for that call only."""
        key = (batch, S)
        if key in self.positions:
            return self.positions[key]
        pos = (torch.arange(batch * S, device=device, dtype=torch.int32) % S + self.length).contiguous()
        if torch.device(device).type == "cuda" and torch.cuda.is_current_stream_capturing():
            self.positions[key] = pos
        return pos


class W8A8Stack:
    """Random-init 4B-shaped stack; `prefill(ids, batch)` returns option probabilities."""

    def __init__(self, cfg: StackConfig = StackConfig(), device="cuda", seed=0, attention: str = "mica",
                 split_keys: bool = False, last_only: bool = True):
        self.cfg = cfg
        self.attention = attention
        # the last layer at the picked rows only (prefill_engine.py:181, 283-339); same bits per row
        self.last_only = last_only
        # continuations over a prefix (Sk > S): divide each query block's keys over several workgroups
        # (attention.key_splits_for).  Off by default: the continuation then matches a full run within
        # bf16 rounding instead of bit for bit.
        self.split_keys = split_keys
        # whole-head RoPE inside the attention kernel (mica_attention_fwd_rope) instead of a pass of its own
        self.fuse_rope = True
        self.device = torch.device(device)
        g = torch.Generator(device=self.device).manual_seed(seed)
        H = cfg.hidden
        self.embed = (torch.randn(cfg.vocab, H, generator=g, device=self.device) * 0.5).to(torch.bfloat16)
        self.layers = [(GDNBlock if cfg.is_gdn(i) else Layer)(cfg, g, self.device) for i in range(cfg.layers)]
        self.final_norm = _rand_norm(H, g, self.device)
        self.lm_head = (torch.randn(cfg.vocab, H, generator=g, device=self.device) * 0.02).to(torch.bfloat16)
        ids = torch.randperm(cfg.vocab, generator=torch.Generator().manual_seed(seed))[: 2 + cfg.n_options]
        self.label_ids = ids.to(self.device)
        self.readout = LabelReadout(self.lm_head, self.label_ids)
        self._rope = None     # (cos, sin) of positions 0 .. size - 1, grown by doubling
        self._retired = []    # earlier tables: a captured graph may still read them

    def _tables(self, n, device):
        """cos / sin of positions 0 .. n - 1: the first n rows of one table, which is regrown (doubled)
        when a longer sequence comes, so memory stays within twice the longest sequence seen.  Every
        entry depends only on its position, so a row is the same in every table."""
        if self._rope is None or self._rope[0].shape[0] < n:
            size = max(n, 4096 if self._rope is None else 2 * self._rope[0].shape[0])
            if self._rope is not None:
                self._retired.append(self._rope)
            self._rope = _rope(size, self.cfg.rot_dim, self.cfg.rope_theta, device)
        cos, sin = self._rope
        return cos[:n], sin[:n]

    def _attention(self, qkv, B, S, past=None, keep=False, pos=None, norms=(None, None), fuse_rope=True):
        """Causal GQA attention per request.  RoPE rotates the q and k heads of the QKV output in place
        (one kernel); the flash-attention kernel (head dim 256, 4 query heads per K/V head) then reads
        [B, S, heads, d] views of it and writes [B, S, heads, d]-contiguous output, i.e. already the O
        projection's [T, heads * d] rows.  Other head shapes, or attention="sdpa", use torch SDPA on the
        same views (enable_gqa, transposed strides, no copies).

        past: (k, v) of a prefix of P tokens; the S rows are then positions P .. P + S - 1 and attend to
        the prefix's keys too (Sk = P + S keys, the queries being the last S); pos: their int32 RoPE
        positions (PrefixState.positions_for).  keep: also return this call's rotated (k, v),
        contiguous (batch 1: a prefix being recorded); norms: the layer's (q_norm, k_norm) weights.

        The attention kernel applies the head norm and the rotation itself (mica_attention_fwd_rope: k in
        place, q as it is loaded, bit-identical to rope_inplace / head_norm_rope first) unless fuse_rope is
        False or self.fuse_rope is off; q then stays untreated in qkv."""
        cfg = self.cfg
        hq, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
        ng = hq if cfg.attn_output_gate else 0          # gate heads between the q and the k heads
        P = 0 if past is None else past[0].shape[1]
        cos, sin = self._tables(P + S, qkv.device)
        mica = self.attention == "mica" and d == _FA_DIM and hq == _FA_GROUP * hk
        # the keys read in place (no prefix, or a tile-aligned one): the kernel norms and rotates
        fused = (mica and fuse_rope and self.fuse_rope and cfg.rot_dim in (64, 128, 256) and P % 32 == 0
                 and (P == 0 or pos is not None))
        if not fused:
            self._rotate(qkv, (0, hq), (ng * d + hq * d, hk), cos, sin, S if P == 0 else None,
                         None if P == 0 else pos, norms)
        q, _, k, v = qkv.view(B, S, hq + ng + 2 * hk, d).split((hq, ng, hk, hk), dim=2)
        state = (k.contiguous(), v.contiguous()) if keep and not fused else None
        if fused:
            ks = key_splits_for(B, S, P + S, hk, cus=_cu_count(qkv.device)) if P and self.split_keys else 1
            hn = (norms[0], norms[1], 1.0, cfg.eps) if cfg.qk_norm else None
            a = causal_gqa_attention(q, k, v, 1.0 / math.sqrt(d), key_splits=ks, prefix=past if P else None,
                                     rope=(cos, sin, pos if P else None), head_norm=hn).view(B * S, hq * d)
            if keep:
                state = (k.contiguous(), v.contiguous())
        elif mica:
            ks = 1
            if P and self.split_keys:
                ks = key_splits_for(B, S, P + S, hk, cus=_cu_count(qkv.device))
            # a tile-aligned prefix's keys are read in place, shared by the batch's rows
            pre = past if P and P % 32 == 0 else None
            if P and pre is None:
                k = torch.cat((past[0].expand(B, -1, -1, -1), k), dim=1)
                v = torch.cat((past[1].expand(B, -1, -1, -1), v), dim=1)
            a = causal_gqa_attention(q, k, v, 1.0 / math.sqrt(d), key_splits=ks, prefix=pre).view(B * S, hq * d)
        else:
            if P:
                k = torch.cat((past[0].expand(B, -1, -1, -1), k), dim=1)
                v = torch.cat((past[1].expand(B, -1, -1, -1), v), dim=1)
            a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                               is_causal=P == 0, attn_mask=None if P == 0 else self._mask(S, P, q.device),
                                               scale=1.0 / math.sqrt(d), enable_gqa=True)
            a = a.transpose(1, 2).reshape(B * S, hq * d).contiguous()
        return (a, state) if keep else a

    def _plain_rope(self) -> bool:
        """RoPE over whole heads and no head norm: the rope_inplace kernel serves it."""
        return not self.cfg.qk_norm and self.cfg.rot_dim == self.cfg.head_dim

    def _rotate(self, rows, q_heads, k_heads, cos, sin, period=None, pos=None, norms=(None, None)):
        """The q / k heads of the projection rows, in place: RoPE (rope_inplace) when the q heads come
        right before the k heads, the heads are rotated whole and not normed; else the head norm (when
        configured) and RoPE on the first rot_dim dims in one head_norm_rope launch.  q_heads / k_heads:
        (column offset, head count); norms: the layer's (q_norm, k_norm) weights or Nones."""
        cfg = self.cfg
        d = cfg.head_dim
        nq, nk = q_heads[1], k_heads[1]
        if self._plain_rope() and (nq == 0 or nk == 0 or k_heads[0] == q_heads[0] + nq * d):
            first = q_heads[0] if nq else k_heads[0]
            view = rows[:, first:] if first else rows
            rope_inplace(view, nq + nk, d, cos, sin, period=period, pos=pos)
            return
        head_norm_rope(rows, d, q_heads, k_heads, norms[0], norms[1], cfg.eps, 1.0, cfg.rot_dim, cos, sin,
                       period=period, pos=pos)

    def _o_input(self, a, gate, keep_gated=False):
        """O projection's int8 input (q, s, gated rows or None): the attention output quantized per
        token, gated first with the output gate when the layers have one (gate_quant; with keep_gated the
        bf16 gated rows too, for a trace)."""
        if gate is None:
            q, s = aot.act_quant(a)
            return q, s, None
        if keep_gated:
            return gate_quant(a, gate, return_gated=True)
        q, s = gate_quant(a, gate)
        return q, s, None

    def _attention_rows(self, qr, kv, B, S, rows, past=None, pos=None, norms=(None, None)):
        """Attention of the last-only pass: one query per request, the picked row rows[b] (int32, a row
        of the packed [B * S] batch), over its request's keys.  qr: the picked rows' query projection
        [B, heads * d]; kv: every row's K / V projection [B * S, 2 * kv_heads * d].  RoPE rotates the
        keys of every row (positions as in _attention) and each query at its own position; the query of
        request b, at position p_b = rows[b] - b S (+ the prefix length), sees keys 0 .. p_b, i.e.
        kv_len[b] = p_b + 1 (the reference's key limit, prefill_engine.py:332-336).  Returns
        [B, heads * d]."""
        cfg = self.cfg
        hq, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
        P = 0 if past is None else past[0].shape[1]
        cos, sin = self._tables(P + S, kv.device)
        self._rotate(kv, (0, 0), (0, hk), cos, sin, S if P == 0 else None, None if P == 0 else pos, norms)
        qpos = (rows - torch.arange(B, device=rows.device, dtype=torch.int32) * S + P).to(torch.int32)
        self._rotate(qr, (0, hq), (0, 0), cos, sin, pos=qpos, norms=norms)
        k, v = kv.view(B, S, 2 * hk, d).split((hk, hk), dim=2)
        q = qr[:, :hq * d].view(B, 1, hq, d)
        kv_len = (qpos + 1).to(torch.int32)
        if self.attention == "mica" and d == _FA_DIM and hq == _FA_GROUP * hk:
            pre = past if P and P % 32 == 0 else None
            if P and pre is None:
                k = torch.cat((past[0].expand(B, -1, -1, -1), k), dim=1)
                v = torch.cat((past[1].expand(B, -1, -1, -1), v), dim=1)
            return causal_gqa_attention(q, k, v, 1.0 / math.sqrt(d), kv_len=kv_len, prefix=pre).view(B, hq * d)
        if P:
            k = torch.cat((past[0].expand(B, -1, -1, -1), k), dim=1)
            v = torch.cat((past[1].expand(B, -1, -1, -1), v), dim=1)
        seen = torch.arange(P + S, device=q.device)[None, :] < kv_len[:, None]
        a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           attn_mask=seen[:, None, None, :], scale=1.0 / math.sqrt(d),
                                           enable_gqa=True)
        return a.transpose(1, 2).reshape(B, hq * d).contiguous()

    def last_layer_forward(self, L, h, B, S, rows, trace=None, past=None, pos=None):
        """The last layer at the picked rows only (prefill_engine.py:283-339): returns the layer's
        output rows [B, hidden] for the packed rows ``rows`` (int32 [B], device), bit-identical to
        layer_forward's output at those rows."""
        cfg = self.cfg
        t = {} if trace is not None else None
        if isinstance(L, GDNBlock):
            init = None if past is None else tuple(x.expand(B, *x.shape[1:]) for x in past)
            full = L.mixer(h, B, initial=init)
            h1 = full.index_select(0, rows)
            if t is not None:
                t.update(kind="gdn_last", h=h, mixer_out=full)
        else:
            q, s, y = _norm_quant(h, L.input_norm, cfg.eps, t is not None)
            kv = L.kv_rows.forward_quantized(q, s)
            qr = L.q_rows.forward_quantized(q.index_select(0, rows), s.index_select(0, rows))
            if t is not None:
                t.update(kind="attention_last", h=h, q=q, s=s, y=y, kv=kv.clone(), qr=qr.clone())
            a = self._attention_rows(qr, kv, B, S, rows, past, pos, (L.q_norm, L.k_norm))
            nq = cfg.heads * cfg.head_dim
            qa, sa, gated = self._o_input(a, qr[:, nq:] if cfg.attn_output_gate else None, t is not None)
            h1 = L.o.forward_quantized(qa, sa, residual=h.index_select(0, rows))
            if t is not None:
                t.update(kv_rope=kv, qr_rope=qr, a=a, gated=gated, qa=qa, sa=sa)
        q2, s2, y2 = _norm_quant(h1, L.post_norm, cfg.eps, t is not None)
        g = L.gate_up.forward_quantized(q2, s2)
        qh, sh = aot.act_quant(g)
        h2 = L.down.forward_quantized(qh, sh, residual=h1)
        if t is not None:
            t.update(rows=rows, h1=h1, q2=q2, s2=s2, y2=y2, g=g, qh=qh, sh=sh, h2=h2)
            trace.append(t)
        return h2

    @staticmethod
    def _mask(S, P, device):
        """Boolean [S, P + S] mask: query i (position P + i) sees keys 0 .. P + i."""
        return torch.arange(P + S, device=device)[None, :] <= (torch.arange(S, device=device)[:, None] + P)

    def layer_forward(self, L, h, B, S, trace=None, past=None, keep=False, pos=None):
        """One decoder layer over B packed sequences of S tokens.  past: this layer's part of a
        PrefixState the sequences continue; keep: also return this layer's state (batch 1)."""
        cfg = self.cfg
        state = None
        if isinstance(L, GDNBlock):
            t = {} if trace is not None else None
            init = None
            if past is not None:
                init = tuple(x.expand(B, *x.shape[1:]) for x in past)
            h1 = L.mixer(h, B, initial=init, keep=keep, trace=t)
            if keep:
                h1, state = h1
            t = dict(kind="gdn", h=h, mixer=t, h1=h1) if trace is not None else None
        else:
            q, s, y = _norm_quant(h, L.input_norm, cfg.eps, trace is not None)
            qkv = L.qkv.forward_quantized(q, s)
            qkv_out = qkv.clone() if trace is not None else None  # RoPE rotates qkv in place
            # a trace keeps the rotated q too: RoPE as a pass of its own there
            a = self._attention(qkv, B, S, past, keep, pos, (L.q_norm, L.k_norm), fuse_rope=trace is None)
            if keep:
                a, state = a
            nq = cfg.heads * cfg.head_dim
            qa, sa, gated = self._o_input(a, qkv[:, nq:2 * nq] if cfg.attn_output_gate else None, trace is not None)
            h1 = L.o.forward_quantized(qa, sa, residual=h)
            t = dict(kind="attention", h=h, q=q, s=s, y=y, qkv=qkv_out, qkv_rope=qkv, a=a, gated=gated, qa=qa,
                     sa=sa, h1=h1) if trace is not None else None
        q2, s2, y2 = _norm_quant(h1, L.post_norm, cfg.eps, trace is not None)
        g = L.gate_up.forward_quantized(q2, s2)
        qh, sh = aot.act_quant(g)
        h2 = L.down.forward_quantized(qh, sh, residual=h1)
        if trace is not None:
            t.update(q2=q2, s2=s2, y2=y2, g=g, qh=qh, sh=sh, h2=h2)
            trace.append(t)
        return (h2, state) if keep else h2

    @torch.no_grad()
    def prefix_state(self, ids) -> PrefixState:
        """Run a prompt prefix (int [P] token ids, one sequence) through every layer and keep the
        state the rest of a prompt continues from.  With P a multiple of PREFIX_ALIGN a continuation
        gives the same bits as running the whole prompt."""
        P = ids.numel()
        if P < 1:
            raise ValueError("an empty prefix has no state")
        h = self.embed.index_select(0, ids.reshape(-1))
        states = []
        for L in self.layers:
            h, st = self.layer_forward(L, h, 1, P, keep=True)
            states.append(st)
        return PrefixState(P, states)

    @torch.no_grad()
    def prefill(self, ids, batch, kinds=None, n_choices=None, trace=None):
        """ids: int [batch * S] packed token ids of `batch` equal-length requests.  Returns
        (logits [batch, 2 + n_options], probs [batch, width]) for the requests' last positions;
        kinds[b] == 'noul' softmaxes logits[:2], otherwise logits[2 : 2 + n_choices[b]]."""
        S = ids.numel() // batch
        rows = torch.arange(batch, device=ids.device, dtype=torch.int32) * S + (S - 1)
        lo, cnt = self.slices(kinds, n_choices, batch, ids.device)
        return self.forward_last(ids, batch, rows, lo, cnt, trace)

    def slices(self, kinds, n_choices, batch, device):
        """The readout's softmax slices per request: [0, 2) for 'noul', [2, 2 + n) for a choice."""
        if kinds is None:
            kinds = ["choice"] * batch
        if n_choices is None:
            n_choices = [self.cfg.n_options] * batch
        lo = torch.tensor([0 if k == "noul" else 2 for k in kinds], dtype=torch.int32, device=device)
        cnt = torch.tensor([2 if k == "noul" else n for k, n in zip(kinds, n_choices)], dtype=torch.int32, device=device)
        return lo, cnt

    @torch.no_grad()
    def forward_last(self, ids, batch, rows, lo, cnt, trace=None, prefix: PrefixState | None = None):
        """The stack over `batch` packed requests of equal (padded) length S = ids.numel() / batch, then
        the readout at the token rows `rows` (int32 [batch], device) with softmax slices lo / cnt.
        Everything stays on the device and no tensor is built from host values, so a HIP graph can
        capture the call (rows / lo / cnt / ids then act as the graph's static inputs).  With a prefix,
        every request continues it: its tokens are positions prefix.length + 0 .. S - 1."""
        S = ids.numel() // batch
        h = self.embed.index_select(0, ids)
        pos = None if prefix is None else prefix.positions_for(batch, S, ids.device)
        past = (lambda i: None) if prefix is None else (lambda i: prefix.layers[i])  # noqa: E731
        n = len(self.layers)
        full = n - 1 if self.last_only and n else n
        for i in range(full):
            h = self.layer_forward(self.layers[i], h, batch, S, trace, past=past(i), pos=pos)
        if full < n:
            h = self.last_layer_forward(self.layers[-1], h, batch, S, rows, trace, past=past(n - 1), pos=pos)
            rows = torch.arange(batch, device=h.device, dtype=torch.int32)   # h now holds the picked rows
        logits, probs = self.readout(h, rows, self.final_norm, self.cfg.eps, offset=0.0, lo=lo, cnt=cnt,
                                     probs_width=self.cfg.n_options)
        if trace is not None:
            trace.append(dict(h_final=h, rows=rows, logits=logits, probs=probs))
        return logits, probs

    def linear_ops_per_token(self):
        """int8 ops per token of the W8A8 linears (2 N K per projection), final readout excluded."""
        c = self.cfg
        attn = (((2 if c.attn_output_gate else 1) * c.heads + 2 * c.kv_heads) * c.head_dim * c.hidden  # QKV (+ gate)
                + c.hidden * c.heads * c.head_dim)                   # O
        hk, hv, D = c.linear_k_heads, c.linear_v_heads, _GDN_DIM
        gdn = ((2 * hk + hv) * D + hv * D + 2 * hv) * c.hidden + c.hidden * hv * D  # in_proj qkv / z / b / a, out
        mlp = 3 * c.intermediate * c.hidden
        n_gdn = sum(c.is_gdn(i) for i in range(c.layers))
        return 2 * ((c.layers - n_gdn) * attn + n_gdn * gdn + c.layers * mlp)
