"""numpy restatement of the reference's W8A8 arithmetic (test infrastructure; see oracle/__init__.py).

Conventions: bf16 tensors are numpy ``uint16`` arrays of bit patterns; every fp32 step is an explicit
``np.float32`` operation, so IEEE single rounding happens exactly where the reference's torch code
rounds.  Reference citations are into akivet/Mica ``v0.5/serving/``.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
QMAX = F32(127.0)   # int8_quant.py:11
EPS = F32(1e-8)     # int8_quant.py:13 (a python float clamped against an fp32 tensor -> fp32)


# ---------------------------------------------------------------- bf16 helpers
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (torch's ``.to(torch.bfloat16)``); NaN -> 0x7fc0."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), rounded)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 and return them as fp32."""
    return bf16_to_f32(f32_to_bf16(x))


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def bf16_ulp(bits: np.ndarray) -> np.ndarray:
    """Size of one bf16 unit in the last place at each value (fp32)."""
    v = np.abs(bf16_to_f32(bits)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return (2.0 ** (e - 7)).astype(np.float32)


# ---------------------------------------------------------------- quantizers
def quant_act(x: np.ndarray, inv_smooth: np.ndarray | None = None, rounding: str = "even"):
    """Per-token symmetric INT8 quantizer.

    rounding='even': int8_quant.quant_act (int8_quant.py:64-73): ``xf = x.float()``, optional
    ``xf * inv_smooth``, ``s = amax.clamp_min(1e-8) / 127``, ``q = round_half_even(xf / s)`` clamped
    to +-127.  rounding='away': the Triton act_quant (kernel_src/kernels.py:26-36):
    ``v = x / scale; r = int(v + 0.5 if v >= 0 else v - 0.5)`` (fp32 add, truncation).

    x: fp32 values (already widened from bf16/fp16), shape [M, K].  Returns (q int8 [M, K], s fp32 [M]).
    """
    xf = np.asarray(x, dtype=np.float32)
    if inv_smooth is not None:
        xf = xf * np.asarray(inv_smooth, dtype=np.float32)
    amax = np.abs(xf).max(axis=-1) if xf.shape[-1] else np.zeros(xf.shape[:-1], np.float32)
    s = np.maximum(amax, EPS) / QMAX
    v = xf / s[..., None]
    if rounding == "even":
        r = np.rint(v)
    elif rounding == "away":
        r = np.trunc(np.where(v >= 0, v + F32(0.5), v - F32(0.5)))
    else:
        raise ValueError(rounding)
    q = np.clip(r, -127, 127).astype(np.int8)
    return q, s.astype(np.float32)


def quant_weight(w: np.ndarray):
    """Per-output-channel weight quantizer, int8_quant.quant_weight (int8_quant.py:54-61)."""
    wf = np.asarray(w, dtype=np.float32)
    s = np.maximum(np.abs(wf).max(axis=1), EPS) / QMAX
    q = np.clip(np.rint(wf / s[:, None]), -127, 127).astype(np.int8)
    return q, s.astype(np.float32)


def smooth_factors(act_amax: np.ndarray, w: np.ndarray, alpha: float = 0.5, lo: float = 1e-4, hi: float = 1e4):
    """SmoothQuant factors per input channel, int8_quant.smooth_factors (int8_quant.py:80-85):
    s = max(a, 1e-8)^alpha / max(wmax, 1e-8)^(1 - alpha) with wmax the column absmax of w [N, K];
    1 where a or wmax is 0; clamped to [lo, hi].  fp32 throughout (pow as fp32 powf)."""
    a = np.asarray(act_amax, np.float32)
    wmax = np.abs(np.asarray(w, np.float32)).max(axis=0)
    num = np.power(np.maximum(a, EPS), np.float32(alpha), dtype=np.float32)
    den = np.power(np.maximum(wmax, EPS), np.float32(1.0 - alpha), dtype=np.float32)
    s = np.where((a > 0) & (wmax > 0), (num / den).astype(np.float32), np.float32(1.0))
    return np.clip(s, np.float32(lo), np.float32(hi)).astype(np.float32)


# ---------------------------------------------------------------- GEMM
def int_gemm(qa: np.ndarray, qw: np.ndarray) -> np.ndarray:
    """acc[m, n] = sum_k qa[m, k] * qw[n, k], exact int32 (int8_quant.int_gemm_exact, int8_quant.py:88-89).

    Evaluated in float64 like the reference: every partial sum is an integer of magnitude
    <= K * 127^2 < 2^53 for K < 5.5e8, so the float64 result is exact.
    """
    qa = np.asarray(qa, dtype=np.int8)
    qw = np.asarray(qw, dtype=np.int8)
    assert qa.shape[1] * 127 * 127 < 2 ** 53
    return (qa.astype(np.float64) @ qw.astype(np.float64).T).astype(np.int32)


def epilogue(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias: np.ndarray | None = None,
             out: str = "bf16"):
    """y = (f32(acc) * sa[m]) * sb[n] (+ bias[n]), then converted to the output dtype.

    int8_runtime.py:186 ``torch_int_mm(qx, w).float() * sx[:, None] * wscale[None, :]``, :190-192
    ``y + bias`` then ``.to(out_dtype)``; Triton kernels.py:65-68 in the same order.
    Returns bf16 bits (out='bf16'), float16 (out='fp16') or float32 (out='fp32').
    """
    y = np.asarray(acc, dtype=np.int32).astype(np.float32) * np.asarray(sa, np.float32)[:, None]
    y = y * np.asarray(sb, np.float32)[None, :]
    if bias is not None:
        y = y + np.asarray(bias, np.float32)[None, :]
    if out == "bf16":
        return f32_to_bf16(y)
    if out == "fp16":
        return f32_to_f16(y)
    return y.astype(np.float32)


def qlinear(x_bits: np.ndarray, qw: np.ndarray, sw: np.ndarray, bias=None, inv_smooth=None,
            rounding: str = "even"):
    """QLinear.forward on bf16 x (int8_runtime.py:172-192): quantize, exact GEMM, epilogue -> bf16 bits."""
    q, s = quant_act(bf16_to_f32(x_bits), inv_smooth, rounding)
    return epilogue(int_gemm(q, qw), s, sw, bias)


# ---------------------------------------------------------------- RMSNorm
def rms_norm(x_bits: np.ndarray, w: np.ndarray, eps: float, offset: float = 1.0,
             residual_bits: np.ndarray | None = None):
    """RMSNorm of fused_kernels.rms_norm, CPU branch (fused_kernels.py:51-56):

    value = x (+ residual, rounded to bf16); xf = value.float()
    y = bf16((xf * rsqrt(mean(xf^2) + eps)) * (offset + w))

    offset=1 is the Qwen3.5 ``(1 + weight)``; offset=0 a plain gamma.  w: fp32 values of the weight.
    mean(xf^2) is evaluated as RN32(exact sum) / K: torch's fp32 summation order is not a fixed
    reference, so the exact sum rounded once is used (the kernel's fp32 tree may differ by ulps;
    tests bound that at one bf16 ulp of y).  rsqrt = 1 / sqrt, two correctly rounded fp32 ops
    (torch CPU's Vectorized<float>::rsqrt).
    Returns (y_bits, value_bits).
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    if residual_bits is not None:
        value = f32_to_bf16(bf16_to_f32(x_bits) + bf16_to_f32(residual_bits))
    else:
        value = x_bits
    xf = bf16_to_f32(value)
    K = xf.shape[-1]
    ss = F32((xf.astype(np.float64) ** 2).sum(axis=-1))  # squares of bf16 values are exact in fp64
    ss = np.asarray(ss, dtype=np.float32)
    mean = ss / F32(K)
    rstd = F32(1.0) / np.sqrt(mean + F32(eps))
    w1 = F32(offset) + np.asarray(w, dtype=np.float32)
    y = (xf * rstd[..., None]) * w1
    return f32_to_bf16(y), value


def rms_norm_quant(x_bits, w, eps, offset=1.0, residual_bits=None, inv_smooth=None, rounding="even"):
    """rms_norm followed by quant_act on its bf16 output (the QLinear input path, int8_runtime.py:181)."""
    y, value = rms_norm(x_bits, w, eps, offset, residual_bits)
    q, s = quant_act(bf16_to_f32(y), inv_smooth, rounding)
    return q, s, y, value


# ---------------------------------------------------------------- SwiGLU / MLP
def silu_mul(g_bits: np.ndarray, u_bits: np.ndarray) -> np.ndarray:
    """h = bf16(bf16(silu(g)) * u) on bf16 inputs.

    CPU path ``F.silu(gate) * up`` (fused_kernels.py:86-87): F.silu on a bf16 tensor computes
    g / (1 + exp(-g)) in fp32 and rounds to bf16, the product of two bf16 tensors is an fp32 product
    rounded to bf16.  Same formula as the Triton swiglu (fused_kernels.py:36-42).  exp(-g) is
    evaluated in float64 and rounded once to fp32 (so it overflows to inf for -g > 88.72, as the fp32
    exp does); 1 + e and the quotient are fp32 operations.
    """
    g = bf16_to_f32(g_bits)
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    act = round_bf16(g / (F32(1.0) + e))
    return f32_to_bf16(act * bf16_to_f32(u_bits))


def pack_gate_up(qg, sg, qu, su, group: int = 64):
    """Interleave gate and up weight rows in groups: [g0..g63, u0..u63, g64..g127, u64..u127, ...].

    Layout contract of the fused gate+up GEMM's SILU_MUL epilogue (the reference keeps separate
    gate/up QLinears, fast_runtime.py:126-132; the fused GEMM is mica_amd's).
    """
    n, k = qg.shape
    assert n % group == 0 and qu.shape == qg.shape
    q = np.stack([qg.reshape(n // group, group, k), qu.reshape(n // group, group, k)], axis=1)
    s = np.stack([sg.reshape(n // group, group), su.reshape(n // group, group)], axis=1)
    return q.reshape(2 * n, k), s.reshape(2 * n)


def gated_mlp(x_bits, qg, sg, qu, su, qd, sd, residual_bits=None, rounding="even"):
    """MLP of fast_runtime._fused_mlp (fast_runtime.py:126-132) on W8A8 linears, plus the block's
    residual add (fork.py:419-422): gate = QLinear(x), up = QLinear(x), h = swi_glu(gate, up),
    out = bf16(residual + QLinear_down(h)).  Returns (out_bits, h_bits)."""
    q, s = quant_act(bf16_to_f32(x_bits), None, rounding)
    g = epilogue(int_gemm(q, qg), s, sg)
    u = epilogue(int_gemm(q, qu), s, su)
    h = silu_mul(g, u)
    qh, sh = quant_act(bf16_to_f32(h), None, rounding)
    d = epilogue(int_gemm(qh, qd), sh, sd)
    if residual_bits is not None:
        d = f32_to_bf16(bf16_to_f32(d) + bf16_to_f32(residual_bits))
    return d, h


# ---------------------------------------------------------------- readout
def readout(h_bits, rows, norm_w, eps, W, offset=1.0, ids=None):
    """Label readout (release_runtime.py:298-306) on body.norm of the last hidden rows
    (prefill_engine.py:280-281, pick :296-304): logits = f32(bf16 normed x) @ W_rows^T.

    h_bits: bf16 bits [T, K]; rows: indices of each request's last token; W: fp32 [L, K] label rows
    (or the full table indexed by ids).  The fp32 dot is evaluated in float64 and rounded once.
    """
    x = np.asarray(h_bits, dtype=np.uint16)[np.asarray(rows)]
    if norm_w is not None:
        x, _ = rms_norm(x, norm_w, eps, offset)
    xf = bf16_to_f32(x).astype(np.float64)
    Wr = np.asarray(W, dtype=np.float32)
    if ids is not None:
        Wr = Wr[np.asarray(ids)]
    return (xf @ Wr.astype(np.float64).T).astype(np.float32)


def softmax(z: np.ndarray) -> np.ndarray:
    """softmax over the last axis (release_runtime.py:517), evaluated in float64."""
    z = np.asarray(z, dtype=np.float64)
    e = np.exp(z - z.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def option_probs(logits: np.ndarray, kind: str, n: int | None = None) -> np.ndarray:
    """Slice + softmax of judge_many.put/finish (release_runtime.py:509-517): [:2] for a noul
    question, [2:2+n] otherwise."""
    z = logits[..., :2] if kind == "noul" else logits[..., 2:2 + n]
    return softmax(z)


def rope(x_bits: np.ndarray, cos_bits: np.ndarray, sin_bits: np.ndarray) -> np.ndarray:
    """Rotate-half rotary embedding in bf16 arithmetic, as transformers' apply_rotary_pos_emb computes
    it for bf16 q / k (q * cos + rotate_half(q) * sin; each product and the sum rounded to bf16).
    x: bf16 bits [..., d]; cos / sin: bf16 bits broadcastable to [..., d / 2].  Returns bf16 bits."""
    x = bf16_to_f32(x_bits)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    c, s = bf16_to_f32(cos_bits), bf16_to_f32(sin_bits)
    y1 = round_bf16(x1 * c) + round_bf16(x2 * -s)
    y2 = round_bf16(x2 * c) + round_bf16(x1 * s)
    return f32_to_bf16(np.concatenate([y1, y2], -1).astype(np.float32))


def causal_gqa_attention(q, k, v, scale: float) -> np.ndarray:
    """float64 softmax(scale q k^T, causal) v per sequence and query head; q [B, Sq, HQ, D], k / v
    [B, Sk, HK, D] with Sk >= Sq, query head h reads key/value head h // (HQ // HK) (the attention of
    the full-attention layers; torch SDPA with enable_gqa computes the same).  The queries are the
    last Sq positions: query t sees keys u <= t + Sk - Sq (kernel_src/kernels.py:92-98, the n_q < n_k
    shift of the reference's kernel)."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    B, S, HQ, D = q.shape
    Sk = k.shape[1]
    assert Sk >= S
    grp = HQ // k.shape[2]
    out = np.zeros((B, S, HQ, D))
    mask = np.arange(Sk)[None, :] > (np.arange(S)[:, None] + (Sk - S))
    for b in range(B):
        for h in range(HQ):
            s = scale * q[b, :, h] @ k[b, :, h // grp].T
            s[mask] = -np.inf
            s -= s.max(1, keepdims=True)
            p = np.exp(s)
            out[b, :, h] = (p / p.sum(1, keepdims=True)) @ v[b, :, h // grp]
    return out


# ---------------------------------------------------------------- full-attention extras
def sigmoid_bf16(g_bits: np.ndarray) -> np.ndarray:
    """bf16(sigmoid(g)) on bf16 g, torch.sigmoid's fp32 steps for a bf16 tensor: 1 / (1 + exp(-g)) with
    exp(-g) in float64 rounded once to fp32 (inf past the fp32 range, as the fp32 exp), then the fp32 sum
    and IEEE quotient, rounded to bf16 (the gate of the full-attention layers, fast_runtime.py:240)."""
    g = bf16_to_f32(g_bits)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    return f32_to_bf16(F32(1.0) / (F32(1.0) + e))


def gate_mul(a_bits: np.ndarray, g_bits: np.ndarray) -> np.ndarray:
    """The output gate o * sigmoid(gate) on bf16 tensors (fast_runtime.py:240,
    prefill_engine.py:331): the fp32 product of o and bf16(sigmoid(g)), rounded to bf16."""
    return f32_to_bf16(bf16_to_f32(a_bits) * bf16_to_f32(sigmoid_bf16(g_bits)))


def head_rms_norm(x_bits: np.ndarray, w, eps: float, offset: float = 1.0) -> np.ndarray:
    """q_norm / k_norm of the full-attention layers (fast_runtime.py:232-233): the RMSNorm of rms_norm over
    the last axis (each head of head_dim values), with the zero-centred weight (offset 1)."""
    return rms_norm(x_bits, w, eps, offset)[0]


def rope_partial(x_bits: np.ndarray, cos_bits: np.ndarray, sin_bits: np.ndarray, rot_dim: int) -> np.ndarray:
    """Partial rotary embedding (rope_one, prefill_engine.py:83-89): rope on the first rot_dim dims of each
    head, the other dims unchanged.  cos / sin: bf16 bits broadcastable to [..., rot_dim / 2]."""
    x = np.asarray(x_bits, dtype=np.uint16)
    rot = rope(x[..., :rot_dim], cos_bits, sin_bits)
    return np.concatenate([rot, x[..., rot_dim:]], -1)
