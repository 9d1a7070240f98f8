"""CPU oracle for the gated-delta-net (GDN) token mixer -- TEST INFRASTRUCTURE ONLY.

Restates, in numpy, the arithmetic of the reference's GDN layer step (v0.5/serving/lib/fork.py
``gdn_step`` -> ``_gdn_inputs`` -> ``_gdn_scan``, fork.py:20-149):

  gate            g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b)      (fork.py:124-125)
  causal_conv1d   depthwise causal convolution of width 4 over time + SiLU       (fork.py:94-113)
  l2norm          q, k rows divided by sqrt(sum x^2 + 1e-6)  (use_qk_l2norm_in_kernel=True, fork.py:145)
  gated_delta_rule the recurrence the reference's ``chunk_gated_delta_rule`` computes (fork.py:137-147;
                  flash-linear-attention 0.5.2, absent here, or the transformers torch fallback)
  gated_rmsnorm   attn.norm(out, z): RMSNorm over head_v_dim, times silu(z)        (fork.py:148)

Two forms of the scan are given: ``gated_delta_rule`` is the definitional per-token recurrence
(float64), and ``gated_delta_rule_chunked`` the chunked WY form (the same algebra the reference's
GPU kernels and torch fallback use, long_input_state.py:29-68), also in float64.  tests/test_gdn_oracle.py
pins them against each other, against closed forms (exact memorisation with orthonormal keys,
pure decay) and against the torch implementations shipped with the installed transformers package.

Nothing in ``mica_amd`` may import this module.
"""
from __future__ import annotations

import numpy as np

from .w8a8 import bf16_to_f32, f32_to_bf16


def softplus(x: np.ndarray) -> np.ndarray:
    """torch.nn.functional.softplus with beta=1, threshold=20 (linear above 20)."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def gdn_gate(a: np.ndarray, b: np.ndarray, A_log: np.ndarray, dt_bias: np.ndarray):
    """g = -exp(A_log) * softplus(a + dt_bias) and beta = sigmoid(b) per token and value head
    (fork.py:124-125).  a, b: [..., HV]; A_log, dt_bias: [HV].  Returned in float64."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    g = -np.exp(np.asarray(A_log, np.float64)) * softplus(a + np.asarray(dt_bias, np.float64))
    beta = 1.0 / (1.0 + np.exp(-b))
    return g, beta


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def causal_conv1d(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None, init: np.ndarray | None = None,
                  activation: bool = True) -> np.ndarray:
    """Depthwise causal convolution over time, as ``causal_conv1d_fn`` / the F.conv1d fallback in
    ``_gdn_inputs`` (fork.py:94-113): out[b, t, c] = sum_j w[c, j] * x[b, t - W + 1 + j, c] (+ bias[c]),
    with x at negative times taken from ``init`` [B, C, W - 1] (zeros when None), then SiLU.
    x: [B, T, C] (channel-last, as the reference's channel-last path hands it over); w: [C, W]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, T, C = x.shape
    W = w.shape[1]
    pre = np.zeros((B, W - 1, C)) if init is None else np.transpose(np.asarray(init, np.float64), (0, 2, 1))
    full = np.concatenate([pre, x], axis=1)  # [B, W - 1 + T, C]
    out = np.zeros((B, T, C))
    for j in range(W):
        out += w[:, j][None, None, :] * full[:, j:j + T, :]
    if bias is not None:
        out += np.asarray(bias, np.float64)[None, None, :]
    return silu(out) if activation else out


def l2norm(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """x / sqrt(sum(x^2) + eps) over the last axis (the l2norm of use_qk_l2norm_in_kernel)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def expand_heads(x: np.ndarray, hv: int) -> np.ndarray:
    """q / k of HK heads repeated for HV value heads: head h reads key head h // (HV // HK)
    (``repeat_interleave`` on the head axis, fork.py:134-136).  x: [B, T, HK, D]."""
    hk = x.shape[2]
    assert hv % hk == 0
    return np.repeat(x, hv // hk, axis=2)


def gated_delta_rule(q, k, v, g, beta, scale: float | None = None, initial_state=None):
    """The gated delta rule, token by token (float64).  Per batch b and value head h, with state
    S [Dk, Dv] (zeros or ``initial_state[b, h]``):

        S <- exp(g_t) S;  S <- S + k_t (beta_t (v_t - S^T k_t))^T;  o_t = S^T (scale q_t)

    q, k: [B, T, H(K), Dk] (key heads are repeated to the value heads), v: [B, T, HV, Dv],
    g, beta: [B, T, HV].  scale defaults to Dk ** -0.5.  Returns (o [B, T, HV, Dv], S [B, HV, Dk, Dv])."""
    v = np.asarray(v, np.float64)
    B, T, HV, Dv = v.shape
    q = expand_heads(np.asarray(q, np.float64), HV)
    k = expand_heads(np.asarray(k, np.float64), HV)
    Dk = q.shape[-1]
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    scale = Dk ** -0.5 if scale is None else scale
    S = np.zeros((B, HV, Dk, Dv)) if initial_state is None else np.array(initial_state, np.float64)
    o = np.zeros((B, T, HV, Dv))
    for t in range(T):
        S *= np.exp(g[:, t])[:, :, None, None]
        kt = k[:, t]                                    # [B, HV, Dk]
        mem = np.einsum("bhk,bhkv->bhv", kt, S)
        delta = (v[:, t] - mem) * beta[:, t][:, :, None]
        S += kt[:, :, :, None] * delta[:, :, None, :]
        o[:, t] = np.einsum("bhk,bhkv->bhv", q[:, t] * scale, S)
    return o, S


def gated_delta_rule_chunked(q, k, v, g, beta, scale: float | None = None, initial_state=None, chunk: int = 64):
    """The same recurrence in the chunked WY form (float64), per chunk of C tokens with in-chunk
    cumulative log decays G (long_input_state.py:29-68 restates it for the state only):

        L[i, j] = beta_i (k_i . k_j) exp(G_i - G_j) for j < i;  T = (I + L)^-1
        W = T (beta * exp(G) * K);  U = T (beta * V)
        v_new = U - W S;  o = scale (exp(G) * (Q S) + ((Q K^T) o exp(G_i - G_j), j <= i) v_new)
        S <- exp(G_last) S + (exp(G_last - G) * K)^T v_new
    """
    v = np.asarray(v, np.float64)
    B, T, HV, Dv = v.shape
    q = expand_heads(np.asarray(q, np.float64), HV)
    k = expand_heads(np.asarray(k, np.float64), HV)
    Dk = q.shape[-1]
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    scale = Dk ** -0.5 if scale is None else scale
    S = np.zeros((B, HV, Dk, Dv)) if initial_state is None else np.array(initial_state, np.float64)
    o = np.zeros((B, T, HV, Dv))
    for b in range(B):
        for h in range(HV):
            St = S[b, h]
            for c0 in range(0, T, chunk):
                c1 = min(T, c0 + chunk)
                n = c1 - c0
                K = k[b, c0:c1, h]
                Q = q[b, c0:c1, h]
                V = v[b, c0:c1, h]
                bt = beta[b, c0:c1, h]
                G = np.cumsum(g[b, c0:c1, h])
                D = np.exp(G[:, None] - G[None, :])
                L = np.tril(bt[:, None] * (K @ K.T) * D, -1)
                Tm = np.linalg.inv(np.eye(n) + L)
                W = Tm @ (bt[:, None] * np.exp(G)[:, None] * K)
                U = Tm @ (bt[:, None] * V)
                v_new = U - W @ St
                P = np.tril((Q @ K.T) * D)
                o[b, c0:c1, h] = scale * (np.exp(G)[:, None] * (Q @ St) + P @ v_new)
                St = np.exp(G[-1]) * St + (np.exp(G[-1] - G)[:, None] * K).T @ v_new
            S[b, h] = St
    return o, S


def gated_rmsnorm(x_bits: np.ndarray, z_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """attn.norm(out, z) of the reference's GDN (fork.py:148; Qwen3_5RMSNormGated): over the last
    axis, h = bf16(x * rsqrt(mean(x^2) + eps)); h = bf16(w * h); y = bf16(h * silu(f32(z))).
    bf16 tensors are uint16 bit patterns; returns bf16 bits."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    ms = (x * x).mean(-1, keepdims=True)
    h = bf16_to_f32(f32_to_bf16((x / np.sqrt(ms + eps)).astype(np.float32)))
    h = bf16_to_f32(f32_to_bf16((bf16_to_f32(w_bits) * h).astype(np.float32)))
    z = bf16_to_f32(z_bits).astype(np.float64)
    return f32_to_bf16((h * silu(z)).astype(np.float32))
