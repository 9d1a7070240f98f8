"""Pins the GDN oracle (oracle/gdn.py) before it checks the HIP kernels.

The reference ships no vectors for its GDN layer; its scan lives in flash-linear-attention 0.5.2
(absent here) with the transformers torch functions as fallback.  Each oracle function is pinned by:
  * closed forms: a single token, pure decay (beta = 0), exact memorisation of orthonormal keys;
  * the two independent restatements agreeing (per-token recurrence vs chunked WY form, any chunk);
  * the installed transformers package's torch_recurrent / torch_chunk_gated_delta_rule, l2norm and
    Qwen3_5RMSNormGated, and torch's F.conv1d / F.softplus, as library routines;
  * planted mistakes: plausible wrong variants fail at least one of the above.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as G
from oracle import w8a8 as O


def _inputs(rng, B=2, T=37, HK=2, HV=4, Dk=16, Dv=8, init=True):
    q = G.l2norm(rng.standard_normal((B, T, HK, Dk)))
    k = G.l2norm(rng.standard_normal((B, T, HK, Dk)))
    v = rng.standard_normal((B, T, HV, Dv))
    g = -rng.uniform(0.0, 0.5, (B, T, HV))
    beta = rng.uniform(0.0, 1.0, (B, T, HV))
    S0 = rng.standard_normal((B, HV, Dk, Dv)) * 0.3 if init else None
    return q, k, v, g, beta, S0


def test_single_token_closed_form():
    rng = np.random.default_rng(1)
    q, k, v, g, beta, _ = _inputs(rng, B=1, T=1, HK=1, HV=1, init=False)
    o, S = G.gated_delta_rule(q, k, v, g, beta, scale=0.5)
    want_S = beta[0, 0, 0] * np.outer(k[0, 0, 0], v[0, 0, 0])
    np.testing.assert_allclose(S[0, 0], want_S, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(o[0, 0, 0], 0.5 * beta[0, 0, 0] * (q[0, 0, 0] @ k[0, 0, 0]) * v[0, 0, 0], rtol=1e-12)


def test_pure_decay_closed_form():
    rng = np.random.default_rng(2)
    q, k, v, g, beta, S0 = _inputs(rng)
    beta[:] = 0.0
    o, S = G.gated_delta_rule(q, k, v, g, beta, initial_state=S0)
    cum = np.cumsum(g, axis=1)                                  # [B, T, HV]
    np.testing.assert_allclose(S, np.exp(cum[:, -1])[:, :, None, None] * S0, rtol=1e-12)
    qe = G.expand_heads(q, 4) * q.shape[-1] ** -0.5
    want = np.exp(cum)[..., None] * np.einsum("bthk,bhkv->bthv", qe, S0)
    np.testing.assert_allclose(o, want, rtol=1e-10, atol=1e-13)


def test_exact_memorisation_of_orthonormal_keys():
    """beta = 1, no decay, orthonormal keys: the delta rule stores each value exactly, so after the
    sequence S^T k_j = v_j for every j, and reading with q_t = k_j (j <= t) returns v_j."""
    rng = np.random.default_rng(3)
    Dk, Dv, T = 16, 8, 12
    basis, _ = np.linalg.qr(rng.standard_normal((Dk, Dk)))
    k = basis[:T][None, :, None, :]
    v = rng.standard_normal((1, T, 1, Dv))
    S0 = rng.standard_normal((1, 1, Dk, Dv))
    q = np.roll(k, 1, axis=1)  # q_t = k_{t-1} (q_0 = k_{T-1}: not yet stored at t = 0)
    o, S = G.gated_delta_rule(q, k, v, np.zeros((1, T, 1)), np.ones((1, T, 1)), scale=1.0, initial_state=S0)
    np.testing.assert_allclose(k[0, :, 0] @ S[0, 0], v[0, :, 0], atol=1e-12)
    np.testing.assert_allclose(o[0, 1:, 0], v[0, :-1, 0], atol=1e-12)
    # with chunks shorter than the sequence, the chunked form does the same
    oc, Sc = G.gated_delta_rule_chunked(q, k, v, np.zeros((1, T, 1)), np.ones((1, T, 1)), scale=1.0,
                                        initial_state=S0, chunk=5)
    np.testing.assert_allclose(oc, o, atol=1e-12)
    np.testing.assert_allclose(Sc, S, atol=1e-12)


@pytest.mark.parametrize("chunk", [64, 16, 7])
def test_chunked_form_equals_recurrence(chunk):
    rng = np.random.default_rng(4)
    q, k, v, g, beta, S0 = _inputs(rng, T=150)
    o1, S1 = G.gated_delta_rule(q, k, v, g, beta, initial_state=S0)
    o2, S2 = G.gated_delta_rule_chunked(q, k, v, g, beta, initial_state=S0, chunk=chunk)
    np.testing.assert_allclose(o2, o1, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(S2, S1, rtol=1e-9, atol=1e-11)


def _transformers_gdn():
    try:
        from transformers.models.qwen3_5 import modeling_qwen3_5 as m
    except Exception as e:  # pragma: no cover - the package is part of the image
        pytest.skip(f"transformers qwen3_5 unavailable: {e}")
    return m


def test_against_transformers_torch_functions():
    """The transformers torch fallback (the reference's scan when flash-linear-attention is absent),
    in float32, with its own l2norm: both its recurrent and chunked functions agree with the oracle."""
    m = _transformers_gdn()
    rng = np.random.default_rng(5)
    B, T, HK, HV, Dk, Dv = 2, 100, 2, 4, 32, 16
    q = rng.standard_normal((B, T, HK, Dk))
    k = rng.standard_normal((B, T, HK, Dk))
    v = rng.standard_normal((B, T, HV, Dv))
    g = -rng.uniform(0.0, 0.3, (B, T, HV))
    beta = rng.uniform(0.0, 1.0, (B, T, HV))
    S0 = rng.standard_normal((B, HV, Dk, Dv)) * 0.3
    want_o, want_S = G.gated_delta_rule(G.l2norm(q), G.l2norm(k), v, g, beta, initial_state=S0)
    t = lambda a: torch.tensor(a, dtype=torch.float32)
    rq, rk = (t(G.expand_heads(a, HV)) for a in (q, k))
    for fn in (m.torch_recurrent_gated_delta_rule, m.torch_chunk_gated_delta_rule):
        o, S = fn(rq, rk, t(v), g=t(g), beta=t(beta), initial_state=t(S0), output_final_state=True,
                  use_qk_l2norm_in_kernel=True)
        np.testing.assert_allclose(o.double().numpy(), want_o, rtol=2e-4, atol=2e-5)
        np.testing.assert_allclose(S.double().numpy(), want_S, rtol=2e-4, atol=2e-5)
    np.testing.assert_allclose(m.l2norm(t(q)).double().numpy(), G.l2norm(q), rtol=1e-5, atol=1e-6)


def test_gate_against_torch():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((5, 7)) * 8.0
    b = rng.standard_normal((5, 7)) * 4.0
    A_log = rng.standard_normal(7)
    dt_bias = rng.standard_normal(7)
    g, beta = G.gdn_gate(a, b, A_log, dt_bias)
    ta = torch.tensor(a)
    want_g = -torch.tensor(A_log).exp() * F.softplus(ta + torch.tensor(dt_bias))
    np.testing.assert_allclose(g, want_g.numpy(), rtol=1e-12)
    np.testing.assert_allclose(beta, torch.tensor(b).sigmoid().numpy(), rtol=1e-12)
    assert (g <= 0).all()


def test_causal_conv1d_against_torch_and_brute_force():
    rng = np.random.default_rng(7)
    B, T, C, W = 2, 9, 6, 4
    x = rng.standard_normal((B, T, C))
    w = rng.standard_normal((C, W))
    bias = rng.standard_normal(C)
    init = rng.standard_normal((B, C, W - 1))
    out = G.causal_conv1d(x, w, bias, init, activation=False)
    # brute force
    for b in range(B):
        for t in range(T):
            for c in range(C):
                acc = bias[c]
                for j in range(W):
                    s = t - W + 1 + j
                    acc += w[c, j] * (x[b, s, c] if s >= 0 else init[b, c, W - 1 + s])
                assert abs(out[b, t, c] - acc) < 1e-12
    # torch depthwise conv on [B, C, T] with the initial states prepended (the reference's F.conv1d path)
    full = torch.cat([torch.tensor(init), torch.tensor(x).transpose(1, 2)], -1)
    ref = F.conv1d(full, torch.tensor(w)[:, None, :], torch.tensor(bias), groups=C)
    np.testing.assert_allclose(out, ref.transpose(1, 2).numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(G.causal_conv1d(x, w, bias, init), F.silu(ref).transpose(1, 2).numpy(), rtol=1e-12)
    # no initial state = zero history
    np.testing.assert_allclose(G.causal_conv1d(x, w, None, None, False),
                               G.causal_conv1d(x, w, None, np.zeros_like(init), False), rtol=0, atol=0)


def test_gated_rmsnorm_against_transformers_module():
    m = _transformers_gdn()
    rng = np.random.default_rng(8)
    x = O.f32_to_bf16(rng.standard_normal((64, 128)).astype(np.float32) * 3)
    z = O.f32_to_bf16(rng.standard_normal((64, 128)).astype(np.float32) * 2)
    w = O.f32_to_bf16(rng.normal(1.0, 0.2, 128).astype(np.float32))
    mod = m.Qwen3_5RMSNormGated(128, eps=1e-6).to(torch.bfloat16)
    tb = lambda bits: torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    with torch.no_grad():
        mod.weight.copy_(tb(w))
        ref = mod(tb(x), tb(z)).view(torch.int16).numpy().view(np.uint16)
    got = G.gated_rmsnorm(x, z, w, 1e-6)
    diff = np.abs(O.bf16_to_f32(got).astype(np.float64) - O.bf16_to_f32(ref))
    assert (diff <= O.bf16_ulp(ref)).all()
    assert (got == ref).mean() > 0.99


@pytest.mark.parametrize("mutant", ["decay_sign", "beta_dropped", "qk_swapped", "decay_after_update",
                                    "no_scale"])
def test_planted_mistakes_fail_the_library_check(mutant):
    """Plausible wrong restatements of the recurrence are caught by the comparison with the
    transformers torch function (the check the oracle itself passes above)."""
    m = _transformers_gdn()
    rng = np.random.default_rng(9)
    q, k, v, g, beta, S0 = _inputs(rng, T=20, Dk=16, Dv=8)
    HV = v.shape[2]
    t = lambda a: torch.tensor(a, dtype=torch.float32)
    lib_o, lib_S = m.torch_recurrent_gated_delta_rule(t(G.expand_heads(q, HV)), t(G.expand_heads(k, HV)), t(v),
                                                      g=t(g), beta=t(beta), initial_state=t(S0),
                                                      output_final_state=True)

    def wrong():
        if mutant == "decay_sign":
            return G.gated_delta_rule(q, k, v, -g, beta, initial_state=S0)
        if mutant == "beta_dropped":
            return G.gated_delta_rule(q, k, v, g, np.ones_like(beta), initial_state=S0)
        if mutant == "qk_swapped":
            return G.gated_delta_rule(k, q, v, g, beta, initial_state=S0)
        if mutant == "no_scale":
            return G.gated_delta_rule(q, k, v, g, beta, scale=1.0, initial_state=S0)
        # decay applied after the delta update instead of before it
        B, T, _, Dv = v.shape
        qq, kk = G.expand_heads(q, HV), G.expand_heads(k, HV)
        S = S0.copy()
        o = np.zeros((B, T, HV, Dv))
        for i in range(T):
            mem = np.einsum("bhk,bhkv->bhv", kk[:, i], S)
            S = S + kk[:, i][..., None] * ((v[:, i] - mem) * beta[:, i][..., None])[:, :, None, :]
            S = S * np.exp(g[:, i])[:, :, None, None]
            o[:, i] = np.einsum("bhk,bhkv->bhv", qq[:, i] * q.shape[-1] ** -0.5, S)
        return o, S

    good_o, good_S = G.gated_delta_rule(q, k, v, g, beta, initial_state=S0)
    close = lambda a, b: np.allclose(a, b.double().numpy(), rtol=2e-4, atol=2e-5)
    assert close(good_o, lib_o) and close(good_S, lib_S)
    o, S = wrong()
    assert not (close(o, lib_o) and close(S, lib_S))
