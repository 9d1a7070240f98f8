"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

The reference ships no golden vectors for this path, so each oracle function is pinned by:
  * known answers derived independently from the mathematics (tests/golden/kat_w8a8.json, made by
    tests/golden/make_golden.py in pure Python with explicit fp32 rounding -- no numpy, no oracle);
  * the reference's own CPU code path restated with the same torch calls (oracle/cpu_path.py) on
    seeded inputs of the benchmark distributions -- bit-exact where the reference is deterministic;
  * brute force on tiny inputs, closed forms and invariants;
  * planted mistakes: plausible wrong variants of the oracle must fail at least one of the above.
"""
import numpy as np
import pytest
import torch

from oracle import cpu_path
from oracle import w8a8 as O

RNG_SEED = 1234


def _bf16_from_torch(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _torch_from_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _act(rng, shape, outliers=8):
    """X ~ N(0, 1) bf16 with `outliers` channels x20 (the benchmark activation distribution)."""
    x = rng.standard_normal(shape).astype(np.float32)
    if outliers:
        cols = rng.permutation(shape[-1])[:outliers]
        x[..., cols] *= 20.0
    return O.f32_to_bf16(x)


# ------------------------------------------------------------------------------- known answers
def test_kat_quant(kat):
    for case in kat["quant"]:
        x = O.bf16_to_f32(np.array(case["x_bf16"], np.uint16))[None, :]
        inv = np.array(case["inv"], np.float32) if "inv" in case else None
        for mode, key in (("even", "q_even"), ("away", "q_away")):
            q, s = O.quant_act(x, inv, mode)
            assert q[0].tolist() == case[key], (mode, case)
            assert s.view(np.uint32)[0] == case["s_bits"]


def test_kat_quant_weight(kat):
    """quant_weight (int8_quant.py:54-61) against pure-Python known answers: ties at s = 1 and 1/2, an
    all-zero row, rows under the 1e-8 floor, single-element rows, a constant row; and row for row the
    same bits as the activation quantizer applied to the weight's rows (the same formula per row)."""
    for case in kat["quant_weight"]:
        w = np.array(case["w_f32_bits"], np.uint32).view(np.float32)
        q, s = O.quant_weight(w)
        assert q.tolist() == case["q"], case
        assert s.view(np.uint32).tolist() == case["s_bits"], case
        qa, sa = O.quant_act(w)
        assert np.array_equal(q, qa) and np.array_equal(s.view(np.uint32), sa.view(np.uint32))


def test_kat_gemm(kat):
    for case in kat["gemm"]:
        A = np.array(case["A"], np.int8)
        B = np.array(case["B"], np.int8)
        acc = O.int_gemm(A, B)
        assert acc.tolist() == case["acc"]
        bias = None if case["bias"] is None else np.array(case["bias"], np.float32)
        y = O.epilogue(acc, np.array(case["sa"], np.float32), np.array(case["sb"], np.float32), bias)
        assert y.tolist() == case["y_bf16"]


def test_kat_rms_norm(kat):
    for case in kat["rms_norm"]:
        y, _ = O.rms_norm(np.array(case["x_bf16"], np.uint16)[None, :], np.array(case["w"], np.float32),
                          case["eps"], case["offset"])
        assert y[0].tolist() == case["y_bf16"]


def test_kat_silu_and_softmax(kat):
    c = kat["silu_mul"]
    h = O.silu_mul(np.array(c["g_bf16"], np.uint16), np.array(c["u_bf16"], np.uint16))
    assert h.tolist() == c["h_bf16"]
    for case in kat["softmax"]:
        np.testing.assert_allclose(O.softmax(np.array(case["z"])), case["p"], rtol=0, atol=1e-7)


# ----------------------------------------------- cross-check against the reference's CPU code path
@pytest.mark.parametrize("rows,k,smooth", [(64, 2560, False), (64, 2560, True), (33, 9728, False), (5, 4096, True)])
def test_quant_act_matches_reference_cpu_path(rows, k, smooth):
    rng = np.random.default_rng(RNG_SEED + k)
    xb = _act(rng, (rows, k))
    inv = (rng.uniform(0.2, 5.0, k).astype(np.float32)) if smooth else None
    q, s = O.quant_act(O.bf16_to_f32(xb), inv)
    qt, st = cpu_path.quant_act(_torch_from_bf16(xb), None if inv is None else torch.from_numpy(inv))
    assert np.array_equal(q, qt.numpy())
    assert np.array_equal(s.view(np.uint32), st.numpy().view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(48, 96, 2560), (7, 64, 4096), (17, 32, 9728)])
def test_qlinear_matches_reference_cpu_path(m, n, k):
    rng = np.random.default_rng(RNG_SEED + m)
    xb = _act(rng, (m, k))
    qw = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sw = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    for b in (None, bias):
        y = O.qlinear(xb, qw, sw, b)
        yt = cpu_path.qlinear(_torch_from_bf16(xb), torch.from_numpy(qw), torch.from_numpy(sw),
                              None if b is None else torch.from_numpy(b))
        assert np.array_equal(y, _bf16_from_torch(yt))
    # the int32 accumulators against torch._int_mm
    q, _ = O.quant_act(O.bf16_to_f32(xb))
    acc = cpu_path.torch_int_mm(torch.from_numpy(q), torch.from_numpy(qw)).numpy()
    assert np.array_equal(O.int_gemm(q, qw), acc)


@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_rms_norm_matches_reference_cpu_path(offset):
    rng = np.random.default_rng(RNG_SEED)
    xb = _act(rng, (256, 2560))
    rb = _act(rng, (256, 2560), outliers=0)
    w = O.round_bf16(rng.normal(1.0 - offset, 0.1, 2560).astype(np.float32))
    for res in (None, rb):
        y, v = O.rms_norm(xb, w, 1e-6, offset, res)
        wt = _torch_from_bf16(O.f32_to_bf16(w))
        out = cpu_path.rms_norm(_torch_from_bf16(xb), wt, 1e-6, None if res is None else _torch_from_bf16(res),
                                offset=offset)
        yt = out if res is None else out[0]
        if res is not None:
            assert np.array_equal(v, _bf16_from_torch(out[1]))
        yt = _bf16_from_torch(yt)
        diff = np.abs(O.bf16_to_f32(y) - O.bf16_to_f32(yt))
        # torch's fp32 summation order differs from the exactly rounded sum: at most one bf16 ulp
        assert np.all(diff <= O.bf16_ulp(y) * 1.0001)
        assert np.mean(y == yt) > 0.999


def test_swiglu_matches_reference_cpu_path():
    rng = np.random.default_rng(RNG_SEED)
    g = O.f32_to_bf16(rng.standard_normal(200_000).astype(np.float32) * 4)
    u = O.f32_to_bf16(rng.standard_normal(200_000).astype(np.float32))
    h = O.silu_mul(g, u)
    ht = _bf16_from_torch(cpu_path.swi_glu(_torch_from_bf16(g), _torch_from_bf16(u)))
    diff = np.abs(O.bf16_to_f32(h) - O.bf16_to_f32(ht))
    assert np.all(diff <= O.bf16_ulp(h) * 1.0001)
    assert np.mean(h == ht) > 0.999


def test_mlp_block_matches_reference_cpu_path():
    rng = np.random.default_rng(RNG_SEED)
    T, H, I = 16, 256, 512
    xb = _act(rng, (T, H))
    res = _act(rng, (T, H), outliers=0)
    mk = lambda n, k: (rng.integers(-127, 128, (n, k), dtype=np.int8), rng.uniform(1e-3, 1e-2, n).astype(np.float32))  # noqa: E731
    (qg, sg), (qu, su), (qd, sd) = mk(I, H), mk(I, H), mk(H, I)
    out, _ = O.gated_mlp(xb, qg, sg, qu, su, qd, sd, res)
    tt = lambda a: torch.from_numpy(a)  # noqa: E731
    ot = cpu_path.mlp(_torch_from_bf16(xb), (tt(qg), tt(sg)), (tt(qu), tt(su)), (tt(qd), tt(sd)),
                      _torch_from_bf16(res))
    ot = _bf16_from_torch(ot)
    # h can differ by one bf16 ulp (library exp), which moves the requantized row slightly
    rel = np.abs(O.bf16_to_f32(out) - O.bf16_to_f32(ot)) / (np.abs(O.bf16_to_f32(ot)) + 1e-2)
    assert np.mean(out == ot) > 0.95 and rel.max() < 2e-2


def test_readout_matches_reference_cpu_path():
    rng = np.random.default_rng(RNG_SEED)
    T, K, L = 64, 2560, 257
    h = _act(rng, (T, K))
    rows = np.array([7, 20, 63])
    w = O.round_bf16(rng.normal(0, 0.1, K).astype(np.float32))
    W = rng.normal(0, 0.02, (L, K)).astype(np.float32)
    z = O.readout(h, rows, w, 1e-6, W)
    zt = cpu_path.readout(_torch_from_bf16(h[rows]), _torch_from_bf16(O.f32_to_bf16(w)), 1e-6,
                          torch.from_numpy(W)).numpy()
    np.testing.assert_allclose(z, zt, rtol=1e-4, atol=1e-4)
    p = O.option_probs(z, "choice", 255)
    pt = torch.softmax(torch.from_numpy(zt)[:, 2:257], -1).numpy()
    np.testing.assert_allclose(p, pt, atol=1e-6)


# ----------------------------------------------------------------------- brute force / closed forms
def test_int_gemm_brute_force():
    rng = np.random.default_rng(5)
    A = rng.integers(-127, 128, (3, 48), dtype=np.int8)
    B = rng.integers(-127, 128, (4, 48), dtype=np.int8)
    ref = [[sum(int(A[m, k]) * int(B[n, k]) for k in range(48)) for n in range(4)] for m in range(3)]
    assert O.int_gemm(A, B).tolist() == ref


def test_quant_act_brute_force_exact_rationals():
    """q = clamp(round_half_even(x / s)) with x / s rounded to fp32 -- evaluated with exact rationals."""
    from fractions import Fraction

    rng = np.random.default_rng(9)
    x = O.round_bf16(rng.standard_normal((4, 64)).astype(np.float32) * 3)
    q, s = O.quant_act(x)
    for r in range(4):
        amax = max(abs(float(v)) for v in x[r])
        s_ref = np.float32(Fraction(amax) / 127)  # correctly rounded scale
        assert np.float32(s[r]) == s_ref
        for k in range(64):
            t = float(np.float32(Fraction(float(x[r, k])) / Fraction(float(s_ref))))
            assert q[r, k] == int(np.clip(round(t), -127, 127))  # python round() is half-even


def test_quant_invariants():
    rng = np.random.default_rng(3)
    x = O.bf16_to_f32(_act(rng, (128, 512)))
    q, s = O.quant_act(x)
    assert q.min() >= -127 and q.max() <= 127
    assert np.all(np.abs(q).max(axis=1) == 127)          # the absmax element maps to +-127
    err = np.abs(q.astype(np.float32) * s[:, None] - x)
    assert np.all(err <= s[:, None] * (0.5 + 1e-5))       # round-trip error <= half a step (+ fp32 rounding of x / s)
    q2, s2 = O.quant_act(x * np.float32(4.0))           # power-of-two scaling commutes
    assert np.array_equal(q, q2) and np.array_equal(s2, s * np.float32(4.0))
    z, sz = O.quant_act(np.zeros((2, 16), np.float32))
    assert not z.any() and np.all(sz == np.float32(1e-8) / np.float32(127))


def test_rms_norm_closed_forms():
    # unit-RMS row and eps = 0: y == bf16(x * w1)
    x = np.array([[1.0, -1.0] * 32], np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y, _ = O.rms_norm(O.f32_to_bf16(x), w, 0.0, offset=0.0)
    assert np.array_equal(y, O.f32_to_bf16(x * w))
    # scaling x by 2^k leaves y unchanged when eps = 0
    rng = np.random.default_rng(2)
    xb = _act(rng, (4, 256))
    y1, _ = O.rms_norm(xb, w[:1].repeat(256), 0.0, 1.0)
    y2, _ = O.rms_norm(O.f32_to_bf16(O.bf16_to_f32(xb) * 8), w[:1].repeat(256), 0.0, 1.0)
    assert np.array_equal(y1, y2)


# ------------------------------------------------------------------------------ planted mistakes
def _wrong_epilogue_order(acc, sa, sb, bias=None):
    y = acc.astype(np.float32) * (sa[:, None] * sb[None, :])
    return O.f32_to_bf16(y if bias is None else y + bias[None, :])


_QUANT_ACT, _RMS_NORM, _QUANT_WEIGHT = O.quant_act, O.rms_norm, O.quant_weight  # originals, for planting


def _wrong_weight_round_away(w):
    return _QUANT_ACT(np.asarray(w, np.float32), None, "away")


def _wrong_weight_no_eps_floor(w):
    return _wrong_no_eps_floor(w)


def _wrong_weight_per_column(w):
    q, s = _QUANT_WEIGHT(np.asarray(w, np.float32).T)
    return q.T, s


def _wrong_round_away(x, inv=None, rounding="even"):
    return _QUANT_ACT(x, inv, "away")


def _wrong_no_eps_floor(x, inv=None, rounding="even"):
    xf = np.asarray(x, np.float32)
    s = np.abs(xf).max(-1) / np.float32(127)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.clip(np.nan_to_num(np.rint(xf / s[:, None])), -127, 127).astype(np.int8)
    return q, s


def _wrong_transposed_gemm(qa, qw):
    return (qa.astype(np.float64) @ qw.astype(np.float64)[:, : qa.shape[1]].T).astype(np.int32) \
        if qw.shape[0] >= qa.shape[1] else (qa.astype(np.float64)[:, ::-1] @ qw.astype(np.float64).T).astype(np.int32)


def _wrong_norm_no_offset(x_bits, w, eps, offset=1.0, residual_bits=None):
    return _RMS_NORM(x_bits, w, eps, 0.0, residual_bits)


def _wrong_norm_fused_scale(x_bits, w, eps, offset=1.0, residual_bits=None):
    xf = O.bf16_to_f32(x_bits)
    ss = np.float32((xf.astype(np.float64) ** 2).sum(-1))
    rstd = np.float32(1) / np.sqrt(np.float32(ss) / np.float32(xf.shape[-1]) + np.float32(eps))
    return O.f32_to_bf16(xf * (rstd[..., None] * (np.float32(offset) + w))), x_bits


def _kat_failures(kat, monkey):
    """Run the KAT checks with one oracle function replaced; return the number of failing checks."""
    fails = 0
    for check in (test_kat_quant, test_kat_quant_weight, test_kat_gemm, test_kat_rms_norm):
        with monkey.context() as mp:
            for name, fn in monkey._plant.items():
                mp.setattr(O, name, fn)
            try:
                check(kat)
            except AssertionError:
                fails += 1
    return fails


@pytest.mark.parametrize("name,fn", [
    ("epilogue", _wrong_epilogue_order),
    ("quant_act", _wrong_round_away),
    ("quant_act", _wrong_no_eps_floor),
    ("int_gemm", _wrong_transposed_gemm),
    ("rms_norm", _wrong_norm_no_offset),
    ("rms_norm", _wrong_norm_fused_scale),
    ("quant_weight", _wrong_weight_round_away),
    ("quant_weight", _wrong_weight_no_eps_floor),
    ("quant_weight", _wrong_weight_per_column),
])
def test_planted_mistakes_are_caught(kat, monkeypatch, name, fn):
    monkeypatch._plant = {name: fn}
    assert _kat_failures(kat, monkeypatch) >= 1, f"a wrong {name} passed every known-answer check"


def test_rope_matches_torch_bf16_ops_and_closed_forms():
    """bf16 RoPE: bit-exact against the same formula as torch bf16 tensor ops on the CPU (the model's
    own attention arithmetic); position 0 (cos 1, sin 0) is the identity; a quarter turn maps
    (x1, x2) to (-x2, x1) exactly."""
    rng = np.random.default_rng(31)
    x = O.f32_to_bf16(rng.standard_normal((7, 3, 64)).astype(np.float32) * 4)
    ang = rng.uniform(0, 6.3, (7, 1, 32)).astype(np.float32)
    cb, sb = O.f32_to_bf16(np.cos(ang)), O.f32_to_bf16(np.sin(ang))
    got = O.rope(x, cb, sb)
    tx, tc, ts = (_torch_from_bf16(a) for a in (x, cb, sb))
    cs = torch.cat((tc, tc), -1)
    sn = torch.cat((-ts, ts), -1)
    ref = tx * cs + torch.cat((tx[..., 32:], tx[..., :32]), -1) * sn
    assert np.array_equal(got, _bf16_from_torch(ref))
    one, zero = O.f32_to_bf16(np.ones((1, 1, 32), np.float32)), O.f32_to_bf16(np.zeros((1, 1, 32), np.float32))
    assert np.array_equal(O.rope(x, one, zero), x)
    quarter = O.rope(x, zero, one)
    assert np.array_equal(O.bf16_to_f32(quarter[..., :32]), -O.bf16_to_f32(x[..., 32:]))
    assert np.array_equal(quarter[..., 32:], x[..., :32])


def test_attention_oracle_against_torch_and_closed_forms():
    """Causal GQA attention: torch's math SDPA (float64, CPU) with enable_gqa; the first position
    attends only to itself (o = v_0); equal keys give the running mean of v."""
    import torch.nn.functional as F
    rng = np.random.default_rng(41)
    B, S, HQ, HK, D = 2, 19, 8, 2, 16
    q, k, v = (rng.standard_normal((B, S, h, D)) for h in (HQ, HK, HK))
    got = O.causal_gqa_attention(q, k, v, 0.25)
    tq, tk, tv = (torch.tensor(a).transpose(1, 2) for a in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True, scale=0.25, enable_gqa=True).transpose(1, 2)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(got[:, 0], np.repeat(v[:, 0], HQ // HK, axis=1), rtol=1e-12)
    k_same = np.repeat(k[:, :1], S, axis=1)
    mean = np.cumsum(v, axis=1) / np.arange(1, S + 1)[None, :, None, None]
    np.testing.assert_allclose(O.causal_gqa_attention(q, k_same, v, 0.25), np.repeat(mean, HQ // HK, axis=2),
                               rtol=1e-10, atol=1e-12)


def test_attention_oracle_queries_after_a_prefix():
    """Sq < Sk (the queries are the last Sq positions): torch's math SDPA with the explicit mask
    key u <= t + Sk - Sq; the same rows of the full Sk x Sk attention (queries padded in front);
    a one-query row over Sk keys attends to all of them (plain softmax)."""
    import torch.nn.functional as F
    rng = np.random.default_rng(43)
    B, Sq, Sk, HQ, HK, D = 2, 7, 30, 8, 2, 16
    q = rng.standard_normal((B, Sq, HQ, D))
    k, v = (rng.standard_normal((B, Sk, HK, D)) for _ in range(2))
    got = O.causal_gqa_attention(q, k, v, 0.3)
    mask = torch.arange(Sk)[None, :] <= (torch.arange(Sq)[:, None] + Sk - Sq)
    tq, tk, tv = (torch.tensor(a).transpose(1, 2) for a in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=0.3, enable_gqa=True).transpose(1, 2)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-12)
    qp = np.zeros((B, Sk, HQ, D))
    qp[:, Sk - Sq:] = q
    np.testing.assert_allclose(got, O.causal_gqa_attention(qp, k, v, 0.3)[:, Sk - Sq:], rtol=1e-12, atol=1e-14)
    one = O.causal_gqa_attention(q[:, -1:], k, v, 0.3)
    s = 0.3 * np.einsum("bhd,bkhd->bhk", q[:, -1], np.repeat(k, HQ // HK, axis=2))
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(one[:, 0], np.einsum("bhk,bkhd->bhd", p, np.repeat(v, HQ // HK, axis=2)), rtol=1e-10)


# ---------------------------------------------------------------- full-attention extras
def test_sigmoid_bf16_equals_torch_cpu_on_every_code():
    """sigmoid_bf16 against torch.sigmoid on bf16 CPU tensors (a library, not the reference), for every
    finite bf16 code: identical bits.  Plus closed forms: sigmoid(0) = 0.5, sigmoid(g) + sigmoid(-g) = 1
    within rounding, monotone, 0 / 1 far out."""
    codes = np.arange(65536, dtype=np.uint16)
    g = O.bf16_to_f32(codes)
    fin = np.isfinite(g)
    s = O.sigmoid_bf16(codes)
    t = torch.sigmoid(torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16)).view(torch.int16).numpy()
    assert np.array_equal(s[fin], t.view(np.uint16)[fin])
    assert O.bf16_to_f32(O.sigmoid_bf16(np.array([0], np.uint16)))[0] == 0.5
    sv = O.bf16_to_f32(s[fin])
    order = np.argsort(g[fin], kind="stable")
    assert np.all(np.diff(sv[order]) >= 0)
    pos = codes[fin & (g > 0)]
    neg = pos | np.uint16(0x8000)
    assert np.all(np.abs(O.bf16_to_f32(O.sigmoid_bf16(pos)) + O.bf16_to_f32(O.sigmoid_bf16(neg)) - 1.0) <= 2 ** -8)
    assert O.bf16_to_f32(O.sigmoid_bf16(O.f32_to_bf16(np.array([100.0], np.float32))))[0] == 1.0


def test_gate_mul_matches_torch_bf16_ops():
    """o * torch.sigmoid(gate) on bf16 CPU tensors, the reference's op sequence (fast_runtime.py:240)."""
    rng = np.random.default_rng(40)
    a = O.f32_to_bf16(rng.standard_normal((64, 512)).astype(np.float32) * 3)
    gt = O.f32_to_bf16(rng.standard_normal((64, 512)).astype(np.float32) * 4)
    ta, tg = (torch.from_numpy(x.view(np.int16)).view(torch.bfloat16) for x in (a, gt))
    ref = (ta * torch.sigmoid(tg)).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.gate_mul(a, gt), ref)
    # closed form: a gate of 0 halves a exactly (bf16 * 0.5 is exact)
    assert np.array_equal(O.bf16_to_f32(O.gate_mul(a, np.zeros_like(gt))), O.bf16_to_f32(a) * 0.5)


def test_rope_partial_and_head_norm():
    """rope_partial with rot_dim = head_dim is rope; with rot_dim < head_dim its first rot_dim dims are rope
    of that slice and the rest pass through; head_rms_norm is rms_norm of each head (zero-centred weight)."""
    rng = np.random.default_rng(41)
    x = O.f32_to_bf16(rng.standard_normal((6, 4, 256)).astype(np.float32))
    ang = rng.uniform(-3, 3, (6, 1, 128)).astype(np.float32)
    c, s = O.f32_to_bf16(np.cos(ang)), O.f32_to_bf16(np.sin(ang))
    assert np.array_equal(O.rope_partial(x, c, s, 256), O.rope(x, c, s))
    y = O.rope_partial(x, c[..., :32], s[..., :32], 64)
    assert np.array_equal(y[..., 64:], x[..., 64:])
    assert np.array_equal(y[..., :64], O.rope(x[..., :64], c[..., :32], s[..., :32]))
    # rotate_half pairs dim i with i + 32 inside the 64 rotated dims: a quarter turn maps (a, b) to (-b, a)
    quarter_c = O.f32_to_bf16(np.zeros((1, 1, 32), np.float32))
    quarter_s = O.f32_to_bf16(np.ones((1, 1, 32), np.float32))
    z = O.bf16_to_f32(O.rope_partial(x, quarter_c, quarter_s, 64))
    xf = O.bf16_to_f32(x)
    assert np.array_equal(z[..., :32], -xf[..., 32:64]) and np.array_equal(z[..., 32:64], xf[..., :32])
    w = rng.normal(0, 0.1, 256).astype(np.float32)
    wb = O.round_bf16(w)
    assert np.array_equal(O.head_rms_norm(x, wb, 1e-6), O.rms_norm(x.reshape(-1, 256), wb, 1e-6)[0].reshape(x.shape))
