"""The synthetic W8A8 decoder stack (mica_amd.model) checked stage by stage against the oracle.

Attention is a torch op outside the W8A8 path; every other stage of every layer is recomputed by the
oracle from the kernel's own input to that stage: fused norm + quant (int8 / scales bit-exact given
the kernel's normed row is within one bf16 ulp), QKV / O / down GEMMs with their residual epilogues
(bit-exact), the fused gate+up SiLU epilogue (one bf16 ulp), the requantizations (bit-exact), and the
last-position readout (logits 1e-4 relative, option probabilities 1e-3 absolute).
"""
import sys

import numpy as np
import pytest
import torch

from mica_amd import int8_kernels
from mica_amd.model import StackConfig, W8A8Stack
from oracle import w8a8 as O

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def within_one_ulp(got, ref, min_exact=0.999):
    g, r = O.bf16_to_f32(got), O.bf16_to_f32(ref)
    assert np.all(np.abs(g - r) <= O.bf16_ulp(ref) * 1.0001)
    assert np.mean(got == ref) >= min_exact


def _check_mlp(L, t, cfg, li):
    """The post-attention norm + quant, fused gate+up SiLU, requant and down + residual of one layer,
    each recomputed by the oracle from the kernel's own input to that stage."""
    h1 = bits(t["h1"])
    # post-attention norm + quant
    g2 = O.bf16_to_f32(bits(L.post_norm))
    y2, _ = O.rms_norm(h1, g2, cfg.eps, 0.0)
    q2o, s2o = O.quant_act(O.bf16_to_f32(y2))
    q2, s2 = t["q2"].cpu().numpy(), t["s2"].cpu().numpy()
    assert (np.all(q2 == q2o, axis=1) & (s2 == s2o)).mean() > 0.97
    # fused gate+up SiLU from the kernel's q2, s2 (packed weight: 64-row gate / up groups)
    qp, sp = L.gate_up.qweight.cpu().numpy(), L.gate_up.wscale.cpu().numpy()
    n = qp.shape[0] // 2
    grp = qp.reshape(n // 64, 2, 64, -1)
    sgr = sp.reshape(n // 64, 2, 64)
    qg, qu = grp[:, 0].reshape(n, -1), grp[:, 1].reshape(n, -1)
    sg, su = sgr[:, 0].reshape(n), sgr[:, 1].reshape(n)
    gv = O.epilogue(O.int_gemm(q2, qg), s2, sg)
    uv = O.epilogue(O.int_gemm(q2, qu), s2, su)
    within_one_ulp(bits(t["g"]), O.silu_mul(gv, uv))
    # requant of h and the down projection + residual
    qho, sho = O.quant_act(O.bf16_to_f32(bits(t["g"])))
    assert np.array_equal(t["qh"].cpu().numpy(), qho) and np.array_equal(t["sh"].cpu().numpy(), sho)
    h2 = O.epilogue(O.int_gemm(qho, L.down.qweight.cpu().numpy()), sho, L.down.wscale.cpu().numpy())
    h2 = O.f32_to_bf16(O.bf16_to_f32(h2) + O.bf16_to_f32(bits(t["h1"])))
    assert np.array_equal(bits(t["h2"]), h2), f"layer {li}: down + residual"


@pytest.fixture(autouse=True)
def _strict(monkeypatch):
    monkeypatch.setattr(int8_kernels, "STRICT", True)


def test_small_stack_stage_by_stage(gpu):
    print("[case] small stack", file=sys.stderr, flush=True)
    cfg = StackConfig(layers=2, hidden=512, intermediate=1024, heads=8, kv_heads=2, head_dim=64, vocab=4096,
                      n_options=31)
    st = W8A8Stack(cfg, device=gpu, seed=3)
    B, S = 2, 96
    ids = torch.randint(0, cfg.vocab, (B * S,), generator=torch.Generator().manual_seed(5)).to(gpu)
    trace = []
    logits, probs = st.prefill(ids, B, kinds=["noul", "choice"], n_choices=[2, 17], trace=trace)
    torch.cuda.synchronize()
    for li, (L, t) in enumerate(zip(st.layers, trace[:-1])):
        hb = bits(t["h"])
        g1 = O.bf16_to_f32(bits(L.input_norm))
        yo, _ = O.rms_norm(hb, g1, cfg.eps, 0.0)
        qo, so = O.quant_act(O.bf16_to_f32(yo))
        q, s = t["q"].cpu().numpy(), t["s"].cpu().numpy()
        same = np.all(q == qo, axis=1) & (s == so)
        assert same.mean() > 0.97, f"layer {li}: norm+quant rows differing: {(~same).sum()}"
        # QKV GEMM from the kernel's q, s
        qkv = O.epilogue(O.int_gemm(q, L.qkv.qweight.cpu().numpy()), s, L.qkv.wscale.cpu().numpy())
        assert np.array_equal(bits(t["qkv"]), qkv), f"layer {li}: qkv"
        # in-place RoPE on the q and k heads: bit-exact bf16 arithmetic
        hq, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
        cos, sin = st._tables(S, st.device)
        pos = np.arange(B * S) % S
        xr = qkv.reshape(B * S, hq + 2 * hk, d)
        want = xr.copy()
        want[:, :hq + hk] = O.rope(xr[:, :hq + hk], bits(cos)[pos][:, None, :], bits(sin)[pos][:, None, :])
        assert np.array_equal(bits(t["qkv_rope"]), want.reshape(B * S, -1)), f"layer {li}: rope"
        # O projection + residual from the kernel's attention output
        qa, sa = O.quant_act(O.bf16_to_f32(bits(t["a"])))
        assert np.array_equal(t["qa"].cpu().numpy(), qa) and np.array_equal(t["sa"].cpu().numpy(), sa)
        h1 = O.epilogue(O.int_gemm(qa, L.o.qweight.cpu().numpy()), sa, L.o.wscale.cpu().numpy())
        h1 = O.f32_to_bf16(O.bf16_to_f32(h1) + O.bf16_to_f32(hb))
        assert np.array_equal(bits(t["h1"]), h1), f"layer {li}: o_proj + residual"
        _check_mlp(L, t, cfg, li)
    fin = trace[-1]
    rows = fin["rows"].cpu().numpy()
    W = st.readout.weight.cpu().numpy()
    zo = O.readout(bits(fin["h_final"]), rows, O.bf16_to_f32(bits(st.final_norm)), cfg.eps, W, offset=0.0)
    np.testing.assert_allclose(logits.cpu().numpy(), zo, rtol=1e-4, atol=1e-4)
    p = probs.cpu().numpy()
    np.testing.assert_allclose(p[0, :2], O.option_probs(zo[0], "noul"), atol=1e-3)
    np.testing.assert_allclose(p[1, :17], O.option_probs(zo[1], "choice", 17), atol=1e-3)
    assert not int8_kernels.STATS["fallback"]


def test_full_shape_stack_runs_one_layer(gpu):
    """The 4B shape itself (hidden 2560, intermediate 9728, QKV 6144, vocab 151936) with one layer
    and 2 x 2048 packed tokens: finite option probabilities that sum to one."""
    print("[case] 4B-shaped stack, 1 layer", file=sys.stderr, flush=True)
    st = W8A8Stack(StackConfig(layers=1), device=gpu, seed=1)
    ids = torch.randint(0, st.cfg.vocab, (2 * 2048,), device=gpu)
    logits, probs = st.prefill(ids, 2)
    p = probs.cpu().numpy()
    assert np.isfinite(p).all() and np.allclose(p.sum(1), 1.0, atol=1e-5)
    assert st.linear_ops_per_token() == 2 * (6144 * 2560 + 2560 * 4096 + 3 * 9728 * 2560)


def test_hybrid_stack_gdn_and_attention_layers(gpu):
    """The hybrid layout (full_attention_interval 2: a gated-delta-net layer, then a full-attention
    layer, twice): each GDN mixer output equals the GDN layer module run alone on the same input
    (bit-identical; the module itself is checked stage by stage against the oracle in
    test_gpu_gdn_layer.py), every MLP half is checked against the oracle as above, and the readout
    gives finite probabilities that sum to one."""
    print("[case] hybrid stack", file=sys.stderr, flush=True)
    cfg = StackConfig(layers=4, hidden=512, intermediate=1024, heads=4, kv_heads=1, head_dim=256, vocab=4096,
                      n_options=31, full_attention_interval=2, linear_k_heads=2, linear_v_heads=4)
    st = W8A8Stack(cfg, device=gpu, seed=7)
    assert [type(L).__name__ for L in st.layers] == ["GDNBlock", "Layer", "GDNBlock", "Layer"]
    B, S = 2, 80
    ids = torch.randint(0, cfg.vocab, (B * S,), generator=torch.Generator().manual_seed(9)).to(gpu)
    trace = []
    logits, probs = st.prefill(ids, B, trace=trace)
    torch.cuda.synchronize()
    for li, (L, t) in enumerate(zip(st.layers, trace[:-1])):
        assert t["kind"] == ("gdn" if li % 2 == 0 else "attention")
        if t["kind"] == "gdn":
            again = L.mixer(t["h"], B)
            torch.cuda.synchronize()
            assert torch.equal(again, t["h1"]), f"layer {li}: GDN mixer"
        _check_mlp(L, t, cfg, li)
    p = probs.cpu().numpy()
    assert np.isfinite(p).all() and np.allclose(p.sum(1), 1.0, atol=1e-5)
    hk, hv, H = 2, 4, 512
    gdn_ops = ((2 * hk + hv) * 128 + hv * 128 + 2 * hv) * H + H * hv * 128
    attn_ops = (4 + 2) * 256 * H + H * 4 * 256
    assert st.linear_ops_per_token() == 2 * (2 * gdn_ops + 2 * attn_ops + 4 * 3 * 1024 * H)
    assert not int8_kernels.STATS["fallback"]


def test_config4_full_stack_8x2048(gpu):
    """Config 4 at its size: the 36-layer 4B-shaped stack (hidden 2560, intermediate 9728, QKV 6144,
    vocab 151936) over 8 requests x 2048 packed tokens (M = 16384), logits only at each request's last
    position over 2 + 255 label ids, softmaxed.  The probabilities are finite and sum to one; a second
    run traced at the last layer gives the same bits; that layer's norm + quant, QKV, RoPE, O + residual,
    SiLU epilogue, requant and down + residual are recomputed by the oracle on 64 sampled rows from the
    kernels' own inputs to each stage, and the readout of the 8 last rows on all of them
    (release_runtime.py:298-306, 509-517; prefill_engine.py:283-339)."""
    print("[case] config 4: 36 layers, 8 x 2048 tokens", file=sys.stderr, flush=True)
    cfg = StackConfig()
    assert (cfg.layers, cfg.hidden, cfg.intermediate, cfg.vocab) == (36, 2560, 9728, 151936)
    st = W8A8Stack(cfg, device=gpu, seed=4)
    B, S = 8, 2048
    ids = torch.randint(0, cfg.vocab, (B * S,), generator=torch.Generator().manual_seed(44)).to(gpu)
    logits, probs = st.prefill(ids, B)
    torch.cuda.synchronize()
    p = probs.cpu().numpy()
    assert p.shape == (B, cfg.n_options)
    assert np.isfinite(p).all() and np.allclose(p.sum(1), 1.0, atol=1e-5)

    # the same run with the last layer traced (the trace only keeps tensors the run makes anyway)
    rows_last = torch.arange(B, device=gpu, dtype=torch.int32) * S + (S - 1)
    lo, cnt = st.slices(None, None, B, gpu)
    h = st.embed.index_select(0, ids)
    trace = []
    for i, L in enumerate(st.layers):
        h = st.layer_forward(L, h, B, S, trace if i == cfg.layers - 1 else None)
    logits2, probs2 = st.readout(h, rows_last, st.final_norm, cfg.eps, offset=0.0, lo=lo, cnt=cnt,
                                 probs_width=cfg.n_options)
    torch.cuda.synchronize()
    assert torch.equal(logits2, logits) and torch.equal(probs2, probs), "traced run differs from prefill"

    L, t = st.layers[-1], trace[0]
    rng = np.random.default_rng(4)
    rows = np.unique(np.concatenate([rng.choice(B * S, 60, replace=False), [0, S - 1, S, B * S - 1]]))
    trows = torch.from_numpy(rows).to(gpu)
    sel = lambda x: x.index_select(0, trows)  # noqa: E731
    hb = bits(sel(t["h"]))
    # input norm + quant (the normed bf16 row may differ by one ulp: rows that agree quantize exactly)
    yo, _ = O.rms_norm(hb, O.bf16_to_f32(bits(L.input_norm)), cfg.eps, 0.0)
    qo, so = O.quant_act(O.bf16_to_f32(yo))
    q, s = sel(t["q"]).cpu().numpy(), sel(t["s"]).cpu().numpy()
    same = np.all(q == qo, axis=1) & (s == so)
    print(f"[case] config 4 input norm+quant rows matching the oracle: {same.mean():.4f}", file=sys.stderr)
    assert same.mean() >= 0.95
    # QKV from the kernel's q, s: bit-exact
    qkv = O.epilogue(O.int_gemm(q, L.qkv.qweight.cpu().numpy()), s, L.qkv.wscale.cpu().numpy())
    assert np.array_equal(bits(sel(t["qkv"])), qkv), "qkv"
    # RoPE in place on the q and k heads of those rows (positions t % S)
    hq, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
    cos, sin = st._tables(S, gpu)
    pos = rows % S
    xr = qkv.reshape(rows.size, hq + 2 * hk, d)
    want = xr.copy()
    want[:, :hq + hk] = O.rope(xr[:, :hq + hk], bits(cos)[pos][:, None, :], bits(sin)[pos][:, None, :])
    assert np.array_equal(bits(sel(t["qkv_rope"])), want.reshape(rows.size, -1)), "rope"
    # O projection + residual from the kernel's attention output
    qa, sa = O.quant_act(O.bf16_to_f32(bits(sel(t["a"]))))
    assert np.array_equal(sel(t["qa"]).cpu().numpy(), qa) and np.array_equal(sel(t["sa"]).cpu().numpy(), sa)
    h1 = O.epilogue(O.int_gemm(qa, L.o.qweight.cpu().numpy()), sa, L.o.wscale.cpu().numpy())
    h1 = O.f32_to_bf16(O.bf16_to_f32(h1) + O.bf16_to_f32(hb))
    assert np.array_equal(bits(sel(t["h1"])), h1), "o_proj + residual"
    # post-attention norm + quant, SiLU epilogue, requant, down + residual
    y2, _ = O.rms_norm(h1, O.bf16_to_f32(bits(L.post_norm)), cfg.eps, 0.0)
    q2o, s2o = O.quant_act(O.bf16_to_f32(y2))
    q2, s2 = sel(t["q2"]).cpu().numpy(), sel(t["s2"]).cpu().numpy()
    same2 = np.all(q2 == q2o, axis=1) & (s2 == s2o)
    print(f"[case] config 4 post norm+quant rows matching the oracle: {same2.mean():.4f}", file=sys.stderr)
    assert same2.mean() >= 0.95
    qp, sp = L.gate_up.qweight.cpu().numpy(), L.gate_up.wscale.cpu().numpy()
    n = qp.shape[0] // 2
    grp, sgr = qp.reshape(n // 64, 2, 64, -1), sp.reshape(n // 64, 2, 64)
    gv = O.epilogue(O.int_gemm(q2, grp[:, 0].reshape(n, -1)), s2, sgr[:, 0].reshape(n))
    uv = O.epilogue(O.int_gemm(q2, grp[:, 1].reshape(n, -1)), s2, sgr[:, 1].reshape(n))
    g = bits(sel(t["g"]))
    within_one_ulp(g, O.silu_mul(gv, uv))
    qho, sho = O.quant_act(O.bf16_to_f32(g))
    assert np.array_equal(sel(t["qh"]).cpu().numpy(), qho) and np.array_equal(sel(t["sh"]).cpu().numpy(), sho)
    h2 = O.epilogue(O.int_gemm(qho, L.down.qweight.cpu().numpy()), sho, L.down.wscale.cpu().numpy())
    h2 = O.f32_to_bf16(O.bf16_to_f32(h2) + O.bf16_to_f32(h1))
    assert np.array_equal(bits(sel(t["h2"])), h2), "down + residual"
    # readout of the 8 last rows over all 257 label rows, then the option softmax
    last = rows_last.cpu().numpy()
    W = st.readout.weight.cpu().numpy()
    zo = O.readout(bits(h), last, O.bf16_to_f32(bits(st.final_norm)), cfg.eps, W, offset=0.0)
    np.testing.assert_allclose(logits.cpu().numpy(), zo, rtol=1e-4, atol=1e-4)
    for b in range(B):
        np.testing.assert_allclose(p[b], O.option_probs(zo[b], "choice", cfg.n_options), atol=1e-3)
    assert not int8_kernels.STATS["fallback"]
