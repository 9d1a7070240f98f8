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


def _check_norm_quant(h_bits, norm_w, cfg, y_bits, q, s, what):
    """Fused norm + quant rows: the normed row y within one bf16 ulp of the oracle's norm of h (the fp32
    sum-of-squares order is not pinned), and q, s bit-exact with the oracle's quantizer applied to the
    kernel's own y -- on every row."""
    yo, _ = O.rms_norm(h_bits, O.bf16_to_f32(bits(norm_w)), cfg.eps, 0.0)
    within_one_ulp(y_bits, yo, min_exact=0.99)
    qy, sy = O.quant_act(O.bf16_to_f32(y_bits))
    assert np.array_equal(q, qy) and np.array_equal(s, sy), f"{what} norm + quant: int8 / scale vs the kernel's y"
    same = np.all(q == O.quant_act(O.bf16_to_f32(yo))[0], axis=1)
    print(f"[case] {what} norm+quant rows equal to the oracle's own: {same.mean():.4f}", file=sys.stderr)


@pytest.fixture(autouse=True)
def _strict(monkeypatch):
    monkeypatch.setattr(int8_kernels, "STRICT", True)


def test_small_stack_stage_by_stage(gpu):
    print("[case] small stack", file=sys.stderr, flush=True)
    cfg = StackConfig(layers=2, hidden=512, intermediate=1024, heads=8, kv_heads=2, head_dim=64, vocab=4096,
                      n_options=31)
    st = W8A8Stack(cfg, device=gpu, seed=3, last_only=False)
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
    st = W8A8Stack(cfg, device=gpu, seed=7, last_only=False)
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

    # the same run with the whole last layer (every row) traced: the prefill ran that layer last-only
    # (its query side, attention, O and MLP at the 8 picked rows), which must give the same bits
    rows_last = torch.arange(B, device=gpu, dtype=torch.int32) * S + (S - 1)
    lo, cnt = st.slices(None, None, B, gpu)
    h = st.embed.index_select(0, ids)
    trace = []
    for i, L in enumerate(st.layers):
        h = st.layer_forward(L, h, B, S, trace if i == cfg.layers - 1 else None)
    logits2, probs2 = st.readout(h, rows_last, st.final_norm, cfg.eps, offset=0.0, lo=lo, cnt=cnt,
                                 probs_width=cfg.n_options)
    torch.cuda.synchronize()
    assert torch.equal(logits2, logits) and torch.equal(probs2, probs), "full last layer differs from last-only"

    L, t = st.layers[-1], trace[0]
    rng = np.random.default_rng(4)
    rows = np.unique(np.concatenate([rng.choice(B * S, 60, replace=False), [0, S - 1, S, B * S - 1]]))
    trows = torch.from_numpy(rows).to(gpu)
    sel = lambda x: x.index_select(0, trows)  # noqa: E731
    hb = bits(sel(t["h"]))
    # input norm + quant: the kernel's normed bf16 row within one ulp of the oracle's, and its int8 row and
    # scale bit-exact with the oracle's quantizer applied to that row, for every sampled row
    q, s = sel(t["q"]).cpu().numpy(), sel(t["s"]).cpu().numpy()
    _check_norm_quant(hb, L.input_norm, cfg, bits(sel(t["y"])), q, s, "input")
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
    q2, s2 = sel(t["q2"]).cpu().numpy(), sel(t["s2"]).cpu().numpy()
    _check_norm_quant(h1, L.post_norm, cfg, bits(sel(t["y2"])), q2, s2, "post-attention")
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


def _padded_batch(cfg, gpu, lengths, width, seed):
    """Requests of these lengths padded at the end to a common width, as the engine packs them, and the
    rows of their last real positions."""
    gen = torch.Generator().manual_seed(seed)
    ids = torch.zeros(len(lengths) * width, dtype=torch.long)
    for b, n in enumerate(lengths):
        ids[b * width:b * width + n] = torch.randint(0, cfg.vocab, (n,), generator=gen)
    rows = torch.tensor([b * width + n - 1 for b, n in enumerate(lengths)], dtype=torch.int32)
    return ids.to(gpu), rows.to(gpu)


@pytest.mark.parametrize("interval", [0, 3])
def test_last_only_equals_full_last_layer(gpu, interval):
    """The last-only last layer (prefill_engine.py:283-339: K / V and the keys' RoPE over every row,
    the query projection, attention, O projection and MLP at the picked rows) against the same stack
    running the whole last layer: logits and probabilities bit-identical, for requests padded to a common
    width (picked rows inside the batch, so each query sees only its own request's first keys), with and
    without a prefix state.  interval 3 makes the last layer a gated-delta-net layer (mixer over every
    row, MLP at the picked rows)."""
    print(f"[case] last-only vs full last layer, interval {interval}", file=sys.stderr, flush=True)
    cfg = StackConfig(layers=2, hidden=512, intermediate=1024, heads=4, kv_heads=1, head_dim=256, vocab=4096,
                      n_options=31, full_attention_interval=interval, linear_k_heads=2, linear_v_heads=4)
    last = W8A8Stack(cfg, device=gpu, seed=11)
    full = W8A8Stack(cfg, device=gpu, seed=11, last_only=False)
    assert type(last.layers[-1]).__name__ == ("GDNBlock" if interval == 3 else "Layer")
    lengths, width = [128, 77, 100, 1], 128
    ids, rows = _padded_batch(cfg, gpu, lengths, width, seed=12)
    lo, cnt = last.slices(["choice", "noul", "choice", "choice"], [31, 2, 5, 31], len(lengths), gpu)
    B = len(lengths)
    a = last.forward_last(ids, B, rows, lo, cnt)
    b = full.forward_last(ids, B, rows, lo, cnt)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), "last-only readout differs from the full layer's"
    # continuations of a 64-token prefix
    pre = torch.randint(0, cfg.vocab, (64,), generator=torch.Generator().manual_seed(13)).to(gpu)
    pa, pb = last.prefix_state(pre), full.prefix_state(pre)
    a = last.forward_last(ids, B, rows, lo, cnt, prefix=pa)
    b = full.forward_last(ids, B, rows, lo, cnt, prefix=pb)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), "last-only continuation differs"
    assert not int8_kernels.STATS["fallback"]


def test_last_only_layer_stage_by_stage(gpu):
    """The last-only layer's stages against the oracle from the kernels' own inputs: norm + quant of every
    row, the K / V GEMM over every row and the query GEMM at the picked rows (bit-exact), RoPE of the keys
    and of each query at its own position (bit-exact), then O + residual and the MLP at the picked rows."""
    print("[case] last-only layer stage by stage", file=sys.stderr, flush=True)
    cfg = StackConfig(layers=1, hidden=512, intermediate=1024, heads=4, kv_heads=1, head_dim=256, vocab=4096,
                      n_options=31)
    st = W8A8Stack(cfg, device=gpu, seed=21)
    lengths, width = [96, 33, 64], 96
    ids, rows = _padded_batch(cfg, gpu, lengths, width, seed=22)
    B = len(lengths)
    lo, cnt = st.slices(None, None, B, gpu)
    trace = []
    logits, probs = st.forward_last(ids, B, rows, lo, cnt, trace=trace)
    torch.cuda.synchronize()
    L, t = st.layers[0], trace[0]
    assert t["kind"] == "attention_last"
    hq, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
    hb = bits(t["h"])
    q, s = t["q"].cpu().numpy(), t["s"].cpu().numpy()
    _check_norm_quant(hb, L.input_norm, cfg, bits(t["y"]), q, s, "input")
    W, sw = L.qkv.qweight.cpu().numpy(), L.qkv.wscale.cpu().numpy()
    nq = hq * d
    kv = O.epilogue(O.int_gemm(q, W[nq:]), s, sw[nq:])
    assert np.array_equal(bits(t["kv"]), kv), "K / V GEMM over every row"
    r = rows.cpu().numpy()
    qr = O.epilogue(O.int_gemm(q[r], W[:nq]), s[r], sw[:nq])
    assert np.array_equal(bits(t["qr"]), qr), "query GEMM at the picked rows"
    cos, sin = (bits(x) for x in st._tables(width, gpu))
    kpos = np.arange(B * width) % width
    krot = kv.reshape(B * width, 2 * hk, d).copy()
    krot[:, :hk] = O.rope(krot[:, :hk], cos[kpos][:, None, :], sin[kpos][:, None, :])
    assert np.array_equal(bits(t["kv_rope"]), krot.reshape(B * width, -1)), "RoPE of the keys"
    qpos = r - np.arange(B) * width
    qrot = O.rope(qr.reshape(B, hq, d), cos[qpos][:, None, :], sin[qpos][:, None, :])
    assert np.array_equal(bits(t["qr_rope"]), qrot.reshape(B, -1)), "RoPE of the queries at their positions"
    # attention of each picked query over its own request's first keys (oracle, float64), then O + residual
    kr = O.bf16_to_f32(krot.reshape(B, width, 2 * hk, d)[:, :, :hk])
    vr = O.bf16_to_f32(kv.reshape(B, width, 2 * hk, d)[:, :, hk:])
    a = O.bf16_to_f32(bits(t["a"])).reshape(B, hq, d)
    for b in range(B):
        n = qpos[b] + 1
        want = O.causal_gqa_attention(O.bf16_to_f32(qrot[b])[None, None], kr[b:b + 1, :n], vr[b:b + 1, :n],
                                      1.0 / 16)[0, 0]
        np.testing.assert_allclose(a[b], want, rtol=2e-2, atol=2e-2)
    qa, sa = O.quant_act(O.bf16_to_f32(bits(t["a"])))
    assert np.array_equal(t["qa"].cpu().numpy(), qa) and np.array_equal(t["sa"].cpu().numpy(), sa)
    h1 = O.epilogue(O.int_gemm(qa, L.o.qweight.cpu().numpy()), sa, L.o.wscale.cpu().numpy())
    h1 = O.f32_to_bf16(O.bf16_to_f32(h1) + O.bf16_to_f32(hb[r]))
    assert np.array_equal(bits(t["h1"]), h1), "O + residual at the picked rows"
    q2, s2 = t["q2"].cpu().numpy(), t["s2"].cpu().numpy()
    _check_norm_quant(h1, L.post_norm, cfg, bits(t["y2"]), q2, s2, "post-attention")
    _check_mlp(L, t, cfg, 0)
    fin = trace[-1]
    zo = O.readout(bits(fin["h_final"]), fin["rows"].cpu().numpy(), O.bf16_to_f32(bits(st.final_norm)), cfg.eps,
                   st.readout.weight.cpu().numpy(), offset=0.0)
    np.testing.assert_allclose(logits.cpu().numpy(), zo, rtol=1e-4, atol=1e-4)
    assert not int8_kernels.STATS["fallback"]


def test_last_only_sdpa_path(gpu):
    """Head shapes the flash kernel does not serve take torch SDPA with a per-request key mask at the
    picked rows; it agrees with the full last layer's is_causal SDPA within bf16 rounding."""
    print("[case] last-only SDPA path", file=sys.stderr, flush=True)
    cfg = StackConfig(layers=2, hidden=512, intermediate=1024, heads=8, kv_heads=2, head_dim=64, vocab=4096,
                      n_options=31)
    last = W8A8Stack(cfg, device=gpu, seed=31)
    full = W8A8Stack(cfg, device=gpu, seed=31, last_only=False)
    ids, rows = _padded_batch(cfg, gpu, [64, 40], 64, seed=32)
    lo, cnt = last.slices(None, None, 2, gpu)
    a = last.forward_last(ids, 2, rows, lo, cnt)
    b = full.forward_last(ids, 2, rows, lo, cnt)
    torch.cuda.synchronize()
    np.testing.assert_allclose(a[1].cpu().numpy(), b[1].cpu().numpy(), atol=2e-2)


def test_reference_attention_layer_stage_by_stage(gpu):
    """A full-attention layer with the reference model's extras (q_proj output gate, q / k head norm,
    RoPE on 64 dims; fast_runtime.py:229-241): the gated QKV GEMM bit-exact, head norm + RoPE of the q
    and k heads within two bf16 ulps of the oracle (the gate and v columns untouched), attention against
    the float64 oracle, the gated o_proj input (one ulp of the oracle's gate, int8 bit-exact given the
    kernel's gated row), then O + residual and the MLP as in the other layers."""
    print("[case] reference attention layer", file=sys.stderr, flush=True)
    cfg = StackConfig.reference_model(layers=1, full_attention_interval=0, hidden=512, intermediate=1024,
                                      heads=4, kv_heads=1, vocab=4096, n_options=31)
    st = W8A8Stack(cfg, device=gpu, seed=51, last_only=False)
    B, S = 2, 96
    ids = torch.randint(0, cfg.vocab, (B * S,), generator=torch.Generator().manual_seed(52)).to(gpu)
    trace = []
    st.prefill(ids, B, trace=trace)
    torch.cuda.synchronize()
    L, t = st.layers[0], trace[0]
    hq, hk, d = cfg.heads, cfg.kv_heads, cfg.head_dim
    q, s = t["q"].cpu().numpy(), t["s"].cpu().numpy()
    qkv = O.epilogue(O.int_gemm(q, L.qkv.qweight.cpu().numpy()), s, L.qkv.wscale.cpu().numpy())
    assert qkv.shape[1] == (2 * hq + 2 * hk) * d
    assert np.array_equal(bits(t["qkv"]), qkv), "gated QKV GEMM"
    cos, sin = (bits(x) for x in st._tables(S, gpu))
    pos = np.arange(B * S) % S
    xr = qkv.reshape(B * S, -1, d)
    want = xr.copy()
    for sl, w in ((slice(0, hq), L.q_norm), (slice(2 * hq, 2 * hq + hk), L.k_norm)):
        want[:, sl] = O.rope_partial(O.head_rms_norm(xr[:, sl], O.bf16_to_f32(bits(w)), cfg.eps, 1.0),
                                     cos[pos][:, None, :], sin[pos][:, None, :], 64)
    got = bits(t["qkv_rope"]).reshape(B * S, -1, d)
    assert np.array_equal(got[:, hq:2 * hq], xr[:, hq:2 * hq]) and np.array_equal(got[:, -hk:], xr[:, -hk:])
    heads = np.r_[0:hq, 2 * hq:2 * hq + hk]
    u = np.abs(O.bf16_to_f32(got[:, heads]) - O.bf16_to_f32(want[:, heads])) / O.bf16_ulp(want[:, heads])
    assert u.max() <= 2.0001 and np.mean(got[:, heads] == want[:, heads]) >= 0.99
    # attention on the kernel's rotated q / k
    g4 = got.reshape(B, S, -1, d)
    a_ref = O.causal_gqa_attention(O.bf16_to_f32(g4[:, :, :hq]), O.bf16_to_f32(g4[:, :, 2 * hq:2 * hq + hk]),
                                   O.bf16_to_f32(g4[:, :, 2 * hq + hk:]), 1.0 / 16)
    # row-relative L2 error of each (request, position, head) row <= 0.02: the reference's attention
    # acceptance criterion (int8_runtime.py:445-488, ATTN_TOL; bf16 probabilities and outputs)
    ak = O.bf16_to_f32(bits(t["a"])).reshape(B, S, hq, d)
    rel = np.linalg.norm(ak - a_ref, axis=-1) / np.maximum(np.linalg.norm(a_ref, axis=-1), 1e-30)
    assert rel.max() <= 0.02, f"attention row error {rel.max():.4f}"
    # the gated o_proj input
    gk = bits(t["gated"])
    gref = O.gate_mul(bits(t["a"]), got[:, hq:2 * hq].reshape(B * S, -1))
    u = np.abs(O.bf16_to_f32(gk) - O.bf16_to_f32(gref)) / O.bf16_ulp(gref)
    assert u.max() <= 1.0001 and np.mean(gk == gref) >= 0.999
    qa, sa = O.quant_act(O.bf16_to_f32(gk))
    assert np.array_equal(t["qa"].cpu().numpy(), qa) and np.array_equal(t["sa"].cpu().numpy(), sa)
    h1 = O.epilogue(O.int_gemm(qa, L.o.qweight.cpu().numpy()), sa, L.o.wscale.cpu().numpy())
    h1 = O.f32_to_bf16(O.bf16_to_f32(h1) + O.bf16_to_f32(bits(t["h"])))
    assert np.array_equal(bits(t["h1"]), h1), "o_proj + residual"
    _check_mlp(L, t, cfg, 0)


def test_reference_model_last_only_bit_identical(gpu):
    """The reference model's layout (GDN layers, every fourth full attention with the gate, q / k norm and
    partial RoPE): last-only equals the full last layer bit for bit, padded requests and a prefix too."""
    print("[case] reference model last-only", file=sys.stderr, flush=True)
    cfg = StackConfig.reference_model(layers=4, hidden=512, intermediate=1024, heads=4, kv_heads=1, vocab=4096,
                                      n_options=31, linear_k_heads=2, linear_v_heads=4)
    last = W8A8Stack(cfg, device=gpu, seed=61)
    full = W8A8Stack(cfg, device=gpu, seed=61, last_only=False)
    assert [type(L).__name__ for L in last.layers] == ["GDNBlock"] * 3 + ["Layer"]
    ids, rows = _padded_batch(cfg, gpu, [128, 90, 5], 128, seed=62)
    lo, cnt = last.slices(None, None, 3, gpu)
    a = last.forward_last(ids, 3, rows, lo, cnt)
    b = full.forward_last(ids, 3, rows, lo, cnt)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    p = a[1].cpu().numpy()
    assert np.isfinite(p).all() and np.allclose(p.sum(1), 1.0, atol=1e-5)
    pre = torch.randint(0, cfg.vocab, (64,), generator=torch.Generator().manual_seed(63)).to(gpu)
    a = last.forward_last(ids, 3, rows, lo, cnt, prefix=last.prefix_state(pre))
    b = full.forward_last(ids, 3, rows, lo, cnt, prefix=full.prefix_state(pre))
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
