"""The full-attention layers' extra kernels against the oracle: the per-head q / k RMSNorm with partial RoPE
(mica_head_norm_rope) and the output gate fused with o_proj's quantizer (mica_gate_quant).

Bar: RoPE alone bit-exact (bf16 arithmetic fully determined); the head norm within one bf16 ulp of the
oracle's (its fp32 sum order is not pinned), so norm + RoPE within two; columns outside the q / k heads
untouched.  The gate's sigmoid within one bf16 ulp for every finite bf16 gate (library exp, as SiLU), the
gated row's int8 / scale bit-exact with the oracle quantizer applied to the kernel's own gated row.
"""
import sys

import numpy as np
import pytest
import torch

from mica_amd import fused_kernels
from oracle import w8a8 as O

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def gpu_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def bits_of(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def ulps(got, ref):
    return np.abs(O.bf16_to_f32(got) - O.bf16_to_f32(ref)) / O.bf16_ulp(ref)


def test_sigmoid_every_bf16_gate(gpu):
    """a = 1 (exact), so the gated row is bf16(sigmoid(g)) itself: every finite bf16 code as a gate."""
    note("gate_quant: sigmoid on all bf16 codes")
    codes = np.arange(65536, dtype=np.uint16).reshape(128, 512)
    one = np.full(codes.shape, 0x3F80, np.uint16)
    q, s, y = fused_kernels.gate_quant(gpu_bf16(one), gpu_bf16(codes), return_gated=True)
    yk = bits_of(y)
    fin = np.isfinite(O.bf16_to_f32(codes))
    ref = O.sigmoid_bf16(codes)
    d = ulps(yk[fin], ref[fin])
    assert d.max() <= 1.0001, f"sigmoid off by {d.max():.2f} ulp"
    assert np.mean(yk[fin] == ref[fin]) >= 0.999
    rows = np.all(fin, axis=1)            # rows with a non-finite gate have no defined scale
    qo, so = O.quant_act(O.bf16_to_f32(yk[rows]))
    assert np.array_equal(q.cpu().numpy()[rows], qo) and np.array_equal(s.cpu().numpy()[rows], so)


@pytest.mark.parametrize("m,k", [(300, 4096), (1, 512), (77, 2560)])
def test_gate_quant_matches_oracle(gpu, m, k):
    """The gate read as a strided view of a wider row (the QKV projection output), as the layers pass it."""
    note(f"gate_quant m={m} k={k}")
    rng = np.random.default_rng(m + k)
    a = O.f32_to_bf16(rng.standard_normal((m, k)).astype(np.float32) * 2)
    wide = O.f32_to_bf16(rng.standard_normal((m, 3 * k)).astype(np.float32) * 3)
    tw = gpu_bf16(wide)
    q, s, y = fused_kernels.gate_quant(gpu_bf16(a), tw[:, k:2 * k], return_gated=True)
    yk = bits_of(y)
    ref = O.gate_mul(a, wide[:, k:2 * k])
    assert ulps(yk, ref).max() <= 1.0001 and np.mean(yk == ref) >= 0.999
    qo, so = O.quant_act(O.bf16_to_f32(yk))
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)
    q2, s2 = fused_kernels.gate_quant(gpu_bf16(a), tw[:, k:2 * k])     # without the gated rows: same bits
    assert torch.equal(q2, q) and torch.equal(s2, s)


def _tables(n_pos, rot, theta=1e7):
    inv = 1.0 / (theta ** (np.arange(0, rot, 2, dtype=np.float32) / rot))
    ang = np.arange(n_pos, dtype=np.float32)[:, None] * inv[None, :]
    return O.f32_to_bf16(np.cos(ang)), O.f32_to_bf16(np.sin(ang))


@pytest.mark.parametrize("norm,rot", [(True, 64), (False, 64), (True, 0), (False, 256), (True, 256)])
def test_head_norm_rope_matches_oracle(gpu, norm, rot):
    """Rows laid out as the gated QKV projection: [q (16 heads) | gate (16) | k (4) | v (4)] of 256; q and
    k normed (zero-centred weights, offset 1) and rotated on their first rot dims, positions t % 100;
    gate and v columns untouched."""
    note(f"head_norm_rope norm={norm} rot={rot}")
    rng = np.random.default_rng(7 + rot + norm)
    T, d, hq, hk = 300, 256, 16, 4
    C = (2 * hq + 2 * hk) * d
    x = O.f32_to_bf16(rng.standard_normal((T, C)).astype(np.float32) * 2)
    wq = O.f32_to_bf16(rng.normal(0, 0.1, d).astype(np.float32))
    wk = O.f32_to_bf16(rng.normal(0, 0.1, d).astype(np.float32))
    cos, sin = _tables(128, rot) if rot else (None, None)
    tx = gpu_bf16(x)
    fused_kernels.head_norm_rope(tx, d, (0, hq), (2 * hq * d, hk), gpu_bf16(wq) if norm else None,
                                 gpu_bf16(wk) if norm else None, 1e-6, 1.0, rot,
                                 None if cos is None else gpu_bf16(cos), None if sin is None else gpu_bf16(sin),
                                 period=100)
    got = bits_of(tx).reshape(T, -1, d)
    xr = x.reshape(T, -1, d)
    pos = np.arange(T) % 100
    want = xr.copy()
    for sl, w in ((slice(0, hq), wq), (slice(2 * hq, 2 * hq + hk), wk)):
        seg = xr[:, sl]
        if norm:
            seg = O.head_rms_norm(seg, O.bf16_to_f32(w), 1e-6, 1.0)
        if rot:
            seg = O.rope_partial(seg, cos[pos][:, None, :], sin[pos][:, None, :], rot)
        want[:, sl] = seg
    untouched = np.r_[hq:2 * hq, 2 * hq + hk:2 * hq + 2 * hk]
    assert np.array_equal(got[:, untouched], xr[:, untouched]), "gate / v columns changed"
    heads = np.r_[0:hq, 2 * hq:2 * hq + hk]
    g, w = got[:, heads], want[:, heads]
    if not norm:
        assert np.array_equal(g, w), "RoPE alone must be bit-exact"
    else:
        tol = 2.0001 if rot else 1.0001
        assert ulps(g, w).max() <= tol, f"{ulps(g, w).max():.2f} ulp"
        assert np.mean(g == w) >= 0.99


def test_head_norm_rope_positions_tensor(gpu):
    """Positions given per row (a continuation after a prefix), k heads only (the last-only K / V rows)."""
    note("head_norm_rope with a positions tensor")
    rng = np.random.default_rng(11)
    T, d, hk = 64, 256, 4
    x = O.f32_to_bf16(rng.standard_normal((T, 2 * hk * d)).astype(np.float32))
    wk = O.f32_to_bf16(rng.normal(0, 0.1, d).astype(np.float32))
    cos, sin = _tables(400, 64)
    pos = (np.arange(T) + 300).astype(np.int32)
    tx = gpu_bf16(x)
    fused_kernels.head_norm_rope(tx, d, (0, 0), (0, hk), None, gpu_bf16(wk), 1e-6, 1.0, 64, gpu_bf16(cos),
                                 gpu_bf16(sin), pos=torch.from_numpy(pos).cuda())
    got = bits_of(tx).reshape(T, -1, d)
    xr = x.reshape(T, -1, d)
    want = O.rope_partial(O.head_rms_norm(xr[:, :hk], O.bf16_to_f32(wk), 1e-6, 1.0), cos[pos][:, None, :],
                          sin[pos][:, None, :], 64)
    assert np.array_equal(got[:, hk:], xr[:, hk:])
    assert ulps(got[:, :hk], want).max() <= 2.0001 and np.mean(got[:, :hk] == want) >= 0.99
