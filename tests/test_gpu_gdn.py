"""GDN kernels (mica_amd/csrc/gdn.hip) against the GDN oracle (oracle/gdn.py), through the C ABI.

Tolerances (floating point; stated per test):
  * conv + SiLU (+ l2norm): each bf16 output within one bf16 ulp of the oracle's float64 value
    rounded to bf16 (the kernel sums in fp32), and >= 99 % of them bit-equal;
  * chunked scan: the kernel rounds T, W, U, the state, v_new and the masked Q K^T to bf16 where they
    enter a matrix product (as the reference's kernels do), so outputs are compared in relative
    Frobenius norm per (sequence, head): <= 1e-2 for o and for the final state (measured: ~3e-3),
    against the float64 recurrence on the same bf16 inputs;
  * gated RMSNorm + quant: three chained bf16 roundings (normalised, weighted, gated), so y is within
    two bf16 ulps of the oracle (one ulp of difference in the fp32 rstd can cross two rounding
    boundaries) and >= 99 % bit-equal; q is exact given the kernel's y and within 1 of the oracle's.
Size-independent checks at the benchmark shape (8 x 2048 tokens, 16 key / 32 value heads): a scan
split at a chunk boundary and continued from the returned state is bit-identical to the unsplit scan;
one (sequence, head) pair is checked against the oracle.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import gdn as G
from oracle import w8a8 as O

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _f64(t):
    return t.detach().float().cpu().double().numpy()


def _rel(a, b):
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_causal_conv1d_empty_sequence_keeps_the_state(gpu):
    """T = 0: no output rows, and the final state is the initial one (zeros without one), as the
    scan's final state is for an empty input."""
    from mica_amd import gdn
    print("[case] conv T=0", file=sys.stderr, flush=True)
    B, C = 2, 256
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(C, 4, generator=g) * 0.5).to(torch.bfloat16).to(gpu)
    h0 = torch.randn(B, C, 3, generator=g).to(torch.bfloat16).to(gpu)
    x = torch.empty(B, 0, C, dtype=torch.bfloat16, device=gpu).transpose(1, 2)
    for init in (h0, None):
        stale = torch.full((B, C, 3), 7.0, dtype=torch.bfloat16, device=gpu)
        y, fin = gdn.causal_conv1d_fn(x, w, initial_states=init, return_final_states=True,
                                      final_states_out=stale, activation="silu")
        torch.cuda.synchronize()
        assert y.shape == (B, C, 0)
        assert torch.equal(fin, h0 if init is not None else torch.zeros_like(h0))


@pytest.mark.parametrize("B,T,C,n_norm,init,bias", [(2, 37, 1024, 4, True, True), (1, 5, 8192, 32, False, False),
                                                     (3, 64, 512, 0, True, False), (1, 2, 256, 2, True, True)])
def test_causal_conv1d_matches_oracle(gpu, B, T, C, n_norm, init, bias):
    from mica_amd import gdn
    g = torch.Generator().manual_seed(B * 1000 + T)
    x = (torch.randn(B, T, C, generator=g) * 2).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=g) * 0.5).to(torch.bfloat16)
    bs = (torch.randn(C, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    h0 = (torch.randn(B, C, 3, generator=g)).to(torch.bfloat16) if init else None
    xd = x.to(gpu).transpose(1, 2)  # channel-last [B, C, T] view, as the reference hands it over
    y, fin = gdn.causal_conv1d_fn(xd, w.to(gpu), None if bs is None else bs.to(gpu),
                                  initial_states=None if h0 is None else h0.to(gpu), return_final_states=True,
                                  activation="silu", l2norm_heads=n_norm)
    torch.cuda.synchronize()
    ref = G.causal_conv1d(_f64(x), _f64(w), None if bs is None else _f64(bs), None if h0 is None else _f64(h0))
    ref_bits = O.f32_to_bf16(ref.astype(np.float32))
    if n_norm:
        r = O.bf16_to_f32(ref_bits).astype(np.float64).reshape(B, T, C // 128, 128)
        r[:, :, :n_norm] = G.l2norm(r[:, :, :n_norm])
        ref_bits = O.f32_to_bf16(r.reshape(B, T, C).astype(np.float32))
    got = _bits(y.transpose(1, 2))
    diff = np.abs(O.bf16_to_f32(got).astype(np.float64) - O.bf16_to_f32(ref_bits))
    assert (diff <= O.bf16_ulp(ref_bits)).all(), diff.max()
    assert (got == ref_bits).mean() >= 0.99
    # final state: the last 3 inputs (history included when T < 3)
    full = np.concatenate([np.zeros((B, C, 3), np.uint16) if h0 is None else _bits(h0), _bits(x).transpose(0, 2, 1)], -1)
    assert (_bits(fin) == full[:, :, -3:]).all()


def _scan_inputs(seed, B, T, HK, HV, init):
    g = torch.Generator().manual_seed(seed)
    q = G.l2norm(torch.randn(B, T, HK, 128, generator=g).double().numpy())
    k = G.l2norm(torch.randn(B, T, HK, 128, generator=g).double().numpy())
    qb = torch.tensor(q, dtype=torch.bfloat16)
    kb = torch.tensor(k, dtype=torch.bfloat16)
    vb = torch.randn(B, T, HV, 128, generator=g).to(torch.bfloat16)
    a = torch.randn(B, T, HV, generator=g) * 2
    bb = torch.randn(B, T, HV, generator=g) * 2
    A_log = torch.rand(HV, generator=g) * 2 - 1
    dt_bias = torch.randn(HV, generator=g) * 0.5
    gg, beta = G.gdn_gate(a.numpy(), bb.numpy(), A_log.numpy(), dt_bias.numpy())
    gt = torch.tensor(gg, dtype=torch.float32)
    bt = torch.tensor(beta, dtype=torch.float32).to(torch.bfloat16)
    h0 = torch.randn(B, HV, 128, 128, generator=g) * 0.2 if init else None
    return qb, kb, vb, gt, bt, h0


@pytest.mark.parametrize("B,T,HK,HV,init", [(2, 200, 2, 4, True), (1, 64, 1, 2, False), (2, 1, 2, 2, True),
                                            (1, 130, 2, 4, False)])
def test_chunk_gated_delta_rule_matches_recurrence(gpu, B, T, HK, HV, init):
    from mica_amd import gdn
    qb, kb, vb, gt, bt, h0 = _scan_inputs(B * 7 + T, B, T, HK, HV, init)
    o, hT = gdn.chunk_gated_delta_rule(qb.to(gpu), kb.to(gpu), vb.to(gpu), gt.to(gpu), bt.to(gpu),
                                       initial_state=None if h0 is None else h0.to(gpu), output_final_state=True)
    torch.cuda.synchronize()
    ro, rS = G.gated_delta_rule(_f64(qb), _f64(kb), _f64(vb), _f64(gt), _f64(bt),
                                initial_state=None if h0 is None else _f64(h0))
    go, gS = _f64(o), _f64(hT)
    worst_o = max(_rel(go[b, :, h], ro[b, :, h]) for b in range(B) for h in range(HV))
    worst_s = max(_rel(gS[b, h], rS[b, h]) for b in range(B) for h in range(HV))
    print(f"relative error: o {worst_o:.2e}, final state {worst_s:.2e}")
    assert worst_o <= 1e-2 and worst_s <= 1e-2


def test_scan_with_l2norm_in_kernel_and_empty_input(gpu):
    from mica_amd import gdn
    qb, kb, vb, gt, bt, h0 = _scan_inputs(5, 1, 70, 1, 2, True)
    raw_q = (qb.float() * 3).to(torch.bfloat16)  # not normalised: the l2norm runs in front of the scan
    o, hT = gdn.chunk_gated_delta_rule(raw_q.to(gpu), kb.to(gpu), vb.to(gpu), gt.to(gpu), bt.to(gpu),
                                       initial_state=h0.to(gpu), output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)
    ro, rS = G.gated_delta_rule(G.l2norm(_f64(raw_q)), G.l2norm(_f64(kb)), _f64(vb), _f64(gt), _f64(bt),
                                initial_state=_f64(h0))
    assert _rel(_f64(o), ro) <= 1e-2 and _rel(_f64(hT), rS) <= 1e-2
    # T = 0: no output rows, the final state is the initial state
    o0, h0out = gdn.chunk_gated_delta_rule(qb[:, :0].to(gpu), kb[:, :0].to(gpu), vb[:, :0].to(gpu),
                                           gt[:, :0].to(gpu), bt[:, :0].to(gpu), initial_state=h0.to(gpu),
                                           output_final_state=True)
    torch.cuda.synchronize()
    assert o0.shape == (1, 0, 2, 128) and torch.equal(h0out.cpu(), h0)


def test_scan_dv_split_is_bit_identical(gpu):
    """With fewer (sequence, head) pairs than CUs the scan splits the value columns over 2 or 4
    workgroups per pair; every output element keeps its arithmetic, so a sequence scanned alone (4-way
    split), with three others (2-way) or with seven others (no split) gives the same bits."""
    from mica_amd import gdn
    B, T, HK, HV = 8, 200, 16, 32
    qb, kb, vb, gt, bt, h0 = _scan_inputs(17, B, T, HK, HV, True)
    q, k, v, g, beta, s0 = (t.to(gpu) for t in (qb, kb, vb, gt, bt, h0))
    o8, h8 = gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=s0, output_final_state=True)
    for n in (1, 4):
        o, hT = gdn.chunk_gated_delta_rule(q[:n], k[:n], v[:n], g[:n], beta[:n], initial_state=s0[:n],
                                           output_final_state=True)
        torch.cuda.synchronize()
        assert torch.equal(o, o8[:n]) and torch.equal(hT, h8[:n]), n


def test_scan_at_benchmark_shape_split_is_bit_identical(gpu):
    """8 sequences x 2048 tokens, 16 key / 32 value heads (the GDN layer of the 4B model at the prefill
    benchmark's shape).  Scanning tokens [0, 1024) then [1024, 2048) from the returned state gives the
    same bits as one scan; one (sequence, head) pair is checked against the float64 recurrence."""
    from mica_amd import gdn
    B, T, HK, HV = 8, 2048, 16, 32
    qb, kb, vb, gt, bt, _ = _scan_inputs(11, B, T, HK, HV, False)
    q, k, v, g, beta = (t.to(gpu) for t in (qb, kb, vb, gt, bt))
    o, hT = gdn.chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True)
    o1, h1 = gdn.chunk_gated_delta_rule(q[:, :1024], k[:, :1024], v[:, :1024], g[:, :1024], beta[:, :1024],
                                        output_final_state=True)
    o2, h2 = gdn.chunk_gated_delta_rule(q[:, 1024:], k[:, 1024:], v[:, 1024:], g[:, 1024:], beta[:, 1024:],
                                        initial_state=h1, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([o1, o2], 1), o) and torch.equal(h2, hT)
    assert torch.isfinite(o.float()).all()
    b, h = 5, 19
    ro, rS = G.gated_delta_rule(_f64(qb[b:b + 1, :, h // 2:h // 2 + 1]), _f64(kb[b:b + 1, :, h // 2:h // 2 + 1]),
                                _f64(vb[b:b + 1, :, h:h + 1]), _f64(gt[b:b + 1, :, h:h + 1]),
                                _f64(bt[b:b + 1, :, h:h + 1]))
    assert _rel(_f64(o[b, :, h]), ro[0, :, 0]) <= 1e-2
    assert _rel(_f64(hT[b, h]), rS[0, 0]) <= 1e-2


@pytest.mark.parametrize("M,N", [(37, 4096), (1, 512), (256, 8192)])
def test_gated_rmsnorm_quant_matches_oracle(gpu, M, N):
    from mica_amd import gdn
    g = torch.Generator().manual_seed(M + N)
    x = (torch.randn(M, N, generator=g) * 3).to(torch.bfloat16)
    z = (torch.randn(M, N, generator=g) * 2).to(torch.bfloat16)
    w = (torch.randn(128, generator=g) * 0.2 + 1).to(torch.bfloat16)
    q, s, y = gdn.gated_rmsnorm_quant(x.to(gpu), z.to(gpu), w.to(gpu), 1e-6, want_y=True)
    torch.cuda.synchronize()
    ref_y = G.gated_rmsnorm(_bits(x).reshape(M, N // 128, 128), _bits(z).reshape(M, N // 128, 128), _bits(w),
                            1e-6).reshape(M, N)
    got_y = _bits(y)
    ulps = np.abs(O.bf16_to_f32(got_y).astype(np.float64) - O.bf16_to_f32(ref_y)) / O.bf16_ulp(ref_y)
    print(f"max {ulps.max():.0f} ulp, {(got_y == ref_y).mean() * 100:.3f} % bit-equal")
    assert ulps.max() <= 2 and (got_y == ref_y).mean() >= 0.99
    # the quantiser is exact given the kernel's y
    rq, rs = O.quant_act(O.bf16_to_f32(got_y))
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    rq2, _ = O.quant_act(O.bf16_to_f32(ref_y))
    assert np.abs(q.cpu().numpy().astype(int) - rq2).max() <= 1


@pytest.mark.parametrize("M,HV", [(300, 32), (7, 4), (1, 1)])
def test_gdn_gate_matches_oracle(gpu, M, HV):
    """g = -exp(A_log) softplus(a + dt_bias) within 1e-6 relative of the float64 formula applied to the
    fp32 sum a + dt_bias (the reference adds in fp32, a.float() + self.dt_bias; below the threshold
    softplus ~ exp passes that sum's rounding on as a relative error of up to |x| 2^-24, so the oracle
    takes the same rounded sum), with fp32 exp and log1p a few ulps apart; values below 1e-30 compared
    absolutely.  beta = sigmoid(b) within one bf16 ulp of the float64 value rounded to bf16; a spans
    both sides of the softplus threshold 20."""
    from mica_amd import gdn
    g = torch.Generator().manual_seed(M * 31 + HV)
    a = (torch.randn(M, HV, generator=g) * 12).to(torch.bfloat16)
    b = (torch.randn(M, HV, generator=g) * 6).to(torch.bfloat16)
    A_log = torch.rand(HV, generator=g) * 4 - 2
    dt = torch.randn(HV, generator=g) * 2
    gg, beta = gdn.gdn_gate(a.to(gpu), b.to(gpu), A_log.to(gpu), dt.to(gpu))
    torch.cuda.synchronize()
    x32 = (a.float() + dt).double().numpy()  # the reference's fp32 sum
    rg, rb = G.gdn_gate(x32, _f64(b), A_log.double().numpy(), np.zeros(HV))
    assert gg.dtype == torch.float32 and beta.dtype == torch.bfloat16
    np.testing.assert_allclose(gg.cpu().double().numpy(), rg, rtol=1e-6, atol=1e-30)
    ref_b = O.f32_to_bf16(rb.astype(np.float32))
    assert (np.abs(O.bf16_to_f32(_bits(beta)).astype(np.float64) - O.bf16_to_f32(ref_b)) <= O.bf16_ulp(ref_b)).all()
    # strided rows (the a / b columns of a wider projection output) give the same values
    wide = torch.cat([a, b], 1).to(gpu)
    g2, b2 = gdn.gdn_gate(wide[:, :HV], wide[:, HV:], A_log.to(gpu), dt.to(gpu))
    assert torch.equal(g2, gg) and torch.equal(b2, beta)
