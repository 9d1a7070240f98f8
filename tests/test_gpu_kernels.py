"""Parity of the gfx950 kernels with the CPU oracle, through the drop-in surface and the C ABI.

Bar (from the hot path's contract): int8 activations, fp32 scales and int32 accumulators bit-exact;
bf16 outputs bit-exact where the reference's arithmetic is fully determined (quantizer, GEMM epilogue)
and within one bf16 ulp where it is not (the fp32 summation order inside RMSNorm, library exp in
SiLU); option probabilities within 1e-3 absolute.  Shapes are the benchmark configurations; the
largest ones are checked on a seeded sample of rows (rows of a GEMM are independent).
"""
import sys

import numpy as np
import pytest
import torch

from mica_amd import fused_kernels, int8_kernels, int8_runtime
from mica_amd.readout import LabelReadout
from oracle import w8a8 as O

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def to_gpu_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def bits_of(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def act_bits(rng, shape, outliers=8, scale=1.0):
    x = rng.standard_normal(shape).astype(np.float32) * scale
    if outliers:
        x[..., rng.permutation(shape[-1])[:outliers]] *= 20.0
    return O.f32_to_bf16(x)


def assert_within_one_ulp(got_bits, ref_bits, min_exact=0.999):
    g, r = O.bf16_to_f32(got_bits), O.bf16_to_f32(ref_bits)
    ulps = np.abs(g - r) / O.bf16_ulp(ref_bits)
    bad = np.flatnonzero(ulps > 1.0001)
    assert bad.size == 0, (f"{bad.size} of {ulps.size} elements differ by more than one bf16 ulp (max "
                           f"{ulps.max():.2f}); first: got {g.ravel()[bad[:5]]} want {r.ravel()[bad[:5]]}")
    assert np.mean(got_bits == ref_bits) >= min_exact, f"exact fraction {np.mean(got_bits == ref_bits):.6f}"


def assert_equal_diag(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    if got.dtype == np.float16:
        got, want = got.view(np.uint16), want.view(np.uint16)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    if bad.size:
        gv, wv = got.ravel()[bad[:6]], want.ravel()[bad[:6]]
        raise AssertionError(f"{what}: {bad.size} of {got.size} differ; at {bad[:6]} got {gv} want {wv}")


@pytest.fixture(autouse=True)
def _strict_and_clean(monkeypatch):
    monkeypatch.setattr(int8_kernels, "STRICT", True)
    yield
    torch.cuda.synchronize()


# ------------------------------------------------------------------------------ quantizer
def test_act_quant_known_answers(gpu, kat):
    for i, case in enumerate(kat["quant"]):
        note(f"act_quant KAT {i}")
        x = to_gpu_bf16(np.array(case["x_bf16"], np.uint16)[None, :])
        inv = torch.tensor(case["inv"], dtype=torch.float32, device=gpu) if "inv" in case else None
        for mode, key in (("even", "q_even"), ("away", "q_away")):
            q, s = int8_kernels.act_quant(x, inv, rounding=mode)
            assert q.cpu()[0].tolist() == case[key], (i, mode)
            assert s.cpu().numpy().view(np.uint32)[0] == case["s_bits"]


@pytest.mark.parametrize("m,k,smooth,rounding,dtype", [
    (512, 2560, False, "even", torch.bfloat16),      # config 0 activations
    (4096, 9728, False, "even", torch.bfloat16),     # the down projection's input
    (1500, 4096, False, "away", torch.bfloat16),
    (608, 9216, True, "even", torch.bfloat16),       # reference shape with SmoothQuant factors
    (200, 2560, False, "even", torch.float16),
    (48, 2560, True, "away", torch.float32),
    (3, 8, False, "even", torch.bfloat16),           # smallest K
    (7, 1000, False, "even", torch.bfloat16),        # K not a multiple of 512 (masked chunks)
    (333, 2560, True, "even", torch.bfloat16),       # smoothed, factors held in LDS
    (129, 1000, True, "away", torch.bfloat16),       # the same with masked chunks
    (64, 2048, True, "even", torch.float16),         # fp16 rows on the LDS-factor path
])
def test_act_quant_bit_exact(gpu, m, k, smooth, rounding, dtype):
    note(f"act_quant m={m} k={k} smooth={smooth} {rounding} {dtype}")
    rng = np.random.default_rng(m * 7 + k)
    xb = act_bits(rng, (m, k))
    xf = O.bf16_to_f32(xb)
    if dtype == torch.float16:
        xf = xf.astype(np.float16).astype(np.float32)
    x = torch.from_numpy(xf).to(dtype).cuda()
    inv = rng.uniform(0.2, 5.0, k).astype(np.float32) if smooth else None
    q, s = int8_kernels.act_quant(x, None if inv is None else torch.from_numpy(inv).cuda(), rounding=rounding)
    qo, so = O.quant_act(x.float().cpu().numpy(), inv, rounding)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


# ------------------------------------------------------------------------------ RMSNorm + quant
def test_rms_norm_known_answers(gpu, kat):
    for i, case in enumerate(kat["rms_norm"]):
        note(f"rms_norm KAT {i}")
        x = to_gpu_bf16(np.array(case["x_bf16"], np.uint16)[None, :])
        w = torch.tensor(case["w"], dtype=torch.float32, device=gpu)
        y = fused_kernels.rms_norm(x, w, case["eps"], offset=case["offset"])
        assert bits_of(y)[0].tolist() == case["y_bf16"], i


@pytest.mark.parametrize("T", [256, 4096, 32768])
@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_rmsnorm_quant_config1(gpu, T, offset):
    """Config 1: X bf16 [T, 2560] ~N(0,1) + 8 outlier channels x20, gamma ~N(1, 0.1) (offset 0: a plain
    gamma; offset 1: the same multiplier written as 1 + w), eps 1e-6."""
    note(f"rmsnorm_quant T={T} offset={offset}")
    rng = np.random.default_rng(T)
    K = 2560
    xb = act_bits(rng, (T, K))
    gamma = O.round_bf16(rng.normal(1.0, 0.1, K).astype(np.float32))
    w = gamma - np.float32(offset)
    wt = to_gpu_bf16(O.f32_to_bf16(w))
    x = to_gpu_bf16(xb)
    q, s, y = fused_kernels.rms_norm_quant(x, wt, 1e-6, offset=offset, return_normed=True)
    yk = bits_of(y)
    yo, _ = O.rms_norm(xb, O.bf16_to_f32(O.f32_to_bf16(w)), 1e-6, offset)
    # the normed row: within one bf16 ulp of the oracle (fp32 summation order), nearly always equal
    assert_within_one_ulp(yk, yo)
    # int8 and scales: bit-exact against the reference quantizer applied to the kernel's own row
    qo, so = O.quant_act(O.bf16_to_f32(yk))
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    # and wherever the normed row matches, the whole output matches the oracle end to end
    same = np.all(yk == yo, axis=1)
    qe, se = O.quant_act(O.bf16_to_f32(yo))
    assert np.array_equal(q.cpu().numpy()[same], qe[same])
    note(f"rmsnorm_quant T={T} offset={offset}: {same.mean():.5f} of rows equal the oracle's bf16 row, "
         f"{np.mean(yk == yo):.7f} of elements")
    # observed 0.988 (T = 256) to 0.991 of rows (rows whose fp32 sum of squares rounds the other way)
    assert same.mean() > 0.98


def test_rmsnorm_quant_residual_and_smoothing(gpu):
    note("rmsnorm_quant residual + inv_smooth")
    rng = np.random.default_rng(77)
    T, K = 333, 2560
    xb, rb = act_bits(rng, (T, K)), act_bits(rng, (T, K), outliers=0)
    w = O.round_bf16(rng.normal(0.0, 0.1, K).astype(np.float32))
    inv = rng.uniform(0.3, 3.0, K).astype(np.float32)
    q, s, y, v = fused_kernels.rms_norm_quant(to_gpu_bf16(xb), to_gpu_bf16(O.f32_to_bf16(w)), 1e-6,
                                              inv_smooth=torch.from_numpy(inv).cuda(), residual=to_gpu_bf16(rb),
                                              return_normed=True)
    yo, vo = O.rms_norm(xb, w, 1e-6, 1.0, rb)
    assert np.array_equal(bits_of(v), vo)  # the residual sum is exact bf16 arithmetic
    yk = bits_of(y)
    assert_within_one_ulp(yk, yo)
    qo, so = O.quant_act(O.bf16_to_f32(yk), inv)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("T,K,n", [(333, 2560, 3), (64, 1000, 3), (257, 9728, 3), (130, 2560, 4), (50, 512, 4)])
def test_rmsnorm_quant_multi_consumers(gpu, T, K, n):
    """One norm quantized for n consumers (one unsmoothed, the others with different SmoothQuant factors;
    rows of up to 2560 keep the factors in LDS, 4 consumers being its largest size): each output is
    bit-identical to the single-consumer launch, and to the reference quantizer applied to the kernel's
    normed row times that consumer's factors."""
    note(f"rmsnorm_quant_multi T={T} K={K} n={n}")
    rng = np.random.default_rng(T + K)
    xb, rb = act_bits(rng, (T, K)), act_bits(rng, (T, K), outliers=0)
    x, r = to_gpu_bf16(xb), to_gpu_bf16(rb)
    w = O.round_bf16(rng.normal(0.0, 0.1, K).astype(np.float32))
    wt = to_gpu_bf16(O.f32_to_bf16(w))
    invs = [None] + [rng.uniform(0.3, 3.0, K).astype(np.float32) for _ in range(n - 1)]
    tinvs = [None if v is None else torch.from_numpy(v).cuda() for v in invs]
    outs, v = fused_kernels.rms_norm_quant_multi(x, wt, 1e-6, tinvs, residual=r)
    _, _, y, v1 = fused_kernels.rms_norm_quant(x, wt, 1e-6, residual=r, return_normed=True)
    assert np.array_equal(bits_of(v), bits_of(v1))
    yk = bits_of(y)
    for i, ((q, s), inv, tinv) in enumerate(zip(outs, invs, tinvs)):
        q1, s1, _ = fused_kernels.rms_norm_quant(x, wt, 1e-6, inv_smooth=tinv, residual=r)
        assert np.array_equal(q.cpu().numpy(), q1.cpu().numpy()), f"consumer {i}"
        assert np.array_equal(s.cpu().numpy().view(np.uint32), s1.cpu().numpy().view(np.uint32)), f"consumer {i}"
        qo, so = O.quant_act(O.bf16_to_f32(yk), inv)
        assert np.array_equal(q.cpu().numpy(), qo), f"consumer {i} vs oracle"
        assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32)), f"consumer {i} vs oracle"


@pytest.mark.parametrize("T,n,res,rounding", [
    (4096, 3, True, "even"),    # q / k / v of a smoothed model at T = 4096: every row resident at once
    (4096, 2, False, "even"),   # gate / up
    (333, 3, True, "away"),
    (5, 1, True, "even"),       # fewer rows than waves in a workgroup
    (20000, 3, True, "even"),   # more rows than resident waves: the grid-stride kernel
])
def test_rmsnorm_quant_all_consumers_smoothed(gpu, T, n, res, rounding):
    """Every consumer with its own SmoothQuant factors (K = 2560): each output is bit-exact with the
    reference quantizer applied to the kernel's normed row times that consumer's factors; the normed
    row is within one bf16 ulp of the oracle's and the residual sum exact."""
    note(f"rmsnorm_quant all smoothed T={T} n={n} res={res} {rounding}")
    rng = np.random.default_rng(T * 3 + n)
    K = 2560
    xb, rb = act_bits(rng, (T, K)), act_bits(rng, (T, K), outliers=0)
    w = O.round_bf16(rng.normal(0.0, 0.1, K).astype(np.float32))
    wt = to_gpu_bf16(O.f32_to_bf16(w))
    invs = [rng.uniform(0.05, 20.0, K).astype(np.float32) for _ in range(n)]
    tinvs = [torch.from_numpy(v).cuda() for v in invs]
    outs = fused_kernels.rms_norm_quant_multi(to_gpu_bf16(xb), wt, 1e-6, tinvs,
                                              residual=to_gpu_bf16(rb) if res else None, rounding=rounding)
    if res:
        outs, v = outs
    got = fused_kernels.rms_norm_quant(to_gpu_bf16(xb), wt, 1e-6, residual=to_gpu_bf16(rb) if res else None,
                                       return_normed=True)
    y = got[2]
    yo, vo = O.rms_norm(xb, w, 1e-6, 1.0, rb if res else None)
    if res:
        assert np.array_equal(bits_of(v), vo)
        assert np.array_equal(bits_of(v), bits_of(got[3]))
    yk = bits_of(y)
    assert_within_one_ulp(yk, yo)
    for i, ((q, s), inv) in enumerate(zip(outs, invs)):
        qo, so = O.quant_act(O.bf16_to_f32(yk), inv, rounding)
        assert_equal_diag(q.cpu().numpy(), qo, f"consumer {i} q")
        assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32)), f"consumer {i} s"


def test_shared_norm_qlinears_match_separate_path(gpu):
    """SharedNormQLinears (one norm + quant launch for q/k/v-style consumers, then a GEMM each) gives the
    bits of the reference's call pattern: rms_norm, then each QLinear quantizing with its own factors."""
    note("shared-norm qlinears")
    rng = np.random.default_rng(5)
    T, K = 300, 2560
    h = to_gpu_bf16(act_bits(rng, (T, K)))
    nw = to_gpu_bf16(O.f32_to_bf16(O.round_bf16(rng.normal(0.0, 0.1, K).astype(np.float32))))
    lins = []
    for n, smooth in ((1024, True), (512, False), (512, True)):
        qw = torch.from_numpy(rng.integers(-127, 128, (n, K), dtype=np.int8)).cuda()
        sw = torch.from_numpy(rng.uniform(1e-3, 1e-2, n).astype(np.float32)).cuda()
        inv = torch.from_numpy(rng.uniform(0.5, 2.0, K).astype(np.float32)).cuda() if smooth else None
        lins.append(int8_runtime.QLinear.from_quantized(qw, sw, inv_smooth=inv))
    mod = int8_runtime.SharedNormQLinears(nw, 1e-6, lins)
    l0 = int8_kernels.STATS["launch"]
    outs = mod(h)
    torch.cuda.synchronize()
    assert int8_kernels.STATS["launch"] - l0 == 1 + len(lins)
    y = fused_kernels.rms_norm(h, nw, 1e-6)
    for lin, o in zip(lins, outs):
        assert np.array_equal(bits_of(o), bits_of(lin(y)))


def test_shared_norm_qlinears_share_equal_factors(gpu):
    """Linears with the same SmoothQuant factors (both None, or equal vectors held separately) share one
    int8 input and one GEMM over their stacked weights: 1 + (distinct factor sets) launches, each output
    bit-identical to its own QLinear on the normed rows, the members' weights row views of the stack."""
    note("shared-norm qlinears, shared inputs")
    rng = np.random.default_rng(6)
    T, K = 260, 2560
    h = to_gpu_bf16(act_bits(rng, (T, K)))
    nw = to_gpu_bf16(O.f32_to_bf16(O.round_bf16(rng.normal(0.0, 0.1, K).astype(np.float32))))
    inv = rng.uniform(0.5, 2.0, K).astype(np.float32)
    for plan, groups in ((((2048, None), (1024, None), (32, None), (32, None)), 1),   # the GDN in_proj shapes
                         (((512, "a"), (256, None), (512, "a"), (64, None)), 2)):   # equal factors, two copies
        lins = []
        for n, fac in plan:
            qw = torch.from_numpy(rng.integers(-127, 128, (n, K), dtype=np.int8)).cuda()
            sw = torch.from_numpy(rng.uniform(1e-3, 1e-2, n).astype(np.float32)).cuda()
            lins.append(int8_runtime.QLinear.from_quantized(
                qw, sw, inv_smooth=None if fac is None else torch.from_numpy(inv.copy()).cuda()))
        mod = int8_runtime.SharedNormQLinears(nw, 1e-6, lins)
        assert len(mod.groups) == groups
        l0 = int8_kernels.STATS["launch"]
        outs = mod(h)
        torch.cuda.synchronize()
        assert int8_kernels.STATS["launch"] - l0 == 1 + groups
        y = fused_kernels.rms_norm(h, nw, 1e-6)
        for lin, o, (n, _) in zip(lins, outs, plan):
            assert o.shape == (T, n)
            assert np.array_equal(bits_of(o), bits_of(lin(y)))
        for gi, grp in enumerate(mod.groups):
            if len(grp) > 1:
                base = mod._stacked[gi][0].untyped_storage().data_ptr()
                assert all(lins[i].qweight.untyped_storage().data_ptr() == base for i in grp)


def test_rms_norm_op_matches_reference_surface(gpu):
    """fused_kernels.rms_norm(x, w, eps, residual) -> y / (y, summed), the reference's signature."""
    note("rms_norm op")
    rng = np.random.default_rng(5)
    xb, rb = act_bits(rng, (64, 4096)), act_bits(rng, (64, 4096))
    w = O.round_bf16(rng.normal(0, 0.1, 4096).astype(np.float32))
    wt = to_gpu_bf16(O.f32_to_bf16(w))
    y = fused_kernels.rms_norm(to_gpu_bf16(xb), wt, 1e-6)
    assert_within_one_ulp(bits_of(y), O.rms_norm(xb, w, 1e-6)[0])
    y2, summed = fused_kernels.rms_norm(to_gpu_bf16(xb), wt, 1e-6, to_gpu_bf16(rb))
    yo, vo = O.rms_norm(xb, w, 1e-6, 1.0, rb)
    assert np.array_equal(bits_of(summed), vo)
    assert_within_one_ulp(bits_of(y2), yo)


# ------------------------------------------------------------------------------ GEMM
def test_gemm_known_answers(gpu, kat):
    for i, case in enumerate(kat["gemm"]):
        note(f"gemm KAT {i}")
        A = torch.tensor(case["A"], dtype=torch.int8, device=gpu)
        B = torch.tensor(case["B"], dtype=torch.int8, device=gpu)
        acc = int8_kernels.mm_i8_int32(A, B)
        assert acc.cpu().tolist() == case["acc"]
        sa = torch.tensor(case["sa"], dtype=torch.float32, device=gpu)
        sb = torch.tensor(case["sb"], dtype=torch.float32, device=gpu)
        bias = None if case["bias"] is None else torch.tensor(case["bias"], dtype=torch.float32, device=gpu)
        y = int8_kernels.mm_i8(A, sa, B, sb, bias)
        assert bits_of(y).tolist() == case["y_bf16"]


def _rand_gemm(rng, m, n, k):
    A = rng.integers(-127, 128, (m, k), dtype=np.int8)
    B = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    return A, B, sa, sb


@pytest.mark.parametrize("m,n,k", [
    (512, 9728, 2560),     # config 0
    (300, 1000, 2560),     # ragged M and N
    (256, 2560, 9728),     # down projection K
    (96, 2560, 4096),      # o_proj K
    (1, 32, 2560),         # single row, the reference's N=32 projection
    (17, 300, 2576),       # K not a multiple of the 128-byte slab
    (258, 514, 16),        # K of one chunk
    (130, 2704, 2576),     # 11 tiles as 128 x 128 quarters, cut by both the M and the N edge
    (130, 2704, 2560),     # the same quarters with K a multiple of 256 (the 16x16x64 kernel)
    (70, 1002, 512),       # N not a multiple of 4: element stores after the staged epilogue
    (64, 260, 256),        # one pair of 128-byte slabs; N a multiple of 4 but not of 8
])
def test_gemm_int32_and_epilogue_bit_exact(gpu, m, n, k):
    note(f"gemm m={m} n={n} k={k}")
    rng = np.random.default_rng(m + n + k)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    acc = int8_kernels.mm_i8_int32(tA, tB).cpu().numpy()
    ref = O.int_gemm(A, B)
    assert_equal_diag(acc, ref, "int32 accumulators")
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    tsa, tsb, tbias = (torch.from_numpy(v).cuda() for v in (sa, sb, bias))
    y = int8_kernels.mm_i8(tA, tsa, tB, tsb)
    assert_equal_diag(bits_of(y), O.epilogue(ref, sa, sb), "bf16 epilogue")
    yb = int8_kernels.mm_i8(tA, tsa, tB, tsb, tbias)
    assert np.array_equal(bits_of(yb), O.epilogue(ref, sa, sb, bias))
    y32 = int8_kernels.mm_i8(tA, tsa, tB, tsb, tbias, out_dtype=torch.float32)
    assert np.array_equal(y32.cpu().numpy().view(np.uint32), O.epilogue(ref, sa, sb, bias, "fp32").view(np.uint32))
    y16 = int8_kernels.mm_i8(tA, tsa, tB, tsb, out_dtype=torch.float16)
    assert_equal_diag(y16.cpu().numpy(), O.epilogue(ref, sa, sb, None, "fp16"), "fp16 epilogue")


def test_gemm_extreme_accumulators(gpu):
    """|acc| up to K * 127^2 = 1.57e8 at K = 9728 (above 2^24: the int32 -> fp32 conversion rounds)."""
    note("gemm extremes")
    m, n, k = 64, 256, 9728
    A = np.full((m, k), -127, np.int8)
    A[1::2] = 127
    B = np.full((n, k), -127, np.int8)
    B[::3, ::2] = 127
    acc = int8_kernels.mm_i8_int32(torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()).cpu().numpy()
    assert np.array_equal(acc, O.int_gemm(A, B))
    assert np.abs(acc).max() == k * 127 * 127


@pytest.mark.parametrize("m", [1, 100, 128, 200, 300, 700])
def test_gemm_silu_m_halves(gpu, m):
    """The fused gate+up SiLU epilogue at N = 3072 runs as one round of 128 x 128 tiles (one gate / up
    group each; rows past M in the last tile row), within one bf16 ulp of the oracle; with 32768 more
    weight rows the same columns come from whole tiles and 128 x 256 halves along M (a lower half wholly
    past M skipped, one cut by it, or both full), with the same bits."""
    note(f"gemm silu m-halves m={m}")
    rng = np.random.default_rng(m + 5)
    n, k = 3072, 2560
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    grp = B.reshape(n // 128, 2, 64, k)
    sgr = sb.reshape(n // 128, 2, 64)
    gv = O.epilogue(O.int_gemm(A, grp[:, 0].reshape(n // 2, k)), sa, sgr[:, 0].reshape(n // 2))
    uv = O.epilogue(O.int_gemm(A, grp[:, 1].reshape(n // 2, k)), sa, sgr[:, 1].reshape(n // 2))
    y = int8_kernels.mm_i8(*(torch.from_numpy(v).cuda() for v in (A, sa, B, sb)), epilogue="silu_mul")
    assert_within_one_ulp(bits_of(y), O.silu_mul(gv, uv))
    # here every M runs as one round of 128 x 128 tiles of one gate / up group each; with 32768 more
    # weight rows (more 128 x 128 tiles than CUs: whole tiles, then M-halves or whole tiles for the tail)
    # the same columns come out with the same bits: rows and column groups are independent
    B2 = np.concatenate([B, rng.integers(-127, 128, (32768, k), dtype=np.int8)])
    sb2 = np.concatenate([sb, rng.uniform(1e-3, 1e-2, 32768).astype(np.float32)])
    y2 = int8_kernels.mm_i8(*(torch.from_numpy(v).cuda() for v in (A, sa, B2, sb2)), epilogue="silu_mul")
    assert np.array_equal(bits_of(y2)[:, : n // 2], bits_of(y)), "128 x 128 SiLU tiles differ from the other schedules"


def test_gemm_requant_output(gpu):
    """mm_i8(..., requant=True): the per-token int8 quantization of the GEMM's output, bit-exact with the
    oracle's quant_act of that output (the gate+up SiLU product h feeding the down projection, and a
    plain bf16 output)."""
    note("gemm requant")
    rng = np.random.default_rng(21)
    m, n, k = 300, 1024, 2560
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    tA, tB, tsa, tsb = (torch.from_numpy(v).cuda() for v in (A, B, sa, sb))
    for epi in ("silu_mul", "none"):
        out = int8_kernels.mm_i8(tA, tsa, tB, tsb, epilogue=epi)
        q, s = int8_kernels.mm_i8(tA, tsa, tB, tsb, epilogue=epi, requant=True)
        qo, so = O.quant_act(O.bf16_to_f32(bits_of(out)))
        assert np.array_equal(q.cpu().numpy(), qo), epi
        assert np.array_equal(s.cpu().numpy(), so), epi


@pytest.mark.parametrize("m,n,k", [(700, 2560, 9728), (130, 1004, 512)])
def test_gemm_residual_epilogue(gpu, m, n, k):
    note(f"gemm residual m={m} n={n} k={k}")
    rng = np.random.default_rng(3 + m)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    res = act_bits(rng, (m, n), outliers=0)
    y = int8_kernels.mm_i8(*(torch.from_numpy(v).cuda() for v in (A, sa, B, sb)), residual=to_gpu_bf16(res))
    d = O.epilogue(O.int_gemm(A, B), sa, sb)
    ref = O.f32_to_bf16(O.bf16_to_f32(d) + O.bf16_to_f32(res))
    assert np.array_equal(bits_of(y), ref)


@pytest.mark.parametrize("m,n,k,epi", [
    (4096, 2560, 4096, "residual"),  # the O projection at T = 4096: 160 whole tiles -> 256 tiles of 256 x 160
    (4096, 2560, 9728, "bias"),      # the down projection's shape
    (3900, 2504, 2560, "residual"),  # both edges ragged; the last tile's upper half 24 columns wide
    (3900, 2500, 512, "fp16"),       # N not a multiple of 8: element stores
    (4096, 2504, 1024, "fp16"),      # fp16 rows in 16-byte units: the AGPR kernel's 4 x 1 wave grid
])
def test_gemm_narrow_tiles_bit_exact(gpu, m, n, k, epi):
    """One partial round of whole tiles (more than half the CUs busy) runs as 256 x 160 tiles when those
    still fit one round.  Bit-exact with the oracle, int32 accumulators included."""
    note(f"gemm narrow m={m} n={n} k={k} epi={epi}")
    rng = np.random.default_rng(m * 7 + n + k)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    tA, tB, tsa, tsb = (torch.from_numpy(v).cuda() for v in (A, B, sa, sb))
    acc = O.int_gemm(A, B)
    if epi == "residual":
        res = act_bits(rng, (m, n), outliers=0)
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, residual=to_gpu_bf16(res))
        ref = O.f32_to_bf16(O.bf16_to_f32(O.epilogue(acc, sa, sb)) + O.bf16_to_f32(res))
        assert_equal_diag(bits_of(y), ref, "bf16 + residual")
    elif epi == "bias":
        bias = rng.uniform(-1, 1, n).astype(np.float32)
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, torch.from_numpy(bias).cuda())
        assert_equal_diag(bits_of(y), O.epilogue(acc, sa, sb, bias), "bf16 + bias")
    else:
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, out_dtype=torch.float16)
        assert_equal_diag(y.cpu().numpy(), O.epilogue(acc, sa, sb, None, "fp16"), "fp16")


@pytest.mark.parametrize("m,n,k,epi", [
    (512, 9728, 2560, "none"),       # config 0: 76 whole tiles -> one round of 244 tiles of 128 x 160
    (500, 9696, 2560, "residual"),   # both edges ragged: the last row tile 116 rows, the last column tile 96 wide
    (768, 6144, 1024, "bias"),       # 72 tiles -> 234 tiles of 128 x 160
    (640, 6400, 512, "fp16"),        # the shortest K of the AGPR kernels, fp16 output
])
def test_gemm_small_tiles_bit_exact(gpu, m, n, k, epi):
    """Fewer whole 256 x 256 tiles than CUs, too many for four quarters each to fit one round: one round
    of 128 x 160 tiles.  Bit-exact with the oracle on every output."""
    note(f"gemm small tiles m={m} n={n} k={k} epi={epi}")
    rng = np.random.default_rng(m * 3 + n + k)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    tA, tB, tsa, tsb = (torch.from_numpy(v).cuda() for v in (A, B, sa, sb))
    acc = O.int_gemm(A, B)
    if epi == "residual":
        res = act_bits(rng, (m, n), outliers=0)
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, residual=to_gpu_bf16(res))
        ref = O.f32_to_bf16(O.bf16_to_f32(O.epilogue(acc, sa, sb)) + O.bf16_to_f32(res))
        assert_equal_diag(bits_of(y), ref, "bf16 + residual")
    elif epi == "bias":
        bias = rng.uniform(-1, 1, n).astype(np.float32)
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, torch.from_numpy(bias).cuda())
        assert_equal_diag(bits_of(y), O.epilogue(acc, sa, sb, bias), "bf16 + bias")
    elif epi == "fp16":
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, out_dtype=torch.float16)
        assert_equal_diag(y.cpu().numpy(), O.epilogue(acc, sa, sb, None, "fp16"), "fp16")
    else:
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb)
        assert_equal_diag(bits_of(y), O.epilogue(acc, sa, sb), "bf16")


def test_gemm_headline_full_size(gpu):
    """The benchmarked GEMM itself, M=4096 K=2560 N=9728 (every tile, including the partial last round
    of tiles), bit-exact: int32 accumulators and the bf16 output.  Then a size-independent property
    of the epilogue at the same size: scaling sa by 2^j scales every finite output by exactly 2^j."""
    note("gemm headline 4096x9728x2560")
    m, n, k = 4096, 9728, 2560
    rng = np.random.default_rng(4096)
    xb = act_bits(rng, (m, k))
    A, sa = O.quant_act(O.bf16_to_f32(xb))
    B = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    tA, tB, tsa, tsb = (torch.from_numpy(v).cuda() for v in (A, B, sa, sb))
    ref = O.int_gemm(A, B)
    assert_equal_diag(int8_kernels.mm_i8_int32(tA, tB).cpu().numpy(), ref, "int32 accumulators")
    y = bits_of(int8_kernels.mm_i8(tA, tsa, tB, tsb))
    assert_equal_diag(y, O.epilogue(ref, sa, sb), "bf16 output")
    pow2 = np.float32(2.0) ** rng.integers(-3, 4, m).astype(np.float32)
    y2 = bits_of(int8_kernels.mm_i8(tA, torch.from_numpy(sa * pow2).cuda(), tB, tsb))
    want = O.f32_to_bf16(O.bf16_to_f32(y) * pow2[:, None])
    assert_equal_diag(y2, want, "epilogue linearity in sa")


@pytest.mark.parametrize("m,n,k,epi", [
    (4096, 4352, 8192, "none"),      # 272 tiles: 256 whole, then 16 as 128 x 128 quarters (M > 256)
    (700, 2560, 9728, "residual"),   # 96 tiles of 128 x 160 leave room for 2 parts only: quarters
    (300, 3072, 8192, "silu_mul"),   # 36 tiles of 128 x 256 in 3 parts along K, then the SiLU epilogue
    (200, 2560, 8256, "none"),       # int32: 256 x 256 stream-K split, ranges straddle tiles; bf16: quarters
    (256, 2560, 9728, "none"),       # 32 tiles of 128 x 160 in 3 parts (the int32 output: stream-K split)
    (512, 2560, 4096, "none"),       # K below both split thresholds: quarters, workspace unused
])
def test_gemm_split_schedule_bit_exact(gpu, m, n, k, epi):
    """split=True (a workspace: remainder tiles split along K where that serves best, int32 partial sums
    through the workspace) gives the same bits as the oracle, twice in a row (the arrival counters must
    come back to zero)."""
    note(f"gemm split m={m} n={n} k={k} epi={epi}")
    rng = np.random.default_rng(m + n + k + 1)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    tA, tB, tsa, tsb = (torch.from_numpy(v).cuda() for v in (A, B, sa, sb))
    acc = O.int_gemm(A, B)
    for rep in range(2):
        assert_equal_diag(int8_kernels.mm_i8_int32(tA, tB, split=True).cpu().numpy(), acc, f"int32 (call {rep})")
    if epi == "silu_mul":
        n2 = n // 2
        grp = B.reshape(n // 128, 2, 64, k)
        sgr = sb.reshape(n // 128, 2, 64)
        gv = O.epilogue(O.int_gemm(A, grp[:, 0].reshape(n2, k)), sa, sgr[:, 0].reshape(n2))
        uv = O.epilogue(O.int_gemm(A, grp[:, 1].reshape(n2, k)), sa, sgr[:, 1].reshape(n2))
        ref = O.silu_mul(gv, uv)
        for rep in range(2):
            assert_within_one_ulp(bits_of(int8_kernels.mm_i8(tA, tsa, tB, tsb, epilogue="silu_mul", split=True)), ref)
        return
    res = act_bits(rng, (m, n), outliers=0) if epi == "residual" else None
    ref = O.epilogue(acc, sa, sb)
    if res is not None:
        ref = O.f32_to_bf16(O.bf16_to_f32(ref) + O.bf16_to_f32(res))
    for rep in range(2):
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, residual=None if res is None else to_gpu_bf16(res), split=True)
        assert_equal_diag(bits_of(y), ref, f"bf16 (call {rep})")


@pytest.mark.parametrize("m,n,k,epi", [
    (128, 2560, 9728, "residual"),   # one short request's down projection: 16 tiles of 128 x 160, 3 parts
    (128, 4096, 8192, "silu_mul"),   # SiLU epilogue: 16 tiles of 128 x 256, 3 parts of 21 or 22 slabs
    (77, 6144, 8192, "none"),        # ragged M (51 empty rows in every tile), 39 tiles, 3 parts
    (512, 2560, 9728, "bias_fp16"),  # fp16 output with a bias, 64 tiles, 3 parts
    (64, 2560, 16384, "none"),       # the most parts: 128 slabs in 6 parts, 16 tiles
    (256, 2560, 8192, "bias_residual"),  # bias and residual together (bf16), 32 tiles, 3 parts
])
def test_gemm_small_m_split_bit_exact(gpu, m, n, k, epi):
    """Few 128-row tiles and a long K, with a workspace: every tile is split along K over several
    workgroups whose int32 partial sums the tile's last part adds.  Integer sums are exact in any order,
    so the output equals the unsplit schedule's bit for bit and the oracle's (the SiLU within the
    one-ulp bound of its own test), on two calls in a row (the arrival counts come back to zero)."""
    note(f"gemm small-M split m={m} n={n} k={k} epi={epi}")
    rng = np.random.default_rng(m + n + k + 7)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    tA, tB, tsa, tsb = (torch.from_numpy(v).cuda() for v in (A, B, sa, sb))
    if epi == "silu_mul":
        n2 = n // 2
        grp = B.reshape(n // 128, 2, 64, k)
        sgr = sb.reshape(n // 128, 2, 64)
        gv = O.epilogue(O.int_gemm(A, grp[:, 0].reshape(n2, k)), sa, sgr[:, 0].reshape(n2))
        uv = O.epilogue(O.int_gemm(A, grp[:, 1].reshape(n2, k)), sa, sgr[:, 1].reshape(n2))
        plain = bits_of(int8_kernels.mm_i8(tA, tsa, tB, tsb, epilogue="silu_mul"))
        assert_within_one_ulp(plain, O.silu_mul(gv, uv))
        for rep in range(2):
            got = bits_of(int8_kernels.mm_i8(tA, tsa, tB, tsb, epilogue="silu_mul", split=True))
            assert np.array_equal(got, plain), f"split SiLU output differs from the unsplit one (call {rep})"
        return
    acc = O.int_gemm(A, B)
    kw, res, bias = {}, None, None
    if epi == "residual":
        res = act_bits(rng, (m, n), outliers=0)
        kw["residual"] = to_gpu_bf16(res)
        ref = O.f32_to_bf16(O.bf16_to_f32(O.epilogue(acc, sa, sb)) + O.bf16_to_f32(res))
    elif epi == "bias_fp16":
        bias = rng.uniform(-1, 1, n).astype(np.float32)
        kw.update(bias=torch.from_numpy(bias).cuda(), out_dtype=torch.float16)
        ref = O.epilogue(acc, sa, sb, bias, "fp16")
    elif epi == "bias_residual":
        bias = rng.uniform(-1, 1, n).astype(np.float32)
        res = act_bits(rng, (m, n), outliers=0)
        kw.update(bias=torch.from_numpy(bias).cuda(), residual=to_gpu_bf16(res))
        ref = O.f32_to_bf16(O.bf16_to_f32(O.epilogue(acc, sa, sb, bias)) + O.bf16_to_f32(res))
    else:
        ref = O.epilogue(acc, sa, sb)

    def out(**extra):
        y = int8_kernels.mm_i8(tA, tsa, tB, tsb, kw.get("bias"), kw.get("out_dtype", torch.bfloat16),
                               residual=kw.get("residual"), **extra)
        return y.cpu().numpy() if y.dtype == torch.float16 else bits_of(y)

    plain = out()
    assert_equal_diag(plain, ref, "unsplit")
    for rep in range(2):
        got = out(split=True)
        assert_equal_diag(got, ref, f"split (call {rep})")
        assert np.array_equal(got.view(np.uint16), plain.view(np.uint16)), f"split != unsplit (call {rep})"


@pytest.mark.parametrize("m,n,k", [(32768, 6144, 2560), (32768, 2560, 4096)])
def test_gemm_config3_long_context_sampled_rows(gpu, m, n, k):
    """Config 3 (T = 32768 packed prefill): QKV 2560 -> 6144 and O 4096 -> 2560, checked exactly on a
    seeded sample of rows spread over all M tiles."""
    note(f"gemm config3 m={m} n={n} k={k}")
    rng = np.random.default_rng(m + n)
    A, B, sa, sb = _rand_gemm(rng, m, n, k)
    y = int8_kernels.mm_i8(*(torch.from_numpy(v).cuda() for v in (A, sa, B, sb)))
    rows = np.unique(np.concatenate([rng.choice(m, 384, replace=False), [0, 255, 256, m - 1]]))
    ref = O.epilogue(O.int_gemm(A[rows], B), sa[rows], sb)
    assert np.array_equal(bits_of(y[torch.from_numpy(rows).cuda()]), ref)


# ------------------------------------------------------------------------------ QLinear / MLP
def test_qlinear_config0_end_to_end(gpu):
    """Config 0: X bf16 [512, 2560] (8 outlier channels x20) -> per-token int8 (half-even) -> int32 GEMM
    with W int8 [9728, 2560], sw ~U(1e-3, 1e-2) -> bf16; 2 launches, bit-exact."""
    note("qlinear config0")
    rng = np.random.default_rng(0)
    xb = act_bits(rng, (512, 2560))
    qw = rng.integers(-127, 128, (9728, 2560), dtype=np.int8)
    sw = rng.uniform(1e-3, 1e-2, 9728).astype(np.float32)
    lin = int8_runtime.QLinear.from_quantized(torch.from_numpy(qw).cuda(), torch.from_numpy(sw).cuda())
    l0 = int8_kernels.STATS["launch"]
    y = lin(to_gpu_bf16(xb))
    torch.cuda.synchronize()
    assert int8_kernels.STATS["launch"] - l0 == 2
    assert np.array_equal(bits_of(y), O.qlinear(xb, qw, sw))
    # rows_forward: one quantization, a GEMM per row range (the GDN qkv split)
    outs = lin.rows_forward(to_gpu_bf16(xb[:64]), [(0, 2048), (2048, 4096), (4096, 9728)])
    ref = O.qlinear(xb[:64], qw, sw)
    assert np.array_equal(np.concatenate([bits_of(o) for o in outs], 1), ref)


def test_smoothed_qlinear_from_bf16_linear_on_device(gpu):
    """A QLinear converted on the GPU from a random bf16 nn.Linear with SmoothQuant factors from synthetic
    activation absmax (int8_runtime.py:108-127, int8_quant.py:54-61, 80-85): its int8 weights, scales and
    inverse factors equal the oracle's weight quantizer on the smoothed fp32 weight, bit for bit, and
    its forward equals oracle.qlinear with those buffers (quantize with inv_smooth, exact GEMM, epilogue
    with bias)."""
    note("smoothed qlinear convert")
    torch.manual_seed(12)
    N, K = 1024, 2560
    lin = torch.nn.Linear(K, N, bias=True).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.mul_(20.0)
    rng = np.random.default_rng(12)
    amax = rng.uniform(0.05, 4.0, K).astype(np.float32)
    amax[::61] *= 25.0
    smooth = int8_runtime.smooth_factors(torch.from_numpy(amax), lin.weight.detach())     # on the CPU, once
    q = int8_runtime.QLinear(lin.cuda(), smooth)
    torch.cuda.synchronize()
    s = smooth.numpy()
    wf = lin.weight.detach().float().cpu().numpy() * s[None, :]
    qo, so = O.quant_weight(wf)
    inv = (np.float32(1) / s).astype(np.float32)
    assert_equal_diag(q.qweight.cpu().numpy(), qo, "qweight")
    assert_equal_diag(q.wscale.cpu().numpy().view(np.uint32), so.view(np.uint32), "wscale")
    assert_equal_diag(q.inv_smooth.cpu().numpy().view(np.uint32), inv.view(np.uint32), "inv_smooth")
    x = rng.standard_normal((300, K)).astype(np.float32) * (amax / 3)[None, :]
    xb = O.f32_to_bf16(x)
    bias = lin.bias.detach().float().cpu().numpy()
    y = q(to_gpu_bf16(xb))
    assert_equal_diag(bits_of(y), O.qlinear(xb, qo, so, bias=bias, inv_smooth=inv), "forward")


def test_convert_body_on_device(gpu, tmp_path):
    """int8_runtime.convert over a small body on the GPU with statistics read from a packed s.pt-layout
    file: every target linear becomes a QLinear; smoothed exactly where the file has its absmax; each
    one's forward equals the oracle's on its own buffers."""
    note("convert body")
    from torch import nn
    torch.manual_seed(3)
    H = 256
    body = nn.Module()
    body.layers = nn.ModuleList()
    for i in range(2):
        layer = nn.Module()
        layer.mlp = nn.Module()
        layer.mlp.gate_proj, layer.mlp.up_proj = nn.Linear(H, 512), nn.Linear(H, 512)
        layer.mlp.down_proj = nn.Linear(512, H, bias=False)
        body.layers.append(layer)
    body = body.to(torch.bfloat16).cuda()
    names = [n for n, *_ in int8_runtime.target_linears(body)]
    rng = np.random.default_rng(3)
    have = names[::2]
    lens = [512 if n.endswith("down_proj") else H for n in have]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    torch.save({"h": torch.tensor([int8_runtime.name_key(n) for n in have], dtype=torch.int64),
                "o": torch.from_numpy(offs), "v": torch.from_numpy(rng.uniform(0.1, 20, offs[-1]).astype(np.float32))},
               tmp_path / "s.pt")
    stats = int8_runtime.load_stats(tmp_path / "s.pt")
    assert int8_runtime.convert(body, stats) == (len(names), len(have))
    for name, _, _, _ in [(n, None, None, None) for n in names]:
        mod = body
        for part in name.split("."):
            mod = mod[int(part)] if part.isdigit() else getattr(mod, part)
        assert isinstance(mod, int8_runtime.QLinear) and (mod.inv_smooth is not None) == (name in have), name
        x = O.f32_to_bf16(rng.standard_normal((40, mod.in_features)).astype(np.float32) * 3)
        inv = None if mod.inv_smooth is None else mod.inv_smooth.cpu().numpy()
        bias = None if mod.bias is None else mod.bias.cpu().numpy()
        ref = O.qlinear(x, mod.qweight.cpu().numpy(), mod.wscale.cpu().numpy(), bias=bias, inv_smooth=inv)
        assert_equal_diag(bits_of(mod(to_gpu_bf16(x))), ref, name)


def test_qlinear_reference_selftest(gpu):
    """The reference's own acceptance criterion (int8_runtime.selftest) on its shipped shapes."""
    note("reference selftest")
    shapes = [(32, 2560, False), (1024, 2560, True), (2048, 2560, False), (4096, 2560, False),
              (8192, 2560, False), (9216, 2560, False), (2560, 4096, False), (2560, 9216, False)]
    out = int8_runtime.selftest(shapes, "cuda")
    assert out["ok"], out


def test_fused_gate_up_silu_epilogue(gpu):
    note("gate_up silu epilogue")
    rng = np.random.default_rng(11)
    m, inter, k = 1000, 1536, 2560
    xb = act_bits(rng, (m, k))
    qg, qu = (rng.integers(-127, 128, (inter, k), dtype=np.int8) for _ in range(2))
    sg, su = (rng.uniform(1e-3, 1e-2, inter).astype(np.float32) for _ in range(2))
    q, s = O.quant_act(O.bf16_to_f32(xb))
    qp, sp = int8_runtime.pack_gate_up(*(torch.from_numpy(v) for v in (qg, sg, qu, su)))
    h = int8_kernels.mm_i8(torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), qp.cuda(), sp.cuda(),
                           epilogue="silu_mul")
    g = O.epilogue(O.int_gemm(q, qg), s, sg)
    u = O.epilogue(O.int_gemm(q, qu), s, su)
    assert_within_one_ulp(bits_of(h), O.silu_mul(g, u))


def test_gated_mlp_config2(gpu):
    """Config 2 at T = 4096: fused gate+up (N = 2 x 9728) with the SiLU epilogue, requantization, down
    GEMM (K = 9728) with the residual add.  Each stage is checked against the oracle applied to the
    kernel's own input of that stage, on a seeded sample of rows."""
    note("gated mlp config2")
    rng = np.random.default_rng(2)
    T, H, I = 4096, 2560, 9728
    hb = act_bits(rng, (T, H))
    gamma = O.round_bf16(rng.normal(1.0, 0.1, H).astype(np.float32))
    mk = lambda n, k: (rng.integers(-127, 128, (n, k), dtype=np.int8), rng.uniform(1e-3, 1e-2, n).astype(np.float32))  # noqa: E731
    (qg, sg), (qu, su), (qd, sd) = mk(I, H), mk(I, H), mk(H, I)
    gate = int8_runtime.QLinear.from_quantized(torch.from_numpy(qg).cuda(), torch.from_numpy(sg).cuda())
    up = int8_runtime.QLinear.from_quantized(torch.from_numpy(qu).cuda(), torch.from_numpy(su).cuda())
    down = int8_runtime.QLinear.from_quantized(torch.from_numpy(qd).cuda(), torch.from_numpy(sd).cuda())
    mlp = int8_runtime.W8A8MLP(to_gpu_bf16(O.f32_to_bf16(gamma)), 1e-6, int8_runtime.GateUpQLinear(gate, up), down,
                               offset=0.0)
    h = to_gpu_bf16(hb)
    # stage by stage
    q, s = fused_kernels.rms_norm_quant(h, mlp.norm_weight, 1e-6, offset=0.0)
    hg = mlp.gate_up.forward_quantized(q, s)
    qh, sh = int8_kernels.act_quant(hg)
    out = mlp.down.forward_quantized(qh, sh, residual=h)
    l0 = int8_kernels.STATS["launch"]
    out2 = mlp(h)
    torch.cuda.synchronize()
    assert int8_kernels.STATS["launch"] - l0 == 4
    assert torch.equal(out, out2)
    rows = np.sort(rng.choice(T, 256, replace=False))
    tr = torch.from_numpy(rows).cuda()
    qn, sn = q[tr].cpu().numpy(), s[tr].cpu().numpy()
    g = O.epilogue(O.int_gemm(qn, qg), sn, sg)
    u = O.epilogue(O.int_gemm(qn, qu), sn, su)
    hk = bits_of(hg[tr])
    assert_within_one_ulp(hk, O.silu_mul(g, u))
    qo, so = O.quant_act(O.bf16_to_f32(hk))
    assert np.array_equal(qh[tr].cpu().numpy(), qo)
    assert np.array_equal(sh[tr].cpu().numpy().view(np.uint32), so.view(np.uint32))
    d = O.epilogue(O.int_gemm(qo, qd), so, sd)
    ref = O.f32_to_bf16(O.bf16_to_f32(d) + O.bf16_to_f32(hb[rows]))
    assert np.array_equal(bits_of(out[tr]), ref)


def test_swi_glu_op(gpu, kat):
    note("swi_glu op")
    c = kat["silu_mul"]
    h = fused_kernels.swi_glu(to_gpu_bf16(np.array(c["g_bf16"], np.uint16)), to_gpu_bf16(np.array(c["u_bf16"],
                                                                                                   np.uint16)))
    assert bits_of(h).tolist() == c["h_bf16"]
    rng = np.random.default_rng(8)
    g = O.f32_to_bf16(rng.standard_normal(1_000_003).astype(np.float32) * 4)
    u = O.f32_to_bf16(rng.standard_normal(1_000_003).astype(np.float32))
    assert_within_one_ulp(bits_of(fused_kernels.swi_glu(to_gpu_bf16(g), to_gpu_bf16(u))), O.silu_mul(g, u))


def test_silu_every_bf16_gate(gpu):
    """The SiLU of every finite bf16 gate value (u = 1, so h = bf16(silu(g))) is bit-exact against the
    oracle's float64 exp and IEEE fp32 quotient: the device formula (v_exp_f32, v_rcp_f32 + one Newton
    step) that the swi_glu kernel shares with the GEMMs' SiLU epilogue, on this hardware."""
    note("silu over all bf16 codes")
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = g[np.isfinite(O.bf16_to_f32(g))]
    u = np.full(g.shape, O.f32_to_bf16(np.array([1.0], np.float32))[0], np.uint16)
    ref = O.silu_mul(g, u)
    got = bits_of(fused_kernels.swi_glu(to_gpu_bf16(g), to_gpu_bf16(u)))
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} gate codes differ, first {g[bad[:5]]}: got {got[bad[:5]]} want {ref[bad[:5]]}"


# ------------------------------------------------------------------------------ readout
def test_readout_config4_shape(gpu, kat):
    """8 requests x 2048 packed tokens, hidden 2560: final RMSNorm at each last position, fp32 dot with
    2 + 255 label rows gathered from a 151936-row table, softmax over [:2] (noul) or [2:2+n]."""
    note("readout")
    rng = np.random.default_rng(4)
    B, S, K, V = 8, 2048, 2560, 151936
    h = act_bits(rng, (B * S, K), scale=0.5)
    rows = np.arange(B) * S + S - 1
    norm_w = O.round_bf16(rng.normal(0, 0.1, K).astype(np.float32))
    ids = rng.choice(V, 257, replace=False)
    table_rows = O.f32_to_bf16(rng.normal(0, 0.02, (257, K)).astype(np.float32))
    table = np.zeros((V, K), np.uint16)
    table[ids] = table_rows
    tt = to_gpu_bf16(table)
    ro = LabelReadout(tt, torch.from_numpy(ids).cuda())
    kinds = ["noul", "choice", "choice", "noul", "choice", "choice", "choice", "noul"]
    ns = [2, 255, 7, 2, 100, 3, 255, 2]
    lo = [0 if k == "noul" else 2 for k in kinds]
    logits, probs = ro(to_gpu_bf16(h), torch.from_numpy(rows).cuda(), to_gpu_bf16(O.f32_to_bf16(norm_w)), 1e-6,
                       lo=torch.tensor(lo).cuda(), cnt=torch.tensor(ns).cuda(), probs_width=255)
    zo = O.readout(h, rows, norm_w, 1e-6, O.bf16_to_f32(table_rows))
    np.testing.assert_allclose(logits.cpu().numpy(), zo, rtol=1e-4, atol=1e-4)
    p = probs.cpu().numpy()
    for b in range(B):
        po = O.option_probs(zo[b], kinds[b], ns[b])
        np.testing.assert_allclose(p[b, : ns[b]], po, atol=1e-3)
        assert abs(p[b, : ns[b]].sum() - 1) < 1e-5
    # the un-gathered table indexed by id inside the kernel gives the same logits
    ro2 = LabelReadout(tt, torch.from_numpy(ids).cuda(), gather=False)
    l2, _ = ro2(to_gpu_bf16(h), torch.from_numpy(rows).cuda(), to_gpu_bf16(O.f32_to_bf16(norm_w)), 1e-6)
    np.testing.assert_allclose(l2.cpu().numpy(), logits.cpu().numpy(), rtol=1e-5, atol=1e-5)
    # softmax known answers through the kernel: logits chosen so probs are closed forms
    for case in kat["softmax"]:
        z = np.array(case["z"], np.float32)
        n = len(z)
        x = np.zeros((1, 64), np.float32)
        x[0, 0] = 1.0
        W = np.zeros((n, 64), np.float32)
        W[:, 0] = z
        r3 = LabelReadout(torch.from_numpy(W).cuda(), list(range(n)))
        r3.weight = torch.from_numpy(W).cuda()
        _, pk = r3(to_gpu_bf16(O.f32_to_bf16(x)), torch.tensor([0]).cuda())
        np.testing.assert_allclose(pk.cpu().numpy()[0, :n], case["p"], atol=1e-6)


def test_gather_logits_function(gpu):
    """readout.gather_logits (fp32 and bf16 label rows; 0 = the No / Yes pair, n = the first n options)
    against the oracle's readout and option softmax."""
    from mica_amd.readout import gather_logits
    note("gather_logits")
    rng = np.random.default_rng(6)
    T, K, L = 600, 2560, 257
    h = act_bits(rng, (T, K), scale=0.5)
    rows = np.array([99, 299, 599, 0])
    norm_w = O.round_bf16(rng.normal(0, 0.1, K).astype(np.float32))
    W = O.round_bf16(rng.normal(0, 0.02, (L, K)).astype(np.float32))
    ns = [0, 255, 5, 0]
    zo = O.readout(h, rows, norm_w, 1e-6, W)
    for wt in (torch.from_numpy(W).cuda(), to_gpu_bf16(O.f32_to_bf16(W))):
        p = gather_logits(to_gpu_bf16(h), torch.from_numpy(rows).cuda(), to_gpu_bf16(O.f32_to_bf16(norm_w)), 1e-6,
                          wt, ns, offset=1.0).cpu().numpy()
        for b, n in enumerate(ns):
            kind, cnt = ("noul", 2) if n == 0 else ("choice", n)
            np.testing.assert_allclose(p[b, :cnt], O.option_probs(zo[b], kind, cnt), atol=1e-3)
            assert not p[b, cnt:].any()


def test_readout_bad_indices_give_nan_not_a_fault(gpu):
    note("readout bad indices")
    h = torch.zeros(4, 64, dtype=torch.bfloat16, device=gpu)
    table = torch.randn(10, 64, device=gpu).to(torch.bfloat16)
    ro = LabelReadout(table, torch.tensor([1, 2, 3], device=gpu), gather=False)
    ro.ids = torch.tensor([1, 2, 99], dtype=torch.int32, device=gpu)  # 99 is past the table
    logits, _ = ro(h, torch.tensor([0, 7], device=gpu))  # row 7 is past h
    z = logits.cpu()
    assert torch.isnan(z[1]).all() and torch.isnan(z[0, 2]) and not torch.isnan(z[0, :2]).any()


def test_no_fallbacks_were_taken(gpu):
    assert not int8_kernels.STATS["fallback"], int8_kernels.STATS["fallback"]


def test_rope_inplace_positions_and_period(gpu):
    """rope_inplace against the oracle's bf16 RoPE, with an explicit position array (ragged requests)
    and with period-derived positions; heads past n_heads and out-of-table positions stay as they were."""
    from mica_amd.fused_kernels import rope_inplace
    print("[case] rope", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(77)
    T, H, d, n_heads, n_pos = 300, 6, 128, 4, 256
    x = (torch.randn(T, H * d, generator=g) * 3).to(torch.bfloat16)
    ang = torch.rand(n_pos, d // 2, generator=g) * 6.3
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    pos = torch.cat([torch.arange(100), torch.arange(150), torch.arange(50) + 230]).to(torch.int32)  # 20 past n_pos
    xb = bits_of(x).reshape(T, H, d)
    for use_pos in (True, False):
        y = x.to(gpu)
        rope_inplace(y, n_heads, d, cos.to(gpu), sin.to(gpu), period=None if use_pos else 64,
                     pos=pos.to(gpu) if use_pos else None)
        torch.cuda.synchronize()
        p = pos.numpy() if use_pos else np.arange(T) % 64
        want = xb.copy()
        ok = p < n_pos
        pc = np.minimum(p, n_pos - 1)
        rot = O.rope(xb[:, :n_heads], bits_of(cos)[pc][:, None, :], bits_of(sin)[pc][:, None, :])
        want[ok, :n_heads] = rot[ok]
        assert np.array_equal(bits_of(y.cpu()).reshape(T, H, d), want)


@pytest.mark.parametrize("B,S,HK", [(2, 100, 1), (1, 64, 2), (1, 33, 1), (2, 1, 1)])
def test_causal_gqa_attention_matches_oracle(gpu, B, S, HK):
    """Flash attention (head dim 256, 4 query heads per key/value head) against the float64 oracle on
    the same bf16 inputs, q / k / v as strided views of one fused QKV buffer: relative Frobenius
    error <= 1e-2 per (sequence, head) (P is rounded to bf16 for the PV product, as in the reference's
    kernel and SDPA's flash path)."""
    from mica_amd.attention import causal_gqa_attention
    print(f"[case] attention B={B} S={S} HK={HK}", file=sys.stderr, flush=True)
    HQ, D = 4 * HK, 256
    g = torch.Generator().manual_seed(B * 100 + S)
    qkv = (torch.randn(B, S, HQ + 2 * HK, D, generator=g) * 1.5).to(torch.bfloat16)
    dq = qkv.to(gpu)
    q, k, v = dq[:, :, :HQ], dq[:, :, HQ:HQ + HK], dq[:, :, HQ + HK:]
    o = causal_gqa_attention(q, k, v)
    torch.cuda.synchronize()
    f = qkv.float().numpy()
    ref = O.causal_gqa_attention(f[:, :, :HQ], f[:, :, HQ:HQ + HK], f[:, :, HQ + HK:], D ** -0.5)
    got = o.float().cpu().numpy()
    worst = max(np.linalg.norm(got[b, :, h] - ref[b, :, h]) / np.linalg.norm(ref[b, :, h])
                for b in range(B) for h in range(HQ))
    print(f"relative error {worst:.2e}", file=sys.stderr)
    assert worst <= 1e-2


@pytest.mark.parametrize("B,Sq,Sk,HK,splits", [
    (2, 64, 1000, 1, 4),     # a continuation over a prefix: few query blocks, many keys
    (1, 33, 33, 1, 2),       # Sq == Sk: the diagonal tile's split holds keys above some queries
    (3, 40, 300, 2, 7),      # splits of unequal length, ragged last tiles
    (1, 1, 2048, 1, 64),     # one query row, the most splits
    (1, 96, 100, 1, 5),      # more splits than some blocks have tiles (empty splits)
])
def test_attention_split_keys_matches_oracle(gpu, B, Sq, Sk, HK, splits):
    """mica_attention_fwd_split (each query block's keys over several workgroups, partial softmax states
    merged) against the float64 oracle with Sk > Sq: relative error <= 1e-2 per (sequence, head), and
    at most twice the unsplit kernel's own error (+ 1e-3)."""
    from mica_amd.attention import causal_gqa_attention
    note(f"attention split B={B} Sq={Sq} Sk={Sk} HK={HK} splits={splits}")
    HQ, D = 4 * HK, 256
    g = torch.Generator().manual_seed(B * 1000 + Sq + Sk)
    q = (torch.randn(B, Sq, HQ, D, generator=g) * 1.5).to(torch.bfloat16)
    kv = (torch.randn(B, Sk, 2 * HK, D, generator=g) * 1.5).to(torch.bfloat16)
    dq, dkv = q.to(gpu), kv.to(gpu)
    k, v = dkv[:, :, :HK], dkv[:, :, HK:]
    o = causal_gqa_attention(dq, k, v, key_splits=splits)
    o1 = causal_gqa_attention(dq, k, v)
    torch.cuda.synchronize()
    f = kv.float().numpy()
    ref = O.causal_gqa_attention(q.float().numpy(), f[:, :, :HK], f[:, :, HK:], D ** -0.5)
    def worst(out):
        got = out.float().cpu().numpy()
        return max(np.linalg.norm(got[b, :, h] - ref[b, :, h]) / np.linalg.norm(ref[b, :, h])
                   for b in range(B) for h in range(HQ))
    w_split, w_one = worst(o), worst(o1)
    note(f"relative error: split {w_split:.2e}, unsplit {w_one:.2e}")
    assert w_split <= 1e-2
    # P is rounded to bf16 against a different running maximum in each split, so the two kernels differ
    # by rounding noise of the same size as the unsplit kernel's own error, not by a bias
    assert w_split <= 2.0 * w_one + 1e-3


@pytest.mark.parametrize("B,P,Sn,Sq,HK,splits,use_len", [
    (3, 64, 96, 96, 1, 1, False),     # continuations of one prefix: every new row a query
    (2, 256, 40, 40, 2, 1, False),    # ragged last tile of the new keys
    (4, 1024, 64, 64, 1, 5, False),   # split keys over the prefix and the new keys
    (3, 128, 70, 1, 1, 1, True),      # the last-only pass: one query per sequence at kv_len
    (2, 32, 33, 1, 1, 3, True),       # one prefix tile, split, per-sequence key counts
])
def test_attention_shared_prefix_equals_concatenated_keys(gpu, B, P, Sn, Sq, HK, splits, use_len):
    """mica_attention_fwd_prefix (a key prefix shared by every sequence, read in place) against the same
    kernel on the prefix expanded and concatenated to every sequence's keys: bit-identical outputs (each
    query sees the same key tiles in the same order), and the concatenated run against the oracle."""
    from mica_amd.attention import causal_gqa_attention
    note(f"attention prefix B={B} P={P} Sn={Sn} Sq={Sq} HK={HK} splits={splits} kv_len={use_len}")
    HQ, D = 4 * HK, 256
    g = torch.Generator().manual_seed(B * 100 + P + Sn + Sq)
    q = (torch.randn(B, Sq, HQ, D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
    kvp = (torch.randn(1, P, 2 * HK, D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
    kvn = (torch.randn(B, Sn, 2 * HK, D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
    kp, vp = kvp[:, :, :HK], kvp[:, :, HK:]
    kn, vn = kvn[:, :, :HK], kvn[:, :, HK:]
    kv_len = None
    if use_len:   # each sequence's query at a different position of its new keys
        kv_len = torch.tensor([P + Sn - 3 * b for b in range(B)], dtype=torch.int32, device=gpu)
    o = causal_gqa_attention(q, kn, vn, key_splits=splits, kv_len=kv_len, prefix=(kp, vp))
    kc = torch.cat((kp.expand(B, -1, -1, -1), kn), dim=1)
    vc = torch.cat((vp.expand(B, -1, -1, -1), vn), dim=1)
    oc = causal_gqa_attention(q, kc, vc, key_splits=splits, kv_len=kv_len)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), oc.view(torch.int16)), "shared prefix differs from concatenated keys"
    # the concatenated run against the oracle (queries at the last Sq of each sequence's kv_len keys)
    kcf, vcf, qf = kc.float().cpu().numpy(), vc.float().cpu().numpy(), q.float().cpu().numpy()
    for b in range(B):
        n = P + Sn if kv_len is None else int(kv_len[b])
        ref = O.causal_gqa_attention(qf[b:b + 1], kcf[b:b + 1, :n], vcf[b:b + 1, :n], D ** -0.5)[0]
        got = oc[b].float().cpu().numpy()
        err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert err <= 1e-2, (b, err)


@pytest.mark.parametrize("B,P,S,HK,splits,n_pos,use_pos", [
    (2, 0, 200, 1, 1, 4096, False),    # plain prefill, ragged last query block
    (1, 0, 1024, 4, 1, 4096, False),   # the layer's head count
    (1, 0, 70, 1, 1, 50, False),       # rows past the table stay unrotated
    (2, 64, 96, 2, 1, 4096, True),     # continuation of a prefix, explicit positions
    (2, 64, 96, 2, 3, 200, True),      # the same with split keys, some positions off the table
])
def test_attention_fused_rope_equals_rope_then_attention(gpu, B, P, S, HK, splits, n_pos, use_pos):
    """mica_attention_fwd_rope (the rotary embedding folded into the attention) against rope_inplace over
    the q and k heads of a fused QKV buffer followed by the plain kernel: k is rotated in place to the
    same bits, q is left as it was in memory, and the outputs are bit-identical."""
    from mica_amd.attention import causal_gqa_attention
    from mica_amd.fused_kernels import rope_inplace
    from mica_amd.model import _rope
    note(f"attention rope B={B} P={P} S={S} HK={HK} splits={splits} n_pos={n_pos} pos={use_pos}")
    HQ, D = 4 * HK, 256
    g = torch.Generator().manual_seed(B * 1000 + P + S + HK)
    qkv = (torch.randn(B * S, (HQ + 2 * HK) * D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
    cos, sin = _rope(n_pos, D, 1e6, gpu)
    pos = None
    if use_pos:   # P + (t % S), every tenth row pushed past the table
        p_ = torch.arange(B * S, dtype=torch.int32) % S + P
        p_[::10] += n_pos
        pos = p_.to(gpu)
    pre = None
    if P:
        kvp = (torch.randn(1, P, 2 * HK, D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
        pre = (kvp[:, :, :HK], kvp[:, :, HK:])

    def views(buf):
        q, k, v = buf.view(B, S, HQ + 2 * HK, D).split((HQ, HK, HK), dim=2)
        return q, k, v

    ref = qkv.clone()
    rope_inplace(ref, HQ + HK, D, cos, sin, period=None if use_pos else S, pos=pos)
    rq, rk, rv = views(ref)
    want = causal_gqa_attention(rq, rk, rv, key_splits=splits, prefix=pre)
    fused = qkv.clone()
    fq, fk, fv = views(fused)
    got = causal_gqa_attention(fq, fk, fv, key_splits=splits, prefix=pre, rope=(cos, sin, pos))
    torch.cuda.synchronize()
    assert torch.equal(fk.view(torch.int16), rk.view(torch.int16)), "keys rotated differently"
    q0 = views(qkv)[0]
    assert torch.equal(fq.view(torch.int16), q0.view(torch.int16)), "q was modified in memory"
    assert torch.equal(fv.view(torch.int16), rv.view(torch.int16)), "v was modified"
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "fused rope attention differs"


@pytest.mark.parametrize("B,P,S,rot,norms,n_pos,use_pos", [
    (2, 0, 200, 64, "qk", 4096, False),     # the reference model's layers: both head norms, RoPE on 64 dims
    (1, 0, 300, 256, "qk", 4096, False),
    (2, 64, 96, 128, "k", 200, True),       # a prefix continuation, k norm only, some positions off the table
    (1, 0, 70, 64, "", 50, False),          # partial RoPE alone
    (2, 0, 100, 0, "qk", 1, False),         # head norms alone
])
def test_attention_fused_head_norm_rope_equals_passes(gpu, B, P, S, rot, norms, n_pos, use_pos):
    """mica_attention_fwd_rope with head norms and partial RoPE against head_norm_rope over the q and k
    heads of a fused QKV buffer (output gate heads between them) followed by the plain kernel: k treated
    in place to the same bits, q and the gate heads left as they were, bit-identical outputs."""
    from mica_amd.attention import causal_gqa_attention
    from mica_amd.fused_kernels import head_norm_rope
    from mica_amd.model import _rope
    note(f"attention head norm rope B={B} P={P} S={S} rot={rot} norms={norms!r} n_pos={n_pos} pos={use_pos}")
    HK, D = 4, 256
    HQ = 4 * HK
    g = torch.Generator().manual_seed(B * 1000 + P + S + rot)
    cols = 2 * HQ + 2 * HK                      # q, gate, k, v heads
    qkv = (torch.randn(B * S, cols * D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
    qw = (torch.randn(D, generator=g) * 0.1).to(torch.bfloat16).to(gpu) if "q" in norms else None
    kw = (torch.randn(D, generator=g) * 0.1).to(torch.bfloat16).to(gpu) if "k" in norms else None
    cos, sin = _rope(n_pos, rot, 1e7, gpu) if rot else (None, None)
    pos = None
    if use_pos:
        p_ = torch.arange(B * S, dtype=torch.int32) % S + P
        p_[::10] += n_pos
        pos = p_.to(gpu)
    pre = None
    if P:
        kvp = (torch.randn(1, P, 2 * HK, D, generator=g) * 1.5).to(torch.bfloat16).to(gpu)
        pre = (kvp[:, :, :HK], kvp[:, :, HK:])

    def views(buf):
        q, _, k, v = buf.view(B, S, cols, D).split((HQ, HQ, HK, HK), dim=2)
        return q, k, v

    ref = qkv.clone()
    head_norm_rope(ref, D, (0, HQ), (2 * HQ * D, HK), qw, kw, 1e-6, 1.0, rot, cos, sin,
                   period=None if use_pos else S, pos=pos)
    rq, rk, rv = views(ref)
    want = causal_gqa_attention(rq, rk, rv, prefix=pre)
    fused = qkv.clone()
    fq, fk, fv = views(fused)
    got = causal_gqa_attention(fq, fk, fv, prefix=pre, rope=(cos, sin, pos) if rot else None,
                               head_norm=(qw, kw, 1.0, 1e-6))
    torch.cuda.synchronize()
    assert torch.equal(fk.view(torch.int16), rk.view(torch.int16)), "keys treated differently"
    untouched = torch.cat((qkv[:, :2 * HQ * D], qkv[:, (2 * HQ + HK) * D:]), 1)
    kept = torch.cat((fused[:, :2 * HQ * D], fused[:, (2 * HQ + HK) * D:]), 1)
    assert torch.equal(kept.view(torch.int16), untouched.view(torch.int16)), "q, gate or v modified in memory"
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "fused head norm / rope attention differs"


def test_attn_fwd_reference_selftest_cases(gpu):
    """int8_kernels.attn_fwd under the reference's own attention self-test (int8_runtime.py:444-488):
    its shapes (b, n, keys) with prefix keys, q as a transposed [b, n, hq, d] tensor and head-major k / v,
    checked against the float64 oracle with the reference's row tolerance 0.02."""
    print("[case] attn_fwd self-test cases", file=sys.stderr, flush=True)
    hq, rep, d, scale = 16, 4, 256, 0.0625
    hk = hq // rep
    assert int8_kernels.attn_keys(gpu) == ["attn|bf16|hd256|hq16|r4|s0.0625|m64"]
    g = torch.Generator().manual_seed(20261022)
    worst = 0.0
    for b, n, s in ((1, 1, 37), (2, 13, 13), (1, 48, 200), (1, 130, 130), (2, 70, 333)):
        q = torch.randn(b, n, hq, d, generator=g).to(torch.bfloat16)
        k = torch.randn(b, hk, s, d, generator=g).to(torch.bfloat16)
        v = torch.randn(b, hk, s, d, generator=g).to(torch.bfloat16)
        o = int8_kernels.attn_fwd(q.to(gpu).transpose(1, 2), k.to(gpu), v.to(gpu), scale)
        torch.cuda.synchronize()
        assert o is not None and o.shape == (b, hq, n, d)
        # oracle on the last n positions: pad the queries in front so query row i sits at position s - n + i
        qp = torch.zeros(b, s, hq, d)
        qp[:, s - n:] = q.float()
        ref = O.causal_gqa_attention(qp.numpy(), k.float().transpose(1, 2).numpy(), v.float().transpose(1, 2).numpy(),
                                     scale)[:, s - n:]
        got = o.float().cpu().transpose(1, 2).numpy()
        err = (np.linalg.norm(got - ref, axis=-1) / np.linalg.norm(ref, axis=-1)).max()
        worst = max(worst, err)
        assert err <= 0.02, (b, n, s, err)
    print(f"worst row error {worst:.2e}", file=sys.stderr)
