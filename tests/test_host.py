"""Host-side logic of the drop-in surface, on the CPU: the reference's miss convention
(None + a counted reason), the no-CPU-compute rule, weight-side helpers and layouts."""
import numpy as np
import pytest
import torch

from mica_amd import fused_kernels, int8_kernels, int8_runtime
from mica_amd.readout import LabelReadout
from oracle import w8a8 as O


@pytest.fixture
def lenient(monkeypatch):
    monkeypatch.setattr(int8_kernels, "STRICT", False)
    int8_kernels.STATS["fallback"].clear()
    return int8_kernels.STATS


def test_cpu_inputs_miss_like_the_reference(lenient):
    x = torch.randn(4, 64).to(torch.bfloat16)
    assert int8_kernels.act_quant(x) is None
    assert lenient["fallback"] == {"act_input": 1}
    q = torch.zeros(4, 64, dtype=torch.int8)
    s = torch.ones(4)
    assert int8_kernels.mm_i8(q, s, q, s) is None
    assert lenient["fallback"]["no_container"] == 1
    assert int8_kernels.mm_i8(q, s, q.float(), s) is None
    assert lenient["fallback"]["mm_input"] == 1
    assert int8_kernels.mm_i8(q, s, q[:, :32], s) is None
    assert lenient["fallback"]["mm_contiguous"] == 1
    assert int8_kernels.mm_i8(q, s.double(), q, s) is None
    assert lenient["fallback"]["mm_scales"] == 1
    qa = torch.zeros(1, 4, 8, 256, dtype=torch.bfloat16)
    ka = torch.zeros(1, 1, 8, 256, dtype=torch.bfloat16)
    assert int8_kernels.attn_fwd(qa, ka, ka, 0.0625) is None      # CPU tensors (int8_kernels.py:431-438)
    assert lenient["fallback"]["attn_input"] == 1
    assert int8_kernels.attn_fwd(qa, ka[:, :, :4], ka[:, :, :4], 0.0625) is None  # fewer keys than queries
    assert lenient["fallback"]["attn_input"] == 2
    assert int8_kernels.attn_keys() == []                          # no gfx950 device here


def test_strict_mode_raises_on_a_miss(monkeypatch):
    monkeypatch.setattr(int8_kernels, "STRICT", True)
    with pytest.raises(int8_kernels.KernelMiss):
        int8_kernels.act_quant(torch.randn(2, 16))


def test_no_cpu_compute_path():
    x = torch.randn(4, 64).to(torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        fused_kernels.rms_norm(x, w, 1e-6)
    with pytest.raises(ValueError, match="GPU only"):
        fused_kernels.rms_norm_quant(x, w, 1e-6)
    with pytest.raises(ValueError, match="GPU only"):
        fused_kernels.swi_glu(x, x)
    lin = torch.nn.Linear(64, 32, bias=False).to(torch.bfloat16)
    q = int8_runtime.QLinear(lin)
    with pytest.raises(ValueError, match="GPU only"):
        q(x)


def test_available_reports_without_a_gpu():
    ok, why = int8_kernels.available()
    if not torch.cuda.is_available():
        assert not ok and "GPU" in why


def test_qlinear_weight_quantization_matches_the_oracle():
    torch.manual_seed(0)
    lin = torch.nn.Linear(256, 48, bias=True).to(torch.bfloat16)
    q = int8_runtime.QLinear(lin)
    qo, so = O.quant_weight(lin.weight.detach().float().numpy())
    assert np.array_equal(q.qweight.numpy(), qo)
    assert np.array_equal(q.wscale.numpy().view(np.uint32), so.view(np.uint32))
    assert q.bias.dtype == torch.float32 and q.inv_smooth is None
    assert q.weight.shape == (48, 256)


def test_smoothing_buffers():
    torch.manual_seed(1)
    lin = torch.nn.Linear(128, 16, bias=False).to(torch.bfloat16)
    amax = torch.rand(128) * 4 + 0.05
    sm = int8_runtime.smooth_factors(amax, lin.weight)
    q = int8_runtime.QLinear(lin, sm)
    torch.testing.assert_close(q.inv_smooth, 1.0 / sm.float())
    # the dequantized weight approximates the original: per row, within one int8 step of the
    # smoothed row mapped back through inv_smooth
    w = lin.weight.detach().float()
    step = q.wscale[:, None] * q.inv_smooth[None, :]
    assert torch.all((q.weight.float() - w).abs() <= step * 0.5 + w.abs() * 2 ** -7)


def test_empty_and_from_quantized_shells():
    e = int8_runtime.QLinear.empty(2560, 9728, smooth=False)
    assert e.qweight.shape == (9728, 2560) and e.qweight.device.type == "meta" and e.inv_smooth is None
    qw = torch.randint(-127, 128, (64, 32), dtype=torch.int8)
    f = int8_runtime.QLinear.from_quantized(qw, torch.rand(64))
    assert f.out_features == 64 and f.in_features == 32


def test_pack_gate_up_layout_matches_the_oracle():
    rng = np.random.default_rng(0)
    qg = rng.integers(-127, 128, (256, 32), dtype=np.int8)
    qu = rng.integers(-127, 128, (256, 32), dtype=np.int8)
    sg = rng.random(256).astype(np.float32)
    su = rng.random(256).astype(np.float32)
    q, s = int8_runtime.pack_gate_up(*map(torch.from_numpy, (qg, sg, qu, su)))
    qo, so = O.pack_gate_up(qg, sg, qu, su)
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    # group j of 128 packed rows = gate rows 64j.. then up rows 64j..
    assert np.array_equal(q[128:192].numpy(), qg[64:128]) and np.array_equal(q[192:256].numpy(), qu[64:128])
    with pytest.raises(ValueError):
        int8_runtime.pack_gate_up(torch.from_numpy(qg[:100]), torch.from_numpy(sg[:100]),
                                  torch.from_numpy(qu[:100]), torch.from_numpy(su[:100]))


def test_label_readout_gathers_rows_once():
    table = torch.randn(1000, 64).to(torch.bfloat16)
    ids = [5, 999, 0, 17]
    r = LabelReadout(table, ids)
    assert r.weight.dtype == torch.float32 and r.weight.shape == (4, 64)
    assert torch.equal(r.weight, table[ids].float())
    r2 = LabelReadout(table, ids, gather=False)
    assert r2.ids.tolist() == ids and r2.weight.data_ptr() == table.data_ptr()
    with pytest.raises(ValueError, match="GPU only"):
        r(torch.zeros(8, 64, dtype=torch.bfloat16), [1, 2])


def _tile_of(pid, tiles_m, tiles_n, group_m=4, xcds=8):
    """The GEMM kernel's workgroup -> tile map (tile_of in mica_amd/csrc/gemm_i8.hip)."""
    nt = tiles_m * tiles_n
    per, rem = divmod(nt, xcds)
    x, local = pid % xcds, pid // xcds
    t = x * per + min(x, rem) + local
    width = group_m * tiles_n
    first = (t // width) * group_m
    gsize = min(tiles_m - first, group_m)
    inn = t % width
    return first + inn % gsize, inn // gsize


@pytest.mark.parametrize("m,n", [(4096, 9728), (512, 9728), (32768, 6144), (32768, 2560), (4096, 19456),
                                 (4096, 2560), (1, 32), (300, 1000), (16384, 9728), (257, 257), (2048, 768)])
def test_gemm_tile_map_is_a_bijection(m, n):
    """Every workgroup of the launch gets a distinct in-range tile and every tile is covered (checked
    before the kernel ever runs on a GPU)."""
    tm_, tn_ = -(-m // 256), -(-n // 256)
    seen = {_tile_of(p, tm_, tn_) for p in range(tm_ * tn_)}
    assert len(seen) == tm_ * tn_
    assert all(0 <= a < tm_ and 0 <= b < tn_ for a, b in seen)


# ------------------------------------------------------------------ GEMM split-tile (stream-K) schedule
def _gemm_schedule(M, N, K, cus, min_slabs=4):
    """mica_mm_i8's schedule choice (gemm_i8.hip): (dp_tiles, sk_tiles, grid)."""
    tiles = -(-M // 256) * -(-N // 256)
    nk = -(-K // 64)
    rem = tiles % cus
    if rem and rem * nk >= min_slabs * cus:
        return tiles - rem, rem, cus
    return tiles, 0, tiles


def _sk_begin(g, W, G):
    return g * W // G


def _sk_owner(i, W, G):
    return ((i + 1) * G + W - 1) // W - 1


@pytest.mark.parametrize("m,n,k", [(4096, 9728, 2560), (4096, 6144, 2560), (4096, 2560, 4096), (4096, 2560, 9728),
                                   (512, 9728, 2560), (4096, 19456, 2560), (32768, 6144, 2560), (300, 1000, 2576),
                                   (16384, 2560, 9728), (1, 9728, 2560), (2048, 4096, 2560)])
@pytest.mark.parametrize("cus", [256, 304, 80])
def test_gemm_split_schedule_covers_every_slab_once(m, n, k, cus):
    """Replays the kernel's work loop on the CPU: every (tile, slab) is computed exactly once; every
    split tile is finished by exactly one contributor, the one that counts itself last; the partial
    slots it reads are exactly those the other contributors wrote, and no slot is written twice."""
    dp, sk, G = _gemm_schedule(m, n, k, cus)
    nk = -(-k // 64)
    tiles_m, tiles_n = -(-m // 256), -(-n // 256)
    W = sk * nk
    done = {}
    written = {}              # (g, seg) -> tile
    contrib = {}              # tile -> set of g
    for g in range(G):
        pid = g
        while pid < dp:
            t = _tile_of(pid, tiles_m, tiles_n)
            for s in range(nk):
                done[(t, s)] = done.get((t, s), 0) + 1
            pid += G
        if not sk:
            continue
        b, e = _sk_begin(g, W, G), _sk_begin(g + 1, W, G)
        assert e > b, "a workgroup without stream-K work would break the arrival count"
        it = b
        while it < e:
            rel, k0 = divmod(it, nk)
            k1 = nk if nk - k0 < e - it else k0 + (e - it)
            t = _tile_of(dp + rel, tiles_m, tiles_n)
            for s in range(k0, k1):
                done[(t, s)] = done.get((t, s), 0) + 1
            if k0 != 0 or k1 != nk:
                seg = 1 if rel * nk > b else 0
                assert (g, seg) not in written
                written[(g, seg)] = rel
                contrib.setdefault(rel, set()).add(g)
            it += k1 - k0
    assert len(done) == tiles_m * tiles_n * nk and set(done.values()) == {1}
    for rel, gs in contrib.items():
        tb = rel * nk
        g0, g1 = _sk_owner(tb, W, G), _sk_owner(tb + nk - 1, W, G)
        assert gs == set(range(g0, g1 + 1)), "the arrival target g1 - g0 + 1 must count the real contributors"
        for g in gs:  # the slot the finisher reads for g is the one g wrote for this tile
            assert written[(g, 1 if tb > _sk_begin(g, W, G) else 0)] == rel
