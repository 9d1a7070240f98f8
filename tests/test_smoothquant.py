"""SmoothQuant statistics and the bf16 -> W8A8 conversion (int8_runtime.name_key / load_stats / convert,
reference int8_runtime.py:84-105, 195-206; int8_quant.py:80-85, 99-110), on the CPU.

Pinned by: the reference's own statistics file, summarised in tests/golden/stats_sample.json (its 248
keys all resolve to qualified linear names under our hash; sampled entries' lengths, first values and
sums); synthetic files in both of its layouts; closed forms of the SmoothQuant factors; and the oracle's
weight quantizer (itself pinned by known answers in test_oracle.py) on converted linears."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from mica_amd import int8_runtime as R
from oracle import w8a8 as O

HERE = Path(__file__).resolve().parent
SAMPLE = json.loads((HERE / "golden" / "stats_sample.json").read_text())
REF_STATS = Path("/root/reference/v0.5/serving/lib/kernels/s.pt")


def test_name_keys_match_the_reference_file():
    for e in SAMPLE["sample"]:
        assert R.name_key(e["name"]) == e["key"]
    keys = {R.name_key(n) for n in SAMPLE["names"]}
    assert len(keys) == len(SAMPLE["names"]) == SAMPLE["count"] == 248


def _packed(names, lengths, seed=0):
    rng = np.random.default_rng(seed)
    offs = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    vals = rng.uniform(0.01, 50.0, int(offs[-1])).astype(np.float32)
    keys = np.array([R.name_key(n) for n in names], np.int64)
    return {"h": torch.from_numpy(keys), "o": torch.from_numpy(offs), "v": torch.from_numpy(vals)}, offs, vals


def test_load_stats_packed_layout(tmp_path):
    names = ["layers.0.mlp.gate_proj", "layers.0.mlp.down_proj", "layers.3.self_attn.o_proj"]
    data, offs, vals = _packed(names, [16, 40, 24])
    f = tmp_path / "s.pt"
    torch.save(data, f)
    st = R.load_stats(f)
    assert len(st) == 3
    for i, n in enumerate(names):
        assert np.array_equal(st.get(n).numpy(), vals[offs[i]:offs[i + 1]])
    assert st.get("layers.0.mlp.up_proj") is None
    bad = dict(data, o=torch.tensor([0, 16, 10, 80]))
    torch.save(bad, f)
    with pytest.raises(ValueError):
        R.load_stats(f)


def test_load_stats_amax_layout(tmp_path):
    amax = {"layers.1.mlp.up_proj": torch.rand(8)}
    torch.save({"amax": amax}, tmp_path / "a.pt")
    got = R.load_stats(tmp_path / "a.pt")
    assert torch.equal(got["layers.1.mlp.up_proj"], amax["layers.1.mlp.up_proj"])


@pytest.mark.skipif(not REF_STATS.is_file(), reason="the reference tree is not present")
def test_load_stats_reads_the_reference_file():
    st = R.load_stats(REF_STATS)
    assert len(st) == SAMPLE["count"]
    assert all(st.get(n) is not None for n in SAMPLE["names"])
    assert sum(st.get(n).numel() for n in SAMPLE["names"]) == SAMPLE["values"]
    for e in SAMPLE["sample"]:
        v = st.get(e["name"])
        assert v.numel() == e["len"] and v[:8].tolist() == e["first"]
        assert float(v.double().sum()) == e["sum"]


def test_smooth_factors_closed_forms():
    a = torch.tensor([4.0, 0.0, 1e-12, 1e6, 9.0])
    w = torch.tensor([[1.0, 2.0, 3.0, 1e-6, 0.0], [-1.0, 0.5, 0.0, 0.0, 0.0]])
    s = R.smooth_factors(a, w)
    # sqrt(4) / sqrt(1) = 2; a = 0 -> 1; tiny a clamps to 1e-4; huge ratio clamps to 1e4; wmax = 0 -> 1
    assert np.array_equal(s.numpy(), np.array([2.0, 1.0, 1e-4, 1e4, 1.0], np.float32))
    assert np.array_equal(O.smooth_factors(a.numpy(), w.numpy()), s.numpy())
    rng = np.random.default_rng(1)
    a = rng.uniform(0.05, 100, 512).astype(np.float32)
    w = (rng.standard_normal((64, 512)) * 0.05).astype(np.float32)
    st, so = R.smooth_factors(torch.from_numpy(a), torch.from_numpy(w)).numpy(), O.smooth_factors(a, w)
    # fp32 pow is library math (not bit-pinned): each pow may differ by an ulp or two between torch and
    # numpy, the quotient then by a few
    assert np.all(np.abs(st.view(np.int32) - so.view(np.int32)) <= 4)


class _Attn(nn.Module):
    def __init__(self, h):
        super().__init__()
        self.q_proj, self.k_proj, self.v_proj = nn.Linear(h, 2 * h), nn.Linear(h, h // 2), nn.Linear(h, h // 2)
        self.o_proj = nn.Linear(2 * h, h)


class _Mixer(nn.Module):
    def __init__(self, h):
        super().__init__()
        self.in_proj_qkv, self.in_proj_z = nn.Linear(h, 3 * h), nn.Linear(h, h)
        self.in_proj_a, self.in_proj_b = nn.Linear(h, 4), nn.Linear(h, 4)
        self.out_proj = nn.Linear(h, h)


class _Mlp(nn.Module):
    def __init__(self, h):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = nn.Linear(h, 2 * h), nn.Linear(h, 2 * h), nn.Linear(2 * h, h)


class _Layer(nn.Module):
    def __init__(self, h, attention):
        super().__init__()
        if attention:
            self.self_attn = _Attn(h)
        else:
            self.linear_attn = _Mixer(h)
        self.mlp = _Mlp(h)
        self.norm = nn.LayerNorm(h)


def _body(h=32, seed=0):
    torch.manual_seed(seed)
    body = nn.Module()
    body.layers = nn.ModuleList([_Layer(h, attention=(i % 2 == 1)) for i in range(4)])
    return body.to(torch.bfloat16)


def test_target_linears_names_and_groups():
    body = _body()
    names = [n for n, *_ in R.target_linears(body)]
    assert names[:8] == ["layers.0.linear_attn.in_proj_qkv", "layers.0.linear_attn.in_proj_z",
                         "layers.0.linear_attn.in_proj_a", "layers.0.linear_attn.in_proj_b",
                         "layers.0.linear_attn.out_proj", "layers.0.mlp.gate_proj", "layers.0.mlp.up_proj",
                         "layers.0.mlp.down_proj"]
    assert len(names) == 2 * 8 + 2 * 7
    assert [n for n, *_ in R.target_linears(body, layers=[1], modules="attn")] == [
        f"layers.1.self_attn.{m}" for m in ("q_proj", "k_proj", "v_proj", "o_proj")]
    assert len(R.target_linears(body, layers=[0, 1, 9], modules=["mlp", "o_proj"])) == 3 + 4
    with pytest.raises(ValueError):
        R.target_linears(body, modules=["lm_head"])


def test_convert_smooths_where_statistics_exist():
    body = _body()
    lins = {n: c.weight.detach().clone() for n, _, _, c in R.target_linears(body)}
    rng = np.random.default_rng(5)
    amax = {n: torch.from_numpy(rng.uniform(0.05, 30, w.shape[1]).astype(np.float32))
            for i, (n, w) in enumerate(lins.items()) if i % 3 != 2}
    replaced, smoothed = R.convert(body, amax)
    assert (replaced, smoothed) == (len(lins), len(amax))
    for name, w in lins.items():
        mod = body
        for part in name.split("."):
            mod = mod[int(part)] if part.isdigit() else getattr(mod, part)
        assert isinstance(mod, R.QLinear)
        wf = w.float().numpy()
        if name in amax:
            s = R.smooth_factors(amax[name], w).numpy()
            assert np.array_equal(mod.inv_smooth.numpy(), (np.float32(1) / s).astype(np.float32))
            wf = wf * s[None, :]
        else:
            assert mod.inv_smooth is None
        qo, so = O.quant_weight(wf)
        assert np.array_equal(mod.qweight.numpy(), qo), name
        assert np.array_equal(mod.wscale.numpy().view(np.uint32), so.view(np.uint32)), name


def test_parse_modules_specs():
    """Module specs as int8_quant.parse_modules reads them (int8_quant.py:16-30)."""
    assert R.parse_modules(None) == R.LINEAR_NAMES
    assert R.parse_modules("attn,mlp") == ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                           "down_proj")
    assert R.parse_modules("ffn") == R.parse_modules("mlp") == ("gate_proj", "up_proj", "down_proj")
    assert R.parse_modules(" o_proj , ,mlp,o_proj") == ("o_proj", "gate_proj", "up_proj", "down_proj")
    assert R.parse_modules(["gdn", "out_proj", "q_proj"]) == ("in_proj_qkv", "in_proj_z", "in_proj_a",
                                                             "in_proj_b", "out_proj", "q_proj")
    assert R.parse_modules("all") == R.LINEAR_NAMES
    with pytest.raises(ValueError, match="lm_head"):
        R.parse_modules("mlp,lm_head")


def test_parse_layers_specs():
    """Layer specs as int8_quant.parse_layers reads them (int8_quant.py:33-51)."""
    assert R.parse_layers(None) == list(range(16))
    assert R.parse_layers(None, 8) == list(range(8))
    assert R.parse_layers("0-3, 8,2,,10-10") == [0, 1, 2, 3, 8, 10]
    assert R.parse_layers([5, 1, 5, 30], 16) == [1, 5]
    assert R.parse_layers(range(20, 40), 36) == list(range(20, 36))


def test_target_linears_default_layers_and_string_specs():
    torch.manual_seed(0)
    body = nn.Module()
    body.layers = nn.ModuleList([_Layer(16, attention=True) for _ in range(20)])
    assert {n.split(".")[1] for n, *_ in R.target_linears(body)} == {str(i) for i in range(16)}
    got = [n for n, *_ in R.target_linears(body, layers="17-18", modules="ffn,o_proj")]
    assert got == [f"layers.{i}.{m}" for i in (17, 18)
                   for m in ("self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")]
    # convert with no layer spec converts every layer, as the reference's convert does
    assert R.convert(body, None, modules="o_proj") == (20, 0)


def test_weight_scale_division_modes():
    """'ieee' (default) is the CPU path's quotient amax / 127; 'reciprocal' is fl(amax * fl(1/127)), what
    torch computes for the same expression on a GPU.  Both pinned against numpy fp32; they differ on
    some channels, so the option is not a no-op."""
    rng = np.random.default_rng(11)
    w = torch.from_numpy(rng.standard_normal((4096, 64)).astype(np.float32) * rng.uniform(0.01, 3, (4096, 1))
                         .astype(np.float32))
    amax = np.maximum(np.abs(w.numpy()).max(1), np.float32(1e-8)).astype(np.float32)
    q_i, s_i = R.quant_weight(w)
    q_r, s_r = R.quant_weight(w, division="reciprocal")
    ieee = (amax / np.float32(127)).astype(np.float32)
    recip = (amax * (np.float32(1) / np.float32(127))).astype(np.float32)
    assert np.array_equal(s_i.numpy().view(np.uint32), ieee.view(np.uint32))
    assert np.array_equal(s_r.numpy().view(np.uint32), recip.view(np.uint32))
    assert 0 < np.count_nonzero(ieee != recip) < ieee.size // 4
    qo, so = O.quant_weight(w.numpy())
    assert np.array_equal(q_i.numpy(), qo) and np.array_equal(s_i.numpy(), so)
    # q rounds w / s with the chosen s (IEEE quotient, half-even, clamp)
    assert np.array_equal(q_r.numpy(), np.clip(np.rint(w.numpy() / s_r.numpy()[:, None]), -127, 127).astype(np.int8))
    with pytest.raises(ValueError):
        R.quant_weight(w, division="fast")
    lin = nn.Linear(64, 4096, bias=False)
    lin.weight.data = w.to(torch.bfloat16)
    mod = R.QLinear(lin, division="reciprocal")
    assert np.array_equal(mod.wscale.numpy(), R.quant_weight(w.to(torch.bfloat16), "reciprocal")[1].numpy())
