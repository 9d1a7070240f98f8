"""The int8 checkpoint surface (int8_runtime.linear_shapes / load_linears) on synthetic files written in
the reference's ``model-int8.safetensors`` layout (format ``int8-w8a8/1``, int8_runtime.py:639-716):
``<prefix>.qweight`` int8 [N, K], ``.wscale`` fp32 [N], optional ``.inv_smooth`` fp32 [K] and ``.bias``
fp32 [N], other tensors as they are, and tied parameters listed in the ``ties`` metadata.  The reference
ships no checkpoint; these files are made here with safetensors."""
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from mica_amd import int8_runtime
from oracle import w8a8 as O

H, I, KD, VD = 256, 512, 128, 192   # hidden, MLP width, linear-attention key / value widths


def _model_tensors(rng):
    t = {}

    def lin(prefix, n, k, smooth=True, bias=False):
        t[prefix + ".qweight"] = torch.from_numpy(rng.integers(-127, 128, (n, k), dtype=np.int8))
        t[prefix + ".wscale"] = torch.from_numpy(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
        if smooth:
            t[prefix + ".inv_smooth"] = torch.from_numpy(rng.uniform(0.5, 2.0, k).astype(np.float32))
        if bias:
            t[prefix + ".bias"] = torch.from_numpy(rng.normal(0, 0.1, n).astype(np.float32))

    # layer 0: linear attention (GDN), layer 1: full attention; both with a gated MLP
    lin("model.layers.0.linear_attn.in_proj_qkv", 2 * KD + VD, H)
    lin("model.layers.0.linear_attn.in_proj_z", VD, H, smooth=False)
    lin("model.layers.0.linear_attn.out_proj", H, VD)
    lin("model.layers.1.self_attn.q_proj", H, H, bias=True)
    lin("model.layers.1.self_attn.o_proj", H, H)
    for i in (0, 1):
        lin(f"model.layers.{i}.mlp.gate_proj", I, H)
        lin(f"model.layers.{i}.mlp.up_proj", I, H)
        lin(f"model.layers.{i}.mlp.down_proj", H, I)
        t[f"model.layers.{i}.input_layernorm.weight"] = torch.zeros(H, dtype=torch.bfloat16)
    t["model.embed_tokens.weight"] = torch.randn(1000, H).to(torch.bfloat16)
    t["mtp.layers.0.mlp.gate_proj.qweight"] = torch.zeros(I, H, dtype=torch.int8)  # skipped by linear_shapes
    t["mtp.layers.0.mlp.gate_proj.wscale"] = torch.ones(I)
    return t


def _write(tmp_path, tensors, meta):
    save_file(tensors, str(tmp_path / int8_runtime.FILE), metadata=meta)
    (tmp_path / "config.json").write_text(json.dumps({"text_config": {
        "hidden_size": H, "linear_num_key_heads": 2, "linear_key_head_dim": KD // 2,
        "linear_num_value_heads": 3, "linear_value_head_dim": VD // 3}}))


@pytest.fixture
def ckpt(tmp_path):
    rng = np.random.default_rng(0)
    t = _model_tensors(rng)
    _write(tmp_path, t, {"format": "int8-w8a8/1", "ties": json.dumps({"lm_head.weight": "model.embed_tokens.weight"})})
    return tmp_path, t


def test_linear_shapes_from_headers(ckpt):
    folder, _ = ckpt
    shapes = int8_runtime.linear_shapes(folder)
    want = {(2 * KD + VD, H, False), (VD, H, False), (H, VD, False), (H, H, True), (H, H, False), (I, H, False),
            (H, I, False), (KD, H, False)}  # the q / k and v row ranges of in_proj_qkv (KD, VD) added
    assert set(shapes) == want


def test_load_linears_builds_qlinear_buffers(ckpt):
    folder, t = ckpt
    linears, tensors = int8_runtime.load_linears(folder, device="cpu")
    assert len(linears) == 12  # 11 decoder-layer linears + the multi-token-prediction gate_proj
    q = linears["model.layers.1.self_attn.q_proj"]
    assert torch.equal(q.qweight, t["model.layers.1.self_attn.q_proj.qweight"])
    assert torch.equal(q.bias, t["model.layers.1.self_attn.q_proj.bias"])
    assert torch.equal(q.inv_smooth, t["model.layers.1.self_attn.q_proj.inv_smooth"])
    assert linears["model.layers.0.linear_attn.in_proj_z"].inv_smooth is None
    assert (q.out_features, q.in_features) == (H, H)
    # the dequantized weight (int8_runtime.py:145-149): qweight * wscale * inv_smooth
    w = q.weight.float().numpy()
    ref = (t["model.layers.1.self_attn.q_proj.qweight"].float() * t["model.layers.1.self_attn.q_proj.wscale"][:, None]
           * t["model.layers.1.self_attn.q_proj.inv_smooth"][None, :]).to(torch.bfloat16).float().numpy()
    assert np.array_equal(w, ref)
    assert torch.equal(tensors["lm_head.weight"], tensors["model.embed_tokens.weight"])
    assert "model.layers.0.input_layernorm.weight" in tensors


@pytest.mark.parametrize("case", ["format", "dtype", "wscale_shape", "inv_shape", "tie_missing", "tie_duplicate"])
def test_load_linears_rejects(tmp_path, case):
    rng = np.random.default_rng(1)
    t = _model_tensors(rng)
    meta = {"format": "int8-w8a8/1", "ties": json.dumps({"lm_head.weight": "model.embed_tokens.weight"})}
    pre = "model.layers.1.self_attn.o_proj"
    if case == "format":
        meta["format"] = "int8-w8a8/0"
    elif case == "dtype":
        t[pre + ".qweight"] = t[pre + ".qweight"].to(torch.int16)
    elif case == "wscale_shape":
        t[pre + ".wscale"] = t[pre + ".wscale"][:-1].clone()
    elif case == "inv_shape":
        t[pre + ".inv_smooth"] = torch.ones(H + 8)
    elif case == "tie_missing":
        meta["ties"] = json.dumps({"lm_head.weight": "model.nonexistent.weight"})
    elif case == "tie_duplicate":
        t["lm_head.weight"] = t["model.embed_tokens.weight"].clone()
    _write(tmp_path, t, meta)
    with pytest.raises(ValueError, match="invalid_model"):
        int8_runtime.load_linears(tmp_path, device="cpu")


@pytest.mark.gpu
def test_loaded_linear_runs_bit_exact(gpu, ckpt):
    """A QLinear loaded from the file (smoothing + bias) computes the reference's arithmetic on the GPU."""
    folder, t = ckpt
    linears, _ = int8_runtime.load_linears(folder, device=gpu)
    pre = "model.layers.1.self_attn.q_proj"
    lin = linears[pre]
    rng = np.random.default_rng(2)
    x = O.f32_to_bf16(rng.standard_normal((77, H)).astype(np.float32))
    y = lin(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(gpu))
    ref = O.qlinear(x, t[pre + ".qweight"].numpy(), t[pre + ".wscale"].numpy(), bias=t[pre + ".bias"].numpy(),
                    inv_smooth=t[pre + ".inv_smooth"].numpy())
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), ref)


# ------------------------------------------------- linear_shapes on the bf16 checkpoint routes
def _bf16_linear(t, prefix, n, k, bias=False):
    t[prefix + ".weight"] = torch.zeros(n, k, dtype=torch.bfloat16)
    if bias:
        t[prefix + ".bias"] = torch.zeros(n, dtype=torch.bfloat16)


def _config(folder, nested=True, **over):
    cfg = {"hidden_size": H, "linear_num_key_heads": 2, "linear_key_head_dim": KD // 2,
           "linear_num_value_heads": 3, "linear_value_head_dim": VD // 3}
    cfg.update(over)
    (folder / "config.json").write_text(json.dumps({"text_config": cfg} if nested else cfg))


def test_linear_shapes_sharded_bf16(tmp_path):
    """Shards named by model.safetensors.index.json: 'weight' leaves of decoder-layer linears only; a shard
    the index lists but the folder lacks is skipped; a bias counts when it sits in the same shard."""
    a, b = {}, {}
    _bf16_linear(a, "model.language_model.layers.0.linear_attn.in_proj_qkv", 2 * KD + VD, H)
    _bf16_linear(a, "model.language_model.layers.0.mlp.gate_proj", I, H)
    _bf16_linear(a, "model.language_model.layers.3.self_attn.q_proj", H, H, bias=True)
    a["model.language_model.layers.0.input_layernorm.weight"] = torch.zeros(H, dtype=torch.bfloat16)
    a["model.language_model.embed_tokens.weight"] = torch.zeros(64, H, dtype=torch.bfloat16)
    _bf16_linear(b, "model.language_model.layers.1.mlp.down_proj", H, I)
    _bf16_linear(b, "mtp.layers.0.mlp.down_proj", H + 16, I)              # multi-token-prediction: skipped
    _bf16_linear(b, "model.visual.blocks.0.mlp.up_proj", 48, 32)           # not under layers.<i>: skipped
    _bf16_linear(b, "model.language_model.layers.2.self_attn.k_proj", 64, H)
    b["model.language_model.layers.2.self_attn.k_proj.qweight"] = torch.zeros(8, H, dtype=torch.int8)  # wrong leaf
    b["model.language_model.layers.2.mlp.gate_proj.weight"] = torch.zeros(I, dtype=torch.bfloat16)   # not 2-D
    save_file(a, str(tmp_path / "model-00001-of-00003.safetensors"))
    save_file(b, str(tmp_path / "model-00002-of-00003.safetensors"))
    wm = {k: "model-00001-of-00003.safetensors" for k in a}
    wm.update({k: "model-00002-of-00003.safetensors" for k in b})
    wm["model.language_model.layers.5.mlp.up_proj.weight"] = "model-00003-of-00003.safetensors"  # absent shard
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    _config(tmp_path)
    assert int8_runtime.linear_shapes(tmp_path) == sorted({
        (2 * KD + VD, H, False), (KD, H, False), (VD, H, False),    # in_proj_qkv and its q/k and v row ranges
        (I, H, False), (H, H, True), (H, I, False), (64, H, False)})


def test_linear_shapes_single_file_and_config_forms(tmp_path):
    """No index: model.safetensors alone.  The in_proj_qkv split reads a flat config as well as a nested
    text_config, and only applies to a bias-free [2 KD + VD, H] linear."""
    t = {}
    _bf16_linear(t, "model.layers.0.linear_attn.in_proj_qkv", 2 * KD + VD, H)
    _bf16_linear(t, "model.layers.0.linear_attn.out_proj", H, VD)
    save_file(t, str(tmp_path / "model.safetensors"))
    _config(tmp_path, nested=False)
    assert int8_runtime.linear_shapes(tmp_path) == sorted({(2 * KD + VD, H, False), (KD, H, False), (VD, H, False),
                                                           (H, VD, False)})
    _config(tmp_path, linear_num_value_heads=4)     # widths that do not add up to the stored linear: no split
    assert int8_runtime.linear_shapes(tmp_path) == sorted({(2 * KD + VD, H, False), (H, VD, False)})
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": H}))    # keys missing: no split, no error
    assert int8_runtime.linear_shapes(tmp_path) == sorted({(2 * KD + VD, H, False), (H, VD, False)})
    (tmp_path / "config.json").unlink()                                     # no config at all
    assert int8_runtime.linear_shapes(tmp_path) == sorted({(2 * KD + VD, H, False), (H, VD, False)})
    t2 = {}
    _bf16_linear(t2, "model.layers.0.linear_attn.in_proj_qkv", 2 * KD + VD, H, bias=True)
    save_file(t2, str(tmp_path / "model.safetensors"))
    _config(tmp_path)
    assert int8_runtime.linear_shapes(tmp_path) == [(2 * KD + VD, H, True)]   # biased: not split


def test_linear_shapes_prefers_int8_file(ckpt):
    """With model-int8.safetensors present, bf16 shards in the same folder are not read."""
    folder, _ = ckpt
    t = {}
    _bf16_linear(t, "model.layers.0.mlp.gate_proj", 4 * I, H)
    save_file(t, str(folder / "model.safetensors"))
    assert (4 * I, H, False) not in int8_runtime.linear_shapes(folder)


def test_linear_shapes_empty_folder(tmp_path):
    assert int8_runtime.linear_shapes(tmp_path) == []
