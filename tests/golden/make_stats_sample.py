"""Summarise the reference's SmoothQuant statistics file into a small fixture.

    python tests/golden/make_stats_sample.py [/path/to/reference]

Loads v0.5/serving/lib/kernels/s.pt with torch's weights-only loader (the file is data: int64 keys and
offsets and fp32 absmax values; no code in it runs) and writes tests/golden/stats_sample.json: the
number of linears, the qualified name of every key (found by hashing the candidate names
layers.{i}.{module path} of a 32-layer body), and for a few linears their key, length, first values
and float64 sum.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
MODULES = ("linear_attn.in_proj_qkv", "linear_attn.in_proj_z", "linear_attn.in_proj_a", "linear_attn.in_proj_b",
           "linear_attn.out_proj", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
SAMPLE = ("layers.0.linear_attn.in_proj_qkv", "layers.3.self_attn.q_proj", "layers.3.self_attn.o_proj",
          "layers.17.mlp.down_proj", "layers.30.linear_attn.in_proj_b")


def key(name):
    return int.from_bytes(hashlib.sha256(name.encode("utf-8")).digest()[:8], "little", signed=True)


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    ref = Path(argv[0]) if argv else Path("/root/reference")
    d = torch.load(str(ref / "v0.5" / "serving" / "lib" / "kernels" / "s.pt"), map_location="cpu", weights_only=True)
    keys, offs, vals = d["h"].tolist(), d["o"].tolist(), d["v"]
    by_key = {k: (offs[i], offs[i + 1]) for i, k in enumerate(keys)}
    names = sorted(n for n in (f"layers.{i}.{m}" for i in range(32) for m in MODULES) if key(n) in by_key)
    sample = []
    for n in SAMPLE:
        a, b = by_key[key(n)]
        v = vals[a:b]
        sample.append({"name": n, "key": key(n), "len": b - a, "first": v[:8].tolist(),
                       "sum": float(v.double().sum())})
    out = {"count": len(keys), "values": int(vals.numel()), "names": names, "sample": sample}
    (HERE / "stats_sample.json").write_text(json.dumps(out, indent=0) + "\n", encoding="utf-8")
    print(f"{len(keys)} linears, {len(names)} names resolved")


if __name__ == "__main__":
    main()
