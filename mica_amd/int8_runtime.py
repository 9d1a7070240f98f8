"""W8A8 linear modules on the gfx950 kernels: a drop-in ``QLinear`` (akivet/Mica
v0.5/serving/lib/int8_runtime.py:108-192), the fused gate+up projection of the gated MLP, and the
reference's numerical self-test (int8_runtime.py:362-443).

Buffers follow the reference (int8_runtime.py:124-127): ``qweight`` int8 [N, K] (K-contiguous),
``wscale`` fp32 [N], ``inv_smooth`` fp32 [K] or None, ``bias`` fp32 [N] or None.
"""
from __future__ import annotations

import json
import re
import time
import types
from pathlib import Path

import torch
from torch import nn

from . import int8_kernels as aot
from .fused_kernels import rms_norm_quant, rms_norm_quant_multi

EPS = 1e-08              # int8_quant.py:13
QMAX = 127.0             # int8_quant.py:11
ALPHA = 0.5              # int8_runtime.py:10
GATE_UP_GROUP = 64       # rows per gate / up group of the fused gate+up weight
SELFTEST_ROWS = (3, 48, 200, 608, 1500)   # int8_runtime.py:288
SELFTEST_TOL = 1.05                       # int8_runtime.py:289
SELFTEST_SEED = 20261022                  # int8_runtime.py:290


def quant_weight(w: torch.Tensor):
    """Per-output-channel symmetric int8 (int8_quant.quant_weight, int8_quant.py:54-61); offline."""
    wf = w.float()
    s = wf.abs().amax(1).clamp_min(EPS) / QMAX
    q = torch.round(wf / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


def smooth_factors(act_amax, w, alpha=ALPHA, lo=0.0001, hi=10000.0):
    """SmoothQuant factors (int8_quant.smooth_factors, int8_quant.py:80-85); offline."""
    a = act_amax.float().to(w.device)
    wmax = w.float().abs().amax(0)
    s = a.clamp_min(EPS).pow(alpha) / wmax.clamp_min(EPS).pow(1.0 - alpha)
    s = torch.where((a > 0) & (wmax > 0), s, torch.ones_like(s))
    return s.clamp(lo, hi)


def _hit(r, what):
    """A kernel miss inside a module is an error: the modules have no torch or CPU fallback."""
    if r is None:
        reasons = ", ".join(f"{k}={v}" for k, v in aot.STATS["fallback"].items())
        raise RuntimeError(f"mica_amd {what} kernel miss (misses so far: {reasons})")
    return r


def _require_gpu(x):
    if not x.is_cuda:
        raise ValueError("mica_amd W8A8 modules run on the GPU only (got a CPU tensor)")


class QLinear(nn.Module):
    """W8A8 linear: per-token int8 activations x per-channel int8 weights, bf16 out.

    forward(x) = 2 launches (act_quant + mm_i8), as the reference asserts in its self-test
    (int8_runtime.py:385-402); forward_quantized(qx, sx) = 1 launch for callers that produced the
    int8 activations themselves (the fused RMSNorm + quantizer).
    """

    def __init__(self, linear, smooth=None, backend="aot", keep_bf16=False):
        super().__init__()
        w = linear.weight.detach()
        self.register_buffer("w16", w.contiguous() if keep_bf16 else None)
        self.in_features, self.out_features = w.shape[1], w.shape[0]
        self.out_dtype, self.backend, self.mode = w.dtype, backend, "int8"
        wf = w.float()
        if smooth is not None:
            smooth = smooth.float().to(w.device)
            wf = wf * smooth[None, :]
            self.register_buffer("inv_smooth", (1.0 / smooth).contiguous())
        else:
            self.inv_smooth = None
        q, s = quant_weight(wf)
        self.register_buffer("qweight", q.contiguous())
        self.register_buffer("wscale", s.contiguous())
        self.register_buffer("bias", None if linear.bias is None else linear.bias.detach().float().contiguous())

    @classmethod
    def from_quantized(cls, qweight, wscale, bias=None, inv_smooth=None, out_dtype=torch.bfloat16):
        """Wrap already-quantized buffers (the layout of int8_runtime.load_file, :748-776)."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.register_buffer("w16", None)
        self.out_features, self.in_features = qweight.shape
        self.out_dtype, self.backend, self.mode = out_dtype, "aot", "int8"
        self.register_buffer("qweight", qweight.contiguous())
        self.register_buffer("wscale", wscale.float().contiguous())
        if inv_smooth is not None:
            self.register_buffer("inv_smooth", inv_smooth.float().contiguous())
        else:
            self.inv_smooth = None
        self.register_buffer("bias", None if bias is None else bias.float().contiguous())
        return self

    @classmethod
    def empty(cls, in_features, out_features, out_dtype=torch.bfloat16, backend="aot", smooth=True, bias=False):
        """Meta-device shell to be filled by a loader (int8_runtime.py:129-144)."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.register_buffer("w16", None)
        self.in_features, self.out_features = in_features, out_features
        self.out_dtype, self.backend, self.mode = out_dtype, backend, "int8"

        def meta(*shape, dtype=torch.float32):
            return torch.empty(*shape, dtype=dtype, device="meta")

        if smooth:
            self.register_buffer("inv_smooth", meta(in_features))
        else:
            self.inv_smooth = None
        self.register_buffer("qweight", meta(out_features, in_features, dtype=torch.int8))
        self.register_buffer("wscale", meta(out_features))
        self.register_buffer("bias", meta(out_features) if bias else None)
        return self

    @property
    def weight(self):
        w = self.qweight.float() * self.wscale.reshape(-1, 1)
        return (w * self.inv_smooth[None, :] if self.inv_smooth is not None else w).to(self.out_dtype)

    def _quant(self, x2):
        return _hit(aot.act_quant(x2.contiguous(), self.inv_smooth), "act_quant")

    def _mm(self, qx, sx, qw, sw, b, residual=None):
        return _hit(aot.mm_i8(qx, sx, qw, sw, b, self.out_dtype, residual=residual), "mm_i8")

    def rows_forward(self, x, ranges):
        """Quantize once, one GEMM per output-row range (int8_runtime.py:153-170)."""
        _require_gpu(x)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        qx, sx = self._quant(x2)
        outs = []
        for lo, hi in ranges:
            b = None if self.bias is None else self.bias[lo:hi]
            y = self._mm(qx, sx, self.qweight[lo:hi], self.wscale[lo:hi], b)
            outs.append(y.reshape(*shape[:-1], hi - lo))
        return outs

    def forward(self, x, residual=None):
        """y = QLinear(x) (int8_runtime.py:172-192); ``residual`` (same shape as y) is added in the
        GEMM epilogue after the bf16 rounding, i.e. ``residual + QLinear(x)``."""
        if self.w16 is not None and PRECISION["mode"] == "bf16":
            y = nn.functional.linear(x, self.w16, None if self.bias is None else self.bias.to(self.w16.dtype))
            return y if residual is None else residual + y
        _require_gpu(x)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.shape[0] == 0:
            return x.new_zeros(*shape[:-1], self.out_features, dtype=self.out_dtype)
        qx, sx = self._quant(x2)
        res = None if residual is None else residual.reshape(-1, self.out_features)
        return self._mm(qx, sx, self.qweight, self.wscale, self.bias, res).reshape(*shape[:-1], self.out_features)

    def forward_quantized(self, qx, sx, residual=None):
        """GEMM + epilogue on activations already quantized per token (e.g. by rms_norm_quant)."""
        _require_gpu(qx)
        if qx.shape[0] == 0:
            return torch.zeros(0, self.out_features, dtype=self.out_dtype, device=qx.device)
        return self._mm(qx, sx, self.qweight, self.wscale, self.bias, residual)


PRECISION = {"mode": "int8"}  # int8_runtime.py:21


def pack_gate_up(qg, sg, qu, su, group: int = GATE_UP_GROUP):
    """Interleave gate and up rows in groups of ``group``: [g_0..g_63, u_0..u_63, g_64.., u_64.., ...].

    Within one 128-row group the fused GEMM's SILU_MUL epilogue finds gate column c and up column c in
    the same lane, so silu(gate) * up never leaves registers."""
    n, k = qg.shape
    if qu.shape != (n, k) or n % group:
        raise ValueError(f"gate/up weights must both be [N, K] with N % {group} == 0")
    q = torch.stack((qg.reshape(n // group, group, k), qu.reshape(n // group, group, k)), 1).reshape(2 * n, k)
    s = torch.stack((sg.reshape(n // group, group), su.reshape(n // group, group)), 1).reshape(2 * n)
    return q.contiguous(), s.float().contiguous()


class GateUpQLinear(nn.Module):
    """gate_proj and up_proj of a gated MLP as one W8A8 GEMM (N = 2 x intermediate) whose epilogue
    returns h = bf16(bf16(silu(gate)) * up) -- the reference's gate QLinear, up QLinear and swi_glu
    (fast_runtime.py:126-132) in one launch, with the same roundings."""

    def __init__(self, gate: QLinear, up: QLinear):
        super().__init__()
        if gate.inv_smooth is not None or up.inv_smooth is not None:
            raise ValueError("the fused gate+up GEMM shares one activation quantization: no smoothing")
        if gate.bias is not None or up.bias is not None:
            raise ValueError("the fused gate+up GEMM has no bias")
        q, s = pack_gate_up(gate.qweight, gate.wscale, up.qweight, up.wscale)
        self.register_buffer("qweight", q)
        self.register_buffer("wscale", s)
        self.in_features = gate.in_features
        self.out_features = gate.out_features

    def forward_quantized(self, qx, sx):
        _require_gpu(qx)
        return _hit(aot.mm_i8(qx, sx, self.qweight, self.wscale, None, torch.bfloat16, epilogue="silu_mul"),
                    "fused gate+up mm_i8")

    def forward(self, x):
        _require_gpu(x)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        qx, sx = _hit(aot.act_quant(x2), "act_quant")
        return self.forward_quantized(qx, sx).reshape(*shape[:-1], self.out_features)


class W8A8MLP(nn.Module):
    """post_attention_layernorm + gated MLP + residual of one decoder layer (fork.py:419-422), as
    3 launches: fused RMSNorm+quant, fused gate+up GEMM with SiLU epilogue, act_quant of h, and the
    down GEMM with the residual add in its epilogue (4 launches in total)."""

    def __init__(self, norm_weight, eps, gate_up: GateUpQLinear, down: QLinear, offset=1.0):
        super().__init__()
        self.register_buffer("norm_weight", norm_weight.contiguous())
        self.eps, self.offset = float(eps), float(offset)
        self.gate_up, self.down = gate_up, down

    def forward(self, h):
        shape = h.shape
        q, s = rms_norm_quant(h, self.norm_weight, self.eps, offset=self.offset)
        g = self.gate_up.forward_quantized(q, s)
        qh, sh = _hit(aot.act_quant(g), "act_quant")
        out = self.down.forward_quantized(qh, sh, residual=h.reshape(-1, shape[-1]))
        return out.reshape(shape)


class SharedNormQLinears(nn.Module):
    """An RMSNorm and the W8A8 linears that consume its output: the reference model's q/k/v
    projections, or its linear-attention in_proj_qkv / in_proj_z / in_proj_a / in_proj_b (each a
    QLinear with its own SmoothQuant factors, int8_runtime.py:124-127, fed by one input_layernorm,
    fork.py:394-422).  forward(h) normalizes h once, quantizes it for every linear in one kernel
    (each with that linear's inv_smooth) and runs one GEMM per linear: 1 + len(linears) launches."""

    def __init__(self, norm_weight, eps, linears, offset=1.0):
        super().__init__()
        if not 1 <= len(linears) <= 4:
            raise ValueError("SharedNormQLinears takes 1 to 4 linears")
        if len({q.in_features for q in linears}) != 1:
            raise ValueError("the linears must share their input width")
        self.register_buffer("norm_weight", norm_weight.contiguous())
        self.eps, self.offset = float(eps), float(offset)
        self.linears = nn.ModuleList(linears)

    def forward(self, h, residual=None):
        """Returns [y_i] for each linear (and the summed input with a residual: ([y_i], h + residual))."""
        _require_gpu(h)
        shape = h.shape
        r = rms_norm_quant_multi(h, self.norm_weight, self.eps, [q.inv_smooth for q in self.linears],
                                 residual=residual, offset=self.offset)
        qs, summed = (r, None) if residual is None else r
        outs = [lin.forward_quantized(qx, sx).reshape(*shape[:-1], lin.out_features)
                for lin, (qx, sx) in zip(self.linears, qs)]
        return outs if residual is None else (outs, summed)


# ---------------------------------------------------------------------------------- checkpoints
FILE = "model-int8.safetensors"   # int8_runtime.py:639
FILE_FORMAT = "int8-w8a8/1"       # int8_runtime.py:640
LINEAR_NAMES = ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj",   # int8_quant.py:6-9
                "q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _safetensors_header(path):
    """The JSON header of a .safetensors file (8-byte little-endian length, then JSON); no tensor data
    is read."""
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        if not 0 < n < (1 << 30):
            raise ValueError(f"{path}: not a safetensors file")
        return json.loads(f.read(n).decode("utf-8"))


def linear_shapes(folder):
    """(N, K, has_bias) of every decoder-layer W8A8 linear in a checkpoint folder, from file headers only
    (int8_runtime.linear_shapes, int8_runtime.py:312-355): the ``qweight`` buffers of a
    ``model-int8.safetensors``, else the ``weight`` of the bf16 ``model*.safetensors`` shards.  The
    linear-attention in_proj_qkv also contributes its q / k and v row ranges, which rows_forward runs
    as separate GEMMs, when config.json gives the head sizes.  Multi-token-prediction layers (``mtp``)
    are skipped.  These are the shapes the self-test checks before a model is served."""
    folder = Path(folder)
    if (folder / FILE).is_file():
        files, leaf = [folder / FILE], "qweight"
    else:
        index = folder / "model.safetensors.index.json"
        names = (sorted(set(json.loads(index.read_text(encoding="utf-8"))["weight_map"].values()))
                 if index.is_file() else ["model.safetensors"])
        files, leaf = [folder / n for n in names if (folder / n).is_file()], "weight"
    layer = re.compile(r"(?:^|\.)layers\.\d+\.")
    out = set()
    for path in files:
        head = _safetensors_header(path)
        for key, info in head.items():
            if key == "__metadata__" or key.startswith("mtp") or not layer.search(key):
                continue
            parts = key.split(".")
            if len(parts) < 2 or parts[-1] != leaf or parts[-2] not in LINEAR_NAMES or len(info["shape"]) != 2:
                continue
            n, k = info["shape"]
            out.add((n, k, key[: -len(leaf)] + "bias" in head))
    try:
        cfg = json.loads((folder / "config.json").read_text(encoding="utf-8"))
        cfg = cfg.get("text_config", cfg)
        hidden = cfg["hidden_size"]
        kd = cfg["linear_num_key_heads"] * cfg["linear_key_head_dim"]
        vd = cfg["linear_num_value_heads"] * cfg["linear_value_head_dim"]
        if (2 * kd + vd, hidden, False) in out:
            out |= {(kd, hidden, False), (vd, hidden, False)}
    except (OSError, KeyError, ValueError):
        pass
    return sorted(out)


def load_linears(path, device="cuda"):
    """Read a ``model-int8.safetensors`` (format ``int8-w8a8/1``, int8_runtime.py:666-716) into this
    package's modules.

    Returns (linears, tensors): ``linears`` maps every prefix that has a ``<prefix>.qweight`` to a
    QLinear built from its ``qweight`` (int8 [N, K]), ``wscale`` (fp32 [N]), optional ``inv_smooth``
    (fp32 [K]) and optional ``bias`` (fp32 [N]); ``tensors`` holds every other tensor, with the file's
    ``ties`` metadata (alias -> source key) resolved to the source tensor.  A file that is not in this
    format, or whose buffers disagree in dtype or shape, raises ValueError('invalid_model') as the
    reference's loader does."""
    from safetensors import safe_open

    path = Path(path)
    if path.is_dir():
        path = path / FILE
    dev = torch.device(device)
    with safe_open(str(path), framework="pt", device=str(dev) if dev.type == "cuda" else "cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FILE_FORMAT:
            raise ValueError("invalid_model")
        keys = set(f.keys())
        ties = json.loads(meta.get("ties") or "{}")
        if any(t not in keys for t in ties.values()) or any(a in keys for a in ties):
            raise ValueError("invalid_model")
        prefixes = {k[: -len(".qweight")] for k in keys if k.endswith(".qweight")}
        owned = set()
        linears = {}
        for pre in sorted(prefixes):
            qw = f.get_tensor(pre + ".qweight")
            sw = f.get_tensor(pre + ".wscale") if pre + ".wscale" in keys else None
            inv = f.get_tensor(pre + ".inv_smooth") if pre + ".inv_smooth" in keys else None
            bias = f.get_tensor(pre + ".bias") if pre + ".bias" in keys else None
            if qw.dtype != torch.int8 or qw.dim() != 2 or sw is None:
                raise ValueError("invalid_model")
            n, k = qw.shape
            if sw.dtype != torch.float32 or tuple(sw.shape) != (n,):
                raise ValueError("invalid_model")
            if inv is not None and (inv.dtype != torch.float32 or tuple(inv.shape) != (k,)):
                raise ValueError("invalid_model")
            if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (n,)):
                raise ValueError("invalid_model")
            linears[pre] = QLinear.from_quantized(qw, sw, bias=bias, inv_smooth=inv)
            owned |= {pre + "." + leaf for leaf in ("qweight", "wscale", "inv_smooth", "bias")}
        tensors = {k: f.get_tensor(k) for k in sorted(keys - owned)}
    for alias, source in ties.items():
        tensors[alias] = tensors[source] if source in tensors else None
        if tensors[alias] is None:
            raise ValueError("invalid_model")
    return linears, tensors


# ---------------------------------------------------------------------------------- self-test
def _emulated_quant(x, inv_smooth):
    """The self-test's exact INT8 emulation of the quantizer (int8_quant.quant_act, int8_quant.py:64-73),
    in torch on the test's device: the yardstick the kernels' error is measured against."""
    xf = x.float()
    if inv_smooth is not None:
        xf = xf * inv_smooth
    s = xf.abs().amax(-1).clamp_min(EPS) / QMAX
    return torch.round(xf / s[:, None]).clamp(-127, 127).to(torch.int8), s


def _row_rel(a, b):
    return float(((a - b).norm(dim=-1) / b.norm(dim=-1).clamp_min(1e-30)).max())


def selftest(shapes, device, rows=SELFTEST_ROWS, seed=SELFTEST_SEED):
    """The reference's acceptance test (int8_runtime.py:362-443), on mica_amd's kernels.

    For every (N, K, has_bias) and every row count, with and without SmoothQuant factors: QLinear(x)
    must take exactly 2 kernel launches, be finite, and its row-relative L2 error against the fp32
    dequantized product must be <= 1.05 x that of an exact INT8 emulation.
    """
    t0 = time.perf_counter()
    out = {"ok": False, "reason": "", "checked": 0, "worst_ratio": 0.0}
    try:
        dev = torch.device(device)
        g = torch.Generator().manual_seed(seed)
        launches0 = aot.STATS["launch"]
        for n, k, has_bias in shapes:
            n, k = int(n), int(k)
            w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
            amax = torch.rand(k, generator=g) * 4 + 0.05
            amax[::61] *= 25.0
            b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(dev) if has_bias else None
            lin = types.SimpleNamespace(weight=w.to(dev), bias=b)
            for smooth in (smooth_factors(amax, w, ALPHA), None):
                q = QLinear(lin, smooth)
                wd = q.qweight.float() * q.wscale[:, None]
                if q.inv_smooth is not None:
                    wd = wd * q.inv_smooth[None, :]
                for m in rows:
                    x = (torch.randn(m, k, generator=g) * amax / 3).to(torch.bfloat16).to(dev)
                    l0, f0 = aot.STATS["launch"], dict(aot.STATS["fallback"])
                    y = q(x).float()
                    launched = aot.STATS["launch"] - l0
                    if launched != 2:
                        miss = {r: c - f0.get(r, 0) for r, c in aot.STATS["fallback"].items() if c != f0.get(r, 0)}
                        out["reason"] = f"N {n} K {k} M {m}: {launched} launches (expected 2), misses {miss}"
                        return out
                    ref = x.float() @ wd.t()
                    qx, sx = _emulated_quant(x, q.inv_smooth)
                    emu = (qx.double() @ q.qweight.double().t()).float() * sx[:, None] * q.wscale[None, :]
                    if q.bias is not None:
                        ref, emu = ref + q.bias, emu + q.bias
                    emu = emu.to(q.out_dtype).float()
                    noise, err = _row_rel(emu, ref), _row_rel(y, ref)
                    if not bool(torch.isfinite(y).all()):
                        out["reason"] = f"non-finite output (N {n}, K {k}, M {m})"
                        return out
                    if not err <= SELFTEST_TOL * noise:
                        out["reason"] = (f"N {n} K {k} M {m}: error {err:.4g} > {SELFTEST_TOL:.2f} x INT8 noise "
                                         f"{noise:.4g}")
                        return out
                    out["worst_ratio"] = max(out["worst_ratio"], err / max(noise, 1e-30))
                    out["checked"] += 1
        if dev.type == "cuda":
            torch.cuda.synchronize(dev)
        out.update(ok=True, reason="ok", launches=aot.STATS["launch"] - launches0)
        out["worst_ratio"] = round(out["worst_ratio"], 5)
    except Exception as exc:  # noqa: BLE001 -- the reference reports any failure as a reason string
        out["reason"] = f"{type(exc).__name__}: {exc}"[:300]
    finally:
        out["seconds"] = round(time.perf_counter() - t0, 2)
    return out
