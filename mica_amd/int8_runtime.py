"""W8A8 linear modules on the gfx950 kernels: a drop-in ``QLinear`` (akivet/Mica
v0.5/serving/lib/int8_runtime.py:108-192), the fused gate+up projection of the gated MLP, and the
reference's numerical self-test (int8_runtime.py:362-443).

Buffers follow the reference (int8_runtime.py:124-127): ``qweight`` int8 [N, K] (K-contiguous),
``wscale`` fp32 [N], ``inv_smooth`` fp32 [K] or None, ``bias`` fp32 [N] or None.
"""
from __future__ import annotations

import hashlib
import json
import struct
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


def _ieee_div(num: torch.Tensor, den: float) -> torch.Tensor:
    """num / den with the IEEE fp32 quotient on every device.  torch turns a division of a GPU tensor by a
    Python scalar into a multiplication by the scalar's reciprocal, which misses the quotient by one ulp
    for a few values (measured: 29 of 1024 weight scales); a divisor tensor on the same device keeps the
    quotient, which is what the reference's CPU path computes."""
    return num / torch.full((), den, dtype=num.dtype, device=num.device)


SCALE_DIVISION = ("ieee", "reciprocal")


def quant_weight(w: torch.Tensor, division: str = "ieee"):
    """Per-output-channel symmetric int8 (int8_quant.quant_weight, int8_quant.py:54-61); offline.

    ``division`` picks how the scale max(amax, 1e-8) / 127 is rounded.  'ieee' (default): the IEEE fp32
    quotient on any device (see _ieee_div), the bits of the reference's CPU path.  'reciprocal':
    fl(amax * fl(1 / 127)), the bits torch produces on a GPU for the same expression (a division by a
    Python scalar becomes a multiplication by its fp32 reciprocal), i.e. the bits of weights the reference
    converts on the GPU (release_runtime.py:267-272 -> int8_runtime.apply -> convert).  The two differ by
    one ulp on a few per cent of channels; q is then rounded from w / s with either s."""
    if division not in SCALE_DIVISION:
        raise ValueError(f"division must be one of {SCALE_DIVISION}, got {division!r}")
    wf = w.float()
    amax = wf.abs().amax(1).clamp_min(EPS)
    if division == "ieee":
        s = _ieee_div(amax, QMAX)
    else:
        s = amax * torch.full((), 1.0, dtype=torch.float32, device=amax.device).div_(QMAX)
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

    def __init__(self, linear, smooth=None, backend="aot", keep_bf16=False, division="ieee"):
        """From a bf16 linear (int8_runtime.py:109-127): SmoothQuant factors folded into the weight, which
        is then quantized per output channel; ``division`` is quant_weight's scale rounding."""
        super().__init__()
        w = linear.weight.detach()
        self.register_buffer("w16", w.contiguous() if keep_bf16 else None)
        self.in_features, self.out_features = w.shape[1], w.shape[0]
        self.out_dtype, self.backend, self.mode = w.dtype, backend, "int8"
        wf = w.float()
        if smooth is not None:
            smooth = smooth.float().to(w.device)
            wf = wf * smooth[None, :]
            self.register_buffer("inv_smooth", (torch.ones_like(smooth) / smooth).contiguous())
        else:
            self.inv_smooth = None
        q, s = quant_weight(wf, division)
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
        return _hit(aot.mm_i8(qx, sx, qw, sw, b, self.out_dtype, residual=residual,
                              split="auto"), "mm_i8")

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
        return _hit(aot.mm_i8(qx, sx, self.qweight, self.wscale, None, torch.bfloat16, epilogue="silu_mul",
                              split="auto"), "fused gate+up mm_i8")

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
    fork.py:394-422).  forward(h) normalizes h once and quantizes it for every linear in one kernel
    (each with that linear's inv_smooth).

    Linears whose factors are the same (both None, or equal vectors) get the same int8 input, so they
    share it: one quantized copy and one GEMM over their weights stacked along N, whose output columns
    are each linear's output (a column view of the shared [.., sum N] result; every element's
    arithmetic is the linear's own, so the values are those of separate GEMMs).  The reference quantizes
    once per linear (int8_runtime.py:180-186).  The members' buffers become row views of the stacked
    ones, so the weights are not held twice.  1 + (number of distinct factor sets) launches."""

    def __init__(self, norm_weight, eps, linears, offset=1.0):
        super().__init__()
        if not 1 <= len(linears) <= 4:
            raise ValueError("SharedNormQLinears takes 1 to 4 linears")
        if len({q.in_features for q in linears}) != 1:
            raise ValueError("the linears must share their input width")
        self.register_buffer("norm_weight", norm_weight.contiguous())
        self.eps, self.offset = float(eps), float(offset)
        self.linears = nn.ModuleList(linears)
        self.groups = []      # lists of linear indices that share one int8 input
        for i, q in enumerate(linears):
            for grp in self.groups:
                r = linears[grp[0]]
                if _same_factors(r.inv_smooth, q.inv_smooth) and r.out_dtype == q.out_dtype and \
                        (r.bias is None) == (q.bias is None):
                    grp.append(i)
                    break
            else:
                self.groups.append([i])
        self._stacked = {}    # group index -> (qweight, wscale, bias) stacked along N

    def _stack(self, gi):
        """The group's stacked buffers, made on first use (the members may be filled by a loader after
        construction) and again whenever a member's buffers were replaced since."""
        grp = [self.linears[i] for i in self.groups[gi]]
        st = self._stacked.get(gi)
        if st is not None:
            qw = st[0]
            off, ok = 0, True
            for q in grp:
                ok = ok and q.qweight.data_ptr() == qw.data_ptr() + off * qw.stride(0)
                off += q.out_features
            if ok:
                return st
        qw = torch.cat([q.qweight for q in grp]).contiguous()
        sw = torch.cat([q.wscale for q in grp]).contiguous()
        b = None if grp[0].bias is None else torch.cat([q.bias for q in grp]).contiguous()
        off = 0
        for q in grp:   # the members read row views of the stacked buffers
            n = q.out_features
            q.qweight, q.wscale = qw[off:off + n], sw[off:off + n]
            if b is not None:
                q.bias = b[off:off + n]
            off += n
        self._stacked[gi] = (qw, sw, b)
        return self._stacked[gi]

    def forward(self, h, residual=None):
        """Returns [y_i] for each linear (and the summed input with a residual: ([y_i], h + residual))."""
        _require_gpu(h)
        shape = h.shape
        firsts = [self.linears[grp[0]] for grp in self.groups]
        r = rms_norm_quant_multi(h, self.norm_weight, self.eps, [q.inv_smooth for q in firsts],
                                 residual=residual, offset=self.offset)
        qs, summed = (r, None) if residual is None else r
        outs = [None] * len(self.linears)
        for gi, (grp, (qx, sx)) in enumerate(zip(self.groups, qs)):
            if len(grp) == 1:
                lin = self.linears[grp[0]]
                outs[grp[0]] = lin.forward_quantized(qx, sx).reshape(*shape[:-1], lin.out_features)
                continue
            qw, sw, b = self._stack(gi)
            if qx.shape[0] == 0:
                y = torch.zeros(0, qw.shape[0], dtype=self.linears[grp[0]].out_dtype, device=qx.device)
            else:
                y = _hit(aot.mm_i8(qx, sx, qw, sw, b, self.linears[grp[0]].out_dtype,
                                   split="auto"), "mm_i8")
            off = 0
            for i in grp:
                n = self.linears[i].out_features
                outs[i] = y[:, off:off + n].reshape(*shape[:-1], n)
                off += n
        return outs if residual is None else (outs, summed)


def _same_factors(a, b) -> bool:
    """Two linears' SmoothQuant factors give the same int8 input: both absent, or equal vectors."""
    if a is None or b is None:
        return a is None and b is None
    return a is b or (a.shape == b.shape and a.device == b.device and bool(torch.equal(a, b)))


# ---------------------------------------------------------------------------------- checkpoints
FILE = "model-int8.safetensors"   # int8_runtime.py:639
FILE_FORMAT = "int8-w8a8/1"       # int8_runtime.py:640
LINEAR_NAMES = ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj",   # int8_quant.py:6-9
                "q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


# ---------------------------------------------------------------- SmoothQuant statistics and conversion
def name_key(name: str) -> int:
    """The key of a linear's activation statistics in the reference's ``s.pt``: the first 8 bytes of the
    SHA-256 of its qualified name (``layers.{i}.{path}``), little-endian, signed (int8_runtime.py:84-85).
    The file stores only these keys, so the hash is part of its format."""
    return int.from_bytes(hashlib.sha256(name.encode("utf-8")).digest()[:8], "little", signed=True)


class ActStats:
    """Per-linear input absmax (fp32 [K]) packed as in ``s.pt``: ``h`` int64 [L] name keys, ``o`` int64
    [L + 1] offsets into ``v`` fp32, linear i's values being v[o[i]:o[i + 1]] (int8_runtime.py:88-98)."""

    def __init__(self, keys, offsets, values):
        keys, offsets = [int(k) for k in keys.tolist()], [int(o) for o in offsets.tolist()]
        if len(offsets) != len(keys) + 1 or offsets[0] < 0 or offsets[-1] > values.numel() or \
                any(b < a for a, b in zip(offsets, offsets[1:])):
            raise ValueError("activation statistics: offsets do not partition the values")
        self._span = {k: (offsets[i], offsets[i + 1]) for i, k in enumerate(keys)}
        self._values = values

    def get(self, name: str):
        """The absmax vector of the linear called ``name``, or None if the file has none for it."""
        span = self._span.get(name_key(name))
        return None if span is None else self._values[span[0]:span[1]]

    def __len__(self):
        return len(self._span)


def load_stats(path):
    """Read a SmoothQuant statistics file (int8_runtime.load_stats, int8_runtime.py:101-105) with torch's
    weights-only loader (no code in the file runs): the packed ``h`` / ``o`` / ``v`` layout becomes an
    ActStats; a plain ``{"amax": {name: tensor}}`` file gives that mapping."""
    data = torch.load(str(path), map_location="cpu", weights_only=True)
    if not isinstance(data, dict):
        raise ValueError(f"{path}: not an activation statistics file")
    if "amax" in data:
        return data["amax"]
    if not {"h", "o", "v"} <= set(data):
        raise ValueError(f"{path}: expected 'amax' or the packed 'h' / 'o' / 'v' tensors")
    return ActStats(data["h"], data["o"], data["v"].float())


MODULE_GROUPS = {"gdn": LINEAR_NAMES[:5], "attn": LINEAR_NAMES[5:9], "mlp": LINEAR_NAMES[9:]}  # int8_quant.py:6-9
MODULE_GROUPS["ffn"] = MODULE_GROUPS["mlp"]
MODULE_GROUPS["all"] = LINEAR_NAMES
DEFAULT_LAYERS = range(0, 16)     # int8_quant.py:10


def parse_modules(spec=None) -> tuple:
    """The linear names a module spec selects (int8_quant.parse_modules, int8_quant.py:16-30): None is all
    twelve; otherwise a comma-separated string or a sequence whose items are group names ('gdn', 'attn',
    'mlp' or its alias 'ffn', 'all') or linear names, blank items ignored, expanded in order with
    repeats dropped.  A name that is neither raises ValueError."""
    if spec is None:
        return LINEAR_NAMES
    items = [str(x).strip() for x in (spec.split(",") if isinstance(spec, str) else spec)]
    names = dict.fromkeys(n for item in items if item for n in MODULE_GROUPS.get(item, (item,)))
    unknown = [n for n in names if n not in LINEAR_NAMES]
    if unknown:
        raise ValueError(f"unknown module names {unknown}; known {list(LINEAR_NAMES)}")
    return tuple(names)


def parse_layers(spec=None, n_layers=None) -> list:
    """Sorted distinct layer indices of a layer spec (int8_quant.parse_layers, int8_quant.py:33-51): None is
    layers 0-15 (DEFAULT_LAYERS); a string is comma-separated indices and inclusive ranges ('0-3,8');
    anything else an iterable of indices.  With ``n_layers``, indices >= n_layers are dropped."""
    if spec is None:
        spec = DEFAULT_LAYERS
    if isinstance(spec, str):
        picked = set()
        for part in filter(None, (p.strip() for p in spec.split(","))):
            lo, sep, hi = part.partition("-")
            picked.update(range(int(lo), int(hi) + 1) if sep else (int(part),))
        spec = picked
    out = sorted({int(i) for i in spec})
    return out if n_layers is None else [i for i in out if i < n_layers]


def target_linears(body, layers=None, modules=None):
    """(qualified name, parent module, attribute, nn.Linear) of every linear ``modules`` selects
    (parse_modules) inside ``body.layers[i]`` for the layers ``layers`` selects (parse_layers: None is
    layers 0-15, as in the reference), in layer order and module-tree order; the qualified name is
    ``layers.{i}.{path}`` as the statistics file keys it (int8_quant.target_linears, int8_quant.py:99-110)."""
    wanted = set(parse_modules(modules))
    found = []
    for i in parse_layers(layers, len(body.layers)):
        for path, parent in body.layers[i].named_modules():
            for attr, child in parent.named_children():
                if attr in wanted and isinstance(child, nn.Linear):
                    found.append((f"layers.{i}." + (f"{path}." if path else "") + attr, parent, attr, child))
    return found


def convert(body, stats=None, alpha=ALPHA, layers=None, modules=None, division="ieee"):
    """Replace the body's bf16 linears by W8A8 QLinears in place (int8_runtime.convert,
    int8_runtime.py:195-206): a linear whose input absmax is in ``stats`` (load_stats) is smoothed with
    SmoothQuant factors (alpha 0.5) folded into its weight before quantization, the others are quantized
    as they are.  ``layers`` None converts every layer, as the reference's convert does (it passes all of
    them to target_linears); ``division`` is quant_weight's scale rounding.  Returns (linears replaced,
    linears smoothed)."""
    replaced = smoothed = 0
    layers = range(len(body.layers)) if layers is None else layers
    for name, parent, attr, child in target_linears(body, layers, modules):
        amax = None if stats is None else stats.get(name)
        smooth = None if amax is None else smooth_factors(amax, child.weight.detach(), alpha)
        setattr(parent, attr, QLinear(child, smooth, division=division))
        replaced += 1
        smoothed += smooth is not None
    return replaced, smoothed


def _tensor_shapes(path) -> dict:
    """{tensor name: shape tuple} of a .safetensors file, read from its JSON header alone (an 8-byte
    little-endian length, then the JSON); no tensor data is touched."""
    with open(path, "rb") as f:
        (size,) = struct.unpack("<Q", f.read(8))
        if not 0 < size < (1 << 30):
            raise ValueError(f"{path}: not a safetensors file")
        header = json.loads(f.read(size))
    return {name: tuple(entry["shape"]) for name, entry in header.items() if name != "__metadata__"}


def _weight_sources(folder: Path):
    """The files whose headers describe the linears, and the leaf name of a linear's matrix in them:
    the int8 file and its ``qweight`` buffers when present; otherwise the bf16 ``weight`` matrices of the
    shards that ``model.safetensors.index.json`` lists (those present in the folder), or of
    ``model.safetensors`` when there is no index."""
    if (folder / FILE).is_file():
        return [folder / FILE], "qweight"
    index = folder / "model.safetensors.index.json"
    shards = {"model.safetensors"}
    if index.is_file():
        shards = set(json.loads(index.read_text(encoding="utf-8"))["weight_map"].values())
    return [folder / name for name in sorted(shards) if (folder / name).is_file()], "weight"


def _is_layer_linear(name: str, leaf: str) -> bool:
    """True for ``<...>.layers.<i>.<...>.<linear>.<leaf>`` with <linear> one of LINEAR_NAMES, outside the
    multi-token-prediction head (names starting with ``mtp``)."""
    parts = name.split(".")
    if name.startswith("mtp") or len(parts) < 3 or parts[-1] != leaf or parts[-2] not in LINEAR_NAMES:
        return False
    return any(a == "layers" and b.isdigit() for a, b in zip(parts[:-2], parts[1:-1]))


def _qkv_row_ranges(folder: Path):
    """(hidden, q/k width, v width) of the linear-attention in_proj_qkv from config.json (its
    ``text_config`` when nested), or None when the file or a key is missing."""
    try:
        cfg = json.loads((folder / "config.json").read_text(encoding="utf-8"))
        text = cfg.get("text_config", cfg)
        return (text["hidden_size"], text["linear_num_key_heads"] * text["linear_key_head_dim"],
                text["linear_num_value_heads"] * text["linear_value_head_dim"])
    except (OSError, KeyError, ValueError):
        return None


def linear_shapes(folder):
    """(N, K, has_bias) of every decoder-layer W8A8 linear in a checkpoint folder, sorted, from file
    headers only: the shape set the self-test is run on before a model is served (the output of
    int8_runtime.linear_shapes, int8_runtime.py:312-355).  A linear has a bias when ``<prefix>.bias`` is
    in the same file.  When config.json gives the linear-attention head sizes and a bias-free
    in_proj_qkv [2 KD + VD, H] is present, its q / k rows [KD, H] and v rows [VD, H] are added too:
    rows_forward runs those ranges as GEMMs of their own."""
    folder = Path(folder)
    files, leaf = _weight_sources(folder)
    found = set()
    for path in files:
        shapes = _tensor_shapes(path)
        for name, shape in shapes.items():
            if len(shape) == 2 and _is_layer_linear(name, leaf):
                prefix = name[: -len(leaf) - 1]
                found.add((shape[0], shape[1], prefix + ".bias" in shapes))
    widths = _qkv_row_ranges(folder)
    if widths is not None:
        hidden, kd, vd = widths
        if (2 * kd + vd, hidden, False) in found:
            found.update({(kd, hidden, False), (vd, hidden, False)})
    return sorted(found)


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
    s = _ieee_div(xf.abs().amax(-1).clamp_min(EPS), QMAX)
    return torch.round(xf / s[:, None]).clamp(-127, 127).to(torch.int8), s


def _row_rel(a, b):
    return float(((a - b).norm(dim=-1) / b.norm(dim=-1).clamp_min(1e-30)).max())


def _selftest_case(q, x, wd):
    """One QLinear call of the self-test: (output fp32, kernel launches it took, its row-relative error
    against the fp32 dequantized product, the INT8 emulation's error against the same product)."""
    before = aot.STATS["launch"]
    y = q(x).float()
    launches = aot.STATS["launch"] - before
    exact = x.float() @ wd.t()
    qx, sx = _emulated_quant(x, q.inv_smooth)
    emulated = (qx.double() @ q.qweight.double().t()).float() * sx[:, None] * q.wscale[None, :]
    if q.bias is not None:
        exact, emulated = exact + q.bias, emulated + q.bias
    emulated = emulated.to(q.out_dtype).float()
    return y, launches, _row_rel(y, exact), _row_rel(emulated, exact)


def selftest(shapes, device, backend="aot", rows=SELFTEST_ROWS, seed=SELFTEST_SEED):
    """The reference's acceptance test (int8_runtime.py:362-443), on mica_amd's kernels; same positional
    signature, ``selftest(shapes, device, backend)``, which the reference's self-test child calls
    (int8_runtime.py:292).  ``backend`` must be 'aot': there is no other backend here.

    For every (N, K, has_bias) and every row count, with and without SmoothQuant factors: QLinear(x)
    must take exactly 2 kernel launches, be finite, and its row-relative L2 error against the fp32
    dequantized product must be <= 1.05 x that of an exact INT8 emulation.  The random draws follow the
    reference's order (same seed, same calls), so both judge the same inputs.

    Returns a dict: ``ok`` and ``reason`` (the keys the reference's callers read; reason "ok" or what
    failed), ``cases`` (QLinear calls checked), ``max_err_vs_noise`` (largest error / INT8-noise ratio),
    ``kernel_launches`` and ``elapsed_s``.
    """
    started = time.perf_counter()
    report = {"ok": False, "reason": "", "cases": 0, "max_err_vs_noise": 0.0}
    try:
        if backend != "aot":
            report["reason"] = f"backend {backend!r} is not available: mica_amd runs the 'aot' kernels only"
            return report
        dev = torch.device(device)
        g = torch.Generator().manual_seed(seed)
        first_launch = aot.STATS["launch"]
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
                    misses_before = dict(aot.STATS["fallback"])
                    y, launches, err, noise = _selftest_case(q, x, wd)
                    case = f"QLinear {n}x{k} on {m} rows"
                    if launches != 2:
                        new = {r: c - misses_before.get(r, 0) for r, c in aot.STATS["fallback"].items()
                               if c != misses_before.get(r, 0)}
                        report["reason"] = f"{case} took {launches} kernel launches instead of 2 (misses: {new})"
                        return report
                    if not bool(torch.isfinite(y).all()):
                        report["reason"] = f"{case} produced a non-finite value"
                        return report
                    if not err <= SELFTEST_TOL * noise:
                        report["reason"] = (f"{case}: relative error {err:.4g} exceeds {SELFTEST_TOL} times the "
                                            f"INT8 emulation's {noise:.4g}")
                        return report
                    report["max_err_vs_noise"] = max(report["max_err_vs_noise"], err / max(noise, 1e-30))
                    report["cases"] += 1
        if dev.type == "cuda":
            torch.cuda.synchronize(dev)
        report.update(ok=True, reason="ok", kernel_launches=aot.STATS["launch"] - first_launch,
                      max_err_vs_noise=round(report["max_err_vs_noise"], 5))
    except Exception as exc:  # noqa: BLE001 -- any failure is reported in `reason`, as the reference does
        report["reason"] = f"self-test raised {type(exc).__name__}: {exc}"[:300]
    finally:
        report["elapsed_s"] = round(time.perf_counter() - started, 2)
    return report
