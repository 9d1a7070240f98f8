"""The reference's own CPU path, restated with the same torch calls (test infrastructure and the CPU
baseline of bench.py; see oracle/__init__.py).  Citations are into akivet/Mica ``v0.5/serving/``.

This is what the reference runs when its GPU launchers miss: ``int8_quant.quant_act`` ->
``int8_quant.torch_int_mm`` -> ``.float() * sx * wscale`` -> ``.to(bf16)``, the eager RMSNorm and
``F.silu(g) * u``.  tests/test_oracle.py checks it bit-for-bit against ``oracle.w8a8``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

EPS = 1e-08   # int8_quant.py:13
QMAX = 127.0  # int8_quant.py:11


def quant_act(x: torch.Tensor, inv_smooth: torch.Tensor | None = None):
    """int8_quant.quant_act, int8 mode (int8_quant.py:64-73)."""
    xf = x.float()
    if inv_smooth is not None:
        xf = xf * inv_smooth
    s = xf.abs().amax(-1).clamp_min(EPS) / QMAX
    q = torch.round(xf / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


def torch_int_mm(qx: torch.Tensor, qw: torch.Tensor) -> torch.Tensor:
    """int8_quant.torch_int_mm (int8_quant.py:92-96): pads M <= 16 to 32 rows for _int_mm."""
    m = qx.shape[0]
    if m <= 16:
        qx = torch.cat((qx, qx.new_zeros(32 - m, qx.shape[1])), 0)
    return torch._int_mm(qx, qw.t())[:m]


def qlinear(x: torch.Tensor, qweight: torch.Tensor, wscale: torch.Tensor, bias=None, inv_smooth=None,
            out_dtype=torch.bfloat16) -> torch.Tensor:
    """QLinear.forward's fallback branch (int8_runtime.py:176-192)."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    if x2.shape[0] == 0:
        return x.new_zeros(*shape[:-1], qweight.shape[0], dtype=out_dtype)
    qx, sx = quant_act(x2, inv_smooth)
    y = torch_int_mm(qx, qweight).float() * sx[:, None] * wscale[None, :]
    if bias is not None:
        y = y + bias
    return y.to(out_dtype).reshape(*shape[:-1], qweight.shape[0])


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual=None, offset: float = 1.0):
    """fused_kernels.rms_norm, CPU branch (fused_kernels.py:51-56); offset=1 is its (1 + weight)."""
    value = x if residual is None else x + residual
    xf = value.float()
    y = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * (offset + weight.float())
    y = y.to(x.dtype)
    return y if residual is None else (y, value)


def swi_glu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """fused_kernels.swi_glu, CPU branch (fused_kernels.py:86-87)."""
    return F.silu(gate) * up


def mlp(x, gate, up, down, residual=None):
    """fast_runtime._fused_mlp (fast_runtime.py:126-132) with three W8A8 linears given as
    (qweight, wscale) pairs, plus the block's residual add (fork.py:419-422)."""
    g = qlinear(x, *gate)
    u = qlinear(x, *up)
    d = qlinear(swi_glu(g, u), *down)
    return d if residual is None else residual + d


def readout(x_last: torch.Tensor, norm_w: torch.Tensor, eps: float, label_w: torch.Tensor, offset=1.0):
    """body.norm then the fp32 label-row readout (prefill_engine.py:281, release_runtime.py:304-306)."""
    x = rms_norm(x_last, norm_w, eps, offset=offset)
    return F.linear(x.float(), label_w).float()
