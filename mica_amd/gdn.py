"""Gated delta net (GDN) token mixer on the gfx950 HIP kernels.

The reference's GDN layer step (akivet/Mica v0.5/serving/lib/fork.py ``gdn_step`` -> ``_gdn_inputs``
-> ``_gdn_scan``, :20-149) calls three operators this module replaces:

  causal_conv1d_fn(x, weight, bias, initial_states, activation)      fork.py:94-113, :163-175
      the causal-conv1d package's function on channel-last activations; ``l2norm_heads`` also
      l2-normalises the q / k heads of the result (use_qk_l2norm_in_kernel, fork.py:145)
  chunk_gated_delta_rule(q, k, v, g, beta, ...)                      fork.py:137-147
      flash-linear-attention 0.5.2's function (same signature and return value); grouped value
      heads are read in place instead of repeat_interleave'd (fork.py:134-136)
  gated_rmsnorm_quant(x, z, weight, eps)                             fork.py:148 + out_proj's act_quant
      attn.norm(out, z) fused with the INT8 quantisation of out_proj's input
  gdn_gate(a, b, A_log, dt_bias)                                     fork.py:124-125
      the decay g and write strength beta from the in_proj_a / in_proj_b outputs

Everything runs on the GPU through libmica_amd.so; there is no CPU path (a CPU tensor raises
ValueError) and no fallback.
"""
from __future__ import annotations

import torch

from . import _lib
from .int8_kernels import _aligned, _gpu_ok, _launched, _on, _stream

HEAD_DIM = 128
CHUNK = 64


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("mica_amd GDN kernels run on the GPU only (got a CPU tensor)")
    dev = ts[0].device
    if not _gpu_ok(dev):
        raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
    return dev


def _rc(rc, what):
    rc = _lib.check(rc, what)
    if rc:
        raise ValueError(f"{what}: unsupported input ({_lib.status_name(rc)})")
    _launched()


def _w_dtype(t):
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype == torch.float32:
        return _lib.FP32
    raise ValueError(f"conv weight must be bf16 or fp32, got {t.dtype}")


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None, return_final_states=False,
                     final_states_out=None, activation=None, l2norm_heads: int = 0, eps: float = 1e-6):
    """Depthwise causal convolution of x [B, C, T] (channel-last in memory: x.stride(1) == 1) with
    weight [C, W] (W <= 4), optional bias [C], optional initial_states [B, C, W - 1] (bf16), then
    SiLU when activation is 'silu' / 'swish'.  Returns y [B, C, T] bf16 (a channel-last view), and
    the final states [B, C, W - 1] when return_final_states.  l2norm_heads > 0 also divides each of
    the first l2norm_heads 128-channel groups of every token by its l2 norm (+ eps)."""
    if seq_idx is not None:
        raise ValueError("seq_idx is not supported")
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"activation {activation!r} not supported")
    dev = _need_gpu(x, weight, bias, initial_states)
    if x.dim() != 3 or x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be bf16 [B, C, T] with channels contiguous (channel-last)")
    B, C, T = x.shape
    w = weight if weight.dim() == 2 else weight.reshape(C, -1)
    if w.shape[0] != C or not w.is_contiguous():
        raise ValueError("weight must be a contiguous [C, W] tensor")
    wd = _w_dtype(w)
    if bias is not None and (bias.dtype != w.dtype or bias.numel() != C or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous [C] tensor of the weight's dtype")
    width = w.shape[1]
    init = None
    if initial_states is not None:
        init = initial_states.to(torch.bfloat16).contiguous()
        if init.shape != (B, C, width - 1):
            raise ValueError("initial_states must be [B, C, W - 1]")
    fin = None
    if return_final_states:
        fin = final_states_out if final_states_out is not None else torch.empty(
            (B, C, width - 1), dtype=torch.bfloat16, device=dev)
        if fin.shape != (B, C, width - 1) or fin.dtype != torch.bfloat16 or not fin.is_contiguous():
            raise ValueError("final_states_out must be a contiguous bf16 [B, C, W - 1] tensor")
    y = torch.empty((B, T, C), dtype=torch.bfloat16, device=dev)
    if not _aligned(x, y):
        raise ValueError("x must be 16-byte aligned")
    L = _lib.load()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    sbx = x.stride(0) if B > 1 else T * x.stride(2)
    _rc(_on(dev, lambda: L.mica_causal_conv1d(
        x.data_ptr(), sbx, x.stride(2), w.data_ptr(), ptr(bias), wd, width, ptr(init), ptr(fin), y.data_ptr(),
        T * C, C, B, T, C, 1 if activation is not None else 0, int(l2norm_heads), float(eps), _stream(dev))),
        "mica_causal_conv1d")
    out = y.transpose(1, 2)
    return (out, fin) if return_final_states else out


_ONES = {}


def l2norm_heads(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x [B, T, H, 128] bf16 divided by its l2 norm over the last axis (+ eps), per (b, t, h):
    the width-1 identity convolution with every head normalised."""
    if x.dim() != 4 or x.shape[-1] != HEAD_DIM or x.stride(3) != 1 or x.stride(2) != HEAD_DIM:
        raise ValueError("expected bf16 [B, T, H, 128] with contiguous heads")
    B, T, H, _ = x.shape
    C = H * HEAD_DIM
    key = (x.device, C)
    ones = _ONES.get(key)
    if ones is None:
        ones = _ONES[key] = torch.ones((C, 1), dtype=torch.float32, device=x.device)
    view = x.as_strided((B, C, T), (x.stride(0), 1, x.stride(1)))
    y = causal_conv1d_fn(view, ones, activation=None, l2norm_heads=H, eps=eps)
    return y.transpose(1, 2).reshape(B, T, H, HEAD_DIM)


def _heads_view(t, name):
    if t.dim() != 4 or t.shape[-1] != HEAD_DIM or t.dtype != torch.bfloat16 or t.stride(3) != 1 or \
            t.stride(2) != HEAD_DIM:
        raise ValueError(f"{name} must be bf16 [B, T, H, 128] with contiguous heads")
    B, T, H, _ = t.shape
    return t.stride(0) if B > 1 else T * t.stride(1), t.stride(1)


def gdn_workspace_bytes(B: int, T: int, HV: int) -> int:
    return int(_lib.load().mica_gdn_workspace_bytes(B, T, HV))


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                           use_qk_l2norm_in_kernel=False, cu_seqlens=None, head_first=False):
    """flash-linear-attention's chunk_gated_delta_rule on the gfx950 kernels.
    q, k: bf16 [B, T, HK, 128]; v: bf16 [B, T, HV, 128] (HV a multiple of HK; value head h reads key
    head h // (HV // HK)); g: [B, T, HV] log decays; beta: [B, T, HV]; initial_state: [B, HV, 128, 128].
    Returns (o bf16 [B, T, HV, 128], final_state fp32 [B, HV, 128, 128] or None)."""
    if cu_seqlens is not None or head_first:
        raise ValueError("cu_seqlens / head_first layouts are not supported")
    dev = _need_gpu(q, k, v, g, beta, initial_state)
    if use_qk_l2norm_in_kernel:
        q, k = l2norm_heads(q), l2norm_heads(k)
    sbq, ldq = _heads_view(q, "q")
    sbk, ldk = _heads_view(k, "k")
    sbv, ldv = _heads_view(v, "v")
    B, T, HK, _ = q.shape
    HV = v.shape[2]
    if k.shape != q.shape or v.shape[:2] != (B, T) or HV % HK:
        raise ValueError("q / k / v shapes do not match")
    g = g.to(torch.float32).contiguous()
    if beta.dtype not in (torch.bfloat16, torch.float32):
        beta = beta.float()
    beta = beta.contiguous()
    if g.shape != (B, T, HV) or beta.shape != (B, T, HV):
        raise ValueError("g and beta must be [B, T, HV]")
    h0 = None
    if initial_state is not None:
        h0 = initial_state.to(torch.float32).contiguous()
        if h0.shape != (B, HV, HEAD_DIM, HEAD_DIM):
            raise ValueError("initial_state must be [B, HV, 128, 128]")
    hT = torch.empty((B, HV, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev) if output_final_state else None
    o = torch.empty((B, T, HV, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    nbytes = gdn_workspace_bytes(B, T, HV)
    ws = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=dev)
    if not _aligned(q, k, v, o, ws, *[t for t in (h0, hT) if t is not None]):
        raise ValueError("q / k / v / states must be 16-byte aligned")
    scale = HEAD_DIM ** -0.5 if scale is None else float(scale)
    L = _lib.load()
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    _rc(_on(dev, lambda: L.mica_gdn_chunk(
        q.data_ptr(), sbq, ldq, k.data_ptr(), sbk, ldk, v.data_ptr(), sbv, ldv, g.data_ptr(), beta.data_ptr(),
        _lib.BF16 if beta.dtype == torch.bfloat16 else _lib.FP32, ptr(h0), ptr(hT), o.data_ptr(), scale,
        B, T, HK, HV, ws.data_ptr(), nbytes, _stream(dev))), "mica_gdn_chunk")
    return o, hT


def gdn_gate(a, b, A_log, dt_bias):
    """The GDN layer's decay and write strength (fork.py:124-125) in one launch:
    g = -exp(A_log) * softplus(a + dt_bias) (fp32) and beta = sigmoid(b) (bf16), per token and value
    head.  a, b: bf16 [..., HV] (rows may be strided); A_log, dt_bias: [HV].  Returns (g, beta) shaped
    like a."""
    dev = _need_gpu(a, b, A_log, dt_bias)
    HV = a.shape[-1]
    af, bf = a.reshape(-1, HV), b.reshape(-1, HV)
    if af.dtype != torch.bfloat16 or bf.dtype != torch.bfloat16 or af.stride(1) != 1 or bf.stride(1) != 1 or \
            bf.shape != af.shape:
        raise ValueError("gdn_gate takes bf16 a and b of one shape [..., HV] with contiguous heads")
    A = A_log.to(torch.float32).contiguous()
    dt = dt_bias.to(torch.float32).contiguous()
    if A.numel() != HV or dt.numel() != HV:
        raise ValueError("A_log and dt_bias must have HV elements")
    M = af.shape[0]
    g = torch.empty((M, HV), dtype=torch.float32, device=dev)
    beta = torch.empty((M, HV), dtype=torch.bfloat16, device=dev)
    L = _lib.load()
    _rc(_on(dev, lambda: L.mica_gdn_gate(af.data_ptr(), af.stride(0), bf.data_ptr(), bf.stride(0), A.data_ptr(),
                                         dt.data_ptr(), g.data_ptr(), beta.data_ptr(), M, HV, _stream(dev))),
        "mica_gdn_gate")
    return g.view(a.shape), beta.view(a.shape)


def gated_rmsnorm_quant(x, z, weight, eps: float = 1e-6, want_y: bool = False):
    """attn.norm(x, z) over 128-wide heads, then per-token INT8 (half-even) of the [.., HV * 128] row.
    Returns (q int8 [M, N], s fp32 [M]) or, with want_y, (q, s, y bf16 [M, N])."""
    dev = _need_gpu(x, z, weight)
    N = x.shape[-1]
    xf = x.reshape(-1, N)
    zf = z.reshape(-1, N)
    if xf.dtype != torch.bfloat16 or zf.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("gated_rmsnorm_quant takes bf16 x, z and weight")
    if xf.stride(1) != 1 or zf.stride(1) != 1 or weight.numel() != HEAD_DIM or not weight.is_contiguous():
        raise ValueError("x / z rows must be contiguous and weight [128]")
    M = xf.shape[0]
    q = torch.empty((M, N), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev) if want_y else None
    if not _aligned(xf, zf, weight, q, *([y] if y is not None else [])):
        raise ValueError("gated_rmsnorm_quant requires 16-byte aligned rows")
    L = _lib.load()
    _rc(_on(dev, lambda: L.mica_gated_rmsnorm_quant(
        xf.data_ptr(), xf.stride(0), zf.data_ptr(), zf.stride(0), weight.data_ptr(), float(eps),
        None if y is None else y.data_ptr(), N, q.data_ptr(), N, s.data_ptr(), M, N, _stream(dev))),
        "mica_gated_rmsnorm_quant")
    return (q, s, y) if want_y else (q, s)


class GDNLayer(torch.nn.Module):
    """The token-mixing half of a gated-delta-net decoder layer on the W8A8 path (fork.gdn_step and the
    layer's residual around it, fork.py:20-149): h + out_proj(norm_z(GDN(conv(in_proj(rmsnorm(h)))))).

      1. input RMSNorm, quantized per token once for the four projections (in_proj_qkv, in_proj_z,
         in_proj_b, in_proj_a; each a QLinear with its own SmoothQuant factors)  -> 1 + 4 launches
      2. causal conv + SiLU over the q / k / v channels, q / k l2-normalised  -> 1 launch
      3. g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)  (fork.py:124-125)  -> 1 launch
      4. chunked gated delta rule  -> 2 launches
      5. gated RMSNorm fused with out_proj's quantisation, out_proj GEMM with the residual add in its
         epilogue  -> 2 launches
    Input h: [B * T, hidden] bf16 rows of B sequences of T tokens each.  With keep=True the layer also
    returns (conv state, recurrent state) for continuation."""

    def __init__(self, norm_weight, eps, in_qkv, in_z, in_b, in_a, conv_weight, A_log, dt_bias, norm_z_weight,
                 out_proj, num_k_heads: int, num_v_heads: int, norm_offset: float = 1.0, z_eps: float = 1e-6):
        super().__init__()
        from .int8_runtime import SharedNormQLinears

        self.inproj = SharedNormQLinears(norm_weight, eps, [in_qkv, in_z, in_b, in_a], offset=norm_offset)
        self.register_buffer("conv_weight", conv_weight.contiguous())
        self.register_buffer("A_log", A_log.float().contiguous())
        self.register_buffer("dt_bias", dt_bias.float().contiguous())
        self.register_buffer("norm_z_weight", norm_z_weight.to(torch.bfloat16).contiguous())
        self.out_proj = out_proj
        self.hk, self.hv = int(num_k_heads), int(num_v_heads)
        self.z_eps = float(z_eps)
        if in_qkv.out_features != (2 * self.hk + self.hv) * HEAD_DIM or in_z.out_features != self.hv * HEAD_DIM:
            raise ValueError("projection widths do not match the head counts (head dims 128)")

    @torch.no_grad()
    def forward(self, h, batch: int, initial=None, keep: bool = False, trace=None):
        T = h.shape[0] // batch
        mixed, z, b, a = self.inproj(h)
        C = mixed.shape[-1]
        init_conv = None if initial is None else initial[0]
        conv = causal_conv1d_fn(mixed.view(batch, T, C).transpose(1, 2), self.conv_weight, activation="silu",
                                initial_states=init_conv, return_final_states=keep, l2norm_heads=2 * self.hk)
        conv, conv_state = conv if keep else (conv, None)
        x = conv.transpose(1, 2)                            # [B, T, C] (contiguous memory)
        kd = self.hk * HEAD_DIM
        q = x[..., :kd].unflatten(-1, (self.hk, HEAD_DIM))
        k = x[..., kd:2 * kd].unflatten(-1, (self.hk, HEAD_DIM))
        v = x[..., 2 * kd:].unflatten(-1, (self.hv, HEAD_DIM))
        g, beta = gdn_gate(a, b, self.A_log, self.dt_bias)
        o, rec = chunk_gated_delta_rule(q, k, v, g.view(batch, T, self.hv), beta.view(batch, T, self.hv),
                                        initial_state=None if initial is None else initial[1],
                                        output_final_state=keep)
        qo, so = gated_rmsnorm_quant(o.view(batch * T, -1), z, self.norm_z_weight, self.z_eps)
        out = self.out_proj.forward_quantized(qo, so, residual=h)
        if trace is not None:
            trace.update(mixed=mixed, z=z, b=b, a=a, conv=x, g=g, beta=beta, o=o, qo=qo, so=so, out=out)
        return (out, (conv_state, rec)) if keep else out
