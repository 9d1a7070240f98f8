"""Last-position label readout on the gfx950 kernel: only the allowed answer rows of the output
embedding are ever multiplied, and only at each request's last token.

Reference: the readout closure built in HFJudge.__init__ (akivet/Mica
v0.5/serving/lib/release_runtime.py:298-306) applied to ``body.norm`` of the last hidden row
(prefill_engine.py:280-304), then the slice + softmax of judge_many (release_runtime.py:509-517).
"""
from __future__ import annotations

import torch

from . import _lib
from .int8_kernels import DT, _gpu_ok, _launched, _on, _stream


class LabelReadout:
    """Readout over label rows of the output embedding.

    ``gather=True`` copies the rows once as fp32, as the reference does (release_runtime.py:301);
    ``gather=False`` keeps the bf16 table and indexes it by id inside the kernel.
    """

    def __init__(self, lm_head_weight: torch.Tensor, ids, gather: bool = True):
        ids = torch.as_tensor(ids, dtype=torch.long, device=lm_head_weight.device)
        self.n_labels = int(ids.numel())
        if gather:
            self.weight = lm_head_weight.detach().index_select(0, ids).float().contiguous()
            self.ids = None
        else:
            if lm_head_weight.dtype != torch.bfloat16:
                raise ValueError("an un-gathered table must be bf16")
            self.weight = lm_head_weight.detach().contiguous()
            self.ids = ids.to(torch.int32).contiguous()

    def __call__(self, h, rows, norm_weight=None, eps=1e-6, offset=1.0, lo=None, cnt=None, probs_width=None):
        """h: [T, K] bf16 hidden states (packed requests); rows: int [B] index of each request's last
        token; norm_weight: the final RMSNorm weight or None (h already normed).
        lo / cnt: int [B] start and length of each request's softmax slice (None: all labels).
        Returns (logits fp32 [B, L], probs fp32 [B, width])."""
        if not h.is_cuda:
            raise ValueError("mica_amd readout runs on the GPU only (got a CPU tensor)")
        if h.dtype != torch.bfloat16 or h.dim() != 2 or h.stride(1) != 1:
            raise ValueError("h must be a 2-D bf16 tensor with unit feature stride")
        dev = h.device
        if not _gpu_ok(dev):
            raise RuntimeError(f"mica_amd kernels need a gfx950 GPU (device {dev})")
        K = h.shape[1]
        rows = torch.as_tensor(rows, device=dev).to(torch.int32).contiguous()
        B = rows.numel()
        L = self.n_labels
        logits = torch.empty((B, L), dtype=torch.float32, device=dev)
        if lo is not None:
            if probs_width is None:
                # the width is read from host values only: a device tensor would need a synchronising
                # read, which stalls the stream and cannot be captured in a HIP graph
                if isinstance(cnt, torch.Tensor) and cnt.is_cuda:
                    raise ValueError("give probs_width when cnt is a device tensor")
                host = torch.as_tensor(cnt, dtype=torch.int64)
                probs_width = int(host.max()) if host.numel() else 0
            lo = torch.as_tensor(lo, device=dev).to(torch.int32).contiguous()
            cnt = torch.as_tensor(cnt, device=dev).to(torch.int32).contiguous()
            width = probs_width if B else 0
        else:
            width = L
        probs = torch.zeros((B, max(width, 1)), dtype=torch.float32, device=dev)
        nw = None if norm_weight is None else norm_weight.contiguous()
        lib = _lib.load()
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        wdt = _lib.FP32 if self.weight.dtype == torch.float32 else _lib.BF16
        rc = _lib.check(_on(dev, lambda: lib.mica_gather_logits(
            h.data_ptr(), h.stride(0), h.shape[0], rows.data_ptr(), B, ptr(nw),
            DT[nw.dtype] if nw is not None else 0, float(offset), float(eps), self.weight.data_ptr(), wdt,
            self.weight.stride(0), self.weight.shape[0], ptr(self.ids), L, K, logits.data_ptr(), ptr(lo), ptr(cnt),
            probs.data_ptr(), probs.shape[1], _stream(dev))), "mica_gather_logits")
        if rc > 0:
            raise ValueError(f"readout does not support this input ({_lib.status_name(rc)})")
        _launched()
        return logits, probs


def gather_logits(h, last_idx, norm_w, eps, label_W, n_opts, offset=1.0):
    """The readout as one function: the final RMSNorm of h at each request's last token (rows
    last_idx of the packed [T, K] bf16 h), fp32 dots with the label rows label_W ([L, K] fp32 or bf16:
    No, Yes, then the option labels, as gathered by release_runtime.py:298-302), and the softmax of
    each request's slice (release_runtime.py:509-517): n_opts[b] == 0 reads the No / Yes pair, n > 0
    the first n option labels.  n_opts is one int for every request or one per request.  Returns the
    probabilities, fp32 [B, max slice] (zero past each request's slice); one kernel launch pair."""
    if label_W.dtype not in (torch.float32, torch.bfloat16) or label_W.dim() != 2:
        raise ValueError("label_W must be a 2-D fp32 or bf16 tensor")
    ro = LabelReadout.__new__(LabelReadout)
    ro.weight, ro.ids, ro.n_labels = label_W.contiguous(), None, int(label_W.shape[0])
    B = int(torch.as_tensor(last_idx).numel())
    ns = [int(n_opts)] * B if isinstance(n_opts, int) else [int(n) for n in n_opts]
    if len(ns) != B or any(n < 0 or n > ro.n_labels - 2 for n in ns):
        raise ValueError("n_opts must give 0 (No / Yes) or 1 .. L - 2 options for every request")
    lo = torch.tensor([0 if n == 0 else 2 for n in ns], dtype=torch.int32)
    cnt = [2 if n == 0 else n for n in ns]
    _, probs = ro(h, last_idx, norm_w, eps, offset, lo=lo, cnt=torch.tensor(cnt, dtype=torch.int32),
                  probs_width=max(cnt) if cnt else 0)
    return probs
