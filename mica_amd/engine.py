"""Last-position prefill engine with HIP-graph buckets.

The reference's PrefillEngine (v0.5/serving/lib/prefill_engine.py:171-418) runs a batch of requests
through the model and keeps only each request's last position for the label readout; request widths
are rounded up to a bucket, and each (bucket) shape is captured once as a CUDA graph and replayed with
the token ids and the last positions copied into the graph's static inputs (capture :370-389, replay
:391-409).  This engine does the same over ``mica_amd.model.W8A8Stack`` on HIP graphs
(torch.cuda.CUDAGraph on ROCm): requests are padded at the end to a common width (causal attention
keeps the padding out of every real position), packed [batch, width], and run by the stack's
``forward_last``; the readout reads row b * width + len_b - 1.

Prefix reuse (the reference's header, :214-268): ``PrefillEngine(stack, header=ids)`` runs the fixed
header once at construction (its first multiple of 64 tokens, ``model.PREFIX_ALIGN``) and keeps every
layer's state; a request that starts with those tokens then runs only its remaining tokens, continuing
the header's attention keys / values and GDN states, with the same bits as a full run.  A caller can
also pass any ``PrefixState`` (``stack.prefix_state``) that a batch of requests continues, e.g. the
shared start of several questions about one state; such batches run eagerly (graphs are captured for the
header and for no prefix only).
"""
from __future__ import annotations

import torch

from .model import PREFIX_ALIGN

BUCKET = 64          # width granularity (tokens)
GRAPH_MAX = 4096     # widest bucket that is captured; wider batches run eagerly
GRAPH_WARMUP = 2     # eager runs on a side stream before a capture (prefill_engine.py:375-378)


class _Graph:
    def __init__(self, batch, width, device):
        self.ids = torch.zeros(batch * width, dtype=torch.long, device=device)
        self.rows = torch.zeros(batch, dtype=torch.int32, device=device)
        self.lo = torch.zeros(batch, dtype=torch.int32, device=device)
        self.cnt = torch.ones(batch, dtype=torch.int32, device=device)
        self.graph = None
        self.out = None


class PrefillEngine:
    def __init__(self, stack, graph: bool = True, bucket: int = BUCKET, graph_max: int = GRAPH_MAX, header=None):
        self.stack = stack
        self.device = stack.device
        self.graph = bool(graph) and self.device.type == "cuda"
        self.bucket, self.graph_max = int(bucket), int(graph_max)
        self.graphs, self.pool, self.side = {}, None, None
        self.captures = 0
        self.header = None           # (token ids [Hc] on the device, PrefixState), Hc = aligned header length
        if header is not None:
            ids = torch.as_tensor(list(header), dtype=torch.long)
            hc = ids.numel() // PREFIX_ALIGN * PREFIX_ALIGN
            if hc:
                ids = ids[:hc].to(self.device)
                self.header = (ids, stack.prefix_state(ids))

    def header_hit(self, requests) -> bool:
        """Whether every request starts with the header's cached tokens and has at least one more."""
        if self.header is None:
            return False
        ids, st = self.header
        return all(r.numel() > st.length and torch.equal(r.reshape(-1)[:st.length], ids) for r in requests)

    def plan(self, lengths):
        """(batch, padded width, graphed) for requests of these lengths."""
        if not lengths or min(lengths) < 1:
            raise ValueError("every request needs at least one token")
        width = -(-max(lengths) // self.bucket) * self.bucket
        return len(lengths), width, self.graph and width <= self.graph_max

    def _pack(self, requests, width, out=None):
        ids = out if out is not None else torch.zeros(len(requests) * width, dtype=torch.long, device=self.device)
        ids.zero_()
        for b, r in enumerate(requests):
            ids[b * width:b * width + r.numel()].copy_(r.reshape(-1))
        return ids

    def _inputs(self, lengths, width, kinds, n_choices):
        rows = [b * width + n - 1 for b, n in enumerate(lengths)]
        lo, cnt = self.stack.slices(kinds, n_choices, len(lengths), "cpu")
        return torch.tensor(rows, dtype=torch.int32), lo, cnt

    @torch.no_grad()
    def run(self, requests, kinds=None, n_choices=None, prefix=None):
        """Eager: pack, run, read out.  Returns (logits [B, 2 + n_options], probs [B, n_options])."""
        lengths = [int(r.numel()) for r in requests]
        B, width, _ = self.plan(lengths)
        ids = self._pack(requests, width)
        rows, lo, cnt = (t.to(self.device) for t in self._inputs(lengths, width, kinds, n_choices))
        return self.stack.forward_last(ids, B, rows, lo, cnt, prefix=prefix)

    def capture(self, batch, width, prefix=None):
        g = _Graph(batch, width, self.device)
        g.prefix = prefix            # the graph reads the prefix's tensors on every replay
        g.rows.copy_(torch.arange(batch, dtype=torch.int32, device=self.device) * width + (width - 1))
        fn = lambda: self.stack.forward_last(g.ids, batch, g.rows, g.lo, g.cnt, prefix=prefix)  # noqa: E731
        if self.pool is None:
            self.pool = torch.cuda.graph_pool_handle()
        # one side stream for every warm-up and capture: the warm-ups give it the GEMM split workspace
        # (int8_kernels.gemm_workspace, per stream), which the captured GEMMs then use
        if self.side is None:
            self.side = torch.cuda.Stream(device=self.device)
        side = self.side
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(GRAPH_WARMUP):
                fn()
        torch.cuda.current_stream(self.device).wait_stream(side)
        g.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g.graph, pool=self.pool, stream=side), torch.no_grad():
            g.out = fn()
        self.graphs[batch, width, prefix is not None] = g
        self.captures += 1
        return g

    @torch.no_grad()
    def __call__(self, requests, kinds=None, n_choices=None, prefix=None):
        """Prefill `requests` (1-D int token-id tensors on the device) and return their last-position
        (logits, probs).  Graphed shapes return fresh copies of the graph's static outputs.  prefix: a
        PrefixState every request continues (the requests then hold only the tokens after it); without
        one, requests that all start with the engine's header continue the header's state."""
        if prefix is None and self.header_hit(requests):
            prefix = self.header[1]
            requests = [r.reshape(-1)[prefix.length:] for r in requests]
        lengths = [int(r.numel()) for r in requests]
        B, width, graphed = self.plan(lengths)
        header = self.header is not None and prefix is self.header[1]
        if not graphed or (prefix is not None and not header):
            return self.run(requests, kinds, n_choices, prefix)
        g = self.graphs.get((B, width, header)) or self.capture(B, width, prefix)
        self._pack(requests, width, g.ids)
        rows, lo, cnt = self._inputs(lengths, width, kinds, n_choices)
        g.rows.copy_(rows, non_blocking=False)
        g.lo.copy_(lo, non_blocking=False)
        g.cnt.copy_(cnt, non_blocking=False)
        g.graph.replay()
        return g.out[0].clone(), g.out[1].clone()
