"""The HIP-graph prefill engine (mica_amd.engine) against eager execution and against running each
request alone.  A graph is replayed several times with other eager work and synchronisations in
between, and every replay must give the eager result bit for bit (integer GEMMs, per-row norms and
quantisers, causal attention that keeps the end padding out of every real position)."""
import sys

import pytest
import torch

from mica_amd.engine import PrefillEngine
from mica_amd.model import StackConfig, W8A8Stack

pytestmark = pytest.mark.gpu


def _stack(gpu, hybrid=False):
    cfg = StackConfig(layers=2, hidden=512, intermediate=1024, heads=4, kv_heads=1, head_dim=256, vocab=4096,
                      n_options=31, full_attention_interval=2 if hybrid else 0, linear_k_heads=2,
                      linear_v_heads=4)
    return W8A8Stack(cfg, device=gpu, seed=7)


@pytest.mark.parametrize("hybrid", [False, True])
def test_graph_replays_match_eager_and_single_requests(gpu, hybrid):
    """hybrid: a gated-delta-net layer then an attention layer (conv, gate, chunked scan and gated
    norm inside the graph; the GDN recurrence is causal, so end padding leaves real positions alone)."""
    print(f"[case] engine graph vs eager hybrid={hybrid}", file=sys.stderr, flush=True)
    st = _stack(gpu, hybrid)
    g = torch.Generator().manual_seed(3)
    lens = [37, 64, 5]
    reqs = [torch.randint(0, st.cfg.vocab, (n,), generator=g).to(gpu) for n in lens]
    kinds, nch = ["choice", "noul", "choice"], [31, 2, 9]
    eager = PrefillEngine(st, graph=False)
    ref_logits, ref_probs = eager(reqs, kinds, nch)
    torch.cuda.synchronize()
    eng = PrefillEngine(st, graph=True)
    other = [torch.randint(0, st.cfg.vocab, (100,), generator=g).to(gpu)]
    for rep in range(3):
        logits, probs = eng(reqs, kinds, nch)
        torch.cuda.synchronize()
        assert torch.equal(logits, ref_logits), rep
        assert torch.equal(probs, ref_probs), rep
        eager(other)                      # eager work of another shape between replays
        torch.cuda.synchronize()
    assert eng.captures == 1
    # each request alone (no padding, batch 1) gives the same last-position logits
    for b, r in enumerate(reqs):
        lo, pr = st.prefill(r, 1, kinds=[kinds[b]], n_choices=[nch[b]])
        torch.cuda.synchronize()
        assert torch.equal(lo[0], ref_logits[b]), b
        assert torch.allclose(pr[0], ref_probs[b], atol=0, rtol=0), b


def test_engine_shape_buckets(gpu):
    st = _stack(gpu)
    eng = PrefillEngine(st, graph=True, bucket=64, graph_max=128)
    assert eng.plan([1, 64]) == (2, 64, True)
    assert eng.plan([65]) == (1, 128, True)
    assert eng.plan([129]) == (1, 192, False)   # wider than graph_max: eager
    with pytest.raises(ValueError):
        eng.plan([])


@pytest.mark.parametrize("hybrid", [False, True])
def test_prefix_continuation_is_bit_identical(gpu, hybrid):
    """A prompt continued from the PrefixState of its first P tokens (P a multiple of 64) gives the
    full run's logits and probabilities bit for bit: attention over the prefix's rotated keys and
    values plus its own, GDN conv and recurrent states carried over; a batch of different
    continuations shares one prefix state."""
    print(f"[case] prefix continuation hybrid={hybrid}", file=sys.stderr, flush=True)
    st = _stack(gpu, hybrid)
    g = torch.Generator().manual_seed(5)
    P = 128
    head = torch.randint(0, st.cfg.vocab, (P,), generator=g)
    tails = [torch.randint(0, st.cfg.vocab, (n,), generator=g) for n in (5, 64, 100)]
    kinds, nch = ["choice", "noul", "choice"], [31, 2, 7]
    full = [torch.cat((head, t)).to(gpu) for t in tails]
    pre = st.prefix_state(head.to(gpu))
    assert pre.length == P
    eager = PrefillEngine(st, graph=False)
    ref = [eager([f], [k], [n]) for f, k, n in zip(full, kinds, nch)]
    got = eager([t.to(gpu) for t in tails], kinds, nch, prefix=pre)
    torch.cuda.synchronize()
    for b in range(3):
        assert torch.equal(got[0][b], ref[b][0][0]), b
        assert torch.equal(got[1][b], ref[b][1][0]), b


def test_header_engine_graphs_match_full_runs(gpu):
    """PrefillEngine(header=...) keeps the header's first multiple of 64 tokens as a prefix state;
    requests that start with it run only the rest, captured in a graph and replayed with eager work
    in between, and give the same bits as full eager runs."""
    print("[case] header engine graphs", file=sys.stderr, flush=True)
    st = _stack(gpu, hybrid=True)
    g = torch.Generator().manual_seed(9)
    header = torch.randint(0, st.cfg.vocab, (150,), generator=g)   # 128 tokens cached, 22 run per request
    reqs = [torch.cat((header, torch.randint(0, st.cfg.vocab, (n,), generator=g))).to(gpu) for n in (3, 40, 77)]
    kinds, nch = ["noul", "choice", "choice"], [2, 31, 12]
    plain = PrefillEngine(st, graph=False)
    ref = plain(reqs, kinds, nch)
    eng = PrefillEngine(st, graph=True, header=header.tolist())
    assert eng.header[1].length == 128 and eng.header_hit(reqs)
    other = [torch.randint(0, st.cfg.vocab, (70,), generator=g).to(gpu)]   # no header: a full run
    assert not eng.header_hit(other)
    for rep in range(3):
        out = eng(reqs, kinds, nch)
        torch.cuda.synchronize()
        assert torch.equal(out[0], ref[0]) and torch.equal(out[1], ref[1]), rep
        o2 = eng(other)
        torch.cuda.synchronize()
        assert torch.equal(o2[0], plain(other)[0]), rep
    assert eng.captures == 2      # one graph continuing the header, one without
