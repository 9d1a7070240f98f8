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
