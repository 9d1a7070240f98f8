"""Host-side bookkeeping of the layer stack, on the CPU: the RoPE table that grows by doubling (a
continuation's rows must equal a full run's, and a table a graph may hold is never freed) and the
continuation positions a PrefixState keeps."""
import types

import torch

from mica_amd.model import PrefixState, StackConfig, W8A8Stack, _rope


def _holder():
    return types.SimpleNamespace(cfg=StackConfig(head_dim=256), _rope=None, _retired=[])


def test_rope_table_grows_by_doubling_and_keeps_rows():
    st = _holder()
    cos, sin = W8A8Stack._tables(st, 100, "cpu")
    assert cos.shape == (100, 128) and cos.is_contiguous() and st._rope[0].shape[0] == 4096
    first = st._rope
    cos2, sin2 = W8A8Stack._tables(st, 5000, "cpu")         # regrow: 2 x 4096
    assert st._rope[0].shape[0] == 8192 and st._retired == [first]
    assert torch.equal(cos2[:100], cos) and torch.equal(sin2[:100], sin)
    c3, s3 = W8A8Stack._tables(st, 9000, "cpu")              # doubled again: 16384 rows
    assert st._rope[0].shape[0] == 16384 and len(st._retired) == 2
    # every row equals a table built for exactly that many positions
    cf, sf = _rope(9000, 256, st.cfg.rope_theta, "cpu")
    assert torch.equal(c3, cf) and torch.equal(s3, sf)
    W8A8Stack._tables(st, 40000, "cpu")                      # beyond twice: exactly what is asked
    assert st._rope[0].shape[0] == 40000 and len(st._retired) == 3


def test_prefix_positions_are_not_kept_for_eager_runs():
    """Positions of an eager continuation are made per call: serving many request lengths eagerly does
    not grow the prefix's memory (only shapes captured in a HIP graph are kept)."""
    pre = PrefixState(128, [])
    p = pre.positions_for(3, 64, "cpu")
    assert p.dtype == torch.int32 and p.numel() == 3 * 64
    assert torch.equal(p.view(3, 64), (torch.arange(64) + 128).int().expand(3, 64))
    for S in range(1, 300):
        pre.positions_for(2, S, "cpu")
    assert pre.positions == {}
    pre.positions[(3, 64)] = p                                 # a captured shape: served from the cache
    assert pre.positions_for(3, 64, "cpu") is p
