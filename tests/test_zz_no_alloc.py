"""mica_mm_i8_noalloc (the GEMM entry point that allocates nothing: its split schedule's workspace is a
static device array of the library) against mica_mm_i8 with a workspace, both called through the C ABI.

Bar: bit-identical outputs (int8 x int8 -> int32 accumulators, then the same epilogue).  Two calls in a
row, the second smaller, so the shared scratch's arrival counters must come back to zero after each
launch; a split round larger than the scratch is rejected with MICA_MISS_RANGE."""
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from mica_amd import _lib, int8_kernels
from oracle import w8a8 as O

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def _operands(rng, m, n, k, dev):
    A = torch.from_numpy(rng.integers(-127, 128, (m, k), dtype=np.int8)).to(dev)
    B = torch.from_numpy(rng.integers(-127, 128, (n, k), dtype=np.int8)).to(dev)
    sa = torch.from_numpy(rng.uniform(1e-3, 1e-2, m).astype(np.float32)).to(dev)
    sb = torch.from_numpy(rng.uniform(1e-3, 1e-2, n).astype(np.float32)).to(dev)
    return A, B, sa, sb


def _call(noalloc, A, B, sa, sb, out, out_code, epi_code, residual=None):
    L = _lib.load()
    m, k = A.shape
    n = B.shape[0]
    n_out = out.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    res = None if residual is None else residual.data_ptr()
    args = (A.data_ptr(), k, B.data_ptr(), k, sa.data_ptr(), sb.data_ptr(), None, res, n_out, out.data_ptr(), n_out,
            out_code, m, n, k, epi_code)
    if noalloc:
        return L.mica_mm_i8_noalloc(*args, stream)
    ws, ws_bytes = int8_kernels.gemm_workspace(A.device)
    return L.mica_mm_i8(*args, ws, ws_bytes, stream)


def _both(A, B, sa, sb, dtype, epi_code, n_out, residual=None):
    code = {torch.bfloat16: _lib.BF16, torch.int32: _lib.INT32}[dtype]
    outs = []
    for noalloc in (False, True):
        out = torch.full((A.shape[0], n_out), -1, dtype=dtype, device=A.device)  # no stale zeros
        rc = _call(noalloc, A, B, sa, sb, out, code, epi_code, residual)
        assert rc == 0, f"{'mica_mm_i8_noalloc' if noalloc else 'mica_mm_i8'} returned {rc} ({_lib.status_name(rc)})"
        outs.append(out)
    torch.cuda.synchronize()
    return outs


def _same(a, b, what):
    ab, bb = a.view(torch.int16) if a.dtype == torch.bfloat16 else a, b.view(torch.int16) if b.dtype == torch.bfloat16 else b
    diff = (ab != bb).sum().item()
    assert diff == 0, f"{what}: {diff} of {a.numel()} outputs differ between mica_mm_i8_noalloc and mica_mm_i8"


def test_scratch_size_is_stated(gpu):
    assert _lib.load().mica_mm_i8_noalloc_scratch_bytes() == 4096 + 64 * 2 * 256 * 1024


@pytest.mark.parametrize("calls", [
    # (m, n, k, epilogue) per call; the second call of each pair is smaller
    # split rounds of 10 then 5 tiles of 256 x 256 (int32), 32 then 8 of 128 x 160 in 3 parts (bf16)
    ((256, 2560, 9728, "scale"), (128, 1280, 8192, "scale")),
    # SiLU epilogue: 16 then 4 tiles of 128 x 256 in 3 parts
    ((200, 2048, 8192, "silu_mul"), (64, 1024, 8192, "silu_mul")),
    # no split (K below both thresholds): quarter / half tiles
    ((512, 2560, 4096, "scale"), (300, 1000, 2576, "scale")),
])
def test_noalloc_matches_mica_mm_i8_twice(gpu, calls):
    rng = np.random.default_rng(7)
    for i, (m, n, k, epi) in enumerate(calls):
        note(f"noalloc call {i}: m={m} n={n} k={k} epi={epi}")
        A, B, sa, sb = _operands(rng, m, n, k, gpu)
        if epi == "silu_mul":
            a, b = _both(A, B, sa, sb, torch.bfloat16, _lib.EPI_SILU_MUL, n // 2)
            _same(a, b, f"silu call {i}")
            continue
        a, b = _both(A, B, sa, sb, torch.int32, _lib.EPI_SCALE, n)
        _same(a, b, f"int32 call {i}")
        rows = np.unique(np.r_[0, m - 1, rng.integers(0, m, 6)])   # noalloc's accumulators against the oracle
        want = O.int_gemm(A.cpu().numpy()[rows], B.cpu().numpy())
        assert np.array_equal(b.cpu().numpy()[rows], want), f"int32 call {i}: noalloc differs from the oracle"
        res = torch.randn(m, n, device=gpu).to(torch.bfloat16)
        a, b = _both(A, B, sa, sb, torch.bfloat16, _lib.EPI_SCALE, n, residual=res)
        _same(a, b, f"bf16 + residual call {i}")


def test_noalloc_rejects_a_split_round_beyond_the_scratch(gpu):
    """17 tiles of 256 x 256 with int32 outputs at K = 8192, M <= 256 would split over 68 workgroups:
    more than the scratch holds."""
    note("noalloc reject m=200 n=4352 k=8192 int32")
    rng = np.random.default_rng(3)
    A, B, sa, sb = _operands(rng, 200, 4352, 8192, gpu)
    out = torch.empty((200, 4352), dtype=torch.int32, device=gpu)
    assert _call(True, A, B, sa, sb, out, _lib.INT32, _lib.EPI_SCALE) == 5  # MICA_MISS_RANGE
    # the existing entry point serves it (its workspace is sized for every CU)
    assert _call(False, A, B, sa, sb, out, _lib.INT32, _lib.EPI_SCALE) == 0
    torch.cuda.synchronize()


def _capture_child():
    """Run in a fresh process: the process's first mica_mm_i8_noalloc calls are made inside a HIP-graph
    capture (torch.cuda.graph) on a split shape, so the scratch lookup and its counter clear happen
    under capture.  The graph is replayed three times, with eager work and synchronisation between the
    replays, and every replay is compared with eager mica_mm_i8 (own workspace) and, for the int32
    accumulators, with the oracle on sampled rows.  Prints one JSON line."""
    dev = torch.device("cuda", 0)
    L = _lib.load()
    rng = np.random.default_rng(21)
    m, n, k = 256, 2560, 9728                    # split: 10 tiles of 256 x 256 (int32), 32 of 128 x 160 (bf16)
    A, B, sa, sb = _operands(rng, m, n, k, dev)
    eager_i32 = torch.empty((m, n), dtype=torch.int32, device=dev)
    eager_bf16 = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    assert _call(False, A, B, sa, sb, eager_i32, _lib.INT32, _lib.EPI_SCALE) == 0
    assert _call(False, A, B, sa, sb, eager_bf16, _lib.BF16, _lib.EPI_SCALE) == 0
    out_i32 = torch.full((m, n), -1, dtype=torch.int32, device=dev)
    out_bf16 = torch.full((m, n), -1, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = [_call(True, A, B, sa, sb, out_i32, _lib.INT32, _lib.EPI_SCALE),
              _call(True, A, B, sa, sb, out_bf16, _lib.BF16, _lib.EPI_SCALE)]
    result = {"rc": rc, "replays": []}
    rows = np.unique(np.r_[0, m - 1, rng.integers(0, m, 6)])
    want = O.int_gemm(A.cpu().numpy()[rows], B.cpu().numpy())
    for r in range(3):
        out_i32.fill_(-1)
        out_bf16.fill_(-1)
        (A.float() @ B[:64].float().t().contiguous()).sum().item()   # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        result["replays"].append({
            "int32_differs": int((out_i32 != eager_i32).sum().item()),
            "bf16_differs": int((out_bf16.view(torch.int16) != eager_bf16.view(torch.int16)).sum().item()),
            "oracle_rows_equal": bool(np.array_equal(out_i32.cpu().numpy()[rows], want)),
        })
    print(json.dumps(result), flush=True)


def test_noalloc_first_call_under_graph_capture(gpu):
    """A caller under HIP-graph capture whose first noalloc call is the captured one (see _capture_child)."""
    note("noalloc first call inside graph capture: m=256 n=2560 k=9728, child process")
    here = Path(__file__).resolve().parent
    code = f"import sys; sys.path[:0] = [{str(here.parent)!r}, {str(here)!r}]; import test_zz_no_alloc as t; t._capture_child()"
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240,
                          env=dict(os.environ), cwd=str(here.parent))
    assert proc.returncode == 0, proc.stderr[-3000:]
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    assert r["rc"] == [0, 0], r
    assert len(r["replays"]) == 3
    for i, rep in enumerate(r["replays"]):
        assert rep == {"int32_differs": 0, "bf16_differs": 0, "oracle_rows_equal": True}, (i, r)
