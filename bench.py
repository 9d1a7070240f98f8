#!/usr/bin/env python3
"""Benchmark of the W8A8 linear-layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extra]

A step is one launch of the W8A8 GEMM at the headline 4B shape (M = T = 4096 tokens, K = 2560,
N = 9728, per-token x per-channel scale epilogue, bf16 out) on synthetic seeded inputs already
resident in HBM; `value` is its throughput in TOPS (2 M N K int8 ops per launch).  The JSON line
also carries the roofline of that kernel, the CPU baseline (the reference's CPU path: quant_act ->
torch._int_mm -> scale epilogue, timed on this host's cores) and, unless --no-extra, the other hot
path measurements: fused RMSNorm + quant GB/s (T = 4096, 32768), the GEMMs of the 4B layer and
the per-layer hot path in tokens/s.

Timing: W untimed warm-up launches, then exactly K launches bracketed by device synchronisation,
HIP events recorded on the stream the kernels run on (torch's current stream), average per launch.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "W8A8 GEMM TOPS (% INT8 peak) + prefill tokens/s, 4B shapes, T=4096"
PEAK_INT8_TOPS = 5000.0    # MI355X dense INT8 matrix peak, 5.0 POP/s (spec sheet; no sparsity)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, 8 TB/s
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak, 2.5 PFLOP/s
HIDDEN, INTER, QKV_N, O_K, LAYERS = 2560, 9728, 6144, 4096, 36


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # untimed launches before each timed block: after an idle host phase the first ~100 launches run
    # ~10 % slower (113.5 us steady vs ~125 us for the headline GEMM) while the clocks come back up
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="skip the 36-layer prefill measurement")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="only run the profiled kernels (headline GEMM, norm+quant T=32768, a 256 MiB copy) "
                         "for rocprofv3 counter passes")
    ap.add_argument("--summarize", nargs=2, metavar=("ROCPROF_DIR", "OUT_TXT"),
                    help="write a text summary of rocprofv3 CSV output (kernel stats or counters)")
    ap.add_argument("--command", default="", help="with --summarize: the command that produced ROCPROF_DIR")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="rebuild profiles/gemm_i8_m4096_n9728_k2560_traffic.json from a FETCH_SIZE and a WRITE_SIZE "
                         "pass of --pmc-workload (rocprofv3 output folders) and exit")
    return ap.parse_args()


def extra_warmup(args):
    """Untimed launches before each extra line's timed block: at least 100, so short kernels are timed
    at the clocks of a busy GPU (the headline's own warmup is exactly --warmup)."""
    return max(args.warmup, 100)


class Timer:
    """HIP events on the current stream around a block of launches."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # an untimed spin kernel ahead of the start event, long enough for the host to queue every timed
        # launch behind it: the events then bracket back-to-back GPU work, not the host's launch rate
        # (a 5 us kernel launched through ctypes otherwise waits on the host at the start of the block)
        torch.cuda._sleep(int(2e9 * 20e-6 * steps) + 1_000_000)
        s.record()
        for _ in range(steps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / steps  # ms per launch


def gemm_launcher(torch, lib, qx, sx, qw, sw, out, residual=None, epilogue=0, split=False):
    """A zero-allocation closure over the C ABI (what the drop-in mm_i8 calls, minus torch.empty)."""
    from mica_amd import int8_kernels

    M, K = qx.shape
    N = qw.shape[0]
    n_out = out.shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    ws, ws_bytes = int8_kernels.gemm_workspace(qx.device) if split else (None, 0)
    args = (qx.data_ptr(), K, qw.data_ptr(), K, sx.data_ptr(), sw.data_ptr(), None,
            None if residual is None else residual.data_ptr(), n_out, out.data_ptr(), n_out, 0, M, N, K, epilogue,
            ws, ws_bytes, stream)
    fn = lib.mica_mm_i8

    def launch():
        rc = fn(*args)
        if rc != 0:
            raise RuntimeError(f"mica_mm_i8 returned {rc}")
    return launch


def synthetic(torch, dev, M, K, N, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:8]] *= 20.0
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.empty(N).uniform_(1e-3, 1e-2, generator=g)
    return x.to(torch.bfloat16).to(dev), qw.to(dev), sw.to(dev)


def cpu_model() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_time(fn, budget_s, min_reps=3, max_reps=30):
    """Median wall time of fn after one warm-up, over at least min_reps runs or budget_s seconds."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(torch, M, K, N):
    """The reference's CPU path (oracle/cpu_path: its torch calls restated), timed on this host's cores:
    the headline W8A8 linear (the reported value), the eager RMSNorm of config 1 at T = 4096, and one
    36-layer-stack layer of config 4 at M = 16384 tokens (extrapolated to the stack).  About 20 s."""
    import math

    import torch.nn.functional as F

    from oracle import cpu_path

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1)

    def act(m, k):
        x = torch.randn(m, k, generator=g)
        x[:, torch.randperm(k, generator=g)[:8]] *= 20.0
        return x.to(torch.bfloat16)

    def weight(n, k):
        return torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8), \
            torch.empty(n).uniform_(1e-3, 1e-2, generator=g)

    x = act(M, K)
    qw, sw = weight(N, K)
    med, reps = _cpu_time(lambda: cpu_path.qlinear(x, qw, sw), 10.0)
    out = {
        "value": round(2.0 * M * N * K / med / 1e12, 4),
        "unit": "TOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"W8A8 linear M={M} K={K} N={N}: quant_act (round half even) + torch._int_mm + fp32 scale "
                   f"epilogue -> bf16 (oracle/cpu_path.qlinear), median of {reps} runs, {med * 1e3:.1f} ms"),
        "cpu_model": cpu_model(),
    }
    # config 1's eager RMSNorm (fused_kernels.py:51-56) + quant_act at T = 4096
    T = 4096
    h, nw = act(T, K), (torch.randn(K, generator=g) * 0.1 + 1.0).to(torch.bfloat16)
    med_n, reps_n = _cpu_time(lambda: cpu_path.rms_norm(h, nw, 1e-6, offset=0.0), 3.0)
    med_q, reps_q = _cpu_time(lambda: cpu_path.quant_act(cpu_path.rms_norm(h, nw, 1e-6, offset=0.0)), 3.0)
    nbytes = T * (2 * K + K + 4) + 2 * K
    out["rmsnorm_T4096"] = {"rmsnorm_ms": round(med_n * 1e3, 2), "rmsnorm_then_quant_ms": round(med_q * 1e3, 2),
                            "GB/s": round(nbytes / med_q / 1e9, 2),
                            "note": f"eager RMSNorm (cpu_path.rms_norm), then quant_act; medians of {reps_n} / {reps_q}"}
    # config 4: one layer of the 36-layer stack at M = 8 x 2048 tokens on the CPU path, attention (torch
    # SDPA in fp32, causal, 16 / 4 heads of 256, per request) timed once; the stack = 36 layers
    B, S, HQ, HK, D = 8, 2048, 16, 4, 256
    Mt = B * S
    hs = act(Mt, HIDDEN)
    w_in, w_post = nw, nw
    qkv_w, o_w = weight(QKV_N, HIDDEN), weight(HIDDEN, O_K)
    gate_w, up_w, down_w = weight(INTER, HIDDEN), weight(INTER, HIDDEN), weight(HIDDEN, INTER)
    t0 = time.perf_counter()
    y = cpu_path.rms_norm(hs, w_in, 1e-6, offset=0.0)
    qkv = cpu_path.qlinear(y, *qkv_w)
    t_qkv = time.perf_counter()
    q, k, v = qkv.view(B, S, HQ + 2 * HK, D).float().split((HQ, HK, HK), dim=2)
    a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True,
                                       scale=1 / math.sqrt(D), enable_gqa=True)
    a = a.transpose(1, 2).reshape(Mt, HQ * D).to(torch.bfloat16)
    t_att = time.perf_counter()
    h1 = hs + cpu_path.qlinear(a, *o_w)
    y2 = cpu_path.rms_norm(h1, w_post, 1e-6, offset=0.0)
    h2 = h1 + cpu_path.qlinear(cpu_path.swi_glu(cpu_path.qlinear(y2, *gate_w), cpu_path.qlinear(y2, *up_w)), *down_w)
    t1 = time.perf_counter()
    del h2
    linear_s = (t_qkv - t0) + (t1 - t_att)
    layer_s = t1 - t0
    out["c4_stack_extrapolated"] = {
        "layer_ms": round(layer_s * 1e3, 1), "layer_linear_ms": round(linear_s * 1e3, 1),
        "layer_attention_ms": round((t_att - t_qkv) * 1e3, 1),
        "ms_per_prefill": round(LAYERS * layer_s * 1e3, 1),
        "tokens_per_s": round(Mt / (LAYERS * layer_s), 1),
        "note": ("one layer of the 36-layer stack at 8 x 2048 tokens on the reference's CPU path (eager RMSNorm, "
                 "quant_act + torch._int_mm + epilogue per linear, F.silu(g) * u, fp32 SDPA per request), run "
                 "once; x 36 layers (extrapolated), readout excluded")}
    return out


TRAFFIC_JSON = ROOT / "profiles" / "gemm_i8_m4096_n9728_k2560_traffic.json"
GEMM_SOURCES = ("gemm_i8.hip", "gemm_i8_agpr.hip", "gemm_i8_wide.hip", "gemm_i8_common.h", "common.h")


def gemm_sources_digest() -> str:
    """First 16 hex digits of the SHA-256 over the GEMM kernels' sources: the traffic figure is valid for
    the kernels built from exactly these."""
    import hashlib
    h = hashlib.sha256()
    for name in GEMM_SOURCES:
        h.update((ROOT / "mica_amd" / "csrc" / name).read_bytes())
    return h.hexdigest()[:16]


def traffic_from_profiles():
    """(HBM bytes per headline GEMM launch, note) from the committed rocprofv3 counter passes
    (profiles/gemm_i8_m4096_n9728_k2560_traffic.json, written by --traffic); (None, why) when there is
    none or it was measured on other GEMM sources than the ones built here."""
    if not TRAFFIC_JSON.is_file():
        return None, "no traffic measurement committed"
    try:
        d = json.loads(TRAFFIC_JSON.read_text())
    except (ValueError, OSError) as ex:
        return None, f"traffic file unreadable: {ex}"[:120]
    if d.get("sources_sha16") != gemm_sources_digest():
        return None, "traffic measurement is of other GEMM sources (run the FETCH_SIZE / WRITE_SIZE passes and --traffic)"
    return d.get("hbm_bytes_per_launch"), ("traffic: " + TRAFFIC_JSON.relative_to(ROOT).as_posix() +
                                           ", rocprofv3 FETCH_SIZE + WRITE_SIZE passes over --pmc-workload, "
                                           "scaled by the 256 MiB copy's factors; sources " + d["sources_sha16"])


def write_traffic(fetch_dir, write_dir, commands=()):
    """Rebuild the traffic file from a FETCH_SIZE pass and a WRITE_SIZE pass of --pmc-workload (their
    rocprofv3 output folders): the headline GEMM's KiB per dispatch, scaled by the factors that make the
    256 MiB copy of the same run read and write 256 MiB, stamped with the GEMM sources' digest."""
    import csv
    import glob

    def per_run(folder, counter):
        f = sorted(glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True))[0]
        disp = {}
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == counter:
                disp[int(r["Dispatch_Id"])] = (r["Kernel_Name"], float(r["Counter_Value"]))
        runs, cur = [], None
        for i in sorted(disp):
            k, v = disp[i]
            if cur is not None and cur[0] == k:
                cur[1].append(v)
            else:
                cur = (k, [v])
                runs.append(cur)
        long_runs = [r for r in runs if len(r[1]) >= 20]
        if len(long_runs) != len(PMC_WORKLOADS):
            raise SystemExit(f"{folder}: {len(long_runs)} runs of 20 dispatches, expected {len(PMC_WORKLOADS)}")
        return {name: sum(v) / len(v) for name, (_, v) in zip(PMC_WORKLOADS, long_runs)}

    fetch, write = per_run(fetch_dir, "FETCH_SIZE"), per_run(write_dir, "WRITE_SIZE")
    copied = 256 << 20
    ff, wf = copied / (fetch["copy_256MiB"] * 1024), copied / (write["copy_256MiB"] * 1024)
    head = "gemm_headline_4096x9728x2560"
    fb, wb = fetch[head] * 1024 * ff, write[head] * 1024 * wf
    M, K, N = 4096, HIDDEN, INTER
    out = {"workload": "M=4096 K=2560 N=9728", "sources_sha16": gemm_sources_digest(), "commands": list(commands),
           "fetch_size_kib_per_dispatch": round(fetch[head], 1), "write_size_kib_per_dispatch": round(write[head], 1),
           "copy_calibration": {"bytes_copied": copied, "fetch_size_kib": round(fetch["copy_256MiB"], 1),
                                "write_size_kib": round(write["copy_256MiB"], 1), "fetch_factor": round(ff, 4),
                                "write_factor": round(wf, 4)},
           "fetch_bytes_per_launch": int(fb), "write_bytes_per_launch": int(wb), "hbm_bytes_per_launch": int(fb + wb),
           "algorithmic_bytes_per_launch": M * K + N * K + 2 * M * N + 4 * (M + N),
           "note": "FETCH_SIZE / WRITE_SIZE count L2 (TCC) traffic to the memory fabric; fetches served by the 256 MB "
                   "Infinity Cache are included, so this is an upper bound on HBM bytes."}
    TRAFFIC_JSON.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {TRAFFIC_JSON}: {out['hbm_bytes_per_launch']} bytes per launch", flush=True)


def main():
    args = parse()
    if args.summarize:
        summarize(*args.summarize, command=args.command)
        return
    if args.traffic:
        write_traffic(*args.traffic, commands=[c for c in args.command.split(" ;; ") if c])
        return
    if args.pmc_workload:
        pmc_workload()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the hot path is a single-GPU "
              f"kernel set; requests shard across GPUs as independent processes)", file=sys.stderr)
        sys.exit(2)
    import torch

    from mica_amd import _lib, fused_kernels, int8_kernels

    ok, why = int8_kernels.available("cuda")
    if not ok:
        raise SystemExit(f"mica_amd kernels unavailable: {why}")
    int8_kernels.STRICT = True
    dev = torch.device("cuda", torch.cuda.current_device())
    lib = _lib.load()
    info = _lib.device_info(dev.index)
    timer = Timer(torch)

    # ---- headline: the W8A8 GEMM at M=4096, K=2560, N=9728 -------------------------------------
    # (inputs here; its timed block runs last, after the other measurements' GPU work, so it is timed
    # at the clocks of a busy GPU rather than right after the idle host phase of the CPU baseline)
    M, K, N = 4096, HIDDEN, INTER
    x, qw, sw = synthetic(torch, dev, M, K, N, seed=0)
    qx, sx = int8_kernels.act_quant(x)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ops = 2.0 * M * N * K
    result = {"metric": METRIC}
    cpu = cpu_baseline(torch, M, K, N) if not args.no_cpu_baseline else None

    if not args.no_extra:
        extra = {"timing": "each line: at least 100 untimed launches, then an untimed spin kernel while the host queues "
                           "the timed block, then its timed block (HIP events); "
                           "cold-cache line: median of single launches after a 512 MiB fill"}
        # the headline GEMM with cold caches: before each launch a 512 MiB fill evicts the operands from
        # L2 and the 256 MB Infinity Cache; each launch is timed on its own (events around the GEMM only)
        flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        gemm = gemm_launcher(torch, lib, qx, sx, qw, sw, out)
        times = []
        for i in range(args.warmup + 20):
            flush.fill_(i & 0xff)
            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s_ev.record()
            gemm()
            e_ev.record()
            e_ev.synchronize()
            if i >= args.warmup:
                times.append(s_ev.elapsed_time(e_ev))
        del flush
        ms_c = statistics.median(times)
        extra["gemm_headline_cold_caches"] = {"us": round(ms_c * 1e3, 2), "TOPS": round(ops / (ms_c * 1e-3) / 1e12, 1),
                                              "pct_peak": round(100 * ops / (ms_c * 1e-3) / 1e12 / PEAK_INT8_TOPS, 1),
                                              "launches": len(times), "note": "median; 512 MiB fill before each"}
        # the same shape through ROCm's own int8 GEMM (torch._int_mm: int32 out, no scale epilogue), for
        # reference
        try:
            qwt = qw.t()
            ms_v = timer.run(lambda: torch._int_mm(qx, qwt), max(args.steps // 4, 10), extra_warmup(args))
            extra["vendor_int8_gemm_same_shape"] = {
                "us": round(ms_v * 1e3, 2), "TOPS": round(ops / (ms_v * 1e-3) / 1e12, 1),
                "note": "torch._int_mm(qx, qw.t()) on M=4096 K=2560 N=9728 (int32 out); the headline kernel "
                        "also applies the scale epilogue and writes bf16"}
        except RuntimeError as ex:
            extra["vendor_int8_gemm_same_shape"] = {"error": str(ex)[:160]}
        # fused RMSNorm + quant (config 1): T * (2K + K + 4) + 2K algorithmic bytes
        for T in (256, 4096, 32768):
            g = torch.Generator().manual_seed(T)
            h = torch.randn(T, K, generator=g)
            h[:, torch.randperm(K, generator=g)[:8]] *= 20
            h = h.to(torch.bfloat16).to(dev)
            w = (torch.randn(K, generator=g) * 0.1 + 1.0).to(torch.bfloat16).to(dev)
            q = torch.empty(T, K, dtype=torch.int8, device=dev)
            s = torch.empty(T, dtype=torch.float32, device=dev)
            stream = torch.cuda.current_stream().cuda_stream
            a = (h.data_ptr(), _lib.BF16, K, None, K, w.data_ptr(), _lib.BF16, 0.0, 1e-6, None, q.data_ptr(), K,
                 s.data_ptr(), None, K, None, K, T, K, 0, stream)

            def norm(a=a):
                if lib.mica_rmsnorm_quant(*a) != 0:
                    raise RuntimeError("mica_rmsnorm_quant failed")
            ms_n = timer.run(norm, max(args.steps, 50), extra_warmup(args))
            nbytes = T * (2 * K + K + 4) + 2 * K
            gbs = nbytes / (ms_n * 1e-3) / 1e9
            extra[f"rmsnorm_quant_T{T}"] = {"us": round(ms_n * 1e3, 2), "GB/s": round(gbs, 1),
                                           "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes}
            if T == 4096:
                # one norm for 3 consumers (the q / k / v pattern), unsmoothed and with SmoothQuant factors,
                # through the C ABI on preallocated outputs: T * (2K + 3 (K + 4)) + 2K (+ 3 * 4K) bytes
                import ctypes
                P = ctypes.c_void_p
                invs = [(torch.rand(K, generator=g) + 0.5).to(dev) for _ in range(3)]
                q3 = [torch.empty(T, K, dtype=torch.int8, device=dev) for _ in range(3)]
                s3 = [torch.empty(T, dtype=torch.float32, device=dev) for _ in range(3)]
                qp, sp = (P * 3)(*[t.data_ptr() for t in q3]), (P * 3)(*[t.data_ptr() for t in s3])
                ld3 = (ctypes.c_int * 3)(K, K, K)
                for tag, iv in (("", [None] * 3), ("_smoothed", [t.data_ptr() for t in invs])):
                    ivp = (P * 3)(*iv)
                    a3 = (h.data_ptr(), _lib.BF16, K, None, K, w.data_ptr(), _lib.BF16, 0.0, 1e-6, 3, ivp, qp, ld3, sp,
                          None, K, None, K, T, K, 0, stream)

                    def norm3(a3=a3):
                        if lib.mica_rmsnorm_quant_multi(*a3) != 0:
                            raise RuntimeError("mica_rmsnorm_quant_multi failed")
                    ms_3 = timer.run(norm3, 50, extra_warmup(args))
                    b3 = T * (2 * K + 3 * (K + 4)) + 2 * K + (12 * K if tag else 0)
                    extra[f"rmsnorm_quant_3consumers{tag}_T4096"] = {
                        "us": round(ms_3 * 1e3, 2), "GB/s": round(b3 / (ms_3 * 1e-3) / 1e9, 1),
                        "frac_hbm": round(b3 / (ms_3 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": b3}
        # the 4B layer's GEMMs at T = 4096 and the per-layer W8A8 hot path
        T = 4096
        layer = {}
        shapes = {"qkv": (QKV_N, HIDDEN), "o": (HIDDEN, O_K), "gate_up": (2 * INTER, HIDDEN), "down": (HIDDEN, INTER)}
        bufs = {}
        for name, (n, k) in shapes.items():
            xx, ww, ss = synthetic(torch, dev, T, k, n, seed=n + k)
            qa, sa = int8_kernels.act_quant(xx)
            epi = 1 if name == "gate_up" else 0
            o = torch.empty(T, n // 2 if epi else n, dtype=torch.bfloat16, device=dev)
            res = torch.randn(T, n, device=dev).to(torch.bfloat16) if name in ("o", "down") else None
            fn = gemm_launcher(torch, lib, qa, sa, ww, ss, o, residual=res, epilogue=epi)
            ms_g = timer.run(fn, max(args.steps // 4, 20), extra_warmup(args))
            t = 2.0 * T * n * k / (ms_g * 1e-3) / 1e12
            layer[name] = {"us": round(ms_g * 1e3, 2), "TOPS": round(t, 1), "pct_peak": round(100 * t / PEAK_INT8_TOPS, 1)}
            bufs[name] = (qa, sa, ww, ss, o, res, fn)
        # requant of h [T, 9728] between gate_up and down
        hh = bufs["gate_up"][4]
        qh = torch.empty(T, INTER, dtype=torch.int8, device=dev)
        sh = torch.empty(T, dtype=torch.float32, device=dev)
        st = torch.cuda.current_stream().cuda_stream
        ra = (hh.data_ptr(), _lib.BF16, INTER, None, qh.data_ptr(), INTER, sh.data_ptr(), T, INTER, 0, st)

        def requant():
            if lib.mica_act_quant(*ra) != 0:
                raise RuntimeError("mica_act_quant failed")
        ms_r = timer.run(requant, 50, extra_warmup(args))
        rbytes = T * (2 * INTER + INTER + 4)
        layer["requant_h"] = {"us": round(ms_r * 1e3, 2), "GB/s": round(rbytes / (ms_r * 1e-3) / 1e9, 1)}
        ms_norm = extra["rmsnorm_quant_T4096"]["us"] / 1e3
        per_layer_ms = 2 * ms_norm + ms_r + sum(layer[k]["us"] for k in shapes) / 1e3
        layer["hot_path_us_per_layer"] = round(per_layer_ms * 1e3, 1)
        layer["hot_path_tokens_per_s_36_layers"] = round(T / (LAYERS * per_layer_ms * 1e-3), 1)
        layer["note"] = ("per 4B layer at T=4096: 2 fused RMSNorm+quant, QKV, O(+residual), fused gate+up with SiLU "
                         "epilogue, requant of h, down(+residual); attention (a torch op) not included")
        extra["layer_T4096"] = layer
        # config 2's gated MLP block at T = 4096: fused gate+up (SiLU epilogue), requant of h, down + residual
        blk_us = layer["gate_up"]["us"] + layer["requant_h"]["us"] + layer["down"]["us"]
        blk_ops = 2.0 * T * (2 * INTER) * HIDDEN + 2.0 * T * HIDDEN * INTER
        extra["c2_gated_mlp_T4096"] = {"us": round(blk_us, 2), "TOPS": round(blk_ops / (blk_us * 1e-6) / 1e12, 1),
                                       "frac_int8_peak": round(blk_ops / (blk_us * 1e-6) / 1e12 / PEAK_INT8_TOPS, 4),
                                       "note": "sum of the three launches' times (gate_up, requant_h, down)"}
        # config 0 (one W8A8 linear on 512 tokens) and config 3 (T = 32768 projections), GEMM launches alone
        for tag, (m, n, k) in (("gemm_c0_512x2560x9728", (512, INTER, HIDDEN)),
                               ("gemm_c3_qkv_32768x2560x6144", (32768, QKV_N, HIDDEN)),
                               ("gemm_c3_o_32768x4096x2560", (32768, HIDDEN, O_K))):
            xx, ww, ss = synthetic(torch, dev, m, k, n, seed=m + n + k)
            qa, sa = int8_kernels.act_quant(xx)
            o = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            ms_g = timer.run(gemm_launcher(torch, lib, qa, sa, ww, ss, o), max(args.steps // 4, 20), extra_warmup(args))
            t = 2.0 * m * n * k / (ms_g * 1e-3) / 1e12
            extra[tag] = {"us": round(ms_g * 1e3, 2), "TOPS": round(t, 1), "frac_int8_peak": round(t / PEAK_INT8_TOPS, 4),
                          "M": m, "K": k, "N": n}
            del xx, ww, ss, qa, sa, o
        extra["gdn_8x2048"] = gdn_token_mixer(torch, dev, timer, args)
        extra["attention_8x2048"] = attention_extra(torch, dev, timer, args)
        result["extra"] = extra
        result["prefill_tokens_per_s"] = layer["hot_path_tokens_per_s_36_layers"]

    if not args.no_stack:
        result["stack"] = stack_prefill(torch, dev)
        result["stack_hybrid"] = hybrid_prefill(torch, dev)
        result["prefill_tokens_per_s"] = result["stack"]["tokens_per_s"]
    ms = timer.run(gemm_launcher(torch, lib, qx, sx, qw, sw, out), args.steps, args.warmup)
    tops = ops / (ms * 1e-3) / 1e12
    traffic, traffic_note = traffic_from_profiles()
    head = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded: X bf16 ~N(0,1) with 8 outlier channels x20, quantized per token; "
                "W int8 uniform [-127,127], per-channel scales ~U(1e-3,1e-2))",
        "config": {"workload": "W8A8 GEMM M=4096 K=2560 N=9728 (4B MLP projection at T=4096), int8 x int8 -> "
                               "int32 on MFMA, per-token x per-channel scale epilogue, bf16 out",
                   "M": M, "K": K, "N": N, "T": M, "parallelism": "none (1 GPU)",
                   "timing": "HIP events around the K timed launches, after the W warmup launches and an untimed "
                             "spin kernel that lets the host queue them; measured after the other lines of this run "
                             "(GPU clocks of a busy GPU)"},
        "pct_int8_peak": round(100.0 * tops / PEAK_INT8_TOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(tops / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "note": "INT8 TOP/s (2 M N K per launch / mean launch time); peak = MI355X dense INT8 5.0 "
                             "POP/s; " + traffic_note},
        "device": {**info, "derived_int8_peak_tops": round(info["cu_count"] * info["clock_khz"] * 1e3 * 8192 / 1e12,
                                                           1)},
    }
    result.pop("metric")
    head.update(result)
    if cpu is not None:
        head["cpu_baseline"] = cpu
    print(json.dumps(head), flush=True)


def gdn_token_mixer(torch, dev, timer, args):
    """The GDN layer's token mixer of the 4B model (16 key / 32 value heads of 128, conv width 4) on
    8 sequences x 2048 tokens: conv + SiLU + q/k l2norm over the 8192 projected channels, the chunked
    gated delta rule (prep + scan), and the gated RMSNorm fused with out_proj's int8 quantisation.
    Algorithmic bytes count each input read once and each output written once; the scan's flops are
    the chunked form's matrix products (11.5 MFLOP per 64-token chunk and value head)."""
    from mica_amd import gdn

    B, T, HK, HV, D = 8, 2048, 16, 32, 128
    C = 2 * HK * D + HV * D
    g = torch.Generator(device=dev).manual_seed(7)
    mixed = torch.randn(B, T, C, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(C, 4, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    conv = gdn.causal_conv1d_fn(mixed.transpose(1, 2), w, activation="silu", l2norm_heads=2 * HK).transpose(1, 2)
    q = conv[..., :HK * D].unflatten(-1, (HK, D))
    k = conv[..., HK * D:2 * HK * D].unflatten(-1, (HK, D))
    v = conv[..., 2 * HK * D:].unflatten(-1, (HV, D))
    gg = -torch.rand(B, T, HV, device=dev, generator=g) * 0.5
    beta = torch.rand(B, T, HV, device=dev, generator=g).to(torch.bfloat16)
    z = torch.randn(B * T, HV * D, device=dev, generator=g).to(torch.bfloat16)
    nw = torch.ones(D, device=dev, dtype=torch.bfloat16)
    out = {}
    steps = max(args.steps // 10, 10)
    ms = timer.run(lambda: gdn.causal_conv1d_fn(mixed.transpose(1, 2), w, activation="silu", l2norm_heads=2 * HK),
                   steps, extra_warmup(args))
    nb = 2 * B * T * C * 2 + C * 4 * 2
    out["conv_silu_l2norm"] = {"us": round(ms * 1e3, 1), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                               "frac_hbm": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": nb}
    ms = timer.run(lambda: gdn.chunk_gated_delta_rule(q, k, v, gg, beta, output_final_state=True), steps,
                   extra_warmup(args))
    flops = 11.5e6 * B * HV * (T // 64)
    nb = B * T * (2 * HK * D * 2 + 2 * HV * D * 2 + HV * 6) + B * HV * D * D * 4
    out["chunk_gated_delta_rule"] = {"us": round(ms * 1e3, 1), "Mtokens/s": round(B * T / (ms * 1e-3) / 1e6, 2),
                                     "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                                     "frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                     "GB/s": round(nb / (ms * 1e-3) / 1e9, 1), "flops": flops, "bytes": nb}
    ms = timer.run(lambda: gdn.gated_rmsnorm_quant(v.reshape(B * T, HV * D), z, nw), steps, extra_warmup(args))
    nb = B * T * HV * D * 5 + B * T * 4 + D * 2
    out["gated_rmsnorm_quant"] = {"us": round(ms * 1e3, 1), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                                  "frac_hbm": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": nb}
    out["token_mixer_us"] = round(sum(x["us"] for x in out.values()), 1)
    out["note"] = ("8 x 2048 tokens, 16 key / 32 value heads of 128; excludes the in/out projections (W8A8 "
                   "GEMMs); chunk_gated_delta_rule = prep (chunk-parallel WY) + scan (sequential) kernels")
    return out


def attention_extra(torch, dev, timer, args):
    """Causal GQA attention of the full-attention layers (16 query / 4 K/V heads of 256) on 8 x 2048
    tokens, q / k / v as views of one fused QKV buffer: the flash-attention kernel against torch SDPA
    on the same views.  FLOPs: 4 B HQ D S^2 / 2 (the causal half of QK^T and PV)."""
    import math

    import torch.nn.functional as F

    from mica_amd.attention import causal_gqa_attention

    B, S, HQ, HK, D = 8, 2048, 16, 4, 256
    g = torch.Generator(device=dev).manual_seed(11)
    qkv = torch.randn(B * S, (HQ + 2 * HK) * D, device=dev, generator=g).to(torch.bfloat16)
    q, k, v = qkv.view(B, S, HQ + 2 * HK, D).split((HQ, HK, HK), dim=2)
    flops = 4.0 * B * HQ * D * S * S / 2
    steps = max(args.steps // 20, 5)
    ms = timer.run(lambda: causal_gqa_attention(q, k, v), steps, extra_warmup(args))
    ms_ref = timer.run(lambda: F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                                              is_causal=True, scale=1 / math.sqrt(D), enable_gqa=True),
                       steps, extra_warmup(args))
    t = flops / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 1), "TFLOP/s": round(t, 1), "frac_bf16_peak": round(t / PEAK_BF16_TFLOPS, 4),
            "sdpa_us": round(ms_ref * 1e3, 1), "speedup_vs_sdpa": round(ms_ref / ms, 2), "flops": flops}


def stack_prefill(torch, dev, reps=3):
    """Config 4: the 36-layer 4B-shaped W8A8 stack on 8 requests x 2048 packed tokens, readout of 255
    option ids at each request's last position.  Attention (16 query / 4 K/V heads of 256) runs on the
    flash-attention kernel; RoPE on the in-place kernel."""
    from mica_amd.model import StackConfig, W8A8Stack

    st = W8A8Stack(StackConfig(), device=dev, seed=0)
    B, S = 8, 2048
    ids = torch.randint(0, st.cfg.vocab, (B * S,), generator=torch.Generator().manual_seed(0)).to(dev)
    st.prefill(ids, B)  # warm-up
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        _, probs = st.prefill(ids, B)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    ops = st.linear_ops_per_token() * B * S
    ok = bool(torch.isfinite(probs).all()) and bool(torch.allclose(probs.sum(1), torch.ones(B, device=dev)))
    engine = engine_latency(torch, dev, st)
    engine["serve_8_questions_8k_state"] = serving_latency(torch, dev, st)
    del st
    torch.cuda.empty_cache()
    return {"workload": "36 layers, hidden 2560, inter 9728, QKV 6144 (16 / 4 heads of 256), vocab 151936; "
                        "8 requests x 2048 tokens packed; last-position readout over 255 option ids + softmax",
            "ms_per_prefill": round(ms, 2), "tokens_per_s": round(B * S / (ms * 1e-3), 1),
            "w8a8_linear_TOP": round(ops / 1e12, 2), "linear_TOPS_incl_attention_time": round(ops / (ms * 1e-3) / 1e12, 1),
            "probs_valid": ok, "reps": reps, "engine": engine}


def hybrid_prefill(torch, dev, reps=3):
    """The reference model's hybrid layout and attention at the same shape (StackConfig.reference_model):
    32 layers, every fourth full attention (16 / 4 heads of 256 with the q_proj output gate, per-head
    q / k RMSNorm and RoPE on 64 dims: QKV N = 10240) and the other 24 gated-delta-net layers (16 key /
    32 value heads of 128: W8A8 input projections 8192 + 4096 + 32 + 32, conv, chunked scan, gated norm
    + quant, W8A8 out_proj), each followed by the same W8A8 MLP; 8 requests x 2048 tokens, last-position
    readout (last layer last-only)."""
    from mica_amd.model import StackConfig, W8A8Stack

    st = W8A8Stack(StackConfig.reference_model(), device=dev, seed=0)
    B, S = 8, 2048
    ids = torch.randint(0, st.cfg.vocab, (B * S,), generator=torch.Generator().manual_seed(0)).to(dev)
    st.prefill(ids, B)  # warm-up
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        _, probs = st.prefill(ids, B)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    ops = st.linear_ops_per_token() * B * S
    ok = bool(torch.isfinite(probs).all()) and bool(torch.allclose(probs.sum(1), torch.ones(B, device=dev)))
    # single requests (the GDN scan then has one workgroup per value head: 32)
    single = {}
    g = torch.Generator().manual_seed(6)
    for S1 in (512, 4096):
        ids1 = torch.randint(0, st.cfg.vocab, (S1,), generator=g).to(dev)
        st.prefill(ids1, 1)
        torch.cuda.synchronize()
        s.record()
        for _ in range(reps):
            st.prefill(ids1, 1)
        e.record()
        torch.cuda.synchronize()
        ms1 = s.elapsed_time(e) / reps
        single[f"B1_S{S1}"] = {"ms": round(ms1, 2), "tokens_per_s": round(S1 / (ms1 * 1e-3), 1)}
    del st
    torch.cuda.empty_cache()
    return {"workload": "32 layers (24 gated-delta-net + 8 full attention with output gate, q / k head norm and "
                        "RoPE on 64 dims), hidden 2560, inter 9728; 8 requests x 2048 tokens packed; "
                        "last-position readout over 255 option ids + softmax",
            "ms_per_prefill": round(ms, 2), "tokens_per_s": round(B * S / (ms * 1e-3), 1),
            "w8a8_linear_TOP": round(ops / 1e12, 2), "probs_valid": ok, "reps": reps, "single_request": single}


def engine_latency(torch, dev, st, reps=5):
    """The prefill engine (HIP-graph buckets, mica_amd.engine) on the 36-layer stack: per-call time of
    one 128-token and one 512-token request (~430 launches each) and of 8 x 2048 tokens, eager vs a
    replayed graph (inputs copied in, outputs copied out)."""
    from mica_amd.engine import PrefillEngine

    out = {}
    g = torch.Generator().manual_seed(5)
    for B, S in ((1, 128), (1, 512), (8, 2048)):
        reqs = [torch.randint(0, st.cfg.vocab, (S,), generator=g).to(dev) for _ in range(B)]
        for mode in ("eager", "graph"):
            eng = PrefillEngine(st, graph=mode == "graph")
            eng(reqs)
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(reps):
                eng(reqs)
            e.record()
            torch.cuda.synchronize()
            ms = s.elapsed_time(e) / reps
            out[f"{mode}_B{B}_S{S}"] = {"ms": round(ms, 3), "tokens_per_s": round(B * S / (ms * 1e-3), 1)}
            del eng
    torch.cuda.empty_cache()
    return out


def serving_latency(torch, dev, st, reps=3):
    """One /v1/systemone request end to end on the 36-layer stack (mica_amd.contract.answer: validation,
    prompts, tokens, engine, typed answers): 8 questions (Noul, Choice, Score) about one synthetic state
    of ~8 K tokens (UTF-8 bytes as tokens), with the prompts' common start run once (share_prefix) and
    with every prompt run in full; the shared start also with the continuations' attention split over
    the prefix keys (W8A8Stack.split_keys).  Wall time per request, host work included."""
    from mica_amd import contract
    from mica_amd.engine import PrefillEngine

    state = " ".join(f"record {i}: value {i * 37 % 101}, status {'open' if i % 3 else 'closed'}." for i in range(220))
    qs = {}
    for i in range(8):
        kind = ("noul", "choice", "score")[i % 3]
        q = {"type": kind, "instructions": f"Question {i}: what does record {i * 11} say?"}
        if kind == "choice":
            q["criteria"] = {f"c{j}": f"value {j * 10}" for j in range(6)}
        elif kind == "score":
            q["criteria"] = ["low", "medium", "high", "very high"]
        qs[f"q{i}"] = q
    req = {"state": state, "questions": qs}
    out = {}
    for share, split in ((True, False), (True, True), (False, False)):
        st.split_keys = split  # the continuations' attention over the prefix keys split over workgroups
        judge = contract.EngineJudge(PrefillEngine(st, graph=False), lambda t: list(t.encode("utf-8")),
                                     share_prefix=share)
        resp = contract.answer(req, judge)   # warm-up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            resp = contract.answer(req, judge)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / reps * 1e3
        out[("shared_prefix_split_keys" if split else "shared_prefix") if share else "full_prompts"] = {
            "ms": round(ms, 1), "prompt_tokens": sum(len(t) for t in judge.last_prompts),
            "tokens_run": sum(len(t) for t in judge.last_prompts) - judge.shared_tokens,
            "answers": len(resp["answers"])}
        del judge
    st.split_keys = False
    torch.cuda.empty_cache()
    return out


# the --pmc-workload runs, in launch order, 20 back-to-back launches each (the counter summaries label
# the runs of >= 20 dispatches of one kernel with these names, in this order)
PMC_WORKLOADS = (
    "gemm_headline_4096x9728x2560", "gemm_qkv_4096x6144x2560", "gemm_o_residual_4096x2560x4096",
    "gemm_gate_up_silu_4096x19456x2560", "gemm_down_residual_4096x2560x9728", "gemm_c0_512x9728x2560",
    "gemm_c3_qkv_32768x6144x2560", "gemm_c3_o_32768x2560x4096", "rmsnorm_quant_T4096", "rmsnorm_quant_T32768",
    "rmsnorm_quant_3consumers_smoothed_T4096", "act_quant_h_4096x9728", "copy_256MiB",
)


def pmc_workload():
    """The kernels the committed counter summaries describe (PMC_WORKLOADS), each launched 20 times."""
    import torch

    from mica_amd import _lib, int8_kernels

    dev = torch.device("cuda", torch.cuda.current_device())
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    T = 4096
    x, _, _ = synthetic(torch, dev, T, HIDDEN, 16, seed=0)
    qx, sx = int8_kernels.act_quant(x)
    h = torch.randn(T, INTER, device=dev).to(torch.bfloat16)
    qh, sh = int8_kernels.act_quant(h)
    a4 = torch.randn(T, O_K, device=dev).to(torch.bfloat16)
    qa, sa = int8_kernels.act_quant(a4)
    res = torch.randn(T, HIDDEN, device=dev).to(torch.bfloat16)

    def gemm(n, k, qa_, sa_, epilogue=0, residual=None):
        g = torch.Generator(device="cpu").manual_seed(n + k)
        qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
        sw = torch.empty(n).uniform_(1e-3, 1e-2, generator=g).to(dev)
        out = torch.empty(qa_.shape[0], n // 2 if epilogue else n, dtype=torch.bfloat16, device=dev)
        return gemm_launcher(torch, lib, qa_, sa_, qw, sw, out, residual=residual, epilogue=epilogue)

    def activations(m, k, seed):
        xx, _, _ = synthetic(torch, dev, m, k, 16, seed=seed)
        return int8_kernels.act_quant(xx)

    def norm3_smoothed(rows):
        import ctypes
        P = ctypes.c_void_p
        g = torch.Generator().manual_seed(rows)
        hx = torch.randn(rows, HIDDEN, device=dev).to(torch.bfloat16)
        w = torch.ones(HIDDEN, device=dev).to(torch.bfloat16)
        invs = [(torch.rand(HIDDEN, generator=g) + 0.5).to(dev) for _ in range(3)]
        q3 = [torch.empty(rows, HIDDEN, dtype=torch.int8, device=dev) for _ in range(3)]
        s3 = [torch.empty(rows, dtype=torch.float32, device=dev) for _ in range(3)]
        keep = (hx, w, invs, q3, s3)
        ivp, qp = (P * 3)(*[t.data_ptr() for t in invs]), (P * 3)(*[t.data_ptr() for t in q3])
        sp, ld3 = (P * 3)(*[t.data_ptr() for t in s3]), (ctypes.c_int * 3)(HIDDEN, HIDDEN, HIDDEN)
        args = (hx.data_ptr(), _lib.BF16, HIDDEN, None, HIDDEN, w.data_ptr(), _lib.BF16, 0.0, 1e-6, 3, ivp, qp, ld3,
                sp, None, HIDDEN, None, HIDDEN, rows, HIDDEN, 0, st)

        def run(keep=keep):
            if lib.mica_rmsnorm_quant_multi(*args) != 0:
                raise RuntimeError("mica_rmsnorm_quant_multi failed")
        return run

    def norm(rows):
        hx = torch.randn(rows, HIDDEN, device=dev).to(torch.bfloat16)
        w = torch.ones(HIDDEN, device=dev).to(torch.bfloat16)
        q = torch.empty(rows, HIDDEN, dtype=torch.int8, device=dev)
        s = torch.empty(rows, dtype=torch.float32, device=dev)
        args = (hx.data_ptr(), _lib.BF16, HIDDEN, None, HIDDEN, w.data_ptr(), _lib.BF16, 0.0, 1e-6, None,
                q.data_ptr(), HIDDEN, s.data_ptr(), None, HIDDEN, None, HIDDEN, rows, HIDDEN, 0, st)

        def run():
            if lib.mica_rmsnorm_quant(*args) != 0:
                raise RuntimeError("mica_rmsnorm_quant failed")
        return run

    qo = torch.empty(T, INTER, dtype=torch.int8, device=dev)
    so = torch.empty(T, dtype=torch.float32, device=dev)
    rq = (h.data_ptr(), _lib.BF16, INTER, None, qo.data_ptr(), INTER, so.data_ptr(), T, INTER, 0, st)

    def requant():
        if lib.mica_act_quant(*rq) != 0:
            raise RuntimeError("mica_act_quant failed")

    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    runs = {
        "gemm_headline_4096x9728x2560": gemm(INTER, HIDDEN, qx, sx),
        "gemm_qkv_4096x6144x2560": gemm(QKV_N, HIDDEN, qx, sx),
        "gemm_o_residual_4096x2560x4096": gemm(HIDDEN, O_K, qa, sa, residual=res),
        "gemm_gate_up_silu_4096x19456x2560": gemm(2 * INTER, HIDDEN, qx, sx, epilogue=1),
        "gemm_down_residual_4096x2560x9728": gemm(HIDDEN, INTER, qh, sh, residual=res),
        "gemm_c0_512x9728x2560": gemm(INTER, HIDDEN, *activations(512, HIDDEN, 1)),
        "gemm_c3_qkv_32768x6144x2560": gemm(QKV_N, HIDDEN, *activations(32768, HIDDEN, 2)),
        "gemm_c3_o_32768x2560x4096": gemm(HIDDEN, O_K, *activations(32768, O_K, 3)),
        "rmsnorm_quant_3consumers_smoothed_T4096": norm3_smoothed(4096),
        "rmsnorm_quant_T4096": norm(4096),
        "rmsnorm_quant_T32768": norm(32768),
        "act_quant_h_4096x9728": requant,
        # 256 MiB read + 256 MiB written: the calibration of FETCH_SIZE / WRITE_SIZE
        "copy_256MiB": lambda: dst.copy_(src),
    }
    marker = torch.zeros(1, device=dev)
    torch.cuda.synchronize()
    for name in PMC_WORKLOADS:
        marker.fill_(1.0)  # one other kernel between two runs, so that runs of the same kernel stay apart
        for _ in range(20):
            runs[name]()
        torch.cuda.synchronize()
    print("pmc workload done", flush=True)


def summarize(indir, out_txt, command="", top=16):
    """Text summary of rocprofv3 CSV output: kernel time statistics (--stats), per-dispatch durations
    by launch shape (--kernel-trace) and/or per-dispatch counter means (--pmc), top entries only.
    FETCH_SIZE / WRITE_SIZE are also converted to bytes with the factors that make the 256 MiB copy
    of the --pmc-workload read and write exactly 256 MiB."""
    import csv
    import glob
    from collections import defaultdict

    lines = [f"# rocprofv3 summary of {indir}"]
    if command:
        lines.append(f"# command: {command}")
    stats = sorted(glob.glob(os.path.join(indir, "**", "*kernel_stats.csv"), recursive=True))
    for f in stats:
        rows = list(csv.DictReader(open(f)))
        lines.append(f"# kernel statistics ({os.path.basename(f)})")
        lines.append(f"{'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'pct':>6}  kernel")
        for r in rows[:top]:
            name = r["Name"]
            lines.append(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} {float(r['MinNs']) / 1e3:10.2f} "
                         f"{float(r['MaxNs']) / 1e3:10.2f} {float(r['Percentage']):6.2f}  {name[:150]}")
    traces = sorted(glob.glob(os.path.join(indir, "**", "*kernel_trace.csv"), recursive=True))
    for f in traces:
        groups = defaultdict(list)
        rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Start_Timestamp"]))
        for r in rows:
            grid = (int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
            groups[(r["Kernel_Name"][:150], grid)].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        # runs of >= 20 back-to-back dispatches of one kernel and launch shape, in launch order (a
        # timed loop of the bench is one such run: its warm-up launches, then its timed launches)
        runs, cur = [], None
        for r in rows:
            key = (r["Kernel_Name"][:150], int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
            d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            if cur is not None and cur[0] == key:
                cur[1].append(d)
            else:
                cur = (key, [d])
                runs.append(cur)
        lines.append(f"# runs of >= 20 back-to-back dispatches, in launch order ({os.path.basename(f)})")
        lines.append(f"{'run':>4} {'calls':>6} {'avg_us':>10} {'avg_last':>10} {'avg_end50':>10} {'min_us':>10} "
                     f"{'max_us':>10} {'grid':>9}  kernel  (avg_last: all calls but the first 20; avg_end50: the "
                     f"last 50 calls, the timed ones of a --steps 50 run)")
        for i, (key, v) in enumerate(r_ for r_ in runs if len(r_[1]) >= 20):
            tail = v[20:] if len(v) > 20 else v
            end = v[-50:]
            lines.append(f"{i:4d} {len(v):6d} {sum(v) / len(v) / 1e3:10.2f} {sum(tail) / len(tail) / 1e3:10.2f} "
                         f"{sum(end) / len(end) / 1e3:10.2f} {min(v) / 1e3:10.2f} {max(v) / 1e3:10.2f} {key[1]:9d}  {key[0]}")
        lines.append(f"# per-dispatch durations by kernel and launch shape ({os.path.basename(f)})")
        lines.append(f"{'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'grid':>9} {'wg':>5}  kernel")
        for (k, (gx, wx)), v in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
            lines.append(f"{len(v):6d} {sum(v) / len(v) / 1e3:10.2f} {min(v) / 1e3:10.2f} {max(v) / 1e3:10.2f} "
                         f"{gx:9d} {wx:5d}  {k}")
    pmc = sorted(glob.glob(os.path.join(indir, "**", "*counter_collection.csv"), recursive=True))
    for f in pmc:
        # dispatches in launch order; runs of >= 20 back-to-back dispatches of one kernel are the
        # --pmc-workload's runs, labelled with PMC_WORKLOADS in order (other kernels keep their names)
        disp = {}
        for r in csv.DictReader(open(f)):
            d = disp.setdefault(int(r["Dispatch_Id"]), {"kernel": r["Kernel_Name"][:150], "c": {}})
            d["c"][r["Counter_Name"]] = float(r["Counter_Value"])
        order = [disp[i] for i in sorted(disp)]
        runs, cur = [], None
        for d in order:
            if cur is not None and cur[0] == d["kernel"]:
                cur[1].append(d)
            else:
                cur = (d["kernel"], [d])
                runs.append(cur)
        long_runs = [r_ for r_ in runs if len(r_[1]) >= 20]
        labels = {}
        if len(long_runs) == len(PMC_WORKLOADS):
            for (k, ds), name in zip(long_runs, PMC_WORKLOADS):
                for d in ds:
                    labels[id(d)] = f"[{name}] {k}"
        agg = defaultdict(list)
        for d in order:
            key = labels.get(id(d), d["kernel"])
            for c, v in d["c"].items():
                agg[(key, c)].append(v)
        lines.append(f"# counters per dispatch, mean over dispatches ({os.path.basename(f)})")
        for (k, c), v in sorted(agg.items()):
            lines.append(f"{c:28s} {sum(v) / len(v):16.1f}  n={len(v):3d}  {k}")
        labelled = any(k.startswith("[copy_256MiB]") for k, _ in agg)
        copy = {c: sum(v) / len(v) for (k, c), v in agg.items()
                if (k.startswith("[copy_256MiB]") if labelled else ("copyBuffer" in k or "copy_kernel" in k))
                and c in ("FETCH_SIZE", "WRITE_SIZE") and sum(v) > 0}
        for c, kib in copy.items():
            factor = (256 << 20) / (kib * 1024.0)
            lines.append(f"# calibration: the 256 MiB copy (256 MiB read, 256 MiB written) counts {c} = {kib:.1f} KiB "
                         f"-> bytes = KiB x 1024 x {factor:.4f}")
            for (k, c2), v in sorted(agg.items()):
                if c2 == c and "copyBuffer" not in k and not k.startswith("[copy_256MiB]"):
                    lines.append(f"{c2 + '_bytes':28s} {sum(v) / len(v) * 1024.0 * factor:16.0f}  {k}")
        # derived figures per kernel.  GRBM_GUI_ACTIVE comes summed over the XCCs; rocprofv3's own
        # MfmaUtil divides the SIMD-summed MFMA busy cycles by the per-XCC active cycles x SIMD count
        simds, xccs = 1024, 8  # MI355X, unless the run's agent info says otherwise
        for ai in glob.glob(os.path.join(os.path.dirname(f), "*agent_info.csv")):
            for a in csv.DictReader(open(ai)):
                if a.get("Name", "").startswith("gfx"):
                    simds, xccs = int(a["Simd_Count"]), int(a["Num_Xcc"])
        per = defaultdict(dict)
        for (k, c), v in agg.items():
            per[k][c] = sum(v) / len(v)
        for k, d in sorted(per.items()):
            if "SQ_VALU_MFMA_BUSY_CYCLES" in d and d.get("GRBM_GUI_ACTIVE"):
                util = 100.0 * d["SQ_VALU_MFMA_BUSY_CYCLES"] / (d["GRBM_GUI_ACTIVE"] / xccs * simds)
                lines.append(f"{'MFMA_util_pct':28s} {util:16.2f}  (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / "
                             f"{xccs} XCCs x {simds} SIMDs), rocprofv3's MfmaUtil)  {k}")
            if "SQ_INSTS_VALU_MFMA_MOPS_I8" in d:
                lines.append(f"{'int8_ops_per_dispatch':28s} {d['SQ_INSTS_VALU_MFMA_MOPS_I8'] * 512:16.4g}"
                             f"  (SQ_INSTS_VALU_MFMA_MOPS_I8 x 512)  {k}")
            if "SQ_LDS_BANK_CONFLICT" in d and d.get("SQ_LDS_IDX_ACTIVE"):
                active = d["SQ_LDS_IDX_ACTIVE"] - d["SQ_LDS_BANK_CONFLICT"]
                lines.append(f"{'LDS_conflict_per_access':28s} {d['SQ_LDS_BANK_CONFLICT'] / max(active, 1.0):16.4f}"
                             f"  (SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT))  {k}")
    with open(out_txt, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print(f"wrote {out_txt} ({len(lines)} lines)")


if __name__ == "__main__":
    main()
