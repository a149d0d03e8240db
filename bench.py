#!/usr/bin/env python3
"""Benchmark of the W4A16 decode GEMV on one MI355X.

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50] [--configs all|c0,c3,...]

Metric: HBM read GB/s and % of the measured read roof of the
W4A16 GEMV at M=4096, K=4096, B=1, with p50 latency. One "step" is one GEMV
launch over packed weights resident in HBM. `--warmup` untimed steps run
first; then exactly `--steps` steps run back-to-back, captured in one HIP
graph, step i reading weight copy i mod n where the n copies total more than
640 MB, as in a decode pass over many layers. Each step's output is released
when the next step's is kept (the caching allocator hands the block back, as
it does in a decode loop and in the reference's timing loop); only the last
one is held, to check the replays against an eager launch. Before each of 5 timed replays
a 1 GiB read is enqueued on the same stream, outside the events: it flushes
the L2s and the 256 MB Infinity Cache, so every replay starts cold whatever
--steps is. The timed span is bracketed inside the graph on the GPU's own
clock: after one untimed lead-in step, a timestamp kernel (s_memrealtime,
100 MHz), the `--steps` steps, a second timestamp kernel; the bracket's own
cost, measured by a graph of the two timestamps alone, is subtracted. So the
span holds exactly the timed steps and not the fixed start cost of a graph
launch, which is reported as `graph_replay_overhead_us` (events around the
whole replay: `p50_us_outer`). Per-step time = span / steps, p50 over the 5
replays. `value` = algorithmic bytes / p50 per-step time.

The reference's protocol (a cache flush, then events around one call,
bench/common.py:64-108) is reported beside it: on MI355X the event markers
alone cost ~6 us, more than this GEMV, so it measures the timer.

Also reported on the same line: the read roof (best 1 GiB STREAM read), the
copy roof, the read floor (the fastest launch shape of a kernel that only
reads the headline's bytes), the empty-kernel timing floors, every kernel
variant at the headline shape, the other four configurations, a roofline
object for the headline kernel (named by dk_gemv_describe), the fp16 GEMM
ridge point, and the CPU baseline: the reference's CPU path (fp32
dequantize + F.linear, python/decode_kernel/reference.py:17-26) in torch on
this host's cores.

Prints exactly one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "decode-kernel_amd"))
sys.path.insert(0, str(REPO))

METRIC = "HBM read GB/s & % of measured read roof, W4A16 GEMV 4096x4096 B=1; p50 us"

# name -> (M, K, batches, variants timed). The headline is c0 B=1 with the
# default op (v5). Seeds follow the config index.
CONFIGS = {
    "c0": (4096, 4096, [1], ["v5", "v0", "v1", "v1_wpr2", "v1_wpr4", "v2", "v3", "v4", "reuse",
                             "v5_paired"]),
    "c1": (11008, 4096, [1], ["v5", "v4", "reuse", "v5_paired"]),
    "c2": (4096, 11008, [1], ["v5", "v4", "reuse", "v5_paired"]),
    "c3": (4096, 4096, [1, 2, 4, 8, 16, 32, 48, 64, 128, 256], ["reuse", "v5", "v4"]),
    "c4a": (28672, 8192, [1], ["v5", "v4", "reuse", "v5_paired"]),
    "c4b": (8192, 28672, [1], ["v5", "v4", "reuse", "v5_paired"]),
}
# c3 beyond the BASELINE batches: the reference's own sweep continues to
# B = 256 (bench/bench.py:36, 261-264); there only the reuse path (the
# batch op, w4a16_linear's choice) and the fp16 baseline are timed.
C3_BASELINE_BATCHES = (1, 2, 4, 8, 16)
# The margin over the B = 1 time that names c3's crossover batch.
C3_CROSSOVER_MARGIN = 0.25
VARIANTS = {
    "v0": dict(version=0), "v1": dict(version=1), "v1_wpr2": dict(version=1, warps_per_row=2),
    "v1_wpr4": dict(version=1, warps_per_row=4), "v2": dict(version=2), "v3": dict(version=3),
    "v4": dict(version=4, split_k=4), "v5": dict(version=5),
    "reuse": dict(version=5, reuse_weights=True),
    "v5_paired": None,  # the v5 GEMV on weights repacked into the paired layout
}
EXPECTED_STAMP = {"v0": 0, "v1": 1, "v1_wpr2": 12, "v1_wpr4": 14, "v2": 2, "v3": 3, "v4": 4,
                  "v5": 5, "reuse": 15, "v5_paired": 25}
PROFILE_TRAFFIC = REPO / "profiles" / "traffic_c0_gemv_v5_lds.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--configs", default="all",
                    help="comma list of c0,c1,c2,c3,c4a,c4b or 'all' (c0 is always run)")
    ap.add_argument("--other-steps", type=int, default=None,
                    help="timed steps per variant outside the headline (default: --steps)")
    ap.add_argument("--flush", choices=["read", "write", "none"], default="read")
    ap.add_argument("--flush-bytes", type=int, default=1 << 30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-quantizer", action="store_true",
                    help="skip the device quantizer measurement")
    ap.add_argument("--no-mlp", action="store_true", help="skip the MLP decode step measurement")
    ap.add_argument("--no-fp16-baseline", action="store_true",
                    help="skip the cross-precision torch fp16 F.linear rows")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="budget of the CPU baseline sample")
    ap.add_argument("--out", type=Path, default=None, help="also write the full JSON here")
    return ap.parse_args()


def make_inputs(m, k, batch, seed):
    """Synthetic inputs: W ~ N(0, 0.02) fp32, x ~ N(0,1) fp16 (PCG64), quantized
    on the CPU by the package's quantizer, then copied to HBM."""
    import torch

    from decode_kernel.quantize import quantize_and_pack
    from dk_bench.common import synthetic_case

    w, x = synthetic_case(m, k, batch, seed)
    packed, scales = quantize_and_pack(torch.from_numpy(w))
    del w
    return (packed.cuda(), scales.cuda(), torch.from_numpy(x).cuda(), packed, scales, x)


class LastOutput:
    """Keeps only the latest step's output. Holding all `steps` outputs of a
    graph would make every step write fresh pages (at B >= 4 on 4096 x 4096,
    0.2 us per step); a decode loop, like the reference's timing loop, writes
    into the block its previous output freed."""

    def __init__(self):
        self.y = None

    def __call__(self, y):
        self.y = y


def bench_variant(ext, copies, x, variant, steps, flush, warmup=1, y_ref=None,
                  call_level_flush=None):
    """Exactly `steps` launches of one variant back-to-back (HIP graph), step
    i on weight copy i mod len(copies), after `warmup` untimed launches and a
    1 GiB pre-roll per replay, so every step reads cold weights."""
    from dk_bench.common import bytes_moved_w4, flop_gemv, time_gpu, time_graph_steps

    pk, sc = copies
    kw = VARIANTS[variant]
    if variant == "v5_paired":
        pk = [ext.repack_paired(p) for p in pk]

        def call(p, s, xx):
            return ext.w4a16_gemv_paired(p, s, xx)
    else:
        def call(p, s, xx):
            return ext.w4a16_gemv(p, s, xx, **kw)
    y0 = call(pk[0], sc[0], x)
    stamp = int(ext.last_kernel_stamp())
    if stamp != EXPECTED_STAMP[variant]:
        raise RuntimeError(f"{variant}: dispatch stamp {stamp}, expected {EXPECTED_STAMP[variant]}")
    if y_ref is not None and not torch_equal(y0, y_ref):
        raise RuntimeError(f"{variant}: output differs from the checked headline output")
    n = len(pk)
    last = LastOutput()
    st, graph = time_graph_steps(lambda i: last(call(pk[i % n], sc[i % n], x)), steps=steps,
                                 warmup=warmup, preroll=flush)
    # Every replayed step recomputes the same product: the last one must equal
    # the eager result bit for bit (graph replays checked against eager work).
    if not torch_equal(last.y, y0):
        raise RuntimeError(f"{variant}: graph replay output differs from the eager launch")
    del graph, last
    m, k, b = pk[0].shape[0], pk[0].shape[1] * 8, x.shape[0]
    moved = bytes_moved_w4(m, k, b)
    row = {
        "impl": variant, "stamp": stamp, "bytes_moved": moved, "weight_copies": n,
        "gbps": moved / (st["median_us"] * 1e3),
        "gbps_mean": moved / (st["mean_us"] * 1e3),
        "tflops": flop_gemv(m, k, b) / (st["median_us"] * 1e-6) / 1e12,
        **st,
    }
    if call_level_flush is not None:
        from decode_kernel import gemv

        ev = time_gpu(lambda: gemv(pk[0], sc[0], x, **kw), warmup=20, iters=300,
                      flush=call_level_flush)
        row["call_events"] = {k2: ev[k2] for k2 in ("median_us", "iqr_us", "mean_us", "iters")}
    return row


def bench_torch_fp16(pd, sd, x, steps, flush):
    """Cross-precision baseline (labelled as such, as the reference's bench
    does, bench/bench.py:1-9): torch F.linear on the dequantized weights in
    fp16 (hipBLASLt/rocBLAS), back-to-back over weight copies totalling
    > 640 MB. It moves 4x the weight bytes of the W4A16 kernel."""
    import torch

    from decode_kernel import dequantize
    from dk_bench.common import bytes_moved_fp16, time_graph_steps

    w16 = dequantize(pd, sd, dtype=torch.float16)
    n = max(2, (640 << 20) // (w16.numel() * 2) + 1)
    ws = [w16] + [w16.clone() for _ in range(n - 1)]
    st, graph = time_graph_steps(lambda i: torch.nn.functional.linear(x, ws[i % n]), steps=steps,
                                 preroll=flush)
    del graph, ws, w16
    m, k, b = pd.shape[0], pd.shape[1] * 8, x.shape[0]
    moved = bytes_moved_fp16(m, k, b)
    return {"impl": "torch_fp16_linear", "precision": "fp16",
            "note": "fp16 weights (cross-precision baseline)",
            "bytes_moved": moved, "gbps": moved / (st["median_us"] * 1e3), "weight_copies": n,
            **st}


def torch_equal(a, b) -> bool:
    import torch

    return bool(torch.equal(a, b))


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _timed_calls(fn, budget_s, max_calls):
    fn()  # warm: page in, thread pools
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end and len(times) < max_calls:
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) / 1e3)
    times.sort()
    return times


def cpu_baseline(packed, scales, x, budget_s):
    """The reference's CPU path, restated in torch as decode_kernel.reference
    (python/decode_kernel/reference.py:17-26: fp32 dequantize, then F.linear)
    on this host with torch's intra-op threads set to the cores this process
    may use (capped by OMP_NUM_THREADS, the box's CPU share), for a bounded
    number of calls. Labelled extras: the fp32 GEMM alone with W dequantized
    beforehand, and the oracle's numpy port (single-threaded unpack)."""
    import numpy as np
    import torch

    from decode_kernel.reference import linear_fp32
    from dk_bench.common import bytes_moved_w4
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    threads = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores) or cores))
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        xt = torch.from_numpy(np.asarray(x))
        times = _timed_calls(lambda: linear_fp32(xt, packed, scales), budget_s, 400)
        from decode_kernel.quantize import dequantize

        w32 = dequantize(packed, scales, dtype=torch.float32)
        x32 = xt.float()
        mm = _timed_calls(lambda: torch.nn.functional.linear(x32, w32), min(5.0, budget_s / 3), 2000)
        del w32
    finally:
        torch.set_num_threads(prev_threads)
    p, s, xv = packed.numpy(), scales.numpy(), np.asarray(x)
    port = _timed_calls(lambda: oracle.linear_fp32(xv, p, s), min(5.0, budget_s / 3), 50)
    m, k, b = p.shape[0], p.shape[1] * 8, xv.shape[0]
    moved = bytes_moved_w4(m, k, b)
    med = times[len(times) // 2]
    return {
        "value": moved / (med * 1e3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"c0 M={m} K={k} B={b}: {len(times)} calls of decode_kernel.reference."
                   f"linear_fp32 (torch fp32 dequantize + F.linear, the reference's CPU path "
                   f"reference.py:17-26) with torch.set_num_threads({threads}), median of "
                   f"~{budget_s:.0f} s"),
        "p50_us": med, "iqr_us": times[(3 * len(times)) // 4] - times[len(times) // 4],
        "calls": len(times), "torch_threads": threads, "host_cpus": cores,
        "cpu_model": _cpu_model(),
        "matmul_only": {"p50_us": mm[len(mm) // 2], "calls": len(mm), "torch_threads": threads,
                        "note": "F.linear with W dequantized beforehand (not the reference path)"},
        "numpy_port": {"p50_us": port[len(port) // 2], "calls": len(port),
                       "note": "oracle.linear_fp32: numpy unpack single-threaded, BLAS sgemv"},
    }


def bench_quantizer(roof_gbps, cpu_seconds):
    """The device quantizer (dk_quantize_pack_f32) at the largest weight,
    c4a 28672 x 8192 (235 M weights, 940 MB fp32 read per launch, more than
    the Infinity Cache holds), checked bit-for-bit against the torch
    formulation on the same GPU before it is timed. The oracle's numpy
    quantizer is timed beside it on a bounded row sample on this host."""
    import numpy as np
    import torch

    from decode_kernel import _cuda
    from decode_kernel.quantize import quantize_and_pack_torch
    from dk_bench.common import time_repeated
    from oracle import oracle

    m, k = 28672, 8192
    gen = torch.Generator(device="cuda").manual_seed(3000)
    w = torch.randn(m, k, device="cuda", generator=gen) * 0.02
    packed, scales = _cuda.quantize_and_pack(w)
    tp, ts = quantize_and_pack_torch(w)
    if not (torch.equal(packed, tp) and torch.equal(scales.view(torch.int16), ts.view(torch.int16))):
        raise RuntimeError("device quantizer differs from the torch formulation at c4a")
    del tp, ts
    st = time_repeated(lambda: _cuda.quantize_and_pack(w), reps=20)
    moved = m * k * 4 + m * k // 2 + (m * k // 128) * 2
    out = {
        "shape": [m, k], "bytes_moved": moved, "p50_us": st["median_us"], "iqr_us": st["iqr_us"],
        "gbps": moved / (st["median_us"] * 1e3), "weights_per_s": m * k / (st["median_us"] * 1e-6),
        "timer": "events around 20 back-to-back launches, p50 of 5 trials",
    }
    out["pct_of_read_roof"] = 100.0 * out["gbps"] / roof_gbps
    rows = 1024
    wc = w[:rows].cpu().numpy()
    del w, packed, scales
    torch.cuda.empty_cache()
    oracle.quantize_and_pack(wc)
    times = []
    t_end = time.perf_counter() + cpu_seconds
    while time.perf_counter() < t_end and len(times) < 50:
        t0 = time.perf_counter_ns()
        oracle.quantize_and_pack(wc)
        times.append((time.perf_counter_ns() - t0) / 1e9)
    times.sort()
    med = times[len(times) // 2]
    out["cpu_baseline"] = {
        "weights_per_s": rows * k / med, "kind": "port", "cores": 1,
        "sample": f"oracle.quantize_and_pack (numpy) on {rows} rows of c4a, median of {len(times)}",
        "seconds_for_c4a_extrapolated": m * k / (rows * k / med),
    }
    return out


MLP_SHAPES = {
    "llama7b": (11008, 4096),
    "llama70b_tp8": (3584, 8192),
    "llama70b": (28672, 8192),
}


MLP_BATCHES = (1, 8)


def bench_mlp(roof_gbps, steps, flush=None):
    """One MLP decode step (gate/up fused with SiLU*mul, then the down GEMV)
    per shape at B = 1 and B = 8, back-to-back in a HIP graph over weight
    copies that total > 640 MB (cold weights), against the unfused
    composition a caller writes with the GEMV (w4a16_linear's choice of
    path: the reuse path for a batch): three GEMVs and a SiLU*mul between
    them. Keys: the shape name at B = 1, name_bB for a batch."""
    import torch

    from decode_kernel import gate_up_silu, gemv, mlp_decode, quantize_and_pack
    from dk_bench.common import mlp_bytes, time_graph_steps

    out = {}
    for name, (i, h) in MLP_SHAPES.items():
        gen = torch.Generator(device="cuda").manual_seed(4000 + i)
        one = []
        for shape in ((i, h), (i, h), (h, i)):
            one += list(quantize_and_pack(torch.randn(*shape, device="cuda", generator=gen) * 0.02))
        nbytes = sum(t.numel() * t.element_size() for t in one)
        copies = [one] + [[t.clone() for t in one] for _ in range(max(1, (640 << 20) // nbytes))]
        n = len(copies)
        for batch in MLP_BATCHES:
            x = torch.randn(batch, h, device="cuda", generator=gen).half()
            y0 = mlp_decode(x, *copies[0])
            last = LastOutput()
            # The first timing on a fresh set of weight copies runs slow
            # (as for the GEMV variants): one discarded run first.
            for _ in range(2):
                st, graph = time_graph_steps(lambda k: last(mlp_decode(x, *copies[k % n])),
                                             steps=steps, preroll=flush)
            if not torch.equal(last.y, y0):
                raise RuntimeError(f"mlp {name} B={batch}: graph replay output differs from the "
                                   f"eager step")
            del graph, last
            reuse = batch > 1

            def unfused(k):
                gp, gs, up, us, dp, ds = copies[k % n]
                g = gemv(gp, gs, x, reuse_weights=reuse)
                u = gemv(up, us, x, reuse_weights=reuse)
                return gemv(dp, ds, (torch.nn.functional.silu(g.float()) * u.float()).half(),
                            reuse_weights=reuse)

            st_u, graph = time_graph_steps(unfused, steps=steps, preroll=flush)
            del graph
            # Each launch of the fused step alone: gate/up (with SiLU*mul) on
            # its own, and the down projection on the h it produces (the GEMV
            # w4a16_linear picks, as mlp_decode runs it).
            hs = [gate_up_silu(x, *copies[kk][:4]) for kk in range(2)]
            st_gu, graph = time_graph_steps(lambda kk: gate_up_silu(x, *copies[kk % n][:4]),
                                            steps=steps, preroll=flush)
            del graph
            st_dn, graph = time_graph_steps(
                lambda kk: gemv(copies[kk % n][4], copies[kk % n][5], hs[kk % 2],
                                reuse_weights=batch > 1), steps=steps, preroll=flush)
            del graph, hs
            moved = mlp_bytes(i, h, batch)
            w_gu = 2 * (i * h // 2 + i * h // 128 * 2)
            w_dn = i * h // 2 + i * h // 128 * 2
            out[name if batch == 1 else f"{name}_b{batch}"] = {
                "I": i, "H": h, "batch": batch, "bytes_moved": moved, "weight_copies": n,
                "fused_p50_us": st["median_us"], "fused_gbps": moved / (st["median_us"] * 1e3),
                "fused_pct_of_read_roof": 100.0 * moved / (st["median_us"] * 1e3) / roof_gbps,
                "unfused_p50_us": st_u["median_us"], "speedup": st_u["median_us"] / st["median_us"],
                "launches": {"fused": 2, "unfused": 6},
                "gate_up_p50_us": st_gu["median_us"],
                "gate_up_pct_of_read_roof": 100.0 * (w_gu + 2 * batch * (h + i)) /
                (st_gu["median_us"] * 1e3) / roof_gbps,
                "down_p50_us": st_dn["median_us"],
                "down_pct_of_read_roof": 100.0 * (w_dn + 2 * batch * (h + i)) /
                (st_dn["median_us"] * 1e3) / roof_gbps,
                "gate_up_share": st_gu["median_us"] / (st_gu["median_us"] + st_dn["median_us"]),
            }
        del copies
        torch.cuda.empty_cache()
    return out


def c3_crossover(results: dict, margin: float):
    """c3's crossover (where the decode's cost stops
    hiding under the HBM time): per batch the reuse path's per-step time
    against its B = 1 time and against torch fp16 F.linear; the smallest
    batch whose time exceeds the B = 1 time by more than `margin`, and the
    smallest batch at which the fp16 baseline is at least as fast."""
    rows = []
    for r in results.values():
        if r["M"] != 4096 or r["K"] != 4096 or not r.get("c3"):
            continue
        reuse = next((k for k in r["kernels"] if k["impl"] == "reuse"), None)
        if reuse is None:
            continue
        f16 = r.get("torch_fp16")
        rows.append((r["batch"], reuse["median_us"], f16["p50_us"] if f16 else None))
    rows.sort()
    if not rows or rows[0][0] != 1:
        return None
    t1 = rows[0][1]
    return {
        "margin": margin,
        "b1_us": t1,
        "first_batch_over_margin": next((b for b, t, _ in rows if t > (1.0 + margin) * t1), None),
        "fp16_overtakes_at": next((b for b, t, f in rows if f is not None and f <= t), None),
        "per_batch": [{"batch": b, "reuse_us": round(t, 3), "over_b1": round(t / t1, 3),
                       "torch_fp16_us": None if f is None else round(f, 3),
                       "fp16_over_w4a16": None if f is None else round(f / t, 3)}
                      for b, t, f in rows],
        "note": ("reuse path (the batch op w4a16_linear picks) per step at M = K = 4096; "
                 "first_batch_over_margin: smallest B whose time exceeds (1 + margin) x the "
                 "B = 1 time; fp16_overtakes_at: smallest B where torch fp16 F.linear on the "
                 "dequantized weights (4x the weight bytes) is at least as fast"),
    }


def kernel_of(m, k, b, **cfg):
    """The kernel the C ABI dispatches for this call (dk_gemv_describe)."""
    from decode_kernel import _abi

    return _abi.describe(_abi.load(), m, k, b, **{kk: int(v) for kk, v in cfg.items()})


def profiled_traffic(kernel: str):
    """HBM bytes per launch of the headline kernel from the committed PMC
    summary, if that summary was taken for this same kernel; else None."""
    if not PROFILE_TRAFFIC.exists():
        return None, "no committed PMC summary"
    try:
        rec = json.loads(PROFILE_TRAFFIC.read_text())
    except Exception as exc:  # unreadable summary
        return None, f"unreadable PMC summary: {exc}"
    if rec.get("kernel") != kernel:
        return None, f"committed PMC summary is for {rec.get('kernel')!r}, not this kernel"
    return rec.get("hbm_bytes_per_launch"), rec.get("source", str(PROFILE_TRAFFIC))


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE "
              f"{world}). The W4A16 GEMV has no multi-GPU path in this build: rows would shard "
              f"across GPUs with no communication beyond an optional all-gather of y.",
              file=sys.stderr)
        sys.exit(2)
    other_steps = args.other_steps if args.other_steps is not None else args.steps

    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    from decode_kernel import _cuda  # the HIP extension; no fallback exists
    from dk_bench.ceilings import (measure_copy, measure_event_floor, measure_gemm_fp16,
                                   measure_read, measure_read_floor, measure_read_same_size)
    from decode_kernel.quantize import dequantize
    from dk_bench.common import (MI355X_HBM_PEAK_GBPS, Flush, bytes_moved_w4, meta_dict,
                                 time_direct_steps, weight_copies)

    wanted = list(CONFIGS) if args.configs == "all" else ["c0"] + [
        c for c in args.configs.split(",") if c and c != "c0"]
    for c in wanted:
        if c not in CONFIGS:
            raise SystemExit(f"unknown config {c}")

    log("[bench] read roof (1 GiB STREAM read), copy roof")
    roof = measure_read(1 << 30)
    copy_roof = measure_copy(1 << 30)
    flush = Flush(args.flush_bytes, args.flush)
    preroll = flush if args.flush != "none" else None
    floor = measure_event_floor(preroll=preroll)
    lead = flush if flush.kind == "read" else Flush(args.flush_bytes, "read")
    floor_direct = time_direct_steps(lambda i: _cuda.empty_kernel(), 200, lead)
    log(f"[bench] read roof {roof['gbps']:.1f} GB/s (blocks {roof['block_sweep_gbps']}); copy "
        f"{copy_roof['gbps']:.1f} GB/s; empty kernel {floor['back_to_back']['median_us']:.2f} "
        f"us/launch back-to-back in a graph, {floor_direct['median_us']:.2f} direct, "
        f"{floor['call']['median_us']:.2f} us with events around one call")
    read_floor = measure_read_floor(bytes_moved_w4(4096, 4096, 1), preroll=preroll)
    rf = read_floor["best"]
    log(f"[bench] read floor at the headline's bytes: {rf['median_us']:.3f} us/launch "
        f"({rf['blocks']} x {rf['threads']} lanes, {rf['loads']} loads/lane, nt={rf['nt']})")

    results = {}
    headline = None
    headline_long = None
    headline_direct = None
    cpu = None
    for ci, name in enumerate(CONFIGS):
        if name not in wanted:
            continue
        m, k, batches, variants = CONFIGS[name]
        for b in batches:
            log(f"[bench] {name} M={m} K={k} B={b}")
            pd, sd, xd, p_cpu, s_cpu, x_cpu = make_inputs(m, k, b, seed=1000 + ci)
            y_ref = None
            if name == "c0":
                # The reference's gate before timing: within 1e-2 of an fp32
                # dequantize-then-matmul of the same weights (on the GPU).
                y_ref = _cuda.w4a16_gemv(pd, sd, xd)
                y32 = xd.float() @ dequantize(pd, sd).t()
                err = float((y_ref.float() - y32).abs().max())
                del y32
                if not err < 1e-2:
                    raise RuntimeError(f"headline kernel fails the 1e-2 gate: {err}")
            copies = weight_copies(pd, sd)
            del pd, sd
            entry = {"M": m, "K": k, "batch": b, "kernels": [], "c3": name == "c3"}
            if b == 1:
                same = measure_read_same_size(copies[0], preroll=preroll)
                entry["same_size_read"] = same
                log(f"   same-size STREAM read {same['median_us']:7.2f} us  {same['gbps']:8.1f} GB/s")
            first = True
            for v in variants:
                if v == "v0" and name != "c0":
                    continue
                if name == "c3" and b not in C3_BASELINE_BATCHES and v != "reuse":
                    continue
                headline_row = name == "c0" and v == "v5"
                steps = args.steps if headline_row else other_steps
                if first:
                    # The first timings after a new set of weight copies run
                    # up to 8% slow on MI355X, whichever kernel comes first:
                    # one untimed run of the first variant precedes the
                    # timed runs, and every variant is then timed once.
                    bench_variant(_cuda, copies, xd, v, steps, preroll, warmup=1)
                    first = False
                r = bench_variant(_cuda, copies, xd, v, steps, preroll,
                                  warmup=args.warmup if headline_row else 1,
                                  y_ref=y_ref if v == "v5" else None,
                                  call_level_flush=flush if headline_row else None)
                r["kernel"] = (None if v == "v5_paired" else
                               kernel_of(m, k, b, **VARIANTS[v])["kernel"])
                r["pct_of_read_roof"] = 100.0 * r["gbps"] / roof["gbps"]
                if "same_size_read" in entry:
                    r["pct_of_same_size_read"] = 100.0 * r["gbps"] / entry["same_size_read"]["gbps"]
                entry["kernels"].append(r)
                log(f"   {v:8s} {r['median_us']:8.2f} us/step  {r['gbps']:8.1f} GB/s  "
                    f"{r['pct_of_read_roof']:5.1f}% of read roof")
                if headline_row:
                    # The same kernel launched directly (no graph), back to
                    # back behind queued work, on the same GPU-clock bracket.
                    pk_, sc_ = copies
                    nc = len(pk_)
                    headline_direct = time_direct_steps(
                        lambda i: _cuda.w4a16_gemv(pk_[i % nc], sc_[i % nc], xd), 200, lead)
                    log(f"   v5 direct launches {headline_direct['median_us']:8.2f} us/step")
                if headline_row and args.steps != 1000:
                    # The same kernel over 1000 steps in the same run: the
                    # per-step figure must not depend on the step count.
                    headline_long = bench_variant(_cuda, copies, xd, v, 1000, preroll,
                                                  warmup=args.warmup)
                    log(f"   v5 at 1000 steps {headline_long['median_us']:8.2f} us/step")
            if (b == 1 or name == "c3") and not args.no_fp16_baseline:
                # Beside every c3 batch, as the reference's sweep has a
                # cuBLAS column at every B (bench/bench.py:128-139), compared
                # with the batch op there (the reuse path) and with v5 at B = 1.
                r16 = bench_torch_fp16(copies[0][0], copies[1][0], xd, other_steps, preroll)
                cmp_impl = "reuse" if name == "c3" else "v5"
                v5row = next(r for r in entry["kernels"] if r["impl"] == cmp_impl)
                pct16 = 100.0 * r16["gbps"] / roof["gbps"]
                entry["torch_fp16"] = {"precision": "fp16", "p50_us": r16["median_us"],
                                       "gbps": r16["gbps"], "pct_of_read_roof": pct16,
                                       "compared_with": cmp_impl,
                                       "w4a16_v5_speedup": r16["median_us"] / v5row["median_us"]}
                if pct16 > 90.0:
                    # bench/common.py:145-171 of the reference: an fp16 row above 90% of the
                    # read roof is not reported as a hit of the roof.
                    entry["torch_fp16"]["flag_over_roof"] = True
                    entry["torch_fp16"]["flag_note"] = (
                        f"{pct16:.1f}% of read-only STREAM exceeds 90%; do not report as a hit "
                        f"of the roof")
                log(f"   torch fp16 F.linear {r16['median_us']:8.2f} us/step (cross-precision; "
                    f"{pct16:.1f}% of read roof; {cmp_impl} is "
                    f"{entry['torch_fp16']['w4a16_v5_speedup']:.2f}x faster)")
            results[f"{name}_B{b}"] = entry
            if name == "c0":
                headline = next(r for r in entry["kernels"] if r["impl"] == "v5")
                if not args.no_cpu_baseline:
                    log(f"[bench] CPU baseline (~{args.cpu_seconds:.0f} s)")
                    cpu = cpu_baseline(p_cpu, s_cpu, x_cpu, args.cpu_seconds)
                    log(f"   torch linear_fp32 {cpu['p50_us']:.1f} us/call with "
                        f"{cpu['torch_threads']} threads ({cpu['value']:.2f} GB/s)")
            del copies, xd, p_cpu, s_cpu, x_cpu
            torch.cuda.empty_cache()

    mlp = None
    if not args.no_mlp:
        log("[bench] MLP decode step (fused gate/up + SiLU*mul, then down), B=1 and 8")
        mlp = bench_mlp(roof["gbps"], steps=other_steps, flush=preroll)
        for name, r in mlp.items():
            log(f"   {name:13s} fused {r['fused_p50_us']:8.2f} us  {r['fused_gbps']:8.1f} GB/s  "
                f"{r['fused_pct_of_read_roof']:5.1f}% of read roof; unfused {r['unfused_p50_us']:8.2f} us; "
                f"gate/up alone {r['gate_up_p50_us']:.2f} us, down alone {r['down_p50_us']:.2f} us")

    quant = None
    if not args.no_quantizer:
        log("[bench] device quantizer at c4a")
        quant = bench_quantizer(roof["gbps"], min(args.cpu_seconds, 5.0))
        log(f"   quantize_and_pack {quant['p50_us']:8.2f} us  {quant['gbps']:8.1f} GB/s  "
            f"{quant['pct_of_read_roof']:5.1f}% of read roof")

    log("[bench] fp16 GEMM (ridge point)")
    gemm = measure_gemm_fp16()
    ridge = gemm["tflops"] * 1e12 / (roof["gbps"] * 1e9)

    kernel = kernel_of(4096, 4096, 1)["kernel"]
    if headline["kernel"] != kernel:
        raise RuntimeError(f"headline kernel {headline['kernel']} is not the dispatched {kernel}")
    traffic, traffic_source = profiled_traffic(kernel)
    achieved = headline["bytes_moved"] / (headline["mean_us"] * 1e3)
    line = {
        "metric": METRIC,
        "value": headline["gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": headline["median_us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16 (int4 weights, fp16 activations, fp32 accumulate)",
        "data": "synthetic: W~N(0,0.02) fp32 quantized to int4 group 128, x~N(0,1) fp16, PCG64 seeds",
        "config": {"workload": "c0: W4A16 GEMV M=4096 K=4096 B=1 group 128 (BASELINE configs[0])",
                   "M": 4096, "K": 4096, "batch": 1, "group_size": 128, "kernel": "v5",
                   "stamp": headline["stamp"], "parallelism": "single GPU"},
        "p50_us": headline["median_us"],
        "iqr_us": headline["iqr_us"],
        "pct_of_read_roof": 100.0 * headline["gbps"] / roof["gbps"],
        "read_roof_gbps": roof["gbps"],
        "copy_roof_gbps": copy_roof["gbps"],
        "timer": ("`warmup` untimed steps, then exactly `steps` GEMV launches back-to-back in one "
                  "HIP graph over weight copies totalling > 640 MB, after one untimed lead-in "
                  "step; a 1 GiB read before each replay, outside the timed span (cold caches); "
                  "the span bracketed inside the graph by two GPU wall-clock timestamp kernels, "
                  "the bracket's own cost subtracted; p50 over 5 replays of span/steps"),
        "timer_kind": headline["timer"],
        "p50_us_outer": headline["outer_median_us"],
        "graph_replay_overhead_us": headline["replay_overhead_us"],
        "p50_us_1000_steps": (headline_long["median_us"] if headline_long is not None
                              else headline["median_us"]),
        "same_size_read_gbps": results["c0_B1"]["same_size_read"]["gbps"],
        "pct_of_same_size_read": headline["pct_of_same_size_read"],
        "floor_read_us": rf["median_us"],
        "floor_read_shape": {kk: rf[kk] for kk in ("kind", "blocks", "threads", "loads", "nt")},
        "pct_of_floor_read": 100.0 * rf["median_us"] / headline["median_us"],
        "p50_us_reference_protocol": headline["call_events"]["median_us"],
        "empty_kernel_us_back_to_back": floor["back_to_back"]["median_us"],
        "empty_kernel_us_call_events": floor["call"]["median_us"],
        "empty_kernel_us_direct": floor_direct["median_us"],
        "p50_us_direct": headline_direct["median_us"] if headline_direct else None,
        "reference_protocol_flush": flush.describe(),
        "gemm_fp16_tflops": gemm["tflops"],
        "ridge_flop_per_byte": ridge,
        "arithmetic_intensity": 2.0 * 4096 * 4096 / headline["bytes_moved"],
        "roofline": {
            "bound": "hbm", "achieved": achieved, "peak": MI355X_HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": achieved / MI355X_HBM_PEAK_GBPS, "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel": kernel, "mean_us": headline["mean_us"],
            "algorithmic_bytes": headline["bytes_moved"],
        },
        "cpu_baseline": cpu,
        "crossover": c3_crossover(results, C3_CROSSOVER_MARGIN),
        "quantizer": quant,
        "mlp": mlp,
        "configs": {
            key: {"M": r["M"], "K": r["K"], "batch": r["batch"],
                  "same_size_read_gbps": (round(r["same_size_read"]["gbps"], 1)
                                          if "same_size_read" in r else None),
                  "torch_fp16_linear": r.get("torch_fp16"),
                  "kernels": {row["impl"]: {"p50_us": round(row["median_us"], 3),
                                            "iqr_us": round(row["iqr_us"], 3),
                                            "gbps": round(row["gbps"], 1),
                                            "pct_read_roof": round(row["pct_of_read_roof"], 2)}
                              for row in r["kernels"]}}
            for key, r in results.items()
        },
    }
    if args.out:
        full = {"line": line, "meta": meta_dict(), "read_roof": roof, "copy_roof": copy_roof,
                "timing_floor": floor, "read_floor": read_floor, "gemm_fp16": gemm,
                "results": results}
        args.out.parent.mkdir(parents=True, exist_ok=True)
        args.out.write_text(json.dumps(full, indent=2) + "\n")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
