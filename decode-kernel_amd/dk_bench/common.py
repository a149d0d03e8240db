"""Shared benchmark helpers: HIP-event timer, cache flush, bytes and roofs.

Restates bench/common.py of the reference for MI355X:
  * time_graph_steps: exactly K GEMV steps back-to-back, captured in one HIP
    graph over enough weight copies that every step reads cold weights, the
    replay bracketed by events; per-step time = elapsed / K (the metric);
  * time_gpu: the reference's protocol, a flush, then events around exactly
    one call (bench/common.py:64-108); on MI355X the event markers alone add
    ~6 us, more than a small GEMV takes, so it is reported beside the metric;
  * time_repeated: back-to-back launches between two events (STREAM probes);
  * the flush defaults to a read-only sweep of 1 GiB (the reference wrote
    64 MB, bench/common.py:54-61): larger than the 256 MB Infinity Cache and
    the 8 x 4 MB L2s, and read-only so the timed kernel never competes with
    the write-back of a dirty flush buffer;
  * bytes_moved_w4 / flop_gemv: bench/common.py:111-125.
"""

from __future__ import annotations

import json
import os
import platform
import statistics
import subprocess
from dataclasses import asdict, dataclass
from datetime import datetime, timezone
from typing import Callable, Optional

import torch

GROUP_SIZE = 128
FLUSH_BYTES_DEFAULT = 1 << 30
COLD_WORKING_SET = 640 << 20
MI355X_HBM_PEAK_GBPS = 8000.0


def bytes_moved_w4(m: int, k: int, batch: int) -> int:
    """Algorithmic HBM bytes if W is read once: packed W + scales + x + y."""
    return m * (k // 2) + m * (k // GROUP_SIZE) * 2 + batch * k * 2 + batch * m * 2


def mlp_bytes(i: int, h: int, batch: int) -> int:
    """Algorithmic HBM bytes of one MLP decode step: the three weight
    matrices and their scales, x, h written and read back, and y."""
    w = 3 * (i * h // 2 + i * h // GROUP_SIZE * 2)
    return w + batch * h * 2 + 2 * batch * i * 2 + batch * h * 2


def synthetic_case(m: int, k: int, batch: int, seed: int, w_std: float = 0.02):
    """Benchmark inputs: W ~ N(0, w_std) fp32 and x ~ N(0, 1) fp16, both from
    one PCG64 stream seeded with `seed` (numpy arrays)."""
    import numpy as np

    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(w_std)).astype(np.float32)
    x = rng.standard_normal((batch, k), dtype=np.float32).astype(np.float16)
    return w, x


def bytes_moved_fp16(m: int, k: int, batch: int) -> int:
    return m * k * 2 + batch * k * 2 + batch * m * 2


def arithmetic_intensity_w4(m: int, k: int, batch: int) -> float:
    """FLOP per algorithmic byte (bench/common.py:128-129)."""
    return flop_gemv(m, k, batch) / bytes_moved_w4(m, k, batch)


def flop_gemv(m: int, k: int, batch: int) -> int:
    return 2 * m * k * batch


class Flush:
    """Evicts L2 and the Infinity Cache between timed iterations."""

    def __init__(self, nbytes: int = FLUSH_BYTES_DEFAULT, kind: str = "read"):
        from decode_kernel import _cuda

        if kind not in ("read", "write", "none"):
            raise ValueError(kind)
        self.kind = kind
        self.nbytes = nbytes if kind != "none" else 0
        self._cuda = _cuda
        if kind == "none":
            return
        self.buf = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
        self.partials = torch.empty(_cuda.stream_recommended_blocks(), dtype=torch.float32,
                                    device="cuda")

    def __call__(self) -> None:
        if self.kind == "read":
            self._cuda.stream_read(self.buf, self.partials)
        elif self.kind == "write":
            self._cuda.stream_write(self.buf)

    def describe(self) -> dict:
        return {"kind": self.kind, "bytes": self.nbytes}


def time_gpu(fn: Callable[[], object], warmup: int, iters: int,
             flush: Optional[Flush] = None) -> dict:
    """Median / IQR / mean of one `fn()` call between two torch events on the
    current stream (the reference's protocol, bench/common.py:64-108)."""
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for _ in range(warmup):
        if flush is not None:
            flush()
        fn()
    torch.cuda.synchronize()
    import time

    t0 = time.perf_counter()
    for i in range(iters):
        if flush is not None:
            flush()
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    out = _stats([s.elapsed_time(e) * 1000.0 for s, e in zip(starts, ends)])
    out.update({"warmup": warmup, "wall_s_timed_loop": wall_s, "timer": "call_events",
                "flush": flush.describe() if flush is not None else None})
    return out


def _stats(us: list[float]) -> dict:
    us = sorted(us)
    n = len(us)
    return {
        "median_us": us[n // 2],
        "q1_us": us[n // 4],
        "q3_us": us[(3 * n) // 4],
        "iqr_us": us[(3 * n) // 4] - us[n // 4],
        "mean_us": statistics.fmean(us),
        "stdev_us": statistics.pstdev(us) if n > 1 else 0.0,
        "min_us": us[0],
        "max_us": us[-1],
        "iters": n,
    }


def weight_copies(packed: torch.Tensor, scales: torch.Tensor,
                  min_bytes: int = COLD_WORKING_SET) -> tuple[list, list]:
    """Enough device copies of (packed, scales) that cycling through them
    reads more than `min_bytes` (the 256 MB Infinity Cache plus the 8 x 4 MB
    L2s, with margin) between two uses of the same copy: every GEMV step then
    reads cold weights from HBM, without a flush kernel in the timed span."""
    per = packed.numel() * 4 + scales.numel() * 2
    n = max(2, -(-min_bytes // per))
    return [packed.clone() for _ in range(n)], [scales.clone() for _ in range(n)]


def _replays(graph, trials, preroll, after=None):
    """`trials` replays, each after `preroll` and bracketed by events on the
    replay stream; returns the outer times in us and the `after()` values."""
    import time

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    outer, extra, walls = [], [], []
    for _ in range(trials):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if preroll is not None:
            preroll()
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        outer.append(start.elapsed_time(end) * 1000.0)
        if after is not None:
            extra.append(after())
    return outer, extra, walls


_BRACKET = {}  # (trials) -> cost of the timestamp bracket itself, in clock ticks


def time_graph_steps(step: Callable[[int], object], steps: int, trials: int = 5,
                     warmup: int = 1, preroll: Optional[Callable[[], None]] = None) -> dict:
    """Per-step time of exactly `steps` back-to-back steps, `step(i)` for
    i = 0..steps-1, captured in one HIP graph and replayed `trials` times.

    `warmup` untimed eager steps run first (at least one: allocator and code
    objects), then one untimed replay loads the graph. Before each timed
    replay `preroll` (a 1 GiB read, ~0.2 ms) is enqueued on the same stream
    outside the timed span: every replay starts with the L2s and the
    Infinity Cache flushed.

    The timed span is bracketed on the GPU's own clock: the graph is [one
    untimed lead-in step (`step(steps)`, the next weight copy), a timestamp
    kernel, the `steps` steps, a timestamp kernel]; the two timestamps
    (s_memrealtime, a vector store each) bracket exactly the timed steps,
    and the cost of the bracket itself, measured by a graph of the two
    timestamp kernels alone, is subtracted. A graph launch's fixed start
    cost (about 10 us per replay on MI355X) thus falls outside the span,
    as it does when a decode pass replays one graph over hundreds of kernels.
    Events around the whole replay on the host's side are kept beside it
    (`outer_median_us`, per step), and their difference per replay is
    `replay_overhead_us`. Without the bench library the outer events are the
    measurement. Per-step time = span / steps; p50 over the replays."""
    try:
        from . import benchlib

        khz = benchlib.wall_clock_khz()
        inner = khz > 0
    except Exception:
        inner, khz = False, 0
    for i in range(max(1, warmup)):
        step(i % steps)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    if inner:
        ts = torch.zeros(2, dtype=torch.int64, device="cuda")
        with torch.cuda.graph(graph):
            step(steps)  # lead-in, untimed
            benchlib.timestamp(ts, 0)
            for i in range(steps):
                step(i)
            benchlib.timestamp(ts, 1)
        if trials not in _BRACKET:
            tb = torch.zeros(2, dtype=torch.int64, device="cuda")
            bracket = torch.cuda.CUDAGraph()
            with torch.cuda.graph(bracket):
                benchlib.timestamp(tb, 0)
                benchlib.timestamp(tb, 1)
            bracket.replay()
            _, ticks, _ = _replays(bracket, 2 * trials, preroll,
                                   lambda: int(tb[1].item()) - int(tb[0].item()))
            _BRACKET[trials] = sorted(ticks)[len(ticks) // 2]
    else:
        with torch.cuda.graph(graph):
            for i in range(steps):
                step(i)
    graph.replay()
    torch.cuda.synchronize()
    if inner:
        outer, ticks, walls = _replays(graph, trials, preroll,
                                       lambda: int(ts[1].item()) - int(ts[0].item()))
        per_in = [(t - _BRACKET[trials]) * 1e3 / khz / steps for t in ticks]
        if not all(0.0 < a <= b / steps * 1.001 for a, b in zip(per_in, outer)):
            inner = False  # implausible: the outer events bound the bracketed span
    else:
        outer, _, walls = _replays(graph, trials, preroll)
    per_out = [o / steps for o in outer]
    out = _stats(per_in if inner else per_out)
    out.update({"steps": steps, "trials": trials, "warmup": max(1, warmup),
                "timer": "gpu_clock_bracket_in_graph" if inner else "events_around_graph_replay",
                "outer_median_us": _stats(per_out)["median_us"],
                "replay_overhead_us": ((_stats(per_out)["median_us"] - out["median_us"]) * steps
                                       if inner else None),
                "bracket_us": _BRACKET[trials] * 1e3 / khz if inner else None,
                "preroll": "1 GiB read before each replay" if preroll is not None else None,
                "wall_s_per_replay": statistics.fmean(walls)})
    return out, graph


def time_direct_steps(step: Callable[[int], object], steps: int, flush: Flush,
                      trials: int = 5, lead_reads: int = 24) -> dict:
    """Per-step time of exactly `steps` direct launches (`step(i)`, no graph)
    back-to-back on the current stream, bracketed by the same GPU-clock
    timestamp kernels as time_graph_steps. The launches are queued behind
    `lead_reads` 1 GiB reads (~4 ms of GPU work), so the host has enqueued
    all of them before the GPU reaches the first: the span measures the
    GPU's cadence, not the host's launch rate (which is checked: the host's
    enqueue time must fit inside the lead reads). The bracket's own cost is
    measured the same way and subtracted. p50 over `trials`."""
    import time

    from . import benchlib

    khz = benchlib.wall_clock_khz()
    ts = torch.zeros(2, dtype=torch.int64, device="cuda")
    step(0)
    torch.cuda.synchronize()
    per, host = [], []
    for _ in range(trials):
        for _ in range(lead_reads):
            flush()
        benchlib.timestamp(ts, 0)
        benchlib.timestamp(ts, 1)
        torch.cuda.synchronize()
        bracket = int(ts[1]) - int(ts[0])
        for _ in range(lead_reads):
            flush()
        t0 = time.perf_counter()
        benchlib.timestamp(ts, 0)
        for i in range(steps):
            step(i)
        benchlib.timestamp(ts, 1)
        host.append((time.perf_counter() - t0) * 1e6)
        torch.cuda.synchronize()
        per.append((int(ts[1]) - int(ts[0]) - bracket) * 1e3 / khz / steps)
    out = _stats(per)
    out.update({"steps": steps, "trials": trials, "timer": "gpu_clock_bracket_direct_launches",
                "host_enqueue_us_per_step": statistics.median(host) / steps,
                "host_kept_ahead": max(host) < lead_reads * 150.0})
    return out


def time_repeated(fn: Callable[[], object], reps: int, trials: int = 5) -> dict:
    """Per-launch time of `reps` back-to-back launches between two events (the
    STREAM method: the event overhead is shared by `reps` launches)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    per = []
    for _ in range(trials):
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        per.append(start.elapsed_time(end) * 1000.0 / reps)
    out = _stats(per)
    out.update({"reps": reps, "trials": trials, "timer": "events_around_repeated_launches"})
    return out


def gpu_info() -> dict:
    if not torch.cuda.is_available():
        return {"name": "none"}
    p = torch.cuda.get_device_properties(0)
    info = {
        "name": torch.cuda.get_device_name(0),
        "gcn_arch": getattr(p, "gcnArchName", None),
        "total_memory_bytes": int(p.total_memory),
        "multi_processor_count": int(p.multi_processor_count),
        "l2_cache_bytes": int(getattr(p, "L2_cache_size", 0)),
    }
    info["amd_smi"] = _smi()
    return info


def _smi() -> dict:
    for cmd in (["amd-smi", "static", "--asic", "--clock", "--json"],
                ["rocm-smi", "--showclocks", "--json"]):
        try:
            out = subprocess.run(cmd, capture_output=True, text=True, timeout=20)
            if out.returncode == 0 and out.stdout.strip():
                return {"cmd": " ".join(cmd), "raw": out.stdout.strip()[:4000]}
        except Exception as exc:  # tool missing on this host
            last = str(exc)
            continue
    return {"error": locals().get("last", "no smi tool")}


@dataclass
class RunMeta:
    gpu: dict
    host: str
    platform: str
    torch: str
    hip: Optional[str]
    timestamp: str
    git: Optional[str]
    host_cpus: int


def collect_meta() -> RunMeta:
    git = None
    try:
        git = subprocess.check_output(["git", "rev-parse", "--short", "HEAD"], text=True,
                                      timeout=5, stderr=subprocess.DEVNULL).strip()
    except Exception:
        pass
    return RunMeta(
        gpu=gpu_info(),
        host=platform.node(),
        platform=platform.platform(),
        torch=torch.__version__,
        hip=getattr(torch.version, "hip", None),
        timestamp=datetime.now(timezone.utc).isoformat(),
        git=git,
        host_cpus=len(os.sched_getaffinity(0)),
    )


def meta_dict() -> dict:
    return asdict(collect_meta())


def save_json(path, payload: dict) -> None:
    from pathlib import Path

    p = Path(path)
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_text(json.dumps(payload, indent=2) + "\n")
