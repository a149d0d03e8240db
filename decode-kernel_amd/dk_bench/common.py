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


def time_graph_steps(step: Callable[[int], object], steps: int, trials: int = 5,
                     warmup: int = 1, preroll: Optional[Callable[[], None]] = None) -> dict:
    """Per-step time of exactly `steps` back-to-back steps, `step(i)` for
    i = 0..steps-1, captured in one HIP graph and replayed `trials` times.

    `warmup` untimed eager steps run first (at least one: allocator and code
    objects), then one untimed replay loads the graph. Before each timed
    replay `preroll` (a 1 GiB read, ~0.2 ms) is enqueued on the same stream
    outside the events: the GPU is busy with it while the host enqueues the
    start event and the graph's launches, so the timed span holds only the
    steps back-to-back, whatever `steps` is, and every replay starts with
    the L2s and the Infinity Cache flushed. Each replay is bracketed by
    events on the stream it runs on; per-step time = elapsed / steps."""
    import time

    for i in range(max(1, warmup)):
        step(i % steps)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    per, walls = [], []
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
        per.append(start.elapsed_time(end) * 1000.0 / steps)
    out = _stats(per)
    out.update({"steps": steps, "trials": trials, "warmup": max(1, warmup),
                "timer": "events_around_graph_replay",
                "preroll": "1 GiB read before each replay" if preroll is not None else None,
                "wall_s_per_replay": statistics.fmean(walls)})
    return out, graph


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
