"""Hardware ceilings for one MI355X, measured before the GEMV is judged.

    python -m dk_bench.ceilings [--bytes N] [--out PATH]   (from decode-kernel_amd/)

STREAM probes over a buffer of at least 1 GiB (past the 256 MB Infinity
Cache and the 8 x 4 MB L2s), as bench/ceilings.py:1-13 of the reference did
with 512 MB on NVIDIA parts:
  * read:  grid-stride sum, read-only, bytes counted once  <- GEMV denominator
  * copy:  read + write, bytes counted twice
  * write: fill, bytes counted once
Each probe is timed as 20 back-to-back launches between two events (the
STREAM method), and the read roof is the best of a few grid sizes. Also
reported: an empty kernel per launch back-to-back and with events around one
call (the timing floors), and an fp16 GEMM for the ridge point.
"""

from __future__ import annotations

import argparse
from pathlib import Path

import torch

from .common import meta_dict, save_json, time_gpu, time_graph_steps, time_repeated

DEFAULT_STREAM_BYTES = 1 << 30


def _measure(fn, nbytes: int, factor: float, reps: int = 20) -> dict:
    stats = time_repeated(fn, reps=reps)
    return {"nbytes": nbytes, "bytes_factor": factor,
            "gbps": factor * nbytes / (stats["median_us"] * 1e3), **stats}


def measure_read(nbytes: int = DEFAULT_STREAM_BYTES, block_counts=(2048, 4096, 8192)) -> dict:
    """Best read rate over a few grid sizes (the roof is the best measured)."""
    from decode_kernel import _cuda

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    best, sweep = None, {}
    for blocks in block_counts:
        partials = torch.empty(blocks, dtype=torch.float32, device="cuda")
        out = _measure(lambda: _cuda.stream_read(src, partials), nbytes, 1.0)
        out["checksum_ok"] = float(partials.double().sum()) == float(nbytes // 4)
        out["blocks"] = blocks
        sweep[blocks] = round(out["gbps"], 1)
        if best is None or out["gbps"] > best["gbps"]:
            best = out
    best["kind"] = "stream_read_sum"
    best["block_sweep_gbps"] = sweep
    best["recommended_blocks"] = int(_cuda.stream_recommended_blocks())
    return best


def measure_copy(nbytes: int = DEFAULT_STREAM_BYTES) -> dict:
    from decode_kernel import _cuda

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    out = _measure(lambda: _cuda.d2d_copy(src, dst), nbytes, 2.0)
    out["kind"] = "d2d_copy"
    return out


def measure_write(nbytes: int = DEFAULT_STREAM_BYTES) -> dict:
    from decode_kernel import _cuda

    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = _measure(lambda: _cuda.stream_write(dst), nbytes, 1.0)
    out["kind"] = "stream_write_fill"
    return out


def measure_event_floor(steps: int = 500, preroll=None) -> dict:
    """An empty kernel: per launch when launches run back-to-back (graph
    replay; the floor under every per-step time here), and with events around
    a single call (the floor under the reference's protocol)."""
    from decode_kernel import _cuda

    b2b, _ = time_graph_steps(lambda i: _cuda.empty_kernel(), steps=steps, preroll=preroll)
    call = time_gpu(lambda: _cuda.empty_kernel(), warmup=50, iters=500)
    return {"back_to_back": b2b, "call": call}


def measure_read_same_size(packed_copies: list, preroll=None) -> dict:
    """Read-only STREAM over the GEMV's own weight buffers, back-to-back over
    the copies: the best a kernel that only reads those bytes achieves."""
    from decode_kernel import _cuda

    best = None
    for blocks in (1024, 2048, 4096):
        partials = torch.empty(blocks, dtype=torch.float32, device="cuda")
        n = len(packed_copies)
        st, _ = time_graph_steps(lambda i: _cuda.stream_read(packed_copies[i % n], partials),
                                 steps=4 * n, preroll=preroll)
        nbytes = packed_copies[0].numel() * 4
        st.update({"blocks": blocks, "nbytes": nbytes, "gbps": nbytes / (st["median_us"] * 1e3)})
        if best is None or st["gbps"] > best["gbps"]:
            best = st
    return best


def measure_read_floor(nbytes: int, preroll=None, grids=(256, 512, 1024, 2048, 4096),
                       threads=(256, 512, 1024), loads=(1, 2, 4, 8), max_passes: int = 2,
                       steps: int = 200, stride_blocks=(512, 1024, 2048, 4096, 8192)) -> dict:
    """The read floor at `nbytes`: the fastest per-launch time of a kernel that
    only reads that many bytes, over launch shapes of the read probe
    (dk_bench/libdk_bench.so): `grids` workgroups of `threads` lanes, `loads`
    16-byte loads per lane all issued before the first wait, with and without
    the non-temporal hint; shapes needing more than `max_passes` passes over
    the buffer are skipped. The grid-stride STREAM read (one load per lane
    per step, `stride_blocks` workgroups of 256 lanes: the kernel of the read
    roof and the same-size read) is swept beside them (`threads` 256,
    `loads` 0 in the rows), so the floor is never above the same-size read.
    Each shape is timed back-to-back over buffer copies totalling > 640 MB
    (cold), `steps` launches per graph, p50 of 5 replays after a 1 GiB
    pre-roll. Returns the best shape and the sweep."""
    from decode_kernel import _cuda

    from . import benchlib
    from .common import COLD_WORKING_SET

    nbytes = (nbytes + 15) // 16 * 16
    n = max(2, -(-COLD_WORKING_SET // nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(n)]
    pieces = nbytes // 16
    sweep, best = [], None
    for g in stride_blocks:
        partials = torch.empty(g, dtype=torch.float32, device="cuda")
        st, _ = time_graph_steps(lambda i: _cuda.stream_read(bufs[i % n], partials), steps=steps,
                                 preroll=preroll)
        row = {"blocks": g, "threads": 256, "loads": 0, "nt": False, "kind": "grid_stride",
               "median_us": st["median_us"], "gbps": nbytes / (st["median_us"] * 1e3)}
        sweep.append(row)
        if best is None or row["median_us"] < best["median_us"]:
            best = row
    for t in threads:
        partials = torch.empty(max(grids) * t // 64, dtype=torch.float32, device="cuda")
        for g in grids:
            for ld in loads:
                if -(-pieces // (g * t * ld)) > max_passes:
                    continue
                for nt in (False, True):
                    st, _ = time_graph_steps(
                        lambda i: benchlib.read_probe(bufs[i % n], partials, g, t, ld, nt),
                        steps=steps, preroll=preroll)
                    row = {"blocks": g, "threads": t, "loads": ld, "nt": nt, "kind": "probe",
                           "median_us": st["median_us"], "gbps": nbytes / (st["median_us"] * 1e3)}
                    sweep.append(row)
                    if best is None or row["median_us"] < best["median_us"]:
                        best = row
    del bufs
    return {"nbytes": nbytes, "copies": n, "best": best,
            "sweep": sorted(sweep, key=lambda r: r["median_us"])}


def measure_gemm_fp16(n: int = 8192, warmup: int = 10, iters: int = 30) -> dict:
    a = torch.randn(n, n, device="cuda", dtype=torch.float16)
    b = torch.randn(n, n, device="cuda", dtype=torch.float16)
    stats = time_gpu(lambda: torch.mm(a, b), warmup=warmup, iters=iters, flush=None)
    return {"n": n, "tflops": 2.0 * n ** 3 / (stats["median_us"] * 1e-6) / 1e12, **stats}


def measure_all(nbytes: int = DEFAULT_STREAM_BYTES, gemm: bool = True) -> dict:
    read = measure_read(nbytes)
    out = {
        "hbm_read": read,
        "hbm_copy": measure_copy(nbytes),
        "hbm_write": measure_write(nbytes),
        "event_floor": measure_event_floor(),
        "hbm_denominator": "read",
    }
    if gemm:
        g = measure_gemm_fp16()
        out["gemm_fp16"] = g
        out["ridge_flop_per_byte"] = g["tflops"] * 1e12 / (read["gbps"] * 1e9)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--bytes", type=int, default=DEFAULT_STREAM_BYTES)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--out", type=Path, default=None)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("a GPU is required")
    if args.bytes % 16 or args.bytes < (1 << 30):
        raise SystemExit("--bytes must be a multiple of 16 and at least 1 GiB")
    payload = {"meta": meta_dict(), **measure_all(args.bytes, gemm=not args.no_gemm)}
    if args.out:
        save_json(args.out, payload)
    r, c, w = payload["hbm_read"], payload["hbm_copy"], payload["hbm_write"]
    print(f"STREAM buffer {args.bytes / 2**30:.2f} GiB")
    print(f"read  {r['gbps']:.1f} GB/s  (denominator, checksum_ok={r['checksum_ok']})")
    print(f"copy  {c['gbps']:.1f} GB/s   write {w['gbps']:.1f} GB/s")
    fl = payload["event_floor"]
    print(f"empty kernel {fl['back_to_back']['median_us']:.2f} us/launch back-to-back, "
          f"{fl['call']['median_us']:.2f} us with events around one call")
    if "gemm_fp16" in payload:
        print(f"fp16 GEMM {payload['gemm_fp16']['tflops']:.1f} TFLOP/s, "
              f"ridge {payload['ridge_flop_per_byte']:.0f} FLOP/B")


if __name__ == "__main__":
    main()
