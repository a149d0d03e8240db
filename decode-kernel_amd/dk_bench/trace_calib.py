"""Live per-launch times of a set of kernels, to set beside a rocprofv3 kernel
trace of the same command.

    python decode-kernel_amd/dk_bench/trace_calib.py [--steps 200]
    rocprofv3 --kernel-trace --stats -d OUT -- python decode-kernel_amd/dk_bench/trace_calib.py

For each kernel it times `--steps` launches back to back twice: captured in
one HIP graph (as bench.py times a step) and launched directly behind queued
work (dk_bench.common.time_direct_steps), both on the GPU-clock bracket.
Kernels: the empty kernel (the launch floor), the product's GEMV at c0, c2,
c4a (one batch row) and c3 B = 16 (the weight-reuse path), and, at each
one-row configuration, the grid-stride read of the same weight bytes. Each
launch reads cold weights (copies totalling > 640 MB).

Without a profiler the numbers are the kernels' back-to-back cadence. Under
rocprofv3's kernel trace every dispatch gets its own completion signal, and
dispatches shorter than about 6 us no longer run back to back (the trace's
own per-step time rises to about 9 us), so they start on an idle GPU and
trace 0.3-0.5 us longer than their live cadence; longer kernels keep running
back to back and trace within a few percent of it. The pair of runs measures
that per-dispatch overhead for kernels of every length on the path.
Prints one JSON object (kernel name -> times in us).
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve()
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parents[2]))

CASES = {"c0": (4096, 4096, 1), "c2": (4096, 11008, 1), "c4a": (28672, 8192, 1),
         "c3_B16": (4096, 4096, 16)}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--steps", type=int, default=200)
    args = ap.parse_args()

    import torch

    from decode_kernel import _abi, _cuda, gemv
    from decode_kernel.quantize import quantize_and_pack
    from dk_bench.common import (Flush, synthetic_case, time_direct_steps, time_graph_steps,
                                 weight_copies)

    def log(*a):
        print(*a, file=sys.stderr, flush=True)

    flush = Flush()
    lib = _abi.load()
    out = {}
    g, _ = time_graph_steps(lambda i: _cuda.empty_kernel(), steps=args.steps, preroll=flush)
    d = time_direct_steps(lambda i: _cuda.empty_kernel(), args.steps, flush)
    out["empty_kernel"] = {"graph_us": g["median_us"], "direct_us": d["median_us"]}
    log("empty_kernel", out["empty_kernel"])
    for name, (m, k, b) in CASES.items():
        w, x = synthetic_case(m, k, b, seed=1000)
        p, s = quantize_and_pack(torch.from_numpy(w))
        pk, sc = weight_copies(p.cuda(), s.cuda())
        xd = torch.from_numpy(x).cuda()
        n = len(pk)
        kw = dict(reuse_weights=True) if b > 1 else {}
        kernel = _abi.describe(lib, m, k, b, **{kk: int(v) for kk, v in kw.items()})["kernel"]
        g, graph = time_graph_steps(lambda i: gemv(pk[i % n], sc[i % n], xd, **kw),
                                    steps=args.steps, preroll=flush)
        del graph
        d = time_direct_steps(lambda i: gemv(pk[i % n], sc[i % n], xd, **kw), args.steps, flush)
        out[f"{name}: {kernel.split('(')[0]}"] = {"graph_us": g["median_us"],
                                                 "direct_us": d["median_us"]}
        if b == 1:
            part = torch.empty(2048, dtype=torch.float32, device="cuda")
            g, graph = time_graph_steps(lambda i: _cuda.stream_read(pk[i % n], part),
                                        steps=args.steps, preroll=flush)
            del graph
            d = time_direct_steps(lambda i: _cuda.stream_read(pk[i % n], part), args.steps, flush)
            out[f"{name}: stream_read of the weight bytes"] = {
                "graph_us": g["median_us"], "direct_us": d["median_us"],
                "bytes": pk[0].numel() * 4}
        log(name, kernel.split("(")[0], out)
        del pk, sc
        torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
