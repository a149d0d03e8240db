"""Load-only ablation of the streaming GEMV at one batch row.

    python -m dk_bench.ablation [--configs c0,c1,c2,c4a,c4b] [--steps 400] [--out PATH]
    (from decode-kernel_amd/, after build_ext.py)

For each configuration the product kernel (the shape dk_gemv_describe
reports for it) is timed next to the same kernel with its arithmetic
replaced (dk_bench/libdk_bench.so, never part of the product):
  * no decode: the stage's activation pieces are still read from LDS, and
    XOR-folded with the weight words instead of decoded and multiplied;
  * loads only: the weight words and scales are folded, no LDS reads;
and next to two reads of the same bytes: the STREAM read probe over the
weight bytes (`same-size read`) and the best launch shape of the read probe
over the algorithmic bytes (`read floor`). Everything runs back-to-back in
HIP graphs over weight copies totalling > 640 MB (cold), after a 1 GiB
pre-roll per replay, p50 of 5 replays, microseconds per step; each kernel
is timed twice (product, no decode, loads only, then again) and the lower
median is kept.
This answers the reference's open question (README.md:44): how much of the
GEMV's time is the decode, and how much is moving the bytes.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

import torch

SHAPES = {"c0": (4096, 4096), "c1": (11008, 4096), "c2": (4096, 11008),
          "c4a": (28672, 8192), "c4b": (8192, 28672)}


def gpu_case(m: int, k: int, seed: int):
    """W ~ N(0, 0.02) quantized on the GPU (same bits as the CPU quantizer),
    x ~ N(0, 1) fp16, one batch row."""
    from decode_kernel import _cuda

    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(m, k, device="cuda", generator=gen) * 0.02
    packed, scales = _cuda.quantize_and_pack(w)
    del w
    x = torch.randn(1, k, device="cuda", generator=gen).half()
    return packed, scales, x


def run(configs, steps: int) -> dict:
    from decode_kernel import _abi, _cuda

    from . import benchlib
    from .ceilings import measure_read_floor, measure_read_same_size
    from .common import Flush, bytes_moved_w4, time_graph_steps, weight_copies

    lib = _abi.load()
    flush = Flush()
    out = {}
    for name in configs:
        m, k = SHAPES[name]
        packed, scales, x = gpu_case(m, k, seed=1000 + list(SHAPES).index(name))
        desc = _abi.describe(lib, m, k, 1)
        kern = benchlib.parse_kernel(desc["kernel"])
        if kern is None:
            raise RuntimeError(f"{name}: the product runs {desc['kernel']}, not a stage-loop kernel")
        pk, sc = weight_copies(packed, scales)
        n = len(pk)
        y_prod = _cuda.w4a16_gemv(pk[0], sc[0], x)
        y = torch.empty_like(y_prod)
        benchlib.run_kernel(kern, 0, pk[0], sc[0], x, y)
        torch.cuda.synchronize()
        if not torch.equal(y, y_prod):
            raise RuntimeError(f"{name}: bench-library instance {kern} differs from the product")
        row = {"M": m, "K": k, "kernel": desc["kernel"], "shape": [kern[0], *kern[1]],
               "bytes_moved": bytes_moved_w4(m, k, 1)}
        timings = {
            "product": lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x),
            "no_decode": lambda i: benchlib.run_kernel(kern, 1, pk[i % n], sc[i % n], x, y),
            "loads_only": lambda i: benchlib.run_kernel(kern, 2, pk[i % n], sc[i % n], x, y),
        }
        # Each variant is timed twice, in the order product, no decode, loads
        # only, then again; the lower of its two medians is reported (the
        # first timings after a new set of weight copies run up to 8% slow
        # on MI355X, whichever kernel comes first).
        for rnd in range(2):
            for key, fn in timings.items():
                st, _ = time_graph_steps(fn, steps=steps, preroll=flush)
                row.setdefault(key + "_runs_us", []).append(st["median_us"])
        for key in timings:
            row[key + "_us"] = min(row[key + "_runs_us"])
        row["same_size_read_us"] = measure_read_same_size(pk, preroll=flush)["median_us"]
        floor = measure_read_floor(row["bytes_moved"], preroll=flush)
        row["read_floor_us"] = floor["best"]["median_us"]
        row["read_floor_shape"] = {kk: floor["best"][kk]
                                   for kk in ("kind", "blocks", "threads", "loads", "nt")}
        out[name] = row
        print(f"{name:4s} product {row['product_us']:7.2f}  no decode {row['no_decode_us']:7.2f}  "
              f"loads only {row['loads_only_us']:7.2f}  same-size read {row['same_size_read_us']:7.2f}  "
              f"read floor {row['read_floor_us']:7.2f} us", flush=True)
        del pk, sc, packed, scales, x
        torch.cuda.empty_cache()
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--configs", default="c0,c1,c2,c4a,c4b")
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--out", type=Path, default=None)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("a GPU is required")
    res = run([c for c in args.configs.split(",") if c], args.steps)
    if args.out:
        args.out.parent.mkdir(parents=True, exist_ok=True)
        args.out.write_text(json.dumps(res, indent=2) + "\n")


if __name__ == "__main__":
    main()
