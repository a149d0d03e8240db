"""Fixed workload for rocprofv3 runs (kernel trace and PMC counters).

    rocprofv3 --pmc FETCH_SIZE -d OUT -- python decode-kernel_amd/dk_bench/profile_run.py --config c0

Runs, each after a 1 GiB read-only flush so every launch starts cold:
  * `--copies` launches of the d2d copy over a 64 MiB buffer: known traffic
    (64 MiB read + 64 MiB written) that calibrates FETCH_SIZE / WRITE_SIZE;
  * `--reps` launches of each GEMV variant at each benchmark configuration
    (comma-separated lists), or of another operation on the path (the MLP
    step, the paired-layout GEMV, the device quantizer:
    `--config mlp7b|mlp70b|mlp70b_tp8|mlp70b_tp8_b8|paired_c0|paired_c4b|quant_c4a`). Variants
    `no_decode` and `loads_only` run the kernel the product dispatches at one
    batch row with the ablation maths of dk_bench/libdk_bench.so (the same
    loads; the decode replaced, or the decode and the activation reads from
    LDS), so a counter run shows whether they move the product's bytes.
Replaces the reference's ncu launcher (bench/ncu_launch.py:13-34).
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve()
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parents[2]))

SHAPES = {"c0": (4096, 4096, 1), "c1": (11008, 4096, 1), "c2": (4096, 11008, 1),
          "c3b4": (4096, 4096, 4), "c3b8": (4096, 4096, 8), "c3b12": (4096, 4096, 12),
          "c3b16": (4096, 4096, 16), "c3b48": (4096, 4096, 48), "c3b128": (4096, 4096, 128),
          "c3b256": (4096, 4096, 256), "c4ab4": (28672, 8192, 4),
          "c4a": (28672, 8192, 1), "c4ab8": (28672, 8192, 8), "c4b": (8192, 28672, 1),
          # shapes of the reuse path's two-tile and split-K routes
          "m6144k8192b16": (6144, 8192, 16), "m1024k16384b16": (1024, 16384, 16),
          "m1024k28672b16": (1024, 28672, 16)}
VARIANTS = {"v5": dict(version=5), "v2": dict(version=2), "v4": dict(version=4, split_k=4),
            "reuse": dict(version=5, reuse_weights=True), "v1": dict(version=1),
            # w4a16_linear's choice: the reuse path for a batch, v5 at one row
            # (python/decode_kernel/__init__.py:71-74)
            "linear": None}
ABLATIONS = {"no_decode": 1, "loads_only": 2}
COPY_BYTES = 64 << 20


def _mlp(i: int, h: int, b: int = 1):
    def run(reps, flush):
        import torch

        from decode_kernel import mlp_decode, quantize_and_pack

        gen = torch.Generator(device="cuda").manual_seed(i)
        ws = []
        for shape in ((i, h), (i, h), (h, i)):
            ws += list(quantize_and_pack(torch.randn(*shape, device="cuda", generator=gen) * 0.02))
        x = torch.randn(b, h, device="cuda", generator=gen).half()
        for _ in range(reps):
            flush()
            mlp_decode(x, *ws)
    return run


def _paired(m: int, k: int):
    def run(reps, flush):
        import torch

        from decode_kernel import gemv_paired, quantize_and_pack, repack_paired

        gen = torch.Generator(device="cuda").manual_seed(m)
        p, s = quantize_and_pack(torch.randn(m, k, device="cuda", generator=gen) * 0.02)
        p = repack_paired(p)
        x = torch.randn(1, k, device="cuda", generator=gen).half()
        for _ in range(reps):
            flush()
            gemv_paired(p, s, x)
    return run


def _quant(reps, flush):
    import torch

    from decode_kernel import _cuda

    w = torch.randn(28672, 8192, device="cuda") * 0.02
    for _ in range(reps):
        flush()
        _cuda.quantize_and_pack(w)


# Other operations on the path, by name: the MLP step at the Llama-7B and
# 70B shapes and at the 70B TP = 8 shard (one and eight batch rows), the
# paired-layout GEMV at c0 and c4b, the device quantizer.
OTHER_OPS = {"mlp7b": _mlp(11008, 4096), "mlp70b": _mlp(28672, 8192),
             "mlp70b_tp8": _mlp(3584, 8192), "mlp70b_tp8_b8": _mlp(3584, 8192, 8),
             "paired_c0": _paired(4096, 4096), "paired_c4b": _paired(8192, 28672),
             "quant_c4a": _quant}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", default="c0",
                    help="comma-separated: " + ", ".join(sorted(SHAPES) + sorted(OTHER_OPS)))
    ap.add_argument("--variant", default="v5",
                    help="comma-separated: " + ", ".join(sorted(VARIANTS) + sorted(ABLATIONS)))
    ap.add_argument("--reps", type=int, default=50)
    ap.add_argument("--copies", type=int, default=5)
    ap.add_argument("--sclk", action="store_true",
                    help="print the shader clock (clock probe kernel) before and after the "
                         "workload, so SCLK-cycle counters convert to time in the same run")
    args = ap.parse_args()
    configs = args.config.split(",")
    variants = args.variant.split(",")
    for c in configs:
        if c not in SHAPES and c not in OTHER_OPS:
            ap.error(f"unknown config {c}")
    for v in variants:
        if v not in VARIANTS and v not in ABLATIONS:
            ap.error(f"unknown variant {v}")

    import torch

    from decode_kernel import _abi, _cuda, gemv
    from decode_kernel.quantize import quantize_and_pack
    from dk_bench.common import Flush, bytes_moved_w4
    from dk_bench.common import synthetic_case

    def sclk(when):
        if args.sclk:
            from dk_bench import benchlib

            print(json.dumps({"sclk_mhz": {"when": when, "one_wave": benchlib.sclk_mhz(),
                                           "all_cus": benchlib.sclk_mhz(blocks=1024)}}),
                  flush=True)

    sclk("start")
    flush = Flush()
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(args.copies):
        flush()
        _cuda.d2d_copy(src, dst)
    for config in configs:
        if config in OTHER_OPS:
            OTHER_OPS[config](args.reps, flush)
            torch.cuda.synchronize()
            print(json.dumps({"config": config, "reps": args.reps, "copy_bytes": COPY_BYTES}),
                  flush=True)
            continue
        m, k, b = SHAPES[config]
        w, x = synthetic_case(m, k, b, seed=1000)
        packed, scales = quantize_and_pack(torch.from_numpy(w))
        pd, sd, xd = packed.cuda(), scales.cuda(), torch.from_numpy(x).cuda()
        for variant in variants:
            if variant in ABLATIONS:
                from dk_bench import benchlib

                kern = benchlib.parse_kernel(_abi.describe(_abi.load(), m, k, b)["kernel"])
                if kern is None:
                    raise SystemExit(f"{config}: no ablation of the dispatched kernel")
                y = torch.empty(b, m, dtype=torch.float16, device="cuda")
                for _ in range(args.reps):
                    flush()
                    benchlib.run_kernel(kern, ABLATIONS[variant], pd, sd, xd, y)
            else:
                kw = VARIANTS[variant]
                if kw is None:
                    kw = dict(version=5, reuse_weights=b > 1)
                for _ in range(args.reps):
                    flush()
                    gemv(pd, sd, xd, **kw)
            torch.cuda.synchronize()
            print(json.dumps({"config": config, "variant": variant, "M": m, "K": k, "B": b,
                              "reps": args.reps, "copy_bytes": COPY_BYTES,
                              "algorithmic_bytes": bytes_moved_w4(m, k, b)}), flush=True)
    sclk("end")


if __name__ == "__main__":
    main()
