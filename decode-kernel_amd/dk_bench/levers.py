"""Launch-shape and kernel-variant sweeps behind the routing choices.

    python -m dk_bench.levers floor|c0|v4|split|reuse|rsplit|mlp|cache|all [--steps 300] [--out PATH]
    (from decode-kernel_amd/, after build_ext.py)

  floor  read-probe launch shapes at the algorithmic bytes of c0, c1 and c2
         (grid, lanes, loads per lane, non-temporal hint): the read floor;
  c0     one-stage GEMV variants at M = K = 4096, B = 1 (activations through
         LDS or in registers, weights issued first or last, one or two waves
         per row, 4 to 16 waves per workgroup) and streaming-kernel shapes,
         against the product;
  v4     the product's split-K kernel at every instantiated shape (rows per
         wave, chunks per lane per stage, waves per workgroup, 2-8 waves per
         row, prefetch) and the cross-workgroup ticket form (a sample, also
         without the reduction), at short and tall rows, against the
         product's v5 and v4;
  split  the split-K kernel's shapes against the product's v5 (B = 1) over
         the shapes the streaming kernel's launch rules were set on;
  reuse  the weight-reuse tile kernels (operands loaded directly, or staged
         in LDS by the buffer-load-to-LDS path, single or double buffered)
         at 3-32 batch rows over the shapes the reuse path's launch rules
         were set on, against the product's reuse path;
  rsplit the reuse path's split-K tiles (2-8 slices, both forms) and the
         single-pass tiles at M <= 2048 on long rows, 5-33 batch rows,
         against the product's reuse path;
  mlp    the fused gate/up tile kernels (all three forms) at 3-32 batch rows on
         Llama MLP shapes, against the product's fused gate/up;
  cache  the product at one batch row with its weight copies cycled over
         > 640 MB (cold, as bench.py), 128 or 64 MB (inside the Infinity
         Cache) or two copies (largely in the L2s).
Every variant that computes y is checked against the product's v5 output
(bit-exact where the summation order is the same, else within 1e-3 plus one
fp16 ulp) before it is timed. Timing as in bench.py: HIP graphs of `steps`
launches over weight copies totalling > 640 MB (cold), a 1 GiB pre-roll
before each of 5 replays, p50 microseconds per launch.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

import torch

V4_PROBLEMS = {"c0": (4096, 4096), "c2": (4096, 11008), "m1024_k28672": (1024, 28672),
               "m512_k28672": (512, 28672), "m2048_k16384": (2048, 16384),
               "m2048_k11008": (2048, 11008), "m1024_k8192": (1024, 8192), "c4b": (8192, 28672)}
V5_C0_SHAPES = [(1, 2, 8, True), (1, 2, 8, False), (1, 2, 16, True), (1, 2, 16, False),
                (1, 2, 4, True), (1, 1, 16, True), (1, 1, 8, True)]


def _close(a, b) -> bool:
    a32, b32 = a.float(), b.float()
    ulp = torch.clamp(b32.abs(), min=2.0 ** -14) * 2.0 ** -10
    return bool(((a32 - b32).abs() <= 1e-3 + ulp).all())


def _time(fn, steps, flush, runs: int = 1) -> float:
    """p50 us per step; with runs > 1 the lowest of that many timings (the
    first timings after a new set of weight copies run up to 8% slow on
    MI355X, so the product, timed first on each shape, is timed twice)."""
    from .common import time_graph_steps

    return min(time_graph_steps(fn, steps=steps, preroll=flush)[0]["median_us"]
               for _ in range(runs))


def sweep_floor(flush, steps: int) -> dict:
    from .ceilings import measure_read_floor
    from .common import bytes_moved_w4

    out = {}
    for name, (m, k) in {"c0": (4096, 4096), "c1": (11008, 4096), "c2": (4096, 11008)}.items():
        fl = measure_read_floor(bytes_moved_w4(m, k, 1), preroll=flush, steps=steps)
        out[name] = fl
        b = fl["best"]
        print(f"floor {name}: {b['median_us']:.3f} us ({b['gbps']:.0f} GB/s) at {b['blocks']} x "
              f"{b['threads']} lanes, {b['loads']} loads, nt={b['nt']}; next: "
              + ", ".join(f"{r['median_us']:.3f}" for r in fl["sweep"][1:6]), flush=True)
    return out


def sweep_c0(flush, steps: int) -> dict:
    from decode_kernel import _cuda

    from . import benchlib
    from .ablation import gpu_case
    from .common import weight_copies

    packed, scales, x = gpu_case(4096, 4096, seed=1000)
    pk, sc = weight_copies(packed, scales)
    n = len(pk)
    y_prod = _cuda.w4a16_gemv(pk[0], sc[0], x)
    y = torch.empty_like(y_prod)
    rows = {"product_v5": _time(lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x), steps, flush,
                                runs=2)}
    print(f"c0 product v5 {rows['product_v5']:.3f} us", flush=True)
    for shape in V5_C0_SHAPES:
        benchlib.v5(0, shape, pk[0], sc[0], x, y)
        torch.cuda.synchronize()
        if not torch.equal(y, y_prod):
            raise RuntimeError(f"v5 {shape} differs from the product at c0")
        key = "v5_R{}_U{}_W{}_{}".format(*shape[:3], "pf" if shape[3] else "nopf")
        rows[key] = _time(lambda i: benchlib.v5(0, shape, pk[i % n], sc[i % n], x, y), steps, flush)
        print(f"c0 {key} {rows[key]:.3f} us", flush=True)
    for w, s in ((4, 1), (8, 1), (16, 1), (8, 2), (16, 2)):
        for lds in (True, False):
            for wf in (False, True):
                benchlib.onestage(w, s, lds, wf, pk[0], sc[0], x, y)
                torch.cuda.synchronize()
                ok = torch.equal(y, y_prod) if s == 1 else _close(y, y_prod)
                if not ok:
                    raise RuntimeError(f"onestage W{w} S{s} lds={lds} wf={wf} differs at c0")
                key = f"onestage_W{w}_S{s}_{'lds' if lds else 'regs'}_{'wfirst' if wf else 'xfirst'}"
                rows[key] = _time(lambda i: benchlib.onestage(w, s, lds, wf, pk[i % n], sc[i % n], x,
                                                              y), steps, flush)
                print(f"c0 {key} {rows[key]:.3f} us", flush=True)
    return rows


SPLIT_PROBLEMS = [(4096, 4096), (4096, 11008), (4096, 5120), (4096, 6144), (3328, 5120),
                  (8192, 5120), (11008, 5120), (13824, 5120), (4096, 8192), (5120, 8192),
                  (8192, 8192), (4096, 14336), (4096, 28672), (8192, 28672), (28672, 8192),
                  (11008, 4096), (14336, 4096), (2048, 16384), (2048, 4096), (1024, 28672),
                  (1024, 11008), (512, 28672), (512, 4096), (512, 8320)]
V4S_SHAPES = [(r, u, w, k, pf) for k, us in ((2, (1, 2, 4)), (4, (1, 2)), (8, (1,)))
              for r in (1, 2) for u in us for w in (4, 8, 16) for pf in (True, False)
              if w >= k and (r, u) != (2, 4)]


def sweep_v4(flush, steps: int) -> dict:
    """Split-K two ways, against the product's v5 and v4: the product's
    kernel (gemv_v4_split: S waves per row inside the streaming kernel's
    stage loop) at every shape the measurement library instantiates, and
    across workgroups with a ticket reduction (gemv_v4_lds, a sample of
    shapes, also without the reduction)."""
    from decode_kernel import _cuda

    from . import benchlib
    from .ablation import gpu_case
    from .common import weight_copies

    out = {}
    gen = 1 << 20
    for name, (m, k) in V4_PROBLEMS.items():
        packed, scales, x = gpu_case(m, k, seed=2000 + m + k)
        pk, sc = weight_copies(packed, scales)
        n = len(pk)
        y_prod = _cuda.w4a16_gemv(pk[0], sc[0], x)
        y = torch.empty_like(y_prod)
        rows = {"product_v5": _time(lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x), steps, flush,
                                    runs=2)}
        for sk in (2, 4, 8, 16):
            rows[f"product_v4_s{sk}"] = _time(
                lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x, version=4, split_k=sk), steps,
                flush)
        print(f"v4 {name}: product v5 {rows['product_v5']:.3f}; product v4 " + ", ".join(
            f"s{sk} {rows[f'product_v4_s{sk}']:.3f}" for sk in (2, 4, 8, 16)), flush=True)
        for shape in V4S_SHAPES:
            if benchlib.v4s(shape, pk[0], sc[0], x, y) == 3:
                raise RuntimeError(f"v4 split {shape} is not instantiated")
            torch.cuda.synchronize()
            if not _close(y, y_prod):
                raise RuntimeError(f"v4 split {shape} differs from v5 at {name}")
            key = "split_R{}_U{}_W{}_S{}_{}".format(*shape[:4], "pf" if shape[4] else "nopf")
            rows[key] = _time(lambda i: benchlib.v4s(shape, pk[i % n], sc[i % n], x, y), steps,
                              flush)
            print(f"v4 {name} {key}: {rows[key]:.3f} us", flush=True)
        for splits in (2, 4):
            ws = torch.empty(splits * m, dtype=torch.float32, device="cuda")
            tickets = torch.zeros(m, dtype=torch.int64, device="cuda")
            for shape in ((1, 1, 16, True), (1, 4, 8, True), (2, 1, 4, True)):
                gen += 64
                benchlib.v4(shape, 0, splits, pk[0], sc[0], x, y, ws, tickets, gen)
                torch.cuda.synchronize()
                if not _close(y, y_prod):
                    raise RuntimeError(f"v4 {shape} S{splits} differs from v5 at {name}")
                key = "groups_S{}_R{}_U{}_W{}_{}".format(splits, *shape[:3],
                                                         "pf" if shape[3] else "nopf")
                g = gen + 64
                gen += 128
                full = _time(lambda i: benchlib.v4(shape, 0, splits, pk[i % n], sc[i % n], x, y, ws,
                                                   tickets, g), steps, flush)
                part = _time(lambda i: benchlib.v4(shape, 2, splits, pk[i % n], sc[i % n], x, y, ws,
                                                   tickets, g), steps, flush)
                rows[key] = {"us": full, "partials_only_us": part}
                print(f"v4 {name} {key}: {full:.3f} us (partials only {part:.3f})", flush=True)
        out[name] = rows
        del pk, sc, packed, scales, x
        torch.cuda.empty_cache()
    return out


def sweep_split(flush, steps: int) -> dict:
    """The split-K kernel at every instantiated shape against the product's
    v5 at B = 1, over SPLIT_PROBLEMS."""
    from decode_kernel import _cuda

    from . import benchlib
    from .ablation import gpu_case
    from .common import weight_copies

    out = {}
    for m, k in SPLIT_PROBLEMS:
        name = f"m{m}_k{k}"
        packed, scales, x = gpu_case(m, k, seed=3000 + m + k)
        pk, sc = weight_copies(packed, scales)
        n = len(pk)
        y_prod = _cuda.w4a16_gemv(pk[0], sc[0], x)
        y = torch.empty_like(y_prod)
        rows = {"product_v5": _time(lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x), steps, flush,
                                    runs=2)}
        for shape in V4S_SHAPES:
            benchlib.v4s(shape, pk[0], sc[0], x, y)
            torch.cuda.synchronize()
            if not _close(y, y_prod):
                raise RuntimeError(f"v4 split {shape} differs from v5 at {name}")
            key = "R{}_U{}_W{}_S{}_{}".format(*shape[:4], "pf" if shape[4] else "nopf")
            rows[key] = _time(lambda i: benchlib.v4s(shape, pk[i % n], sc[i % n], x, y), steps,
                              flush)
        best = min((v, kk) for kk, v in rows.items() if kk != "product_v5")
        print(f"split {name}: product v5 {rows['product_v5']:.3f}; best {best[1]} {best[0]:.3f}",
              flush=True)
        out[name] = rows
        del pk, sc, packed, scales, x
        torch.cuda.empty_cache()
    return out


REUSE_PROBLEMS = [(4096, 4096), (4096, 11008), (3072, 8192), (11008, 4096), (6144, 8192),
                  (5120, 5120), (28672, 8192), (8192, 28672), (2048, 16384), (2048, 8192),
                  (2048, 4096), (1536, 8192), (2560, 8192), (1024, 4096)]
REUSE_BATCHES = (3, 4, 5, 8, 12, 16, 32)
# (kind, waves, tiles per wave, groups per block, paired scales): kind 0
# operands loaded directly, 1 staged in LDS, 2 staged and double buffered.
REUSE_SHAPES = [(0, 8, 1, 2, True), (0, 8, 1, 4, False), (0, 16, 1, 4, False), (0, 16, 1, 2, False),
                (0, 8, 2, 2, True), (0, 8, 2, 4, False),
                (1, 8, 1, 2, True), (1, 16, 1, 2, True), (1, 8, 2, 2, True), (1, 4, 1, 2, True),
                (1, 4, 2, 2, True), (1, 8, 1, 4, True), (1, 4, 1, 4, True), (1, 4, 2, 4, True),
                (2, 4, 1, 2, True), (2, 6, 1, 2, True), (2, 4, 2, 2, True), (2, 6, 2, 2, True),
                (3, 4, 1, 2, True), (3, 6, 1, 2, True), (4, 4, 1, 2, True), (4, 6, 1, 2, True),
                (3, 4, 2, 2, True), (3, 6, 2, 2, True), (3, 8, 1, 2, True), (3, 8, 2, 2, True)]
# kinds 3 and 4: double buffered with 4 and 2 x loads per block (batches of
# up to 8 and 4 rows; skipped above).
_REUSE_KINDS = ("tiles", "lds", "pf", "pfx4", "pfx2")
_REUSE_MAX_B = {3: 8, 4: 4}


def sweep_reuse(flush, steps: int) -> dict:
    """Tile kernels of the reuse path against the product's reuse path."""
    from decode_kernel import _cuda

    from . import benchlib
    from .ablation import gpu_case
    from .common import weight_copies

    out = {}
    for m, k in REUSE_PROBLEMS:
        packed, scales, _ = gpu_case(m, k, seed=4000 + m + k)
        pk, sc = weight_copies(packed, scales)
        n = len(pk)
        gen = torch.Generator(device="cuda").manual_seed(m + k)
        xall = torch.randn(max(REUSE_BATCHES), k, device="cuda", generator=gen).half()
        for b in REUSE_BATCHES:
            x = xall[:b].contiguous()
            name = f"m{m}_k{k}_b{b}"
            y_prod = _cuda.w4a16_gemv(pk[0], sc[0], x, reuse_weights=True)
            y = torch.empty_like(y_prod)
            rows = {"product_reuse": _time(
                lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x, reuse_weights=True), steps, flush,
                runs=2)}
            for shape in REUSE_SHAPES:
                kind, ks, rt, sg, pairs = shape
                if b > _REUSE_MAX_B.get(kind, b):
                    continue
                y.fill_(float("nan"))
                if benchlib.reuse(kind, ks, rt, sg, pairs, pk[0], sc[0], x, y) == 3:
                    raise RuntimeError(f"reuse {shape} is not instantiated")
                torch.cuda.synchronize()
                if not _close(y, y_prod):
                    raise RuntimeError(f"reuse {shape} differs from the product at {name}")
                key = "{}_KS{}_RT{}_SG{}{}".format(_REUSE_KINDS[kind], ks, rt, sg,
                                                   "_pairs" if pairs else "")
                rows[key] = _time(lambda i: benchlib.reuse(kind, ks, rt, sg, pairs, pk[i % n],
                                                           sc[i % n], x, y), steps, flush)
            best = min((v, kk) for kk, v in rows.items())
            print(f"reuse {name}: product {rows['product_reuse']:.3f}; best {best[1]} {best[0]:.3f}",
                  flush=True)
            out[name] = rows
        del pk, sc, packed, scales, xall
        torch.cuda.empty_cache()
    return out


RSPLIT_PROBLEMS = [(1024, 8192), (1024, 14336), (1024, 16384), (512, 28672), (1024, 28672),
                   (600, 65536), (768, 12288), (512, 16384), (512, 8192), (2048, 16384)]
RSPLIT_BATCHES = (5, 8, 12, 16, 33)
RSPLIT_SINGLE = [(1, 8, 1, 2), (1, 8, 1, 4), (2, 4, 1, 2), (2, 6, 1, 2)]
# (kind, waves, tiles per wave, slices): kind 0 operands loaded directly,
# 1 double-buffered LDS staging.
RSPLIT_SHAPES = [(0, 8, 2, 4), (1, 4, 1, 2), (1, 4, 1, 4), (1, 4, 1, 8), (1, 6, 1, 4),
                 (1, 4, 2, 4), (1, 4, 2, 2)]


def sweep_rsplit(flush, steps: int) -> dict:
    """Split-K and single-pass tiles of the reuse path against the product's
    reuse path, at M <= 2048 on long rows."""
    from decode_kernel import _cuda

    from . import benchlib
    from .ablation import gpu_case
    from .common import weight_copies

    out = {}
    for m, k in RSPLIT_PROBLEMS:
        packed, scales, _ = gpu_case(m, k, seed=4000 + m + k)
        pk, sc = weight_copies(packed, scales)
        n = len(pk)
        gen = torch.Generator(device="cuda").manual_seed(m + k)
        xall = torch.randn(max(RSPLIT_BATCHES), k, device="cuda", generator=gen).half()
        ws = torch.empty(max(benchlib.reuse_split_workspace(rt, s_, m, max(RSPLIT_BATCHES))
                             for _, _, rt, s_ in RSPLIT_SHAPES), dtype=torch.uint8, device="cuda")
        for b in RSPLIT_BATCHES:
            x = xall[:b].contiguous()
            name = f"m{m}_k{k}_b{b}"
            y_prod = _cuda.w4a16_gemv(pk[0], sc[0], x, reuse_weights=True)
            y = torch.empty_like(y_prod)
            rows = {"product_reuse": _time(
                lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x, reuse_weights=True), steps, flush,
                runs=2)}
            for kind, ks, rt, sg in RSPLIT_SINGLE:
                y.fill_(float("nan"))
                if benchlib.reuse(kind, ks, rt, sg, True, pk[0], sc[0], x, y) == 3:
                    raise RuntimeError(f"reuse {(kind, ks, rt, sg)} is not instantiated")
                torch.cuda.synchronize()
                if not _close(y, y_prod):
                    raise RuntimeError(f"reuse {(kind, ks, rt, sg)} differs from the product at {name}")
                rows[f"{_REUSE_KINDS[kind]}_KS{ks}_RT{rt}_SG{sg}"] = _time(
                    lambda i: benchlib.reuse(kind, ks, rt, sg, True, pk[i % n], sc[i % n], x, y),
                    steps, flush)
            for kind, ks, rt, s_ in RSPLIT_SHAPES:
                y.fill_(float("nan"))
                if benchlib.reuse_split(kind, ks, rt, s_, pk[0], sc[0], x, y, ws) == 3:
                    raise RuntimeError(f"split {(kind, ks, rt, s_)} is not instantiated")
                torch.cuda.synchronize()
                if not _close(y, y_prod):
                    raise RuntimeError(f"split {(kind, ks, rt, s_)} differs from the product at {name}")
                rows["{}_KS{}_RT{}_S{}".format("split" if kind == 0 else "splitpf", ks, rt, s_)] = \
                    _time(lambda i: benchlib.reuse_split(kind, ks, rt, s_, pk[i % n], sc[i % n], x, y,
                                                         ws), steps, flush)
            best = min((v, kk) for kk, v in rows.items())
            print(f"rsplit {name}: product {rows['product_reuse']:.3f}; best {best[1]} {best[0]:.3f}",
                  flush=True)
            out[name] = rows
        del pk, sc, packed, scales, xall, ws
        torch.cuda.empty_cache()
    return out


MLP_PROBLEMS = [(11008, 4096), (3584, 8192), (2752, 4096), (14336, 4096), (28672, 8192)]
MLP_BATCHES = (3, 4, 8, 16, 32)
MLP_SHAPES = [(0, 8, True), (1, 8, True), (1, 4, True), (2, 4, True), (2, 6, True), (3, 4, True),
              (3, 6, True)]


def sweep_mlp(flush, steps: int) -> dict:
    """Fused gate/up tile kernels against the product's fused gate/up."""
    from decode_kernel import gate_up_silu

    from . import benchlib
    from .ablation import gpu_case

    out = {}
    for i_dim, h_dim in MLP_PROBLEMS:
        gp, gs, _ = gpu_case(i_dim, h_dim, seed=5000 + i_dim)
        upk, us, _ = gpu_case(i_dim, h_dim, seed=6000 + i_dim)
        # Copies of both matrices totalling > 640 MB, so every step reads cold weights.
        per = (gp.numel() * 4 + gs.numel() * 2) * 2
        n = max(2, -(-(640 << 20) // per))
        gps = [gp.clone() for _ in range(n)]
        gss = [gs.clone() for _ in range(n)]
        ups = [upk.clone() for _ in range(n)]
        uss = [us.clone() for _ in range(n)]
        gen = torch.Generator(device="cuda").manual_seed(i_dim + h_dim)
        xall = torch.randn(max(MLP_BATCHES), h_dim, device="cuda", generator=gen).half()
        for b in MLP_BATCHES:
            x = xall[:b].contiguous()
            name = f"i{i_dim}_h{h_dim}_b{b}"
            h_prod = gate_up_silu(x, gps[0], gss[0], ups[0], uss[0])
            hbuf = torch.empty_like(h_prod)
            rows = {"product": _time(lambda j: gate_up_silu(x, gps[j % n], gss[j % n], ups[j % n],
                                                            uss[j % n]), steps, flush, runs=2)}
            for shape in MLP_SHAPES:
                kind, ks, pairs = shape
                if b > _REUSE_MAX_B.get(kind, b):
                    continue
                hbuf.fill_(float("nan"))
                if benchlib.gate_up(kind, ks, pairs, gps[0], gss[0], ups[0], uss[0], x, hbuf) == 3:
                    raise RuntimeError(f"gate/up {shape} is not instantiated")
                torch.cuda.synchronize()
                if not _close(hbuf, h_prod):
                    raise RuntimeError(f"gate/up {shape} differs from the product at {name}")
                key = "{}_KS{}".format(_REUSE_KINDS[kind], ks)
                rows[key] = _time(lambda j: benchlib.gate_up(kind, ks, pairs, gps[j % n], gss[j % n],
                                                             ups[j % n], uss[j % n], x, hbuf),
                                  steps, flush)
            best = min((v, kk) for kk, v in rows.items())
            print(f"mlp {name}: product {rows['product']:.3f}; best {best[1]} {best[0]:.3f}",
                  flush=True)
            out[name] = rows
        del gps, gss, ups, uss, gp, gs, upk, us, xall
        torch.cuda.empty_cache()
    return out


CACHE_PROBLEMS = [(4096, 4096), (8192, 3584), (4096, 11008)]
# Working sets the weight copies are cycled over: past the Infinity Cache
# (cold, as bench.py), inside it but past the L2s, and two copies.
CACHE_SETS = {"cold": 640 << 20, "mall_128MB": 128 << 20, "mall_64MB": 64 << 20, "two_copies": 0}


def sweep_cache(flush, steps: int) -> dict:
    """The product at one batch row with its weights cold in HBM against
    the same copies cycled within the Infinity Cache or the L2s."""
    from decode_kernel import _cuda

    from .ablation import gpu_case
    from .common import weight_copies

    out = {}
    for m, k in CACHE_PROBLEMS:
        packed, scales, x = gpu_case(m, k, seed=7000 + m + k)
        rows = {}
        for name, nbytes in CACHE_SETS.items():
            pk, sc = weight_copies(packed, scales, min_bytes=nbytes)
            n = len(pk)
            rows[name] = _time(lambda i: _cuda.w4a16_gemv(pk[i % n], sc[i % n], x), steps, flush,
                               runs=2)
            del pk, sc
        print(f"cache m{m}_k{k}: " + "  ".join(f"{kk} {v:.3f}" for kk, v in rows.items()),
              flush=True)
        out[f"m{m}_k{k}"] = rows
        del packed, scales, x
        torch.cuda.empty_cache()
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("what", choices=["floor", "c0", "v4", "split", "reuse", "rsplit", "mlp", "cache",
                                     "all"])
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--out", type=Path, default=None)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("a GPU is required")
    from .common import Flush

    flush = Flush()
    res = {}
    if args.what in ("floor", "all"):
        res["floor"] = sweep_floor(flush, args.steps)
    if args.what in ("c0", "all"):
        res["c0"] = sweep_c0(flush, args.steps)
    if args.what in ("v4", "all"):
        res["v4"] = sweep_v4(flush, args.steps)
    if args.what in ("split", "all"):
        res["split"] = sweep_split(flush, args.steps)
    if args.what in ("reuse", "all"):
        res["reuse"] = sweep_reuse(flush, args.steps)
    if args.what in ("rsplit", "all"):
        res["rsplit"] = sweep_rsplit(flush, args.steps)
    if args.what in ("mlp", "all"):
        res["mlp"] = sweep_mlp(flush, args.steps)
    if args.what in ("cache", "all"):
        res["cache"] = sweep_cache(flush, args.steps)
    if args.out:
        args.out.parent.mkdir(parents=True, exist_ok=True)
        args.out.write_text(json.dumps(res, indent=2) + "\n")


if __name__ == "__main__":
    main()
