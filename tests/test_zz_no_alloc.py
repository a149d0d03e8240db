"""dk_w4a16_gemv_noalloc, the entry point that allocates nothing, through the
C ABI against dk_w4a16_gemv with a caller workspace (same kernels, so the
same bits), on two calls in a row per path, the second with a smaller input:
the reuse path's split-K tiles (the scratch's user: the double-buffered
split, then the split for rows of an odd number of groups) and paths
without scratch. Also: a captured call replays with eager split-K calls of
other shapes between the replays (each rewrites the scratch's tickets and
partials), and, in a fresh process, the first call into the library is a
captured one. (Every call's workspace fits the scratch, which
a CPU test of test_abi.py checks over a grid of shapes, so the refusal of
a larger one has no call to test.)
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


def _lib():
    from decode_kernel import _abi

    return _abi, _abi.load()


def _case(m, k, b, seed):
    w, x = oracle.make_case(m, k, b, seed=seed, w_std=0.05)
    packed, scales = oracle.quantize_and_pack(w)
    y_ref = oracle.linear_f64(x, packed, scales)
    return (torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda(),
            torch.from_numpy(x).cuda(), y_ref)


def _call_noalloc(lib, cfg, pd, sd, xd, y, m, k, b):
    return lib.dk_w4a16_gemv_noalloc(pd.data_ptr(), sd.data_ptr(), xd.data_ptr(), y.data_ptr(),
                                     m, k, b, ctypes.byref(cfg),
                                     torch.cuda.current_stream().cuda_stream)


def _call_ws(abi, lib, cfg, pd, sd, xd, m, k, b, with_ws=True):
    need = lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(cfg)) if with_ws else 0
    ws = (torch.randint(-(2 ** 62), 2 ** 62, ((need + 7) // 8,), dtype=torch.int64, device="cuda")
          if need else None)
    y = torch.empty(b, m, dtype=torch.float16, device="cuda")
    abi.check(lib, lib.dk_w4a16_gemv(pd.data_ptr(), sd.data_ptr(), xd.data_ptr(), y.data_ptr(), m,
                                     k, b, ctypes.byref(cfg), ws.data_ptr() if need else None,
                                     need, torch.cuda.current_stream().cuda_stream))
    return y


def _tight(y, y_ref, label):
    err = np.abs(y.float().cpu().numpy().astype(np.float64) - y_ref)
    assert err.max() < 1e-2, f"{label}: {err.max():.3e}"
    assert (err <= 0.5 * oracle.fp16_ulp(y_ref) + 1e-3).all(), label


# (config, first call (M, K, B), second, smaller call); the reuse path's
# split-K tiles take the scratch, the others none.
PATHS = [
    (dict(version=5, reuse_weights=1), (1024, 16384, 16), (1000, 16512, 13)),
    (dict(version=5, reuse_weights=1), (4096, 11008, 64), (2048, 9216, 33)),
    (dict(version=4, split_k=4), (4096, 11008, 1), (1000, 1024, 3)),
    (dict(version=5), (4096, 4096, 1), (333, 640, 2)),
]


@pytest.mark.parametrize("cfg,first,second", PATHS)
def test_noalloc_matches_the_workspace_entry(cfg, first, second):
    abi, lib = _lib()
    c = abi.default_config(lib, **cfg)
    for (m, k, b), seed in ((first, 1), (second, 2)):
        print(f"[noalloc] {cfg} M={m} K={k} B={b}", flush=True)
        need = lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(c))
        assert need <= abi.DK_NOALLOC_SCRATCH_BYTES
        pd, sd, xd, y_ref = _case(m, k, b, seed=seed + m)
        y = torch.empty(b, m, dtype=torch.float16, device="cuda")
        abi.check(lib, _call_noalloc(lib, c, pd, sd, xd, y, m, k, b))
        y_ws = _call_ws(abi, lib, c, pd, sd, xd, m, k, b)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ws), f"{cfg} M={m} K={k} B={b}: differs from dk_w4a16_gemv"
        _tight(y, y_ref, f"noalloc {cfg} M={m} K={k} B={b}")


# The captured call and the calls between its replays all take their
# tickets and partials from the one scratch array: the between-calls use
# other slice counts and tile counts (so other ticket slots and partial
# offsets), and each rewrites what the next replay finds there.
BETWEEN = [(1024, 28672, 16), (1000, 16512, 13)]


def test_noalloc_graph_replays_with_eager_calls_between():
    abi, lib = _lib()
    c = abi.default_config(lib, reuse_weights=1)
    m, k, b = 1024, 16384, 16
    pd, sd, xd, y_ref = _case(m, k, b, seed=4)
    assert lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(c)) > 0  # uses the scratch
    between = []
    for i, (m2, k2, b2) in enumerate(BETWEEN):
        assert lib.dk_gemv_workspace_bytes(m2, k2, b2, ctypes.byref(c)) > 0, (m2, k2, b2)
        between.append(((m2, k2, b2), _case(m2, k2, b2, seed=5 + i)))
    y_eager = torch.empty(b, m, dtype=torch.float16, device="cuda")
    abi.check(lib, _call_noalloc(lib, c, pd, sd, xd, y_eager, m, k, b))
    torch.cuda.synchronize()
    y_graph = torch.empty(b, m, dtype=torch.float16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        abi.check(lib, _call_noalloc(lib, c, pd, sd, xd, y_graph, m, k, b))
    for rep in range(4):
        print(f"[noalloc] replay {rep}", flush=True)
        graph.replay()
        (m2, k2, b2), (p2, s2, x2, y2_ref) = between[rep % len(between)]
        y_between = torch.empty(b2, m2, dtype=torch.float16, device="cuda")
        abi.check(lib, _call_noalloc(lib, c, p2, s2, x2, y_between, m2, k2, b2))
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), f"replay {rep}"
        _tight(y_between, y2_ref, f"eager call between replays {rep} M={m2} K={k2} B={b2}")
        y_graph.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y_graph, y_eager), "last replay"
    _tight(y_graph, y_ref, "graph")


_CHILD = r"""
import ctypes, sys
import numpy as np
import torch
sys.path[:0] = [{pkg!r}, {repo!r}]
from decode_kernel import _abi
from oracle import oracle

lib = _abi.load()
m, k, b = 1024, 16384, 16
c = _abi.default_config(lib, reuse_weights=1)
assert lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(c)) > 0
w, x = oracle.make_case(m, k, b, seed=11, w_std=0.05)
packed, scales = oracle.quantize_and_pack(w)
y_ref = oracle.linear_f64(x, packed, scales)
pd, sd, xd = (torch.from_numpy(a).cuda() for a in (packed, scales, x))
y = torch.empty(b, m, dtype=torch.float16, device="cuda")
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = lib.dk_w4a16_gemv_noalloc(pd.data_ptr(), sd.data_ptr(), xd.data_ptr(), y.data_ptr(),
                                   m, k, b, ctypes.byref(c),
                                   torch.cuda.current_stream().cuda_stream)
assert rc == 0, lib.dk_last_error().decode()
for rep in range(3):
    y.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    err = np.abs(y.float().cpu().numpy().astype(np.float64) - y_ref)
    assert (err <= 0.5 * oracle.fp16_ulp(y_ref) + 1e-3).all(), (rep, err.max())
print("child ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture():
    """In a fresh process whose first call into the library is a captured
    dk_w4a16_gemv_noalloc (the per-device scratch address is looked up
    inside the capture), the replays give the oracle's result."""
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parents[1]
    code = _CHILD.format(pkg=str(repo / "decode-kernel_amd"), repo=str(repo))
    print("[noalloc] child process: first call inside capture", flush=True)
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                          timeout=100)
    assert proc.returncode == 0 and "child ok" in proc.stdout, proc.stdout + proc.stderr
