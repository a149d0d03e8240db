"""CPU checks of the drop-in boundary: the C-ABI library loads, exports every
entry point include/decode_kernel/*.h declares, and rejects bad arguments on
the host (no compute call needs a GPU here). Also checks the torch extension
exposes the reference's pybind surface (csrc/bindings.cpp:114-129).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from decode_kernel import _abi

REPO = Path(__file__).resolve().parents[1]
HEADERS = sorted((REPO / "include").rglob("*.h"))


def _declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(dk_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not _abi.LIB_PATH.exists():
        pytest.fail(f"{_abi.LIB_PATH} is not built (python decode-kernel_amd/build_ext.py)")
    return _abi.load()


def test_header_declarations_found():
    names = _declared_functions()
    assert "dk_w4a16_gemv" in names and "dk_stream_read" in names
    assert names == set(_abi.EXPORTS), names ^ set(_abi.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.dk_abi_version() == (1 << 16) | 4


def test_default_config_matches_reference(lib):
    # include/decode_kernel/gemv_w4a16.h:22-27: V5, split_k 4, no reuse, 1 warp/row.
    cfg = _abi.default_config(lib)
    assert (cfg.version, cfg.split_k, cfg.reuse_weights, cfg.warps_per_row) == (5, 4, 0, 1)


@pytest.mark.parametrize(
    "overrides,msg",
    [
        ({"version": 6}, "version must be 0..5"),
        ({"version": -1}, "version must be 0..5"),
        ({"split_k": 0}, "split_k must be in [1, 32]"),
        ({"split_k": 33}, "split_k must be in [1, 32]"),
        ({"warps_per_row": 9}, "warps_per_row must be in [1, 8]"),
        ({"warps_per_row": 2, "version": 5}, "streaming v1 only"),
        ({"warps_per_row": 2, "version": 1, "reuse_weights": 1}, "streaming v1 only"),
    ],
)
def test_validate_rejects_reference_ranges(lib, overrides, msg):
    cfg = _abi.default_config(lib, **overrides)
    rc = lib.dk_gemv_validate(64, 256, 1, ctypes.byref(cfg))
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT
    assert msg in lib.dk_last_error().decode()


def test_validate_k_multiple_of_group(lib):
    cfg = _abi.default_config(lib)
    assert lib.dk_gemv_validate(4, 200, 1, ctypes.byref(cfg)) == _abi.DK_ERR_INVALID_ARGUMENT
    assert "divisible by group size 128" in lib.dk_last_error().decode()
    assert lib.dk_gemv_validate(4, 256, 1, ctypes.byref(cfg)) == _abi.DK_OK


def test_empty_problem_is_a_noop(lib):
    # csrc/gemv_w4a16.cu:571: M, K or B <= 0 returns before any launch; no
    # pointers are touched, so this is safe without a GPU.
    cfg = _abi.default_config(lib)
    for m, k, b in [(0, 128, 1), (4, 0, 1), (4, 128, 0), (-1, 128, 1)]:
        rc = lib.dk_w4a16_gemv(None, None, None, None, m, k, b, ctypes.byref(cfg), None, 0, None)
        assert rc == _abi.DK_OK


def test_null_and_misaligned_pointers_rejected(lib):
    cfg = _abi.default_config(lib)
    rc = lib.dk_w4a16_gemv(None, None, None, None, 4, 128, 1, ctypes.byref(cfg), None, 0, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "NULL" in lib.dk_last_error().decode()
    fake = 0x10000
    rc = lib.dk_w4a16_gemv(fake + 4, fake, fake, fake, 4, 128, 1, ctypes.byref(cfg), None, 0, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "16-byte aligned" in lib.dk_last_error().decode()


def test_split_k_needs_no_workspace(lib):
    # v4 splits K over the waves of one workgroup and adds the slices through
    # LDS: no workspace for any version (only the reuse path's optional
    # split-K tiles take one), so a NULL workspace is accepted.
    for v in range(6):
        for sk in (1, 4, 32):
            c = _abi.default_config(lib, version=v, split_k=sk)
            for m, k, b in ((4096, 4096, 1), (4096, 11008, 5), (64, 256, 2)):
                assert lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(c)) == 0, (v, sk, m, k, b)
    # The launch is one gemv_v4_split<R, U, W, S, NB, prefetch>: S waves per
    # row (at most split_k, K / 128 and 8), W / S * R rows per workgroup.
    for m, k, b, sk in ((4096, 11008, 1, 4), (1024, 28672, 1, 32), (512, 28672, 1, 8),
                        (333, 8192, 3, 7), (64, 128, 2, 4)):
        d = _abi.describe(lib, m, k, b, version=4, split_k=sk)
        assert d["kernel"].startswith("void dk::gemv_v4_split<"), d["kernel"]
        r, u, w, s, nb = (int(a) for a in d["kernel"].split("<", 1)[1].split(">", 1)[0].split(",")[:5])
        assert 1 <= s <= min(sk, k // 128, 8) and w % s == 0, (m, k, b, sk, d["kernel"])
        assert d["block"] == [64 * w, 1, 1] and d["launches"] == 1
        assert d["grid"] == [-(-m // (w // s * r)), -(-b // nb), 1], (m, k, b, sk, d)


def test_reference_workspace_contract_checks(lib):
    # dk_w4a16_gemv_ref_workspace keeps the reference's v4 contract (a
    # caller-zeroed fp32 [B, M] buffer, include/decode_kernel/gemv_w4a16.h:33):
    # v4 without it is rejected before any launch; the checks of
    # dk_w4a16_gemv come first.
    fake = 0x10000
    cfg = _abi.default_config(lib, version=4)
    rc = lib.dk_w4a16_gemv_ref_workspace(fake, fake, fake, fake, 64, 256, 1, ctypes.byref(cfg),
                                         None, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "[B, M]" in lib.dk_last_error().decode()
    rc = lib.dk_w4a16_gemv_ref_workspace(fake, fake, fake, fake, 64, 200, 1, ctypes.byref(cfg),
                                         fake, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "group size" in lib.dk_last_error().decode()
    rc = lib.dk_w4a16_gemv_ref_workspace(fake, fake, fake, fake, 64, 256, 1, ctypes.byref(cfg),
                                         fake + 2, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "4-byte aligned" in lib.dk_last_error().decode()
    # M, K or B <= 0: no-op, as in the reference.
    assert lib.dk_w4a16_gemv_ref_workspace(None, None, None, None, 0, 256, 1, ctypes.byref(cfg),
                                           None, None) == _abi.DK_OK


def test_describe_names_the_dispatched_kernel(lib):
    # dk_gemv_describe runs the dispatch without launching (no GPU needed) and
    # names the kernel as a rocprofv3 trace does.
    d = _abi.describe(lib, 4096, 4096, 1)
    assert d["kernel"].startswith("void dk::gemv_v5_lds<1, 2, 8, 1, true, dk::LayoutLogical, 5")
    assert d["grid"] == [512, 1, 1] and d["block"] == [512, 1, 1] and d["launches"] == 1
    d = _abi.describe(lib, 4096, 11008, 1, version=4, split_k=4)
    assert d["kernel"].startswith("void dk::gemv_v4_split<")
    assert _abi.describe(lib, 4096, 4096, 16, reuse_weights=1)["kernel"].startswith(
        "void dk::gemv_reuse_pf<4, 1, 8>")
    assert _abi.describe(lib, 28672, 8320, 4, reuse_weights=1)["kernel"].startswith(
        "void dk::gemv_reuse<8, 2, 2, false>")
    assert _abi.describe(lib, 4096, 4096, 2, reuse_weights=1)["kernel"].startswith(
        "void dk::gemv_v5_lds<") and ", 15, " in _abi.describe(lib, 4096, 4096, 2,
                                                              reuse_weights=1)["kernel"]
    # With the optional workspace the reuse path splits K; without it, not.
    assert "gemv_reuse_split_pf<" in _abi.describe(lib, 1024, 16384, 16, reuse_weights=1)["kernel"]
    assert "gemv_reuse_pf<" in _abi.describe(lib, 1024, 16384, 16, workspace_bytes=0,
                                             reuse_weights=1)["kernel"]
    assert _abi.describe(lib, 4096, 4096, 1, version=1, warps_per_row=4)["kernel"].startswith(
        "dk::gemv_v1_multiwave(")
    # Invalid calls fail as dk_w4a16_gemv would.
    with pytest.raises(_abi.DkError, match="group size"):
        _abi.describe(lib, 64, 200, 1)


# The dispatch each routing rule in dk_gemv.hip gives, read back without a
# GPU (dk_gemv_describe): (M, K, B, config) -> kernel name prefix, grid.
ROUTES = [
    ((4096, 4096, 1), {}, "dk::gemv_v5_lds<1, 2, 8, 1, true, dk::LayoutLogical, 5,", [512, 1, 1]),
    ((4096, 11008, 1), {}, "dk::gemv_v4_split<1, 1, 16, 2, 1, true,", [512, 1, 1]),
    ((512, 28672, 1), {}, "dk::gemv_v4_split<1, 2, 8, 4, 1, false,", [256, 1, 1]),
    ((1024, 28672, 1), {}, "dk::gemv_v4_split<2, 2, 8, 4, 1, false,", [256, 1, 1]),
    ((8192, 28672, 1), {}, "dk::gemv_v5_lds<2, 1, 16, 1, true,", [256, 1, 1]),
    ((4096, 4096, 2), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [512, 1, 1]),
    ((4096, 4096, 4), dict(reuse_weights=1), "dk::gemv_reuse_pf<6, 1, 2>", [256, 1, 1]),
    ((4096, 4096, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<6, 1, 4>", [256, 1, 1]),
    ((4096, 4096, 16), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 8>", [256, 1, 1]),
    ((4096, 4096, 32), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 2, true, 2>", [128, 2, 1]),
    ((4096, 11008, 32), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 8>", [128, 2, 1]),
    ((3072, 8192, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<8, 1, 4>", [192, 1, 1]),
    ((3072, 8192, 3), dict(reuse_weights=1), "dk::gemv_reuse_pf<8, 1, 4>", [192, 1, 1]),
    ((4096, 4096, 3), dict(reuse_weights=1), "dk::gemv_reuse_pf<6, 1, 2>", [256, 1, 1]),
    ((4096, 11008, 4), dict(reuse_weights=1), "dk::gemv_reuse_lds<16, 1, true, 2>", [256, 1, 1]),
    ((4096, 3968, 4), dict(reuse_weights=1), "dk::gemv_reuse<8, 1, 2, false>", [256, 1, 1]),
    ((2048, 4096, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<6, 1, 4>", [128, 1, 1]),
    ((2048, 4224, 8), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 1, 16, 4, true, dk::LayoutLogical, 15,",
     [128, 2, 1]),
    ((2560, 8192, 4), dict(reuse_weights=1), "dk::gemv_reuse_pf<8, 1, 4>", [160, 1, 1]),
    ((28672, 8192, 4), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 2>", [896, 1, 1]),
    ((28672, 8192, 2), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 2>", [896, 1, 1]),
    ((12288, 8192, 2), dict(reuse_weights=1), "dk::gemv_v5_lds<2, 2, 8, 2, false, dk::LayoutLogical, 15,",
     [768, 1, 1]),
    ((12288, 8192, 5), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 4>", [768, 1, 1]),
    ((12416, 8192, 5), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 4>", [388, 1, 1]),
    ((6144, 4096, 3), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 2, true, 2>", [192, 1, 1]),
    ((6144, 3968, 3), dict(reuse_weights=1), "dk::gemv_v5_lds<2, 2, 8, 3, false, dk::LayoutLogical, 15,",
     [384, 1, 1]),
    ((28672, 8320, 4), dict(reuse_weights=1), "dk::gemv_reuse<8, 2, 2, false>", [896, 1, 1]),
    ((28672, 8192, 16), dict(reuse_weights=1), "dk::gemv_reuse_lds<4, 2, true, 2>", [896, 1, 1]),
    ((11008, 4096, 4), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 2>", [688, 1, 1]),
    ((11008, 3968, 4), dict(reuse_weights=1), "dk::gemv_reuse_lds<4, 1, false, 2>", [688, 1, 1]),
    ((11008, 4096, 3), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 2>", [688, 1, 1]),
    ((11008, 4096, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 4>", [688, 1, 1]),
    ((4096, 11008, 5), dict(reuse_weights=1), "dk::gemv_reuse_lds<16, 1, true, 2>", [256, 1, 1]),
    ((6144, 8192, 12), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 8>", [192, 1, 1]),
    ((6144, 8192, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 4>", [192, 1, 1]),
    ((28672, 8192, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 2, 4>", [896, 1, 1]),
    ((8192, 3584, 3), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 2, true, 2>", [256, 1, 1]),
    ((5120, 5120, 4), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 2, true, 2>", [160, 1, 1]),
    ((6144, 8192, 32), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 2, 2>", [192, 1, 1]),
    # Above 16 batch rows, the many-batch tiles: the least reuse whose grid
    # is one round of 144-256 workgroups, else the most reuse (two waves up
    # to 512 workgroups); RT = 1 only above 32 batch rows.
    ((4096, 4096, 48), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 2, 2>", [128, 2, 1]),
    ((4096, 4096, 128), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 4, 2>", [64, 4, 1]),
    ((4096, 4096, 256), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 4, 4>", [64, 4, 1]),
    ((4096, 4096, 257), dict(reuse_weights=1), "dk::gemv_reuse_pfb<2, 4, 4>", [64, 5, 1]),
    ((2048, 8192, 48), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 1, 2>", [128, 2, 1]),
    ((2048, 8192, 32), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 8>", [128, 2, 1]),
    ((8192, 8192, 256), dict(reuse_weights=1), "dk::gemv_reuse_pfb<2, 4, 4>", [128, 4, 1]),
    ((11008, 4096, 32), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 4, 2>", [172, 1, 1]),
    ((1000, 1024, 300), dict(reuse_weights=1), "dk::gemv_reuse_pfb<4, 4, 2>", [16, 10, 1]),
    ((1024, 4096, 64), dict(reuse_weights=1), "dk::gemv_reuse_lds<16, 1, true, 2>", [64, 4, 1]),
    ((4096, 3968, 48), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 2, false, 2>", [128, 3, 1]),
    ((5120, 5120, 12), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 2, true, 2>", [160, 1, 1]),
    ((2048, 16384, 16), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 8>", [128, 1, 1]),
    ((2048, 16384, 8), dict(reuse_weights=1), "dk::gemv_reuse_pf<8, 1, 4>", [128, 1, 1]),
    ((2048, 16512, 16), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 1, false, 4>", [128, 1, 1]),
    ((1024, 16384, 16), dict(reuse_weights=1), "dk::gemv_reuse_split_pf<4, 1>", [64, 1, 2]),
    ((1024, 28672, 16), dict(reuse_weights=1), "dk::gemv_reuse_split_pf<4, 1>", [64, 1, 4]),
    ((512, 28672, 33), dict(reuse_weights=1), "dk::gemv_reuse_split_pf<4, 1>", [32, 3, 2]),
    ((1024, 28672, 33), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 8>", [64, 3, 1]),
    ((777, 28800, 17), dict(reuse_weights=1), "dk::gemv_reuse_split<8, 2, 2>", [25, 2, 2]),
    ((1024, 14336, 16), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 8>", [64, 1, 1]),
    ((512, 8192, 33), dict(reuse_weights=1), "dk::gemv_reuse_lds<8, 1, true, 2>", [32, 3, 1]),
    ((1024, 4096, 8), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [128, 4, 1]),
    ((1024, 4096, 12), dict(reuse_weights=1), "dk::gemv_reuse_pf<4, 1, 8>", [64, 1, 1]),
    # The boundaries the header documents for reuse_weights: the streaming
    # kernel's batch tiles on one side, MFMA tiles on the other.
    ((128, 4096, 64), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [16, 32, 1]),
    ((144, 4096, 64), dict(reuse_weights=1), "dk::gemv_reuse_lds<16, 1, true, 2>", [9, 4, 1]),
    ((512, 8192, 32), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [64, 16, 1]),
    ((1024, 4096, 11), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [128, 6, 1]),
    ((2048, 4096, 4), dict(reuse_weights=1), "dk::gemv_v5_lds<2, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [128, 2, 1]),
    ((2048, 4096, 5), dict(reuse_weights=1), "dk::gemv_reuse_pf<6, 1, 4>", [128, 1, 1]),
    ((2048, 4224, 8), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 1, 16, 4, true, dk::LayoutLogical, 15,",
     [128, 2, 1]),
    ((2048, 4224, 9), dict(reuse_weights=1), "dk::gemv_reuse_lds<16, 1, false, 2>", [128, 1, 1]),
    ((4096, 4096, 2), dict(reuse_weights=1), "dk::gemv_v5_lds<1, 2, 8, 2, true, dk::LayoutLogical, 15,",
     [512, 1, 1]),
    # The waves per row of v4 that the header documents for split_k.
    ((4096, 4096, 1), dict(version=4, split_k=1), "dk::gemv_v4_split<1, 2, 8, 1, 1, true,", [512, 1, 1]),
    ((4096, 4096, 1), dict(version=4, split_k=32), "dk::gemv_v4_split<1, 1, 8, 2, 1, true,",
     [1024, 1, 1]),
    ((1024, 28672, 1), dict(version=4, split_k=4), "dk::gemv_v4_split<2, 2, 8, 4, 1, false,",
     [256, 1, 1]),
    ((1024, 28672, 1), dict(version=4, split_k=2), "dk::gemv_v4_split<1, 4, 8, 2, 1, false,",
     [256, 1, 1]),
    ((512, 8192, 1), dict(version=4, split_k=8), "dk::gemv_v4_split<1, 2, 8, 4, 1, true,", [256, 1, 1]),
    ((1024, 28672, 3), dict(version=4, split_k=32), "dk::gemv_v4_split<1, 1, 8, 2, 4, true,",
     [256, 1, 1]),
]


@pytest.mark.parametrize("shape,kw,kernel,grid", ROUTES)
def test_dispatch_routes(lib, shape, kw, kernel, grid):
    m, k, b = shape
    d = _abi.describe(lib, m, k, b, **kw)
    assert d["kernel"].startswith("void " + kernel), d["kernel"]
    assert d["grid"] == grid and d["launches"] == 1


def test_reuse_split_workspace_size(lib):
    # The reuse path's split-K tiles (M <= 1024 where the tiles run: 12 or
    # more batch rows, 33 or more at M <= 512; S = 4 slices on rows of
    # 28672+ weights at up to 64 tiles of 16 rows x 16 batch rows, S = 2 on
    # 16384+ at up to 64 tiles or 28672+ at up to 128): an 8-byte ticket per
    # tile, padded to 256 bytes, then fp32 partials [S, B, M]. Zero where the
    # path streams or does not split.
    cfg = _abi.default_config(lib, reuse_weights=1)
    ws = lambda m, k, b: lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(cfg))
    assert ws(1024, 16384, 16) == 512 + 2 * 16 * 1024 * 4   # 64 tickets
    assert ws(1024, 28672, 16) == 512 + 4 * 16 * 1024 * 4
    assert ws(1000, 16384, 12) == 512 + 2 * 12 * 1000 * 4  # 63 tickets -> 504 -> 512 bytes
    assert ws(600, 65536, 12) == 512 + 4 * 12 * 600 * 4    # 38 tickets -> 304 -> 512 bytes
    assert ws(600, 65536, 33) == 1024 + 2 * 33 * 600 * 4   # 38 x 3 tickets -> 912 -> 1024 bytes
    assert ws(512, 28672, 33) == 768 + 2 * 33 * 512 * 4
    assert ws(777, 28800, 17) == 1024 + 2 * 17 * 777 * 4   # 49 x 2 tickets -> 784 -> 1024 bytes
    assert ws(1024, 28672, 33) == 0    # 192 tiles: single pass
    assert ws(1024, 14336, 16) == 0    # rows shorter than 16384 weights
    assert ws(512, 28672, 32) == 0     # streaming kernel
    assert ws(1024, 16384, 11) == 0    # streaming kernel
    assert ws(1024, 8192, 16) == 0     # rows of 8192: single-pass tiles
    assert ws(2048, 16384, 16) == 0    # single-pass tiles from 1025 rows
    assert ws(4096, 11008, 64) == 0
    assert ws(4096, 4096, 4) == 0


def test_reuse_split_workspace_fits_the_noalloc_scratch(lib):
    # The split runs on at most 128 tiles with S = 2 or 64 with S = 4, so
    # S * B * M <= 65536 partials and 128 tickets: the workspace never
    # exceeds 263168 bytes, and dk_w4a16_gemv_noalloc's scratch holds every
    # call's.
    cfg = _abi.default_config(lib, reuse_weights=1)
    worst = 0
    for m in list(range(16, 1025, 16)) + [1, 17, 600, 777, 1000, 1023]:
        for b in (1, 12, 13, 16, 17, 24, 32, 33, 48, 64, 65, 100, 128, 640):
            for k in (16384, 16512, 28672, 28800, 65536, 1 << 20):
                worst = max(worst, lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(cfg)))
    assert 0 < worst <= 263168 <= _abi.DK_NOALLOC_SCRATCH_BYTES


def test_probe_argument_checks(lib):
    assert lib.dk_stream_read(None, None, 16, 1, None) == _abi.DK_ERR_INVALID_ARGUMENT
    assert lib.dk_stream_read(0x10000, 0x10000, 15, 1, None) == _abi.DK_ERR_INVALID_ARGUMENT
    assert lib.dk_stream_write(None, 16, 1, None) == _abi.DK_ERR_INVALID_ARGUMENT
    assert lib.dk_d2d_copy(0x10000, 0x10000, 17, None) == _abi.DK_ERR_INVALID_ARGUMENT
    assert lib.dk_d2d_copy(0x10000, 0x10008, 16, None) == _abi.DK_ERR_INVALID_ARGUMENT


def test_quantizer_argument_checks(lib):
    # Every check runs on the host before a launch; empty problems are no-ops.
    assert lib.dk_quantize_pack_f32(None, 0, 128, None, None, None) == _abi.DK_OK
    assert lib.dk_quantize_pack_f32(None, 4, 0, None, None, None) == _abi.DK_OK
    assert lib.dk_quantize_pack_f32(None, -1, 128, None, None, None) == _abi.DK_ERR_INVALID_ARGUMENT
    fake = 0x10000
    rc = lib.dk_quantize_pack_f32(fake, 4, 200, fake, fake, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "group_size=128" in lib.dk_last_error().decode()
    rc = lib.dk_quantize_pack_f32(None, 4, 128, fake, fake, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "NULL" in lib.dk_last_error().decode()
    rc = lib.dk_quantize_pack_f32(fake + 4, 4, 128, fake, fake, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "aligned" in lib.dk_last_error().decode()


def test_mlp_argument_checks(lib):
    fake = 0x10000
    assert lib.dk_mlp_workspace_bytes(11008, 4096, 2) == 2 * 11008 * 2
    assert lib.dk_mlp_workspace_bytes(0, 4096, 2) == 0
    # Empty problems return before touching any pointer.
    assert lib.dk_gate_up_silu(None, None, None, None, None, None, 0, 128, 1, None) == _abi.DK_OK
    assert lib.dk_mlp_decode(None, None, None, None, None, None, None, None, 128, 128, 0, None, 0,
                             None) == _abi.DK_OK
    rc = lib.dk_gate_up_silu(fake, fake, fake, fake, fake, fake, 4, 200, 1, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "128" in lib.dk_last_error().decode()
    rc = lib.dk_gate_up_silu(fake, fake, None, fake, fake, fake, 4, 128, 1, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "NULL" in lib.dk_last_error().decode()
    rc = lib.dk_gate_up_silu(fake, fake, fake + 8, fake, fake, fake, 4, 128, 1, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "16-byte" in lib.dk_last_error().decode()
    # The MLP step checks I % 128 and its workspace before any launch.
    rc = lib.dk_mlp_decode(fake, fake, fake, fake, fake, fake, fake, fake, 200, 128, 1, fake, 4096,
                           None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "I=200" in lib.dk_last_error().decode()
    rc = lib.dk_mlp_decode(fake, fake, fake, fake, fake, fake, fake, fake, 256, 128, 2, fake, 100,
                           None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "1024-byte workspace" in lib.dk_last_error().decode()
    rc = lib.dk_mlp_decode(fake, fake, fake, fake, None, fake, fake, fake, 256, 128, 2, fake, 1024,
                           None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "NULL" in lib.dk_last_error().decode()


def test_paired_layout_argument_checks(lib):
    fake = 0x10000
    assert lib.dk_repack_paired(None, None, 0, 128, None) == _abi.DK_OK
    rc = lib.dk_repack_paired(fake, fake, 4, 200, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "group_size=128" in lib.dk_last_error().decode()
    rc = lib.dk_unpack_paired(fake + 4, fake, 4, 128, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "16-byte" in lib.dk_last_error().decode()
    assert lib.dk_w4a16_gemv_paired(None, None, None, None, 0, 128, 1, None) == _abi.DK_OK
    rc = lib.dk_w4a16_gemv_paired(None, None, None, None, 4, 128, 1, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "NULL" in lib.dk_last_error().decode()
    rc = lib.dk_w4a16_gemv_paired(fake, fake, fake, fake, 4, 200, 1, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "group size" in lib.dk_last_error().decode()
    rc = lib.dk_w4a16_gemv_paired(fake + 8, fake, fake, fake, 4, 128, 1, None)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT and "16-byte" in lib.dk_last_error().decode()


def test_torch_extension_surface():
    from decode_kernel import _cuda

    for name in ("w4a16_gemv", "d2d_copy", "stream_read", "stream_write",
                 "stream_recommended_blocks", "last_kernel_stamp", "quantize_and_pack",
                 "gate_up_silu", "mlp_decode", "repack_paired", "unpack_paired",
                 "w4a16_gemv_paired"):
        assert hasattr(_cuda, name), name
    doc = _cuda.w4a16_gemv.__doc__
    for pat in (r"version: [\w.]*Int = 5", r"split_k: [\w.]*Int = 4",
                r"reuse_weights: bool = False", r"warps_per_row: [\w.]*Int = 1"):
        assert re.search(pat, doc), (pat, doc)
    assert _cuda.ABI_VERSION == (1 << 16) | 4


def test_extension_rejects_cpu_tensors():
    import torch
    from decode_kernel import gemv

    packed = torch.zeros(4, 16, dtype=torch.int32)
    scales = torch.zeros(4, 1, dtype=torch.float16)
    x = torch.zeros(1, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="must be CUDA tensors"):
        gemv(packed, scales, x)


CPP_PROGRAM = r"""
#include "decode_kernel/gemv_w4a16.hpp"
#include <cstdio>
int main() {
  using namespace decode_kernel;
  GemvLaunchConfig cfg;  // the reference's defaults (gemv_w4a16.h:22-27)
  if (cfg.version != KernelVersion::V5 || cfg.split_k != 4 || cfg.reuse_weights ||
      cfg.warps_per_row != 1 || kGroupSize != 128 || kNibblesPerWord != 8 || kWeightsPerInt4 != 32)
    return 2;
  w4a16_gemv(nullptr, nullptr, nullptr, nullptr, 0, 128, 1, cfg, nullptr, nullptr);  // no-op
  try {
    w4a16_gemv(reinterpret_cast<const uint32_t*>(0x10000), reinterpret_cast<const __half*>(0x10000),
               reinterpret_cast<const __half*>(0x10000), reinterpret_cast<__half*>(0x10000), 4, 200,
               1, cfg, nullptr, nullptr);
    return 3;
  } catch (const std::runtime_error& e) {
    std::printf("threw: %s\n", e.what());
  }
  GemvLaunchConfig v4;
  v4.version = KernelVersion::V4;
  // The reference's signature with its v4 contract: a null [B, M] workspace
  // is rejected on the host, before any launch (the reference would fault).
  try {
    w4a16_gemv(reinterpret_cast<const uint32_t*>(0x10000), reinterpret_cast<const __half*>(0x10000),
               reinterpret_cast<const __half*>(0x10000), reinterpret_cast<__half*>(0x10000), 64,
               256, 1, v4, static_cast<float*>(nullptr), nullptr);
    return 4;
  } catch (const std::runtime_error& e) {
    std::printf("v4 threw: %s\n", e.what());
  }
  // The sized overload checks its arguments on the host too.
  try {
    w4a16_gemv(reinterpret_cast<const uint32_t*>(0x10004), reinterpret_cast<const __half*>(0x10000),
               reinterpret_cast<const __half*>(0x10000), reinterpret_cast<__half*>(0x10000), 64,
               256, 1, v4, nullptr, size_t{0}, nullptr);
    return 5;
  } catch (const std::runtime_error& e) {
    std::printf("sized threw: %s\n", e.what());
  }
  std::printf("ws %zu %zu\n", workspace_bytes(4096, 4096, 2, v4), workspace_bytes(4096, 4096, 2, cfg));
  return 0;
}
"""


def test_cpp_namespace_wrapper_compiles_and_validates(tmp_path):
    # include/decode_kernel/gemv_w4a16.hpp mirrors the reference's C++ API
    # (include/decode_kernel/gemv_w4a16.h) over the C ABI; a plain g++ build
    # against it must work, and argument errors must surface as exceptions.
    import shutil
    import subprocess

    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    src = tmp_path / "t.cpp"
    src.write_text(CPP_PROGRAM)
    exe = tmp_path / "t"
    libdir = _abi.LIB_PATH.parent
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{REPO / 'include'}",
                    "-I/opt/rocm/include", str(src), f"-L{libdir}", "-ldk_hip",
                    f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-lamdhip64", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stdout, out.stderr)
    assert "threw: w4a16_gemv: K must be divisible by group size 128" in out.stdout
    assert "v4 threw: w4a16_gemv: v4 needs the caller-zeroed fp32 [B, M] workspace" in out.stdout
    assert "sized threw: w4a16_gemv: packed and x must be 16-byte aligned" in out.stdout
    assert "ws 0 0" in out.stdout


def test_bench_library_loads_and_stays_out_of_the_product(lib):
    # dk_bench/libdk_bench.so holds the measurement-only kernels (read-floor
    # probes, the load-only ablation, shape variants); the product library
    # exports none of its entry points, and it exports only those.
    import subprocess

    from dk_bench import benchlib

    blib = benchlib.load()
    for name in benchlib.EXPORTS:
        assert hasattr(blib, name), name
        assert not hasattr(lib, name), name
    syms = subprocess.run(["nm", "-D", "--defined-only", str(benchlib.LIB_PATH)],
                          capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in syms.splitlines() if " T " in ln}
    assert exported == set(benchlib.EXPORTS), exported
    assert benchlib.parse_v5_shape(_abi.describe(lib, 4096, 4096, 1)["kernel"]) == (1, 2, 8, True)
    assert benchlib.parse_v5_shape(_abi.describe(lib, 4096, 4096, 1, version=4)["kernel"]) is None
    assert benchlib.parse_kernel(_abi.describe(lib, 4096, 4096, 1)["kernel"]) == ("v5", (1, 2, 8, True))
    assert benchlib.parse_kernel(_abi.describe(lib, 4096, 11008, 1)["kernel"]) == \
        ("split", (1, 1, 16, 2, True))
    assert benchlib.parse_kernel(_abi.describe(lib, 4096, 11008, 2)["kernel"]) is None
