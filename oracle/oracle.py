"""CPU oracle for the W4A16 GEMV path: a numpy restatement of the reference.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or as the
timed CPU baseline). The product path (decode_kernel.gemv) never calls it.

Restates, function by function:
  quantize_and_pack   python/decode_kernel/quantize.py:26-51
  unpack_to_int       python/decode_kernel/quantize.py:54-63
  dequantize          python/decode_kernel/quantize.py:66-78
  linear_fp32         python/decode_kernel/reference.py:17-26
  max_abs_err         python/decode_kernel/reference.py:29-30
  bytes_moved_w4, flop_gemv   bench/common.py:111-125
  repack_paired, unpack_paired: no reference counterpart; the kernel-native
    nibble order (q_{2j} at bits 4j, q_{2j+1} at bits 16+4j)
  silu_f64, gate_up_silu_f64, mlp_decode_f64: no reference counterpart;
    the MLP decode step composed from the reference's gemv (linear_f64
    here) and SiLU, x * sigmoid(x), as torch.nn.functional.silu defines it
Nibble semantics: csrc/gemv_w4a16.cu:27-29; layout: include/decode_kernel/gemv_w4a16.h:29-33.

How each function is pinned (tests/test_oracle.py):
  * quantize_and_pack: the reference's known-answer test
    (tests/test_quantize.py:41-53), hand-derived KATs (digit ramp, ties to
    even, fp16 rounding of amax/7 by exact rational arithmetic, zero group),
    the reference's invariants (tests/test_quantize.py:16-38,56-61), and
    element-wise agreement with the independent scalar C restatement
    (oracle/dk_oracle.c).
  * unpack_to_int / dequantize: hand-packed words (0x76543210, 0x88888888,
    ...), round trip with the packer, and the C restatement.
  * linear_fp32: one-hot activations (each output equals one scaled weight),
    all-ones activations (per-group sums), brute-force pure-Python loops on
    tiny shapes, and the C restatement's float64 GEMV.
  * repack_paired / unpack_paired: hand-permuted words (0x76543210 ->
    0x75316420, 0x09ABCDEF -> 0x0ACE9BDF), inverse round trip, and the
    per-nibble definition on random words.
  * silu_f64: silu(0) = 0, the identity silu(-v) = silu(v) - v, limits at
    +-40, and agreement with v * scipy.special.expit(v).
  * gate_up_silu_f64 / mlp_decode_f64: brute-force pure-Python loops on tiny
    shapes, and one-hot activations that select single scaled weights.
The reference ships no golden-vector files; tests/golden/ holds fixtures this
oracle generated after being pinned as above, to catch regressions.
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 128
NIBBLES_PER_WORD = 8
QMIN, QMAX = -7, 7
SCALE_FLOOR = np.float32(1e-8)


def quantize_and_pack(w: np.ndarray, group_size: int = GROUP_SIZE):
    """fp32 W[M, K] -> (packed int32 [M, K/8], scales float16 [M, K/group]).

    Per group: amax in fp32; scale = max(fp32(amax / 7), fp32(1e-8));
    q = clamp(rint_half_even(fp32(w / scale)), -7, 7); pack q & 0xF at bit
    4n of word k//8 for n = k % 8; store scale rounded to fp16 (RNE).
    """
    w = np.asarray(w)
    if w.ndim != 2:
        raise ValueError("weight must be [M, K]")
    m, k = w.shape
    if k % group_size != 0:
        raise ValueError(f"K={k} is not divisible by group_size={group_size}")
    if k % NIBBLES_PER_WORD != 0:
        raise ValueError(f"K={k} is not divisible by {NIBBLES_PER_WORD}")
    g = w.astype(np.float32, copy=False).reshape(m, k // group_size, group_size)
    amax = np.abs(g).max(axis=-1)
    scale = np.maximum(amax / np.float32(QMAX), SCALE_FLOOR).astype(np.float32)
    q = np.clip(np.rint(g / scale[..., None]), QMIN, QMAX).astype(np.int64)
    nib = (q.reshape(m, k // NIBBLES_PER_WORD, NIBBLES_PER_WORD) & 0xF).astype(np.uint32)
    shifts = (4 * np.arange(NIBBLES_PER_WORD, dtype=np.uint32))
    words = np.bitwise_or.reduce(nib << shifts, axis=-1).astype(np.uint32)
    return words.view(np.int32), scale.astype(np.float16)


def unpack_to_int(packed: np.ndarray) -> np.ndarray:
    """int32/uint32 words [M, K/8] -> int32 q [M, K] in [-8, 7]."""
    u = np.asarray(packed).view(np.uint32)
    m, words = u.shape
    shifts = (4 * np.arange(NIBBLES_PER_WORD, dtype=np.uint32))
    nib = ((u[..., None] >> shifts) & np.uint32(0xF)).astype(np.int32)
    q = np.where(nib >= 8, nib - 16, nib)
    return q.reshape(m, words * NIBBLES_PER_WORD).astype(np.int32)


def dequantize(packed: np.ndarray, scales: np.ndarray, group_size: int = GROUP_SIZE,
               dtype=np.float32) -> np.ndarray:
    """W = q * float(scale) [M, K] (exact in fp32: |q| <= 8, scale is fp16)."""
    q = unpack_to_int(packed).astype(dtype)
    m, k = q.shape
    s = np.asarray(scales).astype(dtype).reshape(m, k // group_size, 1)
    return (q.reshape(m, k // group_size, group_size) * s).reshape(m, k)


def _as_batch(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x)
    return x[None, :] if x.ndim == 1 else x


def linear_fp32(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Y[B, M] = fp32(x) @ dequantize(packed, scales)^T, fp32 GEMM (the reference's CPU path)."""
    w = dequantize(packed, scales, dtype=np.float32)
    xv = _as_batch(x).astype(np.float32)
    return xv @ w.T


def linear_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Same product accumulated in float64 (a tighter reference for tests)."""
    w = dequantize(packed, scales, dtype=np.float64)
    xv = _as_batch(x).astype(np.float64)
    return xv @ w.T


def max_abs_err(y_kernel: np.ndarray, y_ref: np.ndarray) -> float:
    a = np.asarray(y_kernel, dtype=np.float64)
    b = np.asarray(y_ref, dtype=np.float64)
    return float(np.abs(a - b).max()) if a.size else 0.0


def fp16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of fp16 at |v| (the granularity of a kernel's fp16 output)."""
    a = np.abs(np.asarray(v, dtype=np.float64)).astype(np.float16)
    return np.spacing(a).astype(np.float64)


def bytes_moved_w4(m: int, k: int, batch: int) -> int:
    """Algorithmic HBM bytes of one GEMV: packed W + scales + x + y."""
    return m * (k // 2) + m * (k // GROUP_SIZE) * 2 + batch * k * 2 + batch * m * 2


def flop_gemv(m: int, k: int, batch: int) -> int:
    return 2 * m * k * batch


def make_case(m: int, k: int, batch: int, seed: int, w_std: float = 0.02):
    """Deterministic inputs: W ~ N(0, w_std) fp32, x ~ N(0, 1) fp16 (PCG64)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((m, k), dtype=np.float32) * np.float32(w_std)).astype(np.float32)
    x = rng.standard_normal((batch, k), dtype=np.float32).astype(np.float16)
    return w, x


def silu_f64(v: np.ndarray) -> np.ndarray:
    """SiLU in float64: v / (1 + exp(-v)) (torch.nn.functional.silu's definition)."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def gate_up_silu_f64(x, gate_packed, gate_scales, up_packed, up_scales) -> np.ndarray:
    """h[B, I] = silu(Wg x) * (Wu x) in float64, before any fp16 rounding."""
    g = linear_f64(x, gate_packed, gate_scales)
    u = linear_f64(x, up_packed, up_scales)
    return silu_f64(g) * u


def mlp_decode_f64(x, gate_packed, gate_scales, up_packed, up_scales, down_packed,
                   down_scales) -> np.ndarray:
    """y[B, H] = Wd fp16(silu(Wg x) * (Wu x)) in float64 around the one fp16
    rounding of h that the step's interface has (h is an fp16 tensor)."""
    h = gate_up_silu_f64(x, gate_packed, gate_scales, up_packed, up_scales).astype(np.float16)
    return linear_f64(h, down_packed, down_scales)


def mlp_bytes(i: int, h: int, batch: int) -> int:
    """Algorithmic HBM bytes of one MLP decode step: the three weight
    matrices and their scales, x, h written and read back, and y."""
    w = 3 * (i * h // 2 + i * h // GROUP_SIZE * 2)
    return w + batch * h * 2 + 2 * batch * i * 2 + batch * h * 2


def repack_paired(packed: np.ndarray) -> np.ndarray:
    """API-format words -> paired words: nibble 2j to bits 4j, nibble 2j+1 to bits 16+4j."""
    w = np.asarray(packed).astype(np.uint32)
    p = np.zeros_like(w)
    for j in range(4):
        p |= ((w >> np.uint32(8 * j)) & np.uint32(0xF)) << np.uint32(4 * j)
        p |= ((w >> np.uint32(8 * j + 4)) & np.uint32(0xF)) << np.uint32(16 + 4 * j)
    return p.view(np.int32)


def unpack_paired(paired: np.ndarray) -> np.ndarray:
    """Inverse of repack_paired."""
    p = np.asarray(paired).astype(np.uint32)
    w = np.zeros_like(p)
    for j in range(4):
        w |= ((p >> np.uint32(4 * j)) & np.uint32(0xF)) << np.uint32(8 * j)
        w |= ((p >> np.uint32(16 + 4 * j)) & np.uint32(0xF)) << np.uint32(8 * j + 4)
    return w.view(np.int32)
