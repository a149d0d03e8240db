"""Pins the CPU oracle (oracle/) before anything is checked against it.

Every function of the oracle is checked against something that is not a
retyping of its own formula: the reference's known-answer test, hand-derived
known answers, exact rational arithmetic, brute-force loops on tiny inputs,
and the independent scalar C restatement (oracle/dk_oracle.c).
"""

from __future__ import annotations

from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle, oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "w4a16_cases.npz"


# ---------------------------------------------------------------- helpers ---
def _round_binary(r: Fraction, mant_bits: int, emin: int) -> Fraction:
    """Exact round-half-even of r > 0 to a binary format with `mant_bits`
    explicit mantissa bits and minimum normal exponent `emin` (no overflow)."""
    if r == 0:
        return Fraction(0)
    e = r.numerator.bit_length() - r.denominator.bit_length()
    if Fraction(2) ** e > r:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant_bits)
    n = r / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl * ulp


def _expected_scale_bits(amax: float) -> int:
    """fp16 bits of fp16(max(fp32(amax/7), fp32(1e-8))) by exact arithmetic."""
    a = Fraction(float(np.float32(amax)))
    s32 = _round_binary(a / 7, 23, -126)
    floor32 = _round_binary(Fraction(1, 10**8), 23, -126)
    s32 = max(s32, floor32)
    s16 = _round_binary(s32, 10, -14)
    return int(np.float16(float(s16)).view(np.uint16))


def _word(packed, m, i):
    return int(np.asarray(packed)[m, i]) & 0xFFFFFFFF


# ------------------------------------------------ reference known answers ---
def test_reference_kat_low_nibble_first():
    # tests/test_quantize.py:41-53: w[0,0]=7, w[0,1]=-7 -> nibbles 0x7, 0x9, scale 1.
    w = np.zeros((1, 128), np.float32)
    w[0, 0], w[0, 1] = 7.0, -7.0
    for impl in (oracle, c_oracle):
        packed, scales = impl.quantize_and_pack(w)
        word = _word(packed, 0, 0)
        assert word & 0xF == 0x7
        assert (word >> 4) & 0xF == 0x9
        assert word == 0x00000097
        assert scales.shape == (1, 1)
        assert scales.view(np.uint16)[0, 0] == 0x3C00  # exactly 1.0


def test_kat_digit_ramp():
    # amax 7 -> scale 1 -> q = w; words by hand: 0x76543210 and 0x09ABCDEF.
    w = np.zeros((1, 128), np.float32)
    w[0, :8] = np.arange(8)
    w[0, 8:15] = -np.arange(1, 8)
    for impl in (oracle, c_oracle):
        packed, _ = impl.quantize_and_pack(w)
        assert _word(packed, 0, 0) == 0x76543210
        assert _word(packed, 0, 1) == 0x09ABCDEF
        assert all(_word(packed, 0, i) == 0 for i in range(2, 16))


def test_kat_ties_to_even():
    # scale 1 exactly; 0.5->0, 1.5->2, 2.5->2, 3.5->4, -0.5->0, -1.5->-2, -2.5->-2, 7->7.
    w = np.zeros((1, 128), np.float32)
    w[0, :8] = [0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, 7.0]
    for impl in (oracle, c_oracle):
        packed, _ = impl.quantize_and_pack(w)
        assert _word(packed, 0, 0) == 0x7EE04220


@pytest.mark.parametrize("amax", [1.0, 0.3, 0.05, 100.0, 3e-4, 6.1e-5, 1e-9, 65504.0 * 7])
def test_scale_rounding_exact(amax):
    # Scale = fp16(fp32(amax / 7)) with the 1e-8 floor, checked by exact rationals.
    w = np.zeros((1, 128), np.float32)
    w[0, 5] = -amax
    for impl in (oracle, c_oracle):
        _, scales = impl.quantize_and_pack(w)
        assert int(scales.view(np.uint16)[0, 0]) == _expected_scale_bits(amax)


def test_zero_group_scale_underflows_to_zero():
    # tests/test_quantize.py:56-61: finite; 1e-8 is below half the fp16 subnormal step.
    w = np.zeros((2, 256), np.float32)
    w[1, 128:] = 0.5
    for impl in (oracle, c_oracle):
        packed, scales = impl.quantize_and_pack(w)
        s = scales.view(np.uint16)
        assert s[0, 0] == 0 and s[0, 1] == 0 and s[1, 0] == 0
        assert np.all(np.asarray(packed)[0] == 0)
        assert np.isfinite(oracle.dequantize(packed, scales)).all()


@pytest.mark.parametrize(
    "word,expected",
    [
        (0x76543210, [0, 1, 2, 3, 4, 5, 6, 7]),
        (0x01234567, [7, 6, 5, 4, 3, 2, 1, 0]),
        (0x88888888, [-8] * 8),
        (0x77777777, [7] * 8),
        (0xFEDCBA98, [-8, -7, -6, -5, -4, -3, -2, -1]),
        (0x00000000, [0] * 8),
    ],
)
def test_unpack_hand_words(word, expected):
    packed = np.array([[word] * 16], dtype=np.uint32).view(np.int32)
    for impl in (oracle, c_oracle):
        q = impl.unpack_to_int(packed)
        assert q.shape == (1, 128)
        assert q[0, :8].tolist() == expected
        assert q[0, 120:].tolist() == expected


# ------------------------------------------------ reference invariants ---
@pytest.mark.parametrize("shape", [(8, 128), (16, 256), (32, 512)])
def test_roundtrip_q_range_and_dequant(shape):
    # tests/test_quantize.py:16-25.
    rng = np.random.Generator(np.random.PCG64(0))
    w = rng.standard_normal(shape, dtype=np.float32)
    packed, scales = oracle.quantize_and_pack(w)
    q = oracle.unpack_to_int(packed)
    assert q.min() >= -7 and q.max() <= 7
    recon = oracle.dequantize(packed, scales)
    s = np.repeat(scales.astype(np.float32), 128, axis=1)
    assert np.array_equal(recon, q.astype(np.float32) * s)  # exact, not just 1e-6


@pytest.mark.parametrize("shape", [(8, 128), (16, 256)])
def test_reconstruction_within_half_step(shape):
    # tests/test_quantize.py:28-38.
    rng = np.random.Generator(np.random.PCG64(0))
    w = rng.standard_normal(shape, dtype=np.float32)
    packed, scales = oracle.quantize_and_pack(w)
    recon = oracle.dequantize(packed, scales)
    s = np.repeat(scales.astype(np.float32), 128, axis=1)
    assert np.all(np.abs(recon - w) <= 0.5 * s + 1e-3)


# ------------------------------------------------ numpy vs scalar C ---
@pytest.mark.parametrize("m,k,seed,std", [(7, 128, 1, 1.0), (33, 384, 2, 0.02), (64, 1024, 3, 0.05),
                                          (16, 11008, 4, 0.02)])
def test_numpy_and_c_restatements_agree(m, k, seed, std):
    w, x = oracle.make_case(m, k, 3, seed, std)
    p1, s1 = oracle.quantize_and_pack(w)
    p2, s2 = c_oracle.quantize_and_pack(w)
    assert np.array_equal(p1, p2)
    assert np.array_equal(s1.view(np.uint16), s2.view(np.uint16))
    assert np.array_equal(oracle.unpack_to_int(p1), c_oracle.unpack_to_int(p1))
    y64 = oracle.linear_f64(x, p1, s1)
    assert np.allclose(y64, c_oracle.gemv_f64(x, p1, s1), rtol=1e-12, atol=1e-12)
    # The fp32 product (the reference's CPU path) stays within fp32 rounding of it.
    assert oracle.max_abs_err(oracle.linear_fp32(x, p1, s1), y64) < 1e-3


def test_fp16_conversion_matches_ieee_on_edges():
    # Hand-written RNE conversion in the C oracle vs numpy's IEEE conversion on
    # every finite fp16 value, the midpoints between neighbours, and one fp32
    # ulp either side of both.
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mid = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    base = np.concatenate([h, mid])
    vals = np.concatenate([base, np.nextafter(base, np.float32(np.inf)),
                           np.nextafter(base, np.float32(0))])
    vals = np.concatenate([vals, -vals[::7]])
    rng = np.random.Generator(np.random.PCG64(5))
    pick = rng.choice(vals.size, 60000, replace=False)
    sub = vals[pick]
    with np.errstate(over="ignore"):
        ref = sub.astype(np.float16).view(np.uint16)
    got = np.array([c_oracle.f32_to_f16_bits(float(v)) for v in sub], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_fp16_rounding_and_doubling():
    # The GPU linearity checks compare y(2x) with 2 y(x): rounding an fp32
    # value t to fp16 commutes with doubling when fp16(t) is normal, and in
    # the subnormal range the two differ by at most 2**-23. Both facts on
    # every fp32 value around the subnormal/normal boundary and a random
    # sample across the range.
    rng = np.random.Generator(np.random.PCG64(9))
    edge = np.arange(0, 3 << 20, 7, dtype=np.uint32) + np.uint32(0x33000000)  # ~2**-25 .. 2**-13
    t = np.concatenate([edge.view(np.float32),
                        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0)])
    t = np.concatenate([t, -t])
    y1 = t.astype(np.float16)
    y2 = (t * np.float32(2)).astype(np.float16)
    normal = np.abs(y1.astype(np.float32)) >= 2.0 ** -14
    assert np.array_equal(y2[normal].view(np.uint16), (y1[normal] * np.float16(2)).view(np.uint16))
    diff = np.abs(y2[~normal].astype(np.float64) - 2 * y1[~normal].astype(np.float64))
    assert diff.max() <= 2.0 ** -23 and (diff > 0).any()  # the exception is real


# ------------------------------------------------ GEMV closed forms ---
def test_gemv_one_hot_picks_single_weights():
    w, _ = oracle.make_case(6, 256, 1, 21, 0.05)
    packed, scales = oracle.quantize_and_pack(w)
    q = oracle.unpack_to_int(packed)
    for k in (0, 1, 7, 8, 127, 128, 200, 255):
        x = np.zeros((1, 256), np.float16)
        x[0, k] = 1.0
        y = oracle.linear_f64(x, packed, scales)[0]
        expect = scales[:, k // 128].astype(np.float64) * q[:, k]
        assert np.array_equal(y, expect)


def test_gemv_ones_gives_group_sums():
    w, _ = oracle.make_case(5, 384, 1, 22, 0.05)
    packed, scales = oracle.quantize_and_pack(w)
    q = oracle.unpack_to_int(packed).reshape(5, 3, 128).sum(-1)
    y = oracle.linear_f64(np.ones((1, 384), np.float16), packed, scales)[0]
    assert np.allclose(y, (q * scales.astype(np.float64)).sum(-1), rtol=0, atol=1e-12)


def test_gemv_brute_force_tiny():
    w, x = oracle.make_case(3, 128, 2, 23, 0.05)
    packed, scales = oracle.quantize_and_pack(w)
    words = np.asarray(packed).view(np.uint32)
    y = oracle.linear_f64(x, packed, scales)
    for b in range(2):
        for m in range(3):
            acc = 0.0
            for k in range(128):
                nib = (int(words[m, k // 8]) >> (4 * (k % 8))) & 0xF
                qv = nib - 16 if nib >= 8 else nib
                acc += float(scales[m, 0]) * qv * float(x[b, k])
            assert abs(acc - y[b, m]) < 1e-12


def test_bytes_moved_matches_reference_formula():
    # bench/common.py:111-117 at 4096x4096 B=1 (8,667,136 B for one c0 launch).
    assert oracle.bytes_moved_w4(4096, 4096, 1) == 8_667_136
    assert oracle.flop_gemv(4096, 4096, 1) == 33_554_432


# ------------------------------------------------ golden fixtures ---
def _golden_cases():
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    return data, names


def test_golden_fixtures_reproduce():
    data, names = _golden_cases()
    assert len(names) >= 5
    for n in names:
        w, x = data[f"{n}/w"], data[f"{n}/x"]
        packed, scales = oracle.quantize_and_pack(w)
        assert np.array_equal(packed, data[f"{n}/packed"]), n
        assert np.array_equal(scales.view(np.uint16), data[f"{n}/scales"].view(np.uint16)), n
        assert np.array_equal(oracle.linear_f64(x, packed, scales), data[f"{n}/y"]), n


# ------------------------------------------------------- MLP decode step ---
def test_silu_closed_forms():
    from scipy.special import expit

    assert oracle.silu_f64(0.0) == 0.0
    v = np.linspace(-30, 30, 601)
    # silu(-v) = -v * sigmoid(-v) = -v * (1 - sigmoid(v)) = silu(v) - v
    np.testing.assert_allclose(oracle.silu_f64(-v), oracle.silu_f64(v) - v, rtol=0, atol=1e-12)
    np.testing.assert_allclose(oracle.silu_f64(v), v * expit(v), rtol=1e-14, atol=1e-300)
    assert abs(oracle.silu_f64(40.0) - 40.0) < 1e-15 * 40 * 1e3
    assert 0 > oracle.silu_f64(-40.0) > -1e-15
    assert oracle.silu_f64(1.0) == pytest.approx(1.0 / (1.0 + np.e ** -1.0), rel=1e-15)


def _brute_linear(x, packed, scales):
    q = [[((int(packed[m, i // 8]) >> (4 * (i % 8))) & 0xF) for i in range(packed.shape[1] * 8)]
         for m in range(packed.shape[0])]
    q = [[v - 16 if v >= 8 else v for v in row] for row in q]
    out = []
    for b in range(x.shape[0]):
        row = []
        for m in range(packed.shape[0]):
            acc = 0.0
            for k in range(len(q[m])):
                acc += float(scales[m, k // 128]) * q[m][k] * float(x[b, k])
            row.append(acc)
        out.append(row)
    return out


def test_gate_up_and_mlp_brute_force_tiny():
    import math

    rng = np.random.Generator(np.random.PCG64(99))
    I, H, B = 128, 128, 2
    gp, gs = oracle.quantize_and_pack(rng.standard_normal((I, H)).astype(np.float32) * 0.1)
    up, us = oracle.quantize_and_pack(rng.standard_normal((I, H)).astype(np.float32) * 0.1)
    dp, ds = oracle.quantize_and_pack(rng.standard_normal((H, I)).astype(np.float32) * 0.1)
    x = rng.standard_normal((B, H)).astype(np.float16)
    g, u = _brute_linear(x, gp, gs), _brute_linear(x, up, us)
    h_ref = np.array([[g[b][i] / (1 + math.exp(-g[b][i])) * u[b][i] for i in range(I)]
                      for b in range(B)])
    h = oracle.gate_up_silu_f64(x, gp, gs, up, us)
    np.testing.assert_allclose(h, h_ref, rtol=1e-12, atol=1e-12)
    y_ref = np.array(_brute_linear(h_ref.astype(np.float16), dp, ds))
    y = oracle.mlp_decode_f64(x, gp, gs, up, us, dp, ds)
    np.testing.assert_allclose(y, y_ref, rtol=1e-12, atol=1e-12)


def test_gate_up_one_hot_selects_weights():
    # x = e_k: g = Wg[:, k], u = Wu[:, k] exactly (scale * q).
    rng = np.random.Generator(np.random.PCG64(5))
    I, H = 64, 256
    gp, gs = oracle.quantize_and_pack(rng.standard_normal((I, H)).astype(np.float32))
    up, us = oracle.quantize_and_pack(rng.standard_normal((I, H)).astype(np.float32))
    x = np.zeros((1, H), np.float16)
    x[0, 131] = 1.0
    wg = oracle.dequantize(gp, gs, dtype=np.float64)[:, 131]
    wu = oracle.dequantize(up, us, dtype=np.float64)[:, 131]
    h = oracle.gate_up_silu_f64(x, gp, gs, up, us)[0]
    np.testing.assert_array_equal(h, wg / (1 + np.exp(-wg)) * wu)


def test_mlp_bytes_formula():
    # 7B MLP: three 11008 x 4096 int4 matrices plus fp16 scales, x, h twice, y.
    w = 11008 * 4096 // 2 + 11008 * 32 * 2
    assert oracle.mlp_bytes(11008, 4096, 1) == 3 * w + 4096 * 2 + 2 * 11008 * 2 + 4096 * 2


# ------------------------------------------------------- paired layout ---
def test_paired_layout_hand_words():
    w = np.array([[0x76543210, 0x09ABCDEF]], dtype=np.uint32).view(np.int32)
    p = oracle.repack_paired(w).view(np.uint32)
    assert int(p[0, 0]) == 0x75316420
    assert int(p[0, 1]) == 0x0ACE9BDF
    np.testing.assert_array_equal(oracle.unpack_paired(oracle.repack_paired(w)), w)


def test_paired_layout_per_nibble_definition():
    rng = np.random.Generator(np.random.PCG64(17))
    w = rng.integers(0, 1 << 32, size=(8, 64), dtype=np.uint64).astype(np.uint32).view(np.int32)
    p = oracle.repack_paired(w).view(np.uint32)
    for (m, i), word in np.ndenumerate(w.view(np.uint32)):
        nib = [(int(word) >> (4 * n)) & 0xF for n in range(8)]
        pw = int(p[m, i])
        for j in range(4):
            assert (pw >> (4 * j)) & 0xF == nib[2 * j]
            assert (pw >> (16 + 4 * j)) & 0xF == nib[2 * j + 1]
    np.testing.assert_array_equal(oracle.unpack_paired(oracle.repack_paired(w)), w)
