"""Pins the oracle's quantisers against the reference's known answers,
invariants and an exact-arithmetic brute force (CPU only)."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import fq_oracle as O


def _bf16_randn(rng, shape, scale=1.0):
    return O.round_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def test_pack_kat_masks_high_nibble():
    # tests/test_kv_quant_int4.py:26-31
    packed = O.pack_int4(np.array([[0, 15, 16, 255]], dtype=np.uint8))
    assert O.unpack_int4(packed).tolist() == [[0, 15, 0, 15]]


def test_pack_layout_low_nibble_is_even_channel():
    # kv_quant.py:104-115: byte k low nibble = x[2k], high nibble = x[2k+1]
    packed = O.pack_int4(np.array([1, 2, 3, 4], dtype=np.uint8))
    assert packed.tolist() == [0x21, 0x43]


def test_pack_roundtrip():
    rng = np.random.default_rng(0)
    x = rng.integers(0, 16, (2, 3, 4, 8)).astype(np.uint8)
    p = O.pack_int4(x)
    assert p.shape == (2, 3, 4, 4)
    assert np.array_equal(O.unpack_int4(p), x)


def test_bf16_rounding_known_values():
    assert O.f32_to_bf16_bits(np.array([1.0], np.float32))[0] == 0x3F80
    # 1 + 2^-8 is exactly half way between 1 and 1 + 2^-7: ties to even (1.0)
    assert O.round_bf16(np.array([1.0 + 2 ** -8], np.float32))[0] == 1.0
    assert O.round_bf16(np.array([1.0 + 3 * 2 ** -8], np.float32))[0] == 1.0 + 2 ** -6
    assert O.round_bf16(np.array([-1.0 - 2 ** -9], np.float32))[0] == -1.0


def test_quantize_k_shapes_and_odd_dim():
    rng = np.random.default_rng(0)
    K = _bf16_randn(rng, (2, 4, 128, 64))
    p, s, m = O.quantize_k_int4(K, 64)
    assert p.shape == (2, 4, 128, 32) and s.shape == (2, 4, 2, 64) and m.shape == (2, 4, 2, 64)
    with pytest.raises(ValueError, match="even head_dim"):
        O.quantize_k_int4(_bf16_randn(rng, (1, 2, 64, 65)), 64)


@pytest.mark.parametrize("dtype,meta", [("bf16", "bf16"), ("f16", "f16"), ("f16", "bf16")])
def test_quantize_k_roundtrip_and_page_max_identity(dtype, meta):
    # tests/test_kv_quant_int4.py:47-66
    rng = np.random.default_rng(42)
    rnd = O.rounder(dtype)
    K = rnd((rng.standard_normal((2, 4, 128, 64)) * 2).astype(np.float32))
    p, s, m = O.quantize_k_int4(K, 64, dtype, meta)
    rec = O.dequant_k(p, s, m, 64)
    tok_s = np.repeat(s, 64, axis=-2)
    assert (np.abs(rec - K) <= tok_s + 1e-2).all()
    page_max = K.reshape(2, 4, 2, 64, 64).max(axis=3)
    page_min = K.reshape(2, 4, 2, 64, 64).min(axis=3)
    # max is recovered up to the half-precision rounding of (max - min) and of
    # the scale (2 roundings of relative size 2^-8 for bf16, 2^-11 for fp16)
    ulp = 2.0 ** (-8 if "bf16" in (dtype, meta) else -11)
    err = np.abs(m.astype(np.float64) + 15 * s - page_max)
    assert (err <= 2 * ulp * (page_max - page_min) + 1e-6).all()
    if meta == dtype:
        assert np.array_equal(m, page_min)          # min stored exactly


def test_quantize_k_codes_equal_exact_rational_rounding():
    """Brute force: each code equals round_half_even((k - mn) / scale) computed
    in exact rational arithmetic, clamped to 0..15, except where the exact
    quotient lies within fp32 resolution of a half-integer."""
    rng = np.random.default_rng(3)
    K = _bf16_randn(rng, (1, 2, 70, 16), 3.0)      # partial last page (70 = 64 + 6)
    p, s, m = O.quantize_k_int4(K, 64)
    codes = O.unpack_int4(p)
    checked = 0
    for h in range(2):
        for t in range(70):
            pg = t // 64
            for d in range(16):
                num = Fraction(float(K[0, h, t, d])) - Fraction(float(m[0, h, pg, d]))
                q = num / Fraction(float(s[0, h, pg, d]))
                fl = q.numerator // q.denominator
                frac = q - fl
                if abs(frac - Fraction(1, 2)) < Fraction(1, 10 ** 5):
                    continue
                exp = fl + 1 if frac > Fraction(1, 2) else fl
                exp = min(max(exp, 0), 15)
                assert codes[0, h, t, d] == exp, (h, t, d)
                checked += 1
    assert checked > 2000


def test_quantize_k_scale_arithmetic_is_in_half_precision():
    # tests/test_selection_flips.py:183-194: a channel whose range is 1.5e-5
    # has (max - min) / 15 <= 1e-6 in bf16 arithmetic, so the scale is the
    # bf16 epsilon clamp; in fp32 the ratio would exceed 1e-6.
    K = np.zeros((1, 1, 64, 2), np.float32)
    K[:, :, 63] = O.round_bf16(np.array([1.5e-5], np.float32))[0]
    hi = K.max(axis=2)
    assert (O.round_bf16(O.round_bf16(hi) * O.INV15) <= 1e-6).all()
    assert (hi / 15 > 1e-6).all()
    _, s, _ = O.quantize_k_int4(K, 64)
    assert np.all(s == O.round_bf16(np.array([1e-6], np.float32))[0])


def test_constant_channel_gives_epsilon_scale_and_zero_codes():
    K = np.full((1, 1, 64, 4), 0.75, np.float32)
    p, s, m = O.quantize_k_int4(K, 64)
    assert np.all(O.unpack_int4(p) == 0)
    assert np.all(m == 0.75)
    assert np.all(s == O.round_bf16(np.array([1e-6], np.float32)))


def test_quantize_v_shapes_roundtrip():
    # tests/test_kv_quant_int4.py:69-87
    rng = np.random.default_rng(1)
    V = _bf16_randn(rng, (2, 4, 32, 64))
    p, s, m = O.quantize_v_int4(V)
    assert p.shape == (2, 4, 32, 32) and s.shape == (2, 4, 32, 1) and m.shape == (2, 4, 32, 1)
    rec = O.dequant_v(p, s, m)
    assert (np.abs(rec - V) <= s + 1e-2).all()


def test_quantize_v_group32_is_independent_per_group():
    rng = np.random.default_rng(2)
    V = O.round_f16(rng.standard_normal((1, 2, 16, 128)).astype(np.float32))
    p, s, m = O.quantize_v_int4(V, group=32, meta="f16")
    assert s.shape == (1, 2, 16, 4)
    for g in range(4):
        pg, sg, mg = O.quantize_v_int4(V[..., 32 * g:32 * g + 32], meta="f16")
        assert np.array_equal(O.unpack_int4(p)[..., 32 * g:32 * g + 32], O.unpack_int4(pg))
        assert np.array_equal(s[..., g:g + 1], sg) and np.array_equal(m[..., g:g + 1], mg)
    rec = O.dequant_v(p, s, m)
    assert (np.abs(rec - V) <= np.repeat(s, 32, axis=-1) * 0.51 + 1e-3).all()


def test_quantize_v_codes_use_fp32_scale_not_stored_meta():
    """kv_quant.py:197-205: codes are computed with the fp32 scale; the stored
    scale is rounded to bf16 afterwards, so for a token whose fp32 scale is not
    bf16-representable, re-deriving codes from the stored meta can differ."""
    rng = np.random.default_rng(11)
    V = _bf16_randn(rng, (1, 1, 4096, 64))
    p, s, m = O.quantize_v_int4(V)
    codes = O.unpack_int4(p).astype(np.int64)
    mn = V.min(-1, keepdims=True)
    sc32 = np.maximum((V.max(-1, keepdims=True) - mn) * O.INV15, O.EPS)
    assert np.array_equal(codes, np.clip(np.rint((V - mn) / sc32), 0, 15))
    alt = np.clip(np.rint((V - m) / s), 0, 15)
    assert not np.array_equal(codes, alt)
