"""Pins the oracle's scoring and selection (CPU only)."""
import math

import numpy as np
import pytest

from oracle import fq_oracle as O


def _sel(scores, retention, sinks=0, window=0, kmax=None):
    s = np.asarray(scores, np.float32)
    return O.select_pages_vectorized(s, retention, sinks, window, kmax)


def test_kat_topk_picks_highest():
    # tests/test_eager_selection.py:22-27
    m = _sel([[[[0.1, 0.9, 0.2, 0.8, 0.3, 0.7]]]], 0.5)
    assert m[0, 0, 0].tolist() == [False, True, False, True, False, True]


def test_kat_retention_rounds_up_to_one():
    # tests/test_eager_selection.py:39-44
    m = _sel([[[[0.1, 0.4, 0.2, 0.3]]]], 0.1)
    assert m.sum() == 1 and m[0, 0, 0, 1]


def test_kat_zero_retention_sinks_and_window():
    # tests/test_eager_selection.py:14-19
    m = _sel(np.zeros((1, 1, 1, 8)), 0.0, sinks=1, window=2)
    assert m[0, 0, 0].tolist() == [True, False, False, False, False, False, True, True]


def test_kat_full_retention_and_clamp():
    # tests/test_select_pages_vectorized.py:45-58
    rng = np.random.default_rng(0)
    assert _sel(rng.standard_normal((1, 4, 1, 16)), 1.0).all()
    assert _sel(rng.standard_normal((1, 2, 1, 4)), 0.0, sinks=10, window=10).all()


def test_kat_per_head_independent():
    # tests/test_eager_selection.py:30-36
    s = np.array([[[[0.9, 0.0, 0.0, 0.1]], [[0.0, 0.0, 0.9, 0.1]]]], np.float32)
    m = _sel(s, 0.25)
    assert m[0, 0, 0, 0] and not m[0, 0, 0, 2] and m[0, 1, 0, 2] and not m[0, 1, 0, 0]


def test_fp32_ceil_rule():
    # tests/test_selection_flips.py:170-180: ceil(fp32(.07) * 100) == 7, not 8
    assert math.ceil(.07 * 100) == 8
    assert O.k_per_head(0.07, 1, 100)[0] == 7


def test_per_head_retention_vector_and_kmax_static():
    rng = np.random.default_rng(42)
    s = rng.standard_normal((1, 6, 1, 32)).astype(np.float32)
    r = np.array([0.0, 0.1, 0.25, 0.5, 0.75, 1.0], np.float32)
    m = _sel(s, r, sinks=2, window=1)
    k = [0, 4, 8, 16, 24, 32]
    for h in range(6):
        top = set(np.argsort(-s[0, h, 0], kind="stable")[:k[h]].tolist())
        expect = top | {0, 1, 31}
        assert set(np.nonzero(m[0, h, 0])[0].tolist()) == expect
    # a static k_max below k_h truncates the top-k (selection.py:107-117)
    m2 = _sel(s, 0.5, kmax=3)
    assert m2.sum(-1).max() == 3


def test_brute_force_against_full_sort():
    rng = np.random.default_rng(7)
    for P in (4, 16, 64, 200):
        s = rng.standard_normal((2, 3, 1, P)).astype(np.float32)
        for r in (0.0, 0.1, 0.25, 0.5, 1.0):
            m = _sel(s, r)
            k = int(np.ceil(np.float32(r) * np.float32(P)))
            for b in range(2):
                for h in range(3):
                    order = sorted(range(P), key=lambda i: (-float(s[b, h, 0, i]), i))
                    assert set(np.nonzero(m[b, h, 0])[0]) == set(order[:k])


def test_ties_go_to_lower_index():
    s = np.array([[[[1.0, 2.0, 2.0, 2.0, 0.5]]]], np.float32)
    m = _sel(s, 0.4)          # k = 2
    assert m[0, 0, 0].tolist() == [False, True, True, False, False]
    z = np.array([[[[-0.0, 0.0, -1.0]]]], np.float32)
    assert _sel(z, 0.3)[0, 0, 0].tolist() == [True, False, False]


def test_compact_kats():
    # tests/test_build_compact_selection.py:8-73
    mask = np.zeros((1, 1, 1, 8), bool)
    mask[..., [1, 3, 5]] = True
    for bm in (4, 8, 16):
        out = O.build_compact_selection(mask, bm)
        assert out.shape == (1, 1, 1, bm) and out.dtype == np.int32
        assert out[0, 0, 0, :3].tolist() == [5, 3, 1]
        assert (out[0, 0, 0, 3:] == -1).all()
    assert (O.build_compact_selection(np.zeros((1, 1, 1, 8), bool), 4) == -1).all()
    assert sorted(O.build_compact_selection(np.ones((1, 1, 1, 4), bool), 4)[0, 0, 0]) == [0, 1, 2, 3]
    m = np.array([[[[True, False, True, True]]]])
    out = O.build_compact_selection(m, 8)
    assert out[0, 0, 0].tolist() == [3, 2, 0, -1, -1, -1, -1, -1]
    # truncation keeps the largest ids (sorted descending, then sliced)
    assert O.build_compact_selection(np.ones((1, 1, 1, 6), bool), 2)[0, 0, 0].tolist() == [5, 4]
    with pytest.raises(ValueError):
        O.build_compact_selection(mask, 0)


def test_compact_no_duplicates_when_topk_overlaps_forced():
    # tests/test_build_compact_selection_overlap.py:9-35
    s = np.zeros((1, 1, 1, 16), np.float32)
    s[0, 0, 0, 0], s[0, 0, 0, 1], s[0, 0, 0, 14] = 10, 9, 1
    m = _sel(s, 0.25, sinks=4, window=2, kmax=4)
    ids = [i for i in O.build_compact_selection(m, 8)[0, 0, 0] if i != -1]
    assert len(ids) == len(set(ids)) and sorted(ids) == np.nonzero(m[0, 0, 0])[0].tolist()


def test_scores_fixed_match_quest_bound_identity():
    # tests/test_eager_criticality.py:42-70: fast form == sum_d max(q mn, q mx)
    rng = np.random.default_rng(11)
    Q = rng.standard_normal((1, 4, 64)).astype(np.float32)
    mn = O.round_bf16(rng.standard_normal((1, 2, 8, 64)).astype(np.float32))
    sc = O.round_bf16((np.abs(rng.standard_normal((1, 2, 8, 64))) + 1e-3).astype(np.float32))
    slow = O.page_scores_quest(Q, mn, mn.astype(np.float64) + 15.0 * sc)
    fast = O.page_scores_fixed(Q, sc, mn)
    assert np.allclose(fast, slow, rtol=1e-3, atol=1e-3)
    ex = O.page_scores_int4_exact(Q, sc, mn)
    assert np.allclose(ex, slow, rtol=1e-12, atol=1e-9)
    # fp32 fixed order stays within fp32 accumulation error of the fp64 value
    assert np.abs(fast - ex).max() < 1e-4 * np.abs(ex).max()


def test_scores_upper_bound_true_page_max_with_exact_summaries():
    # tests/test_eager_criticality.py:17-29
    rng = np.random.default_rng(0)
    Q = rng.standard_normal((1, 1, 8)).astype(np.float32)
    K = rng.standard_normal((1, 1, 16, 8)).astype(np.float32)
    pmin = K.reshape(1, 1, 4, 4, 8).min(3)
    pmax = K.reshape(1, 1, 4, 4, 8).max(3)
    s = O.page_scores_quest(Q, pmin, pmax)
    qk = np.einsum("bhd,bhsd->bhs", Q, K).reshape(1, 1, 4, 4).max(-1)
    assert (s >= qk - 1e-5).all()


def test_scores_fixed_per_kv_sum_and_sensitivity():
    rng = np.random.default_rng(5)
    Q = rng.standard_normal((1, 6, 128)).astype(np.float32)
    mn = O.round_bf16(rng.standard_normal((1, 2, 5, 128)).astype(np.float32))
    sc = O.round_bf16(np.abs(rng.standard_normal((1, 2, 5, 128))).astype(np.float32))
    per_q = O.page_scores_fixed(Q, sc, mn, "per_q_head")
    per_kv = O.page_scores_fixed(Q, sc, mn, "per_kv_head_sum")
    assert np.allclose(per_kv, per_q.reshape(1, 2, 3, 5).sum(2), rtol=1e-5, atol=1e-4)
    # the 15x factor and the relu matter (a dropped term changes the value)
    ex = O.page_scores_int4_exact(Q, sc, mn)
    no_relu = (Q.reshape(1, 2, 3, 128).astype(np.float64) @ (mn + 15 * sc).transpose(0, 1, 3, 2).astype(np.float64)).reshape(1, 6, 5)
    assert np.abs(ex - no_relu).max() > 1.0
    assert np.allclose(per_q, ex, rtol=1e-4, atol=1e-3)


def _rn32_exact(fr):
    """Round a Fraction to the nearest fp32 (ties to even) with integer arithmetic."""
    from fractions import Fraction
    if fr == 0:
        return np.float32(0.0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()   # 2^e ~ a
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    q = max(e - 23, -149)                      # quantum of the fp32 grid at a
    m = a / Fraction(2) ** q
    lo = m.numerator // m.denominator
    rem = m - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    return np.float32(sign * lo * 2.0 ** q)


def test_fma32_is_correctly_rounded():
    # fma32 against exact rational arithmetic: random triples over a wide range of
    # magnitudes, products with fp16/bf16 operands (the scoring case), and triples
    # built so that the fp64 sum lands exactly halfway between fp32 neighbours
    # (where fp64-then-fp32 rounding would round twice)
    from fractions import Fraction
    rng = np.random.default_rng(123)
    a = (rng.standard_normal(4000) * 2.0 ** rng.integers(-20, 20, 4000)).astype(np.float32)
    b = O.round_f16(rng.standard_normal(4000).astype(np.float32))
    c = (rng.standard_normal(4000) * 2.0 ** rng.integers(-30, 30, 4000)).astype(np.float32)
    # ties: products of exactly half an ulp of c (ties go to even)
    n = 200
    c3 = np.full(n, 1.0 + 2.0 ** -23, np.float32)
    a3 = np.full(n, 2.0 ** -24, np.float32)
    b3 = rng.choice([-1.0, 1.0], n).astype(np.float32)
    # double-rounding traps: a*b = +-2^-24 (1 - 2^-36) on c = +-(1 + 2^-23); the fp64
    # sum lands exactly on the fp32 midpoint, the exact sum just short of it
    a4 = np.array([1.0 + 2.0 ** -18, -(1.0 + 2.0 ** -18)], np.float32)
    b4 = np.array([2.0 ** -24 * (1.0 - 2.0 ** -18)] * 2, np.float32)
    c4 = np.array([1.0 + 2.0 ** -23, -(1.0 + 2.0 ** -23)], np.float32)
    A = np.concatenate([a, a3, a4])
    B = np.concatenate([b, b3, b4])
    C = np.concatenate([c, c3, c4])
    got = O.fma32(A, B, C)
    for x, y, z, g in zip(A, B, C, got):
        want = _rn32_exact(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
        assert g == want, (x, y, z, g, want)
    # the traps: exact results 1 + 2^-23 (rounding the fp64 sum again would give 1 + 2^-22)
    assert got[-2] == np.float32(1.0 + 2.0 ** -23) and got[-1] == np.float32(-(1.0 + 2.0 ** -23))
    naive = (A[-2:].astype(np.float64) * B[-2:] + C[-2:]).astype(np.float32)
    assert naive[0] == np.float32(1.0 + 2.0 ** -22)          # the trap is real


def test_scores_fixed_order_brute_force():
    # page_scores_fixed restated one lane at a time with scalar exact FMAs
    from fractions import Fraction
    rng = np.random.default_rng(5)
    Q = rng.standard_normal((1, 2, 128)).astype(np.float32)
    mn = O.round_f16(rng.standard_normal((1, 1, 3, 128)).astype(np.float32))
    sc = O.round_f16(np.abs(rng.standard_normal((1, 1, 3, 128))).astype(np.float32))
    got = O.page_scores_fixed(Q, sc, mn)

    def lane_sums(q, m):
        t = []
        for j in range(16):
            acc = np.float32(q[8 * j] * m[8 * j])
            for i in range(1, 8):
                d = 8 * j + i
                acc = _rn32_exact(Fraction(float(q[d])) * Fraction(float(m[d])) + Fraction(float(acc)))
            t.append(acc)
        t = np.array(t, np.float32)
        idx = np.arange(16)
        for pa in (15 - idx, (idx & ~7) | (7 - (idx & 7)), idx ^ 1, idx ^ 2):
            t = (t + t[pa]).astype(np.float32)
        return t[0]
    for h in range(2):
        for p in range(3):
            q = Q[0, h]
            t1 = lane_sums(q, mn[0, 0, p])
            t2 = lane_sums(np.maximum(q, 0).astype(np.float32), sc[0, 0, p])
            want = np.float32(t1 + np.float32(t2 * np.float32(15.0)))
            assert got[0, h, p] == want
