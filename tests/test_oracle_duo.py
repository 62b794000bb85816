"""Oracle pins for the DuoAttention dispatch's scoring and selection
(duo/fused_dispatch.py:64-72): page_summary_int8, page_scores_quest_fixed
and the per-head loop form select_pages, on the CPU."""
import math

import numpy as np
import torch

from oracle import fq_oracle as O


def _int8_cache(seed, B=1, H=2, S=200, D=16, page=64):
    rng = np.random.default_rng(seed)
    K = O.round_bf16((rng.standard_normal((B, H, S, D)) * rng.lognormal(0, 1, (B, H, 1, D))).astype(np.float32))
    return O.quantize_k_int8(K, page)


def test_page_summary_equals_the_reference_expressions_in_torch():
    """dequantize_k (kv_quant.py:64-75) and compute_page_summary
    (page_summary.py:7-39) evaluated by torch on the CPU, bit for bit,
    including a partial last page (S = 200: 3 pages + 8 tokens)."""
    codes, scale, mn = _int8_cache(1)
    page = 64
    lo, hi = O.page_summary_int8(codes, scale, mn, page)
    c = torch.from_numpy(codes)
    s = torch.from_numpy(scale).to(torch.bfloat16)
    m = torch.from_numpy(mn).to(torch.bfloat16)
    S = c.shape[2]
    spt = s.repeat_interleave(page, dim=2)[:, :, :S]
    mpt = m.repeat_interleave(page, dim=2)[:, :, :S]
    kd = (c.to(torch.float32) * spt.float() + mpt.float()).to(torch.bfloat16).float()
    P = (S + page - 1) // page
    pad = P * page - S
    kmin = torch.nn.functional.pad(kd, (0, 0, 0, pad), value=float("inf")).view(1, 2, P, page, -1).min(3).values
    kmax = torch.nn.functional.pad(kd, (0, 0, 0, pad), value=float("-inf")).view(1, 2, P, page, -1).max(3).values
    assert np.array_equal(lo, kmin.numpy()) and np.array_equal(hi, kmax.numpy())


def test_page_summary_reference_known_answers():
    """test_eager_page_summary.py: page p's min / max are its first / last
    key for increasing keys, and page_size 1 returns the keys themselves
    (through the INT8 codes here, so the keys are the dequantised ones)."""
    codes = np.arange(48, dtype=np.uint8).reshape(1, 1, 12, 4)
    scale = np.full((1, 1, 3, 4), 0.5, np.float32)
    mn = np.zeros((1, 1, 3, 4), np.float32)
    lo, hi = O.page_summary_int8(codes, scale, mn, 4)
    assert np.array_equal(lo[0, 0, 0], codes[0, 0, 0] * 0.5) and np.array_equal(hi[0, 0, 0], codes[0, 0, 3] * 0.5)
    lo1, hi1 = O.page_summary_int8(codes, np.full((1, 1, 12, 4), 0.5, np.float32), np.zeros((1, 1, 12, 4), np.float32), 1)
    assert np.array_equal(lo1[0, 0], codes[0, 0] * 0.5) and np.array_equal(hi1[0, 0], codes[0, 0] * 0.5)


def test_fixed_order_scores_are_the_quest_bound():
    """page_scores_quest_fixed equals the fp64 Quest bound (criticality.py:
    7-31) within fp32 summation error, bounds every key's q.k in its page,
    and equals torch's fp32 maximum(...).sum(-1) within the same error."""
    codes, scale, mn = _int8_cache(2, H=2, S=256, D=128)
    lo, hi = O.page_summary_int8(codes, scale, mn, 64)
    rng = np.random.default_rng(3)
    q = O.round_bf16(rng.standard_normal((1, 4, 128)).astype(np.float32))
    got = O.page_scores_quest_fixed(q, lo, hi)
    exact = O.page_scores_quest(q, lo, hi)
    bound = 140 * 2.0 ** -24 * np.einsum("bhd,bhpd->bhp", np.abs(q).astype(np.float64),
                                         np.maximum(np.abs(np.repeat(lo, 2, 1)), np.abs(np.repeat(hi, 2, 1))))
    assert np.all(np.abs(got - exact) <= bound)
    kd = O.round_bf16(O.dequant_k_int8(codes, scale, mn, 64)).astype(np.float64)
    for h in range(4):
        qk = kd[0, h // 2] @ q[0, h].astype(np.float64)
        assert np.all(exact[0, h] >= qk.reshape(4, 64).max(1) - 1e-9)
    t = torch.maximum(torch.from_numpy(q)[:, :, None] * torch.from_numpy(np.repeat(hi, 2, 1)),
                      torch.from_numpy(q)[:, :, None] * torch.from_numpy(np.repeat(lo, 2, 1))).sum(-1).numpy()
    assert np.all(np.abs(got - t) <= 2 * bound)


def test_fixed_order_is_the_stated_butterfly():
    """A sum whose fp32 result depends on the order: 2^24 in channel 0, 1 in
    channels 1, 4 and 68.  Lane 0 (channels 0-3) rounds 2^24 + 1 back to 2^24;
    lane 1 (channels 4-7) gets lane 17's 1 at the first butterfly step (o = 16)
    and holds 2, which reaches lane 0 at the last step (o = 1): 2^24 + 2.  Any
    left-to-right order over the channels would lose all three 1s."""
    D = 128
    q = np.ones((1, 1, D), np.float32)
    hi = np.zeros((1, 1, 1, D), np.float32)
    hi[0, 0, 0, [0, 1, 4, 68]] = [2.0 ** 24, 1.0, 1.0, 1.0]
    s = O.page_scores_quest_fixed(q, np.zeros_like(hi), hi)
    assert s[0, 0, 0] == np.float32(2.0 ** 24 + 2)


def test_select_pages_loop_form_known_answers():
    """selection.py:9-62 (the per-head loop): the reference's known answers
    (test_eager_selection.py:6-44) and its double-precision k: retention 0.07
    over 100 pages keeps ceil(0.07 * 100) = 8 pages (fp32(0.07) * 100 in
    double), where the vectorized form's fp32 product keeps 7
    (test_selection_flips.py:170-180)."""
    sc = np.array([[[[0.1, 0.9, 0.2, 0.8, 0.3, 0.7]]]], np.float32)
    assert O.select_pages(sc, 0.5, 0, 0)[0, 0, 0].tolist() == [False, True, False, True, False, True]
    z = np.zeros((1, 1, 1, 8), np.float32)
    assert O.select_pages(z, 0.0, 1, 2)[0, 0, 0].tolist() == [True] + [False] * 5 + [True, True]
    assert O.select_pages(np.random.default_rng(0).random((1, 2, 1, 8)).astype(np.float32), 1.0, 0, 0).all()
    four = np.array([[[[0.1, 0.4, 0.2, 0.3]]]], np.float32)
    m = O.select_pages(four, 0.1, 0, 0)
    assert m.sum() == 1 and m[0, 0, 0, 1]
    two = np.stack([np.array([[0.9, 0.0, 0.0, 0.1]]), np.array([[0.0, 0.0, 0.9, 0.1]])], 0)[None].astype(np.float32)
    m = O.select_pages(two, 0.25, 0, 0)
    assert m[0, 0, 0, 0] and not m[0, 0, 0, 2] and m[0, 1, 0, 2] and not m[0, 1, 0, 0]
    hundred = np.arange(100, dtype=np.float32)[None, None, None]
    assert math.ceil(float(np.float32(0.07)) * 100) == 8
    assert O.select_pages(hundred, 0.07, 0, 0).sum() == 8
    assert O.select_pages_vectorized(hundred, 0.07, 0, 0).sum() == 7
    r = np.array([0.07, 0.0], np.float32)
    m = O.select_pages(np.repeat(hundred, 2, 1), r, 1, 0)
    assert m[0, 0].sum() == 9 and m[0, 1].sum() == 1      # + sink page 0


def test_compute_page_summary_reference_known_answers():
    """test_eager_page_summary.py:6-37: increasing keys give each page's first /
    last key; a partial tail page summarises its valid keys; page size 1 gives
    the keys themselves."""
    K = np.arange(1 * 2 * 12 * 8, dtype=np.float32).reshape(1, 2, 12, 8)
    lo, hi = O.compute_page_summary(K, 4)
    assert lo.shape == (1, 2, 3, 8) and np.array_equal(lo[0, 0, 0], K[0, 0, 0]) and np.array_equal(hi[0, 0, 0], K[0, 0, 3])
    K2 = np.random.default_rng(0).standard_normal((1, 1, 10, 4)).astype(np.float32)
    lo2, hi2 = O.compute_page_summary(K2, 4)
    assert lo2.shape == (1, 1, 3, 4) and np.array_equal(hi2[0, 0, 2], K2[0, 0, 8:10].max(0))
    K3 = np.random.default_rng(1).standard_normal((1, 1, 5, 3)).astype(np.float32)
    lo3, hi3 = O.compute_page_summary(K3, 1)
    assert np.array_equal(lo3[:, :, :, :], K3) and np.array_equal(hi3, K3)


def test_page_scores_int8_bound_follows_the_reference_expression():
    """page_scores_int8 (criticality.py:59-74) evaluated by torch on the CPU:
    the fixed-order sum differs only by fp32 summation order, and the bounds
    are the reference's exactly (fp32(K_mn) + 255 * fp32(K_scale))."""
    codes, scale, mn = _int8_cache(5, H=2, S=256, D=128)
    rng = np.random.default_rng(6)
    q = O.round_bf16(rng.standard_normal((1, 4, 128)).astype(np.float32))
    got = O.page_scores_int8_bound_fixed(q, scale, mn)
    kmn = torch.from_numpy(mn).to(torch.bfloat16).float().repeat_interleave(2, dim=1)
    kmx = (torch.from_numpy(mn).to(torch.bfloat16).float() + 255.0 * torch.from_numpy(scale).to(torch.bfloat16).float()
           ).repeat_interleave(2, dim=1)
    qt = torch.from_numpy(q).unsqueeze(2)
    ref = torch.maximum(qt * kmx, qt * kmn).sum(-1).numpy()
    mag = np.einsum("bhd,bhpd->bhp", np.abs(q).astype(np.float64),
                    np.maximum(np.abs(kmn.numpy()), np.abs(kmx.numpy())).astype(np.float64))
    assert np.all(np.abs(got - ref) <= 2 * 140 * 2.0 ** -24 * mag)
    # the bounds themselves are bit-equal to torch's
    hi = (np.asarray(mn, np.float32) + (np.float32(255.0) * np.asarray(scale, np.float32))).astype(np.float32)
    assert np.array_equal(np.repeat(hi, 2, axis=1), kmx.numpy())
