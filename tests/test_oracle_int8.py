"""The INT8 KV family's oracle (kernel/kv_quant.py:18-100, criticality.py:34-125,
sparse_fwd.py:23-157), pinned against known-answer pages, brute force and the
reference tests' properties (test_kv_quant.py ES3/ES9/ES10,
test_page_scores_int8.py EQ18)."""
import math

import numpy as np
import pytest

from oracle import fq_oracle as O


def test_k_known_answer_page_codes_and_scale():
    # one channel spans [0, 255 * 2^-7] in steps of 2^-7: exact bf16 values,
    # scale bf16(bf16(1.9921875) * fp32(1/255)) = 2^-7, codes = the step counts
    t = np.arange(64)
    steps = np.minimum(4 * t, 255)
    steps[-1] = 255                                      # the page maximum is level 255
    k = (steps * 2.0 ** -7).astype(np.float32)
    K = np.zeros((1, 1, 64, 2), np.float32)
    K[0, 0, :, 0] = k
    K[0, 0, :, 1] = 0.5                                  # constant channel: scale clamps to 1e-6 (bf16)
    codes, scale, mn = O.quantize_k_int8(K, 64)
    assert scale[0, 0, 0, 0] == 2.0 ** -7 and mn[0, 0, 0, 0] == 0.0
    assert np.array_equal(codes[0, 0, :, 0], steps)
    assert np.all(codes[0, 0, :, 1] == 0)
    assert scale[0, 0, 0, 1] == O.round_bf16(np.float32(1e-6))


def test_v_known_answer_token_codes():
    # per token: values k * 2^-7 for k in 0..255 over 256 channels -> codes k
    V = (np.arange(256, dtype=np.float32) * 2.0 ** -7)[None, None, None, :]
    codes, scale, mn = O.quantize_v_int8(V)
    assert np.array_equal(codes[0, 0, 0], np.arange(256))
    assert mn[0, 0, 0, 0] == 0.0
    # fp32 scale (1.9921875 * fp32(1/255)) rounded to bf16 afterwards
    assert scale[0, 0, 0, 0] == O.round_bf16(np.float32(1.9921875) * (np.float32(1) / np.float32(255)))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_codes_are_nearest_in_range(dtype):
    # brute force: each K code is the nearest level of the dtype-rounded scale / min
    rng = np.random.default_rng(3)
    K = O.rounder(dtype)(rng.standard_normal((1, 2, 100, 16)).astype(np.float32) * 3)
    codes, _, _ = O.quantize_k_int8(K, 64, dtype, meta="f16" if dtype == "f16" else "bf16")
    sc, mn = O.scale_mn_per_page_channel_int4(K, 64, dtype, inv=O.INV255)
    tok_s = np.repeat(sc, 64, axis=-2)[..., :100, :].astype(np.float64)
    tok_m = np.repeat(mn, 64, axis=-2)[..., :100, :].astype(np.float64)
    x = (K.astype(np.float64) - tok_m) / tok_s
    assert codes.min() >= 0 and codes.max() <= 255
    assert np.all(np.abs(codes - np.clip(x, 0, 255)) <= 0.5 + 1e-5)


def test_shapes_round_trip_partial_page_and_zero_range():
    # test_kv_quant.py: shapes, ES10 round trip within max scale, ES3 partial
    # last page, ES9 constant channel
    rng = np.random.default_rng(0)
    K = O.round_bf16(rng.standard_normal((1, 2, 128, 64)).astype(np.float32))
    codes, scale, mn = O.quantize_k_int8(K, 64)
    assert codes.shape == (1, 2, 128, 64) and codes.dtype == np.uint8 and scale.shape == (1, 2, 2, 64)
    rec = O.round_bf16(O.dequant_k_int8(codes, scale, mn, 64))
    assert np.abs(rec - K).max() <= scale.max() * 1.01
    V = O.round_bf16(rng.standard_normal((1, 2, 128, 64)).astype(np.float32))
    vc, vs, vm = O.quantize_v_int8(V)
    assert vs.shape == (1, 2, 128, 1)
    assert np.abs(O.round_bf16(O.dequant_v_int8(vc, vs, vm)) - V).max() <= vs.max() * 1.01
    Kp = O.round_bf16(rng.standard_normal((1, 1, 100, 64)).astype(np.float32))
    _, sp, _ = O.quantize_k_int8(Kp, 64)
    assert sp.shape == (1, 1, 2, 64)
    Kz = O.round_bf16(rng.standard_normal((1, 1, 64, 64)).astype(np.float32))
    Kz[..., 5] = O.round_bf16(np.float32(0.7))
    c, s, m = O.quantize_k_int8(Kz, 64)
    assert np.all(np.isfinite(s)) and np.abs(O.dequant_k_int8(c, s, m, 64)[..., 5] - Kz[..., 5]).max() <= 1e-2


def test_int8_scores_equal_the_quest_bound_of_the_page_range():
    # EQ18: score = sum_d max(q mn, q (mn + 255 scale)); the fixed-order fp32 scores
    # agree with it to fp32 rounding
    rng = np.random.default_rng(5)
    K = O.round_bf16(rng.standard_normal((1, 2, 256, 64)).astype(np.float32))
    _, ks, km = O.quantize_k_int8(K, 64)
    Q = O.round_bf16(rng.standard_normal((1, 6, 64)).astype(np.float32))
    quest = O.page_scores_quest(Q, km, km.astype(np.float64) + 255.0 * ks.astype(np.float64))
    exact = O.page_scores_int8_exact(Q, ks, km)
    assert np.allclose(exact, quest, rtol=1e-12, atol=1e-9)
    fixed = O.page_scores_fixed(Q, ks, km, "per_q_head", 255.0)
    assert np.allclose(fixed, exact, rtol=1e-5, atol=1e-4)


def test_sparse_int8_attention_matches_brute_force():
    rng = np.random.default_rng(9)
    K = O.round_bf16(rng.standard_normal((1, 2, 150, 16)).astype(np.float32))
    V = O.round_bf16(rng.standard_normal((1, 2, 150, 16)).astype(np.float32))
    ku, ks, km = O.quantize_k_int8(K, 64)
    vu, vs, vm = O.quantize_v_int8(V)
    Q = rng.standard_normal((1, 4, 16)).astype(np.float32)
    mask = np.zeros((1, 4, 3), bool)
    mask[0, 0, [0, 2]] = True
    mask[0, 1, 1] = True
    mask[0, 3] = True                                    # head 2: nothing selected
    O_, lse = O.sparse_int8_attention(Q, ku, ks, km, vu, vs, vm, mask, 64)
    for h in range(4):
        kv = h // 2
        toks = [t for t in range(150) if mask[0, h, t // 64]]
        if not toks:
            assert np.all(O_[0, h] == 0) and lse[0, h] == -np.inf
            continue
        keys = np.array([[float(ku[0, kv, t, d]) * ks[0, kv, t // 64, d] + km[0, kv, t // 64, d]
                          for d in range(16)] for t in toks])
        vals = np.array([[float(vu[0, kv, t, d]) * vs[0, kv, t, 0] + vm[0, kv, t, 0] for d in range(16)]
                         for t in toks])
        logits = keys @ Q[0, h].astype(np.float64) / math.sqrt(16)
        m = logits.max()
        p = np.exp(logits - m)
        assert np.allclose(O_[0, h], p @ vals / p.sum(), rtol=1e-9, atol=1e-12)
        assert abs(lse[0, h] - (m + math.log(p.sum()))) < 1e-9
