"""Pins the oracle's attention, merge, WHT and turbo pieces (CPU only)."""
import math

import numpy as np
import pytest

from oracle import fq_oracle as O


def test_exact_attention_matches_independent_loop():
    # tests/test_profile_contribution.py:42-54 (GQA, page mask, per-head loop)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 4, 8))
    k = rng.standard_normal((1, 2, 7, 8))
    v = rng.standard_normal((1, 2, 7, 8))
    sel = np.array([[[True, False, True], [False, True, False], [True, True, True], [False, False, False]]])
    tm = O.page_mask_to_token_mask(sel, 7, 3)
    out, lse = O.exact_attention(q, k, v, tm)
    for h in range(4):
        valid = tm[0, h]
        if not valid.any():
            assert np.all(out[0, h] == 0) and np.isneginf(lse[0, h])
            continue
        logits = q[0, h] @ k[0, h // 2, valid].T / math.sqrt(8)
        w = np.exp(logits - logits.max())
        w /= w.sum()
        assert np.allclose(out[0, h], w @ v[0, h // 2, valid], atol=1e-12)
        assert np.isclose(lse[0, h], np.log(np.exp(logits).sum()))


def test_empty_mask_zero_and_neg_inf():
    # tests/test_profile_contribution.py:57-61
    out, lse = O.exact_attention(np.ones((1, 2, 4)), np.ones((1, 1, 2, 4)),
                                 np.ones((1, 1, 2, 4)), np.zeros((1, 2, 2), bool))
    assert np.all(out == 0) and np.isneginf(lse).all()


def test_dequant_is_fp32_affine_without_bf16_rounding():
    # tests/test_profile_contribution.py:20-28
    packed = np.array([[[[0xF0, 0xA5], [0x21, 0x43]]]], np.uint8)
    scale = np.full((1, 1, 1, 4), 0.1015625, np.float32)
    mn = np.full((1, 1, 1, 4), 0.19921875, np.float32)
    r = O.dequant_k(packed, scale, mn, 2)
    codes = np.array([[[[0, 15, 5, 10], [1, 2, 3, 4]]]], np.float32)
    assert np.array_equal(r, codes * scale + mn)
    assert not np.array_equal(r, O.round_bf16(r))


def test_all_pages_reduces_to_dense_softmax():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, D, S, ps = 1, 6, 2, 64, 128, 32
    K = O.round_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    V = O.round_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    kp, ks, km = O.quantize_k_int4(K, ps)
    vp, vs, vm = O.quantize_v_int4(V)
    Q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    out, lse = O.sparse_int4_attention(Q, kp, ks, km, vp, vs, vm, np.ones((B, Hq, S // ps), bool), ps)
    kd = O.dequant_k(kp, ks, km, ps).astype(np.float64)
    vd = O.dequant_v(vp, vs, vm).astype(np.float64)
    for h in range(Hq):
        lg = kd[0, h // 3] @ Q[0, h].astype(np.float64) / math.sqrt(D)
        w = np.exp(lg - lg.max())
        assert np.allclose(out[0, h], (w / w.sum()) @ vd[0, h // 3], atol=1e-12)


def test_merge_of_split_equals_unsplit():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 2, 16))
    k = rng.standard_normal((1, 1, 40, 16))
    v = rng.standard_normal((1, 1, 40, 16))
    full, lse_full = O.exact_attention(q, k, v, np.ones((1, 2, 40), bool))
    a, la = O.exact_attention(q, k[:, :, :13], v[:, :, :13], np.ones((1, 2, 13), bool))
    b, lb = O.exact_attention(q, k[:, :, 13:], v[:, :, 13:], np.ones((1, 2, 27), bool))
    assert np.allclose(O.merge_two_attentions(a, la, b, lb), full, atol=1e-12)
    assert np.allclose(np.logaddexp(la, lb), lse_full)


def test_wht_equals_hadamard_matrix_and_self_inverse():
    rng = np.random.default_rng(7)
    for D in (64, 128):
        x = rng.standard_normal((3, D)).astype(np.float32)
        y = O.wht(x)
        assert np.allclose(y, x.astype(np.float64) @ O.hadamard_matrix(D).T, atol=1e-5)
        assert np.abs(O.wht(y) - x).max() < 1e-4
    H = O.hadamard_matrix(8) * math.sqrt(8)
    assert np.array_equal(H @ H.T, 8 * np.eye(8))
    with pytest.raises(ValueError, match="power of 2"):
        O.wht(np.zeros((1, 96), np.float32))


def test_codebook_kats():
    # tests/test_kv_quant_turbo.py:13-30
    cb = O.TURBO_CODEBOOK
    assert np.allclose(np.sort(cb), -np.sort(cb)[::-1])
    small = np.array([-1.0, -0.5, 0.5, 1.0], np.float32)
    x = np.array([-0.9, -0.4, 0.0, 0.6, 1.1], np.float32)
    assert O.quantize_to_codebook(x, small).tolist() == [0, 1, 1, 2, 3]


def test_bit_split_roundtrip_and_layout():
    rng = np.random.default_rng(0)
    idx = rng.integers(0, 8, (1, 4, 16, 64)).astype(np.uint8)
    msb, lsb = O.pack_bit_split(idx)
    assert msb.shape == (1, 4, 16, 8) and lsb.shape == (1, 4, 16, 16)
    assert np.array_equal(O.unpack_bit_split(msb, lsb, 64), idx)
    one = np.zeros((8,), np.uint8)
    one[3] = 7            # msb bit 3 of byte 0; lsb field 3 of byte 0
    m, l = O.pack_bit_split(one)
    assert m.tolist() == [8] and l.tolist() == [0xC0, 0]
    with pytest.raises(ValueError, match="multiple of 8"):
        O.pack_bit_split(np.zeros((12,), np.uint8))


def test_turbo_roundtrip_noise_band():
    # tests/test_kv_quant_turbo.py:95-116
    rng = np.random.default_rng(4)
    K = O.round_bf16(rng.standard_normal((1, 4, 256, 128)).astype(np.float32))
    msb, lsb, st = O.quantize_turbo(K)
    back = O.dequant_turbo_rot(msb, lsb, st, 128).astype(np.float64) @ O.hadamard_matrix(128).T
    err = np.abs(back - K)
    assert err.max() < 1.5 and err.mean() < 0.4


def test_turbo_attention_all_pages_equals_dense_rotated():
    rng = np.random.default_rng(8)
    B, Hq, Hkv, D, S, ps = 1, 2, 1, 64, 64, 16
    K = O.round_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    V = O.round_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    km, kl, kst = O.quantize_turbo(K)
    vm, vl, vst = O.quantize_turbo(V)
    Q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    out, lse = O.sparse_turbo_attention(Q, km, kl, kst, vm, vl, vst, np.ones((B, Hq, S // ps), bool), ps)
    Hm = O.hadamard_matrix(D)
    kd = O.dequant_turbo_rot(km, kl, kst, D).astype(np.float64) @ Hm.T   # back to raw basis
    vd = O.dequant_turbo_rot(vm, vl, vst, D).astype(np.float64) @ Hm.T
    ref, lse_ref = O.exact_attention(Q, kd, vd, np.ones((B, Hq, S), bool))
    assert np.allclose(out, ref, atol=1e-9) and np.allclose(lse, lse_ref)


def test_signed_rotation_preserves_dot_products():
    rng = np.random.default_rng(1)
    s = O.random_signs(3)
    x, y = rng.standard_normal((2, 128))
    assert np.isclose(O.rotate_signed(x, s) @ O.rotate_signed(y, s), x @ y)
    assert np.allclose(O.unrotate_signed(O.rotate_signed(x, s), s), x)
    assert set(np.unique(s)) == {-1.0, 1.0}


def test_selected_pages_path_equals_full_dequant_path():
    rng = np.random.default_rng(12)
    B, Hq, Hkv, D, ps = 2, 6, 2, 128, 64
    S = ps * 10 + 5
    K = O.round_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    V = O.round_bf16(rng.standard_normal((B, Hkv, S, D)).astype(np.float32))
    Q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    kp, ks, km = O.quantize_k_int4(K, ps)
    vp, vs, vm = O.quantize_v_int4(V, 32)
    mask = rng.random((B, Hq, 11)) < 0.4
    mask[1, 2] = False
    a, la = O.sparse_int4_attention(Q, kp, ks, km, vp, vs, vm, mask, ps)
    b, lb = O.sparse_int4_attention_selected(Q, kp, ks, km, vp, vs, vm, mask, ps)
    assert np.allclose(a, b, atol=1e-5) and np.allclose(la[np.isfinite(la)], lb[np.isfinite(lb)], atol=1e-5)
    assert np.array_equal(np.isfinite(la), np.isfinite(lb))


def test_torch_eager_baseline_matches_oracle():
    # oracle/torch_eager.py is bench.py's CPU baseline: same selection and output as the numpy oracle
    import torch

    from oracle import torch_eager as TE
    rng = np.random.default_rng(21)
    Hkv, Hq, D, page, P = 2, 6, 128, 64, 16
    K = O.round_f16(rng.standard_normal((1, Hkv, P * page, D)).astype(np.float32))
    V = O.round_f16(rng.standard_normal((1, Hkv, P * page, D)).astype(np.float32))
    Q = rng.standard_normal((1, Hq, D)).astype(np.float32)
    kp, ks, km = O.quantize_k_int4(K, page, "f16", "f16")
    vp, vs, vm = O.quantize_v_int4(V, 32, "f16")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    for mode in ("per_kv_head_sum", "per_q_head"):
        sc = O.page_scores_fixed(Q, ks, km, mode)
        m = O.select_pages_vectorized(sc[:, :, None, :], 0.25, 4, 2, math.ceil(0.25 * P))[:, :, 0, :]
        if mode == "per_kv_head_sum":
            m = np.repeat(m, Hq // Hkv, axis=1)
        ref, _ = O.sparse_int4_attention(Q, kp, ks, km, vp, vs, vm, m, page)
        out = TE.decode_layer(t(Q[0]), t(kp[0]), t(ks[0]).half(), t(km[0]).half(), t(vp[0]), t(vs[0]).half(),
                              t(vm[0]).half(), retention=0.25, select=mode)
        assert float((out - t(ref[0])).abs().max()) < 1e-5


def test_fp32_rotation_of_the_rotated_decode():
    # rotate_signed_f32 (the kernel's fp32 butterflies) agrees with the exact
    # rotation to fp32 rounding, is exact on a signed basis vector (one
    # Hadamard column / sqrt(128)), and its inverse recovers the input
    rng = np.random.default_rng(9)
    s = O.random_signs(3)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    r = O.rotate_signed_f32(x, s)
    assert r.dtype == np.float32
    assert np.abs(r - O.rotate_signed(x, s)).max() <= 1e-5 * np.abs(x).sum(-1).max()
    e = np.zeros(128, np.float32)
    e[37] = 1.0
    col = O.rotate_signed_f32(e, s)
    assert np.array_equal(np.abs(col), np.full(128, np.float32(1.0) / np.float32(np.sqrt(128)), np.float32))
    assert np.allclose(O.unrotate_signed(r, s), x, atol=1e-5)
