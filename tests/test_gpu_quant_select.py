"""Quantisers, scoring, selection, WHT, tail and merge: HIP vs the CPU oracle (MI355X)."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import TORCH_HALF, Int4Case, make_kv, max_err, to_dev, to_dev_half

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype,meta,S,page", [("bf16", "bf16", 64 * 5, 64), ("f16", "f16", 64 * 4 + 9, 64),
                                               ("f16", "bf16", 200, 32), ("bf16", "bf16", 70, 8)])
def test_quantize_k_bit_exact(dtype, meta, S, page):
    from flashquest_amd.kernel import quantize_k_int4
    rng = np.random.default_rng(S)
    K, _ = make_kv(rng, 2, 3, S, 128, dtype)
    K[0, 0, :, 5] = K[0, 0, 0, 5]                    # a constant channel (epsilon scale)
    kp, ks, km = O.quantize_k_int4(K, page, dtype, meta)
    p, s, m = quantize_k_int4(to_dev_half(K, dtype), page, meta_dtype=TORCH_HALF[meta])
    assert np.array_equal(p.cpu().numpy(), kp)
    assert np.array_equal(_bits(s), O.to_bits(ks, meta))
    assert np.array_equal(_bits(m), O.to_bits(km, meta))


@pytest.mark.parametrize("dtype,meta,group", [("bf16", "bf16", None), ("f16", "f16", 32), ("bf16", "f16", 32)])
def test_quantize_v_bit_exact(dtype, meta, group):
    from flashquest_amd.kernel import quantize_v_int4
    rng = np.random.default_rng(7)
    _, V = make_kv(rng, 2, 3, 333, 128, dtype)
    vp, vs, vm = O.quantize_v_int4(V, group, meta)
    p, s, m = quantize_v_int4(to_dev_half(V, dtype), v_group=group, meta_dtype=TORCH_HALF[meta])
    assert np.array_equal(p.cpu().numpy(), vp)
    assert np.array_equal(_bits(s), O.to_bits(vs, meta))
    assert np.array_equal(_bits(m), O.to_bits(vm, meta))


def test_quantize_into_strided_cache_views():
    from flashquest_amd.kernel import quantize_k_int4
    rng = np.random.default_rng(1)
    K, _ = make_kv(rng, 1, 2, 128, 64)
    store_p = torch.zeros(3, 1, 2, 512, 32, dtype=torch.uint8, device="cuda")
    store_s = torch.zeros(3, 1, 2, 8, 64, dtype=torch.bfloat16, device="cuda")
    store_m = torch.zeros_like(store_s)
    out = (store_p[1, :, :, 64:192], store_s[1, :, :, 1:3], store_m[1, :, :, 1:3])
    quantize_k_int4(to_dev_half(K, "bf16"), 64, out=out)
    kp, ks, km = O.quantize_k_int4(K, 64)
    assert np.array_equal(store_p[1, :, :, 64:192].cpu().numpy(), kp)
    assert np.array_equal(_bits(store_s[1, :, :, 1:3]), O.to_bits(ks, "bf16"))
    assert int(store_p[0].sum()) == 0 and int(store_p[1, :, :, :64].sum()) == 0


@pytest.mark.parametrize("Hq,Hkv,D,meta,Sq", [(24, 8, 128, "bf16", 1), (4, 2, 64, "f16", 1), (6, 2, 128, "bf16", 2)])
def test_page_scores_bit_exact_and_close_to_reference_math(Hq, Hkv, D, meta, Sq):
    from flashquest_amd.eager import page_scores_int4_fast
    case = Int4Case(seed=D + Hq, B=2, Hq=Hq, Hkv=Hkv, S=64 * 37, D=D, meta=meta)
    Q = O.round_bf16(case.rng.standard_normal((2, Hq, Sq, D)).astype(np.float32))
    t = case.device()
    got = page_scores_int4_fast(to_dev_half(Q, "bf16"), t["K_scale"], t["K_mn"]).cpu().numpy()
    assert got.shape == (2, Hq, Sq, case.P)
    for s in range(Sq):
        fixed = O.page_scores_fixed(Q[:, :, s], case.ks, case.km)
        assert np.array_equal(got[:, :, s], fixed)
        exact = O.page_scores_int4_exact(Q[:, :, s], case.ks, case.km)
        assert np.allclose(got[:, :, s], exact, rtol=1e-3, atol=1e-3)    # test_eager_criticality.py:42-70


def test_select_kats_and_brute_force():
    from flashquest_amd.eager import select_pages_vectorized
    s = torch.tensor([[[[0.1, 0.9, 0.2, 0.8, 0.3, 0.7]]]], device="cuda")
    assert select_pages_vectorized(s, 0.5, 0, 0)[0, 0, 0].tolist() == [False, True, False, True, False, True]
    s = torch.tensor([[[[0.1, 0.4, 0.2, 0.3]]]], device="cuda")
    m = select_pages_vectorized(s, 0.1, 0, 0)
    assert m.sum().item() == 1 and m[0, 0, 0, 1]
    z = torch.zeros(1, 1, 1, 8, device="cuda")
    assert select_pages_vectorized(z, 0.0, 1, 2)[0, 0, 0].tolist() == [True] + [False] * 5 + [True, True]
    assert select_pages_vectorized(torch.randn(1, 2, 1, 4, device="cuda"), 0.0, 10, 10).all()
    rng = np.random.default_rng(0)
    for P in (4, 64, 200, 512, 3000):
        sc = rng.standard_normal((2, 3, 1, P)).astype(np.float32)
        sc[0, 0, 0, : P // 4] = 0.5        # many exact ties
        for r in (0.0, 0.1, 0.25, 1.0):
            for kmax in (None, 5):
                ref = O.select_pages_vectorized(sc, r, 3, 2, kmax)
                got = select_pages_vectorized(to_dev(sc), r, 3, 2, k_max_static=kmax).cpu().numpy()
                assert np.array_equal(got, ref), (P, r, kmax)


def test_select_per_head_retention_and_validation():
    from flashquest_amd.eager import select_pages_vectorized
    rng = np.random.default_rng(42)
    sc = rng.standard_normal((1, 6, 1, 32)).astype(np.float32)
    r = np.array([0.0, 0.1, 0.25, 0.5, 0.75, 1.0], np.float32)
    ref = O.select_pages_vectorized(sc, r, 2, 1)
    got = select_pages_vectorized(to_dev(sc), torch.from_numpy(r), 2, 1).cpu().numpy()
    assert np.array_equal(got, ref)
    with pytest.raises(ValueError):
        select_pages_vectorized(to_dev(sc), 1.5, 0, 0)
    with pytest.raises(ValueError):
        select_pages_vectorized(to_dev(sc), torch.ones(5), 0, 0)


def test_build_compact_selection_kats():
    from flashquest_amd.eager import build_compact_selection
    mask = torch.zeros(1, 1, 1, 8, dtype=torch.bool, device="cuda")
    mask[0, 0, 0, [1, 3, 5]] = True
    for bm in (4, 8, 16):
        out = build_compact_selection(mask, bm)
        assert out.shape == (1, 1, 1, bm) and out.dtype == torch.int32
        assert out[0, 0, 0, :3].tolist() == [5, 3, 1] and (out[0, 0, 0, 3:] == -1).all()
    rng = np.random.default_rng(3)
    m = rng.random((2, 3, 1, 700)) < 0.3
    for bm in (1, 50, 700, 900):
        assert np.array_equal(build_compact_selection(to_dev(m), bm).cpu().numpy(), O.build_compact_selection(m, bm))
    with pytest.raises(ValueError):
        build_compact_selection(mask, 0)
    with pytest.raises(ValueError):
        build_compact_selection(mask.int(), 4)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_wht_matches_reference_order(dtype):
    from flashquest_amd.kernel import wht_along_head_dim
    rng = np.random.default_rng(5)
    # every supported width; row counts that leave part of a wave (and of a
    # workgroup) idle, and rows spread over several workgroups
    for D in (8, 16, 32, 64, 128):
        for shape in ((3, 5, D), (67, D), (1, D)):
            x = O.rounder(dtype)(rng.standard_normal(shape).astype(np.float32))
            tdt = torch.float32 if dtype == "f32" else torch.bfloat16
            got = wht_along_head_dim(torch.from_numpy(x).to(tdt).cuda()).float().cpu().numpy()
            assert np.array_equal(got, O.wht(x, dtype)), (D, shape)
    s = O.random_signs(1, 128)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    fx = wht_along_head_dim(torch.from_numpy(x).cuda(), signs=torch.from_numpy(s))
    assert np.allclose(fx.cpu().numpy(), O.rotate_signed(x, s), atol=1e-5)
    back = wht_along_head_dim(fx, signs=torch.from_numpy(s), inverse=True)
    assert np.allclose(back.cpu().numpy(), x, atol=1e-5)
    out = torch.empty_like(fx)
    assert wht_along_head_dim(fx, signs=torch.from_numpy(s), inverse=True, out=out) is out
    assert torch.equal(out, back)
    with pytest.raises(ValueError):
        wht_along_head_dim(fx, out=torch.empty(4, 64, device=fx.device))


def test_turbo_quant_bit_exact():
    from flashquest_amd.kernel import quantize_k_turbo, quantize_v_turbo
    rng = np.random.default_rng(4)
    K, V = make_kv(rng, 1, 2, 130, 128, outliers=False)
    m, l, st, sr, mr = quantize_k_turbo(to_dev_half(K, "bf16"), 64)
    om, ol, ost, osr, omr = O.quantize_k_turbo(K, 64)
    assert np.array_equal(m.cpu().numpy(), om) and np.array_equal(l.cpu().numpy(), ol)
    assert np.array_equal(_bits(st), O.to_bits(ost, "bf16"))
    assert np.array_equal(_bits(sr), O.to_bits(osr, "bf16")) and np.array_equal(_bits(mr), O.to_bits(omr, "bf16"))
    vm, vl, vst = quantize_v_turbo(to_dev_half(V, "bf16"))
    om, ol, ost = O.quantize_turbo(V)
    assert np.array_equal(vm.cpu().numpy(), om) and np.array_equal(vl.cpu().numpy(), ol)


@pytest.mark.parametrize("Hq,Hkv,D", [(6, 2, 128), (4, 4, 64)])
def test_turbo_attention_matches_oracle(Hq, Hkv, D):
    from flashquest_amd.kernel import flash_attn_sparse_turbo_fwd
    rng = np.random.default_rng(Hq)
    B, S, page = 2, 64 * 12, 64
    K, V = make_kv(rng, B, Hkv, S, D, outliers=False)
    km, kl, kst = O.quantize_turbo(K)
    vm, vl, vst = O.quantize_turbo(V)
    Q = O.round_bf16(rng.standard_normal((B, Hq, D)).astype(np.float32))
    mask = rng.random((B, Hq, S // page)) < 0.4
    mask[1, 0] = False
    ref_o, ref_l = O.sparse_turbo_attention(Q, km, kl, kst, vm, vl, vst, mask, page)
    o, lse = flash_attn_sparse_turbo_fwd(
        to_dev_half(Q, "bf16")[:, :, None], to_dev(km), to_dev(kl), to_dev_half(kst, "bf16"), to_dev(vm),
        to_dev(vl), to_dev_half(vst, "bf16"), selection_mask=to_dev(mask)[:, :, None])
    assert max_err(o[:, :, 0], ref_o) <= 2e-3 + 2 ** -8 * np.abs(ref_o).max()
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4


def test_tail_attention_and_merge():
    from flashquest_amd.eager import bf16_dense_attn_with_lse, merge_two_attentions
    rng = np.random.default_rng(9)
    B, Hq, Hkv, D = 2, 6, 2, 128
    for T in (1, 17, 63):
        q = O.round_bf16(rng.standard_normal((B, Hq, D)).astype(np.float32))
        k = O.round_bf16(rng.standard_normal((B, Hkv, T, D)).astype(np.float32))
        v = O.round_bf16(rng.standard_normal((B, Hkv, T, D)).astype(np.float32))
        ro, rl = O.dense_attn_with_lse(q, k, v)
        o, lse = bf16_dense_attn_with_lse(to_dev_half(q, "bf16")[:, :, None], to_dev_half(k, "bf16"),
                                          to_dev_half(v, "bf16"))
        assert o.dtype == torch.bfloat16
        assert max_err(o[:, :, 0], ro) <= 2e-3 + 2 ** -8 * np.abs(ro).max()
        assert max_err(lse[:, :, 0], rl) <= 1e-4
    # merge: split a dense attention in two and merge it back
    k = O.round_bf16(rng.standard_normal((B, Hkv, 40, D)).astype(np.float32))
    v = O.round_bf16(rng.standard_normal((B, Hkv, 40, D)).astype(np.float32))
    full, _ = O.dense_attn_with_lse(q, k, v)
    a = bf16_dense_attn_with_lse(to_dev_half(q, "bf16")[:, :, None], to_dev_half(k[:, :, :13], "bf16"),
                                 to_dev_half(v[:, :, :13], "bf16"))
    b = bf16_dense_attn_with_lse(to_dev_half(q, "bf16")[:, :, None], to_dev_half(k[:, :, 13:], "bf16"),
                                 to_dev_half(v[:, :, 13:], "bf16"))
    m = merge_two_attentions(a[0], a[1], b[0], b[1])
    assert m.dtype == torch.bfloat16
    assert max_err(m[:, :, 0], full) <= 4e-3 + 2 ** -7 * np.abs(full).max()
