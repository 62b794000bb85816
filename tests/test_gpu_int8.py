"""INT8 KV family on HIP vs the CPU oracle (MI355X): quantisers bit-exact
(kv_quant.py:43-89), page scores bit-exact in the library's fp32 order
(criticality.py:77-125), flash_attn_sparse_fwd (sparse_fwd.py:160-228) and the
whole decode step vs exact attention, and the persistent INT8 cache
(persistent_int8.py)."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import TORCH_HALF, Int8Case, make_kv, max_err, to_dev, to_dev_half

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _tol(case, ref):
    return 2e-3 + 2 ** -8 * float(np.abs(ref).max())


@pytest.mark.parametrize("dtype,meta,S,page", [("bf16", "bf16", 64 * 5, 64), ("f16", "bf16", 64 * 4 + 9, 64),
                                               ("f16", "f16", 200, 32), ("f32", "bf16", 130, 64)])
def test_quantize_k_bit_exact(dtype, meta, S, page):
    from flashquest_amd.kernel import quantize_k
    rng = np.random.default_rng(S)
    K, _ = make_kv(rng, 2, 3, S, 128, "bf16" if dtype == "f32" else dtype)
    K[0, 0, :, 5] = K[0, 0, 0, 5]                    # a constant channel (epsilon scale)
    ku, ks, km = O.quantize_k_int8(K, page, dtype, meta)
    Kd = torch.from_numpy(K).cuda() if dtype == "f32" else to_dev_half(K, dtype)
    c, s, m = quantize_k(Kd, page, meta_dtype=TORCH_HALF[meta])
    assert np.array_equal(c.cpu().numpy(), ku)
    assert np.array_equal(_bits(s), O.to_bits(ks, meta))
    assert np.array_equal(_bits(m), O.to_bits(km, meta))


@pytest.mark.parametrize("dtype,meta,D", [("bf16", "bf16", 128), ("f16", "f16", 64), ("bf16", "f16", 128)])
def test_quantize_v_bit_exact(dtype, meta, D):
    from flashquest_amd.kernel import quantize_v
    rng = np.random.default_rng(D)
    _, V = make_kv(rng, 2, 3, 333, D, dtype)
    V[1, 2, 7, :] = V[1, 2, 7, 0]                    # a constant token
    vu, vs, vm = O.quantize_v_int8(V, meta)
    c, s, m = quantize_v(to_dev_half(V, dtype), meta_dtype=TORCH_HALF[meta])
    assert np.array_equal(c.cpu().numpy(), vu)
    assert np.array_equal(_bits(s), O.to_bits(vs, meta))
    assert np.array_equal(_bits(m), O.to_bits(vm, meta))


def test_dequantize_matches_reference_formula():
    from flashquest_amd.kernel import dequantize_k, dequantize_v
    case = Int8Case(seed=2, S=64 * 3 + 5, D=64)
    d = case.device()
    k = dequantize_k(d["K_uint8"], d["K_scale"], d["K_mn"], 64)
    v = dequantize_v(d["V_uint8"], d["V_scale"], d["V_mn"])
    assert np.array_equal(k.float().cpu().numpy(), O.round_bf16(O.dequant_k_int8(case.ku, case.ks, case.km, 64)))
    assert np.array_equal(v.float().cpu().numpy(), O.round_bf16(O.dequant_v_int8(case.vu, case.vs, case.vm)))


@pytest.mark.parametrize("Hq,Hkv,D,meta", [(24, 8, 128, "bf16"), (4, 2, 64, "f16")])
def test_page_scores_int8_bit_exact(Hq, Hkv, D, meta):
    from flashquest_amd.eager import page_scores_int8, page_scores_int8_fast
    case = Int8Case(seed=D + Hq, B=2, Hq=Hq, Hkv=Hkv, S=64 * 37, D=D, meta=meta)
    d = case.device()
    sc = page_scores_int8_fast(case.q_dev(), d["K_scale"], d["K_mn"])
    ref = O.page_scores_fixed(case.Q, case.ks, case.km, "per_q_head", 255.0)
    assert np.array_equal(sc[:, :, 0].cpu().numpy(), ref)
    exact = O.page_scores_int8_exact(case.Q, case.ks, case.km)
    assert np.allclose(ref, exact, rtol=1e-5, atol=1e-3)
    # page_scores_int8 (criticality.py:34-74): the reference's own bounds and terms, fixed order
    sb = page_scores_int8(case.q_dev(), d["K_scale"], d["K_mn"])
    assert np.array_equal(sb[:, :, 0].cpu().numpy(), O.page_scores_int8_bound_fixed(case.Q, case.ks, case.km))
    assert np.allclose(sb[:, :, 0].cpu().numpy(), exact, rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("Hq,Hkv,D,S,dtype,meta", [(24, 8, 128, 64 * 20 + 17, "bf16", "bf16"),
                                                   (8, 8, 64, 64 * 9, "f16", "f16"),
                                                   (16, 2, 128, 64 * 12, "bf16", "bf16"),
                                                   (16, 4, 128, 64 * 7 + 1, "f16", "f16"),
                                                   (8, 8, 128, 64 * 5, "bf16", "f16")])
def test_flash_attn_sparse_fwd_matches_oracle(Hq, Hkv, D, S, dtype, meta):
    from flashquest_amd.kernel import flash_attn_sparse_fwd
    case = Int8Case(seed=S + Hq, B=2, Hq=Hq, Hkv=Hkv, S=S, D=D, dtype=dtype, meta=meta)
    rng = np.random.default_rng(S)
    mask = rng.random((2, Hq, case.P)) < 0.3
    mask[0, 0] = False                                   # an empty selection: O = 0, lse = -inf
    mask[1, -1, -1] = True                               # the partial last page
    o, lse = flash_attn_sparse_fwd(case.q_dev(), **case.device(),
                                   selection_mask=torch.from_numpy(mask[:, :, None, :]).cuda())
    ro, rl = O.sparse_int8_attention(case.Q, case.ku, case.ks, case.km, case.vu, case.vs, case.vm, mask, 64)
    assert max_err(o[:, :, 0], ro) <= _tol(case, ro)
    assert max_err(lse[:, :, 0], rl) <= 1e-4
    assert torch.all(o[0, 0] == 0)


def test_flash_attn_sparse_fwd_errors():
    from flashquest_amd.kernel import flash_attn_sparse_fwd
    case = Int8Case(seed=1, S=64 * 3, D=128)
    d = case.device()
    m = torch.ones(1, 6, 1, 3, dtype=torch.bool, device="cuda")
    q = case.q_dev()
    with pytest.raises(NotImplementedError):
        flash_attn_sparse_fwd(q.expand(1, 6, 2, 128), **d, selection_mask=m)
    with pytest.raises(AssertionError):
        flash_attn_sparse_fwd(q, **d, selection_mask=m[..., :2])


@pytest.mark.parametrize("layers,mode,meta", [(1, "per_q_head", "bf16"), (12, "per_kv_head_sum", "bf16"),
                                              (12, "per_q_head", "f16"), (24, "per_kv_head_sum", "f16")])
def test_quest_decode_int8_matches_oracle_decode_step(layers, mode, meta):
    # 1 and 12 layers: groups split over several workgroups, each selecting;
    # 24 layers x 8 KV heads: one workgroup per group
    from flashquest_amd.eager import quest_decode_int8
    Hq, Hkv, P = 24, 8, 20
    cases = [Int8Case(seed=60 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * (P - 1) + 30, D=128, meta=meta)
             for i in range(layers)]
    dev = [c.device() for c in cases]
    if layers > 1:
        stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
        q = torch.stack([c.q_dev() for c in cases])
    else:
        stacked, q = dev[0], cases[0].q_dev()
    o, lse, mask = quest_decode_int8(q, **stacked, retention=0.3, num_sinks=2, window_pages=1,
                                     select_mode=mode, return_selection=True)
    for i, c in enumerate(cases):
        ref = O.decode_step(c.Q, c.ku, c.ks, c.km, c.vu, c.vs, c.vm, retention=0.3, num_sinks=2,
                            window_pages=1, mode=mode, bits=8)
        oi = o[i] if layers > 1 else o
        li = lse[i] if layers > 1 else lse
        mi = mask[i] if layers > 1 else mask
        assert np.array_equal(mi.cpu().numpy(), ref["mask"]), i
        assert max_err(oi[:, :, 0], ref["O"]) <= _tol(c, ref["O"]), i
        assert max_err(li[:, :, 0], ref["lse"]) <= 1e-4, i


def test_persistent_int8_cache_appends_match_one_quantisation():
    # prefill 150 tokens, then 1 + 40 + 3 decode appends: the completed pages equal
    # the quantisation of the whole stream, the tail holds the rest and zeros after it
    from flashquest_amd.cache import PersistentInt8KVCache
    rng = np.random.default_rng(4)
    K, V = make_kv(rng, 1, 2, 194, 64, "bf16")
    cache = PersistentInt8KVCache(batch_size=1, num_layers=2, num_kv_heads=2, head_dim=64, max_seq_len=256)
    Kd, Vd = to_dev_half(K, "bf16"), to_dev_half(V, "bf16")
    t = 0
    for n in (150, 1, 40, 3):
        cache.update_quantized(Kd[:, :, t:t + n], Vd[:, :, t:t + n], layer_idx=1)
        t += n
    views = cache.get_views(1)
    assert (views["seq_len"], views["completed_len"], views["partial_len"]) == (194, 192, 2)
    ku, ks, km = O.quantize_k_int8(K[:, :, :192], 64)
    vu, vs, vm = O.quantize_v_int8(V[:, :, :192])
    assert np.array_equal(views["K_uint8"].cpu().numpy(), ku)
    assert np.array_equal(views["V_uint8"].cpu().numpy(), vu)
    assert np.array_equal(_bits(views["K_scale"]), O.to_bits(ks, "bf16"))
    assert np.array_equal(_bits(views["V_mn"]), O.to_bits(vm, "bf16"))
    assert torch.equal(views["K_partial"], Kd[:, :, 192:194])
    assert int(cache.K_partial[1, :, :, 2:].abs().sum()) == 0
    assert cache.get_seq_length(0) == 0 and cache.kv_bits == 8
    with pytest.raises(IndexError):
        cache.get_views(2)
    with pytest.raises(RuntimeError):
        cache.update_quantized(Kd[:, :, :100], Vd[:, :, :100], layer_idx=1)
    with pytest.raises(RuntimeError):
        cache.update(Kd, Vd, 0)


@pytest.mark.parametrize("partial", [0, 29])
def test_decode_layer_over_int8_cache_views(partial):
    # the decode branch of the reference's attention patch with kv_bits = 8
    # (llama_persistent_patch.py:143-160, 202-245): INT8 sparse attention on the
    # completed pages, dense bf16 attention on the tail, LSE merge
    from flashquest_amd.cache import PersistentInt8KVCache
    from flashquest_amd.eager.decode import sparse_decode_layer
    rng = np.random.default_rng(31 + partial)
    B, Hq, H, D, P = 1, 6, 2, 128, 12
    S = 64 * P + partial
    K, V = make_kv(rng, B, H, S, D, "bf16")
    Q = O.round_bf16(rng.standard_normal((B, Hq, D)).astype(np.float32))
    cache = PersistentInt8KVCache(batch_size=B, num_layers=1, num_kv_heads=H, head_dim=D, max_seq_len=S)
    cache.update_quantized(to_dev_half(K, "bf16"), to_dev_half(V, "bf16"), 0)
    views = cache.get_views(0)
    out = sparse_decode_layer(to_dev_half(Q, "bf16")[:, :, None, :], views, retention=0.3, num_sinks=1,
                              window_pages=1, page_size=64)
    comp = 64 * P
    ku, ks, km = O.quantize_k_int8(K[:, :, :comp], 64)
    vu, vs, vm = O.quantize_v_int8(V[:, :, :comp])
    ref = O.decode_step(Q, ku, ks, km, vu, vs, vm, retention=0.3, num_sinks=1, window_pages=1, bits=8)
    O_ref = ref["O"]
    if partial:
        ot, lt = O.dense_attn_with_lse(Q, K[:, :, comp:], V[:, :, comp:])
        O_ref = O.merge_two_attentions(O.round_bf16(O_ref), ref["lse"], O.round_bf16(ot), lt)
    assert max_err(out[:, :, 0], O_ref) <= 2e-2
