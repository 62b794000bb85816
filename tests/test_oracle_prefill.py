"""Pins the oracle's prefill restatement (llama_persistent_patch.py:196-201)
against torch's own SDPA on the CPU (the routine the reference calls), closed
forms, and the reference's dequantisers evaluated by torch."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fq_oracle as O


@pytest.mark.parametrize("Hq,Hkv,Sq,Skv", [(6, 2, 5, 5), (4, 4, 3, 9), (8, 2, 17, 40), (3, 1, 1, 7)])
def test_causal_prefill_matches_torch_sdpa(Hq, Hkv, Sq, Skv):
    rng = np.random.default_rng(Sq * 100 + Skv)
    q = rng.standard_normal((2, Hq, Sq, 16))
    k = rng.standard_normal((2, Hkv, Skv, 16))
    v = rng.standard_normal((2, Hkv, Skv, 16))
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    # torch's is_causal with S_q != S_kv is the upper-left aligned mask
    ref = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True, enable_gqa=True).numpy()
    assert np.abs(O.causal_prefill_attention(q, k, v) - ref).max() < 1e-12
    # lower-right alignment = an explicit tril(diagonal = S_kv - S_q) mask
    mask = torch.ones(Sq, Skv, dtype=torch.bool).tril(diagonal=Skv - Sq)
    ref_br = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, enable_gqa=True).numpy()
    assert np.abs(O.causal_prefill_attention(q, k, v, causal_offset=Skv - Sq) - ref_br).max() < 1e-12


def test_causal_prefill_closed_forms():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((1, 1, 6, 8))
    q = rng.standard_normal((1, 2, 6, 8))
    # equal keys: softmax is uniform over the allowed prefix -> running mean of V
    k = np.zeros((1, 1, 6, 8))
    out = O.causal_prefill_attention(q, k, v)
    running_mean = np.cumsum(v[0, 0], axis=0) / np.arange(1, 7)[:, None]
    assert np.allclose(out[0, 0], running_mean) and np.allclose(out[0, 1], running_mean)
    # query 0 sees only key 0
    assert np.allclose(O.causal_prefill_attention(q, rng.standard_normal((1, 1, 6, 8)), v)[0, :, 0], v[0, 0, 0])


@pytest.mark.parametrize("bits,meta,group", [(4, "bf16", None), (4, "f16", 32), (8, "bf16", None), (8, "f16", None)])
def test_dequant_bf16_matches_reference_expression(bits, meta, group):
    rng = np.random.default_rng(bits)
    K = O.round_bf16(rng.standard_normal((1, 2, 150, 64)).astype(np.float32) * 3)
    V = O.round_bf16(rng.standard_normal((1, 2, 150, 64)).astype(np.float32))
    if bits == 4:
        kc, ks, km = O.quantize_k_int4(K, 32, "bf16", meta)
        vc, vs, vm = O.quantize_v_int4(V, group, meta)
        kcodes, vcodes = O.unpack_int4(kc), O.unpack_int4(vc)
    else:
        kc, ks, km = O.quantize_k_int8(K, 32, "bf16", meta)
        vc, vs, vm = O.quantize_v_int8(V, meta)
        kcodes, vcodes = kc, vc
    kd = O.dequant_cache_bf16(kc, "K", ks, km, 32, bits)
    vd = O.dequant_cache_bf16(vc, "V", vs, vm, 32, bits)
    # the reference's expressions (kv_quant.py:184-186, 214-215), evaluated by torch
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    S = K.shape[2]
    ref_k = (t(kcodes).float() * t(ks).repeat_interleave(32, 2)[:, :, :S].float()
             + t(km).repeat_interleave(32, 2)[:, :, :S].float()).to(torch.bfloat16).float().numpy()
    G = vs.shape[-1]
    ref_v = (t(vcodes).float().view(1, 2, S, G, 64 // G) * t(vs).float()[..., None]
             + t(vm).float()[..., None]).view(1, 2, S, 64).to(torch.bfloat16).float().numpy()
    assert np.array_equal(kd, ref_k) and np.array_equal(vd, ref_v)
    # round trip: within half a quantisation step (+ bf16 rounding)
    step_k = np.repeat(ks, 32, axis=-2)[..., :S, :]
    assert np.all(np.abs(kd - K) <= step_k * 0.5 + np.abs(K) * 2 ** -8 + 1e-6)


def test_dequant_turbo_bf16_closed_form():
    # codebook * scale then the normalised Hadamard transform (Sylvester matrix, fp64) -> within one bf16 ulp
    rng = np.random.default_rng(9)
    X = O.round_bf16(rng.standard_normal((1, 2, 40, 128)).astype(np.float32))
    msb, lsb, st = O.quantize_turbo(X)
    got = O.dequant_turbo_bf16(msb, lsb, st)
    rot = O.dequant_turbo_rot(msb, lsb, st, 128).astype(np.float64)
    ref = rot @ O.hadamard_matrix(128).T          # hadamard_matrix is already normalised
    # one bf16 ulp, plus the fp32 butterflies' cancellation on near-zero outputs
    ulp = np.abs(O.round_bf16(ref.astype(np.float32))) * 2 ** -7 + 1e-5
    assert np.all(np.abs(got - ref) <= ulp)
    # and the transform undoes the quantiser's rotation: close to the input
    assert np.abs(got - X).mean() < 0.25
