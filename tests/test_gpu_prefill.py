"""Prefill over the packed cache (llama_persistent_patch.py:196-201) on HIP vs
the CPU oracle: causal GQA attention over cat(dequantised cache, bf16 tail),
INT4 and INT8 codes, both causal alignments, and at a larger size vs torch's
SDPA over the reference's own dequantise-then-concatenate tensors."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fq_oracle as O
from tests.cases import make_kv, to_dev, to_dev_half

pytestmark = pytest.mark.gpu

# bf16 Q/K/V, fp32 softmax, P and O rounded to bf16: |O| <= max|V|, so half a
# bf16 ulp of O plus the P rounding stays well inside this bound
ATOL = 1.5e-2


class PrefillCase:
    def __init__(self, seed, B=1, Hq=6, Hkv=2, S=256, T=0, Sq=None, D=128, page=64, bits=4, meta="bf16",
                 vgroup=None, causal_offset=0):
        rng = np.random.default_rng(seed)
        self.S, self.T, self.page, self.bits, self.off = S, T, page, bits, causal_offset
        self.Sq = S + T if Sq is None else Sq
        K, V = make_kv(rng, B, Hkv, S + T, D, "bf16")
        Kc, Vc = K[:, :, :S], V[:, :, :S]
        self.Kt, self.Vt = K[:, :, S:], V[:, :, S:]
        if bits == 4:
            self.kc, self.ks, self.km = O.quantize_k_int4(Kc, page, "bf16", meta)
            self.vc, self.vs, self.vm = O.quantize_v_int4(Vc, vgroup, meta)
        else:
            self.kc, self.ks, self.km = O.quantize_k_int8(Kc, page, "bf16", meta)
            self.vc, self.vs, self.vm = O.quantize_v_int8(Vc, meta)
        self.meta = meta
        self.Q = O.round_bf16(rng.standard_normal((B, Hq, self.Sq, D)).astype(np.float32))

    def run(self):
        from flashquest_amd.kernel import flash_attn_prefill_int4, flash_attn_prefill_int8
        fn = flash_attn_prefill_int4 if self.bits == 4 else flash_attn_prefill_int8
        m = self.meta
        return fn(to_dev_half(self.Q, "bf16"), to_dev(self.kc), to_dev_half(self.ks, m), to_dev_half(self.km, m),
                  to_dev(self.vc), to_dev_half(self.vs, m), to_dev_half(self.vm, m),
                  to_dev_half(self.Kt, "bf16"), to_dev_half(self.Vt, "bf16"), page_size=self.page,
                  causal_offset=self.off)

    def oracle(self):
        return O.prefill_packed(self.Q, self.kc, self.ks, self.km, self.vc, self.vs, self.vm, self.Kt, self.Vt,
                                page_size=self.page, bits=self.bits, causal_offset=self.off)


def _check(case):
    out = case.run()
    torch.cuda.synchronize()
    ref = case.oracle()
    g = out.float().cpu().numpy()
    assert g.shape == ref.shape
    assert np.isfinite(g).all()
    err = float(np.abs(g - ref).max())
    assert err < ATOL, err
    return err


@pytest.mark.parametrize("Hq,Hkv", [(6, 2), (2, 2), (8, 4), (8, 1), (24, 8), (10, 2), (6, 1), (14, 2)])
def test_prefill_int4_whole_prompt(Hq, Hkv):
    # the first prefill: the cache holds the prompt (completed pages + tail), S_q == S_kv
    _check(PrefillCase(Hq + Hkv, Hq=Hq, Hkv=Hkv, S=320, T=23))


@pytest.mark.parametrize("S,T,Sq,off", [(512, 0, 64, 0), (512, 40, 100, 0), (512, 40, 100, 452),
                                        (1024, 63, 300, 787), (128, 5, 3, 0)])
def test_prefill_int4_chunk(S, T, Sq, off):
    # a later chunk: S_q < S_kv; off 0 is torch's is_causal (the reference's call), S_kv - S_q lower-right
    _check(PrefillCase(S + T + Sq, S=S, T=T, Sq=Sq, causal_offset=off))


@pytest.mark.parametrize("kw", [dict(meta="f16"), dict(vgroup=32), dict(page=32, S=256, T=31),
                                dict(page=128, S=384, T=100), dict(S=0, T=77), dict(S=448, T=0),
                                dict(B=2, S=192, T=9), dict(S=64, T=1, Sq=65)])
def test_prefill_int4_layouts(kw):
    _check(PrefillCase(7, **kw))


@pytest.mark.parametrize("kw", [dict(), dict(meta="f16"), dict(Sq=90, causal_offset=0, T=12),
                                dict(Hq=8, Hkv=2, S=640, T=33), dict(S=0, T=50)])
def test_prefill_int8(kw):
    _check(PrefillCase(11, bits=8, **kw))


def test_prefill_matches_sdpa_at_size():
    """S_kv = 4096 + 37, 24 / 8 heads: vs F.scaled_dot_product_attention over
    the reference's dequantise + concatenate tensors (llama_persistent_patch.py:196-201)."""
    from flashquest_amd.kernel import dequantize_k_int4, dequantize_v_int4, flash_attn_prefill_int4, quantize_k_int4, \
        quantize_v_int4
    torch.manual_seed(0)
    dev = torch.device("cuda:0")
    S, T = 4096, 37
    K = torch.randn(1, 8, S + T, 128, device=dev).to(torch.bfloat16)
    V = torch.randn(1, 8, S + T, 128, device=dev).to(torch.bfloat16)
    q = torch.randn(1, 24, S + T, 128, device=dev).to(torch.bfloat16)
    kp, ks, km = quantize_k_int4(K[:, :, :S].contiguous(), 64)
    vp, vs, vm = quantize_v_int4(V[:, :, :S].contiguous())
    out = flash_attn_prefill_int4(q, kp, ks, km, vp, vs, vm, K[:, :, S:], V[:, :, S:], page_size=64)
    Kf = torch.cat([dequantize_k_int4(kp, ks, km, 64), K[:, :, S:]], dim=2)
    Vf = torch.cat([dequantize_v_int4(vp, vs, vm), V[:, :, S:]], dim=2)
    ref = F.scaled_dot_product_attention(q.float(), Kf.float(), Vf.float(), is_causal=True, enable_gqa=True)
    ref_bf16 = F.scaled_dot_product_attention(q, Kf, Vf, is_causal=True, enable_gqa=True)
    err = (out.float() - ref).abs().max().item()
    err_sdpa = (ref_bf16.float() - ref).abs().max().item()
    assert err < max(2 * err_sdpa, 1e-2), (err, err_sdpa)


def test_prefill_rejects_bad_arguments():
    from flashquest_amd.kernel import flash_attn_prefill_int4
    c = PrefillCase(1, S=128, T=0)
    args = [to_dev(c.kc), to_dev_half(c.ks, "bf16"), to_dev_half(c.km, "bf16"), to_dev(c.vc),
            to_dev_half(c.vs, "bf16"), to_dev_half(c.vm, "bf16")]
    q = to_dev_half(c.Q, "bf16")
    with pytest.raises(ValueError):
        flash_attn_prefill_int4(q[:, :5], *args)                      # H_q not a multiple of H_kv
    with pytest.raises(ValueError):
        flash_attn_prefill_int4(q, *args, causal_offset=-1)
    with pytest.raises(NotImplementedError):
        flash_attn_prefill_int4(q[..., :64].contiguous(), *[a[..., :32] if i in (0, 3) else a[..., :64] if i in (1, 2)
                                                           else a for i, a in enumerate(args)])


@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_over_persistent_cache_views(bits):
    """The patch's prefill step: update_quantized(k, v) then attention over the
    layer's views, for a first chunk and a second chunk (S_q < S_kv, is_causal)."""
    from flashquest_amd.cache import PersistentInt4KVCache, PersistentInt8KVCache
    from flashquest_amd.eager import prefill_attention_layer
    rng = np.random.default_rng(40 + bits)
    B, Hq, H, D = 1, 6, 2, 128
    n1, n2 = 300, 77
    K, V = make_kv(rng, B, H, n1 + n2, D, "bf16")
    Q = O.round_bf16(rng.standard_normal((B, Hq, n1 + n2, D)).astype(np.float32))
    cls = PersistentInt4KVCache if bits == 4 else PersistentInt8KVCache
    cache = cls(batch_size=B, num_layers=1, num_kv_heads=H, head_dim=D, max_seq_len=512)
    for lo, hi in ((0, n1), (n1, n1 + n2)):
        cache.update_quantized(to_dev_half(K[:, :, lo:hi], "bf16"), to_dev_half(V[:, :, lo:hi], "bf16"), 0)
        views = cache.get_views(0)
        out = prefill_attention_layer(to_dev_half(Q[:, :, lo:hi], "bf16"), views, page_size=64)
        comp = views["completed_len"]
        if bits == 4:
            kc, ks, km = O.quantize_k_int4(K[:, :, :comp], 64)
            vc, vs, vm = O.quantize_v_int4(V[:, :, :comp])
        else:
            kc, ks, km = O.quantize_k_int8(K[:, :, :comp], 64)
            vc, vs, vm = O.quantize_v_int8(V[:, :, :comp])
        ref = O.prefill_packed(Q[:, :, lo:hi], kc, ks, km, vc, vs, vm, K[:, :, comp:hi], V[:, :, comp:hi],
                               page_size=64, bits=bits)
        assert float(np.abs(out.float().cpu().numpy() - ref).max()) < ATOL


@pytest.mark.parametrize("kw", [dict(S=512, T=40, Sq=80, causal_offset=472), dict(S=512, T=40, Sq=80, meta="f16"),
                                dict(S=256, T=9, Sq=60, vgroup=32, causal_offset=205), dict(S=960, T=63, Sq=20),
                                dict(S=384, T=7, Sq=33, bits=8, causal_offset=358), dict(S=0, T=40, Sq=40, bits=8)])
def test_prefill_single_pass_path(kw):
    # one row block over at most 1024 attended keys: the kernel dequantises its own tiles
    _check(PrefillCase(5, **kw))


def _turbo_case(seed, B=1, Hq=6, Hkv=2, S=256, T=17, Sq=None):
    rng = np.random.default_rng(seed)
    K, V = make_kv(rng, B, Hkv, S + T, 128, "bf16")
    km, kl, ks = O.quantize_turbo(K[:, :, :S])
    vm, vl, vs = O.quantize_turbo(V[:, :, :S])
    Sq = S + T if Sq is None else Sq
    Q = O.round_bf16(rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32))
    return K, V, Q, (km, kl, ks, vm, vl, vs)


@pytest.mark.parametrize("S,T,Sq,off,Hq,Hkv", [(256, 17, None, 0, 6, 2), (512, 0, None, 0, 8, 2),
                                               (384, 40, 100, 0, 24, 8), (384, 40, 100, 324, 6, 2),
                                               (0, 50, None, 0, 4, 4)])
def test_prefill_turbo(S, T, Sq, off, Hq, Hkv):
    """The TurboQuant prefill: dequantize_k_turbo / dequantize_v_turbo (codebook x scale, inverse WHT,
    bf16; kv_quant.py:366-420), the bf16 tail, causal SDPA."""
    from flashquest_amd.kernel import flash_attn_prefill_turbo
    K, V, Q, (km, kl, ks, vm, vl, vs) = _turbo_case(S + T + Hq, Hq=Hq, Hkv=Hkv, S=S, T=T, Sq=Sq)
    out = flash_attn_prefill_turbo(to_dev_half(Q, "bf16"), to_dev(km), to_dev(kl), to_dev_half(ks, "bf16"),
                                   to_dev(vm), to_dev(vl), to_dev_half(vs, "bf16"),
                                   to_dev_half(K[:, :, S:], "bf16"), to_dev_half(V[:, :, S:], "bf16"),
                                   page_size=64, causal_offset=off)
    Kf = np.concatenate([O.dequant_turbo_bf16(km, kl, ks), K[:, :, S:]], axis=2)
    Vf = np.concatenate([O.dequant_turbo_bf16(vm, vl, vs), V[:, :, S:]], axis=2)
    ref = O.causal_prefill_attention(Q, Kf, Vf, causal_offset=off)
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) < ATOL


def test_prefill_over_persistent_turbo_views():
    from flashquest_amd.cache import PersistentTurboKVCache
    from flashquest_amd.eager import prefill_attention_layer
    rng = np.random.default_rng(77)
    B, Hq, H, n = 1, 6, 2, 333
    K, V = make_kv(rng, B, H, n, 128, "bf16")
    Q = O.round_bf16(rng.standard_normal((B, Hq, n, 128)).astype(np.float32))
    cache = PersistentTurboKVCache(batch_size=B, num_layers=1, num_kv_heads=H, head_dim=128, max_seq_len=512)
    cache.update_quantized(to_dev_half(K, "bf16"), to_dev_half(V, "bf16"), 0)
    views = cache.get_views(0)
    out = prefill_attention_layer(to_dev_half(Q, "bf16"), views, page_size=64)
    comp = views["completed_len"]
    km, kl, ks = O.quantize_turbo(K[:, :, :comp])
    vm, vl, vs = O.quantize_turbo(V[:, :, :comp])
    Kf = np.concatenate([O.dequant_turbo_bf16(km, kl, ks), K[:, :, comp:]], axis=2)
    Vf = np.concatenate([O.dequant_turbo_bf16(vm, vl, vs), V[:, :, comp:]], axis=2)
    ref = O.causal_prefill_attention(Q, Kf, Vf)
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) < ATOL


@pytest.mark.parametrize("kw", [dict(S=8192, T=30, Sq=64, causal_offset=8158), dict(S=4096, T=0, Sq=16, causal_offset=4080),
                                dict(S=4096, T=5, Sq=200, causal_offset=3901, bits=8),
                                dict(S=2048, T=64, Sq=300, Hq=8, Hkv=2, causal_offset=1812)])
def test_prefill_key_range_splits(kw):
    # few query rows over many keys: workgroups take slices of the key range, a merge launch combines them
    _check(PrefillCase(13, **kw))


def test_prefill_key_range_splits_between_128_and_256_workgroups():
    # 10 row blocks x 16 (sequence, KV head) pairs = 160 workgroups: split in 3
    # key ranges so the 480 workgroups fill two rounds of the CUs
    _check(PrefillCase(21, B=2, Hq=24, Hkv=8, S=2048, T=30, Sq=800, causal_offset=2078 - 800))


def test_prefill_turbo_key_range_splits():
    from flashquest_amd.kernel import flash_attn_prefill_turbo
    S, T, Sq = 4096, 20, 48
    K, V, Q, (km, kl, ks, vm, vl, vs) = _turbo_case(3, S=S, T=T, Sq=Sq)
    off = S + T - Sq
    out = flash_attn_prefill_turbo(to_dev_half(Q, "bf16"), to_dev(km), to_dev(kl), to_dev_half(ks, "bf16"),
                                   to_dev(vm), to_dev(vl), to_dev_half(vs, "bf16"),
                                   to_dev_half(K[:, :, S:], "bf16"), to_dev_half(V[:, :, S:], "bf16"),
                                   page_size=64, causal_offset=off)
    Kf = np.concatenate([O.dequant_turbo_bf16(km, kl, ks), K[:, :, S:]], axis=2)
    Vf = np.concatenate([O.dequant_turbo_bf16(vm, vl, vs), V[:, :, S:]], axis=2)
    ref = O.causal_prefill_attention(Q, Kf, Vf, causal_offset=off)
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) < ATOL


@pytest.mark.parametrize("kw", [dict(B=2, S=2048, T=11, Sq=40, causal_offset=2019), dict(B=2, S=640, T=0, Sq=None),
                                dict(page=32, S=2048, T=20, Sq=70, causal_offset=1998, meta="f16", vgroup=32)])
def test_prefill_batch_and_layout_mixes(kw):
    _check(PrefillCase(17, **kw))


def test_prefill_fp16_query_is_cast_like_the_reference():
    # the reference casts q (and the new K/V) to bf16 before the cache and SDPA (llama_persistent_patch.py:183-190)
    c = PrefillCase(19, S=320, T=9)
    from flashquest_amd.kernel import flash_attn_prefill_int4
    m = c.meta
    args = (to_dev(c.kc), to_dev_half(c.ks, m), to_dev_half(c.km, m), to_dev(c.vc), to_dev_half(c.vs, m),
            to_dev_half(c.vm, m), to_dev_half(c.Kt, "bf16"), to_dev_half(c.Vt, "bf16"))
    qb = to_dev_half(c.Q, "bf16")
    o16 = flash_attn_prefill_int4(qb.to(torch.float16), *args, page_size=c.page)
    o = flash_attn_prefill_int4(qb, *args, page_size=c.page)
    # Q holds bf16 values; fp16 holds most of them exactly, so the outputs agree to bf16 rounding
    assert o16.dtype == torch.bfloat16
    assert float((o16.float() - o.float()).abs().max()) < 2e-2
