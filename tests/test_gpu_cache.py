"""Persistent INT4 / INT8 / turbo caches (src/flashquest/cache/persistent_{int4,int8,turbo}.py):
a stream appended in chunks of every shape (single decode tokens, chunks that
end inside a page, exactly on a page, or span several pages) leaves exactly
what quantising the whole stream at once gives (bit-exact codes and metadata,
oracle quantisers), the tail holds the incomplete page, and a decode step over
the cache views matches the oracle's sparse attention merged with the tail."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import TORCH_HALF, max_err, to_dev_half

pytestmark = pytest.mark.gpu

CHUNKS = [1, 5, 58, 64, 70, 1, 1, 127, 3, 200, 1]


def _stream(rng, B, H, S, D):
    K = rng.standard_normal((B, H, S, D)).astype(np.float32) * rng.lognormal(0.0, 1.0, (B, H, 1, D)).astype(np.float32)
    V = rng.standard_normal((B, H, S, D)).astype(np.float32)
    return O.round_bf16(K), O.round_bf16(V)


def _np(t):
    return t.float().cpu().numpy() if t.dtype != torch.uint8 else t.cpu().numpy()


@pytest.mark.parametrize("D,meta,vgroup", [(128, "bf16", None), (128, "f16", 32), (64, "bf16", None),
                                           (64, "f16", 32)])
def test_int4_appends_equal_whole_stream_quantisation(D, meta, vgroup):
    from flashquest_amd.cache import PersistentInt4KVCache
    rng = np.random.default_rng(11 + D)
    B, H, layers, layer = 2, 3, 3, 1
    total = sum(CHUNKS)
    K, V = _stream(rng, B, H, total, D)
    cache = PersistentInt4KVCache(batch_size=B, num_layers=layers, num_kv_heads=H, head_dim=D,
                                  max_seq_len=total + 7, meta_dtype=TORCH_HALF[meta], v_group=vgroup)
    assert cache._kernel_append               # the HIP append path
    pos = 0
    for n in CHUNKS:
        cache.update_quantized(to_dev_half(K[:, :, pos:pos + n], "bf16"), to_dev_half(V[:, :, pos:pos + n], "bf16"),
                               layer)
        pos += n
        v = cache.get_views(layer)
        comp = pos - pos % 64
        assert (v["seq_len"], v["completed_len"], v["partial_len"]) == (pos, comp, pos % 64)
        kp, ks, km = O.quantize_k_int4(K[:, :, :comp], 64, "bf16", meta)
        vp, vs, vm = O.quantize_v_int4(V[:, :, :comp], vgroup, meta)
        for name, ref in (("K_packed", kp), ("K_scale", ks), ("K_mn", km), ("V_packed", vp), ("V_scale", vs),
                          ("V_mn", vm)):
            assert np.array_equal(_np(v[name]), ref), (n, pos, name)
        assert np.array_equal(_np(v["K_partial"]), K[:, :, comp:pos])
        assert np.array_equal(_np(v["V_partial"]), V[:, :, comp:pos])
    assert cache.get_seq_length(layer) == total and cache.get_seq_length(0) == 0
    assert not cache.K_packed[0].any() and not cache.K_scale[2].any()      # other layers untouched


def test_int4_concat_path_and_errors():
    # page size 16 and fp32 new tokens take the concatenate-then-quantise sequence
    from flashquest_amd.cache import PersistentInt4KVCache
    rng = np.random.default_rng(3)
    B, H, D, page = 1, 2, 32, 16
    K, V = _stream(rng, B, H, 75, D)
    cache = PersistentInt4KVCache(batch_size=B, num_layers=1, num_kv_heads=H, head_dim=D, max_seq_len=80,
                                  page_size=page)
    assert not cache._kernel_append
    pos = 0
    for n in (3, 20, 1, 51):
        cache.update_quantized(torch.from_numpy(K[:, :, pos:pos + n]).cuda(), torch.from_numpy(V[:, :, pos:pos + n]).cuda(), 0)
        pos += n
    v = cache.get_views(0)
    comp = pos - pos % page
    kp, ks, km = O.quantize_k_int4(K[:, :, :comp], page, "f32", "bf16")
    vp, vs, vm = O.quantize_v_int4(V[:, :, :comp], None, "bf16")
    # the tail is bf16 and fp32 tokens join it by type promotion, so the first page's
    # scale arithmetic runs in fp32 on bf16-exact values: the same codes and metadata
    assert np.array_equal(_np(v["K_packed"]), kp) and np.array_equal(_np(v["V_packed"]), vp)
    assert np.array_equal(_np(v["K_scale"]), ks) and np.array_equal(_np(v["V_mn"]), vm)
    # the exception types and message keys the reference's tests match on
    # (tests/test_persistent_cache.py:96-107, test_persistent_int4.py:36-74)
    with pytest.raises(IndexError, match="layer_idx"):
        cache.get_views(1)
    with pytest.raises(IndexError, match="layer_idx"):
        cache.update_quantized(torch.zeros(1, 2, 1, D, device="cuda"), torch.zeros(1, 2, 1, D, device="cuda"), -1)
    with pytest.raises(RuntimeError, match="exceeds max_seq_len"):
        cache.update_quantized(torch.zeros(1, 2, 6, D, device="cuda"), torch.zeros(1, 2, 6, D, device="cuda"), 0)
    with pytest.raises(NotImplementedError):
        cache.update(None, None, 0)
    with pytest.raises(ValueError, match="even head_dim"):
        PersistentInt4KVCache(batch_size=1, num_layers=1, num_kv_heads=1, head_dim=7, max_seq_len=8)


@pytest.mark.parametrize("D", [128, 64])
def test_turbo_appends_equal_whole_stream_quantisation(D):
    # fq_turbo_cache_append: after every chunk the completed pages equal the
    # oracle's quantisation of the whole stream so far, bit for bit
    from flashquest_amd.cache import PersistentTurboKVCache
    rng = np.random.default_rng(5 + D)
    B, H = 2, 2
    total = sum(CHUNKS)
    K, V = _stream(rng, B, H, total, D)
    cache = PersistentTurboKVCache(batch_size=B, num_layers=2, num_kv_heads=H, head_dim=D, max_seq_len=total)
    assert cache._kernel_append
    pos = 0
    for n in CHUNKS:
        cache.update_quantized(to_dev_half(K[:, :, pos:pos + n], "bf16"), to_dev_half(V[:, :, pos:pos + n], "bf16"), 1)
        pos += n
        v = cache.get_views(1)
        comp = pos - pos % 64
        assert (v["seq_len"], v["completed_len"], v["partial_len"]) == (pos, comp, pos % 64)
        km, kl, kst, ksr, kmr = O.quantize_k_turbo(K[:, :, :comp], 64, "bf16")
        vm_, vl, vst = O.quantize_turbo(V[:, :, :comp], "bf16")
        for name, ref in (("K_msb", km), ("K_lsb", kl), ("K_scale_turbo", kst), ("K_scale_raw", ksr),
                          ("K_mn_raw", kmr), ("V_msb", vm_), ("V_lsb", vl), ("V_scale_turbo", vst)):
            assert np.array_equal(_np(v[name]), ref), (n, pos, name)
        assert np.array_equal(_np(v["K_partial"]), K[:, :, comp:pos])
        assert np.array_equal(_np(v["V_partial"]), V[:, :, comp:pos])
    assert not cache.K_msb[0].any() and not cache.K_scale_raw[0].any()      # other layer untouched
    with pytest.raises(ValueError, match="multiple of 8"):
        PersistentTurboKVCache(batch_size=1, num_layers=1, num_kv_heads=1, head_dim=12, max_seq_len=8)
    with pytest.raises(ValueError, match="power of two"):
        PersistentTurboKVCache(batch_size=1, num_layers=1, num_kv_heads=1, head_dim=24, max_seq_len=8)


@pytest.mark.parametrize("meta", ["bf16", "f16"])
def test_int8_appends_equal_whole_stream_quantisation(meta):
    # fq_int8_cache_append: codes and metadata equal the oracle's INT8
    # quantisation of the whole stream after every chunk; the tail holds the
    # incomplete page and zeros after it (persistent_int8.py:129-132)
    from flashquest_amd.cache import PersistentInt8KVCache
    rng = np.random.default_rng(17)
    B, H, D = 1, 3, 128
    total = sum(CHUNKS)
    K, V = _stream(rng, B, H, total, D)
    cache = PersistentInt8KVCache(batch_size=B, num_layers=2, num_kv_heads=H, head_dim=D, max_seq_len=total + 3,
                                  meta_dtype=TORCH_HALF[meta])
    assert cache._kernel_append
    pos = 0
    for n in CHUNKS:
        cache.update_quantized(to_dev_half(K[:, :, pos:pos + n], "bf16"), to_dev_half(V[:, :, pos:pos + n], "bf16"), 0)
        pos += n
        v = cache.get_views(0)
        comp = pos - pos % 64
        ku, ks, km = O.quantize_k_int8(K[:, :, :comp], 64, "bf16", meta)
        vu, vs, vm = O.quantize_v_int8(V[:, :, :comp], meta)
        for name, ref in (("K_uint8", ku), ("K_scale", ks), ("K_mn", km), ("V_uint8", vu), ("V_scale", vs),
                          ("V_mn", vm)):
            assert np.array_equal(_np(v[name]), ref), (n, pos, name)
        assert np.array_equal(_np(v["K_partial"]), K[:, :, comp:pos])
        assert not cache.K_partial[0, :, :, pos - comp:].any() and not cache.V_partial[0, :, :, pos - comp:].any()
    with pytest.raises(RuntimeError):
        cache.update(None, None, 0)


@pytest.mark.parametrize("partial", [0, 1, 37])
def test_decode_over_cache_views_matches_oracle(partial):
    # the decode branch of the reference's attention patch over the cache: sparse
    # attention on the completed pages, dense bf16 attention on the tail, LSE merge
    from flashquest_amd.cache import PersistentInt4KVCache
    from flashquest_amd.eager.decode import sparse_decode_layer
    rng = np.random.default_rng(21 + partial)
    B, Hq, H, D, P = 1, 6, 2, 128, 12
    S = 64 * P + partial
    K, V = _stream(rng, B, H, S, D)
    Q = O.round_bf16(rng.standard_normal((B, Hq, D)).astype(np.float32))
    cache = PersistentInt4KVCache(batch_size=B, num_layers=1, num_kv_heads=H, head_dim=D, max_seq_len=S)
    cache.update_quantized(to_dev_half(K[:, :, :S - 1], "bf16"), to_dev_half(V[:, :, :S - 1], "bf16"), 0)
    cache.update_quantized(to_dev_half(K[:, :, S - 1:], "bf16"), to_dev_half(V[:, :, S - 1:], "bf16"), 0)
    views = cache.get_views(0)
    q = to_dev_half(Q, "bf16")[:, :, None, :]
    out = sparse_decode_layer(q, views, retention=0.3, num_sinks=1, window_pages=1, page_size=64)
    comp = 64 * P
    kp, ks, km = O.quantize_k_int4(K[:, :, :comp], 64)
    vp, vs, vm = O.quantize_v_int4(V[:, :, :comp])
    ref = O.decode_step(Q, kp, ks, km, vp, vs, vm, retention=0.3, num_sinks=1, window_pages=1)
    O_ref = ref["O"]
    if partial:
        ot, lt = O.dense_attn_with_lse(Q, K[:, :, comp:], V[:, :, comp:])
        O_ref = O.merge_two_attentions(O.round_bf16(O_ref), ref["lse"], O.round_bf16(ot), lt)
    assert max_err(out[:, :, 0], O_ref) <= 2e-2
