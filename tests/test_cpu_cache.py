"""Host-side checks of the persistent caches (no GPU): the classes mirror the
reference's constructor validation and HF Cache base."""
import pytest


def test_cache_classes_import_and_validate():
    from transformers.cache_utils import Cache

    from flashquest_amd.cache import PersistentInt4KVCache, PersistentTurboKVCache
    assert issubclass(PersistentInt4KVCache, Cache) and issubclass(PersistentTurboKVCache, Cache)
    assert PersistentInt4KVCache.kv_bits == 4 and PersistentTurboKVCache.kv_bits == 3
    with pytest.raises(ValueError):
        PersistentInt4KVCache(batch_size=1, num_layers=1, num_kv_heads=1, head_dim=7, max_seq_len=8, device="cpu")
    with pytest.raises(ValueError):
        PersistentInt4KVCache(batch_size=1, num_layers=1, num_kv_heads=1, head_dim=64, max_seq_len=8, device="cpu",
                              v_group=24)
    with pytest.raises(ValueError):
        PersistentTurboKVCache(batch_size=1, num_layers=1, num_kv_heads=1, head_dim=96, max_seq_len=8, device="cpu")


def test_cpu_cache_views_shapes():
    # buffers and views on the host (no kernel runs): the reference's shapes
    from flashquest_amd.cache import PersistentInt4KVCache
    c = PersistentInt4KVCache(batch_size=2, num_layers=3, num_kv_heads=4, head_dim=128, max_seq_len=200, device="cpu",
                              v_group=32)
    assert c.K_packed.shape == (3, 2, 4, 200, 64) and c.K_scale.shape == (3, 2, 4, 4, 128)
    assert c.V_scale.shape == (3, 2, 4, 200, 4) and c.K_partial.shape == (3, 2, 4, 64, 128)
    v = c.get_views(2)
    assert v["seq_len"] == 0 and v["K_packed"].shape == (2, 4, 0, 64) and v["K_partial"].shape == (2, 4, 0, 128)
    with pytest.raises(IndexError):
        c.get_views(3)
