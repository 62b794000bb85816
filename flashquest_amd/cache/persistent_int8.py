"""Persistent INT8 KV cache (src/flashquest/cache/persistent_int8.py:14-181).

Same buffers, shapes, dtypes and methods as the reference class: uint8 K/V
codes (L, B, H_kv, max_seq_len, D), per-page per-channel K scale/min
(L, B, H_kv, max_pages, D), per-token V scale/min (L, B, H_kv, max_seq_len, 1)
and a bf16 partial-page tail (L, B, H_kv, page_size, D) whose rows after the
staged tokens are kept at zero, as the reference's are.  update_quantized is
one HIP append (fq_int8_cache_append).  Extension: ``meta_dtype`` (bf16, the
reference, or fp16).
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops
from ..kernel.kv_quant import quantize_k, quantize_v
from ._paged import PagedKVCache


class PersistentInt8KVCache(PagedKVCache):
    kv_bits = 8
    _name = "PersistentInt8KVCache"
    _zero_tail_after_append = True

    def __init__(self, *, batch_size: int, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 page_size: int = 64, device: str | torch.device = "cuda", meta_dtype: torch.dtype = torch.bfloat16):
        self._init_paged(batch_size, num_layers, num_kv_heads, head_dim, max_seq_len, page_size, device)
        rows = (num_layers, batch_size, num_kv_heads, max_seq_len)
        pages = (num_layers, batch_size, num_kv_heads, self.max_pages, head_dim)
        self.K_uint8 = torch.zeros(rows + (head_dim,), dtype=torch.uint8, device=self.device)
        self.V_uint8 = torch.zeros(rows + (head_dim,), dtype=torch.uint8, device=self.device)
        self.K_scale = torch.zeros(pages, dtype=meta_dtype, device=self.device)
        self.K_mn = torch.zeros(pages, dtype=meta_dtype, device=self.device)
        self.V_scale = torch.zeros(rows + (1,), dtype=meta_dtype, device=self.device)
        self.V_mn = torch.zeros(rows + (1,), dtype=meta_dtype, device=self.device)
        if self._kernel_append:
            self._desc, _ = _ops.int8_cache(self.K_uint8, self.K_scale, self.K_mn, self.V_uint8, self.V_scale,
                                            self.V_mn, page_size)

    def _append_kernel(self, layer_idx, seen, K_new, V_new):
        L.check(L.lib().fq_int8_cache_append(
            self._desc, layer_idx, self.K_partial.data_ptr(), self._kpart_s, self.V_partial.data_ptr(),
            self._vpart_s, L.dtype_code(self.K_partial.dtype), K_new.data_ptr(), L.strides(K_new, 4),
            V_new.data_ptr(), L.strides(V_new, 4), seen, K_new.shape[2], L.stream_handle(K_new.device)),
            "update_quantized")

    def _quantize_pages(self, layer_idx, tok0, K_pages, V_pages):
        t1, p0 = tok0 + K_pages.shape[2], tok0 // self.page_size
        p1 = p0 + K_pages.shape[2] // self.page_size
        quantize_k(K_pages, self.page_size, meta_dtype=self.K_scale.dtype,
                   out=(self.K_uint8[layer_idx, :, :, tok0:t1], self.K_scale[layer_idx, :, :, p0:p1],
                        self.K_mn[layer_idx, :, :, p0:p1]))
        quantize_v(V_pages, meta_dtype=self.V_scale.dtype,
                   out=(self.V_uint8[layer_idx, :, :, tok0:t1], self.V_scale[layer_idx, :, :, tok0:t1],
                        self.V_mn[layer_idx, :, :, tok0:t1]))

    def get_views(self, layer_idx: int) -> dict:
        """persistent_int8.py:137-169: the completed pages, then the tail."""
        self._check_layer(layer_idx)
        _, done, _, pages = self._counts(layer_idx)
        v = self._tail_views(layer_idx)
        v.update(K_uint8=self.K_uint8[layer_idx, :, :, :done], V_uint8=self.V_uint8[layer_idx, :, :, :done],
                 K_scale=self.K_scale[layer_idx, :, :, :pages], K_mn=self.K_mn[layer_idx, :, :, :pages],
                 V_scale=self.V_scale[layer_idx, :, :, :done], V_mn=self.V_mn[layer_idx, :, :, :done])
        return v

    def update(self, *args, **kwargs):
        """transformers' Cache.update (persistent_int8.py:171-181 raises RuntimeError)."""
        raise RuntimeError("PersistentInt8KVCache.update is not part of the packed-cache protocol; "
                           "use update_quantized() and get_views()")
