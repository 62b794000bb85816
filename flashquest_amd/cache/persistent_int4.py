"""Persistent INT4 KV cache (src/flashquest/cache/persistent_int4.py:14-166).

Same buffers, shapes, dtypes and methods as the reference class: K/V codes
packed two per byte (L, B, H_kv, max_seq_len, D/2), per-page per-channel K
scale/min (L, B, H_kv, max_pages, D), per-token V scale/min (L, B, H_kv,
max_seq_len, G) and a bf16 partial-page tail (L, B, H_kv, page_size, D).
Extensions: ``meta_dtype`` (bf16, the reference, or fp16) and ``v_group``
(None = one V group over all D, the reference; 32 = 32-channel groups).

update_quantized is one HIP append (fq_int4_cache_append): the pages that the
new tokens complete are quantised straight from the tail and the new tokens,
then the rest is staged in the tail (see ``PagedKVCache`` for the other
geometries).
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops
from ..kernel.kv_quant import quantize_k_int4, quantize_v_int4
from ._paged import PagedKVCache


class PersistentInt4KVCache(PagedKVCache):
    kv_bits = 4
    _name = "PersistentInt4KVCache"

    def __init__(self, *, batch_size: int, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 page_size: int = 64, device: str | torch.device = "cuda", meta_dtype: torch.dtype = torch.bfloat16,
                 v_group: int | None = None):
        if head_dim % 2:
            raise ValueError(f"PersistentInt4KVCache packs two 4-bit codes per byte and needs an even head_dim; "
                             f"got {head_dim}")
        if v_group is not None and (v_group < 2 or head_dim % v_group or v_group % 2):
            raise ValueError(f"v_group={v_group} must be an even divisor of head_dim={head_dim}")
        self._init_paged(batch_size, num_layers, num_kv_heads, head_dim, max_seq_len, page_size, device)
        self.v_group = v_group
        G = 1 if v_group is None else head_dim // v_group
        rows = (num_layers, batch_size, num_kv_heads, max_seq_len)
        pages = (num_layers, batch_size, num_kv_heads, self.max_pages, head_dim)
        self.K_packed = torch.zeros(rows + (head_dim // 2,), dtype=torch.uint8, device=self.device)
        self.V_packed = torch.zeros(rows + (head_dim // 2,), dtype=torch.uint8, device=self.device)
        self.K_scale = torch.zeros(pages, dtype=meta_dtype, device=self.device)
        self.K_mn = torch.zeros(pages, dtype=meta_dtype, device=self.device)
        self.V_scale = torch.zeros(rows + (G,), dtype=meta_dtype, device=self.device)
        self.V_mn = torch.zeros(rows + (G,), dtype=meta_dtype, device=self.device)
        self._kernel_append = self._kernel_append and G in (1, head_dim // 32)
        if self._kernel_append:
            self._desc, _ = _ops.int4_cache(self.K_packed, self.K_scale, self.K_mn, self.V_packed, self.V_scale,
                                            self.V_mn, page_size)

    def _append_kernel(self, layer_idx, seen, K_new, V_new):
        L.check(L.lib().fq_int4_cache_append(
            self._desc, layer_idx, self.K_partial.data_ptr(), self._kpart_s, self.V_partial.data_ptr(),
            self._vpart_s, L.dtype_code(self.K_partial.dtype), K_new.data_ptr(), L.strides(K_new, 4),
            V_new.data_ptr(), L.strides(V_new, 4), seen, K_new.shape[2], L.stream_handle(K_new.device)),
            "update_quantized")

    def _quantize_pages(self, layer_idx, tok0, K_pages, V_pages):
        t1, p0 = tok0 + K_pages.shape[2], tok0 // self.page_size
        p1 = p0 + K_pages.shape[2] // self.page_size
        quantize_k_int4(K_pages, self.page_size, out=(self.K_packed[layer_idx, :, :, tok0:t1],
                                                      self.K_scale[layer_idx, :, :, p0:p1],
                                                      self.K_mn[layer_idx, :, :, p0:p1]))
        quantize_v_int4(V_pages, v_group=self.v_group, out=(self.V_packed[layer_idx, :, :, tok0:t1],
                                                            self.V_scale[layer_idx, :, :, tok0:t1],
                                                            self.V_mn[layer_idx, :, :, tok0:t1]))

    def get_views(self, layer_idx: int) -> dict:
        """persistent_int4.py:134-159: the completed pages, then the tail."""
        self._check_layer(layer_idx)
        _, done, _, pages = self._counts(layer_idx)
        v = self._tail_views(layer_idx)
        v.update(K_packed=self.K_packed[layer_idx, :, :, :done], V_packed=self.V_packed[layer_idx, :, :, :done],
                 K_scale=self.K_scale[layer_idx, :, :, :pages], K_mn=self.K_mn[layer_idx, :, :, :pages],
                 V_scale=self.V_scale[layer_idx, :, :, :done], V_mn=self.V_mn[layer_idx, :, :, :done])
        return v
