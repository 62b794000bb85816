"""Persistent TurboQuant KV cache, K3-V3 (src/flashquest/cache/persistent_turbo.py:14-181).

Same buffers as the reference class: 3-bit K and V codes split into a 1-bit
MSB plane (..., D/8) and a 2-bit LSB plane (..., D/4), a per-token bf16 scale
for each, the un-rotated K's per-page per-channel INT4 scale/min (for page
scoring), and bf16 partial-page tails.  update_quantized is one HIP append
(fq_turbo_cache_append): the completed pages' raw K metadata, planes and
scales straight from the tail and the new tokens, then the tail staging.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops
from ..kernel.kv_quant import quantize_k_turbo, quantize_v_turbo
from ._paged import PagedKVCache


class PersistentTurboKVCache(PagedKVCache):
    kv_bits = 3
    _name = "PersistentTurboKVCache"

    def __init__(self, *, batch_size: int, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 page_size: int = 64, device: str | torch.device = "cuda"):
        if head_dim % 8:
            raise ValueError(f"PersistentTurboKVCache: head_dim={head_dim} must be a multiple of 8 "
                             "(one MSB byte holds 8 channels)")
        if head_dim & (head_dim - 1):
            raise ValueError(f"PersistentTurboKVCache: head_dim={head_dim} must be a power of two "
                             "(Walsh-Hadamard rotation)")
        self._init_paged(batch_size, num_layers, num_kv_heads, head_dim, max_seq_len, page_size, device)
        rows = (num_layers, batch_size, num_kv_heads, max_seq_len)
        pages = (num_layers, batch_size, num_kv_heads, self.max_pages, head_dim)
        u8, bf = dict(dtype=torch.uint8, device=self.device), dict(dtype=torch.bfloat16, device=self.device)
        self.K_msb = torch.zeros(rows + (head_dim // 8,), **u8)
        self.K_lsb = torch.zeros(rows + (head_dim // 4,), **u8)
        self.K_scale_turbo = torch.zeros(rows + (1,), **bf)
        self.K_scale_raw = torch.zeros(pages, **bf)
        self.K_mn_raw = torch.zeros(pages, **bf)
        self.V_msb = torch.zeros(rows + (head_dim // 8,), **u8)
        self.V_lsb = torch.zeros(rows + (head_dim // 4,), **u8)
        self.V_scale_turbo = torch.zeros(rows + (1,), **bf)
        if self._kernel_append:
            self._desc, _ = _ops.turbo_cache(self.K_msb, self.K_lsb, self.K_scale_turbo, self.V_msb, self.V_lsb,
                                             self.V_scale_turbo, self.max_pages, page_size)
            self._ksr_s = L.strides(self.K_scale_raw, 5)
            self._kmr_s = L.strides(self.K_mn_raw, 5)

    def _append_kernel(self, layer_idx, seen, K_new, V_new):
        L.check(L.lib().fq_turbo_cache_append(
            self._desc, self.K_scale_raw.data_ptr(), self._ksr_s, self.K_mn_raw.data_ptr(), self._kmr_s, layer_idx,
            self.K_partial.data_ptr(), self._kpart_s, self.V_partial.data_ptr(), self._vpart_s,
            L.dtype_code(self.K_partial.dtype), K_new.data_ptr(), L.strides(K_new, 4), V_new.data_ptr(),
            L.strides(V_new, 4), seen, K_new.shape[2], L.stream_handle(K_new.device)), "update_quantized")

    def _quantize_pages(self, layer_idx, tok0, K_pages, V_pages):
        t1, p0 = tok0 + K_pages.shape[2], tok0 // self.page_size
        p1 = p0 + K_pages.shape[2] // self.page_size
        lay = layer_idx
        quantize_k_turbo(K_pages, self.page_size,
                         out=(self.K_msb[lay, :, :, tok0:t1], self.K_lsb[lay, :, :, tok0:t1],
                              self.K_scale_turbo[lay, :, :, tok0:t1], self.K_scale_raw[lay, :, :, p0:p1],
                              self.K_mn_raw[lay, :, :, p0:p1]))
        quantize_v_turbo(V_pages, out=(self.V_msb[lay, :, :, tok0:t1], self.V_lsb[lay, :, :, tok0:t1],
                                       self.V_scale_turbo[lay, :, :, tok0:t1]))

    def get_views(self, layer_idx: int) -> dict:
        """persistent_turbo.py:149-176: the completed pages, then the tail."""
        self._check_layer(layer_idx)
        _, done, _, pages = self._counts(layer_idx)
        v = self._tail_views(layer_idx)
        lay = layer_idx
        v.update(K_msb=self.K_msb[lay, :, :, :done], K_lsb=self.K_lsb[lay, :, :, :done],
                 K_scale_turbo=self.K_scale_turbo[lay, :, :, :done], K_scale_raw=self.K_scale_raw[lay, :, :, :pages],
                 K_mn_raw=self.K_mn_raw[lay, :, :, :pages], V_msb=self.V_msb[lay, :, :, :done],
                 V_lsb=self.V_lsb[lay, :, :, :done], V_scale_turbo=self.V_scale_turbo[lay, :, :, :done])
        return v
