"""Persistent INT8 KV cache (src/flashquest/cache/persistent_int8.py:14-181).

Same buffers, shapes, dtypes and methods as the reference class: uint8 K/V
codes (L, B, H_kv, max_seq_len, D), per-page per-channel K scale/min
(L, B, H_kv, max_pages, D), per-token V scale/min (L, B, H_kv, max_seq_len, 1)
and a bf16 partial-page tail (L, B, H_kv, page_size, D).  update_quantized
follows the reference's sequence (concatenate the tail and the new tokens,
quantise the completed pages, stage the rest in the tail and zero the rest of
the tail), with the HIP quantisers writing straight into the cache slices.
Extension: ``meta_dtype`` (bf16, the reference, or fp16).
"""
from __future__ import annotations

import torch
from transformers.cache_utils import Cache

from ..kernel.kv_quant import quantize_k, quantize_v


class PersistentInt8KVCache(Cache):
    kv_bits = 8

    def __init__(self, *, batch_size: int, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 page_size: int = 64, device: str | torch.device = "cuda", meta_dtype: torch.dtype = torch.bfloat16):
        self.layers: list = []
        self.layer_class_to_replicate = None
        self.offloading = False
        self._batch_size = batch_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.page_size = page_size
        self.max_pages = (max_seq_len + page_size - 1) // page_size
        dev = torch.device(device)
        shape_kv = (num_layers, batch_size, num_kv_heads, max_seq_len, head_dim)
        shape_kpage = (num_layers, batch_size, num_kv_heads, self.max_pages, head_dim)
        shape_vtok = (num_layers, batch_size, num_kv_heads, max_seq_len, 1)
        shape_partial = (num_layers, batch_size, num_kv_heads, page_size, head_dim)
        self.K_uint8 = torch.zeros(shape_kv, dtype=torch.uint8, device=dev)
        self.V_uint8 = torch.zeros(shape_kv, dtype=torch.uint8, device=dev)
        self.K_scale = torch.zeros(shape_kpage, dtype=meta_dtype, device=dev)
        self.K_mn = torch.zeros(shape_kpage, dtype=meta_dtype, device=dev)
        self.V_scale = torch.zeros(shape_vtok, dtype=meta_dtype, device=dev)
        self.V_mn = torch.zeros(shape_vtok, dtype=meta_dtype, device=dev)
        self.K_partial = torch.zeros(shape_partial, dtype=torch.bfloat16, device=dev)
        self.V_partial = torch.zeros(shape_partial, dtype=torch.bfloat16, device=dev)
        self._seen_tokens = [0] * num_layers

    # transformers' Cache derives these from its layer list, which the patched
    # path leaves empty; the preallocated shapes answer them here.
    @property
    def batch_size(self) -> int:
        return self._batch_size

    @property
    def max_batch_size(self) -> int:
        return self._batch_size

    @property
    def max_cache_len(self) -> int:
        return self.max_seq_len

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seen_tokens[layer_idx]

    def get_max_length(self) -> int:
        return self.max_seq_len

    def _check_layer(self, layer_idx: int):
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise IndexError(f"layer_idx {layer_idx} out of range [0, {self.num_layers})")

    def update_quantized(self, K_new: torch.Tensor, V_new: torch.Tensor, layer_idx: int) -> None:
        """Append K_new, V_new (B, H_kv, S_new, D) to layer_idx's cache
        (persistent_int8.py:72-135)."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        S_new = K_new.shape[2]
        if seen + S_new > self.max_seq_len:
            raise RuntimeError(f"PersistentInt8KVCache: seen+new={seen + S_new} exceeds "
                               f"max_seq_len={self.max_seq_len}")
        page_size = self.page_size
        partial_len = seen % page_size
        K_full = torch.cat([self.K_partial[layer_idx, :, :, :partial_len, :], K_new], dim=2)
        V_full = torch.cat([self.V_partial[layer_idx, :, :, :partial_len, :], V_new], dim=2)
        total = K_full.shape[2]
        n_complete = total // page_size
        complete_len = n_complete * page_size
        lay = layer_idx
        if n_complete > 0:
            tok0 = seen - partial_len
            p0 = tok0 // page_size
            quantize_k(K_full[:, :, :complete_len], page_size, meta_dtype=self.K_scale.dtype,
                       out=(self.K_uint8[lay, :, :, tok0:tok0 + complete_len],
                            self.K_scale[lay, :, :, p0:p0 + n_complete],
                            self.K_mn[lay, :, :, p0:p0 + n_complete]))
            quantize_v(V_full[:, :, :complete_len], meta_dtype=self.V_scale.dtype,
                       out=(self.V_uint8[lay, :, :, tok0:tok0 + complete_len],
                            self.V_scale[lay, :, :, tok0:tok0 + complete_len],
                            self.V_mn[lay, :, :, tok0:tok0 + complete_len]))
        rest = total - complete_len
        if rest > 0:
            self.K_partial[lay, :, :, :rest, :] = K_full[:, :, complete_len:, :]
            self.V_partial[lay, :, :, :rest, :] = V_full[:, :, complete_len:, :]
        if rest < page_size:
            self.K_partial[lay, :, :, rest:, :].zero_()
            self.V_partial[lay, :, :, rest:, :].zero_()
        self._seen_tokens[layer_idx] = seen + S_new

    def get_views(self, layer_idx: int) -> dict:
        """persistent_int8.py:137-169: views up to the completed pages, plus the tail."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        partial_len = seen % self.page_size
        completed_len = seen - partial_len
        n_pages = completed_len // self.page_size
        return {
            "seq_len": seen,
            "completed_len": completed_len,
            "partial_len": partial_len,
            "K_uint8": self.K_uint8[layer_idx, :, :, :completed_len, :],
            "V_uint8": self.V_uint8[layer_idx, :, :, :completed_len, :],
            "K_scale": self.K_scale[layer_idx, :, :, :n_pages, :],
            "K_mn": self.K_mn[layer_idx, :, :, :n_pages, :],
            "V_scale": self.V_scale[layer_idx, :, :, :completed_len, :],
            "V_mn": self.V_mn[layer_idx, :, :, :completed_len, :],
            "K_partial": self.K_partial[layer_idx, :, :, :partial_len, :],
            "V_partial": self.V_partial[layer_idx, :, :, :partial_len, :],
        }

    def update(self, *args, **kwargs):
        """HF Cache.update is unused on the patched path (persistent_int8.py:171-181)."""
        raise RuntimeError("PersistentInt8KVCache.update should not be called directly; "
                           "the flashquest patch uses update_quantized() + get_views().")
