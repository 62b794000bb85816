"""Persistent TurboQuant KV cache, K3-V3 (src/flashquest/cache/persistent_turbo.py:14-167).

Same buffers as the reference class: 3-bit K and V codes split into a 1-bit
MSB plane (..., D/8) and a 2-bit LSB plane (..., D/4), a per-token bf16 scale
for each, the un-rotated K's per-page per-channel INT4 scale/min (for page
scoring), and bf16 partial-page tails.  update_quantized follows the
reference's sequence (concatenate the tail and the new tokens, quantise the
completed pages, stage the rest), with the HIP quantisers writing straight
into the cache slices.
"""
from __future__ import annotations

import torch
from transformers.cache_utils import Cache

from ..kernel.kv_quant import quantize_k_turbo, quantize_v_turbo


class PersistentTurboKVCache(Cache):
    kv_bits = 3

    def __init__(self, *, batch_size: int, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 page_size: int = 64, device: str | torch.device = "cuda"):
        if head_dim % 8 != 0:
            raise ValueError(f"PersistentTurboKVCache requires head_dim multiple of 8 "
                             f"(MSB plane packs 8/byte); got {head_dim}")
        if head_dim & (head_dim - 1) != 0:
            raise ValueError(f"PersistentTurboKVCache requires head_dim power of 2 (WHT); got {head_dim}")
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
        shape_msb = (num_layers, batch_size, num_kv_heads, max_seq_len, head_dim // 8)
        shape_lsb = (num_layers, batch_size, num_kv_heads, max_seq_len, head_dim // 4)
        shape_tok = (num_layers, batch_size, num_kv_heads, max_seq_len, 1)
        shape_kpage = (num_layers, batch_size, num_kv_heads, self.max_pages, head_dim)
        shape_partial = (num_layers, batch_size, num_kv_heads, page_size, head_dim)
        self.K_msb = torch.zeros(shape_msb, dtype=torch.uint8, device=dev)
        self.K_lsb = torch.zeros(shape_lsb, dtype=torch.uint8, device=dev)
        self.K_scale_turbo = torch.zeros(shape_tok, dtype=torch.bfloat16, device=dev)
        self.K_scale_raw = torch.zeros(shape_kpage, dtype=torch.bfloat16, device=dev)
        self.K_mn_raw = torch.zeros(shape_kpage, dtype=torch.bfloat16, device=dev)
        self.V_msb = torch.zeros(shape_msb, dtype=torch.uint8, device=dev)
        self.V_lsb = torch.zeros(shape_lsb, dtype=torch.uint8, device=dev)
        self.V_scale_turbo = torch.zeros(shape_tok, dtype=torch.bfloat16, device=dev)
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
        """Append K_new, V_new (B, H_kv, S_new, D) bf16 (persistent_turbo.py:83-147)."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        S_new = K_new.shape[2]
        if seen + S_new > self.max_seq_len:
            raise RuntimeError(f"PersistentTurboKVCache: seen+new={seen + S_new} exceeds "
                               f"max_seq_len={self.max_seq_len}")
        page_size = self.page_size
        partial_len = seen % page_size
        if partial_len > 0:
            K_full = torch.cat([self.K_partial[layer_idx, :, :, :partial_len, :], K_new], dim=2)
            V_full = torch.cat([self.V_partial[layer_idx, :, :, :partial_len, :], V_new], dim=2)
        else:
            K_full, V_full = K_new, V_new
        total = K_full.shape[2]
        n_complete = total // page_size
        complete_len = n_complete * page_size
        if n_complete > 0:
            t0 = seen - partial_len
            t1 = t0 + complete_len
            p0 = t0 // page_size
            lay = layer_idx
            quantize_k_turbo(K_full[:, :, :complete_len], page_size,
                             out=(self.K_msb[lay, :, :, t0:t1], self.K_lsb[lay, :, :, t0:t1],
                                  self.K_scale_turbo[lay, :, :, t0:t1], self.K_scale_raw[lay, :, :, p0:p0 + n_complete],
                                  self.K_mn_raw[lay, :, :, p0:p0 + n_complete]))
            quantize_v_turbo(V_full[:, :, :complete_len],
                             out=(self.V_msb[lay, :, :, t0:t1], self.V_lsb[lay, :, :, t0:t1],
                                  self.V_scale_turbo[lay, :, :, t0:t1]))
        rest = total - complete_len
        self.K_partial[layer_idx, :, :, :rest, :] = K_full[:, :, complete_len:, :]
        self.V_partial[layer_idx, :, :, :rest, :] = V_full[:, :, complete_len:, :]
        self._seen_tokens[layer_idx] = seen + S_new

    def get_views(self, layer_idx: int) -> dict:
        """persistent_turbo.py:149-176."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        partial_len = seen % self.page_size
        completed_len = seen - partial_len
        n_pages = completed_len // self.page_size
        return {
            "seq_len": seen,
            "completed_len": completed_len,
            "partial_len": partial_len,
            "K_msb": self.K_msb[layer_idx, :, :, :completed_len, :],
            "K_lsb": self.K_lsb[layer_idx, :, :, :completed_len, :],
            "K_scale_turbo": self.K_scale_turbo[layer_idx, :, :, :completed_len, :],
            "K_scale_raw": self.K_scale_raw[layer_idx, :, :, :n_pages, :],
            "K_mn_raw": self.K_mn_raw[layer_idx, :, :, :n_pages, :],
            "V_msb": self.V_msb[layer_idx, :, :, :completed_len, :],
            "V_lsb": self.V_lsb[layer_idx, :, :, :completed_len, :],
            "V_scale_turbo": self.V_scale_turbo[layer_idx, :, :, :completed_len, :],
            "K_partial": self.K_partial[layer_idx, :, :, :partial_len, :],
            "V_partial": self.V_partial[layer_idx, :, :, :partial_len, :],
        }

    def update(self, *args, **kwargs):
        """HF Cache.update is unused on the patched path."""
        raise NotImplementedError("PersistentTurboKVCache.update is not used; the patched forward "
                                  "calls update_quantized directly.")
