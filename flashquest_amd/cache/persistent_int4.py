"""Persistent INT4 KV cache (src/flashquest/cache/persistent_int4.py:14-166).

Same buffers, shapes, dtypes and methods as the reference class: K/V codes
packed two per byte (L, B, H_kv, max_seq_len, D/2), per-page per-channel K
scale/min (L, B, H_kv, max_pages, D), per-token V scale/min (L, B, H_kv,
max_seq_len, G) and a bf16 partial-page tail (L, B, H_kv, page_size, D).
Extensions: ``meta_dtype`` (bf16, the reference, or fp16) and ``v_group``
(None = one V group over all D, the reference; 32 = 32-channel groups).

update_quantized runs one HIP append (fq_int4_cache_append): the pages that
the new tokens complete are quantised straight from the tail and the new
tokens, then the rest is staged in the tail.  Shapes the append kernel does
not take (page size other than 64, head_dim other than 64/128, K_new in
another dtype than the tail) go through the reference's concatenate-then-
quantise sequence on the HIP quantisers.
"""
from __future__ import annotations

import torch
from transformers.cache_utils import Cache

from .. import _lib as L
from .. import _ops
from ..kernel.kv_quant import quantize_k_int4, quantize_v_int4


class PersistentInt4KVCache(Cache):
    kv_bits = 4

    def __init__(self, *, batch_size: int, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 page_size: int = 64, device: str | torch.device = "cuda", meta_dtype: torch.dtype = torch.bfloat16,
                 v_group: int | None = None):
        if head_dim % 2 != 0:
            raise ValueError(f"PersistentInt4KVCache requires even head_dim (2 INT4 per byte); got {head_dim}")
        if v_group is not None and (v_group < 2 or head_dim % v_group or v_group % 2):
            raise ValueError(f"v_group={v_group} must be an even divisor of head_dim={head_dim}")
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
        self.v_group = v_group
        dev = torch.device(device)
        G = 1 if v_group is None else head_dim // v_group
        shape_kv = (num_layers, batch_size, num_kv_heads, max_seq_len, head_dim // 2)
        shape_kpage = (num_layers, batch_size, num_kv_heads, self.max_pages, head_dim)
        shape_vtok = (num_layers, batch_size, num_kv_heads, max_seq_len, G)
        shape_partial = (num_layers, batch_size, num_kv_heads, page_size, head_dim)
        self.K_packed = torch.zeros(shape_kv, dtype=torch.uint8, device=dev)
        self.V_packed = torch.zeros(shape_kv, dtype=torch.uint8, device=dev)
        self.K_scale = torch.zeros(shape_kpage, dtype=meta_dtype, device=dev)
        self.K_mn = torch.zeros(shape_kpage, dtype=meta_dtype, device=dev)
        self.V_scale = torch.zeros(shape_vtok, dtype=meta_dtype, device=dev)
        self.V_mn = torch.zeros(shape_vtok, dtype=meta_dtype, device=dev)
        self.K_partial = torch.zeros(shape_partial, dtype=torch.bfloat16, device=dev)
        self.V_partial = torch.zeros(shape_partial, dtype=torch.bfloat16, device=dev)
        self._seen_tokens = [0] * num_layers
        self._desc = None
        if dev.type == "cuda" and page_size == 64 and head_dim in (64, 128) and G in (1, head_dim // 32):
            self._desc, _ = _ops.int4_cache(self.K_packed, self.K_scale, self.K_mn, self.V_packed, self.V_scale,
                                            self.V_mn, page_size)
            self._kpart_s = L.strides(self.K_partial, 5)
            self._vpart_s = L.strides(self.V_partial, 5)

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
        (persistent_int4.py:69-132)."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        S_new = K_new.shape[2]
        if seen + S_new > self.max_seq_len:
            raise RuntimeError(f"PersistentInt4KVCache: seen+new={seen + S_new} exceeds "
                               f"max_seq_len={self.max_seq_len}")
        if S_new == 0:
            return
        fast = (self._desc is not None and K_new.dtype == self.K_partial.dtype == V_new.dtype
                and K_new.shape == V_new.shape and K_new.stride(-1) == 1 and V_new.stride(-1) == 1
                and K_new.shape[0] == self._batch_size and K_new.shape[1] == self.num_kv_heads
                and K_new.shape[3] == self.head_dim)
        if fast:
            L.require_device(K_new, V_new, self.K_packed)
            L.check(L.lib().fq_int4_cache_append(
                self._desc, layer_idx, self.K_partial.data_ptr(), self._kpart_s, self.V_partial.data_ptr(),
                self._vpart_s, L.dtype_code(self.K_partial.dtype), K_new.data_ptr(), L.strides(K_new, 4),
                V_new.data_ptr(), L.strides(V_new, 4), seen, S_new, L.stream_handle(K_new.device)),
                "update_quantized")
        else:
            self._update_concat(K_new, V_new, layer_idx, seen, S_new)
        self._seen_tokens[layer_idx] = seen + S_new

    def _update_concat(self, K_new, V_new, layer_idx, seen, S_new):
        """The reference's sequence (persistent_int4.py:96-130) on the HIP quantisers."""
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
            tok0 = seen - partial_len
            p0 = tok0 // page_size
            lay = layer_idx
            quantize_k_int4(K_full[:, :, :complete_len], page_size,
                            out=(self.K_packed[lay, :, :, tok0:tok0 + complete_len],
                                 self.K_scale[lay, :, :, p0:p0 + n_complete],
                                 self.K_mn[lay, :, :, p0:p0 + n_complete]))
            quantize_v_int4(V_full[:, :, :complete_len], v_group=self.v_group,
                            out=(self.V_packed[lay, :, :, tok0:tok0 + complete_len],
                                 self.V_scale[lay, :, :, tok0:tok0 + complete_len],
                                 self.V_mn[lay, :, :, tok0:tok0 + complete_len]))
        rest = total - complete_len
        self.K_partial[layer_idx, :, :, :rest, :] = K_full[:, :, complete_len:, :]
        self.V_partial[layer_idx, :, :, :rest, :] = V_full[:, :, complete_len:, :]

    def get_views(self, layer_idx: int) -> dict:
        """persistent_int4.py:134-159: views up to the completed pages, plus the tail."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        partial_len = seen % self.page_size
        completed_len = seen - partial_len
        n_pages = completed_len // self.page_size
        return {
            "seq_len": seen,
            "completed_len": completed_len,
            "partial_len": partial_len,
            "K_packed": self.K_packed[layer_idx, :, :, :completed_len, :],
            "V_packed": self.V_packed[layer_idx, :, :, :completed_len, :],
            "K_scale": self.K_scale[layer_idx, :, :, :n_pages, :],
            "K_mn": self.K_mn[layer_idx, :, :, :n_pages, :],
            "V_scale": self.V_scale[layer_idx, :, :, :completed_len, :],
            "V_mn": self.V_mn[layer_idx, :, :, :completed_len, :],
            "K_partial": self.K_partial[layer_idx, :, :, :partial_len, :],
            "V_partial": self.V_partial[layer_idx, :, :, :partial_len, :],
        }

    def update(self, *args, **kwargs):
        """HF Cache.update is unused on the patched path (persistent_int4.py:161-166)."""
        raise NotImplementedError("PersistentInt4KVCache.update is not used; the patched forward "
                                  "calls update_quantized directly.")
