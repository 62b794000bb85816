"""Bookkeeping shared by the three persistent caches (INT4, INT8, TurboQuant).

Each cache preallocates, per layer, the packed pages of its family for
``max_seq_len`` tokens and a bf16 partial-page tail of ``page_size`` rows; a
layer's token count decides which pages are complete.  Appends run on the GPU
through the family's C-ABI append (page completion straight from the tail and
the new tokens, then tail staging).  Geometries the append kernels do not take
(pages other than 64 tokens, head_dim other than 64 / 128) and new tokens in
another dtype than the tail assemble the token stream on the device and
quantise its completed pages with the family's operator-level quantisers
instead.
"""
from __future__ import annotations

import torch
from transformers.cache_utils import Cache

from .. import _lib as L


class PagedKVCache(Cache):
    """Sizes, token counts, the bf16 tails and the append protocol."""

    kv_bits = 0
    _name = "PagedKVCache"

    def _init_paged(self, batch_size, num_layers, num_kv_heads, head_dim, max_seq_len, page_size, device):
        # transformers' Cache keeps these; the patched decode path never fills them
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
        self.device = torch.device(device)
        tail = (num_layers, batch_size, num_kv_heads, page_size, head_dim)
        self.K_partial = torch.zeros(tail, dtype=torch.bfloat16, device=self.device)
        self.V_partial = torch.zeros(tail, dtype=torch.bfloat16, device=self.device)
        self._seen_tokens = [0] * num_layers
        # the append kernels: 64-token pages, 64 or 128 channels, on the GPU
        self._kernel_append = self.device.type == "cuda" and page_size == 64 and head_dim in (64, 128)
        if self._kernel_append:
            self._kpart_s = L.strides(self.K_partial, 5)
            self._vpart_s = L.strides(self.V_partial, 5)

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
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(f"{self._name}: layer_idx={layer_idx} is not one of its {self.num_layers} layers")

    def _counts(self, layer_idx: int):
        """(tokens, tokens in completed pages, tokens in the tail, completed pages)."""
        seen = self._seen_tokens[layer_idx]
        tail = seen % self.page_size
        return seen, seen - tail, tail, (seen - tail) // self.page_size

    def _tail_views(self, layer_idx: int) -> dict:
        seen, done, tail, _ = self._counts(layer_idx)
        return {"seq_len": seen, "completed_len": done, "partial_len": tail,
                "K_partial": self.K_partial[layer_idx, :, :, :tail, :],
                "V_partial": self.V_partial[layer_idx, :, :, :tail, :]}

    def update_quantized(self, K_new: torch.Tensor, V_new: torch.Tensor, layer_idx: int) -> None:
        """Append K_new, V_new (B, H_kv, S_new, D) to layer ``layer_idx``: the
        pages they complete are quantised into the cache, the remaining tokens
        wait in the layer's bf16 tail."""
        self._check_layer(layer_idx)
        seen = self._seen_tokens[layer_idx]
        if K_new.shape != V_new.shape or K_new.dim() != 4:
            raise ValueError(f"{self._name}: K_new / V_new must share one (B, H_kv, S_new, D) shape; "
                             f"got {tuple(K_new.shape)} and {tuple(V_new.shape)}")
        B, H, S_new, D = K_new.shape
        if (B, H, D) != (self._batch_size, self.num_kv_heads, self.head_dim):
            raise ValueError(f"{self._name}: appended tokens are {tuple(K_new.shape)}, the cache holds "
                             f"(B={self._batch_size}, H_kv={self.num_kv_heads}, D={self.head_dim})")
        if seen + S_new > self.max_seq_len:
            raise RuntimeError(f"{self._name}: {seen} cached + {S_new} new tokens exceeds max_seq_len="
                               f"{self.max_seq_len}")
        if S_new == 0:
            return
        if self._kernel_append and K_new.dtype == V_new.dtype == self.K_partial.dtype:
            L.require_device(K_new, V_new, self.K_partial)
            self._append_kernel(layer_idx, seen, _rows16(K_new), _rows16(V_new))
        else:
            self._append_stream(layer_idx, seen, K_new, V_new)
        self._seen_tokens[layer_idx] = seen + S_new

    def _append_stream(self, layer_idx, seen, K_new, V_new):
        """Other geometries, or new tokens in another dtype than the tail: the
        tail rows and the new tokens as one device stream (in the promoted
        dtype, whose arithmetic the quantisers then use, as the reference's
        concatenation does); its whole pages go through ``_quantize_pages`` at
        their cache position, the remainder becomes the tail."""
        P = self.page_size
        tail = seen % P
        stream_k = torch.cat([self.K_partial[layer_idx, :, :, :tail], K_new], dim=2)
        stream_v = torch.cat([self.V_partial[layer_idx, :, :, :tail], V_new], dim=2)
        whole = stream_k.shape[2] // P * P
        if whole:
            self._quantize_pages(layer_idx, seen - tail, stream_k[:, :, :whole], stream_v[:, :, :whole])
        left = stream_k.shape[2] - whole
        self.K_partial[layer_idx, :, :, :left] = stream_k[:, :, whole:]
        self.V_partial[layer_idx, :, :, :left] = stream_v[:, :, whole:]
        if self._zero_tail_after_append:
            self.K_partial[layer_idx, :, :, left:].zero_()
            self.V_partial[layer_idx, :, :, left:].zero_()

    _zero_tail_after_append = False

    def _append_kernel(self, layer_idx, seen, K_new, V_new):
        raise NotImplementedError

    def _quantize_pages(self, layer_idx, tok0, K_pages, V_pages):
        raise NotImplementedError

    def update(self, *args, **kwargs):
        """transformers' Cache.update: the patched attention appends with
        update_quantized and reads get_views instead."""
        raise NotImplementedError(f"{self._name}.update is not part of the packed-cache protocol; "
                                  "use update_quantized() and get_views()")


def _rows16(t: torch.Tensor) -> torch.Tensor:
    """Contiguous 16-byte aligned channel rows, as the append kernels read them."""
    es = t.element_size()
    if t.stride(-1) == 1 and all((s * es) % 16 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)
