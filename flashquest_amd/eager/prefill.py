"""The prefill branch of the reference's attention patch, on HIP.

Mirrors the S_q > 1 branch of make_quest_persistent_forward
(src/flashquest/eager/llama_persistent_patch.py:196-201): after
update_quantized has written the prompt chunk into the cache, attend q over
cat(dequantised completed pages, bf16 partial page) with torch's is_causal
mask and GQA.  Here the dequantisation happens inside the attention kernel.
"""
from __future__ import annotations

import torch

from ..kernel.prefill import flash_attn_prefill_int4, flash_attn_prefill_int8, flash_attn_prefill_turbo


def prefill_attention_layer(q: torch.Tensor, views: dict, *, page_size: int, causal_offset: int = 0,
                            sm_scale: float | None = None) -> torch.Tensor:
    """llama_persistent_patch.py:196-201 for one layer.

    ``views`` is get_views(layer) of a persistent INT4, INT8 or TurboQuant
    cache (persistent_int4.py:134-159, persistent_int8.py:137-169,
    persistent_turbo.py:149-176), told apart by its keys; q is
    (B, H_q, S_q, D).  causal_offset 0 is the reference's is_causal=True
    (query i attends keys j <= i, upper-left aligned when S_q < S_kv).
    Returns (B, H_q, S_q, D) in q's dtype.
    """
    kw = dict(page_size=page_size, causal_offset=causal_offset, sm_scale=sm_scale)
    if "K_msb" in views:
        out = flash_attn_prefill_turbo(q, views["K_msb"], views["K_lsb"], views["K_scale_turbo"], views["V_msb"],
                                       views["V_lsb"], views["V_scale_turbo"], views["K_partial"], views["V_partial"],
                                       **kw)
    elif "K_uint8" in views:
        out = flash_attn_prefill_int8(q, views["K_uint8"], views["K_scale"], views["K_mn"], views["V_uint8"],
                                      views["V_scale"], views["V_mn"], views["K_partial"], views["V_partial"], **kw)
    else:
        out = flash_attn_prefill_int4(q, views["K_packed"], views["K_scale"], views["K_mn"], views["V_packed"],
                                      views["V_scale"], views["V_mn"], views["K_partial"], views["V_partial"], **kw)
    return out.to(q.dtype)
