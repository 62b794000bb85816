"""Causal prefill attention over the packed INT4 / INT8 cache, on HIP.

The reference runs prefill (S_q > 1) as dequantise the whole cache to bf16,
concatenate the bf16 partial page and call
F.scaled_dot_product_attention(is_causal=True, enable_gqa=True)
(src/flashquest/eager/llama_persistent_patch.py:196-201).  These operators
compute the same attention in one kernel that dequantises K/V tiles on the
fly (codes -> fp32 FMA -> bf16, as dequantize_k_int4 / dequantize_v_int4,
kernel/kv_quant.py:174-186, 208-215, and dequantize_k / dequantize_v,
64-100) and never writes the bf16 cache out.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops


def _prefill_call(fn_name: str, cache_desc, keep, q, K_tail, V_tail, causal_offset: int, sm_scale):
    L.require_device(q, *keep)
    if q.dim() != 4:
        raise ValueError(f"q must be (B, H_q, S_q, D); got {tuple(q.shape)}")
    B, H_q, S_q, D = q.shape
    qb = _ops._ensure_inner_contiguous(q.to(torch.bfloat16), 8)
    if cache_desc.B != B:
        raise ValueError(f"batch mismatch: q has {B}, cache has {cache_desc.B}")
    if D != cache_desc.D:
        raise ValueError(f"head_dim mismatch: q has {D}, the cache has {cache_desc.D}")
    tail = L.Tail()
    tails = ()
    if K_tail is not None and K_tail.shape[-2] > 0:
        L.require_device(K_tail, V_tail)
        if K_tail.shape != V_tail.shape:
            raise ValueError("K_tail and V_tail shapes differ")
        kt = _ops._ensure_inner_contiguous(K_tail.to(torch.bfloat16), 8)
        vt = _ops._ensure_inner_contiguous(V_tail.to(torch.bfloat16), 4)
        tail = L.Tail(kt.data_ptr(), L.strides(kt, 5, 1), vt.data_ptr(), L.strides(vt, 5, 1),
                      L.FQ_BF16, kt.shape[-2], kt.shape[-1])
        tails = (kt, vt)
    out = torch.empty(B, H_q, S_q, D, dtype=torch.bfloat16, device=q.device)
    pq = L.Prefill(qb.data_ptr(), L.strides(qb, 4), out.data_ptr(), L.strides(out, 4), H_q, S_q,
                   int(causal_offset), float(sm_scale) if sm_scale is not None else 0.0, D)
    if fn_name == "fq_prefill_turbo":
        nbytes = L.lib().fq_prefill_turbo_workspace_bytes(cache_desc, tail, pq)
    else:
        nbytes = L.lib().fq_prefill_workspace_bytes(cache_desc, tail, pq, 4 if fn_name.endswith("int4") else 8)
    # the dense bf16 K / V^T of the two-pass path: written in full before it is read
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    L.check(getattr(L.lib(), fn_name)(cache_desc, tail, pq, L.ptr(ws), nbytes, L.stream_handle(q.device)), fn_name)
    del tails
    return out


def flash_attn_prefill_int4(q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, K_tail=None, V_tail=None, *,
                            page_size: int = 64, causal_offset: int = 0, sm_scale: float | None = None):
    """Causal GQA attention of q (B, H_q, S_q, D) over one layer's packed INT4
    cache (B, H_kv, S, D/2) followed by the bf16 tail rows K_tail / V_tail
    (B, H_kv, T, D).  Query i attends keys j <= i + causal_offset
    (0 = torch's is_causal, as the reference's prefill call).  Returns bf16
    (B, H_q, S_q, D)."""
    K_packed = _ops._ensure_inner_contiguous(K_packed, 8)   # one thread loads 8 code bytes
    c, keep = _ops.int4_cache(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size)
    return _prefill_call("fq_prefill_int4", c, keep, q, K_tail, V_tail, causal_offset, sm_scale)


def flash_attn_prefill_int8(q, K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, K_tail=None, V_tail=None, *,
                            page_size: int = 64, causal_offset: int = 0, sm_scale: float | None = None):
    """flash_attn_prefill_int4 over the INT8 cache (one code byte per channel)."""
    K_uint8 = _ops._ensure_inner_contiguous(K_uint8, 16)
    c, keep = _ops.int8_cache(K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, page_size)
    return _prefill_call("fq_prefill_int8", c, keep, q, K_tail, V_tail, causal_offset, sm_scale)


def flash_attn_prefill_turbo(q, K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo, K_tail=None, V_tail=None,
                             *, page_size: int = 64, causal_offset: int = 0, sm_scale: float | None = None):
    """flash_attn_prefill_int4 over the TurboQuant K3-V3 cache: the planes are
    dequantised as dequantize_k_turbo / dequantize_v_turbo
    (kernel/kv_quant.py:366-420: codebook * scale, inverse WHT, bf16) once
    into dense bf16 K / V^T, then attended like the INT4 two-pass path."""
    S = K_msb.shape[-2]
    c, keep = _ops.turbo_cache(K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo,
                               (S + page_size - 1) // page_size, page_size)
    return _prefill_call("fq_prefill_turbo", c, keep, q, K_tail, V_tail, causal_offset, sm_scale)
