"""Quest page criticality from INT4 / INT8 K metadata on HIP.

Mirrors src/flashquest/eager/criticality.py:34-163.
"""
from __future__ import annotations

import torch

from .. import _lib as L


def page_scores_int4_fast(Q: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor) -> torch.Tensor:
    """scores[b, h_q, s, p] = Q.K_mn[p] + 15 * relu(Q).K_scale[p] in fp32, with
    query head h_q reading KV head h_q // (H_q / H_kv).

    The kernel's fp32 evaluation order is fixed (per lane a fused
    multiply-add chain over 8 channels, then a 16-lane butterfly), so the
    scores - and the page selection made from them - are reproducible.

    Args:
        Q: (B, H_q, S_q, D) bf16/fp16/fp32.  K_scale, K_mn: (B, H_kv, P, D) bf16/fp16.
    Returns:
        (B, H_q, S_q, P) fp32.
    """
    B, H_q, S_q, D = Q.shape
    H_kv, P = K_scale.shape[1], K_scale.shape[2]
    if H_q % H_kv != 0:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={H_kv}")
    L.require_device(Q, K_scale, K_mn)
    if K_scale.dtype != K_mn.dtype:
        raise AssertionError("K_scale and K_mn must share a dtype")
    ks = K_scale if K_scale.stride(-1) == 1 else K_scale.contiguous()
    km = K_mn if K_mn.stride(-1) == 1 else K_mn.contiguous()
    out = torch.empty(B, H_q, S_q, P, dtype=torch.float32, device=Q.device)
    L.check(L.lib().fq_page_scores_int4(
        Q.data_ptr(), L.dtype_code(Q.dtype), L.strides(Q, 4), ks.data_ptr(), L.strides(ks, 4),
        km.data_ptr(), L.strides(km, 4), L.dtype_code(ks.dtype), out.data_ptr(), L.strides(out, 4),
        B, H_q, S_q, H_kv, P, D, L.stream_handle(Q.device)), "page_scores_int4_fast")
    return out


def page_scores_int8_fast(Q: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor) -> torch.Tensor:
    """criticality.py:77-125: scores = Q.K_mn[p] + 255 * relu(Q).K_scale[p] in
    fp32 (the INT8 metadata's code range), in the same fixed order as
    page_scores_int4_fast.  Q (B, H_q, S_q, D); K_scale, K_mn (B, H_kv, P, D).
    Returns (B, H_q, S_q, P) fp32."""
    B, H_q, S_q, D = Q.shape
    H_kv, P = K_scale.shape[1], K_scale.shape[2]
    if H_q % H_kv != 0:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={H_kv}")
    L.require_device(Q, K_scale, K_mn)
    if K_scale.dtype != K_mn.dtype:
        raise AssertionError("K_scale and K_mn must share a dtype")
    ks = K_scale if K_scale.stride(-1) == 1 else K_scale.contiguous()
    km = K_mn if K_mn.stride(-1) == 1 else K_mn.contiguous()
    out = torch.empty(B, H_q, S_q, P, dtype=torch.float32, device=Q.device)
    L.check(L.lib().fq_page_scores_int8(
        Q.data_ptr(), L.dtype_code(Q.dtype), L.strides(Q, 4), ks.data_ptr(), L.strides(ks, 4),
        km.data_ptr(), L.strides(km, 4), L.dtype_code(ks.dtype), out.data_ptr(), L.strides(out, 4),
        B, H_q, S_q, H_kv, P, D, L.stream_handle(Q.device)), "page_scores_int8_fast")
    return out


def page_scores_int8(Q: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor) -> torch.Tensor:
    """criticality.py:34-74: the Quest bound from the INT8 page range,
    sum_d max(Q_d * K_mn, Q_d * (K_mn + 255 * K_scale)) in fp32; equal to
    page_scores_int8_fast in exact arithmetic."""
    return page_scores_int8_fast(Q, K_scale, K_mn)
