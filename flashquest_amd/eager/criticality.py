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


def page_scores(Q: torch.Tensor, page_min: torch.Tensor, page_max: torch.Tensor) -> torch.Tensor:
    """criticality.py:7-31: scores[b, h, s, p] = sum_d max(Q_d * max_d, Q_d * min_d)
    in fp32 (a fixed order: 4 channels per lane left to right, then a
    butterfly over the D/4 partial sums).

    Args:
        Q: (B, H, S_q, D) bf16/fp16/fp32.  page_min, page_max: (B, H_b, P, D)
        with H_b = H (the reference's one summary row per head) or any H_b
        dividing H (query head h reads row h // (H / H_b)).
    Returns:
        (B, H, S_q, P) fp32.
    """
    B, H, S_q, D = Q.shape
    H_b, P = page_min.shape[1], page_min.shape[2]
    if page_max.shape != page_min.shape:
        raise ValueError(f"page_min {tuple(page_min.shape)} and page_max {tuple(page_max.shape)} differ")
    if H % H_b != 0:
        raise ValueError(f"H={H} must be divisible by the summaries' {H_b} heads")
    L.require_device(Q, page_min, page_max)
    lo, hi = page_min, page_max
    if hi.dtype != lo.dtype:
        hi = hi.to(lo.dtype)
    out = torch.empty(B, H, S_q, P, dtype=torch.float32, device=Q.device)
    L.check(L.lib().fq_page_scores_quest(
        Q.data_ptr(), L.dtype_code(Q.dtype), L.strides(Q, 4), lo.data_ptr(), L.strides(lo, 4), hi.data_ptr(),
        L.strides(hi, 4), L.dtype_code(lo.dtype), out.data_ptr(), L.strides(out, 4), B, H, S_q, H_b, P, D,
        L.stream_handle(Q.device)), "page_scores")
    return out


def page_scores_int8(Q: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor) -> torch.Tensor:
    """criticality.py:34-74: the Quest bound from the INT8 page range,
    sum_d max(Q_d * K_mn, Q_d * (K_mn + 255 * K_scale)) in fp32 with the
    reference's bounds (fp32(K_mn) and fp32(K_mn) + 255 * fp32(K_scale));
    equal to page_scores_int8_fast in exact arithmetic, and (unlike it) to
    the reference's per-term rounding.  Q (B, H_q, S_q, D); K_scale, K_mn
    (B, H_kv, P, D) bf16/fp16.  Returns (B, H_q, S_q, P) fp32."""
    B, H_q, S_q, D = Q.shape
    H_kv, P = K_scale.shape[1], K_scale.shape[2]
    if H_q % H_kv != 0:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={H_kv}")
    L.require_device(Q, K_scale, K_mn)
    if K_scale.dtype != K_mn.dtype:
        raise AssertionError("K_scale and K_mn must share a dtype")
    out = torch.empty(B, H_q, S_q, P, dtype=torch.float32, device=Q.device)
    L.check(L.lib().fq_page_scores_int8_bound(
        Q.data_ptr(), L.dtype_code(Q.dtype), L.strides(Q, 4), K_scale.data_ptr(), L.strides(K_scale, 4),
        K_mn.data_ptr(), L.strides(K_mn, 4), L.dtype_code(K_scale.dtype), out.data_ptr(), L.strides(out, 4),
        B, H_q, S_q, H_kv, P, D, L.stream_handle(Q.device)), "page_scores_int8")
    return out


def page_scores_int8_summary(Q: torch.Tensor, K_uint8: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor,
                             page_size: int = 64, return_summary: bool = False):
    """The Quest scores of the reference's DuoAttention dispatch
    (duo/fused_dispatch.py:64-67) in one launch: the INT8 keys dequantised to
    bf16 (kv_quant.py:64-75), their per-page per-channel min / max over the
    page's valid tokens (page_summary.py:7-39), and
    sum_d max(Q_d * max_d, Q_d * min_d) in fp32 (criticality.py:7-31), query
    head h_q reading KV head h_q // (H_q / H_kv).

    Args:
        Q: (B, H_q, 1, D) bf16/fp16/fp32.  K_uint8: (B, H_kv, S, D) uint8.
        K_scale, K_mn: (B, H_kv, ceil(S / page_size), D) bf16/fp16.
    Returns:
        (B, H_q, 1, P) fp32 scores; with return_summary also the bf16
        (page_min, page_max), each (B, H_kv, P, D).
    """
    B, H_q, S_q, D = Q.shape
    if S_q != 1:
        raise NotImplementedError(f"page summary scores take one decode query per head (S_q={S_q})")
    H_kv, S = K_uint8.shape[1], K_uint8.shape[2]
    P = K_scale.shape[2]
    if H_q % H_kv != 0:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={H_kv}")
    L.require_device(Q, K_uint8, K_scale, K_mn)
    if K_uint8.dtype != torch.uint8:
        raise AssertionError("K_uint8 must be uint8")
    if K_scale.dtype != K_mn.dtype:
        raise AssertionError("K_scale and K_mn must share a dtype")
    kc = K_uint8
    if kc.stride(-1) != 1 or any(st % 4 for st in kc.stride()[:-1]) or kc.data_ptr() % 4:
        kc = kc.contiguous()
    out = torch.empty(B, H_q, 1, P, dtype=torch.float32, device=Q.device)
    pmin = pmax = None
    if return_summary:
        pmin = torch.empty(B, H_kv, P, D, dtype=torch.bfloat16, device=Q.device)
        pmax = torch.empty_like(pmin)
    z4 = L.i64([0, 0, 0, 0], 4)
    L.check(L.lib().fq_page_scores_int8_summary(
        Q.data_ptr(), L.dtype_code(Q.dtype), L.strides(Q, 4), kc.data_ptr(), L.strides(kc, 4),
        K_scale.data_ptr(), L.strides(K_scale, 4), K_mn.data_ptr(), L.strides(K_mn, 4), L.dtype_code(K_scale.dtype),
        pmin.data_ptr() if pmin is not None else None, pmax.data_ptr() if pmax is not None else None,
        L.strides(pmin, 4) if pmin is not None else z4, out.data_ptr(), L.strides(out, 4),
        B, H_q, H_kv, S, P, D, int(page_size), L.stream_handle(Q.device)), "page_scores_int8_summary")
    return (out, pmin, pmax) if return_summary else out
