"""Top-k page selection and compact id lists on HIP.

Mirrors src/flashquest/eager/selection.py:65-164.  Top-k is a workgroup
radix select over the fp32 scores; equal scores go to the lower page index.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops


def select_pages_vectorized(
    scores: torch.Tensor,
    retention: float | torch.Tensor,
    num_sinks: int,
    window_pages: int,
    *,
    k_max_static: int | None = None,
) -> torch.Tensor:
    """(B, H, S_q, P) scores -> bool mask: per head the top
    k_h = ceil(fp32(r_h) * P) pages (at most k_max_static), plus the first
    ``num_sinks`` and last ``window_pages`` pages."""
    B, H, S_q, P = scores.shape
    L.require_device(scores)
    r = _ops.retention_tensor(retention, H, scores.device)
    sc = scores if scores.dtype == torch.float32 else scores.float()
    mask = torch.empty(B, H, S_q, P, dtype=torch.bool, device=scores.device)
    k_max = -1 if k_max_static is None else min(int(k_max_static), P)
    L.check(L.lib().fq_select_pages(sc.data_ptr(), L.strides(sc, 4), B, H, S_q, P, r.data_ptr(),
                                    int(num_sinks), int(window_pages), k_max, mask.data_ptr(),
                                    L.strides(mask, 4), L.stream_handle(scores.device)),
            "select_pages_vectorized")
    return mask


def select_pages(scores, retention, num_sinks: int, window_pages: int) -> torch.Tensor:
    """selection.py:9-62 (the per-head loop form); same result as the vectorized form."""
    return select_pages_vectorized(scores, retention, num_sinks, window_pages)


def build_compact_selection(mask: torch.Tensor, BUCKET_MAX: int) -> torch.Tensor:
    """(B, H, S_q, P) bool -> (B, H, S_q, BUCKET_MAX) int32: selected ids in
    descending order, then -1 (selection.py:129-164)."""
    if BUCKET_MAX < 1:
        raise ValueError(f"BUCKET_MAX must be >= 1, got {BUCKET_MAX}")
    if mask.dtype != torch.bool:
        raise ValueError(f"mask must be bool, got {mask.dtype}")
    L.require_device(mask)
    B, H, S_q, P = mask.shape
    out = torch.empty(B, H, S_q, BUCKET_MAX, dtype=torch.int32, device=mask.device)
    L.check(L.lib().fq_compact_ids(mask.data_ptr(), L.strides(mask, 4), B, H, S_q, P, BUCKET_MAX,
                                   out.data_ptr(), L.stream_handle(mask.device)), "build_compact_selection")
    return out
