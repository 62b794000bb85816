"""Top-k page selection and compact id lists on HIP.

Mirrors src/flashquest/eager/selection.py:65-164.  Top-k is a workgroup
radix select over the fp32 scores; equal scores go to the lower page index.
"""
from __future__ import annotations

import math

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
    """selection.py:9-62, the per-head loop form.  Its k differs from the
    vectorized form's: each head's fp32 retention is read back to the host
    (``.item()``, a double) and k = ceil(r * P) is taken in double precision
    (r >= 1: every page, r <= 0: none), where select_pages_vectorized rounds
    r * P to fp32 first (selection.py:103).  The two differ when fp32(r * P)
    rounds onto an integer that the double product exceeds.  Like the
    reference, this reads the retention on the host; each head's k is then
    passed to the selection kernel as the retention fp32((k - 1/2) / P), whose
    fp32 ceil(r * P) is exactly k."""
    B, H, S_q, P = scores.shape
    if isinstance(retention, torch.Tensor):
        if retention.shape != (H,):
            raise ValueError(f"per-head retention must be shape ({H},); got {tuple(retention.shape)}")
        r_host = retention.detach().float().cpu().tolist()
    else:
        if not (0.0 <= float(retention) <= 1.0):
            raise ValueError(f"scalar retention must be in [0, 1]; got {retention}")
        r_host = [float(torch.tensor(float(retention), dtype=torch.float32))] * H
    adj = []
    for r in r_host:
        if r >= 1.0:
            adj.append(1.0)
        elif r <= 0.0:
            adj.append(0.0)
        else:
            k = min(math.ceil(r * P), P)
            adj.append(1.0 if k >= P else (k - 0.5) / P)
    r_dev = torch.tensor(adj, dtype=torch.float32).to(scores.device)
    return select_pages_vectorized(scores, r_dev, num_sinks, window_pages)


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
