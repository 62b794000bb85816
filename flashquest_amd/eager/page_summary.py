"""Per-page channel min / max of K on HIP (src/flashquest/eager/page_summary.py:7-39)."""
from __future__ import annotations

import torch

from .. import _lib as L


def compute_page_summary(K: torch.Tensor, page_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(page_min, page_max), each (B, H, ceil(S / page_size), D) in K's dtype:
    per page and channel the minimum and maximum of K (B, H, S, D) over the
    page's tokens; a partial last page summarises only its valid tokens.
    NaN propagates as in torch's min / max."""
    assert page_size > 0
    B, H, S, D = K.shape
    L.require_device(K)
    P = (S + page_size - 1) // page_size
    pmin = torch.empty(B, H, P, D, dtype=K.dtype, device=K.device)
    pmax = torch.empty_like(pmin)
    L.check(L.lib().fq_page_summary(K.data_ptr(), L.dtype_code(K.dtype), L.strides(K, 4), B, H, S, D, int(page_size),
                                    pmin.data_ptr(), pmax.data_ptr(), L.strides(pmin, 4),
                                    L.stream_handle(K.device)), "compute_page_summary")
    return pmin, pmax
