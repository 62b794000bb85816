"""flash_attn_sparse_int4_fwd_compact on the HIP split-K kernel.

Mirrors src/flashquest/kernel/sparse_int4_fwd_compact.py:153-244: the page
selection is a per-query-head int32 id list with -1 sentinels.  Ids outside
[0, P) are skipped like the sentinel; a page listed twice for one head counts
once (lists from build_compact_selection never repeat a page).
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops
from .sparse_int4_fwd import _check_common, _run


def flash_attn_sparse_int4_fwd_compact(
    Q: torch.Tensor,
    K_packed: torch.Tensor,
    K_scale: torch.Tensor,
    K_mn: torch.Tensor,
    V_packed: torch.Tensor,
    V_scale: torch.Tensor,
    V_mn: torch.Tensor,
    *,
    selected_page_ids: torch.Tensor,
    page_size: int = 64,
    sm_scale: float | None = None,
    return_lse: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """selected_page_ids: (B, H_q, 1, BUCKET_MAX) or (B, H_q, BUCKET_MAX) int32."""
    assert selected_page_ids.dtype == torch.int32
    B, H_q, D, H_kv = _check_common(Q, K_packed, V_packed, K_scale)
    if selected_page_ids.dim() == 4:
        sel = selected_page_ids[:, :, 0, :]
    elif selected_page_ids.dim() == 3:
        sel = selected_page_ids
    else:
        raise ValueError(f"selected_page_ids must be 3D or 4D; got {selected_page_ids.dim()}D")
    Bs, H_qs, bucket = sel.shape
    assert Bs == B and H_qs == H_q
    L.require_device(sel)
    if _ops.wants_head_chunks(H_q, H_kv, D, page_size):      # more than 4 query heads per KV head
        return _ops.attend_in_head_chunks(
            Q, H_kv, sel,
            lambda q, ids: flash_attn_sparse_int4_fwd_compact(q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn,
                                                              selected_page_ids=ids, page_size=page_size,
                                                              sm_scale=sm_scale, return_lse=return_lse), return_lse)
    return _run(L.lib().fq_sparse_int4_fwd_ids, Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn,
                page_size, sm_scale, return_lse, sel.data_ptr(), L.strides(sel, 4, 1), bucket)
