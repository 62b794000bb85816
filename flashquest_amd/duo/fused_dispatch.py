"""DuoAttention decode in one call (src/flashquest/duo/fused_dispatch.py:19-78).

quest_duo_fused_sdpa keeps the reference's signature and its three steps over
the INT8 cache, each a HIP launch:

1. Quest scores from the exact page summary of the bf16-dequantised keys
   (dequantize_k -> compute_page_summary -> page_scores, fused_dispatch.py:
   64-67): ``page_scores_int8_summary``, one launch.
2. ``select_pages`` with the per-query-head retention vector: retrieval heads
   keep ``retention``, streaming heads 0, so they select exactly the sink and
   window pages (fused_dispatch.py:56-62, 69-72).
3. ``flash_attn_sparse_fwd`` over that mask (fused_dispatch.py:74-77).

(The decode step ``quest_decode_int8(..., head_pattern=...)`` is the faster
single-launch form of the same pattern; it scores from the page metadata, as
the reference's attention patch does.)
"""
from __future__ import annotations

import torch

from ..eager.criticality import page_scores_int8_summary
from ..eager.selection import select_pages
from ..kernel import flash_attn_sparse_fwd


def quest_duo_fused_sdpa(Q: torch.Tensor, K_uint8: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor,
                         V_uint8: torch.Tensor, V_scale: torch.Tensor, V_mn: torch.Tensor, *,
                         head_pattern: torch.Tensor, page_size: int = 64, retention: float = 0.20,
                         num_sinks: int = 4, window_pages: int = 2) -> torch.Tensor:
    """Q (B, H_q, 1, D); INT8 cache (B, H_kv, S, D) codes, (B, H_kv, P, D) K
    scale/min, (B, H_kv, S, 1) V scale/min; head_pattern (H_kv,) bool, True =
    retrieval.  Returns O (B, H_q, 1, D) in Q's dtype."""
    B, H_q, S_q, D = Q.shape
    if S_q != 1:
        raise NotImplementedError(f"quest_duo_fused_sdpa decodes one token per call (S_q={S_q})")
    H_kv = K_uint8.shape[1]
    if tuple(head_pattern.shape) != (H_kv,):
        raise ValueError(f"head_pattern needs one entry per KV head, shape ({H_kv},); "
                         f"got {tuple(head_pattern.shape)}")
    n_rep = H_q // H_kv
    per_q = head_pattern.bool().cpu().repeat_interleave(n_rep)
    r = torch.where(per_q, torch.full((H_q,), float(retention)), torch.zeros(H_q))
    scores = page_scores_int8_summary(Q, K_uint8, K_scale, K_mn, page_size)
    sel = select_pages(scores, r, num_sinks, window_pages)
    O, _ = flash_attn_sparse_fwd(Q, K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, selection_mask=sel,
                                 page_size=page_size, return_lse=False)
    return O
