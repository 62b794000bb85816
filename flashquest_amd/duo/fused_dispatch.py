"""DuoAttention decode in one fused call (src/flashquest/duo/fused_dispatch.py:19-78).

quest_duo_fused_sdpa keeps the reference's signature over the INT8 cache:
streaming KV heads get retention 0, so their query heads keep exactly the
sink and window pages, retrieval heads the top ``retention`` share of their
pages; scoring, selection and attention then run as one HIP decode step
(quest_decode_int8, per-query-head selection).

Scoring: the reference's helper scores from the dequantised keys' exact page
minimum / maximum (page_summary + page_scores); its attention patch, which
this build follows, scores from the page metadata (min = K_mn, max = K_mn +
255 K_scale; _criticality_scores, llama_persistent_patch.py:152-153 with
criticality.py:98-125).  The two bounds agree where a page channel's codes
reach 0 and 255; the quantiser maps the channel minimum to code 0 and the
maximum to 255 up to the rounding of the half-precision scale, so the
selections can differ only on pages whose scores fall within that rounding of
the k-th score.
"""
from __future__ import annotations

import torch

from ..eager.decode import quest_decode_int8


def quest_duo_fused_sdpa(Q: torch.Tensor, K_uint8: torch.Tensor, K_scale: torch.Tensor, K_mn: torch.Tensor,
                         V_uint8: torch.Tensor, V_scale: torch.Tensor, V_mn: torch.Tensor, *,
                         head_pattern: torch.Tensor, page_size: int = 64, retention: float = 0.20,
                         num_sinks: int = 4, window_pages: int = 2) -> torch.Tensor:
    """Q (B, H_q, 1, D); INT8 cache (B, H_kv, S, D) codes, (B, H_kv, P, D) K
    scale/min, (B, H_kv, S, 1) V scale/min; head_pattern (H_kv,) bool, True =
    retrieval.  Returns O (B, H_q, 1, D) in Q's dtype."""
    if Q.shape[2] != 1:
        raise NotImplementedError(f"quest_duo_fused_sdpa decodes one token per call (S_q={Q.shape[2]})")
    H_kv = K_uint8.shape[1]
    if tuple(head_pattern.shape) != (H_kv,):
        raise ValueError(f"head_pattern needs one entry per KV head, shape ({H_kv},); "
                         f"got {tuple(head_pattern.shape)}")
    O, _ = quest_decode_int8(Q, K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, retention=float(retention),
                             num_sinks=num_sinks, window_pages=window_pages, page_size=page_size,
                             select_mode="per_q_head", return_lse=False, head_pattern=head_pattern.bool())
    return O
