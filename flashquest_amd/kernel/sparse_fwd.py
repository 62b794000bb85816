"""flash_attn_sparse_fwd (INT8 KV) on the HIP split-K kernel.

Mirrors src/flashquest/kernel/sparse_fwd.py:160-228 (signature, shape checks,
exception types, outputs; kernel semantics 23-157: k = code * K_scale[p] +
K_mn[p], v = code * V_scale[t] + V_mn[t], base-2 online softmax, O = acc / l,
lse = (m + log2 l) * ln2, an empty selection gives O = 0 and lse = -inf).
Extensions: Q may also be fp16/fp32 (O takes Q's dtype) and the metadata may
be fp16.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops

_SUPPORTED_HEAD_DIMS = (64, 128)


def flash_attn_sparse_fwd(
    Q: torch.Tensor,
    K_uint8: torch.Tensor,
    K_scale: torch.Tensor,
    K_mn: torch.Tensor,
    V_uint8: torch.Tensor,
    V_scale: torch.Tensor,
    V_mn: torch.Tensor,
    *,
    selection_mask: torch.Tensor,
    page_size: int = 64,
    sm_scale: float | None = None,
    return_lse: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Decode-only sparse attention with INT8 KV (sparse_fwd.py:160-228).

    Args:
        Q: (B, H_q, 1, D).  K_uint8/V_uint8: (B, H_kv, S_kv, D) uint8.
        K_scale, K_mn: (B, H_kv, P, D).  V_scale, V_mn: (B, H_kv, S_kv, 1).
        selection_mask: (B, H_q, 1, P) bool, True = attend.
    Returns:
        (O (B, H_q, 1, D) in Q's dtype, lse (B, H_q, 1) fp32 or None).
    """
    L.require_device(Q, K_uint8, V_uint8, K_scale)
    assert Q.dtype in (torch.bfloat16, torch.float16, torch.float32)
    assert K_uint8.dtype == torch.uint8 and V_uint8.dtype == torch.uint8
    B, H_q, S_q, D = Q.shape
    if S_q != 1:
        raise NotImplementedError(
            f"flash_attn_sparse_fwd: decode-only (S_q={S_q}); use flash_attn_fwd for prefill.")
    if D not in _SUPPORTED_HEAD_DIMS:
        raise NotImplementedError(f"head_dim={D} not in {_SUPPORTED_HEAD_DIMS}")
    Bk, H_kv, S_kv, Dk = K_uint8.shape
    assert (B, D) == (Bk, Dk)
    assert H_q % H_kv == 0
    num_pages = K_scale.shape[2]
    assert selection_mask.shape == (B, H_q, 1, num_pages)
    assert selection_mask.dtype == torch.bool
    if _ops.wants_head_chunks(H_q, H_kv, D, page_size):      # more than 4 query heads per KV head
        return _ops.attend_in_head_chunks(
            Q, H_kv, selection_mask,
            lambda q, m: flash_attn_sparse_fwd(q, K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, selection_mask=m,
                                               page_size=page_size, sm_scale=sm_scale, return_lse=return_lse),
            return_lse)
    Q3 = Q[:, :, 0, :]
    O3 = torch.empty_like(Q3)
    lse = torch.empty(B, H_q, dtype=torch.float32, device=Q.device) if return_lse else None
    cache, keep = _ops.int8_cache(K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, page_size)
    query = _ops.query(Q3, O3, lse, sm_scale)
    ws = L.workspace(Q.device, L.lib().fq_int8_workspace_bytes(cache, H_q))
    mask3 = selection_mask[:, :, 0, :]
    L.check(L.lib().fq_sparse_int8_fwd_mask(cache, query, mask3.data_ptr(), L.strides(mask3, 4, 1),
                                            ws.data_ptr(), ws.numel(), L.stream_handle(Q.device)),
            "flash_attn_sparse_fwd")
    return O3.unsqueeze(2), (lse.unsqueeze(2) if lse is not None else None)
