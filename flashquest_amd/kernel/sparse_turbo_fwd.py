"""flash_attn_sparse_turbo_fwd on the HIP split-K turbo kernel.

Mirrors src/flashquest/kernel/sparse_turbo_fwd.py:254-346.  The Q rotation
and the inverse rotation of O run inside the kernel (in fp32) instead of as
separate bf16 tensor ops around it.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops

_SUPPORTED_HEAD_DIMS = (64, 128)


def flash_attn_sparse_turbo_fwd(
    Q: torch.Tensor,
    K_msb: torch.Tensor,
    K_lsb: torch.Tensor,
    K_scale_turbo: torch.Tensor,
    V_msb: torch.Tensor,
    V_lsb: torch.Tensor,
    V_scale_turbo: torch.Tensor,
    *,
    selection_mask: torch.Tensor,
    page_size: int = 64,
    sm_scale: float | None = None,
    return_lse: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Q (B,H_q,1,D) raw basis; planes (B,H_kv,S,D/8), (B,H_kv,S,D/4) u8;
    scales (B,H_kv,S,1) bf16; selection_mask (B,H_q,1,P) bool.  Returns
    (O (B,H_q,1,D) raw basis, lse (B,H_q,1) fp32 or None)."""
    L.require_device(Q, K_msb, K_lsb, V_msb, V_lsb)
    assert Q.dtype in (torch.bfloat16, torch.float16, torch.float32)
    assert K_msb.dtype == torch.uint8 and K_lsb.dtype == torch.uint8
    assert V_msb.dtype == torch.uint8 and V_lsb.dtype == torch.uint8
    B, H_q, S_q, D = Q.shape
    if S_q != 1:
        raise NotImplementedError(f"flash_attn_sparse_turbo_fwd: decode-only (S_q={S_q})")
    if D not in _SUPPORTED_HEAD_DIMS:
        raise NotImplementedError(f"head_dim={D} not in {_SUPPORTED_HEAD_DIMS}")
    Bk, H_kv, S_kv, _ = K_msb.shape
    assert B == Bk
    assert H_q % H_kv == 0
    num_pages = selection_mask.shape[-1]
    assert selection_mask.shape == (B, H_q, 1, num_pages)
    assert selection_mask.dtype == torch.bool
    assert K_scale_turbo.dtype == torch.bfloat16 and V_scale_turbo.dtype == torch.bfloat16
    if _ops.wants_head_chunks(H_q, H_kv, D, page_size):      # more than 4 query heads per KV head
        return _ops.attend_in_head_chunks(
            Q, H_kv, selection_mask,
            lambda q, m: flash_attn_sparse_turbo_fwd(q, K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo,
                                                     selection_mask=m, page_size=page_size, sm_scale=sm_scale,
                                                     return_lse=return_lse), return_lse)

    Q3 = Q[:, :, 0, :]
    O3 = torch.empty_like(Q3)
    lse = torch.empty(B, H_q, dtype=torch.float32, device=Q.device) if return_lse else None
    cache, keep = _ops.turbo_cache(K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo, num_pages, page_size)
    query = _ops.query(Q3, O3, lse, sm_scale)
    mask3 = selection_mask[:, :, 0, :]
    ws = L.workspace(Q.device, L.lib().fq_turbo_workspace_bytes(cache, H_q))
    L.check(L.lib().fq_sparse_turbo_fwd_mask(cache, query, mask3.data_ptr(), L.strides(mask3, 4, 1),
                                             ws.data_ptr(), ws.numel(), L.stream_handle(Q.device)),
            "flash_attn_sparse_turbo_fwd")
    return O3.unsqueeze(2), (lse.unsqueeze(2) if lse is not None else None)
