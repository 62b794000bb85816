"""flash_attn_sparse_int4_fwd on the HIP split-K kernel.

Mirrors src/flashquest/kernel/sparse_int4_fwd.py:160-248 (signature, shape
checks, exception types, outputs).  Extensions: Q may also be fp16/fp32 (the
output takes Q's dtype), metadata may be fp16, and V metadata may be grouped
per 32 channels ((B, H_kv, S, D/32) instead of (B, H_kv, S, 1)).
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import _ops

_SUPPORTED_HEAD_DIMS = (64, 128)


def _check_common(Q, K_packed, V_packed, K_scale):
    L.require_device(Q, K_packed, V_packed, K_scale)
    assert Q.dtype in (torch.bfloat16, torch.float16, torch.float32)
    assert K_packed.dtype == torch.uint8 and V_packed.dtype == torch.uint8
    B, H_q, S_q, D = Q.shape
    if S_q != 1:
        raise NotImplementedError(f"flash_attn_sparse_int4_fwd: decode-only (S_q={S_q})")
    if D not in _SUPPORTED_HEAD_DIMS:
        raise NotImplementedError(f"head_dim={D} not in {_SUPPORTED_HEAD_DIMS}")
    Bk, H_kv, S_kv, Dp = K_packed.shape
    assert B == Bk
    assert Dp == D // 2, f"K_packed last axis {Dp} != D/2={D // 2}"
    assert H_q % H_kv == 0
    return B, H_q, D, H_kv


def _run(fn, Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size, sm_scale, return_lse, *extra):
    B, H_q, _, D = Q.shape
    Q3 = Q[:, :, 0, :]
    O3 = torch.empty_like(Q3)
    lse = torch.empty(B, H_q, dtype=torch.float32, device=Q.device) if return_lse else None
    cache, keep = _ops.int4_cache(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size)
    query = _ops.query(Q3, O3, lse, sm_scale)
    nbytes = L.lib().fq_workspace_bytes(cache, H_q)
    ws = L.workspace(Q.device, nbytes)
    L.check(fn(cache, query, *extra, ws.data_ptr(), ws.numel(), L.stream_handle(Q.device)),
            "flash_attn_sparse_int4_fwd")
    return O3.unsqueeze(2), (lse.unsqueeze(2) if lse is not None else None)


def flash_attn_sparse_int4_fwd(
    Q: torch.Tensor,
    K_packed: torch.Tensor,
    K_scale: torch.Tensor,
    K_mn: torch.Tensor,
    V_packed: torch.Tensor,
    V_scale: torch.Tensor,
    V_mn: torch.Tensor,
    *,
    selection_mask: torch.Tensor,
    page_size: int = 64,
    sm_scale: float | None = None,
    return_lse: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Decode-only sparse attention over packed INT4 K/V (sparse_int4_fwd.py:160-248).

    Args:
        Q: (B, H_q, 1, D).  K_packed/V_packed: (B, H_kv, S_kv, D/2) uint8.
        K_scale, K_mn: (B, H_kv, P, D).  V_scale, V_mn: (B, H_kv, S_kv, 1 or D/32).
        selection_mask: (B, H_q, 1, P) bool, True = attend.
    Returns:
        (O (B, H_q, 1, D) in Q's dtype, lse (B, H_q, 1) fp32 or None).
    """
    B, H_q, D, H_kv = _check_common(Q, K_packed, V_packed, K_scale)
    num_pages = K_scale.shape[2]
    assert selection_mask.shape == (B, H_q, 1, num_pages)
    assert selection_mask.dtype == torch.bool
    if _ops.wants_head_chunks(H_q, H_kv, D, page_size):      # more than 4 query heads per KV head
        return _ops.attend_in_head_chunks(
            Q, H_kv, selection_mask,
            lambda q, m: flash_attn_sparse_int4_fwd(q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn,
                                                    selection_mask=m, page_size=page_size, sm_scale=sm_scale,
                                                    return_lse=return_lse), return_lse)
    mask3 = selection_mask[:, :, 0, :]
    return _run(L.lib().fq_sparse_int4_fwd_mask, Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn,
                page_size, sm_scale, return_lse, mask3.data_ptr(), L.strides(mask3, 4, 1))
