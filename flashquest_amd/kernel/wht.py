"""Normalised Walsh-Hadamard transform on HIP (src/flashquest/kernel/wht.py:17-41)."""
from __future__ import annotations

import torch

from .. import _lib as L


def wht_along_head_dim(x: torch.Tensor, *, signs: torch.Tensor | None = None,
                       inverse: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """WHT along the last axis (power of two, <= 128); self-inverse.

    Like the reference, each butterfly stage is rounded to x's dtype.
    ``signs`` (D,) fp32 gives the randomised transform WHT(signs * x), and
    with ``inverse=True`` its inverse signs * WHT(x).  ``out`` (contiguous,
    x's shape and dtype) receives the result instead of a new tensor.
    """
    D = x.shape[-1]
    if D == 0 or D & (D - 1) != 0:
        raise ValueError(f"head_dim must be a positive power of 2, got {D}")
    L.require_device(x)
    xc = x.contiguous()
    if out is None:
        out = torch.empty_like(xc)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous() or out.device != x.device:
        raise ValueError("out must be a contiguous tensor of x's shape, dtype and device")
    N = xc.numel() // D
    sp = None
    if signs is not None:
        signs = signs.to(device=x.device, dtype=torch.float32).contiguous()
        sp = signs.data_ptr()
    L.check(L.lib().fq_wht(xc.data_ptr(), L.dtype_code(xc.dtype), D, out.data_ptr(), L.dtype_code(out.dtype), D,
                           N, D, sp, int(inverse), L.dtype_code(xc.dtype), L.stream_handle(x.device)),
            "wht_along_head_dim")
    return out
