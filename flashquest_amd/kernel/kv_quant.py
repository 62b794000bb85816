"""KV quantisers on HIP kernels.

Mirrors src/flashquest/kernel/kv_quant.py: INT8 (18-100: quantize_k /
quantize_v, 255 levels, one code byte per channel), INT4 (104-215) and
TurboQuant K3-V3 (225-420).  Codes and metadata are bit-exact with the reference's CUDA
semantics: K scale arithmetic in the input dtype ((max - min) and "/ 15.0",
the latter as a multiply by fp32(1/15) the way torch's CUDA division by a
Python scalar does), codes by IEEE fp32 division, round-half-even, clamp
0..15; V in fp32.  Extension: ``meta_dtype`` (bf16, the reference, or fp16)
and ``v_group`` (None = per token over all D, the reference; 32 = per token
and 32-channel group).
"""
from __future__ import annotations

import torch

from .. import _lib as L

# kv_quant.py:225-230 (identical K and V codebooks, K3-V3)
K_TURBO_CODEBOOK = torch.tensor(
    [-2.1519, -1.3439, -0.7560, -0.2451, 0.2451, 0.7560, 1.3439, 2.1519], dtype=torch.float32)
V_TURBO_CODEBOOK = K_TURBO_CODEBOOK.clone()


def quantize_k(K: torch.Tensor, page_size: int, *, meta_dtype: torch.dtype = torch.bfloat16, out=None):
    """kv_quant.py:43-61.  K (B, H, S, D) -> (K_uint8 (B,H,S,D) u8, scale
    (B,H,P,D), mn (B,H,P,D)) with P = ceil(S / page_size); scale/min arithmetic
    in K's dtype ("/ 255.0"), codes by fp32 division, round half even, clamp
    0..255, metadata stored as ``meta_dtype`` (bf16 in the reference)."""
    L.require_device(K)
    B, H, S, D = K.shape
    if D % 2 != 0:
        raise ValueError(f"quantize_k requires even head_dim; got {D}")
    P = (S + page_size - 1) // page_size
    if out is None:
        codes = torch.empty(B, H, S, D, dtype=torch.uint8, device=K.device)
        scale = torch.empty(B, H, P, D, dtype=meta_dtype, device=K.device)
        mn = torch.empty(B, H, P, D, dtype=meta_dtype, device=K.device)
    else:
        codes, scale, mn = out
    L.check(L.lib().fq_quantize_k_int8(
        K.data_ptr(), L.dtype_code(K.dtype), L.strides(K, 4), B, H, S, D, page_size,
        codes.data_ptr(), L.strides(codes, 4), scale.data_ptr(), L.strides(scale, 4),
        mn.data_ptr(), L.strides(mn, 4), L.dtype_code(scale.dtype), L.stream_handle(K.device)), "quantize_k")
    return codes, scale, mn


def quantize_v(V: torch.Tensor, *, meta_dtype: torch.dtype = torch.bfloat16, out=None):
    """kv_quant.py:78-89.  V (B, H, S, D) -> (V_uint8 (B,H,S,D) u8, scale
    (B,H,S,1), mn (B,H,S,1)), per token over all D in fp32."""
    L.require_device(V)
    B, H, S, D = V.shape
    if D % 2 != 0:
        raise ValueError(f"quantize_v requires even head_dim; got {D}")
    if out is None:
        codes = torch.empty(B, H, S, D, dtype=torch.uint8, device=V.device)
        scale = torch.empty(B, H, S, 1, dtype=meta_dtype, device=V.device)
        mn = torch.empty(B, H, S, 1, dtype=meta_dtype, device=V.device)
    else:
        codes, scale, mn = out
    L.check(L.lib().fq_quantize_v_int8(
        V.data_ptr(), L.dtype_code(V.dtype), L.strides(V, 4), B, H, S, D,
        codes.data_ptr(), L.strides(codes, 4), scale.data_ptr(), L.strides(scale, 4),
        mn.data_ptr(), L.strides(mn, 4), L.dtype_code(scale.dtype), L.stream_handle(V.device)), "quantize_v")
    return codes, scale, mn


def dequantize_k(K_uint8: torch.Tensor, scale: torch.Tensor, mn: torch.Tensor, page_size: int) -> torch.Tensor:
    """kv_quant.py:64-75 (tensor ops; prefill / test helper, not the decode path).  Returns bf16."""
    S = K_uint8.shape[2]
    s = scale.repeat_interleave(page_size, dim=2)[:, :, :S, :]
    m = mn.repeat_interleave(page_size, dim=2)[:, :, :S, :]
    return (K_uint8.to(torch.float32) * s.float() + m.float()).to(torch.bfloat16)


def dequantize_v(V_uint8: torch.Tensor, scale: torch.Tensor, mn: torch.Tensor) -> torch.Tensor:
    """kv_quant.py:92-97 (tensor ops).  Returns bf16."""
    return (V_uint8.to(torch.float32) * scale.float() + mn.float()).to(torch.bfloat16)


def _pack_int4(x: torch.Tensor) -> torch.Tensor:
    """kv_quant.py:104-115 (tensor op, any device)."""
    if x.shape[-1] % 2 != 0:
        raise ValueError(f"_pack_int4 requires even last axis; got {x.shape[-1]}")
    lo = x[..., 0::2] & 0x0F
    hi = x[..., 1::2] & 0x0F
    return (lo | (hi << 4)).to(torch.uint8)


def _unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """kv_quant.py:118-128."""
    out = torch.empty(*packed.shape[:-1], packed.shape[-1] * 2, dtype=torch.uint8, device=packed.device)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = (packed >> 4) & 0x0F
    return out


def quantize_k_int4(K: torch.Tensor, page_size: int, *, meta_dtype: torch.dtype = torch.bfloat16,
                    out=None):
    """kv_quant.py:152-171.  K (B, H, S, D) -> (K_packed (B,H,S,D/2) u8,
    scale (B,H,P,D), mn (B,H,P,D)) with P = ceil(S / page_size).

    ``out`` = (packed, scale, mn) writes into existing (possibly strided) views.
    """
    L.require_device(K)
    B, H, S, D = K.shape
    if D % 2 != 0:
        raise ValueError(f"quantize_k_int4 requires even head_dim; got {D}")
    P = (S + page_size - 1) // page_size
    if out is None:
        packed = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=K.device)
        scale = torch.empty(B, H, P, D, dtype=meta_dtype, device=K.device)
        mn = torch.empty(B, H, P, D, dtype=meta_dtype, device=K.device)
    else:
        packed, scale, mn = out
    L.check(L.lib().fq_quantize_k_int4(
        K.data_ptr(), L.dtype_code(K.dtype), L.strides(K, 4), B, H, S, D, page_size,
        packed.data_ptr(), L.strides(packed, 4), scale.data_ptr(), L.strides(scale, 4),
        mn.data_ptr(), L.strides(mn, 4), L.dtype_code(scale.dtype), L.stream_handle(K.device)),
        "quantize_k_int4")
    return packed, scale, mn


def quantize_v_int4(V: torch.Tensor, *, v_group: int | None = None,
                    meta_dtype: torch.dtype = torch.bfloat16, out=None):
    """kv_quant.py:189-205.  V (B, H, S, D) -> (V_packed (B,H,S,D/2) u8,
    scale (B,H,S,G), mn (B,H,S,G)) with G = 1 (v_group None) or D / v_group."""
    L.require_device(V)
    B, H, S, D = V.shape
    if D % 2 != 0:
        raise ValueError(f"quantize_v_int4 requires even head_dim; got {D}")
    group = D if v_group is None else int(v_group)
    G = D // group
    if out is None:
        packed = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=V.device)
        scale = torch.empty(B, H, S, G, dtype=meta_dtype, device=V.device)
        mn = torch.empty(B, H, S, G, dtype=meta_dtype, device=V.device)
    else:
        packed, scale, mn = out
    L.check(L.lib().fq_quantize_v_int4(
        V.data_ptr(), L.dtype_code(V.dtype), L.strides(V, 4), B, H, S, D, group,
        packed.data_ptr(), L.strides(packed, 4), scale.data_ptr(), L.strides(scale, 4),
        mn.data_ptr(), L.strides(mn, 4), L.dtype_code(scale.dtype), L.stream_handle(V.device)),
        "quantize_v_int4")
    return packed, scale, mn


def dequantize_k_int4(K_packed, scale, mn, page_size: int) -> torch.Tensor:
    """kv_quant.py:174-186 (tensor ops; prefill / test helper, not the decode path)."""
    q4 = _unpack_int4(K_packed)
    S = q4.shape[2]
    s = scale.repeat_interleave(page_size, dim=2)[:, :, :S, :]
    m = mn.repeat_interleave(page_size, dim=2)[:, :, :S, :]
    return (q4.float() * s.float() + m.float()).to(torch.bfloat16)


def dequantize_v_int4(V_packed, scale, mn) -> torch.Tensor:
    """kv_quant.py:208-215 (tensor ops), also for grouped V metadata."""
    q4 = _unpack_int4(V_packed).float()
    B, H, S, D = q4.shape
    G = scale.shape[-1]
    out = q4.view(B, H, S, G, D // G) * scale.float().unsqueeze(-1) + mn.float().unsqueeze(-1)
    return out.view(B, H, S, D).to(torch.bfloat16)


def _turbo_planes(X: torch.Tensor, out=None):
    L.require_device(X)
    B, H, S, D = X.shape
    if D % 8 != 0:
        raise ValueError(f"turbo quantisation requires head_dim multiple of 8; got {D}")
    if out is None:
        msb = torch.empty(B, H, S, D // 8, dtype=torch.uint8, device=X.device)
        lsb = torch.empty(B, H, S, D // 4, dtype=torch.uint8, device=X.device)
        scale = torch.empty(B, H, S, 1, dtype=torch.bfloat16, device=X.device)
    else:
        msb, lsb, scale = out
    L.check(L.lib().fq_quantize_turbo(
        X.data_ptr(), L.dtype_code(X.dtype), L.strides(X, 4), B, H, S, D,
        msb.data_ptr(), L.strides(msb, 4), lsb.data_ptr(), L.strides(lsb, 4),
        scale.data_ptr(), L.strides(scale, 4), L.stream_handle(X.device)), "quantize_turbo")
    return msb, lsb, scale


def quantize_k_turbo(K: torch.Tensor, page_size: int, *, out=None):
    """kv_quant.py:327-363: (K_msb, K_lsb, K_scale_turbo, K_scale_raw, K_mn_raw).
    The raw INT4-equivalent page metadata (for scoring) is bf16.  ``out`` =
    the five tensors (possibly strided views) to write into."""
    if out is None:
        msb, lsb, st = _turbo_planes(K)
        _, sr, mr = quantize_k_int4(K, page_size, meta_dtype=torch.bfloat16)
        return msb, lsb, st, sr, mr
    msb, lsb, st, sr, mr = out
    _turbo_planes(K, out=(msb, lsb, st))
    # the codes of this INT4 pass are not kept; only the page scale/min are
    scratch = torch.empty(K.shape[:-1] + (K.shape[-1] // 2,), dtype=torch.uint8, device=K.device)
    quantize_k_int4(K, page_size, meta_dtype=sr.dtype, out=(scratch, sr, mr))
    return msb, lsb, st, sr, mr


def quantize_v_turbo(V: torch.Tensor, *, out=None):
    """kv_quant.py:381-405: (V_msb, V_lsb, V_scale_turbo)."""
    return _turbo_planes(V, out=out)
