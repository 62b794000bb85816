"""CPU oracle for the flashquest sparse INT4 / turbo decode-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``flashquest_amd`` imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, as the checker, never as the thing measured or shipped.

It restates, in numpy, the reference's algorithm for every function on the
path.  Paths in citations are relative to the reference repository root.

Rounding conventions (the reference runs its cache writes on CUDA torch):
  * bf16 / fp16 tensor arithmetic is computed in fp32 and rounded to the
    tensor dtype after every op (torch "opmath" semantics);
  * ``tensor / python_scalar`` on CUDA multiplies by the fp32 reciprocal of
    the scalar (torch's CUDA true-division fast path for CPU scalars);
    ``tensor / tensor`` is IEEE fp32 division;
  * ``round`` is round-half-to-even; ``clamp_min(eps)`` on a half tensor is
    ``half(max(float(x), eps))``;
  * ``argmin`` / ``topk`` ties go to the lower index (documented for argmin).
  These rules are checked against torch executing the same operations on the
  GPU (tests/test_gpu_torch_arith_pins.py).

Pinning status (what checks each function; see tests/test_oracle_*.py):
  quantize_k_int4 / quantize_v_int4   closed form + reference KATs + invariants
                                      + brute force over a tiny input space
  pack/unpack int4, bit-split         reference KATs + round trips
  page_scores_*                       reference identity test (Quest bound)
                                      + fp64 closed form + upper-bound invariant
  select_pages_vectorized, compact    reference KATs + brute-force sort
  exact attention / merge / tail      closed forms (dense softmax, merge identity)
  causal_prefill_attention            torch SDPA (is_causal, enable_gqa) on the CPU,
                                      one-key and uniform-key closed forms
  dequant_cache_bf16                  round trip within scale / 2, bf16 rounding
                                      of the fp32 FMA checked elementwise
  wht128                              Sylvester Hadamard matrix, self-inverse
  quantize_*_turbo                    codebook KATs, bit-split round trip;
                                      rms reduction order: parity unpinned
                                      against the reference (torch reduction
                                      order is unspecified); pinned to this
                                      build's sequential order.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
EPS = F32(1e-6)                       # kv_quant.py:14  _EPS = 1e-6
INV15 = F32(1.0) / F32(15.0)          # fp32 reciprocal used by CUDA for "/ 15.0"
INV255 = F32(1.0) / F32(255.0)        # likewise for the INT8 quantisers' "/ 255.0"
LOG2E = 1.4426950408889634

# kv_quant.py:225-229 (K_TURBO_CODEBOOK; V uses the same codebook, :230)
TURBO_CODEBOOK = np.array(
    [-2.1519, -1.3439, -0.7560, -0.2451, 0.2451, 0.7560, 1.3439, 2.1519], dtype=F32)


# ----------------------------------------------------------------------------
# half-precision helpers
# ----------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 -> bf16 (round to nearest even), returned as uint16 bits."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) >> 16).astype(np.uint16)
    r = np.where(np.isnan(x), np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=F32).astype(np.float16).astype(F32)


def rounder(dtype: str):
    """Return the fp32 -> dtype -> fp32 rounding function for a tensor dtype."""
    if dtype == "bf16":
        return round_bf16
    if dtype == "f16":
        return round_f16
    if dtype == "f32":
        return lambda x: np.asarray(x, dtype=F32)
    raise ValueError(dtype)


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values (already representable) -> raw 16-bit storage."""
    if dtype == "bf16":
        return f32_to_bf16_bits(x)
    if dtype == "f16":
        return np.asarray(x, dtype=F32).astype(np.float16).view(np.uint16)
    raise ValueError(dtype)


def from_bits(b: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(b)
    if dtype == "f16":
        return np.asarray(b, dtype=np.uint16).view(np.float16).astype(F32)
    raise ValueError(dtype)


# ----------------------------------------------------------------------------
# INT4 packing (kv_quant.py:104-128)
# ----------------------------------------------------------------------------

def pack_int4(codes: np.ndarray) -> np.ndarray:
    """kv_quant.py:104-115: byte k = c[2k] | c[2k+1] << 4; high input bits masked."""
    codes = np.asarray(codes, dtype=np.uint8)
    if codes.shape[-1] % 2:
        raise ValueError("pack_int4 requires an even last axis")
    lo = codes[..., 0::2] & 0x0F
    hi = codes[..., 1::2] & 0x0F
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """kv_quant.py:118-128."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = (packed >> 4) & 0x0F
    return out


# ----------------------------------------------------------------------------
# Quantisers (kv_quant.py:131-215)
# ----------------------------------------------------------------------------

def scale_mn_per_page_channel_int4(K: np.ndarray, page_size: int, dtype: str = "bf16", inv=None):
    """kv_quant.py:131-149 (INT4, "/ 15.0"); with inv=INV255 kv_quant.py:18-40 (INT8).

    K: (..., S, D) fp32 values exactly representable in ``dtype``.
    Arithmetic happens in the input dtype: (mx - mn) and "/ 15.0" are each
    rounded to ``dtype``; clamp_min(1e-6) likewise.
    Returns (scale, mn), each (..., P, D) fp32 values in ``dtype``.
    """
    rnd = rounder(dtype)
    K = np.asarray(K, dtype=F32)
    *lead, S, D = K.shape
    P = (S + page_size - 1) // page_size
    pad = P * page_size - S
    kmin = np.concatenate([K, np.full((*lead, pad, D), np.inf, F32)], axis=-2) if pad else K
    kmax = np.concatenate([K, np.full((*lead, pad, D), -np.inf, F32)], axis=-2) if pad else K
    mn = kmin.reshape(*lead, P, page_size, D).min(axis=-2)
    mx = kmax.reshape(*lead, P, page_size, D).max(axis=-2)
    diff = rnd(mx - mn)
    scale = rnd(diff * (INV15 if inv is None else inv))
    scale = rnd(np.maximum(scale, EPS))
    return scale, mn


def quantize_k_int4(K: np.ndarray, page_size: int, dtype: str = "bf16", meta: str = "bf16"):
    """kv_quant.py:152-171: per-page, per-channel asymmetric INT4 for K.

    Codes use the dtype-rounded scale/mn (fp32 division, round half even,
    clamp 0..15).  The returned meta is rounded to ``meta`` (the reference
    casts to bf16; ``meta="f16"`` keeps an fp16 copy instead).
    Returns (packed (..., S, D/2) u8, scale (..., P, D) f32, mn (..., P, D) f32)
    where scale/mn hold values representable in ``meta``.
    """
    K = np.asarray(K, dtype=F32)
    *lead, S, D = K.shape
    if D % 2:
        raise ValueError("quantize_k_int4 requires even head_dim")
    scale, mn = scale_mn_per_page_channel_int4(K, page_size, dtype)
    tok_scale = np.repeat(scale, page_size, axis=-2)[..., :S, :]
    tok_mn = np.repeat(mn, page_size, axis=-2)[..., :S, :]
    norm = (K - tok_mn) / tok_scale
    codes = np.clip(np.rint(norm), 0, 15).astype(np.uint8)
    mrnd = rounder(meta)
    return pack_int4(codes), mrnd(scale), mrnd(mn)


def quantize_v_int4(V: np.ndarray, group: int | None = None, meta: str = "bf16"):
    """kv_quant.py:189-205: per-token asymmetric INT4 for V, in fp32.

    ``group=None`` is the reference (one scale/mn per token over all D);
    ``group=32`` quantises each run of 32 channels separately.
    Returns (packed (..., S, D/2), scale (..., S, G), mn (..., S, G)).
    """
    V = np.asarray(V, dtype=F32)
    *lead, S, D = V.shape
    g = D if group is None else group
    if D % 2 or D % g:
        raise ValueError("bad V grouping")
    G = D // g
    Vg = V.reshape(*lead, S, G, g)
    mn = Vg.min(axis=-1, keepdims=True)
    mx = Vg.max(axis=-1, keepdims=True)
    scale = np.maximum((mx - mn) * INV15, EPS)
    codes = np.clip(np.rint((Vg - mn) / scale), 0, 15).astype(np.uint8).reshape(*lead, S, D)
    mrnd = rounder(meta)
    return pack_int4(codes), mrnd(scale[..., 0]), mrnd(mn[..., 0])


def dequant_k(packed, scale, mn, page_size):
    """scripts/profile_contribution.py:79-94: codes*fp32(scale)+fp32(mn), no rounding."""
    codes = unpack_int4(packed).astype(F32)
    S = codes.shape[-2]
    tok_scale = np.repeat(scale, page_size, axis=-2)[..., :S, :]
    tok_mn = np.repeat(mn, page_size, axis=-2)[..., :S, :]
    return codes * tok_scale + tok_mn


def dequant_v(packed, scale, mn):
    """Per-token (or per token-group) V dequant, fp32 (profile_contribution.py:79-94)."""
    codes = unpack_int4(packed).astype(F32)
    *lead, S, D = codes.shape
    G = scale.shape[-1]
    c = codes.reshape(*lead, S, G, D // G)
    return (c * scale[..., None] + mn[..., None]).reshape(*lead, S, D)


# ----------------------------------------------------------------------------
# INT8 KV (kernel/kv_quant.py:18-100, kernel/sparse_fwd.py:23-157)
# ----------------------------------------------------------------------------

def quantize_k_int8(K: np.ndarray, page_size: int, dtype: str = "bf16", meta: str = "bf16"):
    """kv_quant.py:43-61: per-page, per-channel asymmetric uint8 for K.

    scale/mn as kv_quant.py:18-40 in the input dtype ((mx - mn) and "/ 255.0"
    each rounded to ``dtype``, clamp_min(1e-6)); codes by fp32 division with
    those (dtype) values, round half even, clamp 0..255; the meta is returned
    rounded to ``meta`` (the reference casts it to bf16 after the codes).
    Returns (codes (..., S, D) u8, scale (..., P, D) f32, mn (..., P, D) f32).
    """
    K = np.asarray(K, dtype=F32)
    *lead, S, D = K.shape
    scale, mn = scale_mn_per_page_channel_int4(K, page_size, dtype, inv=INV255)
    tok_scale = np.repeat(scale, page_size, axis=-2)[..., :S, :]
    tok_mn = np.repeat(mn, page_size, axis=-2)[..., :S, :]
    codes = np.clip(np.rint((K - tok_mn) / tok_scale), 0, 255).astype(np.uint8)
    mrnd = rounder(meta)
    return codes, mrnd(scale), mrnd(mn)


def quantize_v_int8(V: np.ndarray, meta: str = "bf16"):
    """kv_quant.py:78-89: per-token uint8 for V over all D channels, in fp32
    (mn, mx, scale = max((mx - mn) * fp32(1/255), 1e-6), codes by fp32
    division, round half even, clamp 0..255); meta rounded to ``meta`` after.
    Returns (codes (..., S, D) u8, scale (..., S, 1), mn (..., S, 1))."""
    V = np.asarray(V, dtype=F32)
    mn = V.min(axis=-1, keepdims=True)
    mx = V.max(axis=-1, keepdims=True)
    scale = np.maximum((mx - mn) * INV255, EPS)
    codes = np.clip(np.rint((V - mn) / scale), 0, 255).astype(np.uint8)
    mrnd = rounder(meta)
    return codes, mrnd(scale), mrnd(mn)


def dequant_k_int8(codes, scale, mn, page_size):
    """kv_quant.py:64-75 / sparse_fwd.py:95-96: codes*fp32(scale)+fp32(mn) (fp32, no final rounding)."""
    c = np.asarray(codes).astype(F32)
    S = c.shape[-2]
    tok_scale = np.repeat(np.asarray(scale, F32), page_size, axis=-2)[..., :S, :]
    tok_mn = np.repeat(np.asarray(mn, F32), page_size, axis=-2)[..., :S, :]
    return c * tok_scale + tok_mn


def dequant_v_int8(codes, scale, mn):
    """kv_quant.py:92-97 / sparse_fwd.py:121-126: per-token codes*scale+mn in fp32."""
    return np.asarray(codes).astype(F32) * np.asarray(scale, F32) + np.asarray(mn, F32)


def page_scores_int8_exact(Q, K_scale, K_mn):
    """criticality.py:77-125 in fp64: Q.mn + 255 * relu(Q).scale (GQA view)."""
    Q = np.asarray(Q, np.float64)
    B, Hq, D = Q.shape
    Hkv = K_scale.shape[1]
    rep = Hq // Hkv
    qg = Q.reshape(B, Hkv, rep, D)
    t1 = qg @ np.swapaxes(np.asarray(K_mn, np.float64), -1, -2)
    t2 = np.maximum(qg, 0) @ np.swapaxes(np.asarray(K_scale, np.float64), -1, -2)
    return (t1 + 255.0 * t2).reshape(B, Hq, -1)


def sparse_int8_attention(Q, K_u8, K_scale, K_mn, V_u8, V_scale, V_mn, page_mask, page_size=64,
                          sm_scale=None):
    """flash_attn_sparse_fwd semantics (sparse_fwd.py:23-157, wrapper 160-228), exact.
    Returns (O fp64, lse fp64)."""
    keys = dequant_k_int8(K_u8, K_scale, K_mn, page_size)
    vals = dequant_v_int8(V_u8, V_scale, V_mn)
    S = keys.shape[-2]
    tm = page_mask_to_token_mask(page_mask, S, page_size)
    return exact_attention(Q, keys, vals, tm, sm_scale)


# ----------------------------------------------------------------------------
# Page scoring (eager/criticality.py:7-31, 128-163)
# ----------------------------------------------------------------------------

def page_summary_int8(K_u8, K_scale, K_mn, page_size: int):
    """dequantize_k (kv_quant.py:64-75: codes * fp32(scale) + fp32(mn), then
    bf16) followed by compute_page_summary (page_summary.py:7-39: per page and
    channel the min / max over the page's tokens, a partial last page padded
    with +-inf).  Returns (page_min, page_max) (B, H, P, D) as fp32 values of
    the bf16 keys."""
    kd = round_bf16(dequant_k_int8(K_u8, K_scale, K_mn, page_size))
    B, H, S, D = kd.shape
    P = (S + page_size - 1) // page_size
    pad = P * page_size - S
    lo = np.concatenate([kd, np.full((B, H, pad, D), np.inf, F32)], axis=2)
    hi = np.concatenate([kd, np.full((B, H, pad, D), -np.inf, F32)], axis=2)
    lo = lo.reshape(B, H, P, page_size, D).min(axis=3)
    hi = hi.reshape(B, H, P, page_size, D).max(axis=3)
    return lo.astype(F32), hi.astype(F32)


def compute_page_summary(K, page_size: int):
    """page_summary.py:7-39: per page and channel the min / max of K (B, H, S,
    D) over the page's tokens (a partial last page padded with +-inf, so only
    its valid tokens count).  Returns (page_min, page_max) (B, H, P, D)."""
    K = np.asarray(K)
    B, H, S, D = K.shape
    P = (S + page_size - 1) // page_size
    pad = P * page_size - S
    lo = np.concatenate([K, np.full((B, H, pad, D), np.inf, K.dtype)], axis=2)
    hi = np.concatenate([K, np.full((B, H, pad, D), -np.inf, K.dtype)], axis=2)
    return lo.reshape(B, H, P, page_size, D).min(axis=3), hi.reshape(B, H, P, page_size, D).max(axis=3)


def page_scores_int8_bound_fixed(Q, K_scale, K_mn):
    """page_scores_int8 (criticality.py:34-74) in this build's fixed order:
    the bounds as the reference forms them, min = fp32(K_mn), max = fp32(K_mn)
    + 255 * fp32(K_scale) (fp32 multiply, then fp32 add), then
    page_scores_quest_fixed.  Q (B, H_q, D).  Returns (B, H_q, P) fp32."""
    mn = np.asarray(K_mn, F32)
    mx = (mn + (F32(255.0) * np.asarray(K_scale, F32)).astype(F32)).astype(F32)
    return page_scores_quest_fixed(Q, mn, mx)


def page_scores_quest_fixed(Q, page_min, page_max):
    """page_scores (criticality.py:7-31) with this build's fixed fp32 order:
    term_d = max(q_d * max_d, q_d * min_d) (each product rounded to fp32);
    lane j sums terms 4j .. 4j+3 left to right, then the D/4 lane sums combine
    by the butterfly v_j += v_(j ^ o) for o = D/8, D/16, ..., 1.
    Q (B, H_q, D); summaries (B, H_kv, P, D).  Returns (B, H_q, P) fp32."""
    Q = np.asarray(Q, F32)
    B, Hq, D = Q.shape
    Hkv, P = page_min.shape[1], page_min.shape[2]
    rep = Hq // Hkv
    mn = np.repeat(np.asarray(page_min, F32), rep, axis=1)
    mx = np.repeat(np.asarray(page_max, F32), rep, axis=1)
    q = Q[:, :, None, :]
    term = np.maximum((q * mx).astype(F32), (q * mn).astype(F32)).astype(F32)   # (B, Hq, P, D)
    t4 = term.reshape(B, Hq, P, D // 4, 4)
    v = t4[..., 0].copy()
    for i in range(1, 4):
        v = (v + t4[..., i]).astype(F32)
    nl = D // 4
    idx = np.arange(nl)
    o = nl // 2
    while o >= 1:
        v = (v + v[..., idx ^ o]).astype(F32)
        o //= 2
    return v[..., 0]


def page_scores_quest(Q, page_min, page_max):
    """criticality.py:7-31: sum_d max(q_d*min_d, q_d*max_d), fp64, GQA-broadcast.

    Q: (B, H_q, D); page_min/max: (B, H_kv, P, D).  Returns (B, H_q, P) fp64.
    """
    Q = np.asarray(Q, np.float64)
    B, Hq, D = Q.shape
    Hkv = page_min.shape[1]
    rep = Hq // Hkv
    mn = np.repeat(np.asarray(page_min, np.float64), rep, axis=1)
    mx = np.repeat(np.asarray(page_max, np.float64), rep, axis=1)
    q = Q[:, :, None, :]
    return np.maximum(q * mn, q * mx).sum(-1)


def page_scores_int4_exact(Q, K_scale, K_mn):
    """criticality.py:128-163 in fp64: Q.mn + 15 * relu(Q).scale, Q viewed (B,H_kv,n_rep,D)."""
    Q = np.asarray(Q, np.float64)
    B, Hq, D = Q.shape
    Hkv = K_scale.shape[1]
    if Hq % Hkv:
        raise ValueError("H_q must be divisible by H_kv")
    rep = Hq // Hkv
    qg = Q.reshape(B, Hkv, rep, D)
    t1 = qg @ np.swapaxes(np.asarray(K_mn, np.float64), -1, -2)
    t2 = np.maximum(qg, 0) @ np.swapaxes(np.asarray(K_scale, np.float64), -1, -2)
    return (t1 + 15.0 * t2).reshape(B, Hq, -1)


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded fp32 fused multiply-add RN(a*b + c), elementwise, for
    finite fp32 inputs (the GPU's v_fma_f32 / v_fma_mix_f32 semantics).

    a*b is exact in fp64 (at most 48 significant bits); TwoSum splits the fp64
    sum into s + e exactly; RN32(s) equals RN32(s + e) except when s lies
    exactly halfway between two fp32 neighbours and e != 0, where e decides.
    """
    a = np.asarray(a, F32).astype(np.float64)
    b = np.asarray(b, F32).astype(np.float64)
    c = np.asarray(c, F32).astype(np.float64)
    x = a * b
    s = x + c
    bb = s - x
    e = (x - (s - bb)) + (c - bb)
    r = s.astype(F32)
    d = s - r.astype(np.float64)
    toward = np.where(d > 0, np.float32(np.inf), np.float32(-np.inf)).astype(F32)
    nb = np.nextafter(r, toward)
    gap = np.abs(nb.astype(np.float64) - r.astype(np.float64))
    mid = (d != 0) & (2.0 * np.abs(d) == gap) & (e != 0)
    up = mid & ((e > 0) == (d > 0))       # past the midpoint, away from r
    down = mid & ~up                      # short of the midpoint: r itself
    out = np.where(up, nb, r)
    out = np.where(down, r, out)
    return out.astype(F32)


def _lane_fma_butterfly(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Fixed fp32 evaluation of sum_d a_d * b_d over the last axis D.

    Lane j (of D/8) owns channels 8j..8j+7: t = a_0*b_0 (rounded), then
    t = fma(a_i, b_i, t) for i = 1..7 (fused, one rounding each); lanes are
    then combined the way the HIP kernel's DPP steps do: with 16 lanes first
    v_j += v_(15-j) (row mirror), then within each 8 lanes v_j += v_(7-j)
    (half mirror), then v_j += v_(j^1), then v_j += v_(j^2).  Each step adds a
    value to its partner's, so every lane ends with the same sum.
    """
    a, b = np.broadcast_arrays(np.asarray(a, F32), np.asarray(b, F32))
    D = a.shape[-1]
    nl = D // 8
    pa = a.reshape(*a.shape[:-1], nl, 8)
    pb = b.reshape(*b.shape[:-1], nl, 8)
    t = (pa[..., 0] * pb[..., 0]).astype(F32)
    for i in range(1, 8):
        t = fma32(pa[..., i], pb[..., i], t)
    idx = np.arange(nl)
    partners = []
    if nl == 16:
        partners.append(15 - idx)
    partners += [(idx & ~7) | (7 - (idx & 7)), idx ^ 1, idx ^ 2]
    for pr in partners:
        t = (t + t[..., pr]).astype(F32)
    return t[..., 0]


def page_scores_fixed(Q, K_scale, K_mn, mode: str = "per_q_head", levels: float = 15.0):
    """criticality.py:128-163 with this build's fixed fp32 evaluation order.

    Per (query head r, page p): t1 = sum_d q_d*mn_d, t2 = sum_d relu(q_d)*scale_d
    (per lane an FMA chain, then the butterfly of ``_lane_fma_butterfly``);
    score = t1 + t2*15 (term2 is scaled before the add, criticality.py:161-162).
    mode "per_q_head": (B, H_q, P).
    mode "per_kv_head_sum": (B, H_kv, P), the score of the group's summed query:
    the same formula with q = (q_0 + q_1) + ... and relu(q) = (relu(q_0) +
    relu(q_1)) + ... (fp32, heads in order).  In exact arithmetic it equals the
    sum of the group's per-head scores (both terms are linear in q, relu(q)).
    """
    Q = np.asarray(Q, F32)
    B, Hq, D = Q.shape
    Hkv, P = K_scale.shape[1], K_scale.shape[2]
    rep = Hq // Hkv
    qg = Q.reshape(B, Hkv, rep, 1, D)
    qpos = np.where(qg > 0, qg, F32(0))
    if mode == "per_kv_head_sum":
        qs, ps = qg[:, :, 0].copy(), qpos[:, :, 0].copy()
        for r in range(1, rep):
            qs = (qs + qg[:, :, r]).astype(F32)
            ps = (ps + qpos[:, :, r]).astype(F32)
        qg, qpos = qs[:, :, None], ps[:, :, None]               # one summed row per group
    elif mode != "per_q_head":
        raise ValueError(mode)
    mn = np.asarray(K_mn, F32)[:, :, None, :, :]
    sc = np.asarray(K_scale, F32)[:, :, None, :, :]
    t1 = _lane_fma_butterfly(qg, mn)
    t2 = _lane_fma_butterfly(qpos, sc)
    s = (t1 + (t2 * F32(levels)).astype(F32)).astype(F32)    # (B, Hkv, rows, P); 255 for INT8
    if mode == "per_q_head":
        return s.reshape(B, Hq, P)
    return s[:, :, 0, :]


# ----------------------------------------------------------------------------
# Selection (eager/selection.py:65-164)
# ----------------------------------------------------------------------------

def k_per_head(retention, H: int, P: int) -> np.ndarray:
    """selection.py:92-103: ceil(fp32(r) * fp32(P)) clamped to [0, P]."""
    if np.isscalar(retention):
        if not 0.0 <= float(retention) <= 1.0:
            raise ValueError("scalar retention must be in [0, 1]")
        r = np.full((H,), retention, dtype=F32)
    else:
        r = np.asarray(retention, dtype=F32)
        if r.shape != (H,):
            raise ValueError("per-head retention must be shape (H,)")
    k = np.ceil((r * F32(P)).astype(F32)).astype(np.int64)
    return np.clip(k, 0, P)


def sortable_key(x: np.ndarray) -> np.ndarray:
    """Monotone fp32 -> uint32 map (larger float -> larger key; -0 == +0; NaN largest)."""
    x = np.asarray(x, F32).copy()
    x[x == 0] = 0.0
    x[np.isnan(x)] = np.nan
    u = x.view(np.uint32)
    u = np.where(np.isnan(x), np.uint32(0x7FC00000), u)
    return np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)


def topk_mask_rows(scores: np.ndarray, k: np.ndarray) -> np.ndarray:
    """Per row: the k largest scores, ties to the lower page index."""
    N, P = scores.shape
    key = sortable_key(scores).astype(np.int64)
    mask = np.zeros((N, P), dtype=bool)
    idx = np.arange(P)
    for n in range(N):
        kk = int(k[n])
        if kk <= 0:
            continue
        order = np.lexsort((idx, -key[n]))
        mask[n, order[:kk]] = True
    return mask


def select_pages_vectorized(scores, retention, num_sinks: int, window_pages: int,
                            k_max_static: int | None = None):
    """selection.py:65-126.  scores (B, H, S_q, P) -> bool mask (B, H, S_q, P)."""
    scores = np.asarray(scores, F32)
    B, H, Sq, P = scores.shape
    k_h = k_per_head(retention, H, P)
    k_max = int(k_h.max()) if k_max_static is None else min(int(k_max_static), P)
    k_eff = np.minimum(k_h, k_max)
    rows = scores.transpose(1, 0, 2, 3).reshape(H, B * Sq, P)
    mask = np.zeros((H, B * Sq, P), dtype=bool)
    for h in range(H):
        mask[h] = topk_mask_rows(rows[h], np.full((B * Sq,), k_eff[h]))
    mask = mask.reshape(H, B, Sq, P).transpose(1, 0, 2, 3).copy()
    if num_sinks > 0:
        mask[..., :min(num_sinks, P)] = True
    if window_pages > 0:
        mask[..., P - min(window_pages, P):] = True
    return mask


def select_pages(scores, retention, num_sinks: int, window_pages: int):
    """selection.py:9-62 (the per-head loop form): per head, r = the fp32
    retention read back as a double; r >= 1 selects every page, r <= 0 none,
    otherwise the top ceil(r * P) (double product), then the sink and window
    pages.  scores (B, H, S_q, P) -> bool mask."""
    scores = np.asarray(scores, F32)
    B, H, Sq, P = scores.shape
    if np.isscalar(retention):
        if not 0.0 <= float(retention) <= 1.0:
            raise ValueError("scalar retention must be in [0, 1]")
        r = np.full((H,), retention, dtype=F32)
    else:
        r = np.asarray(retention, dtype=F32)
        if r.shape != (H,):
            raise ValueError("per-head retention must be shape (H,)")
    mask = np.zeros((B, H, Sq, P), dtype=bool)
    for h in range(H):
        rh = float(r[h])
        if rh >= 1.0:
            mask[:, h] = True
            continue
        if rh <= 0.0:
            continue
        k = math.ceil(rh * P)
        rows = scores[:, h].reshape(B * Sq, P)
        mask[:, h] = topk_mask_rows(rows, np.full((B * Sq,), k)).reshape(B, Sq, P)
    if num_sinks > 0:
        mask[..., :min(num_sinks, P)] = True
    if window_pages > 0:
        mask[..., P - min(window_pages, P):] = True
    return mask


def build_compact_selection(mask, BUCKET_MAX: int):
    """selection.py:129-164: selected ids sorted descending, -1 padded / truncated."""
    if BUCKET_MAX < 1:
        raise ValueError("BUCKET_MAX must be >= 1")
    mask = np.asarray(mask, dtype=bool)
    *lead, P = mask.shape
    pos = np.where(mask, np.arange(P, dtype=np.int32), np.int32(-1))
    srt = -np.sort(-pos, axis=-1)
    out = np.full((*lead, BUCKET_MAX), -1, dtype=np.int32)
    n = min(P, BUCKET_MAX)
    out[..., :n] = srt[..., :n]
    return out


def union_lists(qmask_bits: np.ndarray):
    """(G, P) per-group bitmask of selecting query heads -> ascending page lists."""
    out = []
    for g in range(qmask_bits.shape[0]):
        pages = np.nonzero(qmask_bits[g])[0]
        out.append((pages.astype(np.int32), qmask_bits[g][pages].astype(np.int32)))
    return out


# ----------------------------------------------------------------------------
# Attention (sparse_int4_fwd.py:23-157 semantics; profile_contribution.py:120-143)
# ----------------------------------------------------------------------------

def exact_attention(q, keys, values, token_mask, sm_scale=None):
    """Grouped exact attention in fp64 over fp32 dequantised K/V.

    q (B, H_q, D); keys/values (B, H_kv, S, D); token_mask (B, H_q, S) bool.
    Returns (O (B, H_q, D) fp64, lse (B, H_q) fp64 in nats); an empty row
    gives O = 0 and lse = -inf (sparse_int4_fwd.py:147-157).
    """
    q = np.asarray(q, np.float64)
    B, Hq, D = q.shape
    Hkv = keys.shape[1]
    rep = Hq // Hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    k = np.repeat(np.asarray(keys, np.float64), rep, axis=1)
    v = np.repeat(np.asarray(values, np.float64), rep, axis=1)
    logits = np.einsum("bhd,bhsd->bhs", q, k) * sm_scale
    logits = np.where(token_mask, logits, -np.inf)
    m = logits.max(-1, keepdims=True)
    empty = ~np.isfinite(m)
    msafe = np.where(empty, 0.0, m)
    p = np.where(token_mask, np.exp(logits - msafe), 0.0)
    l = p.sum(-1, keepdims=True)
    lsafe = np.where(l == 0, 1.0, l)
    O = np.einsum("bhs,bhsd->bhd", p, v) / lsafe
    lse = np.where(l[..., 0] == 0, -np.inf, msafe[..., 0] + np.log(lsafe[..., 0]))
    return O, lse


def dequant_cache_bf16(codes_or_packed, K_or_V: str, scale, mn, page_size: int = 64, bits: int = 4):
    """The reference's prefill dequantisers, rounded to bf16 like them:
    dequantize_k_int4 / dequantize_v_int4 (kernel/kv_quant.py:174-186, 208-215)
    for bits 4 and dequantize_k / dequantize_v (64-75, 92-97) for bits 8:
    fp32 code * scale + mn, then bf16.  Returns fp32 holding bf16 values."""
    codes = unpack_int4(codes_or_packed) if bits == 4 else np.asarray(codes_or_packed)
    codes = codes.astype(F32)
    scale = np.asarray(scale, F32)
    mn = np.asarray(mn, F32)
    if K_or_V == "K":
        S = codes.shape[-2]
        s = np.repeat(scale, page_size, axis=-2)[..., :S, :]
        m = np.repeat(mn, page_size, axis=-2)[..., :S, :]
        out = (codes * s).astype(F32) + m
    else:
        *lead, S, D = codes.shape
        G = scale.shape[-1]
        c = codes.reshape(*lead, S, G, D // G)
        out = ((c * scale[..., None]).astype(F32) + mn[..., None]).reshape(*lead, S, D)
    return round_bf16(out.astype(F32))


def causal_prefill_attention(q, keys, values, causal_offset: int = 0, sm_scale=None):
    """F.scaled_dot_product_attention(q, K, V, is_causal=True, enable_gqa=True)
    as the reference's prefill calls it (llama_persistent_patch.py:196-201),
    in fp64: query i attends keys j <= i + causal_offset, where torch's
    is_causal is causal_offset = 0 (the upper-left aligned tril(ones(S_q, S_kv)))
    and S_kv - S_q gives the lower-right alignment.  GQA: query head h uses KV
    head h // (H_q / H_kv).  q (B,H_q,S_q,D); keys/values (B,H_kv,S_kv,D)."""
    q = np.asarray(q, np.float64)
    B, Hq, Sq, D = q.shape
    Hkv, Skv = keys.shape[1], keys.shape[2]
    rep = Hq // Hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    k = np.repeat(np.asarray(keys, np.float64), rep, axis=1)
    v = np.repeat(np.asarray(values, np.float64), rep, axis=1)
    logits = np.einsum("bhid,bhjd->bhij", q, k) * sm_scale
    allowed = np.arange(Skv)[None, :] <= np.arange(Sq)[:, None] + causal_offset
    logits = np.where(allowed, logits, -np.inf)
    m = logits.max(-1, keepdims=True)
    p = np.exp(logits - m)
    return np.einsum("bhij,bhjd->bhid", p, v) / p.sum(-1, keepdims=True)


def prefill_packed(q, K_codes, K_scale, K_mn, V_codes, V_scale, V_mn, K_tail, V_tail, *, page_size: int = 64,
                   bits: int = 4, causal_offset: int = 0, sm_scale=None):
    """llama_persistent_patch.py:196-201: cat(dequant(cache), tail) then causal
    SDPA (fp64 over the bf16 K/V the reference builds)."""
    K = dequant_cache_bf16(K_codes, "K", K_scale, K_mn, page_size, bits)
    V = dequant_cache_bf16(V_codes, "V", V_scale, V_mn, page_size, bits)
    if K_tail is not None and K_tail.shape[-2] > 0:
        K = np.concatenate([K, round_bf16(np.asarray(K_tail, F32))], axis=-2)
        V = np.concatenate([V, round_bf16(np.asarray(V_tail, F32))], axis=-2)
    return causal_prefill_attention(q, K, V, causal_offset, sm_scale)


def page_mask_to_token_mask(page_mask, S: int, page_size: int):
    """(B, H_q, P) page mask -> (B, H_q, S) token mask; tokens >= S are dropped."""
    tm = np.repeat(np.asarray(page_mask, bool), page_size, axis=-1)
    return tm[..., :S]


def sparse_int4_attention(Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn,
                          page_mask, page_size=64, sm_scale=None):
    """flash_attn_sparse_int4_fwd semantics (sparse_int4_fwd.py:160-248).

    Q (B,H_q,D); packed (B,H_kv,S,D/2); K meta (B,H_kv,P,D); V meta (B,H_kv,S,G);
    page_mask (B,H_q,P) bool.  Returns (O fp64, lse fp64).
    """
    keys = dequant_k(K_packed, K_scale, K_mn, page_size)
    vals = dequant_v(V_packed, V_scale, V_mn)
    S = keys.shape[-2]
    tm = page_mask_to_token_mask(page_mask, S, page_size)
    return exact_attention(Q, keys, vals, tm, sm_scale)


def sparse_int4_attention_selected(Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn,
                                   page_mask, page_size=64, sm_scale=None):
    """Same result as ``sparse_int4_attention`` but dequantises only the pages
    some query head of a KV group selected (the work a sparse CPU path does).
    fp32 logits/softmax; returns (O fp32, lse fp32)."""
    Q = np.asarray(Q, F32)
    B, Hq, D = Q.shape
    Hkv = K_packed.shape[1]
    S = K_packed.shape[2]
    rep = Hq // Hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    O = np.zeros((B, Hq, D), F32)
    lse = np.full((B, Hq), -np.inf, F32)
    for b in range(B):
        for h in range(Hkv):
            pm = page_mask[b, h * rep:(h + 1) * rep]           # (rep, P)
            pages = np.nonzero(pm.any(0))[0]
            if len(pages) == 0:
                continue
            tok = (pages[:, None] * page_size + np.arange(page_size)).reshape(-1)
            keep = tok < S
            tok = tok[keep]
            codes_k = unpack_int4(K_packed[b, h, tok]).astype(F32)
            codes_v = unpack_int4(V_packed[b, h, tok]).astype(F32)
            pg = tok // page_size
            k = codes_k * K_scale[b, h, pg] + K_mn[b, h, pg]
            G = V_scale.shape[-1]
            v = (codes_v.reshape(len(tok), G, D // G) * V_scale[b, h, tok][..., None]
                 + V_mn[b, h, tok][..., None]).reshape(len(tok), D)
            logits = (Q[b, h * rep:(h + 1) * rep] @ k.T) * F32(sm_scale)      # (rep, T)
            tm = np.repeat(pm[:, pages], page_size, axis=1)[:, keep]
            logits = np.where(tm, logits, -np.inf)
            m = logits.max(1, keepdims=True)
            ok = np.isfinite(m[:, 0])
            p = np.where(tm, np.exp(logits - np.where(ok[:, None], m, 0)), 0).astype(F32)
            l = p.sum(1)
            O[b, h * rep:(h + 1) * rep] = np.where(ok[:, None], (p @ v) / np.where(l > 0, l, 1)[:, None], 0)
            lse[b, h * rep:(h + 1) * rep] = np.where(ok, m[:, 0] + np.log(np.where(l > 0, l, 1)), -np.inf)
    return O, lse


def compact_ids_to_page_mask(ids, P: int):
    """sparse_int4_fwd_compact.py:68-78: -1 slots (and ids outside [0,P)) are skipped."""
    ids = np.asarray(ids)
    B, H, _ = ids.shape
    mask = np.zeros((B, H, P), dtype=bool)
    for b in range(B):
        for h in range(H):
            for p in ids[b, h]:
                if 0 <= p < P:
                    mask[b, h, p] = True
    return mask


def merge_two_attentions(O_a, lse_a, O_b, lse_b):
    """llama_persistent_patch.py:50-61 in fp64 (returns fp64; caller rounds)."""
    m = np.maximum(lse_a, lse_b)
    with np.errstate(invalid="ignore"):
        wa = np.exp(lse_a - m)[..., None]
        wb = np.exp(lse_b - m)[..., None]
    return (wa * O_a + wb * O_b) / (wa + wb)


def dense_attn_with_lse(Q, K, V):
    """llama_persistent_patch.py:30-47: dense attention over the bf16 tail (fp64 here)."""
    B, Hq, D = Q.shape
    S = K.shape[2]
    tm = np.ones((B, Hq, S), dtype=bool)
    return exact_attention(Q, K, V, tm)


# ----------------------------------------------------------------------------
# Walsh-Hadamard / TurboQuant (kernel/wht.py, kv_quant.py:225-420)
# ----------------------------------------------------------------------------

def wht(x: np.ndarray, dtype: str = "f32") -> np.ndarray:
    """wht.py:17-41: butterflies (a+b, a-b) for h = 1, 2, ..., D/2, then / sqrt(D).

    Each stage is rounded to ``dtype``; the final scale multiplies by the fp32
    reciprocal of sqrt(D) (CUDA "/ python_scalar").
    """
    rnd = rounder(dtype)
    x = np.asarray(x, F32)
    D = x.shape[-1]
    if D == 0 or D & (D - 1):
        raise ValueError(f"head_dim must be a positive power of 2, got {D}")
    out = x.copy()
    h = 1
    while h < D:
        o = out.reshape(*out.shape[:-1], D // (2 * h), 2, h)
        a = o[..., 0, :]
        b = o[..., 1, :]
        out = rnd(np.stack([a + b, a - b], axis=-2)).reshape(*x.shape)
        h *= 2
    inv = F32(1.0) / F32(math.sqrt(D))
    return rnd(out * inv)


def hadamard_matrix(D: int) -> np.ndarray:
    """Sylvester Hadamard matrix / sqrt(D) (closed form used to pin ``wht``)."""
    H = np.array([[1.0]])
    while H.shape[0] < D:
        H = np.block([[H, H], [H, -H]])
    return H / math.sqrt(D)


def quantize_to_codebook(x: np.ndarray, codebook=TURBO_CODEBOOK) -> np.ndarray:
    """kv_quant.py:239-250: nearest codepoint index, first index on ties."""
    d = np.abs(np.asarray(x, F32)[..., None] - codebook)
    return d.argmin(-1).astype(np.uint8)


def pack_bit_split(idx: np.ndarray):
    """kv_quant.py:253-279: msb bit i of byte j = d 8j+i; lsb field i of byte j = d 4j+i."""
    idx = np.asarray(idx, np.uint8)
    *pre, D = idx.shape
    if D % 8:
        raise ValueError("last axis must be a multiple of 8")
    msb = ((idx >> 2) & 1).reshape(*pre, D // 8, 8)
    msb = (msb.astype(np.uint32) << np.arange(8, dtype=np.uint32)).sum(-1).astype(np.uint8)
    lsb = (idx & 3).reshape(*pre, D // 4, 4)
    lsb = (lsb.astype(np.uint32) << (2 * np.arange(4, dtype=np.uint32))).sum(-1).astype(np.uint8)
    return msb, lsb


def unpack_bit_split(msb, lsb, D: int):
    """kv_quant.py:282-298."""
    msb = np.asarray(msb, np.uint8)
    lsb = np.asarray(lsb, np.uint8)
    m = ((msb[..., None] >> np.arange(8, dtype=np.uint8)) & 1).reshape(*msb.shape[:-1], D)
    l = ((lsb[..., None] >> (2 * np.arange(4, dtype=np.uint8))) & 3).reshape(*lsb.shape[:-1], D)
    return ((m << 2) | l).astype(np.uint8)


def _rms_seq(x: np.ndarray) -> np.ndarray:
    """sqrt(mean(x^2)) with a fixed fp32 order: sequential sum of squares, / D, sqrt."""
    x = np.asarray(x, F32)
    D = x.shape[-1]
    acc = np.zeros(x.shape[:-1], F32)
    for d in range(D):
        acc = (acc + (x[..., d] * x[..., d]).astype(F32)).astype(F32)
    return np.sqrt((acc / F32(D)).astype(F32)).astype(F32)


def quantize_turbo(X: np.ndarray, dtype: str = "bf16"):
    """kv_quant.py:327-363 / 381-405 (K and V share the transform): WHT (in the
    input dtype) -> per-token rms (clamped >= 1e-6) -> nearest codepoint of the
    8-level codebook -> bit-split planes.  Returns (msb, lsb, scale_bf16_as_f32)."""
    rot = wht(X, dtype)
    rms = np.maximum(_rms_seq(rot), EPS)
    idx = quantize_to_codebook((rot / rms[..., None]).astype(F32))
    msb, lsb = pack_bit_split(idx)
    return msb, lsb, round_bf16(rms)[..., None]


def quantize_k_turbo(K: np.ndarray, page_size: int, dtype: str = "bf16"):
    """kv_quant.py:327-363: turbo planes + raw un-rotated INT4 page meta (bf16)."""
    msb, lsb, st = quantize_turbo(K, dtype)
    sr, mr = scale_mn_per_page_channel_int4(K, page_size, dtype)
    return msb, lsb, st, round_bf16(sr), round_bf16(mr)


def dequant_turbo_rot(msb, lsb, scale, D: int):
    """Rotated-basis dequant: codebook[idx] * fp32(scale)  (sparse_turbo_fwd.py:190-196)."""
    idx = unpack_bit_split(msb, lsb, D)
    return TURBO_CODEBOOK[idx.astype(np.int64)] * np.asarray(scale, F32)


def dequant_turbo_bf16(msb, lsb, scale, D: int = 128):
    """dequantize_k_turbo / dequantize_v_turbo (kernel/kv_quant.py:366-420):
    codebook[idx] * fp32(scale), the fp32 WHT (wht.py:17-41), then bf16."""
    return round_bf16(wht(dequant_turbo_rot(msb, lsb, scale, D), "f32"))


def sparse_turbo_attention(Q, K_msb, K_lsb, K_st, V_msb, V_lsb, V_st, page_mask,
                           page_size=64, sm_scale=None):
    """flash_attn_sparse_turbo_fwd semantics (sparse_turbo_fwd.py:254-346), exact:
    rotate Q, attend in the rotated basis, rotate O back.  fp64 out."""
    Q = np.asarray(Q, np.float64)
    D = Q.shape[-1]
    Hm = hadamard_matrix(D)
    q_rot = Q @ Hm.T
    keys = dequant_turbo_rot(K_msb, K_lsb, K_st, D)
    vals = dequant_turbo_rot(V_msb, V_lsb, V_st, D)
    S = keys.shape[-2]
    tm = page_mask_to_token_mask(page_mask, S, page_size)
    O_rot, lse = exact_attention(q_rot, keys, vals, tm, sm_scale)
    return O_rot @ Hm.T, lse


def random_signs(seed: int, D: int = 128) -> np.ndarray:
    """Seeded +-1 vector for the randomized WHT (config 3)."""
    rng = np.random.default_rng(seed)
    return np.where(rng.random(D) < 0.5, -1.0, 1.0).astype(F32)


def rotate_signed(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """Randomized WHT: WHT(s * x) in fp64 (the rotation applied to K, V and Q)."""
    D = x.shape[-1]
    return (np.asarray(x, np.float64) * signs) @ hadamard_matrix(D).T


def rotate_signed_f32(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """The rotated decode's fp32 rotation of Q (config 3): WHT(s * x) with every
    butterfly rounded to fp32 (h = 1, 2, ..., D/2), then times fp32(1/sqrt(D)).
    s * x is exact; ``wht`` restates the butterflies."""
    return wht(np.asarray(x, F32) * np.asarray(signs, F32), "f32")


def unrotate_signed(y: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """Inverse of ``rotate_signed``: s * WHT(y)."""
    D = y.shape[-1]
    return (np.asarray(y, np.float64) @ hadamard_matrix(D).T) * signs


# ----------------------------------------------------------------------------
# Whole decode step (llama_persistent_patch.py:202-245, completed pages only)
# ----------------------------------------------------------------------------

def decode_step(Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, *, retention,
                num_sinks, window_pages, page_size=64, mode="per_q_head",
                k_max_static=None, bits=4):
    """Score -> select -> sparse attention for one layer.

    Returns dict(scores, mask (B,H_q,P), O fp64, lse fp64).  ``mode``
    "per_kv_head_sum" selects once per KV head from the summed group scores
    and applies that selection to every query head of the group.
    """
    Q = np.asarray(Q, F32)
    B, Hq, D = Q.shape
    Hkv, P = K_scale.shape[1], K_scale.shape[2]
    rep = Hq // Hkv
    scores = page_scores_fixed(Q, K_scale, K_mn, mode, 255.0 if bits == 8 else 15.0)
    if mode == "per_q_head":
        mask = select_pages_vectorized(scores[:, :, None, :], retention, num_sinks,
                                       window_pages, k_max_static)[:, :, 0, :]
    else:
        r = retention if np.isscalar(retention) else np.asarray(retention, F32).reshape(Hkv, rep).max(-1)
        m = select_pages_vectorized(scores[:, :, None, :], r, num_sinks, window_pages,
                                    k_max_static)[:, :, 0, :]
        mask = np.repeat(m, rep, axis=1)
    attn = sparse_int8_attention if bits == 8 else sparse_int4_attention
    O, lse = attn(Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, mask, page_size)
    return {"scores": scores, "mask": mask, "O": O, "lse": lse}
