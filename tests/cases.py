"""Seeded test cases shared by the GPU parity tests (inputs built on the CPU
with numpy, quantised by the oracle, then moved to the device)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import fq_oracle as O

TORCH_HALF = {"bf16": torch.bfloat16, "f16": torch.float16}


def dev():
    return torch.device("cuda:0")


def to_dev_half(a: np.ndarray, dtype: str) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(TORCH_HALF[dtype]).to(dev())


def to_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def make_kv(rng, B, Hkv, S, D, dtype="bf16", outliers=True):
    rnd = O.rounder(dtype)
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    if outliers:
        K = K * rng.lognormal(0.0, 1.0, (B, Hkv, 1, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    return rnd(K), rnd(V)


class Int4Case:
    """Oracle-quantised INT4 cache + query, on the host and on the device."""

    def __init__(self, seed, B=1, Hq=6, Hkv=2, S=1024, D=128, page=64, dtype="bf16", meta="bf16",
                 vgroup=None, outliers=True):
        rng = np.random.default_rng(seed)
        self.B, self.Hq, self.Hkv, self.S, self.D, self.page = B, Hq, Hkv, S, D, page
        self.dtype, self.meta, self.vgroup = dtype, meta, vgroup
        self.K, self.V = make_kv(rng, B, Hkv, S, D, dtype, outliers)
        self.Q = O.rounder(dtype)(rng.standard_normal((B, Hq, D)).astype(np.float32))
        self.kp, self.ks, self.km = O.quantize_k_int4(self.K, page, dtype, meta)
        self.vp, self.vs, self.vm = O.quantize_v_int4(self.V, vgroup, meta)
        self.P = self.ks.shape[-2]
        self.rng = rng

    def device(self):
        return dict(K_packed=to_dev(self.kp), K_scale=to_dev_half(self.ks, self.meta),
                    K_mn=to_dev_half(self.km, self.meta), V_packed=to_dev(self.vp),
                    V_scale=to_dev_half(self.vs, self.meta), V_mn=to_dev_half(self.vm, self.meta))

    def q_dev(self):
        return to_dev_half(self.Q, self.dtype)[:, :, None, :]

    def oracle(self, page_mask):
        return O.sparse_int4_attention(self.Q, self.kp, self.ks, self.km, self.vp, self.vs, self.vm,
                                       page_mask, self.page)


def max_err(gpu: torch.Tensor, ref: np.ndarray) -> float:
    g = gpu.float().cpu().numpy()
    finite = np.isfinite(ref)
    assert np.array_equal(np.isfinite(g), finite), "finite/-inf pattern differs"
    if not finite.any():
        return 0.0
    return float(np.abs(g[finite] - ref[finite]).max())


class Int8Case:
    """Oracle-quantised INT8 cache (kv_quant.py:43-89) + query, host and device."""

    def __init__(self, seed, B=1, Hq=6, Hkv=2, S=1024, D=128, page=64, dtype="bf16", meta="bf16", outliers=True):
        rng = np.random.default_rng(seed)
        self.B, self.Hq, self.Hkv, self.S, self.D, self.page = B, Hq, Hkv, S, D, page
        self.dtype, self.meta = dtype, meta
        self.K, self.V = make_kv(rng, B, Hkv, S, D, dtype, outliers)
        self.Q = O.rounder(dtype)(rng.standard_normal((B, Hq, D)).astype(np.float32))
        self.ku, self.ks, self.km = O.quantize_k_int8(self.K, page, dtype, meta)
        self.vu, self.vs, self.vm = O.quantize_v_int8(self.V, meta)
        self.P = self.ks.shape[-2]

    def device(self):
        return dict(K_uint8=to_dev(self.ku), K_scale=to_dev_half(self.ks, self.meta),
                    K_mn=to_dev_half(self.km, self.meta), V_uint8=to_dev(self.vu),
                    V_scale=to_dev_half(self.vs, self.meta), V_mn=to_dev_half(self.vm, self.meta))

    def q_dev(self):
        return to_dev_half(self.Q, self.dtype)[:, :, None, :]


def fp64_selection_check(q, K_scale, K_mn, got_rows, retention, mode, num_sinks=4, window_pages=2, levels=15.0):
    """Selection against the exact (fp64) page scores, order-independently.

    The reference scores with torch matmuls (criticality.py:128-163) and picks
    with torch.topk (selection.py:103-117); neither fixes an fp32 summation
    order.  Any fp32 evaluation of a score differs from the exact value by at
    most tau = (D + 16) * 2^-24 * sum |terms| (every order of the D products,
    the head sum and the x15 scaling).  A row is *ambiguous* when some page
    inside the exact top-k and some page outside it lie within their taus of
    each other (the margin idea of scripts/profile_contribution.py:194-199,
    249): there the reference itself could pick either.  On every other row
    the selection is fixed by the mathematics, and the GPU must equal it.

    q (1, H_q, D); K_scale / K_mn (1, H_kv, P, D); got_rows: the GPU mask of
    the step, (1, H_q, P) (per-KV-head modes repeat the group's row).
    Returns the counts (rows, ambiguous, mismatched, ambiguous_differing): the
    last is how many ambiguous rows the GPU resolved differently from the
    fp64 top-k (informative only: either choice is within fp32 error).
    """
    q = np.asarray(q, np.float64)[0]
    sc = np.asarray(K_scale, np.float64)[0]
    mn = np.asarray(K_mn, np.float64)[0]
    Hq, D = q.shape
    Hkv, P = sc.shape[0], sc.shape[1]
    rep = Hq // Hkv
    qg = q.reshape(Hkv, rep, D)
    qp = np.maximum(qg, 0.0)
    s = qg @ np.swapaxes(mn, 1, 2) + levels * (qp @ np.swapaxes(sc, 1, 2))          # (Hkv, rep, P)
    a = np.abs(qg) @ np.swapaxes(np.abs(mn), 1, 2) + levels * (qp @ np.swapaxes(sc, 1, 2))
    got = np.asarray(got_rows)[0].reshape(Hkv, rep, P)
    if mode == "per_kv_head_sum":
        s, a, got = s.sum(1, keepdims=True), a.sum(1, keepdims=True), got[:, :1]
        if not np.isscalar(retention):      # a KV head's k: the largest retention of its query heads
            retention = np.asarray(retention, np.float32).reshape(Hkv, rep).max(1)
    s, a, got = s.reshape(-1, P), a.reshape(-1, P), got.reshape(-1, P)
    tau = (D + 16) * 2.0 ** -24 * a
    nrow = s.shape[0]
    k = O.k_per_head(retention, nrow, P) if not np.isscalar(retention) else O.k_per_head(retention, 1, P).repeat(nrow)
    forced = np.zeros(P, bool)
    forced[:min(num_sinks, P)] = True
    if window_pages > 0:
        forced[max(P - window_pages, 0):] = True
    amb = mis = amb_diff = 0
    for i in range(nrow):
        kk = int(k[i])
        order = np.argsort(-s[i], kind="stable")
        top = order[:kk]
        want = forced.copy()
        want[top] = True
        differs = not np.array_equal(want, got[i])
        if 0 < kk < P:
            rest = order[kk:]
            if np.min(s[i, top] - tau[i, top]) <= np.max(s[i, rest] + tau[i, rest]):
                amb += 1
                amb_diff += int(differs)
                continue
        mis += int(differs)
    return nrow, amb, mis, amb_diff


TOL_O = 2e-3      # decode output vs the fp32 oracle, max-abs


def decode_tol(ref_o, out_dtype="f16"):
    """Tolerance for a decode output of type out_dtype against the oracle.

    fp16 / fp32 output: the flat 2e-3 wherever the output type can hold it,
    i.e. max|O| <= 2 (fp16 rounds |O| < 2 by at most 2^-11 * 2 ~ 1e-3, which
    leaves 1e-3 for the kernel).  Larger outputs (the rescale stress cases
    reach |O| ~ 20) add the part of the fp16 rounding, 2^-11 |O|, beyond
    that 1e-3.  bf16 output (the reference's own output type) adds its
    rounding, 2^-8 |O|, which alone exceeds 2e-3 once |O| > 0.5.
    """
    m = float(np.abs(np.asarray(ref_o)).max()) if np.size(ref_o) else 0.0
    if out_dtype == "bf16":
        return TOL_O + 2.0 ** -8 * m
    if out_dtype == "f32":
        return TOL_O
    return TOL_O + max(0.0, 2.0 ** -11 * m - 1e-3)
