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
