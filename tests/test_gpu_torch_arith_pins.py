"""The oracle's restatement of torch arithmetic, checked against torch itself
executing the same operations on the GPU.

The reference's quantisers, selection and turbo codebook search are torch
operations on CUDA tensors (src/flashquest/kernel/kv_quant.py:131-215,
240-250; src/flashquest/eager/selection.py:103-117).  torch on this GPU runs
the same ATen kernels, so running the operation here pins the rule the oracle
(oracle/fq_oracle.py) uses for it:

  * ``half_tensor / 15.0`` (and ``/ 255.0``): a multiply by the fp32
    reciprocal of the scalar, rounded to the tensor's dtype (exhaustive over
    every finite bf16 and fp16 value);
  * ``fp32_tensor / fp32_tensor``: IEEE fp32 division;
  * ``round``: round half to even; ``clamp_min(1e-6)`` on half tensors:
    half(max(float(x), 1e-6));
  * ``argmin`` over |x - codebook|: ties to the lower index
    (oracle.quantize_to_codebook, kv_quant.py:240-250);
  * ``topk(k_max)`` then rank < k: among scores tied with the k-th largest,
    the lower page indices (oracle.select_pages_vectorized, selection.py:
    103-117), with k_max = k and k_max = P.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fq_oracle as O

pytestmark = pytest.mark.gpu

_TORCH = {"bf16": torch.bfloat16, "f16": torch.float16}


def _all_finite(dtype: str) -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = O.from_bits(bits, dtype)
    return x[np.isfinite(x)].astype(np.float32)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("divisor,inv", [(15.0, O.INV15), (255.0, O.INV255)])
def test_half_tensor_divided_by_python_scalar(dtype, divisor, inv):
    x = _all_finite(dtype)
    got = (torch.from_numpy(x).to("cuda", _TORCH[dtype]) / divisor).float().cpu().numpy()
    want = O.rounder(dtype)(x * np.float32(inv))
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all(), (x[~same][:8], got[~same][:8], want[~same][:8])


def test_fp32_tensor_division_is_ieee():
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(1 << 20) * np.exp(rng.uniform(-20, 20, 1 << 20))).astype(np.float32)
    b = (rng.standard_normal(1 << 20) * np.exp(rng.uniform(-20, 20, 1 << 20))).astype(np.float32)
    got = (torch.from_numpy(a).cuda() / torch.from_numpy(b).cuda()).cpu().numpy()
    assert np.array_equal(got, a / b)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_round_and_half_clamp(dtype):
    halves = (np.arange(-40, 41, dtype=np.float32) + np.float32(0.5))
    got = torch.from_numpy(halves).cuda().round().cpu().numpy()
    assert np.array_equal(got, np.rint(halves))
    x = _all_finite(dtype)
    x = x[np.abs(x) < 1e-4]
    got = torch.from_numpy(x).to("cuda", _TORCH[dtype]).clamp_min(1e-6).float().cpu().numpy()
    want = O.rounder(dtype)(np.maximum(x, np.float32(1e-6)))
    assert np.array_equal(got, want)


def test_codebook_argmin_ties_take_the_lower_index():
    cb = O.TURBO_CODEBOOK
    # fp32 values whose distances to two neighbouring codepoints are equal in
    # fp32 arithmetic, plus ordinary values around every midpoint
    xs = []
    for i in range(len(cb) - 1):
        lo = hi = np.float32((np.float64(cb[i]) + np.float64(cb[i + 1])) / 2)
        xs.append(lo)
        for _ in range(64):                  # 64 fp32 steps either side of the midpoint
            lo = np.nextafter(lo, np.float32(-np.inf))
            hi = np.nextafter(hi, np.float32(np.inf))
            xs += [lo, hi]
    x = np.array(xs, dtype=np.float32)
    d = np.abs(x[:, None] - cb[None, :])
    ties = (np.sort(d, axis=1)[:, 0] == np.sort(d, axis=1)[:, 1]).sum()
    assert ties > 0, "no exact ties constructed"
    xt, ct = torch.from_numpy(x).cuda(), torch.from_numpy(cb).cuda()
    got = (xt.unsqueeze(-1) - ct).abs().argmin(dim=-1).cpu().numpy()
    assert np.array_equal(got, O.quantize_to_codebook(x))


@pytest.mark.parametrize("P,k,levels", [(64, 16, 2), (128, 26, 4), (512, 128, 8), (512, 128, 300), (2048, 512, 16)])
def test_topk_ties_take_the_lower_pages(P, k, levels):
    rng = np.random.default_rng(P + k + levels)
    scores = rng.integers(0, levels, size=(16, P)).astype(np.float32)      # heavy ties at the k-th value
    r = np.float32((k - 0.5) / P)                                         # fp32 ceil(r * P) = k
    want = O.select_pages_vectorized(scores[:, None, None, :], r, 0, 0)[:, 0, 0, :]
    st = torch.from_numpy(scores).cuda()
    for k_max in (k, P):
        idx = st.topk(k_max, dim=-1).indices[:, :k]
        got = torch.zeros_like(st, dtype=torch.bool).scatter_(1, idx, True).cpu().numpy()
        assert np.array_equal(got, want), (P, k, levels, k_max)
