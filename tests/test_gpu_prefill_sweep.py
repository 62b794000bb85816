"""A seeded sweep of prefill over the packed cache against the oracle.

Each draw picks batch 1-2, 1-4 KV heads with 1-8 query heads each, page size
32 / 64 / 128, 0 to 32 completed pages, a bf16 tail of 0 to page-1 tokens,
a query count from 1 to all keys, the causal alignment (torch's upper-left
is_causal, or the chunk form causal_offset = S_kv - S_q), INT4 or INT8
codes, bf16 or fp16 metadata and (INT4) per-token or 32-channel V groups.
Between them the draws reach the register-staged short path, the two-pass
dense path and its key-range splits with the merge launch
(llama_persistent_patch.py:196-201 is the reference's prefill call; the
oracle dequantises, concatenates the tail and runs causal attention).
Every draw is printed before it runs, so a failure names its case.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.test_gpu_prefill import ATOL, PrefillCase

pytestmark = pytest.mark.gpu

N_DRAWS = 20


def _draw(rng, bits):
    page = int(rng.choice([32, 64, 64, 128]))
    n_pages = int(rng.choice([0, 1, 3, 9, 17, 32]))
    S = page * n_pages
    T = int(rng.integers(0, page))
    if S + T == 0:
        T = 1
    keys = S + T
    Sq = int(rng.choice([1, 7, 64, 200, keys]))
    Sq = max(1, min(Sq, keys))
    chunk = bool(rng.random() < 0.6)
    Hkv = int(rng.choice([1, 2, 4]))
    return dict(
        B=int(rng.choice([1, 2])), Hkv=Hkv, Hq=Hkv * int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8])), S=S, T=T, Sq=Sq,
        page=page, bits=bits, meta=str(rng.choice(["bf16", "f16"])),
        vgroup=(None if bits == 8 or rng.random() < 0.5 else 32),
        causal_offset=keys - Sq if chunk else 0,
    )


@pytest.mark.parametrize("bits", [4, 8])
def test_random_prefills_match_oracle(bits):
    rng = np.random.default_rng(77 + bits)
    for i in range(N_DRAWS):
        d = _draw(rng, bits)
        print(f"[prefill sweep] int{bits} draw {i}: {d}", flush=True)
        case = PrefillCase(6000 + 100 * bits + i, **d)
        out = case.run()
        torch.cuda.synchronize()
        ref = case.oracle()
        g = out.float().cpu().numpy()
        assert g.shape == ref.shape, d
        assert np.isfinite(g).all(), d
        err = float(np.abs(g - ref).max())
        assert err < ATOL, (err, d)
