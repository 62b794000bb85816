"""A wide seeded sweep of the whole decode step (scores, selection, sparse
attention) against the oracle, INT4 and INT8.

Each draw picks batch 1-3, 1-4 KV heads with 1-8 query heads each, head_dim
64 or 128, 1 to 1024 pages of 64 tokens with a partial last page, bf16 or
fp16 queries with bf16 or fp16 metadata, per-token or 32-channel V groups
(INT4 only: INT8 V metadata is per token), either selection mode, sink and window counts from 0 to past the page
count, a static k_max or none, and a retention in (0, 1]
(tests/test_kernel_sparse_edges.py:149-183 draws ragged shapes the same way
with hypothesis; selection.py:65-126 and sparse_int4_fwd.py / sparse_int8_fwd.py
are the operators).  The selection must equal the oracle's bit for bit, O must
be within the decode tolerance (a flat 2e-3 for fp16 output) and lse within
1e-4.  Every draw is printed before it runs, so a failure names its case.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import Int4Case, Int8Case, decode_tol, max_err

pytestmark = pytest.mark.gpu

N_DRAWS = 24


def _draw(rng):
    Hkv = int(rng.choice([1, 2, 4]))
    rep = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8]))
    P = int(rng.choice([1, 2, 7, 40, 41, 129, 300, 512, 700, 1024]))
    S = max(1, 64 * (P - 1) + int(rng.integers(1, 65)))
    return dict(
        B=int(rng.choice([1, 2, 3])), Hkv=Hkv, Hq=Hkv * rep, D=int(rng.choice([64, 128, 128])), S=S,
        dtype=str(rng.choice(["bf16", "f16"])), meta=str(rng.choice(["bf16", "f16"])),
        vgroup=(None if rng.random() < 0.5 else 32),
        mode=str(rng.choice(["per_q_head", "per_kv_head_sum"])),
        sinks=int(rng.choice([0, 1, 4, 2000])), window=int(rng.choice([0, 1, 2, 2000])),
        retention=float(rng.choice([0.05, 0.2, 0.25, 0.5, 0.9, 1.0])),
        kmax=(None if rng.random() < 0.6 else int(rng.integers(1, P + 1))),
    )


def _check(tag, draw, o, lse, mask, ref):
    torch.cuda.synchronize()
    assert np.array_equal(mask.cpu().numpy(), ref["mask"]), (tag, draw)
    tol = decode_tol(ref["O"], draw["dtype"])
    assert max_err(o[:, :, 0], ref["O"]) <= tol, (tag, draw)
    assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4, (tag, draw)


@pytest.mark.parametrize("bits", [4, 8])
def test_random_decode_steps_match_oracle(bits):
    from flashquest_amd.eager.decode import quest_decode_int4, quest_decode_int8
    rng = np.random.default_rng(31 + bits)
    for i in range(N_DRAWS):
        d = _draw(rng)
        print(f"[sweep] int{bits} draw {i}: {d}", flush=True)
        kw = dict(retention=d["retention"], num_sinks=d["sinks"], window_pages=d["window"],
                  k_max_static=d["kmax"], select_mode=d["mode"], return_selection=True)
        ref_kw = dict(retention=d["retention"], num_sinks=d["sinks"], window_pages=d["window"],
                      k_max_static=d["kmax"], mode=d["mode"])
        seed = 5000 + 100 * bits + i
        if bits == 4:
            c = Int4Case(seed=seed, B=d["B"], Hq=d["Hq"], Hkv=d["Hkv"], S=d["S"], D=d["D"], dtype=d["dtype"],
                         meta=d["meta"], vgroup=d["vgroup"])
            o, lse, mask = quest_decode_int4(c.q_dev(), **c.device(), **kw)
            ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, **ref_kw)
        else:
            c = Int8Case(seed=seed, B=d["B"], Hq=d["Hq"], Hkv=d["Hkv"], S=d["S"], D=d["D"], dtype=d["dtype"],
                         meta=d["meta"])
            o, lse, mask = quest_decode_int8(c.q_dev(), **c.device(), **kw)
            ref = O.decode_step(c.Q, c.ku, c.ks, c.km, c.vu, c.vs, c.vm, bits=8, **ref_kw)
        _check(f"int{bits} draw {i}", d, o, lse, mask, ref)
