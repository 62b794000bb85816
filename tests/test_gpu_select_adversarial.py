"""Page selection on adversarial score sets, through the whole decode step.

The selection inside the attention kernels (and the standalone group
selection of split steps) finds the k-th largest score by one wave's radix
search over 8-bit digits of the sortable key, skipping the bits every key
shares.  Scores here are made to stress exactly that: every page equal, two
distinct values, a block of ties straddling the k-th place, magnitudes
spread over 2^-20..2^2, and sign changes (keys on both sides of the float sign
bit).  Each set is written into the K page metadata, so the oracle
(oracle/fq_oracle.py: page_scores_fixed, the reference's selection rule with
ties to the lower page) scores the same pages; the selection must match bit
for bit and O, lse within the decode tolerance.  Both paths are covered:
two KV groups (split step, standalone group selection) and 192 groups (the
single-launch kernel that selects inside the attention workgroup).
"""
import zlib

import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import Int4Case, max_err

pytestmark = pytest.mark.gpu


def _shape_scores(case, pattern, rng):
    """Rewrite the K page metadata (B, Hkv, P, D) so the page scores follow `pattern`."""
    ks, km = case.ks.copy(), case.km.copy()
    B, H, P, D = ks.shape
    for b in range(B):
        for h in range(H):
            if pattern == "all_equal":
                ks[b, h] = ks[b, h, 0]
                km[b, h] = km[b, h, 0]
            elif pattern == "two_values":
                src = np.where(np.arange(P) % 3 == 0, 0, 1)
                ks[b, h] = ks[b, h, src]
                km[b, h] = km[b, h, src]
            elif pattern == "tie_block":
                # a third of the pages share one page's metadata, the rest random:
                # the k-th place falls inside the tie block for these retentions
                idx = rng.choice(P, P // 3, replace=False)
                ks[b, h, idx] = ks[b, h, idx[0]]
                km[b, h, idx] = km[b, h, idx[0]]
            elif pattern == "wide_exponents":
                # keys spread over 22 binades; pages are only scaled down (or up
                # by at most 4x) so the attention logits stay well conditioned
                e = rng.integers(-20, 3, P).astype(np.float32)
                f = np.exp2(e)[:, None]
                ks[b, h] = ks[b, h] * f
                km[b, h] = km[b, h] * f
            elif pattern == "sign_mix":
                # flip the sign of min for some pages and scale: scores land on
                # both sides of zero
                neg = rng.random(P) < 0.5
                km[b, h, neg] = -np.abs(km[b, h, neg]) * 4.0
                ks[b, h, neg] = ks[b, h, neg] * 0.25
    rnd = O.rounder(case.meta)
    case.ks, case.km = rnd(ks.astype(np.float32)), rnd(km.astype(np.float32))


PATTERNS = ["all_equal", "two_values", "tie_block", "wide_exponents", "sign_mix"]


@pytest.mark.parametrize("pattern", PATTERNS)
@pytest.mark.parametrize("B,retention,mode", [(1, 0.25, "per_kv_head_sum"), (1, 0.5, "per_q_head"),
                                              (96, 0.25, "per_kv_head_sum"), (96, 0.3, "per_q_head")])
def test_selection_on_adversarial_scores(pattern, B, retention, mode):
    from flashquest_amd.eager.decode import quest_decode_int4
    rng = np.random.default_rng(zlib.crc32(f"{pattern}/{B}/{mode}".encode()))
    case = Int4Case(seed=int(rng.integers(1 << 30)), B=B, Hq=6, Hkv=2, S=64 * 64, D=128)
    _shape_scores(case, pattern, rng)
    o, lse, mask = quest_decode_int4(case.q_dev(), **case.device(), retention=retention, num_sinks=2,
                                     window_pages=1, select_mode=mode, return_selection=True)
    ref = O.decode_step(case.Q, case.kp, case.ks, case.km, case.vp, case.vs, case.vm, retention=retention,
                        num_sinks=2, window_pages=1, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(mask.cpu().numpy(), ref["mask"]), (pattern, B, mode)
    tol = 2e-3 + 2.0 ** -8 * float(np.abs(ref["O"]).max())
    assert max_err(o[:, :, 0], ref["O"]) <= tol
    assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4 * max(1.0, float(np.abs(ref["lse"][np.isfinite(ref["lse"])]).max()))


@pytest.mark.parametrize("pattern", PATTERNS)
@pytest.mark.parametrize("P,mode,Hq", [(1000, "per_q_head", 6), (2048, "per_q_head", 6), (1000, "per_kv_head_sum", 6),
                                       (700, "per_q_head", 16)])
def test_selection_on_adversarial_scores_long(pattern, P, mode, Hq):
    """Long steps (more than 512 pages) take the standalone group selection of
    up to 2048 pages: per query head, one wave per row of the group (two rows
    per wave at 8 query heads per KV head)."""
    from flashquest_amd.eager.decode import quest_decode_int4
    rng = np.random.default_rng(zlib.crc32(f"long/{pattern}/{P}/{mode}/{Hq}".encode()))
    case = Int4Case(seed=int(rng.integers(1 << 30)), B=1, Hq=Hq, Hkv=2, S=64 * P, D=128)
    _shape_scores(case, pattern, rng)
    for return_selection in (True, False):
        res = quest_decode_int4(case.q_dev(), **case.device(), retention=0.3, num_sinks=2, window_pages=1,
                                select_mode=mode, return_selection=return_selection)
        ref = O.decode_step(case.Q, case.kp, case.ks, case.km, case.vp, case.vs, case.vm, retention=0.3,
                            num_sinks=2, window_pages=1, mode=mode)
        torch.cuda.synchronize()
        if return_selection:
            assert np.array_equal(res[2].cpu().numpy(), ref["mask"]), (pattern, P, mode)
        o, lse = res[0], res[1]
        tol = 2e-3 + 2.0 ** -8 * float(np.abs(ref["O"]).max())
        assert max_err(o[:, :, 0], ref["O"]) <= tol
        assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4 * max(1.0, float(np.abs(ref["lse"][np.isfinite(ref["lse"])]).max()))
