"""Matrix-core INT4 attention (head_dim 128, 64-token pages): the paths that only
show with many pages per wave, compared with the CPU oracle (MI355X).

The kernel keeps p.v in int32 against a running softmax maximum and V-scale
bound and rescales when a page exceeds either; these cases force such events on
every page (growing logits, growing V scales), none after the first (shrinking),
waves without pages, a partial last page, and every supported query-head ratio
and V grouping.  Splits per KV group are pinned so each wave gets many pages.
"""
import numpy as np
import pytest
import torch

from flashquest_amd import _lib as L
from oracle import fq_oracle as O
from tests.cases import decode_tol, Int4Case, max_err, to_dev

pytestmark = pytest.mark.gpu

TOL_O = 2e-3


def _tol(case, ref_o):
    return decode_tol(ref_o, case.dtype)


def _requantise(case):
    case.kp, case.ks, case.km = O.quantize_k_int4(case.K, case.page, case.dtype, case.meta)
    case.vp, case.vs, case.vm = O.quantize_v_int4(case.V, case.vgroup, case.meta)


def _ramp(case, direction, v_growth):
    """Page p's keys lean towards each KV head's mean query by an amount that
    grows (direction +1) or shrinks (-1) with p; V is scaled by v_growth**p."""
    rnd = O.rounder(case.dtype)
    nrep = case.Hq // case.Hkv
    qdir = case.Q.reshape(case.B, case.Hkv, nrep, case.D).mean(2)
    qdir /= np.linalg.norm(qdir, axis=-1, keepdims=True)
    P, page = case.P, case.page
    for p in range(P):
        frac = p / max(P - 1, 1)
        a = 6.0 * (frac if direction > 0 else 1.0 - frac)
        sl = slice(p * page, min((p + 1) * page, case.S))
        case.K[:, :, sl] = rnd(case.K[:, :, sl] * 0.5 + a * qdir[:, :, None, :])
        case.V[:, :, sl] = rnd(case.V[:, :, sl] * np.float32(v_growth ** p))
    _requantise(case)


def _run(case, mask, splits):
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    with L.attention_splits(splits):
        o, lse = flash_attn_sparse_int4_fwd(case.q_dev(), **case.device(),
                                            selection_mask=to_dev(mask)[:, :, None, :])
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("direction,v_growth", [(1, 1.08), (-1, 1.0), (1, 0.93)])
@pytest.mark.parametrize("splits", [1, 3])
def test_rescale_events_on_every_page(direction, v_growth, splits):
    case = Int4Case(seed=40 + splits, B=1, Hq=6, Hkv=2, S=64 * 64, D=128, page=64, dtype="f16", meta="f16",
                    vgroup=32)
    _ramp(case, direction, v_growth)
    mask = np.ones((1, 6, case.P), bool)
    ref_o, ref_l = case.oracle(mask)
    o, lse = _run(case, mask, splits)
    assert max_err(o[:, :, 0], ref_o) <= _tol(case, ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4


@pytest.mark.parametrize("Hq,Hkv", [(2, 2), (4, 2), (12, 4), (8, 2)])
@pytest.mark.parametrize("vgroup,meta", [(None, "bf16"), (32, "f16"), (32, "bf16")])
def test_head_ratios_groups_partial_page(Hq, Hkv, vgroup, meta):
    case = Int4Case(seed=Hq * 7 + Hkv + (vgroup or 0), B=2, Hq=Hq, Hkv=Hkv, S=64 * 40 + 33, D=128, page=64,
                    dtype="bf16", meta=meta, vgroup=vgroup)
    mask = case.rng.random((2, Hq, case.P)) < 0.5
    mask[:, :, -1] = True                 # the partial last page is always in
    mask[1, 0] = False                    # an empty head
    ref_o, ref_l = case.oracle(mask)
    for splits in (1, 0):
        o, lse = _run(case, mask, splits)
        assert max_err(o[:, :, 0], ref_o) <= _tol(case, ref_o), splits
        assert max_err(lse[:, :, 0], ref_l) <= 1e-4, splits


def test_waves_without_pages_and_empty_groups():
    case = Int4Case(seed=5, B=2, Hq=6, Hkv=2, S=64 * 24, D=128, page=64, dtype="f16", meta="f16", vgroup=32)
    mask = np.zeros((2, 6, case.P), bool)
    mask[0, 0, 5] = True                  # one page in the group: three idle waves
    mask[0, 4, [1, 9]] = True             # two pages, other group
    mask[1, :3, 7] = True                 # same page for all heads of a group
    ref_o, ref_l = case.oracle(mask)      # group (1, head 1) is empty
    for splits in (1, 2, 0):
        o, lse = _run(case, mask, splits)
        assert max_err(o[:, :, 0], ref_o) <= _tol(case, ref_o), splits
        assert max_err(lse[:, :, 0], ref_l) <= 1e-4, splits


def test_split_override_is_restored_and_validated():
    assert L.lib().fq_set_attention_splits(-1) != 0
    with L.attention_splits(2):
        pass
    case = Int4Case(seed=9, B=1, Hq=6, Hkv=2, S=64 * 8, D=128, page=64)
    mask = np.ones((1, 6, case.P), bool)
    ref_o, _ = case.oracle(mask)
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    o, _ = flash_attn_sparse_int4_fwd(case.q_dev(), **case.device(), selection_mask=to_dev(mask)[:, :, None, :])
    assert max_err(o[:, :, 0], ref_o) <= _tol(case, ref_o)


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
@pytest.mark.parametrize("want_mask", [False, True])
@pytest.mark.parametrize("sinks,window,P", [(3, 2, 24), (0, 0, 24), (4, 2, 5), (9, 1, 12), (1, 30, 20)])
def test_fused_decode_selecting_inside_attention(mode, want_mask, sinks, window, P):
    # >= 192 KV groups: one workgroup per group, which selects its own pages from the
    # scores (no selection kernel unless the mask is requested); a partial last page.
    # The forced pages go first in the workgroup's list and are loaded before the
    # selection: none, sinks overlapping the window, forced pages covering every page.
    from flashquest_amd.eager import quest_decode_int4
    L_, Hq, Hkv = 24, 24, 8
    cases = [Int4Case(seed=300 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * (P - 1) + 40, D=128, page=64, dtype="f16",
                      meta="f16", vgroup=32) for i in range(L_)]
    r = np.linspace(0.05, 0.6, Hq).astype(np.float32)
    dev = [c.device() for c in cases]
    stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
    q = torch.stack([c.q_dev() for c in cases])
    out = quest_decode_int4(q, **stacked, retention=torch.from_numpy(r), num_sinks=sinks, window_pages=window,
                            k_max_static=12, select_mode=mode, return_selection=want_mask)
    torch.cuda.synchronize()
    o, lse = out[0], out[1]
    for i, c in enumerate(cases):
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=r, num_sinks=sinks,
                            window_pages=window, mode=mode, k_max_static=12)
        if want_mask:
            assert np.array_equal(out[2][i].cpu().numpy(), ref["mask"]), i
        assert max_err(o[i][:, :, 0], ref["O"]) <= _tol(c, ref["O"]), i
        assert max_err(lse[i][:, :, 0], ref["lse"]) <= 1e-4, i


@pytest.mark.parametrize("mode", ["per_q_head", "per_kv_head_sum"])
def test_fused_decode_ties_take_the_lower_pages(mode):
    # Pages 6.. share one K scale/min (so their scores tie exactly) but not their
    # codes: the top-k boundary cuts through the tie, and the in-kernel selection
    # must keep the lower page indices (selection.py's order), which the output shows.
    from flashquest_amd.eager import quest_decode_int4
    L_, Hq, Hkv, P = 24, 24, 8, 48
    cases = []
    for i in range(L_):
        c = Int4Case(seed=700 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128, page=64, dtype="bf16", meta="bf16")
        c.ks[:, :, 6:, :] = c.ks[:, :, 6:7, :]
        c.km[:, :, 6:, :] = c.km[:, :, 6:7, :]
        cases.append(c)
    r = np.full(Hq, 0.3, np.float32)
    dev = [c.device() for c in cases]
    stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
    q = torch.stack([c.q_dev() for c in cases])
    o, lse = quest_decode_int4(q, **stacked, retention=torch.from_numpy(r), num_sinks=1, window_pages=1,
                               select_mode=mode)
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=r, num_sinks=1,
                            window_pages=1, mode=mode)
        assert max_err(o[i][:, :, 0], ref["O"]) <= _tol(c, ref["O"]), i
        assert max_err(lse[i][:, :, 0], ref["lse"]) <= 1e-4, i


def test_fused_decode_is_deterministic():
    # One workgroup per KV group, each wave a fixed set of pages and a fixed
    # merge order: repeated calls are bit-identical, and match the oracle.
    from flashquest_amd.eager import quest_decode_int4
    L_, Hq, Hkv, P = 24, 24, 8, 40
    cases = [Int4Case(seed=900 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P - 23, D=128, page=64, dtype="bf16", meta="f16",
                      vgroup=32) for i in range(L_)]
    dev = [c.device() for c in cases]
    stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
    q = torch.stack([c.q_dev() for c in cases])
    outs = [quest_decode_int4(q, **stacked, retention=0.5, num_sinks=2, window_pages=1, select_mode="per_q_head")
            for _ in range(3)]
    torch.cuda.synchronize()
    for o, lse in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(lse, outs[0][1])
    o, lse = outs[0]
    for i, c in enumerate(cases):
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=0.5, num_sinks=2,
                            window_pages=1, mode="per_q_head")
        assert max_err(o[i][:, :, 0], ref["O"]) <= _tol(c, ref["O"]), i
        assert max_err(lse[i][:, :, 0], ref["lse"]) <= 1e-4, i
