"""Sparse INT4 decode attention: HIP kernels vs the CPU oracle (MI355X)."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import decode_tol, Int4Case, max_err, to_dev

pytestmark = pytest.mark.gpu

TOL_O = 2e-3      # fp16/bf16 output vs the fp32 oracle (plus output rounding, below)


def _tol(case, ref_o):
    return decode_tol(ref_o, case.dtype)


def _rand_mask(case, frac, rng):
    return rng.random((case.B, case.Hq, case.P)) < frac


@pytest.mark.parametrize("Hq,Hkv,D,page,dtype,meta,vgroup", [
    (6, 2, 128, 64, "bf16", "bf16", None),
    (24, 8, 128, 64, "f16", "f16", 32),
    (4, 2, 64, 32, "bf16", "bf16", None),
    (8, 1, 128, 16, "bf16", "bf16", None),
    (4, 4, 128, 64, "f16", "bf16", None),
    (8, 2, 64, 64, "bf16", "f16", 32),
    (16, 2, 128, 64, "f16", "f16", 32),    # 8 query heads per KV head: chunks of 4 on the matrix cores
    (10, 2, 128, 64, "bf16", "bf16", None),  # 5: chunks of 3 + 2
])
def test_mask_kernel_matches_oracle(Hq, Hkv, D, page, dtype, meta, vgroup):
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    case = Int4Case(seed=Hq * 100 + D + page, B=2, Hq=Hq, Hkv=Hkv, S=16 * page, D=D, page=page,
                    dtype=dtype, meta=meta, vgroup=vgroup)
    mask = _rand_mask(case, 0.3, case.rng)
    mask[0, 0] = False                 # one empty head -> O = 0, lse = -inf
    ref_o, ref_l = case.oracle(mask)
    t = case.device()
    o, lse = flash_attn_sparse_int4_fwd(case.q_dev(), **t, selection_mask=to_dev(mask)[:, :, None, :],
                                        page_size=page)
    torch.cuda.synchronize()
    assert o.dtype == case.q_dev().dtype and o.shape == (case.B, Hq, 1, D)
    assert max_err(o[:, :, 0], ref_o) <= _tol(case, ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4
    assert torch.all(o[0, 0] == 0) and torch.isneginf(lse[0, 0]).all()


def test_all_pages_is_dense_attention_and_partial_last_page():
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    case = Int4Case(seed=7, B=1, Hq=6, Hkv=2, S=64 * 9 + 17, D=128, page=64)
    mask = np.ones((1, 6, case.P), bool)
    ref_o, ref_l = case.oracle(mask)
    o, lse = flash_attn_sparse_int4_fwd(case.q_dev(), **case.device(), selection_mask=to_dev(mask)[:, :, None, :])
    assert max_err(o[:, :, 0], ref_o) <= _tol(case, ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4


def test_empty_mask_gives_exact_zero():
    # tests/test_kernel_sparse_basic.py:78-96
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    case = Int4Case(seed=3, S=512)
    mask = torch.zeros(1, 6, 1, case.P, dtype=torch.bool, device="cuda")
    o, lse = flash_attn_sparse_int4_fwd(case.q_dev(), **case.device(), selection_mask=mask)
    assert torch.all(o == 0) and torch.isneginf(lse).all()
    o2, l2 = flash_attn_sparse_int4_fwd(case.q_dev(), **case.device(), selection_mask=mask, return_lse=False)
    assert l2 is None and torch.all(o2 == 0)


def test_compact_ids_match_mask_kernel_and_padding_invariance():
    # tests/test_sparse_int4_fwd_compact_parity.py:10-48, _padding.py:30-68
    from flashquest_amd.eager import build_compact_selection
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd, flash_attn_sparse_int4_fwd_compact
    for seed in range(4):
        Hq = 64 if seed == 3 else 24     # the last case: 8 query heads per KV head, attended in chunks
        case = Int4Case(seed=40 + seed, B=1, Hq=Hq, Hkv=8, S=64 * 32, D=128)
        mask = to_dev(_rand_mask(case, 0.25, case.rng))[:, :, None, :]
        t = case.device()
        o_m, l_m = flash_attn_sparse_int4_fwd(case.q_dev(), **t, selection_mask=mask)
        for bucket in (case.P, case.P + 7):
            ids = build_compact_selection(mask, bucket)
            o_c, l_c = flash_attn_sparse_int4_fwd_compact(case.q_dev(), **t, selected_page_ids=ids)
            assert torch.equal(o_c, o_m) and torch.equal(l_c, l_m)
    sent = torch.full((1, Hq, 1, 8), -1, dtype=torch.int32, device="cuda")
    o, lse = flash_attn_sparse_int4_fwd_compact(case.q_dev(), **t, selected_page_ids=sent)
    assert torch.all(o == 0) and torch.isneginf(lse).all()


def test_out_of_range_ids_are_skipped():
    # tests/test_sparse_compact_kernel_address_safety.py:7-33
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd, flash_attn_sparse_int4_fwd_compact
    case = Int4Case(seed=5, B=1, Hq=4, Hkv=2, S=64 * 8, D=128)
    t = case.device()
    ids = torch.tensor([[3, -1, 99999, -7, 5]] * 4, dtype=torch.int32, device="cuda")[None]
    mask = torch.zeros(1, 4, 1, case.P, dtype=torch.bool, device="cuda")
    mask[..., 3] = True
    mask[..., 5] = True
    o_c, l_c = flash_attn_sparse_int4_fwd_compact(case.q_dev(), **t, selected_page_ids=ids)
    o_m, l_m = flash_attn_sparse_int4_fwd(case.q_dev(), **t, selection_mask=mask)
    assert torch.equal(o_c, o_m) and torch.equal(l_c, l_m)


def test_wrapper_errors_match_reference():
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    case = Int4Case(seed=1, S=256)
    t = case.device()
    mask = torch.ones(1, 6, 1, case.P, dtype=torch.bool, device="cuda")
    with pytest.raises(NotImplementedError):
        flash_attn_sparse_int4_fwd(case.q_dev().expand(1, 6, 2, 128), **t, selection_mask=mask)
    with pytest.raises(AssertionError):
        flash_attn_sparse_int4_fwd(case.q_dev(), **t, selection_mask=mask.int())


@pytest.mark.parametrize("mode", ["per_q_head", "per_kv_head_sum"])
@pytest.mark.parametrize("Hq,Hkv,P,retention,sinks,window,kmax", [
    (24, 8, 128, 0.20, 4, 2, None),
    (6, 2, 64, 0.25, 1, 1, 16),
    (8, 2, 40, 0.5, 0, 0, None),
    (4, 1, 300, 0.07, 4, 2, None),
])
def test_fused_decode_selection_bit_exact(mode, Hq, Hkv, P, retention, sinks, window, kmax):
    from flashquest_amd.eager import quest_decode_int4
    case = Int4Case(seed=P + Hq, B=2, Hq=Hq, Hkv=Hkv, S=P * 64, D=128)
    ref = O.decode_step(case.Q, case.kp, case.ks, case.km, case.vp, case.vs, case.vm, retention=retention,
                        num_sinks=sinks, window_pages=window, mode=mode, k_max_static=kmax)
    o, lse, mask = quest_decode_int4(case.q_dev(), **case.device(), retention=retention, num_sinks=sinks,
                                     window_pages=window, k_max_static=kmax, select_mode=mode,
                                     return_selection=True)
    torch.cuda.synchronize()
    assert np.array_equal(mask.cpu().numpy(), ref["mask"])
    assert max_err(o[:, :, 0], ref["O"]) <= _tol(case, ref["O"])
    assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4


def test_fused_decode_layers_are_independent():
    from flashquest_amd.eager import quest_decode_int4
    cases = [Int4Case(seed=90 + i, B=1, Hq=6, Hkv=2, S=64 * 48, D=128) for i in range(3)]
    dev = [c.device() for c in cases]
    stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
    q = torch.stack([c.q_dev() for c in cases])
    o, lse = quest_decode_int4(q, **stacked, retention=0.25, num_sinks=4, window_pages=2)
    for i, c in enumerate(cases):
        o1, l1 = quest_decode_int4(c.q_dev(), **dev[i], retention=0.25, num_sinks=4, window_pages=2)
        assert torch.equal(o[i], o1) and torch.equal(lse[i], l1)


def test_retention_vector_and_zero_heads():
    from flashquest_amd.eager import quest_decode_int4
    case = Int4Case(seed=11, B=1, Hq=6, Hkv=2, S=64 * 64, D=128)
    r = np.array([0.0, 0.25, 1.0, 0.1, 0.0, 0.5], np.float32)
    ref = O.decode_step(case.Q, case.kp, case.ks, case.km, case.vp, case.vs, case.vm, retention=r,
                        num_sinks=2, window_pages=1)
    o, lse, mask = quest_decode_int4(case.q_dev(), **case.device(), retention=torch.from_numpy(r),
                                     num_sinks=2, window_pages=1, return_selection=True)
    assert np.array_equal(mask.cpu().numpy(), ref["mask"])
    assert max_err(o[:, :, 0], ref["O"]) <= _tol(case, ref["O"])
