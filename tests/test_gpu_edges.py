"""Edge cases the reference's own tests pin, through this build's GPU path:

* a precomputed ``k_max_static`` selects exactly what the dynamic k does
  (tests/test_select_pages_static_kmax.py:13-45);
* a cache of a single page (tests/test_kernel_sparse_edges.py:98-115);
* a constant-valued channel (zero quantisation range) stays finite and
  matches the oracle (tests/test_kernel_sparse_edges.py:117-146);
* retention 0 with no forced pages attends nothing: O = 0 exactly
  (tests/test_eager_sparse_int8.py:56-75);
* the fused DuoAttention entry refuses prefill and a pattern of the wrong
  shape (tests/test_fused_dispatch.py:82-105).
"""
import math

import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import decode_tol, Int4Case, Int8Case, max_err, to_dev

pytestmark = pytest.mark.gpu


def _tol(dtype, ref_o):
    return decode_tol(ref_o, dtype)


@pytest.mark.parametrize("retention", [0.25, 0.5])
@pytest.mark.parametrize("P", [16, 64, 512])
def test_static_kmax_parity_with_dynamic(retention, P):
    from flashquest_amd.eager.selection import select_pages_vectorized
    g = torch.Generator().manual_seed(0)
    scores = torch.randn(1, 8, 1, P, generator=g).cuda()
    dyn = select_pages_vectorized(scores, retention=retention, num_sinks=4, window_pages=2)
    sta = select_pages_vectorized(scores, retention=retention, num_sinks=4, window_pages=2,
                                  k_max_static=math.ceil(retention * max(P, 512)))
    torch.cuda.synchronize()
    assert torch.equal(dyn, sta)
    ref = O.select_pages_vectorized(scores.cpu().numpy(), retention, 4, 2)
    assert np.array_equal(dyn.cpu().numpy(), ref)


def test_static_kmax_per_head_retention():
    from flashquest_amd.eager.selection import select_pages_vectorized
    g = torch.Generator().manual_seed(0)
    scores = torch.randn(1, 4, 1, 32, generator=g).cuda()
    r = torch.tensor([0.0, 0.25, 0.5, 1.0]).cuda()
    dyn = select_pages_vectorized(scores, retention=r, num_sinks=4, window_pages=2)
    sta = select_pages_vectorized(scores, retention=r, num_sinks=4, window_pages=2, k_max_static=32)
    torch.cuda.synchronize()
    assert torch.equal(dyn, sta)
    ref = O.select_pages_vectorized(scores.cpu().numpy(), r.cpu().numpy(), 4, 2)
    assert np.array_equal(dyn.cpu().numpy(), ref)


@pytest.mark.parametrize("D", [64, 128])
def test_single_page_int4_and_int8(D):
    from flashquest_amd.kernel import flash_attn_sparse_fwd, flash_attn_sparse_int4_fwd
    sel = np.ones((1, 1, 1), bool)
    c4 = Int4Case(seed=11, B=1, Hq=1, Hkv=1, S=64, D=D)
    ref_o, ref_l = c4.oracle(sel)
    o, lse = flash_attn_sparse_int4_fwd(c4.q_dev(), **c4.device(), selection_mask=to_dev(sel)[:, :, None, :])
    c8 = Int8Case(seed=12, B=1, Hq=1, Hkv=1, S=64, D=D)
    ref8_o, ref8_l = O.sparse_int8_attention(c8.Q, c8.ku, c8.ks, c8.km, c8.vu, c8.vs, c8.vm, sel, 64)
    o8, lse8 = flash_attn_sparse_fwd(c8.q_dev(), **c8.device(), selection_mask=to_dev(sel)[:, :, None, :])
    torch.cuda.synchronize()
    assert max_err(o[:, :, 0], ref_o) <= _tol("bf16", ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4
    assert max_err(o8[:, :, 0], ref8_o) <= _tol("bf16", ref8_o)
    assert max_err(lse8[:, :, 0], ref8_l) <= 1e-4


def test_zero_range_channel_is_finite_and_matches_oracle():
    from flashquest_amd.kernel import flash_attn_sparse_fwd, flash_attn_sparse_int4_fwd
    c = Int4Case(seed=21, B=1, Hq=2, Hkv=1, S=128, D=64)
    rnd = O.rounder("bf16")
    c.K[..., 5] = rnd(np.float32(0.7))
    c.V[..., 5] = rnd(np.float32(0.3))
    c.kp, c.ks, c.km = O.quantize_k_int4(c.K, 64, "bf16", "bf16")
    c.vp, c.vs, c.vm = O.quantize_v_int4(c.V, None, "bf16")
    assert np.all(c.ks[..., 5] <= 1e-6)         # zero range: the scale is the quantiser's floor
    sel = np.ones((1, 2, 2), bool)
    ref_o, ref_l = c.oracle(sel)
    o, lse = flash_attn_sparse_int4_fwd(c.q_dev(), **c.device(), selection_mask=to_dev(sel)[:, :, None, :])
    c8 = Int8Case(seed=22, B=1, Hq=2, Hkv=1, S=128, D=64)
    c8.K[..., 5] = rnd(np.float32(0.7))
    c8.V[..., 5] = rnd(np.float32(0.3))
    c8.ku, c8.ks, c8.km = O.quantize_k_int8(c8.K, 64, "bf16", "bf16")
    c8.vu, c8.vs, c8.vm = O.quantize_v_int8(c8.V, "bf16")
    ref8_o, _ = O.sparse_int8_attention(c8.Q, c8.ku, c8.ks, c8.km, c8.vu, c8.vs, c8.vm, sel, 64)
    o8, _ = flash_attn_sparse_fwd(c8.q_dev(), **c8.device(), selection_mask=to_dev(sel)[:, :, None, :])
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(o8).all()
    assert max_err(o[:, :, 0], ref_o) <= _tol("bf16", ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4
    assert max_err(o8[:, :, 0], ref8_o) <= _tol("bf16", ref8_o)


@pytest.mark.parametrize("bits", [4, 8])
def test_no_pages_selected_returns_zero(bits):
    from flashquest_amd.eager.decode import quest_decode_int4, quest_decode_int8
    if bits == 4:
        c = Int4Case(seed=31, B=1, Hq=1, Hkv=1, S=128, D=64)
        o, lse = quest_decode_int4(c.q_dev(), **c.device(), retention=0.0, num_sinks=0, window_pages=0)
    else:
        c = Int8Case(seed=32, B=1, Hq=1, Hkv=1, S=128, D=64)
        o, lse = quest_decode_int8(c.q_dev(), **c.device(), retention=0.0, num_sinks=0, window_pages=0)
    torch.cuda.synchronize()
    assert torch.equal(o, torch.zeros_like(o))
    assert torch.isneginf(lse).all()


def test_fused_duo_rejects_prefill_and_bad_pattern():
    from flashquest_amd.duo import quest_duo_fused_sdpa
    c = Int8Case(seed=41, B=1, Hq=4, Hkv=2, S=64, D=64)
    d = c.device()
    q8 = torch.randn(1, 4, 8, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NotImplementedError):
        quest_duo_fused_sdpa(q8, d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"], d["V_mn"],
                             head_pattern=torch.tensor([True, True]), page_size=64)
    with pytest.raises(ValueError, match="head_pattern"):
        quest_duo_fused_sdpa(c.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"],
                             d["V_mn"], head_pattern=torch.tensor([True, True, True]), page_size=64)


def test_random_shapes_match_oracle_decode():
    """A seeded grid of ragged shapes (tests/test_kernel_sparse_edges.py:149-183
    draws the same ranges with hypothesis): S_kv 64..512 tokens (partial last
    pages), 1-2 KV heads, 1/2/4 query heads each, D 64/128, retention
    0.25/0.5/1: the whole decode step (scores, selection, attention) against
    the oracle, selection bit-exact."""
    from flashquest_amd.eager.decode import quest_decode_int4, quest_decode_int8
    rng = np.random.default_rng(2024)
    for i in range(15):
        S = int(rng.integers(64, 513))
        Hkv = int(rng.choice([1, 2]))
        rep = int(rng.choice([1, 2, 4]))
        D = int(rng.choice([64, 128]))
        r = float(rng.choice([0.25, 0.5, 1.0]))
        kw = dict(retention=r, num_sinks=1, window_pages=1, return_selection=True)
        c = Int4Case(seed=900 + i, B=1, Hq=Hkv * rep, Hkv=Hkv, S=S, D=D)
        o, lse, mask = quest_decode_int4(c.q_dev(), **c.device(), **kw)
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=r, num_sinks=1, window_pages=1)
        c8 = Int8Case(seed=950 + i, B=1, Hq=Hkv * rep, Hkv=Hkv, S=S, D=D)
        o8, lse8, mask8 = quest_decode_int8(c8.q_dev(), **c8.device(), **kw)
        ref8 = O.decode_step(c8.Q, c8.ku, c8.ks, c8.km, c8.vu, c8.vs, c8.vm, retention=r, num_sinks=1,
                             window_pages=1, bits=8)
        torch.cuda.synchronize()
        case = (S, Hkv, rep, D, r)
        assert np.array_equal(mask.cpu().numpy(), ref["mask"]), case
        assert max_err(o[:, :, 0], ref["O"]) <= _tol("bf16", ref["O"]), case
        assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4, case
        assert np.array_equal(mask8.cpu().numpy(), ref8["mask"]), case
        assert max_err(o8[:, :, 0], ref8["O"]) <= _tol("bf16", ref8["O"]), case
        assert max_err(lse8[:, :, 0], ref8["lse"]) <= 1e-4, case


def test_strided_per_head_retention_matches_oracle():
    """A per-head retention that is a strided view of a longer device vector
    (every second entry) selects with those heads' values: each head's k
    follows its own retention, the mask equals the oracle's for the same
    values, INT4 and INT8."""
    from flashquest_amd.eager.decode import quest_decode_int4, quest_decode_int8
    Hkv, rep, S, D = 2, 3, 1024, 128
    Hq = Hkv * rep
    vals = np.array([0.1, 0.9, 0.25, 0.6, 0.4, 0.05], dtype=np.float32)
    wide = torch.zeros(2 * Hq, dtype=torch.float32, device="cuda")
    wide[::2] = torch.from_numpy(vals).cuda()
    wide[1::2] = 1.0                                   # the entries the view skips select everything
    r = wide[::2]
    assert not r.is_contiguous()
    kw = dict(retention=r, num_sinks=1, window_pages=1, return_selection=True)
    c = Int4Case(seed=77, B=1, Hq=Hq, Hkv=Hkv, S=S, D=D)
    o, lse, mask = quest_decode_int4(c.q_dev(), **c.device(), **kw)
    ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=vals, num_sinks=1, window_pages=1)
    c8 = Int8Case(seed=78, B=1, Hq=Hq, Hkv=Hkv, S=S, D=D)
    o8, lse8, mask8 = quest_decode_int8(c8.q_dev(), **c8.device(), **kw)
    ref8 = O.decode_step(c8.Q, c8.ku, c8.ks, c8.km, c8.vu, c8.vs, c8.vm, retention=vals, num_sinks=1,
                         window_pages=1, bits=8)
    torch.cuda.synchronize()
    P = S // 64
    m = mask.cpu().numpy()
    # per head: k = ceil(fp32(r) * P) selected pages plus the forced ones outside them
    for h in range(Hq):
        k = math.ceil(float(np.float32(vals[h]) * np.float32(P)))
        assert k <= m[0, h].sum() <= k + 2, (h, k, int(m[0, h].sum()))
    assert np.array_equal(m, ref["mask"])
    assert max_err(o[:, :, 0], ref["O"]) <= _tol("bf16", ref["O"])
    assert np.array_equal(mask8.cpu().numpy(), ref8["mask"])
    assert max_err(o8[:, :, 0], ref8["O"]) <= _tol("bf16", ref8["O"])
