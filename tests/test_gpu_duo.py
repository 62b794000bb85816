"""DuoAttention head patterns (src/flashquest/duo/, llama_persistent_patch.py:214-220)
through the fused decode, against the oracle: streaming KV heads select
exactly the sink and window pages, retrieval heads the top-k of their scores,
and attention follows the selection.  A (layers, KV heads) pattern in one
multi-layer call gives each layer its own retention row (the single-launch
kernel and the split path agree bit for bit on the selection)."""
import math

import numpy as np
import pytest
import torch

from flashquest_amd import _lib as L
from oracle import fq_oracle as O
from tests.cases import decode_tol, Int4Case, Int8Case, max_err

pytestmark = pytest.mark.gpu


def _forced(P, sinks, window):
    f = np.zeros(P, bool)
    f[:min(sinks, P)] = True
    f[P - min(window, P):] = True
    return f


def _retention_rows(pattern, r, nrep):
    return np.where(np.repeat(pattern, nrep, axis=-1), np.float32(r), np.float32(0))


@pytest.mark.parametrize("mode", ["per_q_head", "per_kv_head_sum"])
@pytest.mark.parametrize("splits", [None, 4])
@pytest.mark.parametrize("Hq", [24, 64])
def test_layer_patterns_in_one_multilayer_call(mode, splits, Hq):
    """Hq = 64: 8 query heads per KV head, two virtual KV heads per KV head in
    the single launch, each reading its layer's retention row."""
    from flashquest_amd.eager.decode import quest_decode_int4
    Lyr, Hkv, P = 24, 8, 40          # 192 groups: the single-launch kernel unless splits are pinned
    rng = np.random.default_rng(123)
    cases = [Int4Case(seed=500 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128, meta="f16", vgroup=32, dtype="f16")
             for i in range(Lyr)]
    pattern = rng.random((Lyr, Hkv)) < 0.5
    pattern[0] = True
    pattern[1] = False
    dev = [c.device() for c in cases]
    stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
    q = torch.stack([c.q_dev() for c in cases])
    kw = dict(retention=0.3, num_sinks=2, window_pages=1, select_mode=mode, return_selection=True,
              head_pattern=torch.from_numpy(pattern))
    if splits is None:
        o, lse, mask = quest_decode_int4(q, **stacked, **kw)
    else:
        with L.attention_splits(splits):
            o, lse, mask = quest_decode_int4(q, **stacked, **kw)
    torch.cuda.synchronize()
    forced = _forced(P, 2, 1)
    rep = Hq // Hkv
    for i, c in enumerate(cases):
        rrow = _retention_rows(pattern[i], 0.3, rep)
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=rrow, num_sinks=2, window_pages=1,
                            mode=mode)
        m = mask[i].cpu().numpy()
        assert np.array_equal(m, ref["mask"]), i
        for h in range(Hkv):
            if not pattern[i, h]:              # streaming head: exactly sinks and window
                assert np.array_equal(m[0, h * rep:(h + 1) * rep], np.broadcast_to(forced, (rep, P))), (i, h)
        tol = decode_tol(ref["O"], "f16")
        assert max_err(o[i][:, :, 0], ref["O"]) <= tol, i
        assert max_err(lse[i][:, :, 0], ref["lse"]) <= 1e-4, i


@pytest.mark.parametrize("mode", ["per_q_head", "per_kv_head_sum"])
def test_layer_patterns_past_512_pages(mode):
    # more than 512 pages: the standalone group selection (per query head one
    # wave per row); streaming heads have retention 0, so only their forced pages
    from flashquest_amd.eager.decode import quest_decode_int4
    Lyr, Hq, Hkv, P = 2, 6, 2, 700
    rng = np.random.default_rng(321)
    cases = [Int4Case(seed=900 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P - 20, D=128) for i in range(Lyr)]
    pattern = np.array([[True, False], [False, True]])
    dev = [c.device() for c in cases]
    stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
    q = torch.stack([c.q_dev() for c in cases])
    o, lse, mask = quest_decode_int4(q, **stacked, retention=0.25, num_sinks=3, window_pages=2, select_mode=mode,
                                     return_selection=True, head_pattern=torch.from_numpy(pattern))
    torch.cuda.synchronize()
    forced = _forced(P, 3, 2)
    rep = Hq // Hkv
    for i, c in enumerate(cases):
        rrow = _retention_rows(pattern[i], 0.25, rep)
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=rrow, num_sinks=3, window_pages=2,
                            mode=mode)
        m = mask[i].cpu().numpy()
        assert np.array_equal(m, ref["mask"]), i
        for h in range(Hkv):
            if not pattern[i, h]:
                assert np.array_equal(m[0, h * rep:(h + 1) * rep], np.broadcast_to(forced, (rep, P))), (i, h)
        tol = 2e-3 + 2.0 ** -8 * float(np.abs(ref["O"]).max())
        assert max_err(o[i][:, :, 0], ref["O"]) <= tol, i
        assert max_err(lse[i][:, :, 0], ref["lse"]) <= 1e-4, i


@pytest.mark.parametrize("D,Hq,Hkv,S,meta,qdt", [(128, 8, 4, 64 * 24, "bf16", "bf16"),
                                                  (128, 24, 8, 64 * 40 + 17, "bf16", "f16"),
                                                  (64, 8, 1, 64 * 9 + 63, "f16", "bf16"),
                                                  (128, 4, 4, 37, "bf16", "f32")])
def test_page_summary_scores_bit_exact(D, Hq, Hkv, S, meta, qdt):
    """The Duo dispatch's scoring (dequantize_k -> compute_page_summary ->
    page_scores, duo/fused_dispatch.py:64-67) in one launch: the bf16 page
    summaries and the fixed-order fp32 scores equal the oracle's bit for bit,
    partial last pages included."""
    from flashquest_amd.eager.criticality import page_scores_int8_summary
    case = Int8Case(seed=D + S, B=2, Hq=Hq, Hkv=Hkv, S=S, D=D, meta=meta, dtype="bf16")
    d = case.device()
    q = case.q_dev() if qdt == "bf16" else case.q_dev().to({"f16": torch.float16, "f32": torch.float32}[qdt])
    sc, pmin, pmax = page_scores_int8_summary(q, d["K_uint8"], d["K_scale"], d["K_mn"], 64, return_summary=True)
    torch.cuda.synchronize()
    lo, hi = O.page_summary_int8(case.ku, case.ks, case.km, 64)
    assert np.array_equal(pmin.float().cpu().numpy(), lo) and np.array_equal(pmax.float().cpu().numpy(), hi)
    ref = O.page_scores_quest_fixed(q[:, :, 0].float().cpu().numpy(), lo, hi)
    assert np.array_equal(sc[:, :, 0].cpu().numpy(), ref)
    # strided codes (a view of a longer cache) give the same scores
    big = torch.zeros(2, Hkv, S + 64, D, dtype=torch.uint8, device=q.device)
    big[:, :, :S] = d["K_uint8"]
    sc2 = page_scores_int8_summary(q, big[:, :, :S], d["K_scale"], d["K_mn"], 64)
    torch.cuda.synchronize()
    assert torch.equal(sc, sc2)


def test_select_pages_loop_form_double_precision_k():
    """select_pages (selection.py:9-62) takes k = ceil(r * P) in double
    precision: 0.07 of 100 pages keeps 8 (the vectorized form keeps 7)."""
    from flashquest_amd.eager.selection import select_pages, select_pages_vectorized
    sc = torch.arange(100, dtype=torch.float32, device="cuda").view(1, 1, 1, 100).repeat(1, 3, 1, 1)
    r = torch.tensor([0.07, 0.0, 1.0])
    m = select_pages(sc, r, 1, 1)
    mv = select_pages_vectorized(sc, r, 1, 1)
    torch.cuda.synchronize()
    ref = O.select_pages(sc.cpu().numpy(), r.numpy(), 1, 1)
    assert np.array_equal(m.cpu().numpy(), ref)
    assert int(m[0, 0].sum()) == 9 and int(mv[0, 0].sum()) == 8        # + sink 0 (the top-k holds window 99)
    assert int(m[0, 1].sum()) == 2 and bool(m[0, 2].all())


@pytest.mark.parametrize("Hq,Hkv,P,pattern", [(8, 4, 24, [True, False, True, False]),
                                               (24, 8, 64, [True] * 8),
                                               (24, 8, 40, [False, True] * 4)])
def test_quest_duo_fused_sdpa_reference_semantics(Hq, Hkv, P, pattern):
    """quest_duo_fused_sdpa against the oracle's restatement of the
    reference's three steps: page summary scores of the bf16-dequantised keys,
    select_pages with retention 0.25 on retrieval heads and 0 on streaming
    heads, INT8 sparse attention over that mask.  The selection is checked
    bit for bit (same fixed score order) and against the fp64 Quest bound
    wherever its top-k boundary is not an fp32 near-tie."""
    from flashquest_amd.duo import quest_duo_fused_sdpa
    from flashquest_amd.eager.criticality import page_scores_int8_summary
    from flashquest_amd.eager.selection import select_pages
    case = Int8Case(seed=77 + P, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128)
    d = case.device()
    pat = torch.tensor(pattern)
    o = quest_duo_fused_sdpa(case.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"],
                             d["V_mn"], head_pattern=pat, retention=0.25, num_sinks=4, window_pages=2)
    torch.cuda.synchronize()
    lo, hi = O.page_summary_int8(case.ku, case.ks, case.km, 64)
    scores = O.page_scores_quest_fixed(case.Q, lo, hi)
    rrow = _retention_rows(pat.numpy(), 0.25, Hq // Hkv)
    mask = O.select_pages(scores[:, :, None, :], rrow, 4, 2)[:, :, 0, :]
    ref_o, _ = O.sparse_int8_attention(case.Q, case.ku, case.ks, case.km, case.vu, case.vs, case.vm, mask, 64)
    assert o.shape == (1, Hq, 1, 128) and o.dtype == torch.bfloat16
    assert max_err(o[:, :, 0], ref_o) <= decode_tol(ref_o, "bf16")
    # the mask itself, through the operators the dispatch calls
    sel = select_pages(page_scores_int8_summary(case.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"]),
                       torch.from_numpy(rrow), 4, 2)
    torch.cuda.synchronize()
    assert np.array_equal(sel[:, :, 0].cpu().numpy(), mask)
    exact = O.page_scores_quest(case.Q, lo, hi)
    k = math.ceil(float(np.float32(0.25)) * P)
    forced = _forced(P, 4, 2)
    rep = Hq // Hkv
    amb = 0
    for h in range(Hq):
        if rrow[h] == 0:
            assert np.array_equal(mask[0, h], forced)
            continue
        order = np.argsort(-exact[0, h], kind="stable")
        mag = np.maximum(np.abs(lo[0, h // rep]), np.abs(hi[0, h // rep])).astype(np.float64)
        tau = 140 * 2.0 ** -24 * (mag @ np.abs(case.Q[0, h]).astype(np.float64))
        top, rest = order[:k], order[k:]
        if np.min(exact[0, h, top] - tau[top]) <= np.max(exact[0, h, rest] + tau[rest]):
            amb += 1
            continue
        want = forced.copy()
        want[top] = True
        assert np.array_equal(mask[0, h], want), h
    print(f"[duo] Hq={Hq} P={P}: ambiguous rows {amb}", flush=True)
    with pytest.raises(ValueError, match="head_pattern"):
        quest_duo_fused_sdpa(case.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"],
                             d["V_mn"], head_pattern=torch.tensor([True] * (Hkv + 1)))


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_compute_page_summary(dtype):
    """compute_page_summary (page_summary.py:7-39) on the GPU: bit for bit
    against the oracle for each K dtype, a partial last page, a strided K view
    and a NaN (propagated by torch's min / max)."""
    from flashquest_amd.eager import compute_page_summary
    rng = np.random.default_rng(11)
    K = rng.standard_normal((2, 3, 64 * 5 + 9, 128)).astype(np.float32)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    Kd = torch.from_numpy(K).to(tdt).cuda()
    Kh = Kd.float().cpu().numpy()
    lo, hi = compute_page_summary(Kd, 64)
    ref_lo, ref_hi = O.compute_page_summary(Kh, 64)
    assert lo.dtype == tdt and lo.shape == (2, 3, 6, 128)
    assert np.array_equal(lo.float().cpu().numpy(), ref_lo) and np.array_equal(hi.float().cpu().numpy(), ref_hi)
    big = torch.zeros(2, 3, Kd.shape[2], 256, dtype=tdt, device="cuda")
    big[..., 64:192] = Kd
    lo2, hi2 = compute_page_summary(big[..., 64:192], 64)
    assert torch.equal(lo2, lo) and torch.equal(hi2, hi)
    Kd[1, 2, 70, 5] = float("nan")
    lo3, hi3 = compute_page_summary(Kd, 64)
    torch.cuda.synchronize()
    assert torch.isnan(lo3[1, 2, 1, 5]) and torch.isnan(hi3[1, 2, 1, 5])
    assert int(torch.isnan(lo3).sum()) == 1 and int(torch.isnan(hi3).sum()) == 1


@pytest.mark.parametrize("H,Hb,Sq,D,qdt", [(4, 4, 1, 128, "bf16"), (8, 2, 3, 128, "f16"), (6, 3, 2, 64, "f32")])
def test_page_scores_bit_exact(H, Hb, Sq, D, qdt):
    """page_scores (criticality.py:7-31) from summaries: bit for bit against
    the oracle's fixed order, one summary row per head (the reference's) or
    shared by a GQA group, several query positions; and the Quest bound."""
    from flashquest_amd.eager import compute_page_summary, page_scores
    rng = np.random.default_rng(H + D)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[qdt]
    K = torch.from_numpy(rng.standard_normal((2, Hb, 64 * 6, D)).astype(np.float32)).to(torch.bfloat16).cuda()
    Q = torch.from_numpy(rng.standard_normal((2, H, Sq, D)).astype(np.float32)).to(tdt).cuda()
    lo, hi = compute_page_summary(K, 64)
    sc = page_scores(Q, lo, hi)
    torch.cuda.synchronize()
    qh = Q.float().cpu().numpy()
    for s in range(Sq):
        ref = O.page_scores_quest_fixed(qh[:, :, s], lo.float().cpu().numpy(), hi.float().cpu().numpy())
        assert np.array_equal(sc[:, :, s].cpu().numpy(), ref), s
        exact = O.page_scores_quest(qh[:, :, s], lo.float().cpu().numpy(), hi.float().cpu().numpy())
        kd = K.float().cpu().numpy().astype(np.float64)
        qk = np.einsum("bhd,bhsd->bhs", qh[:, :, s].astype(np.float64), np.repeat(kd, H // Hb, axis=1))
        assert np.all(exact >= qk.reshape(2, H, 6, 64).max(-1) - 1e-9)
