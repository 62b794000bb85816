"""TurboQuant K3-V3 decode attention on the GPU against the oracle
(src/flashquest/kernel/sparse_turbo_fwd.py:110-346): the fused-layout kernel
(D=128, <= 3 query heads per KV head) with page lists from a mask (splits
merged when few KV groups), the split VALU kernel it hands 4 and 8 query
heads to, and the single-launch fused decode that scores the pages from the
un-rotated K page metadata and selects them itself."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import make_kv, max_err, to_dev, to_dev_half

pytestmark = pytest.mark.gpu


def _turbo_case(rng, B, Hq, Hkv, S, D=128):
    K, V = make_kv(rng, B, Hkv, S, D, outliers=True)
    km, kl, kst, ksr, kmr = O.quantize_k_turbo(K, 64)
    vm, vl, vst = O.quantize_turbo(V)
    Q = O.round_bf16(rng.standard_normal((B, Hq, D)).astype(np.float32))
    return Q, (km, kl, kst, vm, vl, vst), (ksr, kmr)


def _tol(ref):
    return 2e-3 + 2 ** -8 * np.abs(ref).max()


@pytest.mark.parametrize("B,Hq,Hkv", [(2, 6, 2), (1, 3, 3), (3, 4, 2), (1, 2, 1), (2, 8, 2), (1, 8, 1), (1, 10, 2),
                                     (2, 6, 1), (1, 7, 1)])
def test_turbo_mask_attention_matches_oracle(B, Hq, Hkv):
    from flashquest_amd.kernel import flash_attn_sparse_turbo_fwd
    rng = np.random.default_rng(100 + Hq * 7 + Hkv)
    S = 64 * 11 + 13                                    # partial last page
    Q, planes, _ = _turbo_case(rng, B, Hq, Hkv, S)
    P = (S + 63) // 64
    mask = rng.random((B, Hq, P)) < 0.45
    mask[0, 0] = False                                  # a head with nothing selected
    mask[-1, -1, -1] = True                             # the partial page
    ref_o, ref_l = O.sparse_turbo_attention(Q, *planes, mask, 64)
    dev = [to_dev(planes[0]), to_dev(planes[1]), to_dev_half(planes[2], "bf16"), to_dev(planes[3]),
           to_dev(planes[4]), to_dev_half(planes[5], "bf16")]
    o, lse = flash_attn_sparse_turbo_fwd(to_dev_half(Q, "bf16")[:, :, None], *dev,
                                         selection_mask=to_dev(mask)[:, :, None])
    assert max_err(o[:, :, 0], ref_o) <= _tol(ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
@pytest.mark.parametrize("Hq,sinks,window,P", [(24, 3, 2, 20), (24, 0, 0, 20), (16, 9, 1, 12), (8, 4, 2, 6),
                                              (40, 3, 2, 20), (56, 1, 1, 12), (64, 2, 1, 10)])
def test_fused_turbo_decode_matches_oracle(mode, Hq, sinks, window, P):
    # 24 layers x 8 KV heads = 192 KV groups: one workgroup per group, which
    # scores and selects its pages; a second call also writes the kernel's
    # selection as a mask, which must be the oracle's bit for bit
    from flashquest_amd.eager import quest_decode_turbo
    rng = np.random.default_rng(7 + Hq + P)
    Lyr, Hkv = 24, 8
    S = 64 * (P - 1) + 40
    cases = [_turbo_case(rng, 1, Hq, Hkv, S) for _ in range(Lyr)]
    r = np.linspace(0.05, 0.6, Hq).astype(np.float32)
    stack = lambda f: torch.stack([f(c) for c in cases])
    Qd = stack(lambda c: to_dev_half(c[0], "bf16")[:, :, None])
    pl = [stack(lambda c, i=i: to_dev(c[1][i]) if i in (0, 1, 3, 4) else to_dev_half(c[1][i], "bf16"))
          for i in range(6)]
    ksr = stack(lambda c: to_dev_half(c[2][0], "bf16"))
    kmr = stack(lambda c: to_dev_half(c[2][1], "bf16"))
    kw = dict(retention=torch.from_numpy(r), num_sinks=sinks, window_pages=window, k_max_static=8, select_mode=mode)
    o, lse = quest_decode_turbo(Qd, *pl, ksr, kmr, **kw)
    o2, lse2, mask = quest_decode_turbo(Qd, *pl, ksr, kmr, return_selection=True, **kw)
    torch.cuda.synchronize()
    rep = Hq // Hkv
    for i, (Q, planes, raw) in enumerate(cases):
        scores = O.page_scores_fixed(Q, raw[0], raw[1], mode)
        if mode == "per_q_head":
            ref_mask = O.select_pages_vectorized(scores[:, :, None, :], r, sinks, window, 8)[:, :, 0, :]
        else:
            m = O.select_pages_vectorized(scores[:, :, None, :], r.reshape(Hkv, rep).max(-1), sinks, window,
                                          8)[:, :, 0, :]
            ref_mask = np.repeat(m, rep, axis=1)
        assert np.array_equal(mask[i].cpu().numpy(), ref_mask), i
        ref_o, ref_l = O.sparse_turbo_attention(Q, *planes, ref_mask, 64)
        for oo, ll in ((o, lse), (o2, lse2)):
            assert max_err(oo[i][:, :, 0], ref_o) <= _tol(ref_o), i
            assert max_err(ll[i][:, :, 0], ref_l) <= 1e-4, i


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_single_layer_turbo_decode_splits_match_oracle(mode):
    """One layer of 8 KV groups over 200 pages (the reference's per-layer call
    shape): a scoring launch, the attention workgroups select from its scores
    with each group split over several workgroups, and the one-round split
    merge rotates O back.  Selection bit-exact, O and lse against the oracle."""
    from flashquest_amd.eager import quest_decode_turbo
    rng = np.random.default_rng(4242)
    Hq, Hkv, P = 24, 8, 200
    S = 64 * (P - 1) + 40
    Q, planes, raw = _turbo_case(rng, 1, Hq, Hkv, S)
    r = np.linspace(0.1, 0.4, Hq).astype(np.float32)
    Qd = to_dev_half(Q, "bf16")[:, :, None]
    pl = [to_dev(planes[i]) if i in (0, 1, 3, 4) else to_dev_half(planes[i], "bf16") for i in range(6)]
    ksr, kmr = to_dev_half(raw[0], "bf16"), to_dev_half(raw[1], "bf16")
    kw = dict(retention=torch.from_numpy(r), num_sinks=4, window_pages=2, select_mode=mode)
    o, lse, mask = quest_decode_turbo(Qd, *pl, ksr, kmr, return_selection=True, **kw)
    torch.cuda.synchronize()
    scores = O.page_scores_fixed(Q, raw[0], raw[1], mode)
    rep = Hq // Hkv
    if mode == "per_q_head":
        ref_mask = O.select_pages_vectorized(scores[:, :, None, :], r, 4, 2)[:, :, 0, :]
    else:
        m = O.select_pages_vectorized(scores[:, :, None, :], r.reshape(Hkv, rep).max(-1), 4, 2)[:, :, 0, :]
        ref_mask = np.repeat(m, rep, axis=1)
    assert np.array_equal(mask.cpu().numpy(), ref_mask)
    ref_o, ref_l = O.sparse_turbo_attention(Q, *planes, ref_mask, 64)
    assert max_err(o[:, :, 0], ref_o) <= _tol(ref_o)
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4
