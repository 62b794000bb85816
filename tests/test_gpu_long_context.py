"""Decode steps longer than the single-launch kernel's 512 pages, against the CPU oracle.

Past 512 pages per KV group the in-LDS selection no longer holds a group's
keys, so every cache family takes three launches: the scoring launch, the
standalone group selection (one wave per group summed, one wave per query
row per head) and the attention over the selected lists.  These tests run
that path on the bench's synthetic caches (2 layers x 24/8 heads, 1000 pages:
ragged against the 64-lane selection tiles) for INT4, INT8 and TurboQuant in
both selection modes, and check the selection of every group bit-exact
against the oracle's score -> top-k -> forced pages, and O / lse of every
layer against the oracle's fp64 attention over that selection.
"""
import math

import numpy as np
import pytest
import torch

import bench
from oracle import fq_oracle as O

pytestmark = pytest.mark.gpu

LAYERS, P, RET = 2, 1000, 0.25
K = math.ceil(RET * P)
TOL_O, TOL_LSE = 2e-3, 1e-4
KW = dict(retention=RET, num_sinks=4, window_pages=2, k_max_static=K)


def _ref_mask(scores, mode, rep):
    m = O.select_pages_vectorized(scores[:, :, None, :], RET, 4, 2, K)[:, :, 0, :]
    return np.repeat(m, rep, axis=1) if mode == "per_kv_head_sum" else m


def _check(o, lse, ref_o, ref_l):
    got_o = o.float().cpu().numpy()
    assert np.abs(got_o - ref_o).max() <= TOL_O + 2.0 ** -8 * np.abs(ref_o).max()
    assert np.abs(lse.cpu().numpy() - ref_l).max() <= TOL_LSE


def _host(c, keys, l, layer_axis_is_batch):
    out = []
    for k in keys:
        t = (c[k][l:l + 1] if layer_axis_is_batch else c[k][l, 0:1]).cpu()
        out.append(t.numpy() if t.dtype == torch.uint8 else t.float().numpy())
    return out


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_int4_long_step(mode):
    from flashquest_amd.eager.decode import quest_decode_int4
    c = bench.make_cache(LAYERS, 1, P=P, dev=torch.device("cuda:0"))
    keys = ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")
    o, lse, mask = quest_decode_int4(c["Q"], *[c[k] for k in keys], select_mode=mode, return_selection=True, **KW)
    o2, lse2 = quest_decode_int4(c["Q"], *[c[k] for k in keys], select_mode=mode, **KW)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    m_host = mask.cpu().numpy()
    for l in range(LAYERS):
        q = c["Q"][l, 0:1, :, 0].float().cpu().numpy()
        planes = _host(c, keys, l, False)
        ref = _ref_mask(O.page_scores_fixed(q, planes[1], planes[2], mode), mode, 3)
        assert np.array_equal(m_host[l, 0:1], ref), l
        ref_o, ref_l = O.sparse_int4_attention(q, *planes, ref, 64)
        _check(o[l, 0:1, :, 0], lse[l, 0:1, :, 0], ref_o, ref_l)


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_int8_long_step(mode):
    from flashquest_amd.eager.decode import quest_decode_int8
    c = bench.make_int8_cache(LAYERS, P=P, dev=torch.device("cuda:0"))
    keys = ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")
    o, lse, mask = quest_decode_int8(c["Q"], *[c[k] for k in keys], select_mode=mode, return_selection=True, **KW)
    o2, lse2 = quest_decode_int8(c["Q"], *[c[k] for k in keys], select_mode=mode, **KW)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    m_host = mask.cpu().numpy()
    for l in range(LAYERS):
        q = c["Q"][l:l + 1, :, 0].float().cpu().numpy()
        planes = _host(c, keys, l, True)
        ref = _ref_mask(O.page_scores_fixed(q, planes[1], planes[2], mode, 255.0), mode, 3)
        assert np.array_equal(m_host[l:l + 1], ref), l
        ref_o, ref_l = O.sparse_int8_attention(q, *planes, ref, 64)
        _check(o[l:l + 1, :, 0], lse[l:l + 1, :, 0], ref_o, ref_l)


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_turbo_long_step(mode):
    from flashquest_amd.eager.decode import quest_decode_turbo
    c = bench.make_turbo_cache(LAYERS, P=P, dev=torch.device("cuda:0"))
    keys = ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")
    args = [c["Q"]] + [c[k] for k in keys] + [c["K_scale_raw"], c["K_mn_raw"]]
    o, lse, mask = quest_decode_turbo(*args, select_mode=mode, return_selection=True, **KW)
    o2, lse2 = quest_decode_turbo(*args, select_mode=mode, **KW)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    m_host = mask.cpu().numpy()
    for l in range(LAYERS):
        q = c["Q"][l:l + 1, :, 0].float().cpu().numpy()
        ksr, kmr = _host(c, ("K_scale_raw", "K_mn_raw"), l, True)
        ref = _ref_mask(O.page_scores_fixed(q, ksr, kmr, mode), mode, 3)
        assert np.array_equal(m_host[l:l + 1], ref), l
        ref_o, ref_l = O.sparse_turbo_attention(q, *_host(c, keys, l, True), ref, 64)
        _check(o[l:l + 1, :, 0], lse[l:l + 1, :, 0], ref_o, ref_l)
