"""The benchmarked decode at the benchmark configurations' geometries, against the CPU oracle.

The whole-step decode over all layers is one kernel launch when the KV groups
fill the GPU (L*B*H_kv >= 192): every workgroup scores its group's 512 pages,
selects them in LDS (8 keys per lane) and attends.  These tests run exactly
that launch on the bench's own synthetic caches (bench.make_cache: lognormal K
channels, planted pages, fp16 metadata, V in 32-channel groups) and check

* the in-kernel selection of every (layer, sequence, KV head) bit-exact
  against the oracle's score -> top-k -> forced pages, and against the split
  path's separate selection kernel;
* the selection of every sampled (layer, sequence) against the exact fp64
  page scores, independent of any fp32 summation order: equal on every row
  whose top-k boundary is not within fp32 error of another page (such rows
  are counted as ambiguous, with how many of them the GPU resolved unlike
  the fp64 order, and printed);
* O and lse of sampled layers against the oracle's fp64 attention over the
  same selection: a flat 2e-3 max-abs for fp16 output (
  output rounding included); the largest error per configuration is printed;
* that asking for the mask does not change O (same kernel, bitwise);
* the split path (several workgroups per group, merge launch) against the
  fused one within the same tolerance (their fp32 orders differ).

Configs: 0 (one layer, 128 pages, r = 0.20, the small-step single launch the
bench times), 1 (28 layers, r = 0.25, k = 128 of 512), 2 (r = 1: k = P), 3
(rotated INT4: Q rotated, decode, O rotated back) and 4 (batch 16, 3584
groups), in both selection modes where the reference has them; the INT8 and
TurboQuant steps at config 1's geometry with bf16 queries (the reference's)
and with fp16 queries (fp16 output: the flat bar).
"""
import math

import numpy as np
import pytest
import torch

import bench
from flashquest_amd import _lib as L
from flashquest_amd.eager.decode import QuestDecoder, quest_decode_int4
from oracle import fq_oracle as O
from tests.cases import decode_tol, fp64_selection_check

pytestmark = pytest.mark.gpu

TOL_O = 2e-3
TOL_LSE = 1e-4
PLANES = ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")
LAYERS, P = 28, 512


def _tol(ref_o):
    """fp16 output: the flat 2e-3 north-star bar, output rounding included."""
    return TOL_O


def _tol_bf16(ref_o):
    """bf16 output (the reference's own output type): 2e-3 plus the output's
    rounding, 2^-8 |O|."""
    return decode_tol(ref_o, "bf16")


def _report(name, **kw):
    print(f"[at-size] {name}: " + ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.fixture(scope="module")
def cfg1():
    return bench.make_cache(LAYERS, 1, P=P, dev=torch.device("cuda:0"))


def _host(c, l, b):
    """(Q (1,H_q,D), planes) of (layer l, sequence b) as numpy for the oracle."""
    q = c["Q"][l, b:b + 1, :, 0].float().cpu().numpy()
    planes = []
    for k in PLANES:
        t = c[k][l, b:b + 1].cpu()
        planes.append(t.numpy() if t.dtype == torch.uint8 else t.float().numpy())
    return q, planes


def _oracle_mask(q, planes, retention, mode):
    ks, km = planes[1], planes[2]
    scores = O.page_scores_fixed(q, ks, km, mode)
    Hq, Hkv = q.shape[1], ks.shape[1]
    rep = Hq // Hkv
    if mode == "per_q_head":
        return O.select_pages_vectorized(scores[:, :, None, :], retention, 4, 2)[:, :, 0, :]
    # one row per KV head: its k from the largest retention of its query heads
    r_kv = retention if np.isscalar(retention) else np.asarray(retention, np.float32).reshape(Hkv, rep).max(1)
    m = O.select_pages_vectorized(scores[:, :, None, :], r_kv, 4, 2)[:, :, 0, :]
    return np.repeat(m, rep, axis=1)


def _kmax(retention):
    return min(math.ceil(float(np.max(np.asarray(retention))) * P), P)


def _run(c, retention, mode, splits=None, with_mask=True):
    k = _kmax(retention)
    if not np.isscalar(retention):
        retention = torch.as_tensor(np.asarray(retention, np.float32))
    args = [c["Q"]] + [c[x] for x in PLANES]
    kw = dict(retention=retention, num_sinks=4, window_pages=2, k_max_static=k, select_mode=mode,
              return_selection=with_mask)
    if splits is None:
        res = quest_decode_int4(*args, **kw)
    else:
        with L.attention_splits(splits):
            res = quest_decode_int4(*args, **kw)
    torch.cuda.synchronize()
    return res


def _is_fused(c, retention, mode):
    k = _kmax(retention)
    if not np.isscalar(retention):
        retention = torch.as_tensor(np.asarray(retention, np.float32))
    d = QuestDecoder(c["Q"], *[c[x] for x in PLANES], retention=retention, num_sinks=4, window_pages=2,
                     k_max_static=k, select_mode=mode)
    return d.fused


def _check_step(c, retention, mode, sample, mask_sample=None):
    """Fused step vs oracle (selection on mask_sample or every (l, b), O/lse on
    `sample`), vs the split path, and mask-on vs mask-off bitwise."""
    assert _is_fused(c, retention, mode), "the benchmarked configuration must take the single-launch kernel"
    Lc, B = c["Q"].shape[0], c["Q"].shape[1]
    o, lse, mask = _run(c, retention, mode)
    o2, lse2 = _run(c, retention, mode, with_mask=False)
    assert torch.equal(o, o2) and torch.equal(lse, lse2), "mask output changed the fused result"
    os_, lses, masks = _run(c, retention, mode, splits=4)
    assert torch.equal(mask, masks), "fused in-kernel selection differs from the selection kernel"
    m_host = mask.cpu().numpy()
    pairs = mask_sample if mask_sample is not None else [(l, b) for l in range(Lc) for b in range(B)]
    rows = amb = amb_diff = 0
    for l, b in pairs:
        q, planes = _host(c, l, b)
        ref = _oracle_mask(q, planes, retention, mode)
        assert np.array_equal(m_host[l, b:b + 1], ref), f"selection differs from the oracle at layer {l}, seq {b}"
        n, a, mis, ad = fp64_selection_check(q, planes[1], planes[2], m_host[l, b:b + 1], retention, mode)
        assert mis == 0, f"layer {l} seq {b}: {mis} unambiguous rows differ from the fp64 selection"
        rows, amb, amb_diff = rows + n, amb + a, amb_diff + ad
    err_max = lse_max = 0.0
    for l, b in sample:
        q, planes = _host(c, l, b)
        ref_o, ref_l = O.sparse_int4_attention(q, *planes, m_host[l, b:b + 1], 64)
        got_o = o[l, b:b + 1, :, 0].float().cpu().numpy()
        got_l = lse[l, b:b + 1, :, 0].cpu().numpy()
        err_o = float(np.abs(got_o - ref_o).max())
        err_max, lse_max = max(err_max, err_o), max(lse_max, float(np.abs(got_l - ref_l).max()))
        assert err_o <= _tol(ref_o), f"layer {l} seq {b}: max|O - oracle| = {err_o}"
        assert np.abs(got_l - ref_l).max() <= TOL_LSE, f"layer {l} seq {b}: lse"
    d = (o.float() - os_.float()).abs().max().item()
    assert d <= 2 * TOL_O, f"fused vs split O differ by {d}"
    assert (lse - lses).abs().max().item() <= 2 * TOL_LSE
    return mask, dict(rows=rows, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
                      max_abs_O=f"{err_max:.3e}", max_abs_lse=f"{lse_max:.3e}", fused_vs_split=f"{d:.3e}")


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_config1_fused_step(cfg1, mode):
    mask, rec = _check_step(cfg1, 0.25, mode, sample=[(0, 0), (13, 0), (27, 0)])
    _report(f"config1 {mode}", **rec)
    # top-128 plus the 6 forced pages, which the top-k may already hold
    per_head = mask.view(LAYERS, 1, 8, 3, P).sum(-1)
    assert int(per_head.min()) >= 128 and int(per_head.max()) <= 134


def test_config2_all_pages(cfg1):
    mask, rec = _check_step(cfg1, 1.0, "per_kv_head_sum", sample=[(5, 0)])
    _report("config2", **rec)
    assert bool(mask.all()), "retention 1 selects every page"


def test_config1_retention_per_head(cfg1):
    """Different retention per query head (DuoAttention-style vectors), k of
    each head from fp32 ceil(r * P), through the fused kernel."""
    r = np.array([0.25, 0.1, 0.4] * 8, np.float32)
    _, rec = _check_step(cfg1, r, "per_q_head", sample=[(3, 0)], mask_sample=[(l, 0) for l in range(0, LAYERS, 3)])
    _report("config1 per-head retention", **rec)


@pytest.fixture(scope="module", params=[64, 48], ids=["gqa8", "gqa6"])
def cfg1_wide(request):
    """Config 1's caches with 8 or 6 query heads per KV head (64 / 48 heads)."""
    return bench.make_cache(LAYERS, 1, Hq=request.param, P=P, dev=torch.device("cuda:0"))


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_config1_geometry_wide_gqa_one_launch(cfg1_wide, mode):
    """6 and 8 query heads per KV head at config 1's geometry take one launch:
    every KV head runs as two virtual heads of 3 or 4 query heads, one
    workgroup each reading the same cache head; per_kv_head_sum scores the
    sum of all the head's queries in both, so both select the same pages."""
    mask, rec = _check_step(cfg1_wide, 0.25, mode, sample=[(0, 0), (27, 0)],
                            mask_sample=[(0, 0), (13, 0), (27, 0)])
    _report(f"config1 geometry, {cfg1_wide['Q'].shape[2]} query heads, {mode}", **rec)
    nrep = cfg1_wide["Q"].shape[2] // 8
    per_head = mask.view(LAYERS, 1, 8, nrep, P).sum(-1)
    assert int(per_head.min()) >= 128 and int(per_head.max()) <= 134


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_config1_geometry_wide_gqa_retention_per_head(cfg1_wide, mode):
    """Per-head retentions whose largest value falls in either half of a KV
    head's query heads: per_kv_head_sum takes k from the largest retention of
    all the head's queries, not of its own virtual head's."""
    Hq = cfg1_wide["Q"].shape[2]
    r = np.random.default_rng(Hq).uniform(0.05, 0.3, Hq).astype(np.float32)
    _, rec = _check_step(cfg1_wide, r, mode, sample=[(2, 0)], mask_sample=[(l, 0) for l in range(0, LAYERS, 7)])
    _report(f"config1 geometry, {Hq} query heads, per-head retention, {mode}", **rec)


def test_config3_rotated_step():
    """Config 3: K, V rotated by x -> WHT(s x) / sqrt(128) before quantisation.
    The single launch rotates Q in its prologue (fp32) and O back in its
    store.  Against the oracle: the same fp32 rotation of Q (bit-exact, so the
    selection is), attention in the rotated basis, the fp64 inverse rotation
    of its O; and against the split path, which rotates with fq_wht around the
    step."""
    dev = torch.device("cuda:0")
    signs = bench.rotation_signs(dev=dev)
    rc = bench.make_cache(LAYERS, 1, P=P, dev=dev, signs=signs)
    args = [rc["Q"]] + [rc[x] for x in PLANES]
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=128, select_mode="per_kv_head_sum",
              return_selection=True, rotation_signs=signs)
    d = QuestDecoder(*args, retention=0.25, num_sinks=4, window_pages=2, k_max_static=128,
                     select_mode="per_kv_head_sum", rotation_signs=signs)
    assert d.fused
    o, lse, mask = quest_decode_int4(*args, **kw)
    with L.attention_splits(4):
        o_s, lse_s, mask_s = quest_decode_int4(*args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(mask, mask_s)
    s_host = signs.cpu().numpy()
    m_host = mask.cpu().numpy()
    rows = amb = amb_diff = 0
    err_max = 0.0
    for l in range(LAYERS):
        q_raw, planes = _host(rc, l, 0)
        q_rot = O.rotate_signed_f32(q_raw, s_host)
        assert np.array_equal(m_host[l, 0:1], _oracle_mask(q_rot, planes, 0.25, "per_kv_head_sum")), l
        n, a, mis, ad = fp64_selection_check(O.rotate_signed(q_raw, s_host), planes[1], planes[2], m_host[l, 0:1],
                                             0.25, "per_kv_head_sum")
        assert mis == 0, l
        rows, amb, amb_diff = rows + n, amb + a, amb_diff + ad
        if l not in (0, 13, 27):
            continue
        ref_rot, ref_l = O.sparse_int4_attention(q_rot, *planes, m_host[l, 0:1], 64)
        ref_raw = O.unrotate_signed(ref_rot, s_host)
        got = o[l, 0:1, :, 0].float().cpu().numpy()
        err = float(np.abs(got - ref_raw).max())
        err_max = max(err_max, err)
        assert err <= _tol(ref_raw), l
        assert np.abs(lse[l, 0:1, :, 0].cpu().numpy() - ref_l).max() <= TOL_LSE, l
    d = (o.float() - o_s.float()).abs().max().item()
    assert d <= 2 * TOL_O
    assert (lse - lse_s).abs().max().item() <= 2 * TOL_LSE
    _report("config3 rotated", rows=rows, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
            max_abs_O=f"{err_max:.3e}", fused_vs_split=f"{d:.3e}")


def test_config4_batch16():
    dev = torch.device("cuda:0")
    bc = bench.make_cache(LAYERS, 16, P=P, dev=dev)
    rng = np.random.default_rng(4)
    pairs = sorted({(int(l), int(b)) for l, b in zip(rng.integers(0, LAYERS, 48), rng.integers(0, 16, 48))})
    _, rec = _check_step(bc, 0.25, "per_kv_head_sum", sample=[(0, 15), (27, 7)], mask_sample=pairs)
    _report("config4 batch16", **rec)


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_config0_small_step(mode):
    """Config 0 at its benchmark layout: one layer, batch 1, 24 / 8 heads, 8k
    context (128 pages), r = 0.20 (k = 26) + 4 sink and 2 window pages, fp16
    Q and metadata, V in 32-channel groups.  Through the exact object the
    bench times (QuestDecoder: with 8 KV groups and <= 40 pages per group it is
    the small-step single launch), against the oracle's decode step and the
    fp64 selection, and against the split path (scoring launch, selection in
    the attention workgroups, merge launch)."""
    dev = torch.device("cuda:0")
    c0 = bench.make_cache(1, 1, P=128, dev=dev)
    planes = [c0[x] for x in PLANES]
    m0 = torch.zeros(1, 1, 24, 128, dtype=torch.bool, device=dev)
    d0 = QuestDecoder(c0["Q"], *planes, retention=0.2, num_sinks=4, window_pages=2, k_max_static=26,
                      select_mode=mode, mask_out=m0)
    assert d0.fused, "config 0 must take the single launch the bench times"
    d0()
    o = d0.O3.clone()
    with L.attention_splits(4):
        os_, _, ms_ = quest_decode_int4(c0["Q"], *planes, retention=0.2, num_sinks=4, window_pages=2,
                                        k_max_static=26, select_mode=mode, return_selection=True)
    torch.cuda.synchronize()
    assert torch.equal(m0, ms_)
    q, hp = _host(c0, 0, 0)
    ref = O.decode_step(q, *hp, retention=0.2, num_sinks=4, window_pages=2, mode=mode, k_max_static=26)
    assert np.array_equal(m0[0].cpu().numpy(), ref["mask"])
    n, amb, mis, amb_diff = fp64_selection_check(q, hp[1], hp[2], m0[0].cpu().numpy(), 0.2, mode)
    assert mis == 0
    err = float(np.abs(o[0].float().cpu().numpy() - ref["O"]).max())
    assert err <= TOL_O, err
    d = (o.float() - os_[0, :, :, 0].float()).abs().max().item()
    assert d <= 2 * TOL_O
    _report(f"config0 {mode}", rows=n, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
            max_abs_O=f"{err:.3e}", fused_vs_split=f"{d:.3e}")


def _host4(c, keys, l):
    """Layer l of a cache whose layers are folded into the batch axis."""
    out = []
    for k in keys:
        t = c[k][l:l + 1].cpu()
        out.append(t.numpy() if t.dtype == torch.uint8 else t.float().numpy())
    return out


def _qtol(qdtype, ref_o):
    return _tol(ref_o) if qdtype == "f16" else _tol_bf16(ref_o)


@pytest.fixture(scope="module")
def int8_cfg1():
    return bench.make_int8_cache(LAYERS, P=P, dev=torch.device("cuda:0"))


@pytest.fixture(scope="module")
def turbo_cfg1():
    return bench.make_turbo_cache(LAYERS, P=P, dev=torch.device("cuda:0"))


@pytest.mark.parametrize("qdtype", ["bf16", "f16"])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_int8_fused_step_at_size(int8_cfg1, mode, qdtype):
    """The INT8 family (kv_bits 8) at config 1's geometry: 28 layers x 8 KV
    heads x 512 pages, bf16 metadata, through the single-launch kernel; bf16
    queries (the reference's) and fp16 queries (fp16 output, flat 2e-3)."""
    from flashquest_amd.eager.decode import quest_decode_int8
    ic = int8_cfg1
    Q = ic["Q"] if qdtype == "bf16" else ic["Q"].half()
    keys = ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=128, select_mode=mode)
    o, lse, mask = quest_decode_int8(Q, *[ic[k] for k in keys], return_selection=True, **kw)
    o2, lse2 = quest_decode_int8(Q, *[ic[k] for k in keys], **kw)
    with L.attention_splits(4):
        os_, lses, masks = quest_decode_int8(Q, *[ic[k] for k in keys], return_selection=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(mask, masks)
    m_host = mask.cpu().numpy()
    rows = amb = amb_diff = 0
    err_max = 0.0
    for l in range(LAYERS):
        q = Q[l:l + 1, :, 0].float().cpu().numpy()
        planes = _host4(ic, keys, l)
        scores = O.page_scores_fixed(q, planes[1], planes[2], mode, 255.0)
        ref_mask = O.select_pages_vectorized(scores[:, :, None, :], 0.25, 4, 2, 128)[:, :, 0, :]
        if mode == "per_kv_head_sum":
            ref_mask = np.repeat(ref_mask, 3, axis=1)
        assert np.array_equal(m_host[l:l + 1], ref_mask), l
        n, a, mis, ad = fp64_selection_check(q, planes[1], planes[2], m_host[l:l + 1], 0.25, mode, levels=255.0)
        assert mis == 0, l
        rows, amb, amb_diff = rows + n, amb + a, amb_diff + ad
        if l in (0, 27):
            ref_o, ref_l = O.sparse_int8_attention(q, *planes, ref_mask, 64)
            err = float(np.abs(o[l:l + 1, :, 0].float().cpu().numpy() - ref_o).max())
            err_max = max(err_max, err)
            assert err <= _qtol(qdtype, ref_o), (l, err)
            assert np.abs(lse[l:l + 1, :, 0].cpu().numpy() - ref_l).max() <= TOL_LSE
    d = (o.float() - os_.float()).abs().max().item()
    assert d <= 2 * _qtol(qdtype, np.array([2.0]))
    _report(f"int8 {mode} q={qdtype}", rows=rows, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
            max_abs_O=f"{err_max:.3e}", fused_vs_split=f"{d:.3e}")


@pytest.fixture(scope="module", params=[64, 48], ids=["gqa8", "gqa6"])
def int8_wide(request):
    """The INT8 caches of config 1's geometry with 8 or 6 query heads per KV head."""
    return bench.make_int8_cache(LAYERS, Hq=request.param, P=P, dev=torch.device("cuda:0"))


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_int8_wide_gqa_one_launch(int8_wide, mode):
    """6 and 8 query heads per KV head over the INT8 cache at config 1's
    geometry: one launch (two virtual heads of 3 or 4 query heads per KV
    head), selection equal to the oracle's and to the split path's, O within
    the bar on sampled layers."""
    from flashquest_amd.eager.decode import _one_launch, quest_decode_int8
    ic = int8_wide
    Q = ic["Q"]
    Hq = Q.shape[-3]
    keys = ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")
    planes_dev = [ic[k] for k in keys]
    assert _one_launch(8, Q, planes_dev, Hq // 8, 64, mode, 4, 2, 128)
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=128, select_mode=mode)
    o, lse, mask = quest_decode_int8(Q, *planes_dev, return_selection=True, **kw)
    o2, lse2 = quest_decode_int8(Q, *planes_dev, **kw)
    with L.attention_splits(4):
        os_, lses, masks = quest_decode_int8(Q, *planes_dev, return_selection=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(mask, masks)
    m_host = mask.cpu().numpy()
    rows = amb = amb_diff = 0
    err_max = 0.0
    for l in (0, 9, 27):
        q = Q[l:l + 1, :, 0].float().cpu().numpy()
        planes = _host4(ic, keys, l)
        scores = O.page_scores_fixed(q, planes[1], planes[2], mode, 255.0)
        ref_mask = O.select_pages_vectorized(scores[:, :, None, :], 0.25, 4, 2, 128)[:, :, 0, :]
        if mode == "per_kv_head_sum":
            ref_mask = np.repeat(ref_mask, Hq // 8, axis=1)
        assert np.array_equal(m_host[l:l + 1], ref_mask), l
        n, a, mis, ad = fp64_selection_check(q, planes[1], planes[2], m_host[l:l + 1], 0.25, mode, levels=255.0)
        assert mis == 0, l
        rows, amb, amb_diff = rows + n, amb + a, amb_diff + ad
        if l in (0, 27):
            ref_o, ref_l = O.sparse_int8_attention(q, *planes, ref_mask, 64)
            err = float(np.abs(o[l:l + 1, :, 0].float().cpu().numpy() - ref_o).max())
            err_max = max(err_max, err)
            assert err <= _qtol("bf16", ref_o), (l, err)
            assert np.abs(lse[l:l + 1, :, 0].cpu().numpy() - ref_l).max() <= TOL_LSE
    d = (o.float() - os_.float()).abs().max().item()
    assert d <= 2 * _qtol("bf16", np.array([2.0]))
    _report(f"int8 {Hq} query heads {mode}", rows=rows, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
            max_abs_O=f"{err_max:.3e}", fused_vs_split=f"{d:.3e}")


@pytest.mark.parametrize("qdtype", ["bf16", "f16"])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_turbo_fused_step_at_size(turbo_cfg1, mode, qdtype):
    """TurboQuant K3-V3 at config 1's geometry through the single-launch
    kernel; bf16 queries (the reference's) and fp16 queries (flat 2e-3)."""
    from flashquest_amd.eager.decode import quest_decode_turbo
    tc = turbo_cfg1
    Q = tc["Q"] if qdtype == "bf16" else tc["Q"].half()
    keys = ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=128, select_mode=mode)
    args = [Q] + [tc[k] for k in keys] + [tc["K_scale_raw"], tc["K_mn_raw"]]
    o, lse, mask = quest_decode_turbo(*args, return_selection=True, **kw)
    o2, lse2 = quest_decode_turbo(*args, **kw)
    with L.attention_splits(4):
        os_, lses, masks = quest_decode_turbo(*args, return_selection=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(mask, masks)
    m_host = mask.cpu().numpy()
    rows = amb = amb_diff = 0
    err_max = 0.0
    for l in range(LAYERS):
        q = Q[l:l + 1, :, 0].float().cpu().numpy()
        ksr, kmr = _host4(tc, ("K_scale_raw", "K_mn_raw"), l)
        scores = O.page_scores_fixed(q, ksr, kmr, mode)
        ref_mask = O.select_pages_vectorized(scores[:, :, None, :], 0.25, 4, 2, 128)[:, :, 0, :]
        if mode == "per_kv_head_sum":
            ref_mask = np.repeat(ref_mask, 3, axis=1)
        assert np.array_equal(m_host[l:l + 1], ref_mask), l
        n, a, mis, ad = fp64_selection_check(q, ksr, kmr, m_host[l:l + 1], 0.25, mode)
        assert mis == 0, l
        rows, amb, amb_diff = rows + n, amb + a, amb_diff + ad
        if l in (0, 27):
            ref_o, ref_l = O.sparse_turbo_attention(q, *_host4(tc, keys, l), ref_mask, 64)
            err = float(np.abs(o[l:l + 1, :, 0].float().cpu().numpy() - ref_o).max())
            err_max = max(err_max, err)
            assert err <= _qtol(qdtype, ref_o), (l, err)
            assert np.abs(lse[l:l + 1, :, 0].cpu().numpy() - ref_l).max() <= TOL_LSE
    d = (o.float() - os_.float()).abs().max().item()
    assert d <= 2 * _qtol(qdtype, np.array([2.0]))
    _report(f"turbo {mode} q={qdtype}", rows=rows, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
            max_abs_O=f"{err_max:.3e}", fused_vs_split=f"{d:.3e}")


@pytest.fixture(scope="module", params=[64, 48], ids=["gqa8", "gqa6"])
def turbo_wide(request):
    """The TurboQuant caches of config 1's geometry with 8 or 6 query heads per KV head."""
    return bench.make_turbo_cache(LAYERS, Hq=request.param, P=P, dev=torch.device("cuda:0"))


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_turbo_wide_gqa_one_launch(turbo_wide, mode):
    """6 and 8 query heads per KV head over the TurboQuant cache at config 1's
    geometry: one launch (two virtual heads of 3 or 4 query heads per KV
    head), selection equal to the oracle's and to the split path's, O within
    the bar on sampled layers."""
    from flashquest_amd.eager.decode import _one_launch, quest_decode_turbo
    tc = turbo_wide
    Q = tc["Q"]
    Hq = Q.shape[-3]
    keys = ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")
    raw = (tc["K_scale_raw"], tc["K_mn_raw"])
    assert _one_launch(3, Q, [tc[k] for k in keys], Hq // 8, 64, mode, 4, 2, 128, raw=raw)
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=128, select_mode=mode)
    args = [Q] + [tc[k] for k in keys] + list(raw)
    o, lse, mask = quest_decode_turbo(*args, return_selection=True, **kw)
    o2, lse2 = quest_decode_turbo(*args, **kw)
    with L.attention_splits(4):
        os_, lses, masks = quest_decode_turbo(*args, return_selection=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(mask, masks)
    m_host = mask.cpu().numpy()
    rows = amb = amb_diff = 0
    err_max = 0.0
    for l in (0, 9, 27):
        q = Q[l:l + 1, :, 0].float().cpu().numpy()
        ksr, kmr = _host4(tc, ("K_scale_raw", "K_mn_raw"), l)
        scores = O.page_scores_fixed(q, ksr, kmr, mode)
        ref_mask = O.select_pages_vectorized(scores[:, :, None, :], 0.25, 4, 2, 128)[:, :, 0, :]
        if mode == "per_kv_head_sum":
            ref_mask = np.repeat(ref_mask, Hq // 8, axis=1)
        assert np.array_equal(m_host[l:l + 1], ref_mask), l
        n, a, mis, ad = fp64_selection_check(q, ksr, kmr, m_host[l:l + 1], 0.25, mode)
        assert mis == 0, l
        rows, amb, amb_diff = rows + n, amb + a, amb_diff + ad
        if l in (0, 27):
            ref_o, ref_l = O.sparse_turbo_attention(q, *_host4(tc, keys, l), ref_mask, 64)
            err = float(np.abs(o[l:l + 1, :, 0].float().cpu().numpy() - ref_o).max())
            err_max = max(err_max, err)
            assert err <= _qtol("bf16", ref_o), (l, err)
            assert np.abs(lse[l:l + 1, :, 0].cpu().numpy() - ref_l).max() <= TOL_LSE
    d = (o.float() - os_.float()).abs().max().item()
    assert d <= 2 * _qtol("bf16", np.array([2.0]))
    _report(f"turbo {Hq} query heads {mode}", rows=rows, ambiguous_rows=amb, ambiguous_resolved_differently=amb_diff,
            max_abs_O=f"{err_max:.3e}", fused_vs_split=f"{d:.3e}")


def test_read_only_pass_runs_on_config1(cfg1):
    """The bench's ceiling probe (fq_read_decode_pages) takes config 1's cache
    and the decode's own selection mask and completes."""
    from flashquest_amd._probe import read_decode_pages
    planes = [cfg1[k] for k in PLANES]
    _, _, mask = quest_decode_int4(cfg1["Q"], *planes, retention=0.25, num_sinks=4, window_pages=2,
                                   return_selection=True)
    for _ in range(2):
        read_decode_pages(*planes, mask)
    torch.cuda.synchronize()


def test_stream_read_probe_runs_and_checks_its_buffer():
    """The bench's plain-read reference (fq_read_stream) reads a config-1-sized
    buffer, and refuses sizes that are not whole 16-byte chunks."""
    from flashquest_amd._probe import read_stream
    buf = torch.zeros(332717696, dtype=torch.uint8, device="cuda")
    for _ in range(2):
        read_stream(buf)
    torch.cuda.synchronize()
    with pytest.raises(ValueError):
        read_stream(buf[:100])
