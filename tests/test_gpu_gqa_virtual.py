"""6 and 8 query heads per KV head in single-layer decode steps (the
reference's per-layer call pattern, llama_persistent_patch.py:196-245).

The matrix-core kernels take at most 4 query heads per workgroup.  For 6 or 8
the library runs every KV head as two virtual KV heads of 3 or 4 query heads:
a single layer's 8 KV heads are too few to fill the GPU, so the step is the
split form (a scoring launch over the real KV heads, attention workgroups
that each select from those scores and attend a slice of the list, the split
merge).  per_kv_head_sum selects from the summed query of all the head's
queries in every virtual head.  Checked against the oracle (selection bit for
bit, O and lse within the decode bar), with and without a partial-page tail,
and replayed from a HIP graph.
"""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import Int4Case, Int8Case, decode_tol, max_err, to_dev_half

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("Hq", [64, 48])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
@pytest.mark.parametrize("P", [200, 512])
def test_single_layer_step_virtual_heads(bits, Hq, mode, P):
    from flashquest_amd.eager.decode import _one_launch, quest_decode_int4, quest_decode_int8
    S = 64 * (P - 1) + 29
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=None, select_mode=mode)
    ref_kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=None, mode=mode)
    print(f"[virtual heads] bits={bits} Hq={Hq} mode={mode} P={P}", flush=True)
    if bits == 4:
        c = Int4Case(seed=900 + Hq + P, B=1, Hq=Hq, Hkv=8, S=S, D=128, dtype="f16", meta="f16", vgroup=32)
        dev = c.device()
        planes = [dev[k] for k in ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")]
        assert _one_launch(4, c.q_dev(), planes, Hq // 8, 64, mode, 4, 2, None)
        o, lse, mask = quest_decode_int4(c.q_dev(), *planes, return_selection=True, **kw)
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, **ref_kw)
        tol = decode_tol(ref["O"], "f16")
    else:
        c = Int8Case(seed=950 + Hq + P, B=1, Hq=Hq, Hkv=8, S=S, D=128)
        dev = c.device()
        planes = [dev[k] for k in ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")]
        assert _one_launch(8, c.q_dev(), planes, Hq // 8, 64, mode, 4, 2, None)
        o, lse, mask = quest_decode_int8(c.q_dev(), *planes, return_selection=True, **kw)
        ref = O.decode_step(c.Q, c.ku, c.ks, c.km, c.vu, c.vs, c.vm, bits=8, **ref_kw)
        tol = decode_tol(ref["O"], "bf16")
    torch.cuda.synchronize()
    assert np.array_equal(mask.cpu().numpy(), ref["mask"])
    assert max_err(o[:, :, 0], ref["O"]) <= tol
    assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4


@pytest.mark.parametrize("Hq", [64, 48])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_single_layer_step_virtual_heads_with_tail(Hq, mode):
    """The partial page attended inside the attention workgroups of every
    virtual head (split 0 of each), then merged with the pages."""
    from flashquest_amd.eager.decode import quest_decode_int4
    P, T = 300, 37
    c = Int4Case(seed=990 + Hq, B=1, Hq=Hq, Hkv=8, S=64 * P, D=128, dtype="f16", meta="f16", vgroup=32)
    rng = np.random.default_rng(Hq)
    kt = O.round_bf16(rng.standard_normal((1, 8, T, 128)).astype(np.float32))
    vt = O.round_bf16(rng.standard_normal((1, 8, T, 128)).astype(np.float32))
    o, lse = quest_decode_int4(c.q_dev(), **c.device(), retention=0.25, num_sinks=4, window_pages=2,
                               select_mode=mode, K_tail=to_dev_half(kt, "bf16"), V_tail=to_dev_half(vt, "bf16"))
    torch.cuda.synchronize()
    ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=0.25, num_sinks=4, window_pages=2,
                        mode=mode)
    ot, lt = O.dense_attn_with_lse(c.Q, kt, vt)
    ro = O.merge_two_attentions(ref["O"], ref["lse"], ot, lt)
    m = np.maximum(ref["lse"], lt)
    rl = m + np.log(np.exp(ref["lse"] - m) + np.exp(lt - m))
    assert max_err(o[:, :, 0], ro) <= decode_tol(ro, "f16")
    assert max_err(lse[:, :, 0], rl) <= 1e-4


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_per_layer_graph_virtual_heads(mode):
    """Four single-layer steps (64 query / 8 KV heads, 256 pages) captured in
    one HIP graph: every replay, with new queries written in place between
    them, equals the same steps run eagerly bit for bit."""
    from flashquest_amd.eager.decode import QuestDecoder
    layers, P = 4, 256
    cases = [Int4Case(seed=1400 + i, B=1, Hq=64, Hkv=8, S=64 * P, D=128, dtype="f16", meta="f16", vgroup=32)
             for i in range(layers)]
    keys = ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")
    devs = [c.device() for c in cases]
    Qs = [c.q_dev() for c in cases]
    decs = [QuestDecoder(Qs[l], *[devs[l][k] for k in keys], retention=0.25, num_sinks=4, window_pages=2,
                         k_max_static=64, select_mode=mode) for l in range(layers)]
    assert all(d._chunked is None for d in decs), "the library takes these steps itself"
    for d in decs:
        d()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for d in decs:
            d()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for d in decs:
                d()
    torch.cuda.synchronize()
    for rep in range(3):
        for q in Qs:
            q.copy_(torch.randn(q.shape, device=q.device).to(q.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [d.O3.clone() for d in decs]
        for d in decs:
            d()
        torch.cuda.synchronize()
        for l, d in enumerate(decs):
            assert torch.equal(got[l], d.O3), (rep, l)
        assert bool(torch.isfinite(got[0]).all())


@pytest.mark.parametrize("Hq", [64, 48])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_turbo_single_layer_step_virtual_heads(Hq, mode):
    """The same over the TurboQuant cache (scores from the raw K page metadata,
    codebook attention), one layer of the bench's synthetic TurboQuant cache."""
    import bench
    from flashquest_amd.eager.decode import _one_launch, quest_decode_turbo
    P = 300
    tc = bench.make_turbo_cache(1, Hq=Hq, P=P, dev=torch.device("cuda:0"))
    keys = ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")
    raw = (tc["K_scale_raw"], tc["K_mn_raw"])
    Q = tc["Q"]
    assert _one_launch(3, Q, [tc[k] for k in keys], Hq // 8, 64, mode, 4, 2, None, raw=raw)
    o, lse, mask = quest_decode_turbo(Q, *[tc[k] for k in keys], *raw, retention=0.25, num_sinks=4,
                                      window_pages=2, select_mode=mode, return_selection=True)
    torch.cuda.synchronize()
    q = Q[:, :, 0].float().cpu().numpy()
    host = {k: (tc[k].cpu().numpy() if tc[k].dtype == torch.uint8 else tc[k].float().cpu().numpy())
            for k in keys + ("K_scale_raw", "K_mn_raw")}
    scores = O.page_scores_fixed(q, host["K_scale_raw"], host["K_mn_raw"], mode)
    ref_mask = O.select_pages_vectorized(scores[:, :, None, :], 0.25, 4, 2)[:, :, 0, :]
    if mode == "per_kv_head_sum":
        ref_mask = np.repeat(ref_mask, Hq // 8, axis=1)
    assert np.array_equal(mask.cpu().numpy(), ref_mask)
    ref_o, ref_l = O.sparse_turbo_attention(q, *[host[k] for k in keys], ref_mask, 64)
    assert max_err(o[:, :, 0], ref_o) <= decode_tol(ref_o, "bf16")
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4


@pytest.mark.parametrize("bits", [4, 8, 3])
@pytest.mark.parametrize("Hq", [56, 40])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
@pytest.mark.parametrize("layers", [1, 12])
def test_padded_step_five_and_seven_heads(bits, Hq, mode, layers):
    """5 and 7 query heads per KV head as a step of 6 or 8 with a zero query
    head per group (retention 0: it selects only the forced pages); the real
    heads' selection, O and lse against the oracle.  12 layers x 8 KV heads:
    one launch; one layer: the split form."""
    import bench
    from flashquest_amd.eager.decode import _one_launch, _pad_heads, quest_decode_int4, quest_decode_int8, \
        quest_decode_turbo
    P, nrep = 160, Hq // 8
    dev = torch.device("cuda:0")
    print(f"[padded] bits={bits} Hq={Hq} mode={mode} layers={layers}", flush=True)
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, select_mode=mode, return_selection=True)
    if bits == 4:
        c = bench.make_cache(layers, 1, Hq=Hq, P=P, dev=dev)
        keys = ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")
        Q = c["Q"]
        Qp = _pad_heads(Q, Q.dim() - 3, 8, nrep)
        assert _one_launch(4, Qp, [c[k] for k in keys], nrep + 1, 64, mode, 4, 2, None)
        o, lse, mask = quest_decode_int4(Q, *[c[k] for k in keys], **kw)
        host = lambda l: [c[k][l, 0:1].cpu().numpy() if c[k].dtype == torch.uint8 else c[k][l, 0:1].float().cpu().numpy()
                          for k in keys]
        q_of = lambda l: Q[l, 0:1, :, 0].float().cpu().numpy()
        pick = lambda t, l: t[l]
    elif bits == 8:
        c = bench.make_int8_cache(layers, Hq=Hq, P=P, dev=dev)
        keys = ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")
        Q = c["Q"]
        o, lse, mask = quest_decode_int8(Q, *[c[k] for k in keys], **kw)
        host = lambda l: [c[k][l:l + 1].cpu().numpy() if c[k].dtype == torch.uint8 else c[k][l:l + 1].float().cpu().numpy()
                          for k in keys]
        q_of = lambda l: Q[l:l + 1, :, 0].float().cpu().numpy()
        pick = lambda t, l: t[l:l + 1]
    else:
        c = bench.make_turbo_cache(layers, Hq=Hq, P=P, dev=dev)
        keys = ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")
        Q = c["Q"]
        o, lse, mask = quest_decode_turbo(Q, *[c[k] for k in keys], c["K_scale_raw"], c["K_mn_raw"], **kw)
        host = lambda l: [c[k][l:l + 1].cpu().numpy() if c[k].dtype == torch.uint8 else c[k][l:l + 1].float().cpu().numpy()
                          for k in keys + ("K_scale_raw", "K_mn_raw")]
        q_of = lambda l: Q[l:l + 1, :, 0].float().cpu().numpy()
        pick = lambda t, l: t[l:l + 1]
    torch.cuda.synchronize()
    assert o.shape == Q.shape and mask.shape[-2] == Hq
    for l in sorted({0, layers - 1}):
        q, pl = q_of(l), host(l)
        if bits == 3:
            scores = O.page_scores_fixed(q, pl[6], pl[7], mode)
        else:
            scores = O.page_scores_fixed(q, pl[1], pl[2], mode, 255.0 if bits == 8 else 15.0)
        ref_mask = O.select_pages_vectorized(scores[:, :, None, :], 0.25, 4, 2)[:, :, 0, :]
        if mode == "per_kv_head_sum":
            ref_mask = np.repeat(ref_mask, nrep, axis=1)
        got_mask = pick(mask, l).cpu().numpy().reshape(ref_mask.shape)
        assert np.array_equal(got_mask, ref_mask), l
        if bits == 3:
            ref_o, ref_l = O.sparse_turbo_attention(q, *pl[:6], ref_mask, 64)
        elif bits == 8:
            ref_o, ref_l = O.sparse_int8_attention(q, *pl, ref_mask, 64)
        else:
            ref_o, ref_l = O.sparse_int4_attention(q, *pl, ref_mask, 64)
        got_o = pick(o, l)[..., 0, :].reshape(ref_o.shape)
        got_l = pick(lse, l)[..., 0].reshape(ref_l.shape)
        assert max_err(got_o, ref_o) <= decode_tol(ref_o, "f16" if bits == 4 else "bf16"), l
        assert max_err(got_l, ref_l) <= 1e-4, l


@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
def test_padded_decoder_graph(mode):
    """QuestDecoder with 7 query heads per KV head (the padded step: q copied
    into the padded query, O copied out) captured in a HIP graph: every
    replay equals the eager step bit for bit, and the eager step the
    functional operator."""
    import bench
    from flashquest_amd.eager.decode import QuestDecoder, quest_decode_int4
    c = bench.make_cache(12, 1, Hq=56, P=96, dev=torch.device("cuda:0"))
    keys = ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")
    Q = c["Q"]
    d = QuestDecoder(Q, *[c[k] for k in keys], retention=0.25, num_sinks=4, window_pages=2, k_max_static=24,
                     select_mode=mode)
    assert d._padded is not None and d.fused
    d()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        d()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            d()
    torch.cuda.synchronize()
    for rep in range(3):
        Q.copy_(torch.randn(Q.shape, device=Q.device).to(Q.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = d.O3.clone()
        d()
        torch.cuda.synchronize()
        assert torch.equal(got, d.O3), rep
    want, _ = quest_decode_int4(Q, *[c[k] for k in keys], retention=0.25, num_sinks=4, window_pages=2,
                                k_max_static=24, select_mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(want[..., 0, :], d.O3)
