"""Host-side plumbing of the per-call operators (no GPU): descriptors built
from tensors carry exactly the tensors' addresses, strides and shapes, and
scalar retentions become one shared, read-only device vector per (value,
heads, device)."""
import pytest
import torch

from flashquest_amd import _lib as L
from flashquest_amd import _ops


def _planes(lead=(), S=256, P=4, D=128, G=4, meta=torch.float16):
    kp = torch.zeros(*lead, 2, 8, S, D // 2, dtype=torch.uint8)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(*lead, 2, 8, P, D, dtype=meta)
    km = torch.zeros_like(ks)
    vs = torch.zeros(*lead, 2, 8, S, G, dtype=meta)
    vm = torch.zeros_like(vs)
    return kp, ks, km, vp, vs, vm


@pytest.mark.parametrize("lead", [(), (3,)])
def test_int4_descriptor_fields(lead):
    kp, ks, km, vp, vs, vm = _planes(lead)
    c, keep = _ops.int4_cache(kp, ks, km, vp, vs, vm, 64)
    pad = [0] * (1 - len(lead))
    assert c.k_packed == kp.data_ptr() and c.v_mn == vm.data_ptr()
    assert list(c.k_strides) == pad + list(kp.stride()) and list(c.vs_strides) == pad + list(vs.stride())
    assert (c.L, c.B, c.H_kv, c.S, c.P, c.D, c.page_size, c.v_groups) == \
        ((lead[0] if lead else 1), 2, 8, 256, 4, 128, 64, 4)
    assert c.meta_dtype == L.FQ_F16
    assert all(a is b for a, b in zip(keep, (kp, vp, ks, km, vs, vm)))


def test_int4_descriptor_rejects_mixed_ranks_and_copies_misaligned_views():
    kp, ks, km, vp, vs, vm = _planes()
    with pytest.raises(ValueError):
        _ops.int4_cache(kp, ks[0], km, vp, vs, vm, 64)
    # a K-metadata view whose rows are not 8-element aligned is copied, not passed on
    wide = torch.zeros(2, 8, 4, 136, dtype=torch.float16)[..., 3:131]
    c, keep = _ops.int4_cache(kp, wide, km, vp, vs, vm, 64)
    assert keep[2] is not wide and keep[2].is_contiguous() and c.k_scale == keep[2].data_ptr()


def test_query_descriptor_fields():
    q = torch.zeros(2, 24, 128, dtype=torch.bfloat16)
    o = torch.zeros(2, 24, 128, dtype=torch.float32)
    lse = torch.zeros(2, 24, dtype=torch.float32)
    d = _ops.query(q, o, lse, None)
    assert d.q == q.data_ptr() and d.out == o.data_ptr() and d.lse == lse.data_ptr()
    assert list(d.q_strides) == [0] + list(q.stride()) and list(d.lse_strides) == [0] + list(lse.stride())
    assert (d.q_dtype, d.out_dtype, d.H_q) == (L.FQ_BF16, L.FQ_F32, 24)
    assert abs(d.sm_scale - 128 ** -0.5) < 1e-7 and d.retention_layer_stride == 0 and not d.rotation_signs
    nolse = _ops.query(q, o, None, 0.5)
    assert not nolse.lse and list(nolse.lse_strides) == [0, 0, 0] and nolse.sm_scale == 0.5
    with pytest.raises(ValueError):
        _ops.query(q, o[0], None, None)


def test_scalar_retention_vectors_are_shared_and_bounded():
    a = _ops.retention_tensor(0.25, 24, "cpu")
    assert a.shape == (24,) and a.dtype == torch.float32 and bool((a == 0.25).all())
    assert _ops.retention_tensor(0.25, 24, torch.device("cpu")) is a
    b = _ops.retention_tensor(0.5, 24, "cpu")
    assert b is not a and bool((b == 0.5).all())
    assert _ops.retention_tensor(0.25, 12, "cpu") is not a
    for i in range(300):
        _ops.retention_tensor(i / 1000.0, 4, "cpu")
    assert len(_ops._scalar_retention) <= 256
    with pytest.raises(ValueError):
        _ops.retention_tensor(1.5, 24, "cpu")
    per_head = torch.linspace(0, 1, 24)
    assert torch.equal(_ops.retention_tensor(per_head, 24, "cpu"), per_head)


def _turbo_desc(S=256, P=4, D=128, Hkv=2):
    c = L.TurboCache()
    c.k_msb = c.v_msb = c.k_lsb = c.v_lsb = c.k_scale = c.v_scale = 4096
    c.kmsb_strides = c.vmsb_strides = L.i64([0, Hkv * S * D // 8, S * D // 8, D // 8, 1], 5)
    c.klsb_strides = c.vlsb_strides = L.i64([0, Hkv * S * D // 4, S * D // 4, D // 4, 1], 5)
    c.kst_strides = c.vst_strides = L.i64([0, Hkv * S, S, 1, 1], 5)
    c.L, c.B, c.H_kv, c.S, c.P, c.D, c.page_size = 1, 1, Hkv, S, P, D, 64
    return c


@pytest.mark.parametrize("field,value,code,msg", [("v_scale", 4097, "FQ_ERR_UNSUPPORTED", "aligned"),
                                                  ("k_scale", 4097, "FQ_ERR_UNSUPPORTED", "aligned"),
                                                  ("v_lsb", None, "FQ_ERR_INVALID", "NULL cache tensor"),
                                                  ("D", 96, "FQ_ERR_UNSUPPORTED", "head_dim"),
                                                  ("P", 0, "FQ_ERR_UNSUPPORTED", "pages"),
                                                  ("P", 5, "FQ_ERR_INVALID", "tokens of page_size"),
                                                  ("P", 9, "FQ_ERR_INVALID", "tokens of page_size")])
def test_turbo_descriptor_checks_before_any_launch(field, value, code, msg):
    """Every TurboQuant decode entry rejects a misaligned per-token scale, a
    missing plane, an unsupported head_dim or page count, including more pages
    than the planes' tokens fill (the raw K metadata would be read past what
    the caller wrote; no GPU needed: the checks run before anything reaches
    the device)."""
    lib = L.lib()
    c = _turbo_desc()
    setattr(c, field, value)
    want = getattr(L, code)
    z5 = L.i64([0, 0, 0, 0, 1], 5)
    assert lib.fq_quest_decode_turbo(c, 4096, z5, 4096, z5, None, None, 0, 0, -1, 0, None, None, 0, None) == want
    assert msg in lib.fq_last_error().decode()
    assert lib.fq_sparse_turbo_fwd_mask(c, None, None, L.i64([0, 0, 0, 1], 4), None, 0, None) == want
    assert msg in lib.fq_last_error().decode()
    assert lib.fq_quest_select_turbo(c, 4096, z5, 4096, z5, None, None, 0, 0, -1, 0, None, None, 0, None) == want
    assert msg in lib.fq_last_error().decode()
    # the unmodified descriptor passes the cache checks and stops at the missing query
    assert lib.fq_quest_decode_turbo(_turbo_desc(), 4096, z5, 4096, z5, None, None, 0, 0, -1, 0, None, None, 0,
                                     None) == L.FQ_ERR_INVALID
    assert msg not in lib.fq_last_error().decode()


def test_turbo_cache_rejects_more_pages_than_its_tokens():
    """The Python descriptor builder refuses a page count past the planes'
    tokens (a per-token plane's length is not a page count) before any call."""
    S, D = 64 * 3 + 10, 128
    planes = [torch.zeros(1, 2, S, D // 8, dtype=torch.uint8), torch.zeros(1, 2, S, D // 4, dtype=torch.uint8),
              torch.zeros(1, 2, S, 1, dtype=torch.bfloat16)] * 2
    _ops.turbo_cache(*planes, 4, 64)
    with pytest.raises(ValueError, match="pages"):
        _ops.turbo_cache(*planes, 5, 64)
    with pytest.raises(ValueError, match="pages"):
        _ops.turbo_cache(*planes, S, 64)


@pytest.mark.parametrize("stride,ok", [(0, True), (24, True), (48, True), (1, False), (23, False), (-24, False)])
def test_retention_layer_stride_is_zero_or_a_whole_row(stride, ok):
    """fq_query.retention_layer_stride is 0 (one row for every layer) or at
    least H_q (one row per layer); a stride that would make layers read
    overlapping rows is refused before anything reaches the device."""
    kp, ks, km, vp, vs, vm = _planes()
    c, keep = _ops.int4_cache(kp, ks, km, vp, vs, vm, 64)
    q = torch.zeros(2, 24, 128, dtype=torch.float16)
    d = _ops.query(q, torch.zeros_like(q), None, None)
    d.retention_layer_stride = stride
    rc = L.lib().fq_quest_decode_int4(c, d, None, 4, 2, -1, 0, None, None, None, 0, None)
    msg = L.lib().fq_last_error().decode()
    if ok:
        assert "retention layer stride" not in msg
    else:
        assert rc == L.FQ_ERR_INVALID and "retention layer stride" in msg


def test_strided_per_head_retention_is_made_contiguous():
    r = torch.linspace(0, 1, 48)[::2]
    t = _ops.retention_tensor(r, 24, "cpu")
    assert t.is_contiguous() and torch.equal(t, r)


@pytest.mark.parametrize("nrep", [5, 7])
def test_padded_heads_round_trip_and_retention(nrep):
    """The padded step of 5 or 7 query heads per KV head: every group gains
    one zero head at its end, the real heads come back unchanged (as a copy,
    or in place through the grouped view), and the padded retention keeps the
    real heads' values with 0 for the extra head (scalar and per-head)."""
    from flashquest_amd.eager.decode import _pad_heads, _padded_retention, _real_heads
    H_kv, D = 3, 8
    Q = torch.randn(2, 4, H_kv * nrep, 1, D)
    Qp = _pad_heads(Q, 2, H_kv, nrep)
    assert Qp.shape == (2, 4, H_kv * (nrep + 1), 1, D)
    g = Qp.unflatten(2, (H_kv, nrep + 1))
    assert torch.equal(g[:, :, :, nrep], torch.zeros_like(g[:, :, :, nrep]))
    assert torch.equal(_real_heads(Qp, 2, H_kv, nrep), Q)
    Q2 = torch.randn_like(Q)
    _real_heads(Qp, 2, H_kv, nrep, grouped=True).copy_(Q2.unflatten(2, (H_kv, nrep)))
    assert torch.equal(_real_heads(Qp, 2, H_kv, nrep), Q2)       # written in place
    r = _padded_retention(0.3, H_kv * nrep, H_kv, nrep, "cpu")
    want = torch.tensor(([0.3] * nrep + [0.0]) * H_kv, dtype=torch.float32)
    assert torch.equal(r, want)
    per_head = torch.arange(H_kv * nrep, dtype=torch.float32) / 100
    rp = _padded_retention(per_head, H_kv * nrep, H_kv, nrep, "cpu").unflatten(0, (H_kv, nrep + 1))
    assert torch.equal(rp[:, :nrep].flatten(), per_head) and not rp[:, nrep].any()


def test_library_takes_six_and_eight_heads_per_kv_head_itself():
    """fq_quest_fused_int4 (host logic only, no launch): 6 and 8 query heads
    per KV head run on virtual KV heads in the library whether the step is
    one launch (28 layers) or the split form (one layer); 7 does not (the
    Python layer pads it to 8); above 8 the entry refuses the query."""
    Hkv, P, D = 8, 64, 128
    S = P * 64
    for layers in (28, 1):
        planes = (torch.zeros(layers, 1, Hkv, S, D // 2, dtype=torch.uint8),
                  torch.zeros(layers, 1, Hkv, P, D, dtype=torch.float16),
                  torch.zeros(layers, 1, Hkv, P, D, dtype=torch.float16),
                  torch.zeros(layers, 1, Hkv, S, D // 2, dtype=torch.uint8),
                  torch.zeros(layers, 1, Hkv, S, 4, dtype=torch.float16),
                  torch.zeros(layers, 1, Hkv, S, 4, dtype=torch.float16))
        cache, keep = _ops.int4_cache(*planes, 64)
        for Hq, want in ((24, 1), (48, 1), (64, 1), (56, 0)):
            Q3 = torch.zeros(layers, 1, Hq, D, dtype=torch.float16)
            q = _ops.query(Q3, Q3, None, None)
            for mode in (0, 1):
                assert L.lib().fq_quest_fused_int4(cache, q, 4, 2, 16, mode) == want, (layers, Hq, mode)
        Q3 = torch.zeros(layers, 1, 72, D, dtype=torch.float16)
        assert L.lib().fq_quest_fused_int4(cache, _ops.query(Q3, Q3, None, None), 4, 2, 16, 0) < 0
