"""fq_quest_decode_int4_noalloc (the decode step on the library's static
device scratch, for callers that cannot allocate) against fq_quest_decode_int4
with a caller workspace: bit-exact O, lse and selection on two calls in a row,
the second smaller, both on the split path (few KV groups), which is the path
that uses the scratch; and a step too large for the scratch is refused before
any pointer is touched."""
import numpy as np
import pytest
import torch

from flashquest_amd import _lib as L
from flashquest_amd import _ops
from tests.cases import Int4Case

pytestmark = pytest.mark.gpu


def _descriptors(case, retention):
    d = case.device()
    q = case.q_dev()[:, :, 0]
    cache, keep = _ops.int4_cache(d["K_packed"], d["K_scale"], d["K_mn"], d["V_packed"], d["V_scale"], d["V_mn"],
                                  64)
    return cache, keep, q, _ops.retention_tensor(retention, case.Hq, q.device)


def _run(case, noalloc):
    cache, keep, q, r = _descriptors(case, 0.3)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:-1], dtype=torch.float32, device=q.device)
    mask = torch.empty(q.shape[:-1] + (case.P,), dtype=torch.bool, device=q.device)
    query = _ops.query(q, o, lse, None)
    stream = L.stream_handle(q.device)
    if noalloc:
        rc = L.lib().fq_quest_decode_int4_noalloc(cache, query, r.data_ptr(), 2, 1, -1, L.FQ_SELECT_PER_Q_HEAD,
                                                  None, mask.data_ptr(), stream)
    else:
        ws = torch.empty(L.lib().fq_workspace_bytes(cache, case.Hq), dtype=torch.uint8, device=q.device)
        rc = L.lib().fq_quest_decode_int4(cache, query, r.data_ptr(), 2, 1, -1, L.FQ_SELECT_PER_Q_HEAD, None,
                                          mask.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    L.check(rc, "decode")
    torch.cuda.synchronize()
    return o, lse, mask


def test_noalloc_matches_workspace_entry_two_calls():
    torch.cuda.set_device(0)
    big = Int4Case(seed=91, B=3, Hq=24, Hkv=8, S=64 * 100 + 21, D=128, page=64, dtype="f16", meta="f16",
                   vgroup=32)
    small = Int4Case(seed=92, B=1, Hq=6, Hkv=2, S=64 * 20 + 17, D=128, page=64, dtype="bf16", meta="bf16")
    for case in (big, small):
        ref = _run(case, noalloc=False)
        got = _run(case, noalloc=True)
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
        assert bool(got[2].any())


def test_noalloc_refuses_oversized_step_before_touching_memory():
    c = L.Int4Cache()
    c.L, c.B, c.H_kv, c.P, c.D, c.S, c.page_size, c.v_groups = 28, 16, 8, 512, 128, 32768, 64, 4
    q = L.Query()
    q.H_q = 24
    assert L.lib().fq_workspace_bytes(c, 24) > 64 << 20
    rc = L.lib().fq_quest_decode_int4_noalloc(c, q, None, 4, 2, 128, L.FQ_SELECT_PER_KV_HEAD_SUM, None, None, None)
    assert rc == L.FQ_ERR_UNSUPPORTED
    assert b"static buffer" in L.lib().fq_last_error()
