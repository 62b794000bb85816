"""Decode steps captured in a HIP graph (the per-layer call pattern the bench
times as a graph, and the fused multi-layer step) replay correctly: each of
several replays, with the program's own eager work and synchronisations
between them (new queries written in place), equals the same steps run
eagerly on the same inputs bit for bit, and the functional operator within
the decode bar.  The library records no memset into a captured graph; its
workspace is allocated by the eager call before capture."""
import numpy as np
import pytest
import torch

from tests.cases import Int4Case, to_dev_half

pytestmark = pytest.mark.gpu

PLANES = ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")


def _capture(calls):
    for f in calls:                       # eager first: sizes the workspace
        f()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for f in calls:
            f()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for f in calls:
                f()
    torch.cuda.synchronize()
    return graph


@pytest.mark.parametrize("per_layer,mode,tail,Hq", [(True, "per_kv_head_sum", 0, 24), (True, "per_q_head", 37, 24),
                                                    (False, "per_kv_head_sum", 0, 24), (False, "per_q_head", 21, 24),
                                                    (True, "per_q_head", 0, 64), (False, "per_kv_head_sum", 0, 64),
                                                    (True, "per_kv_head_sum", 30, 64)])
def test_graph_replays_equal_the_eager_step(per_layer, mode, tail, Hq):
    """Hq = 64 (8 query heads per KV head): the chunked step, captured."""
    from flashquest_amd.eager.decode import QuestDecoder, quest_decode_int4
    layers, Hkv, P = 6, 8, 40
    cases = [Int4Case(seed=300 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128, dtype="f16", meta="f16", vgroup=32)
             for i in range(layers)]
    dev = [c.device() for c in cases]
    planes = {k: torch.stack([d[k] for d in dev]) for k in PLANES}          # (L, 1, H_kv, ...)
    Q = torch.stack([c.q_dev() for c in cases])                              # (L, 1, H_q, 1, D), written in place
    rng = np.random.default_rng(tail + layers)
    kt = vt = None
    if tail:
        kt = to_dev_half(rng.standard_normal((layers, 1, Hkv, tail, 128)).astype(np.float32), "bf16")
        vt = to_dev_half(rng.standard_normal((layers, 1, Hkv, tail, 128)).astype(np.float32), "bf16")
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, k_max_static=10, select_mode=mode)
    if per_layer:      # the reference's call pattern: one step per layer, in order
        decs = [QuestDecoder(Q[l], *[planes[k][l] for k in PLANES], K_tail=None if kt is None else kt[l],
                             V_tail=None if vt is None else vt[l], **kw) for l in range(layers)]
    else:              # all layers in one step
        decs = [QuestDecoder(Q, *[planes[k] for k in PLANES], K_tail=kt, V_tail=vt, **kw)]
    graph = _capture(decs)
    for rep in range(3):
        Q.copy_(torch.randn(Q.shape, device=Q.device).to(Q.dtype))          # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [d.O3.clone() for d in decs]
        for d in decs:                    # the same steps, eagerly
            d()
        torch.cuda.synchronize()
        for l, d in enumerate(decs):
            assert torch.equal(got[l], d.O3), (rep, l)
        assert bool(torch.isfinite(got[0]).all())
    # and the steps are the functional operator's (within its bar: a
    # different layer grouping may take another split count)
    want, _ = quest_decode_int4(Q, *[planes[k] for k in PLANES], K_tail=kt, V_tail=vt, **kw)
    torch.cuda.synchronize()
    mine = torch.stack([d.O3 for d in decs]) if per_layer else decs[0].O3
    assert float((mine.float() - want[..., 0, :].float()).abs().max()) <= 2e-3
