"""DuoAttention head patterns (src/flashquest/duo/, llama_persistent_patch.py:214-220)
through the fused decode, against the oracle: streaming KV heads select
exactly the sink and window pages, retrieval heads the top-k of their scores,
and attention follows the selection.  A (layers, KV heads) pattern in one
multi-layer call gives each layer its own retention row (the single-launch
kernel and the split path agree bit for bit on the selection)."""
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
def test_layer_patterns_in_one_multilayer_call(mode, splits):
    from flashquest_amd.eager.decode import quest_decode_int4
    Lyr, Hq, Hkv, P = 24, 24, 8, 40          # 192 groups: the single-launch kernel unless splits are pinned
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


def test_quest_duo_fused_sdpa_signature_and_semantics():
    from flashquest_amd.duo import quest_duo_fused_sdpa
    Hq, Hkv, P = 8, 4, 24
    case = Int8Case(seed=77, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128)
    d = case.device()
    pattern = torch.tensor([True, False, True, False])
    o = quest_duo_fused_sdpa(case.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"],
                             d["V_mn"], head_pattern=pattern, retention=0.25, num_sinks=4, window_pages=2)
    torch.cuda.synchronize()
    rrow = _retention_rows(pattern.numpy(), 0.25, Hq // Hkv)
    ref = O.decode_step(case.Q, case.ku, case.ks, case.km, case.vu, case.vs, case.vm, retention=rrow, num_sinks=4,
                        window_pages=2, bits=8)
    assert o.shape == (1, Hq, 1, 128) and o.dtype == torch.bfloat16
    assert max_err(o[:, :, 0], ref["O"]) <= 2e-3 + 2.0 ** -8 * float(np.abs(ref["O"]).max())
    # all-streaming: attention over sinks and window only (duo's EP2)
    o_s = quest_duo_fused_sdpa(case.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"],
                               d["V_mn"], head_pattern=torch.zeros(Hkv, dtype=torch.bool))
    torch.cuda.synchronize()
    forced = np.broadcast_to(_forced(P, 4, 2), (1, Hq, P))
    ro, _ = O.sparse_int8_attention(case.Q, case.ku, case.ks, case.km, case.vu, case.vs, case.vm, forced, 64)
    assert max_err(o_s[:, :, 0], ro) <= 2e-3 + 2.0 ** -8 * float(np.abs(ro).max())
    with pytest.raises(ValueError, match="head_pattern"):
        quest_duo_fused_sdpa(case.q_dev(), d["K_uint8"], d["K_scale"], d["K_mn"], d["V_uint8"], d["V_scale"],
                             d["V_mn"], head_pattern=torch.tensor([True, False, True]))
