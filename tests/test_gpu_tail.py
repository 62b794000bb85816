"""The decode step with a partial page (llama_persistent_patch.py:202-240): the
fused entry attends the selected pages and the bf16 tail together (the tail in
the split-merge launch); the result must match the oracle's sparse attention
merged with the dense tail attention (_merge_two_attentions, fp64 here) for
many layers at once (one workgroup per KV group: the fused kernel attends a
16-bit tail itself; fp32 and padded-row tails) and for one layer (split
groups, the tail in the split merge), tails of 1..64 tokens in bf16, fp16 and
fp32, and an empty selection (the tail alone)."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import Int4Case, Int8Case, max_err, to_dev_half

pytestmark = pytest.mark.gpu


def _dev(x, tdt):
    return torch.from_numpy(x).cuda() if tdt == "f32" else to_dev_half(x, tdt)


def _merged_ref(case, Kt, Vt, retention, sinks, window, mode):
    ref = O.decode_step(case.Q, case.kp, case.ks, case.km, case.vp, case.vs, case.vm, retention=retention,
                        num_sinks=sinks, window_pages=window, mode=mode, k_max_static=None)
    ot, lt = O.dense_attn_with_lse(case.Q, Kt, Vt)
    o = O.merge_two_attentions(ref["O"], ref["lse"], ot, lt)
    m = np.maximum(ref["lse"], lt)
    with np.errstate(invalid="ignore", divide="ignore"):
        lse = m + np.log(np.exp(ref["lse"] - m) + np.exp(lt - m))
    return o, lse


@pytest.mark.parametrize("layers,T,tdt,mode,pad", [(24, 37, "bf16", "per_kv_head_sum", 0),
                                                   (24, 64, "f16", "per_q_head", 0),
                                                   (24, 5, "bf16", "per_q_head", 8),
                                                   (24, 64, "bf16", "per_kv_head_sum", 24),
                                                   (24, 33, "f32", "per_q_head", 0),
                                                   (1, 1, "bf16", "per_q_head", 0),
                                                   (1, 63, "bf16", "per_kv_head_sum", 0)])
def test_fused_tail_matches_sparse_plus_tail_merge(layers, T, tdt, mode, pad):
    from flashquest_amd.eager import quest_decode_int4
    rng = np.random.default_rng(40 + T)
    Hq, Hkv, P = 24, 8, 14
    cases = [Int4Case(seed=500 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128, page=64, dtype="bf16", meta="f16",
                      vgroup=32) for i in range(layers)]
    tails = [(O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32)),
              O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32))) for _ in range(layers)]
    dev = [c.device() for c in cases]
    if layers > 1:
        stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
        q = torch.stack([c.q_dev() for c in cases])
        kt = torch.stack([_dev(t[0], tdt) for t in tails])
        vt = torch.stack([_dev(t[1], tdt) for t in tails])
        if pad:      # rows `pad` elements apart beyond D: views into wider buffers
            kw = torch.zeros(*kt.shape[:-1], 128 + pad, dtype=kt.dtype, device=kt.device)
            vw = torch.zeros_like(kw)
            kw[..., :128] = kt
            vw[..., :128] = vt
            kt, vt = kw[..., :128], vw[..., :128]
    else:
        stacked, q = dev[0], cases[0].q_dev()
        kt, vt = _dev(tails[0][0], tdt), _dev(tails[0][1], tdt)
    o, lse = quest_decode_int4(q, **stacked, retention=0.3, num_sinks=2, window_pages=1, select_mode=mode,
                               K_tail=kt, V_tail=vt)
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        ro, rl = _merged_ref(c, tails[i][0], tails[i][1], 0.3, 2, 1, mode)
        oi = o[i] if layers > 1 else o
        li = lse[i] if layers > 1 else lse
        assert max_err(oi[:, :, 0], ro) <= 2e-3 + 2 ** -8 * np.abs(ro).max(), i
        assert max_err(li[:, :, 0], rl) <= 1e-4, i


def test_fused_tail_with_empty_selection_is_tail_attention():
    from flashquest_amd.eager import quest_decode_int4
    rng = np.random.default_rng(3)
    c = Int4Case(seed=9, B=1, Hq=6, Hkv=2, S=64 * 5, D=128, page=64, dtype="bf16", meta="bf16")
    Kt = O.round_bf16(rng.standard_normal((1, 2, 20, 128)).astype(np.float32))
    Vt = O.round_bf16(rng.standard_normal((1, 2, 20, 128)).astype(np.float32))
    o, lse = quest_decode_int4(c.q_dev(), **c.device(), retention=0.0, num_sinks=0, window_pages=0,
                               K_tail=to_dev_half(Kt, "bf16"), V_tail=to_dev_half(Vt, "bf16"))
    ro, rl = O.dense_attn_with_lse(c.Q, Kt, Vt)
    assert max_err(o[:, :, 0], ro) <= 2e-3 + 2 ** -8 * np.abs(ro).max()
    assert max_err(lse[:, :, 0], rl) <= 1e-4


def test_fused_tail_rejects_long_tails_and_selection_output():
    from flashquest_amd.eager import quest_decode_int4
    c = Int4Case(seed=1, B=1, Hq=6, Hkv=2, S=64 * 3, D=128, page=64, dtype="bf16", meta="bf16")
    kt = torch.zeros(1, 2, 65, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NotImplementedError):
        quest_decode_int4(c.q_dev(), **c.device(), retention=0.5, K_tail=kt, V_tail=kt)
    with pytest.raises(ValueError):
        quest_decode_int4(c.q_dev(), **c.device(), retention=0.5, K_tail=kt[:, :, :3], V_tail=kt[:, :, :3],
                          return_selection=True)


@pytest.mark.parametrize("layers,T,tdt,mode", [(24, 37, "bf16", "per_kv_head_sum"),
                                               (24, 64, "f16", "per_q_head"),
                                               (24, 21, "f32", "per_q_head"),
                                               (1, 1, "bf16", "per_q_head"),
                                               (1, 50, "bf16", "per_kv_head_sum")])
def test_int8_fused_tail_matches_sparse_plus_tail_merge(layers, T, tdt, mode):
    """The same for the INT8 cache (kv_bits 8): quest_decode_int8 with the
    tail, one workgroup per group (the kernel attends the tail) or split groups
    (split 0 of each group attends it), fp32 tails in the split merge."""
    from flashquest_amd.eager.decode import quest_decode_int8
    from tests.cases import Int8Case
    rng = np.random.default_rng(70 + T)
    Hq, Hkv, P = 24, 8, 14
    cases = [Int8Case(seed=700 + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128) for i in range(layers)]
    tails = [(O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32)),
              O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32))) for _ in range(layers)]
    dev = [c.device() for c in cases]
    if layers > 1:
        stacked = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
        q = torch.stack([c.q_dev() for c in cases])
        kt = torch.stack([_dev(t[0], tdt) for t in tails])
        vt = torch.stack([_dev(t[1], tdt) for t in tails])
    else:
        stacked, q = dev[0], cases[0].q_dev()
        kt, vt = _dev(tails[0][0], tdt), _dev(tails[0][1], tdt)
    o, lse = quest_decode_int8(q, **stacked, retention=0.3, num_sinks=2, window_pages=1, select_mode=mode,
                               K_tail=kt, V_tail=vt)
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        ref = O.decode_step(c.Q, c.ku, c.ks, c.km, c.vu, c.vs, c.vm, retention=0.3, num_sinks=2, window_pages=1,
                            mode=mode, bits=8)
        ot, lt = O.dense_attn_with_lse(c.Q, tails[i][0], tails[i][1])
        ro = O.merge_two_attentions(ref["O"], ref["lse"], ot, lt)
        m = np.maximum(ref["lse"], lt)
        rl = m + np.log(np.exp(ref["lse"] - m) + np.exp(lt - m))
        oi = o[i] if layers > 1 else o
        li = lse[i] if layers > 1 else lse
        assert max_err(oi[:, :, 0], ro) <= 2e-3 + 2 ** -8 * np.abs(ro).max(), i
        assert max_err(li[:, :, 0], rl) <= 1e-4, i


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("mode", ["per_kv_head_sum", "per_q_head"])
@pytest.mark.parametrize("T", [0, 37])
def test_single_layer_split_step_matches_oracle(bits, mode, T):
    """One layer of 8 KV groups over 200 pages (the reference's per-layer call
    at a realistic context): a scoring launch, then each group split over
    several attention workgroups that select from its scores, the tail (if
    any) attended by split 0, and the one-round split merge.  Selection
    bit-exact, O and lse against the oracle (with the tail: the oracle's
    sparse attention merged with dense attention over the tail)."""
    from flashquest_amd.eager import quest_decode_int4, quest_decode_int8
    rng = np.random.default_rng(300 + T + bits)
    Hq, Hkv, P = 24, 8, 200
    if bits == 4:
        c = Int4Case(seed=77, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128, page=64, dtype="bf16", meta="f16", vgroup=32)
        fn = quest_decode_int4
    else:
        c = Int8Case(seed=78, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128)
        fn = quest_decode_int8
    kw = dict(retention=0.25, num_sinks=4, window_pages=2, select_mode=mode)
    if T:
        kt = O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32))
        vt = O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32))
        o, lse = fn(c.q_dev(), **c.device(), K_tail=_dev(kt, "bf16"), V_tail=_dev(vt, "bf16"), **kw)
    else:
        o, lse, mask = fn(c.q_dev(), **c.device(), return_selection=True, **kw)
    torch.cuda.synchronize()
    planes = (c.kp, c.ks, c.km, c.vp, c.vs, c.vm) if bits == 4 else (c.ku, c.ks, c.km, c.vu, c.vs, c.vm)
    ref = O.decode_step(c.Q, *planes, retention=0.25, num_sinks=4, window_pages=2, mode=mode, bits=bits)
    ro, rl = ref["O"], ref["lse"]
    if T:
        ot, lt = O.dense_attn_with_lse(c.Q, kt, vt)
        ro = O.merge_two_attentions(ref["O"], ref["lse"], ot, lt)
        m = np.maximum(ref["lse"], lt)
        rl = m + np.log(np.exp(ref["lse"] - m) + np.exp(lt - m))
    else:
        assert np.array_equal(mask.cpu().numpy(), ref["mask"])
    assert max_err(o[:, :, 0], ro) <= 2e-3 + 2 ** -8 * np.abs(ro).max()
    assert max_err(lse[:, :, 0], rl) <= 1e-4


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rep,layers,T,mode", [(5, 1, 37, "per_q_head"), (6, 4, 64, "per_kv_head_sum"),
                                               (7, 1, 1, "per_kv_head_sum"), (7, 4, 20, "per_q_head")])
def test_tail_with_gqa_ratios_above_four(bits, rep, layers, T, mode):
    """GQA ratios 5-7 take the general attention kernels; with a bf16 tail
    the tail is attended in their split merge.  Against the oracle's sparse
    attention merged with the dense tail attention, INT4 and INT8."""
    from flashquest_amd.eager.decode import quest_decode_int4, quest_decode_int8
    rng = np.random.default_rng(90 + rep + T + bits)
    Hkv, P = 2, 9
    Hq = Hkv * rep
    mk = Int4Case if bits == 4 else Int8Case
    cases = [mk(seed=700 + 10 * bits + i, B=1, Hq=Hq, Hkv=Hkv, S=64 * P, D=128, page=64, dtype="bf16", meta="bf16")
             for i in range(layers)]
    tails = [(O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32)),
              O.round_bf16(rng.standard_normal((1, Hkv, T, 128)).astype(np.float32))) for _ in range(layers)]
    dev = [c.device() for c in cases]
    if layers > 1:
        planes = {k: torch.stack([d[k] for d in dev]) for k in dev[0]}
        q = torch.stack([c.q_dev() for c in cases])
        kt = torch.stack([to_dev_half(t[0], "bf16") for t in tails])
        vt = torch.stack([to_dev_half(t[1], "bf16") for t in tails])
    else:
        planes, q = dev[0], cases[0].q_dev()
        kt, vt = to_dev_half(tails[0][0], "bf16"), to_dev_half(tails[0][1], "bf16")
    fn = quest_decode_int4 if bits == 4 else quest_decode_int8
    o, lse = fn(q, **planes, retention=0.3, num_sinks=2, window_pages=1, select_mode=mode, K_tail=kt, V_tail=vt)
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        if bits == 4:
            ro, rl = _merged_ref(c, tails[i][0], tails[i][1], 0.3, 2, 1, mode)
        else:
            ref = O.decode_step(c.Q, c.ku, c.ks, c.km, c.vu, c.vs, c.vm, retention=0.3, num_sinks=2,
                                window_pages=1, mode=mode, bits=8)
            ot, lt = O.dense_attn_with_lse(c.Q, tails[i][0], tails[i][1])
            ro = O.merge_two_attentions(ref["O"], ref["lse"], ot, lt)
            m = np.maximum(ref["lse"], lt)
            rl = m + np.log(np.exp(ref["lse"] - m) + np.exp(lt - m))
        oi = o[i] if layers > 1 else o
        li = lse[i] if layers > 1 else lse
        assert max_err(oi[:, :, 0], ro) <= 2e-3 + 2 ** -8 * np.abs(ro).max(), (rep, i)
        assert max_err(li[:, :, 0], rl) <= 1e-4, (rep, i)
