"""More than 8 query heads per KV head (the reference's kernels take any GQA
ratio, sparse_int4_fwd.py:54-55,201): the library's kernels hold one
selection bit per query head of a group (at most 8), so per-query-head
decode, the mask operators and prefill run the group's query heads in chunks
of at most 4.  Against the oracle at ratios 12 and 16 (head_dim 128 and 64);
per_kv_head_sum above 8 is refused with NotImplementedError."""
import numpy as np
import pytest
import torch

from oracle import fq_oracle as O
from tests.cases import Int4Case, Int8Case, decode_tol, max_err, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 2, 128), (24, 2, 64), (16, 1, 128)])
def test_per_q_head_decode_above_eight_heads_per_group(bits, Hq, Hkv, D):
    from flashquest_amd.eager.decode import quest_decode_int4, quest_decode_int8
    kw = dict(retention=0.3, num_sinks=2, window_pages=1, select_mode="per_q_head", return_selection=True)
    if bits == 4:
        c = Int4Case(seed=1200 + Hq + D, B=2, Hq=Hq, Hkv=Hkv, S=64 * 23 + 9, D=D)
        o, lse, mask = quest_decode_int4(c.q_dev(), **c.device(), **kw)
        ref = O.decode_step(c.Q, c.kp, c.ks, c.km, c.vp, c.vs, c.vm, retention=0.3, num_sinks=2, window_pages=1)
    else:
        c = Int8Case(seed=1300 + Hq + D, B=2, Hq=Hq, Hkv=Hkv, S=64 * 23 + 9, D=D)
        o, lse, mask = quest_decode_int8(c.q_dev(), **c.device(), **kw)
        ref = O.decode_step(c.Q, c.ku, c.ks, c.km, c.vu, c.vs, c.vm, retention=0.3, num_sinks=2, window_pages=1,
                            bits=8)
    torch.cuda.synchronize()
    assert np.array_equal(mask.cpu().numpy(), ref["mask"])
    assert max_err(o[:, :, 0], ref["O"]) <= decode_tol(ref["O"], "bf16")
    assert max_err(lse[:, :, 0], ref["lse"]) <= 1e-4


def test_per_kv_head_sum_above_eight_heads_per_group_is_refused():
    from flashquest_amd.eager.decode import quest_decode_int4
    c = Int4Case(seed=5, B=1, Hq=32, Hkv=2, S=64 * 6, D=128)
    with pytest.raises(NotImplementedError, match="at most 8"):
        quest_decode_int4(c.q_dev(), **c.device(), retention=0.3, select_mode="per_kv_head_sum")


def test_mask_operator_above_eight_heads_per_group():
    from flashquest_amd.kernel import flash_attn_sparse_int4_fwd
    c = Int4Case(seed=77, B=2, Hq=24, Hkv=2, S=64 * 17, D=128, vgroup=32)
    mask = c.rng.random((2, 24, c.P)) < 0.35
    ref_o, ref_l = c.oracle(mask)
    o, lse = flash_attn_sparse_int4_fwd(c.q_dev(), **c.device(), selection_mask=to_dev(mask)[:, :, None, :])
    torch.cuda.synchronize()
    assert max_err(o[:, :, 0], ref_o) <= decode_tol(ref_o, "bf16")
    assert max_err(lse[:, :, 0], ref_l) <= 1e-4


def test_prefill_above_eight_heads_per_group():
    from tests.test_gpu_prefill import ATOL, PrefillCase
    case = PrefillCase(31, B=1, Hq=32, Hkv=2, S=640, T=21)
    out = case.run()
    torch.cuda.synchronize()
    err = float(np.abs(out.float().cpu().numpy() - case.oracle()).max())
    assert err < ATOL, err
