"""The order-independent selection check used by the at-size GPU tests
(tests.cases.fp64_selection_check), pinned on small hand-built inputs: a clear
top-k is accepted, a wrong mask is counted, and a boundary closer than the
fp32 error bound is reported as ambiguous instead of being judged."""
import numpy as np

from tests.cases import fp64_selection_check


def _setup(P=8, D=16, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((1, 2, D)).astype(np.float32)      # 2 query heads, 1 KV head
    km = np.zeros((1, 1, P, D), np.float32)
    ks = np.zeros((1, 1, P, D), np.float32)
    return q, ks, km


def _plant(q, ks, km, scores_per_page):
    """K_mn rows along q_0 + q_1 so that the summed exact score of page p is
    scores_per_page[p] (scale 0: no relu term)."""
    qs = q[0, 0].astype(np.float64) + q[0, 1]
    u = qs / np.dot(qs, qs)
    for p, s in enumerate(scores_per_page):
        km[0, 0, p] = (s * u).astype(np.float32)


def test_clear_topk_is_accepted_and_a_wrong_mask_is_counted():
    q, ks, km = _setup()
    _plant(q, ks, km, [0.0, 5.0, 1.0, 7.0, 2.0, 6.0, 3.0, 4.0])
    want = np.zeros((1, 2, 8), bool)
    want[:, :, [3, 5, 1]] = True               # top-3 by the summed score, no forced pages
    assert fp64_selection_check(q, ks, km, want, 3 / 8, "per_kv_head_sum", 0, 0) == (1, 0, 0, 0)
    bad = want.copy()
    bad[:, :, 1], bad[:, :, 7] = False, True
    assert fp64_selection_check(q, ks, km, bad, 3 / 8, "per_kv_head_sum", 0, 0) == (1, 0, 1, 0)


def test_forced_pages_join_the_expected_set():
    q, ks, km = _setup()
    _plant(q, ks, km, [0.0, 5.0, 1.0, 7.0, 2.0, 6.0, 3.0, 4.0])
    want = np.zeros((1, 2, 8), bool)
    want[:, :, [3, 5, 1, 0, 7]] = True         # top-3 + sink page 0 + window page 7
    assert fp64_selection_check(q, ks, km, want, 3 / 8, "per_kv_head_sum", 1, 1) == (1, 0, 0, 0)


def test_boundary_within_fp32_error_is_ambiguous():
    q, ks, km = _setup()
    _plant(q, ks, km, [0.0, 5.0, 1.0, 7.0, 2.0, 6.0, 5.0 * (1 + 2 ** -22), 4.0])
    # the 3rd and 4th largest (pages 6 and 1) differ by far less than the bound:
    # either mask is accepted as ambiguous, not judged
    for pick, differs in ((6, 0), (1, 1)):
        m = np.zeros((1, 2, 8), bool)
        m[:, :, [3, 5, pick]] = True
        assert fp64_selection_check(q, ks, km, m, 3 / 8, "per_kv_head_sum", 0, 0) == (1, 1, 0, differs)


def test_per_query_head_rows_are_judged_separately():
    q, ks, km = _setup(seed=3)
    rng = np.random.default_rng(5)
    km[:] = rng.standard_normal(km.shape).astype(np.float32)
    s = np.einsum("hd,pd->hp", q[0].astype(np.float64), km[0, 0].astype(np.float64))
    want = np.zeros((1, 2, 8), bool)
    for h in range(2):
        want[0, h, np.argsort(-s[h])[:2]] = True
    assert fp64_selection_check(q, ks, km, want, 0.25, "per_q_head", 0, 0) == (2, 0, 0, 0)
    flipped = want.copy()
    flipped[0, 1] = ~flipped[0, 1]
    assert fp64_selection_check(q, ks, km, flipped, 0.25, "per_q_head", 0, 0) == (2, 0, 1, 0)
