"""Adaptive top-k (adaptive_topk.py:44-51, 76-262, 397-431): the host plan of
veymoe.adaptive against the oracle's restatement, with known answers for the
keep rule and the cache-aware swap.  The weights of the known-answer cases are
exact binary fractions, so every running share is exact."""
import numpy as np
import pytest

from oracle import moe_oracle as mo
from veymoe import adaptive


@pytest.fixture(autouse=True)
def _reset():
    yield
    adaptive.set_threshold(1.0)
    adaptive.set_layer_thresholds()
    adaptive.set_min_keep(1)
    adaptive.set_swap_resident(None, epsilon=0.02, max_rows=4)
    adaptive.set_resident_experts()
    adaptive.set_route_observer()
    adaptive.reset_keep_stats()


@pytest.mark.parametrize("fn", [adaptive.keep_for_mass, mo.keep_for_mass], ids=["product", "oracle"])
def test_keep_for_mass_known_answers(fn):
    w = [4.0, 2.0, 1.0, 1.0]                # shares 0.5, 0.75, 0.875, 1.0
    assert fn(w, 0.5) == 1
    assert fn(w, 0.75) == 2                  # reaching the threshold exactly keeps
    assert fn(w, 0.8) == 3
    assert fn(w, 0.875) == 3
    assert fn(w, 0.9) == 4
    assert fn(w, 1.0) == 4
    assert fn([1.0, 1.0], 1.5) == 2          # never reached: all of them
    assert fn([3.0, 1.0], 0.0) == 1


@pytest.mark.parametrize("fn", [adaptive.swap_row, mo.swap_row], ids=["product", "oracle"])
def test_swap_row_known_answers(fn):
    resident = {10, 13}.__contains__
    # kept 11 (0.30) and 12 (0.20) are cold; dropped 13 (0.19) is resident and
    # within 0.02 of the lighter kept slot only: slot 1 swaps with slot 3
    e, w = fn([11, 12, 14, 13], [0.30, 0.20, 0.10, 0.19], 2, resident, 0.02)
    assert e == [11, 13, 14, 12] and w == [0.30, 0.19, 0.10, 0.20]
    # nothing resident among the dropped: unchanged
    e, w = fn([11, 12, 14], [0.5, 0.3, 0.2], 2, resident, 0.02)
    assert e == [11, 12, 14] and w == [0.5, 0.3, 0.2]
    # every kept expert resident: unchanged
    e, w = fn([10, 13, 12], [0.5, 0.3, 0.2], 2, resident, 0.5)
    assert e == [10, 13, 12]
    # the lightest cold slot chooses first and takes the heaviest candidate;
    # each candidate serves once
    res = {20, 21}.__contains__
    e, w = fn([1, 2, 20, 21], [0.40, 0.35, 0.34, 0.33], 2, res, 0.1)
    assert e == [21, 20, 2, 1] and w == [0.33, 0.34, 0.35, 0.40]


def _rows(rng, t, k, experts):
    inds = np.stack([rng.choice(experts, k, replace=False) for _ in range(t)]).astype(np.int32)
    g = rng.dirichlet(np.full(k, 0.6), size=t).astype(np.float32) * rng.uniform(0.3, 1.0, (t, 1)).astype(np.float32)
    g = mo.bf16r(g)
    g[0, 1] = g[0, 2]                        # a tie inside a row
    return inds, g


@pytest.mark.parametrize("threshold,min_keep,mode", [(0.5, 1, "bf16"), (0.7, 2, "bf16"), (0.9, 1, "f32"),
                                                     (0.3, 4, "bf16")])
def test_plan_equals_the_oracle(threshold, min_keep, mode):
    rng = np.random.default_rng(int(threshold * 100) + min_keep)
    inds, g = _rows(rng, 40, 10, 64)
    adaptive.set_threshold(threshold)
    adaptive.set_min_keep(min_keep)
    p_inds, p_scores, p_keeps, p_width = adaptive.plan(3, inds, g, 1.0, bf16=mode == "bf16")
    o_inds, o_scores, o_keeps = mo.adaptive_routes(inds, g, threshold, mode, min_keep=min_keep)
    width = o_inds.shape[1]
    assert p_keeps == o_keeps and p_width == width
    np.testing.assert_array_equal(p_inds[:, :width], o_inds)
    np.testing.assert_array_equal(p_scores[:, :width], o_scores)
    # slots past the widest row: the row's first expert, score 0
    np.testing.assert_array_equal(p_inds[:, width:], np.repeat(p_inds[:, :1], 10 - width, axis=1))
    assert not p_scores[:, width:].any()
    assert adaptive.last_keeps()[3] == tuple(p_keeps)
    assert adaptive.mean_keeps() == pytest.approx(np.mean(p_keeps))


def test_plan_with_swap_and_resident_masks_equals_the_oracle():
    rng = np.random.default_rng(7)
    inds, g = _rows(rng, 4, 8, 32)
    resident = set(range(0, 32, 3))
    adaptive.set_threshold(0.6)
    adaptive.set_swap_resident(lambda layer, e: layer == 5 and e in resident, epsilon=0.05, max_rows=4)
    adaptive.set_resident_experts({5: {1, 2, 4}})
    p_inds, p_scores, p_keeps, p_width = adaptive.plan(5, inds, g)
    o_inds, o_scores, o_keeps = mo.adaptive_routes(inds, g, 0.6, "bf16", resident={1, 2, 4},
                                                   swap=resident.__contains__, epsilon=0.05)
    width = o_inds.shape[1]
    assert p_keeps == o_keeps and p_width == width
    np.testing.assert_array_equal(p_inds[:, :width], o_inds)
    np.testing.assert_array_equal(p_scores[:, :width], o_scores)
    # above max_rows the swap stands down
    big, gb = _rows(rng, 6, 8, 32)
    q_inds, _, _, _ = adaptive.plan(5, big, gb)
    r_inds, _, _ = mo.adaptive_routes(big, gb, 0.6, "bf16", resident={1, 2, 4})
    np.testing.assert_array_equal(q_inds[:, :r_inds.shape[1]], r_inds)


def test_threshold_one_keeps_every_slot_and_the_plain_renorm():
    rng = np.random.default_rng(3)
    inds, g = _rows(rng, 8, 6, 64)
    p_inds, p_scores, keeps, width = adaptive.plan(None, inds, g)
    assert width == 6
    assert keeps == [6] * 8
    order = np.argsort(-g, axis=1, kind="stable")
    np.testing.assert_array_equal(p_inds, np.take_along_axis(inds, order, axis=1))
    np.testing.assert_array_equal(p_scores, mo.renorm(np.take_along_axis(g, order, axis=1), "bf16"))


def test_observer_sees_rows_before_the_swap():
    seen = []
    adaptive.set_threshold(0.5)
    adaptive.set_route_observer(lambda layer, e, w, k: seen.append((layer, e, w, k)), max_rows=2)
    rng = np.random.default_rng(11)
    inds, g = _rows(rng, 5, 4, 16)
    adaptive.plan(2, inds, g)
    assert len(seen) == 1 and seen[0][0] == 2 and len(seen[0][1]) == 2 and len(seen[0][3]) == 2


def test_exact_routing_reports_every_slot_to_the_observer():
    seen = []
    assert not adaptive.observing()
    adaptive.set_route_observer(lambda layer, e, w, k: seen.append((layer, e, w, k)))
    assert adaptive.observing()
    inds = np.array([[3, 1, 2], [5, 4, 0]], np.int32)
    gates = np.array([[0.5, 0.25, 0.25], [0.75, 0.125, 0.125]], np.float32)
    adaptive.observe_exact(7, inds, gates)
    assert seen == [(7, inds.tolist(), gates.tolist(), [3, 3])]
    adaptive.observe_exact(None, inds, gates)   # no layer id: nothing
    assert len(seen) == 1


# The reference's own known answers for swap_row (models/flashnext/tests/unit/
# test_swap_routing.py:25-81), restated as data: (experts, weights, keep,
# resident experts, epsilon) -> the expected experts, and the weights checked
# there.  The product returns its input list itself when nothing moves
# (the reference asserts identity, :42-54).
_REF_SWAP_CASES = [
    # a cold pick takes a close resident spare (:25-30)
    ([1, 7, 9], [0.5, 0.021, 0.019], 2, {1, 9}, 0.02, [1, 9, 7], {1: 0.019}),
    # a distant spare is left alone (:32-36)
    ([1, 7, 9], [0.5, 0.021, 0.001], 2, {1, 9}, 0.005, [1, 7, 9], {}),
    # nothing moves when every pick is resident (:38-43)
    ([1, 7, 9], [0.5, 0.021, 0.019], 2, {1, 7, 9}, 0.02, [1, 7, 9], {}),
    # nothing moves when no spare is resident (:45-50)
    ([1, 7, 9], [0.5, 0.021, 0.019], 2, {1}, 0.02, [1, 7, 9], {}),
    # it keeps the strongest spare (:59-64)
    ([7, 9, 10], [0.030, 0.029, 0.011], 1, {9, 10}, 0.05, [9, 7, 10], {0: 0.029}),
]


@pytest.mark.parametrize("fn", [adaptive.swap_row, mo.swap_row], ids=["product", "oracle"])
@pytest.mark.parametrize("case", range(len(_REF_SWAP_CASES)))
def test_reference_swap_row_known_answers(fn, case):
    experts, weights, keep, held, eps, want, weight_at = _REF_SWAP_CASES[case]
    got_e, got_w = fn(list(experts), list(weights), keep, held.__contains__, eps)
    assert got_e == want
    for pos, w in weight_at.items():
        assert got_w[pos] == pytest.approx(w)
    # a weight follows its expert (:74-79)
    pairs = dict(zip(got_e, got_w))
    for e, w in zip(experts, weights):
        assert pairs[e] == pytest.approx(w)


def test_reference_swap_row_set_and_identity_rules():
    """test_swap_routing.py:38-57,66-72: unchanged rows are the input list
    itself (product), one spare serves one pick, and the expert and weight
    multisets are preserved."""
    before = [1, 7, 9]
    e, _ = adaptive.swap_row(before, [0.5, 0.021, 0.019], 2, {1, 7, 9}.__contains__, 0.02)
    assert e is before
    e, _ = adaptive.swap_row(before, [0.5, 0.021, 0.019], 2, {1}.__contains__, 0.02)
    assert e is before
    for fn in (adaptive.swap_row, mo.swap_row):
        e, _ = fn([7, 8, 9], [0.021, 0.020, 0.019], 2, {9}.__contains__, 0.02)
        assert e.count(9) == 1 and sorted(e) == [7, 8, 9]
        e, w = fn([1, 7, 9, 10], [0.5, 0.021, 0.020, 0.019], 2, {9, 10}.__contains__, 0.02)
        assert sorted(e) == [1, 7, 9, 10]
        assert sorted(round(v, 6) for v in w) == sorted(round(v, 6) for v in [0.5, 0.021, 0.020, 0.019])


@pytest.mark.parametrize("fn", ["product", "oracle"])
def test_blend_is_a_bf16_scalar(fn):
    """Renorm blend 0.3 rounds to bf16 0.30078125 before it multiplies
    (compiled.py:111 builds mx.array(blend, scores.dtype)).  Row gates
    [0.5, 0.2734375, 0.2265625] at threshold 0.7 keep two slots: topk mass 1,
    kept mass 0.7734375, diff -0.2265625.  By hand: 0.30078125 * -0.2265625 =
    -0.068145751953125 -> bf16 -0.068359375; 1 - 0.068359375 = 0.931640625,
    a tie between 0.9296875 and 0.93359375 -> the even 0.9296875.  Scores:
    0.5 / 0.9296875 = 0.53782 -> 0.5390625, 0.2734375 / 0.9296875 = 0.29412 ->
    0.294921875.  With blend left in fp32 the normalizer would be 0.93359375
    and the first score 0.53515625."""
    inds = np.array([[4, 9, 2]], np.int32)
    gates = np.array([[0.5, 0.2734375, 0.2265625]], np.float32)
    adaptive.set_threshold(0.7)
    if fn == "product":
        _, scores, keeps, width = adaptive.plan(3, inds, gates, 0.3)
        assert keeps == [2] and width == 2
    else:
        _, scores, keeps = mo.adaptive_routes(inds, gates, 0.7, "bf16", blend=0.3)
    np.testing.assert_array_equal(np.asarray(scores)[0, :2], np.array([0.5390625, 0.294921875], np.float32))


def test_keep_stats_count_exact_layers():
    """Layers at threshold 1.0 record k per row too (adaptive_topk.py:236-239),
    so the keep statistics mix exact and adaptive layers as the reference's do."""
    adaptive.set_layer_thresholds({1: 0.5})
    adaptive.record_exact(0, rows=3, k=4)
    assert adaptive.last_keeps()[0] == (4, 4, 4)
    rng = np.random.default_rng(19)
    inds, g = _rows(rng, 2, 4, 16)
    _, _, keeps, _ = adaptive.plan(1, inds, g)
    assert adaptive.last_keeps()[1] == tuple(keeps)
    assert adaptive.mean_keeps() == pytest.approx((12 + sum(keeps)) / 5)
    adaptive.record_exact(None, rows=3, k=4)   # no layer id: nothing
    assert adaptive.mean_keeps() == pytest.approx((12 + sum(keeps)) / 5)
