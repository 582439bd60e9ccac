"""Pins the CPU oracle before anything is checked against it.

Each check is independent of the oracle's own formula: reference known-answer
tests, brute-force loops restating the reference's NumPy projection, closed
forms, float64 mathematics, and full sorts.
"""
import math

import numpy as np
import pytest

from oracle import moe_oracle as mo
from oracle import ref_loops


# ----------------------------------------------------------- KATs ------

def test_weighted_combine_known_answer():
    # models/flashnext/tests/unit/test_metal_runtime.py:222-263
    outputs = np.array([[[1.0, 2.0], [10.0, 20.0], [100.0, 200.0]],
                        [[3.0, 4.0], [30.0, 40.0], [300.0, 400.0]]], dtype=np.float32)
    routes = np.array([[2, 0], [1, 2]], dtype=np.int32)
    scores = np.array([[0.25, 0.75], [0.4, 0.6]], dtype=np.float32)
    expected = np.array([[25.75, 51.5], [192.0, 256.0]], dtype=np.float32)
    first = mo.weighted_combine(outputs, routes, scores)
    np.testing.assert_array_equal(first, expected)
    np.testing.assert_array_equal(mo.weighted_combine(outputs, routes, scores), first)


def test_weighted_combine_rejects_bad_shapes():
    # test_metal_runtime.py:34-48
    with pytest.raises(ValueError):
        mo.weighted_combine(np.zeros((2, 3, 2), np.float32), np.zeros((2, 2), np.int32), np.ones((2, 1), np.float32))
    with pytest.raises(ValueError):
        mo.weighted_combine(np.zeros((2, 3, 2), np.float32), np.array([[0, 3]], np.int32), np.ones((1, 2), np.float32))


def test_bf16_bit_round_trip():
    # models/flashnext/tests/unit/test_swiglu_contract.py:21-23
    raw = np.array([0x0000, 0x3F80, 0x8000, 0x7F80, 0xFFFF], dtype=np.uint16)
    np.testing.assert_array_equal(mo.f32_to_bf16_bits(mo.bf16_bits_to_f32(raw)), raw)


def test_bf16_rounding_is_nearest_even():
    one = 1.0
    ulp = 2.0 ** -7
    cases = {
        one + ulp / 2: one,                 # tie -> even (1.0)
        one + 3 * ulp / 2: one + 2 * ulp,   # tie -> even (mantissa ...10)
        one + ulp / 2 + 2.0 ** -20: one + ulp,
        -(one + ulp / 2): -one,
        3.4e38: math.inf,                   # above the largest bf16 (0x7F7F) by more than half an ulp
    }
    for value, expected in cases.items():
        got = float(mo.bf16r(np.float32(value)))
        assert got == expected, (value, got, expected)


# ------------------------------------------------------- SwiGLU ------

def _all_bf16_values():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = mo.bf16_bits_to_f32(bits)
    return vals[np.isfinite(vals)]


@pytest.mark.parametrize("up_bits", [0x3F80, 0x3F9E, 0xC000])
def test_swiglu_exhaustive_against_float64(up_bits):
    """All 65,536 bf16 gate patterns (the reference's exhaustive scan,
    test_swiglu_contract.py:37-51): the op-by-op bf16 sequence stays within a
    few bf16 ulps of exact silu(g)*u evaluated in float64."""
    gate = _all_bf16_values()
    up = float(mo.bf16_bits_to_f32(np.array([up_bits], np.uint16))[0])
    got = mo.swiglu(gate, np.full_like(gate, up), "bf16").astype(np.float64)
    g64 = gate.astype(np.float64)
    with np.errstate(over="ignore"):
        exact = g64 / (1.0 + np.exp(-g64)) * up
    # outputs that round to zero or overflow are excluded from the relative check
    finite = np.isfinite(exact) & (np.abs(exact) > 1e-30) & np.isfinite(got)
    rel = np.abs(got[finite] - exact[finite]) / np.abs(exact[finite])
    # up to ~6 roundings of 2^-9 each, plus exp's propagated error near 1+e
    assert rel.max() < 6 * 2.0 ** -8, rel.max()
    assert np.all(np.sign(got[finite]) == np.sign(exact[finite]))
    # large negative gates saturate to (-)0, large positive to g*u
    assert got[gate < -100].max() <= 0 or up < 0


def test_swiglu_representative_values():
    # inputs of test_swiglu_contract.py:25-31; expected from float64 mathematics
    gate = mo.bf16_bits_to_f32(np.array([0x0000, 0x3F80, 0xBF80, 0x4120, 0xC120], np.uint16))
    up = mo.bf16_bits_to_f32(np.array([0x3F80, 0x3FA0, 0x3F00, 0x4020, 0xC000], np.uint16))
    got = mo.swiglu(gate, up, "bf16")
    exact = gate.astype(np.float64) / (1 + np.exp(-gate.astype(np.float64))) * up
    np.testing.assert_allclose(got, exact, rtol=2 * 2.0 ** -8, atol=0)
    assert got[0] == 0.0


def test_sigmoid_matches_float64():
    g = np.linspace(-30, 30, 4001).astype(np.float32)
    np.testing.assert_allclose(mo.sigmoid(g, "f32"), 1 / (1 + np.exp(-g.astype(np.float64))), rtol=1e-6, atol=1e-7)


# --------------------------------------------------- projection ------

def _random_proj(rng, experts, out_width, in_width):
    w = rng.integers(0, 2 ** 32, size=(experts, out_width, in_width // 8), dtype=np.uint32)
    s = mo.f32_to_bf16_bits(rng.uniform(0.005, 0.02, (experts, out_width, in_width // 32)).astype(np.float32))
    b = mo.f32_to_bf16_bits(rng.uniform(-0.1, 0.1, (experts, out_width, in_width // 32)).astype(np.float32))
    return w, s, b


@pytest.mark.parametrize("slot_input", [False, True])
def test_projection_matches_reference_loops(slot_input):
    rng = np.random.default_rng(5)
    w, s, b = _random_proj(rng, 3, 8, 64)
    routes = np.array([[2, 0], [1, 2]], dtype=np.int32)
    x = rng.normal(size=(2, 2, 64) if slot_input else (2, 64)).astype(np.float32)
    loops = np.array(ref_loops.projection_loops(x.tolist(), routes.tolist(), w.tolist(), s.tolist(), b.tolist(),
                                                8, slot_input))
    for t in range(2):
        for j in range(2):
            e = routes[t, j]
            src = x[t, j] if slot_input else x[t]
            got = mo.q4_project(src[None], w[e], s[e], b[e])[0]
            np.testing.assert_allclose(got, loops[t, j], rtol=1e-12, atol=1e-12)


def test_nibble_order_one_hot():
    """x = e_k picks s_g * q_k + b_g: pins the MLX nibble order
    (bits 4*(k&7) of word k>>3)."""
    q = np.arange(64) % 16
    words = np.array(ref_loops.pack_nibbles(q.tolist()), dtype=np.uint32)[None]
    s = mo.f32_to_bf16_bits(np.array([[0.5, 0.25]], np.float32))
    b = mo.f32_to_bf16_bits(np.array([[0.0, 1.0]], np.float32))
    for k in (0, 1, 7, 8, 31, 32, 47, 63):
        x = np.zeros((1, 64))
        x[0, k] = 1.0
        got = mo.q4_project(x, words, s, b)[0, 0]
        g = k // 32
        assert got == [0.5, 0.25][g] * q[k] + [0.0, 1.0][g], k


def test_projection_closed_forms():
    rng = np.random.default_rng(7)
    x = rng.normal(size=(3, 96))
    xsum = x.reshape(3, 3, 32).sum(-1)
    s = mo.f32_to_bf16_bits(rng.uniform(0.005, 0.02, (4, 3)).astype(np.float32))
    b = mo.f32_to_bf16_bits(rng.uniform(-0.1, 0.1, (4, 3)).astype(np.float32))
    sf, bf = mo.bf16_bits_to_f32(s).astype(np.float64), mo.bf16_bits_to_f32(b).astype(np.float64)
    zeros = np.zeros((4, 12), np.uint32)
    np.testing.assert_allclose(mo.q4_project(x, zeros, s, b), xsum @ bf.T, rtol=1e-12)
    zero_s = np.zeros_like(s)
    w = rng.integers(0, 2 ** 32, size=(4, 12), dtype=np.uint32)
    np.testing.assert_allclose(mo.q4_project(x, w, zero_s, b), xsum @ bf.T, rtol=1e-12)
    full = np.full((4, 12), 0xFFFFFFFF, np.uint32)
    np.testing.assert_allclose(mo.q4_project(x, full, s, np.zeros_like(b)), 15 * xsum @ sf.T, rtol=1e-12)


def test_projection_equals_dense_dequant_product():
    rng = np.random.default_rng(9)
    w, s, b = _random_proj(rng, 1, 16, 128)
    x = rng.normal(size=(4, 128))
    dense = mo.dequantize(w[0], s[0], b[0])
    np.testing.assert_allclose(mo.q4_project(x, w[0], s[0], b[0]), x @ dense.T, rtol=1e-10, atol=1e-10)


def test_pack_nibbles_round_trip():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=256)
    words = np.array(ref_loops.pack_nibbles(q.tolist()), dtype=np.uint32)
    np.testing.assert_array_equal(mo.unpack_nibbles(words), q)


# ------------------------------------------------------- router ------

def test_softmax_topk_against_full_sort():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(6, 256)).astype(np.float32)
    w = mo.f32_to_bf16_bits(rng.normal(0, 0.02, size=(512, 256)).astype(np.float32))
    inds, scores, gates = mo.route(mo.bf16r(x), w, 10, "bf16")
    # gates: rounded softmax of the rounded logits, summing to one within bf16
    assert np.allclose(gates.astype(np.float64).sum(-1), 1.0, atol=512 * 2 ** -9 / 512 * 4)
    for r in range(6):
        order = sorted(range(512), key=lambda e: (-float(gates[r, e]), e))
        assert inds[r].tolist() == order[:10]
        assert len(set(inds[r].tolist())) == 10
    # renormalised scores: descending, summing to ~1 within the bf16 steps
    assert np.all(np.diff(scores.astype(np.float64), axis=-1) <= 0)
    np.testing.assert_allclose(scores.astype(np.float64).sum(-1), 1.0, atol=10 * 2 ** -8)


def test_topk_tie_rule_prefers_lower_index():
    gates = np.array([[0.25, 0.5, 0.25, 0.5, 0.125]], np.float32)
    assert mo.topk(gates, 3).tolist() == [[1, 3, 0]]


def test_renorm_blend_identity_at_full_selection():
    scores = mo.bf16r(np.array([[0.3, 0.2, 0.1]], np.float32))
    for blend in (0.0, 0.5, 1.0):
        np.testing.assert_array_equal(mo.renorm(scores, "bf16", blend), mo.renorm(scores, "bf16", 1.0))
    expected = mo.bf16r(scores / mo.bf16r(scores.sum()))
    np.testing.assert_array_equal(mo.renorm(scores, "bf16"), expected)


# ------------------------------------------------------ combine ------

def test_fused_combine_shared_forms_are_exact_compositions():
    """The reference's fused-epilogue invariants (test_metal_runtime.py:641-729):
    fused(shared_y) == bf16(unfused + shared_y); fused(shared, gate) ==
    bf16(unfused + bf16(gate * shared))."""
    rng = np.random.default_rng(11)
    down = mo.bf16r(rng.normal(size=(2, 3, 64)).astype(np.float32))
    scores = np.array([[0.375, 0.625, 0.0], [0.2, 0.3, 0.5]], np.float32)
    shared_y = mo.bf16r(((np.arange(128) % 29 - 14) / 32).reshape(2, 64).astype(np.float32))
    unfused = mo.fused_combine(down, scores, "bf16")
    np.testing.assert_array_equal(mo.fused_combine(down, scores, "bf16", shared_y=shared_y),
                                  mo.bf16r(unfused + shared_y))
    gate = mo.bf16r(np.array([[0.333984375], [0.5]], np.float32))
    np.testing.assert_array_equal(mo.fused_combine(down, scores, "bf16", shared=shared_y, shared_gate=gate),
                                  mo.bf16r(unfused + mo.bf16r(shared_y * gate)))
    # the combine itself: fp32 sum in slot order of the products
    manual = np.zeros((2, 64), np.float32)
    for j in range(3):
        manual = manual + down[:, j] * scores[:, j:j + 1]
    np.testing.assert_array_equal(unfused, mo.bf16r(manual))


def test_generic_combine_matches_weighted_combine_in_f32():
    rng = np.random.default_rng(12)
    down = rng.normal(size=(4, 3, 16)).astype(np.float32)
    scores = rng.uniform(size=(4, 3)).astype(np.float32)
    np.testing.assert_allclose(mo.generic_combine(down, scores, "f32"), mo.weighted_combine(down, np.zeros((4, 3),
                               np.int32), scores), rtol=1e-6)


# ------------------------------------------------------ layer --------

def test_layer_lazy_and_dense_experts_agree():
    from veymoe import synth

    spec = synth.LayerSpec("t", 128, 64, 16, 4, 64, 3)
    x = mo.bf16_bits_to_f32(synth.tokens(spec, 21))
    lazy = mo.moe_layer(x, synth.numpy_layer(spec, 21), "bf16")
    dense = mo.moe_layer(x, synth.numpy_layer(spec, 21, materialise=True), "bf16")
    np.testing.assert_array_equal(lazy["output"], dense["output"])
    np.testing.assert_array_equal(lazy["inds"], dense["inds"])


def test_layer_modes_agree_within_bf16_tolerance():
    from veymoe import synth

    spec = synth.LayerSpec("t", 256, 128, 32, 4, 128, 4)
    x = mo.bf16_bits_to_f32(synth.tokens(spec, 3))
    layer = synth.numpy_layer(spec, 3)
    b = mo.moe_layer(x, layer, "bf16")
    f = mo.moe_layer(x, layer, "f32")
    same = np.all(np.sort(b["inds"], 1) == np.sort(f["inds"], 1), axis=1)
    assert same.any()
    assert mo.max_abs_rel(b["output"][same], f["output"][same]) < 2e-2


def test_layer_decode_is_composition_of_parts():
    """Past layer 0 a decode layer is the fused executor call; layer 0 is the
    per-slot expert outputs through the generic combine (expert_cache.py:1434-1443)."""
    from veymoe import synth

    spec = synth.LayerSpec("t", 128, 64, 16, 4, 64, 2)
    x = mo.bf16_bits_to_f32(synth.tokens(spec, 8))
    for layer_id in (1, 0):
        layer = synth.numpy_layer(spec, 8, layer_id)
        out = mo.moe_layer(x, layer, "bf16")
        inds, scores, _ = mo.route(x, layer["router"], 4, "bf16")
        projections = {n: layer[n] for n in ("gate_proj", "up_proj", "down_proj")}
        shared, sg = mo.shared_expert(x, layer, "bf16")
        shared_y = mo.bf16r(sg * shared)
        if layer_id:
            *_, fused = mo.execute(x, inds, projections, "bf16", scores=scores, shared_y=shared_y)
            np.testing.assert_array_equal(out["output"], fused)
        else:
            *_, down, _ = mo.execute(x, inds, projections, "bf16")
            # (y * scores[..., None]).sum(-2) + shared, elementwise bf16 products
            want = mo.bf16r(mo.bf16r(sum(mo.bf16r(down[:, j] * scores[:, j:j + 1]) for j in range(4)))
                            + shared_y)
            np.testing.assert_array_equal(out["output"], want)
            assert not np.array_equal(out["output"], mo.moe_layer(x, layer, "bf16", combine="fused")["output"])


def test_qmm_projection_matches_loops():
    rng = np.random.default_rng(7)
    out_w, in_w = 5, 64
    q = rng.integers(0, 16, (out_w, in_w))
    w = np.array([ref_loops.pack_nibbles(r) for r in q], dtype=np.uint32)
    s = mo.f32_to_bf16_bits(rng.uniform(0.005, 0.02, (out_w, in_w // 32)).astype(np.float32))
    b = mo.f32_to_bf16_bits(rng.uniform(-0.1, 0.1, (out_w, in_w // 32)).astype(np.float32))
    x = mo.bf16r(rng.normal(size=(3, in_w)).astype(np.float32))
    got = mo.qmm_project(x, w, s, b)
    want = np.array(ref_loops.qmm_loops(x.tolist(), w.tolist(), s.tolist(), b.tolist()))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_qmm_projection_equals_vector_form_for_exact_weights():
    """scale 2^-6 and bias -2^-3: every scale*q + bias is exact in bf16, so
    rounding the weights changes nothing."""
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, (4, 96))
    w = np.array([ref_loops.pack_nibbles(r) for r in q], dtype=np.uint32)
    s = mo.f32_to_bf16_bits(np.full((4, 3), 2.0 ** -6, np.float32))
    b = mo.f32_to_bf16_bits(np.full((4, 3), -0.125, np.float32))
    x = rng.normal(size=(2, 96))
    np.testing.assert_allclose(mo.qmm_project(x, w, s, b), mo.q4_project(x, w, s, b), rtol=1e-12, atol=1e-12)


def test_qmm_projection_within_weight_rounding_bound():
    """|qmm - q4| <= sum |x| * half a bf16 step of |w| (2^-9 relative)."""
    rng = np.random.default_rng(9)
    q = rng.integers(0, 16, (6, 128))
    w = np.array([ref_loops.pack_nibbles(r) for r in q], dtype=np.uint32)
    s = mo.f32_to_bf16_bits(rng.uniform(0.005, 0.02, (6, 4)).astype(np.float32))
    b = mo.f32_to_bf16_bits(rng.uniform(-0.1, 0.1, (6, 4)).astype(np.float32))
    x = rng.normal(size=(5, 128))
    dense = mo.dequantize(w, s, b)
    bound = np.abs(x) @ (np.abs(dense) * 2.0 ** -8).T
    diff = np.abs(mo.qmm_project(x, w, s, b) - mo.q4_project(x, w, s, b))
    assert (diff <= bound + 1e-12).all()
    assert diff.max() > 0          # the rounding is really applied
