"""Pins of the decoder-glue oracle (oracle/glue_oracle.py) on the CPU.

RMSNorm (patch_rmsnorm.py:108-135): exact closed forms (a constant row
normalises to the gain; eps = 0 makes it scale invariant), group
independence, the one-/zero-centered gain rule.  Injection
(compile_glue.py:32-35): zero weights, selector weights and exact integer
sums, stream order.  Hyper-connection mix (qwen4_verifier.py:20-33): with
selector Q4 weights every projection picks one input, so the whole chain has
a closed form that an element-by-element loop below states without reshapes;
a swapped reshape axis, a dropped ``/ hc`` or a wrong stream pairing fails it.
"""
import numpy as np
import pytest

from oracle import glue_oracle as go
from oracle import moe_oracle as mo

RNG = np.random.default_rng(8)


def _bf16(values):
    return mo.bf16r(np.asarray(values, dtype=np.float32))


# ---------------------------------------------------------------- rms norm --

def test_rms_norm_of_a_constant_row_is_the_gain():
    w = _bf16(RNG.normal(1.0, 0.3, 64))
    for c in (2.0, -0.5, 8.0):
        y = go.rms_norm(np.full((1, 64), c, np.float32), w, eps=0.0)
        np.testing.assert_array_equal(y[0], _bf16(np.sign(c) * w))


def test_rms_norm_is_scale_invariant_without_eps():
    x = _bf16(RNG.normal(0, 1, (3, 256)))
    w = _bf16(RNG.normal(1.0, 0.2, 256))
    for k in (0.25, 4.0, 1024.0):
        np.testing.assert_array_equal(go.rms_norm(x * np.float32(k), w, 0.0), go.rms_norm(x, w, 0.0))


def test_rms_norm_known_values():
    # [3, 4]: mean of squares 12.5, y = x / sqrt(12.5)
    y = go.rms_norm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32), eps=0.0, mode="f32")
    np.testing.assert_allclose(y[0], [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)], rtol=1e-6)
    # eps enters under the root: [1, 1] with eps 3 -> 1 / 2
    y = go.rms_norm(np.ones((1, 2), np.float32), np.ones(2, np.float32), eps=3.0, mode="f32")
    np.testing.assert_array_equal(y[0], [0.5, 0.5])


def test_rms_norm_groups_normalise_independently():
    x = _bf16(RNG.normal(0, 1, (2, 128)))
    w = _bf16(RNG.normal(1.0, 0.2, 128))
    grouped = go.rms_norm(x, w, 1e-6, group_size=32)
    for g in range(4):
        part = go.rms_norm(x[:, 32 * g:32 * g + 32], w[32 * g:32 * g + 32], 1e-6)
        np.testing.assert_array_equal(grouped[:, 32 * g:32 * g + 32], part)
    assert not np.array_equal(grouped, go.rms_norm(x, w, 1e-6))


def test_zero_centered_gain_adds_one():
    x = _bf16(RNG.normal(0, 1, (2, 64)))
    w = _bf16(RNG.uniform(-0.5, 0.5, 64))
    np.testing.assert_array_equal(go.rms_norm(x, w, 1e-6, one_centered=False),
                                  go.rms_norm(x, (np.float32(1) + w).astype(np.float32), 1e-6))
    assert go.rms_norm(x, np.zeros(64, np.float32), 1e-6, one_centered=False).any()   # gain 1 + 0
    assert not go.rms_norm(x, np.zeros(64, np.float32), 1e-6).any()                    # gain 0


# ------------------------------------------------------------------ inject --

def test_inject_zero_weights_keep_the_streams():
    h = _bf16(RNG.normal(0, 1, (2, 4 * 32)))
    b = _bf16(RNG.normal(0, 1, (2, 32)))
    np.testing.assert_array_equal(go.inject(h, b, np.zeros((2, 4), np.float32)), h)


def test_inject_streams_in_order_with_exact_values():
    # hc = 2, H = 3: stream j gets branch * weights[j]
    h = np.array([[1, 2, 3, 10, 20, 30]], np.float32)
    b = np.array([[1, -1, 2]], np.float32)
    w = np.array([[2, 0.5]], np.float32)
    np.testing.assert_array_equal(go.inject(h, b, w), [[3, 0, 7, 10.5, 19.5, 31]])
    # zero streams with unit weights: the branch tiled hc times
    np.testing.assert_array_equal(go.inject(np.zeros((1, 6), np.float32), b, np.ones((1, 2), np.float32)),
                                  np.tile(b, (1, 2)))


def test_inject_rounds_the_product_then_the_sum():
    # b * w = 2^-8 (1 + 2^-8 - 2^-15) rounds to 2^-8; 1 + 2^-8 is then a tie
    # that goes to the even 1.0.  Without the product's rounding the sum
    # would be above the tie: 1 + 2^-7.
    h = np.array([[1.0]], np.float32)
    b = np.array([[2.0 ** -8 * (1 + 2.0 ** -7)]], np.float32)
    w = np.array([[1 - 2.0 ** -8]], np.float32)
    assert go.inject(h, b, w)[0, 0] == 1.0
    assert mo.bf16r(np.float32(1) + b * w)[0, 0] == 1 + 2.0 ** -7


# ------------------------------------------------------------- hyper mix ----

def _selector(rows, cols, pick):
    """Q4/G32 weights whose row r is the one-hot vector of input pick[r]:
    nibble 1 there, 0 elsewhere, scale 1, bias 0 (so W . x = x[pick[r]])."""
    q = np.zeros((rows, cols), np.uint32)
    q[np.arange(rows), pick] = 1
    words = np.zeros((rows, cols // 8), np.uint32)
    for k in range(8):
        words |= q[:, k::8] << np.uint32(4 * k)
    one = mo.f32_to_bf16_bits(np.ones((rows, cols // 32), np.float32))
    zero = mo.f32_to_bf16_bits(np.zeros((rows, cols // 32), np.float32))
    return words[None], one[None], zero[None]


def test_selector_weights_pick_one_input():
    x = _bf16(RNG.normal(0, 1, (2, 64)))
    pick = np.array([5, 63, 0, 32])
    got = go.linear(x, tuple(a[0] for a in _selector(4, 64, pick)), "bf16")
    np.testing.assert_array_equal(got, x[:, pick])


def test_hyper_mix_follows_the_reference_chain_element_by_element():
    T, hc, H, r = 2, 4, 32, 32
    n = hc * H
    hidden = _bf16(RNG.normal(0, 2, (T, n)))
    norm_w = _bf16(RNG.normal(1.0, 0.2, n))
    pick_down = (7 * np.arange(r) + 3) % n                    # W_down row k reads normed[pick_down[k]]
    pick_up = (5 * np.arange(n) + 1) % r                      # W_up row o reads d[pick_up[o]]
    pick_inj = np.array([1, 40, 77, 120])                     # W_inj row j reads normed[pick_inj[j]]
    down, up, inj = (tuple(a[0] for a in _selector(rows, cols, pick))
                     for rows, cols, pick in ((r, n, pick_down), (n, r, pick_up), (hc, n, pick_inj)))
    mixed, weights, normed = go.hyper_mix(hidden, norm_w, down, up, inj, hc, 1e-6)
    np.testing.assert_array_equal(normed, go.rms_norm(hidden, norm_w, 1e-6))

    def b(v):
        return float(_bf16(np.float32(v)))

    def sig(v):
        return float(mo.sigmoid(np.float32(v), "bf16"))

    for t in range(T):
        d = []
        for k in range(r):
            a = b(normed[t, pick_down[k]] / hc)
            d.append(b(a * sig(a)))
        for h in range(H):
            total = np.float32(0)
            for j in range(hc):
                o = j * H + h                                  # stream j, element h
                m = sig(d[pick_up[o]])
                total = np.float32(total + np.float32(b(m * normed[t, o])))
            assert mixed[t, h] == b(b(total) * b(1.0 / hc)), (t, h)
        for j in range(hc):
            assert weights[t, j] == b(2 * sig(b(normed[t, pick_inj[j]] / hc))), (t, j)


def test_hyper_mix_mixed_is_the_stream_mean_when_the_mix_is_one():
    # a large positive up-projection output saturates the sigmoid at 1.0:
    # mixed = mean of the normalised streams
    T, hc, H, r = 1, 2, 64, 32
    n = hc * H
    hidden = _bf16(RNG.normal(0, 1, (T, n)))
    norm_w = np.ones(n, np.float32)
    down = tuple(a[0] for a in _selector(r, n, np.arange(r)))
    w_up = np.full((1, n, r // 8), 0xFFFFFFFF, np.uint32)   # every nibble 15
    s_up = mo.f32_to_bf16_bits(np.zeros((1, n, 1), np.float32))
    b_up = mo.f32_to_bf16_bits(np.full((1, n, 1), 64.0, np.float32))  # bias 64 on sum(d): large when sum(d) > 0
    inj = tuple(a[0] for a in _selector(hc, n, np.arange(hc)))
    mixed, _w, normed = go.hyper_mix(hidden, norm_w, down, (w_up[0], s_up[0], b_up[0]), inj, hc, 1e-6)
    d_sum = go.linear(go.rms_norm(hidden, norm_w, 1e-6), down, "bf16")
    if float(mo.silu(_bf16(d_sum / hc), "bf16").sum()) <= 0.5:
        pytest.skip("seed gave a small mix input")
    s = normed.reshape(T, hc, H)
    want = _bf16(_bf16(_bf16(s[:, 0] + s[:, 1])) * np.float32(0.5))
    np.testing.assert_array_equal(mixed, want)
