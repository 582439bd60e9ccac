"""Every bf16 gate bit pattern through the SwiGLU epilogue of the HIP gate/up
kernel, against the oracle's op-by-op sequence (metal_runtime.py:267-285).

The reference scans all 65,536 gate patterns at up = 0x3F80 and 0x3F9E
against MLX's bf16 ``silu(gate) * up`` (models/flashnext/tests/unit/
test_swiglu_contract.py:65-83, harness tests/bench/swiglu_contract.py).

Selector projections make the Q4/G32 projections emit chosen values exactly:

* input group g < 64 of token t holds one pattern in its first input and
  zeros elsewhere; group 64 holds a single 1.0 (the constant group);
* gate row r reads group r only (nibble q = 1 on its first input, scale 1,
  bias 0; every other group scale 0, bias 0): gate = x exactly, since the
  kernel's (128 + q) pairing gives 129x - 128x;
* the up row of expert j reads the constant group only (q = 0, scale 0,
  bias u_j): up = u_j.

The pairing multiplies inputs by 128 and 129, so a Q4 projection cannot emit
patterns whose magnitude times 129 leaves the fp32 range (|x| >= 2^120) or
the non-finite ones: those 2,304 patterns are skipped, and the count is
asserted.  A gate of -0 sums to +0 on the way (0 + -0), so its
expected activation is that of +0."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from veymoe.executor import HipMoEExecutor, Q4G32Projection

pytestmark = pytest.mark.gpu

GROUPS = 64            # value groups per token (one pattern each)
HIDDEN = (GROUPS + 1) * 32
INTER = GROUPS         # gate row r selects value group r
TOKENS = 8
UPS = (0x3F80, 0x3F9E)  # the reference's two up patterns


def _patterns():
    bits = np.arange(1 << 16, dtype=np.uint32)
    exponent = (bits >> 7) & 0xFF
    usable = exponent <= 119 + 127        # |x| < 2^120: 129 * x stays finite in fp32
    return bits[usable].astype(np.uint16), int((~usable).sum())


def _selector_projections(device):
    words = HIDDEN // 8
    gate_w = np.zeros((2, INTER, words), np.uint32)
    gate_s = np.zeros((2, INTER, HIDDEN // 32), np.float32)
    gate_b = np.zeros_like(gate_s)
    for r in range(INTER):
        gate_w[:, r, r * 4] = 1              # nibble 0 of the group's first word: input 32 r
        gate_s[:, r, r] = 1.0
    up_w = np.zeros((2, INTER, words), np.uint32)
    up_s = np.zeros((2, INTER, HIDDEN // 32), np.float32)
    up_b = np.zeros_like(up_s)
    for j, u in enumerate(UPS):
        up_b[j, :, GROUPS] = mo.bf16_bits_to_f32(np.array([u], np.uint16))[0]
    down_w = np.zeros((2, HIDDEN, INTER // 8), np.uint32)
    down_m = np.zeros((2, HIDDEN, INTER // 32), np.float32)

    def proj(w, s, b):
        bf = lambda a: torch.from_numpy(mo.f32_to_bf16_bits(a).view(np.int16)).to(device).view(torch.bfloat16)
        return Q4G32Projection(torch.from_numpy(w.view(np.int32)).to(device), bf(s), bf(b))

    return proj(gate_w, gate_s, gate_b), proj(up_w, up_s, up_b), proj(down_w, down_m, down_m)


def test_every_finite_gate_pattern_through_the_gateup_epilogue(device):
    patterns, skipped = _patterns()
    assert skipped == 2304 and patterns.size == 65536 - 2304
    gate, up, down = _selector_projections(device)
    ex = HipMoEExecutor(2, HIDDEN, 2)
    routes = torch.tensor([[0, 1]] * TOKENS, dtype=torch.int32, device=device)
    per_call = TOKENS * GROUPS
    padded = np.concatenate([patterns, np.zeros(-patterns.size % per_call, np.uint16)])
    got_gate, got_act = [], []
    for start in range(0, padded.size, per_call):
        chunk = padded[start:start + per_call].reshape(TOKENS, GROUPS)
        x = np.zeros((TOKENS, HIDDEN), np.uint16)
        x[:, 0:GROUPS * 32:32] = chunk
        x[:, GROUPS * 32] = 0x3F80
        xt = torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
        g, _, _ = ex._run(xt, routes, gate, up, down, INTER, True, None, None, None, None, None, None, None)
        act = ex._run(xt, routes, gate, up, down, INTER, False, None, None, None, None, None, None, None,
                      activations_only=True)
        got_gate.append(g.view(torch.int16).cpu().numpy().view(np.uint16))
        got_act.append(act.view(torch.int16).cpu().numpy().view(np.uint16))
    assert ex.status() == 0
    n = patterns.size
    gate_bits = np.concatenate([a.reshape(TOKENS, 2, GROUPS).transpose(1, 0, 2).reshape(2, -1) for a in got_gate],
                               axis=1)[:, :n]
    act_bits = np.concatenate([a.reshape(TOKENS, 2, GROUPS).transpose(1, 0, 2).reshape(2, -1) for a in got_act],
                              axis=1)[:, :n]
    # the selectors deliver every pattern (-0 arrives as +0)
    want_gate = np.where(patterns == 0x8000, 0, patterns)
    for j in range(2):
        np.testing.assert_array_equal(gate_bits[j], want_gate)
    gate_f = mo.bf16_bits_to_f32(want_gate)
    mismatches = {}
    for j, u in enumerate(UPS):
        up_f = np.full_like(gate_f, mo.bf16_bits_to_f32(np.array([u], np.uint16))[0])
        want = mo.f32_to_bf16_bits(mo.swiglu(gate_f, up_f, "bf16"))
        same = (act_bits[j] == want) | (np.isnan(mo.bf16_bits_to_f32(act_bits[j]))
                                        & np.isnan(mo.bf16_bits_to_f32(want)))
        mismatches[hex(u)] = int((~same).sum())
        bad = np.nonzero(~same)[0][:4]
        assert same.all(), (hex(u), [(hex(patterns[i]), hex(act_bits[j][i]), hex(want[i])) for i in bad])
    print(f"[swiglu] {n} gate patterns x {len(UPS)} up patterns, mismatches {mismatches}, "
          f"{skipped} patterns outside the Q4 projection's range skipped")
