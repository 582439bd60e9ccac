"""The C restatement (CPU baseline) agrees with the NumPy oracle."""
import numpy as np
import pytest

from oracle import moe_oracle as mo
from veymoe import synth


def _c_layer(spec, seed):
    from oracle.cmoe import CDecodeLayer

    layout = spec.layout
    records = np.zeros((spec.experts, layout.record_stride), np.uint8)
    for e in range(spec.experts):
        synth.expert_record(spec, seed, 0, e, out=records[e])
    shared = synth.shared_parts(spec, seed, 0)
    return CDecodeLayer(spec.hidden, spec.inter, spec.experts, spec.top_k, synth.router_weight(spec, seed, 0),
                        records, layout.record_stride, layout.part_offsets(),
                        router_bias=synth.router_bias(spec, seed, 0), shared=shared)


@pytest.mark.parametrize("spec", [synth.CONFIGS["decode_small"], synth.LayerSpec("s", 512, 256, 32, 4, 256, 1)])
def test_c_restatement_matches_numpy_oracle(spec):
    seed = 31
    c = _c_layer(spec, seed)
    layer = synth.numpy_layer(spec, seed)
    for stream in range(3):
        x_bits = synth.tokens(spec, seed, 1, stream=stream)
        inds, scores, y_bits = c.run(x_bits[0])
        # the C restatement is a layer past layer 0: the fused combine
        ref = mo.moe_layer(mo.bf16_bits_to_f32(x_bits), layer, "bf16", combine="fused")
        np.testing.assert_array_equal(inds, ref["inds"][0])
        np.testing.assert_array_equal(scores, ref["scores"][0])
        y = mo.bf16_bits_to_f32(y_bits)
        # fp32 (C) vs float64 (NumPy) accumulation: rare one-ulp bf16 flips
        assert mo.max_abs_rel(y, ref["output"][0]) < 1e-2
