"""GPU parity of the decoder glue around the MoE call (veymoe.glue).

* vm_hyper_mix (qwen4_verifier.py:20-33) against oracle.glue_oracle.hyper_mix
  on the shapes of the reference's own glue test (hc 4, hidden 256, low rank
  32; test_compile_glue.py:17-29) and at hidden 2048: the normalised streams
  within one bf16 step (the mean of squares is summed in another order), the
  branch input and the injection weights within the layer tolerance; with
  selector projections (each output reads one input, so every dot product is
  exact) nearly all values bit for bit.
* The injection in the experts' epilogue (compile_glue.py:32-35): for decode
  and grouped calls, bit for bit the oracle's ``inject`` of the layer's own
  output, also in place.
* ``mlp_branch``: hyper-connection, MoE layer and injection against the oracle
  chain.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, host
from oracle import glue_oracle as go
from oracle import moe_oracle as mo
from veymoe import assemble, synth
from veymoe.glue import HyperConnection, mlp_branch

pytestmark = pytest.mark.gpu

SEED = 123


def _hyper_np(rng, hc, H, r):
    n = hc * H
    norm_w = mo.bf16r(rng.normal(1.0, 0.3, n).astype(np.float32))
    down = synth.q4_projection(rng, r, n)
    up = synth.q4_projection(rng, n, r)
    inj = synth.q4_projection(rng, hc, n)
    return norm_w, down, up, inj


def _hyper_dev(parts, hc, device, dtype=torch.bfloat16, **kw):
    norm_w, down, up, inj = parts
    return HyperConnection(torch.from_numpy(norm_w).to(device).to(dtype),
                           *(assemble.projection(*p, device) for p in (down, up, inj)), hc, **kw)


def _streams(rng, T, n, device, dtype=torch.bfloat16):
    x = mo.bf16r(rng.normal(0, 1.5, (T, n)).astype(np.float32))
    return x, torch.from_numpy(x).to(device).to(dtype)


def _ulps(a, b):
    ia = mo.f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int32)
    ib = mo.f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int32)
    return np.abs(ia - ib)


@pytest.mark.parametrize("hc,H,r,T,group", [(4, 256, 32, 1, 0), (4, 256, 32, 5, 256), (4, 2048, 32, 3, 0),
                                             (2, 512, 64, 37, 0)])
def test_hyper_mix_matches_the_oracle(device, hc, H, r, T, group):
    rng = np.random.default_rng(SEED + H + T)
    parts = _hyper_np(rng, hc, H, r)
    x, xd = _streams(rng, T, hc * H, device)
    hyper = _hyper_dev(parts, hc, device, norm_group=group)
    mixed, same, weights = hyper(xd)
    torch.cuda.synchronize()
    assert same is xd
    want_m, want_w, want_n = go.hyper_mix(x, parts[0], parts[1], parts[2], parts[3], hc, 1e-6, group_size=group)
    normed = hyper._ws[(T, 0, xd.device)][: T * hc * H * 2].view(torch.bfloat16).view(T, hc * H)
    u = _ulps(host(normed), want_n)
    assert u.max() <= 1 and (u == 0).mean() >= 0.99, (u.max(), (u == 0).mean())
    assert_close(host(weights), want_w, f"weights T={T}")
    assert_close(host(mixed), want_m, f"mixed T={T}")


def test_hyper_mix_float32(device):
    hc, H, r, T = 4, 256, 32, 2
    rng = np.random.default_rng(SEED)
    parts = _hyper_np(rng, hc, H, r)
    x, xd = _streams(rng, T, hc * H, device, torch.float32)
    mixed, _, weights = _hyper_dev(parts, hc, device, torch.float32)(xd)
    torch.cuda.synchronize()
    want_m, want_w, _ = go.hyper_mix(x, parts[0], *parts[1:], hc, 1e-6, mode="f32")
    np.testing.assert_allclose(host(mixed), want_m, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(host(weights), want_w, rtol=1e-4, atol=1e-5)


def _selector(rows, cols, pick):
    q = np.zeros((rows, cols), np.uint32)
    q[np.arange(rows), pick] = 1
    words = np.zeros((rows, cols // 8), np.uint32)
    for k in range(8):
        words |= q[:, k::8] << np.uint32(4 * k)
    one = mo.f32_to_bf16_bits(np.ones((rows, cols // 32), np.float32))
    zero = mo.f32_to_bf16_bits(np.zeros((rows, cols // 32), np.float32))
    return words, one, zero


def test_hyper_mix_with_selector_projections_is_nearly_exact(device):
    hc, H, r, T = 4, 256, 32, 3
    n = hc * H
    rng = np.random.default_rng(SEED + 1)
    norm_w = mo.bf16r(rng.normal(1.0, 0.3, n).astype(np.float32))
    parts = (norm_w, _selector(r, n, (7 * np.arange(r) + 3) % n), _selector(n, r, (5 * np.arange(n) + 1) % r),
             _selector(hc, n, np.array([1, 300, 600, 1000])))
    x, xd = _streams(rng, T, n, device)
    mixed, _, weights = _hyper_dev(parts, hc, device)(xd)
    torch.cuda.synchronize()
    want_m, want_w, _ = go.hyper_mix(x, *parts, hc, 1e-6)
    for got, want in ((host(mixed), want_m), (host(weights), want_w)):
        u = _ulps(got, want)
        assert u.max() <= 1 and (u == 0).mean() >= 0.98, (u.max(), (u == 0).mean())


SMALL = synth.LayerSpec("glue_small", 256, 128, 64, 4, 128, 1)


@pytest.mark.parametrize("T", [1, 3, 8, 40])
@pytest.mark.parametrize("in_place", [False, True])
def test_injection_in_the_experts_epilogue_is_exact(device, T, in_place):
    hc = 4
    layer = assemble.build_layer(SMALL, SEED, device, dense=True)
    rng = np.random.default_rng(SEED + T)
    x = assemble.tokens_tensor(SMALL, SEED, device, T, stream=9)
    streams = torch.from_numpy(mo.bf16r(rng.normal(0, 1, (T, hc * SMALL.hidden)).astype(np.float32))).to(device)
    streams = streams.to(torch.bfloat16)
    weights = torch.from_numpy(mo.bf16r(rng.uniform(0, 2, (T, hc)).astype(np.float32))).to(device).to(torch.bfloat16)
    before = host(streams)
    target = streams if in_place else torch.empty_like(streams)
    y = layer.forward(x, inject=(streams, weights, target))
    torch.cuda.synchronize()
    want = go.inject(before, host(y), host(weights))
    np.testing.assert_array_equal(host(target), want)
    # the plain call afterwards leaves no injection behind
    y2 = layer.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))
    np.testing.assert_array_equal(host(target), want)


def test_mlp_branch_matches_the_oracle_chain(device):
    hc, T = 4, 2
    spec = SMALL
    H = spec.hidden
    rng = np.random.default_rng(SEED + 7)
    parts = _hyper_np(rng, hc, H, 32)
    hyper = _hyper_dev(parts, hc, device)
    layer = assemble.build_layer(spec, SEED, device, dense=True)
    x, xd = _streams(rng, T, hc * H, device)
    out = mlp_branch(hyper, layer, xd)
    torch.cuda.synchronize()
    mixed, weights, _ = go.hyper_mix(x, *parts, hc, 1e-6)
    y = mo.moe_layer(mixed, synth.numpy_layer(spec, SEED, 0, materialise=True), "bf16")["output"]
    want = go.inject(x, y, weights)
    assert_close(host(out), want, "mlp branch")
    # in place on the streams
    again = xd.clone()
    mlp_branch(hyper, layer, again, out=again)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))
