"""GPU: the DMA-ring Q4 GEMMs (the default gate/up + SwiGLU and down kernels
of calls above 64 rows) against the chunked GEMM they replace and against the
oracle's matrix form, at every K the ring is built for (512, 1024, 2048,
4096), with the down projection of K 256 left to the chunked GEMM in the same
call, with the shared expert's tile-less GEMMs on the side stream, and with
experts that span several row tiles.

Both kernels compute the matrix form of gather_qmm: every weight rounded to
bf16 once, fp32 sums.  They feed the MFMA the same products in a different
lane order (the ring takes its activation rows in input order, the chunked
GEMM pair-permuted), so they may differ by fp32 rounding order only: a row's
outputs agree within a bf16 step at the output's scale, and both match the
oracle at the layer tolerance."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_device, host
from oracle import moe_oracle as mo
from test_gpu_grouped import _assert_layer, _check_selection, _layer_ref
from veymoe import _lib, assemble, synth
from veymoe.pool import ExpertPool

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _restore_mode():
    lib = _lib.lib()
    saved = lib.vm_grouped_ring(-1)
    yield
    lib.vm_grouped_ring(saved)


def _both(layer, x):
    """Layer outputs and routes with the ring, then with the chunked GEMM."""
    lib = _lib.lib()
    out = {}
    for mode in (1, 0):
        assert lib.vm_grouped_ring(mode) in (0, 1)
        y = layer(x)
        torch.cuda.synchronize()
        out[mode] = (host(y), layer.last_inds.cpu().numpy())
    return out


@pytest.mark.parametrize("hidden,inter,experts,top_k,shared,tokens", [
    (2048, 512, 512, 10, 512, 2048),   # the prefill shape: gate/up K 2048, down K 512, shared expert
    (1024, 256, 64, 4, 0, 2048),       # gate/up K 1024 (the down GEMM's K 256 takes the chunked GEMM)
    (4096, 256, 128, 6, 0, 300),       # gate/up K 4096
    (512, 1024, 64, 4, 1024, 130),     # gate/up K 512, down K 1024, shared expert
], ids=["prefill-k2048", "k1024-2048rows", "k4096", "k512-down1024"])
def test_ring_against_chunked_and_the_oracle(device, hidden, inter, experts, top_k, shared, tokens):
    spec = synth.LayerSpec(f"qring_{hidden}_{inter}", hidden, inter, experts, top_k, shared, tokens)
    seed = 700 + hidden // 256 + tokens
    pool = ExpertPool(spec.layout, experts, layers=1, experts=experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, tokens))
    out = _both(layer, bf16_device(x_np, device))
    (ring, inds), (chunked, inds0) = out[1], out[0]
    np.testing.assert_array_equal(inds, inds0)      # the same router and selection in both calls
    scale = float(np.abs(chunked).max())
    diff = np.abs(ring.astype(np.float64) - chunked.astype(np.float64))
    print(f"[qring] {spec.name} T={tokens}: max |ring - chunked| {diff.max():.3g} (output scale {scale:.3g}), "
          f"identical elements {float((diff == 0).mean()):.4f}", flush=True)
    assert diff.max() <= 2.0 ** -7 * scale
    assert (diff == 0).mean() > 0.9
    sample = np.linspace(0, tokens - 1, min(tokens, 128)).astype(np.int64)
    ref = _layer_ref(spec, seed, x_np, sample)
    same = _check_selection(inds[sample], ref, top_k, max(1, len(sample) // 40), f"{spec.name} T={tokens}")
    _assert_layer(ring[sample], spec, seed, x_np, sample, same, ref, f"ring {spec.name} T={tokens}")


def test_ring_experts_spanning_several_tiles(device):
    """2048 rows over 16 experts top-2: ~256 rows per expert, four or five
    row tiles of 64 each, so an expert's weights stream once per tile and the
    last tile of each is partial; ring = chunked within a bf16 step, and the
    oracle on a sample."""
    spec = synth.LayerSpec("qring_tiles", 1024, 512, 16, 2, 0, 2048)
    seed = 733
    layer = assemble.build_layer(spec, seed, device, dense=True)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, 2048))
    out = _both(layer, bf16_device(x_np, device))
    (ring, inds), (chunked, _) = out[1], out[0]
    scale = float(np.abs(chunked).max())
    assert np.abs(ring.astype(np.float64) - chunked).max() <= 2.0 ** -7 * scale
    sample = np.random.default_rng(3).choice(2048, 64, replace=False)
    ref = _layer_ref(spec, seed, x_np, sample)
    same = _check_selection(inds[sample], ref, spec.top_k, 2, "16 experts T=2048")
    _assert_layer(ring[sample], spec, seed, x_np, sample, same, ref, "ring, experts over several tiles")


def test_ring_mode_switch(device):
    lib = _lib.lib()
    assert lib.vm_grouped_ring(-1) == 1                 # the ring is the default
    assert lib.vm_grouped_ring(0) == 1 and lib.vm_grouped_ring(-1) == 0
    assert lib.vm_grouped_ring(1) == 0 and lib.vm_grouped_ring(-1) == 1
    assert lib.vm_grouped_ring(2) == _lib.VM_EINVAL
