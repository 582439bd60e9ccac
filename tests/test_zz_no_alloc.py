"""vm_moe_layer_static, the layer entry point that allocates nothing (its
workspace is the library's static per-device scratch), against vm_moe_layer
with a caller's workspace: the same bits, on two calls in a row whose second
is smaller, for the decode kernels and for the grouped path.  The caller's
workspace is filled with a pattern first, and the static scratch keeps the
previous call's contents, so neither result can lean on zeroed memory."""
import ctypes

import pytest
import torch

from veymoe import _lib, assemble, synth
from veymoe.device import ptr, stream_handle
from veymoe.pool import ExpertPool

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pooled_layer(device):
    """hidden 2048 / inter 512 / 512 experts top-10 + shared expert, every
    expert resident at a permuted slot behind the slot table."""
    spec = synth.CONFIGS["decode"]
    seed = 4242
    pool = ExpertPool(spec.layout, 600, layers=1, experts=spec.experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    return spec, seed, layer


def _both_entry_points(layer, spec, seed, device, tokens, stream):
    lib = _lib.lib()
    x = assemble.tokens_tensor(spec, seed, device, tokens, stream=stream)
    k = layer.top_k
    outs, inds, scores = [], [], []
    for entry in ("vm_moe_layer", "vm_moe_layer_static"):
        out = torch.full_like(x, float("nan"))
        ind = torch.full((tokens, k), -7, dtype=torch.int32, device=device)
        sc = torch.full((tokens, k), float("nan"), dtype=x.dtype, device=device)
        args = layer.layer_args(x, out, ind, sc)
        args.x, args.output = ptr(x), ptr(out)
        if entry == "vm_moe_layer":
            nbytes = int(args.workspace_bytes)
            ws = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device=device)
            args.workspace, args.workspace_bytes = ptr(ws), nbytes
        else:
            args.workspace, args.workspace_bytes = None, 0
        print(f"[no-alloc] {entry} tokens={tokens}", flush=True)
        _lib.check(getattr(lib, entry)(ctypes.byref(args), stream_handle()))
        torch.cuda.synchronize()
        outs.append(out)
        inds.append(ind)
        scores.append(sc)
    return outs, inds, scores


@pytest.mark.parametrize("sizes", [(8, 1), (48, 12)], ids=["decode", "grouped"])
def test_static_scratch_layer_equals_the_workspace_layer(device, pooled_layer, sizes):
    spec, seed, layer = pooled_layer
    lib = _lib.lib()
    for n, tokens in enumerate(sizes):
        need = lib.vm_moe_layer_workspace(tokens, layer.top_k, spec.hidden, spec.inter, spec.shared_inter,
                                          spec.experts, _lib.VM_BF16)
        assert need <= _lib.VM_STATIC_SCRATCH_BYTES
        outs, inds, scores = _both_entry_points(layer, spec, seed, device, tokens, stream=30 + n)
        assert not torch.isnan(outs[0].float()).any()
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), (sizes, tokens)
        assert torch.equal(inds[0], inds[1]), (sizes, tokens)
        assert torch.equal(scores[0].view(torch.int16), scores[1].view(torch.int16)), (sizes, tokens)


def test_static_scratch_layer_refuses_a_call_above_its_size(device, pooled_layer):
    spec, seed, layer = pooled_layer
    tokens = 2048
    x = assemble.tokens_tensor(spec, seed, device, tokens, stream=5)
    out = torch.empty_like(x)
    args = layer.layer_args(x, out)
    args.workspace, args.workspace_bytes = None, 0
    assert _lib.lib().vm_moe_layer_static(ctypes.byref(args), stream_handle()) == _lib.VM_EWORKSPACE
    assert "static" in _lib.last_error()
