"""The shared expert of grouped calls above 256 rows runs on a second stream
of the calling thread (forked from the caller's stream before the router
GEMM, joined back before the combine).  vm_moe_layer_static never creates
that stream, so it takes the one-stream path, where the shared expert is one
more group of the sorted GEMMs, as every grouped call of up to 256 rows does:
the two entry points must give the same bits (65 rows: both one-stream; 257
and 777 rows: the side stream against the one-stream path).  The
fork and join must also hold inside a captured HIP graph: every replay, with
eager calls between the replays, equals the eager call on the same input."""
import ctypes

import pytest
import torch

from veymoe import _lib, assemble, synth
from veymoe.device import ptr, stream_handle

pytestmark = pytest.mark.gpu

SEED = 57
# hidden 256, inter 128, 64 experts top-4, shared expert of inter 128
SPEC = synth.LayerSpec("shared_stream", 256, 128, 64, 4, 128, 1)


def _call(layer, x, entry):
    out = torch.full_like(x, float("nan"))
    inds = torch.full((x.shape[0], layer.top_k), -7, dtype=torch.int32, device=x.device)
    scores = torch.full((x.shape[0], layer.top_k), float("nan"), dtype=x.dtype, device=x.device)
    args = layer.layer_args(x, out, inds, scores)
    if entry == "vm_moe_layer_static":
        args.workspace, args.workspace_bytes = None, 0
    print(f"[shared-stream] {entry} tokens={x.shape[0]}", flush=True)
    _lib.check(getattr(_lib.lib(), entry)(ctypes.byref(args), stream_handle()))
    torch.cuda.synchronize()
    return out, inds, scores


@pytest.mark.parametrize("tokens", [65, 257, 777])
def test_side_stream_shared_expert_equals_the_one_stream_path(device, tokens):
    layer = assemble.build_layer(SPEC, SEED, device, dense=True)
    need = _lib.lib().vm_moe_layer_workspace(tokens, SPEC.top_k, SPEC.hidden, SPEC.inter, SPEC.shared_inter,
                                             SPEC.experts, _lib.VM_BF16)
    assert need <= _lib.VM_STATIC_SCRATCH_BYTES
    x = assemble.tokens_tensor(SPEC, SEED, device, tokens, stream=tokens)
    side = _call(layer, x, "vm_moe_layer")
    one = _call(layer, x, "vm_moe_layer_static")
    assert not torch.isnan(side[0].float()).any()
    assert torch.equal(side[0].view(torch.int16), one[0].view(torch.int16)), tokens
    assert torch.equal(side[1], one[1]), tokens
    assert torch.equal(side[2].view(torch.int16), one[2].view(torch.int16)), tokens


def test_side_stream_fork_and_join_replay_in_a_graph(device):
    tokens = 300
    layer = assemble.build_layer(SPEC, SEED + 1, device, dense=True)
    lib = _lib.lib()
    x = assemble.tokens_tensor(SPEC, SEED, device, tokens, stream=0)
    out = torch.empty_like(x)
    args = layer.layer_args(x, out)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # an eager call first: the side stream exists before the capture
        _lib.check(lib.vm_moe_layer(ctypes.byref(args), stream_handle(stream)))
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream, capture_error_mode="relaxed"):
        _lib.check(lib.vm_moe_layer(ctypes.byref(args), stream_handle(torch.cuda.current_stream())))
    for step in range(1, 5):
        xi = assemble.tokens_tensor(SPEC, SEED, device, tokens, stream=step)
        want = _call(layer, xi, "vm_moe_layer")[0]
        x.copy_(xi)
        print(f"[shared-stream] graph replay {step}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), step
