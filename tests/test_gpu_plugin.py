"""GPU: the benchmark's --custom-executor arm end to end (bench.py
run_custom_executor; the reference's bench_runtime_layer.py:148-225,
515-640): a target is loaded by name, turned into a runner, validated against
this package's executor on the same token and its ten routed experts, and both
arms are timed.  A target that reports the reference fallback is skipped, not
timed.

Targets: the executor class by module:attribute; a bare module exposing
``build_executor``; a runner function taking ``x, packs, indices, scores``
that computes the layer in plain torch fp32 (dequantised weights, bf16
rounding where the layer stores bf16), an independent check of the built-in
arm; and an executor whose ``last_path`` is ``"reference"``."""
import sys
import types

import pytest
import torch

import bench
from veymoe.executor import HipMoEExecutor

pytestmark = pytest.mark.gpu

SEED = 29


def _dequant(p, slot):
    """w = s*q + b in fp32, [out, in], from the MLX packing (nibble j of
    word i is input 8 i + j)."""
    w = p.weight[slot].to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, device=w.device, dtype=torch.int64) * 4
    q = ((w[..., None] >> shifts) & 15).reshape(w.shape[0], -1).float()
    s = p.scales[slot].float().repeat_interleave(32, dim=-1)
    b = p.biases[slot].float().repeat_interleave(32, dim=-1)
    return s * q + b


def _bf(t):
    return t.to(torch.bfloat16).float()


def torch_runner(x, packs, indices, scores):
    """The routed SwiGLU MoE of one token in torch fp32: gate and up rounded to
    bf16, SwiGLU in bf16 steps, each slot's down output rounded, the score
    combine summed in fp32 slot order and rounded."""
    xf = x.reshape(-1).float()
    y = torch.zeros(packs["down_proj"].weight.shape[1], device=x.device)
    for j, e in enumerate(indices.reshape(-1).tolist()):
        g = _bf(_dequant(packs["gate_proj"], e) @ xf)
        u = _bf(_dequant(packs["up_proj"], e) @ xf)
        act = _bf(_bf(g * _bf(torch.sigmoid(g))) * u)
        d = _bf(_dequant(packs["down_proj"], e) @ act)
        y = y + d * scores.reshape(-1)[j].float()
    return {"output": _bf(y).to(torch.bfloat16).reshape(x.shape)}


class FallbackExecutor:
    """An executor that ran the reference path: the harness must not time it."""

    last_path = "reference"
    fallback_reason = "backend unavailable"

    def __init__(self, expert_count, hidden_size, top_k):
        self.inner = HipMoEExecutor(expert_count, hidden_size, top_k)

    def execute(self, x, packs, indices, scores):
        return torch_runner(x, packs, indices, scores)


@pytest.fixture(scope="module", autouse=True)
def _modules():
    builder = types.ModuleType("vm_gpu_plug_builder")
    builder.build_executor = lambda expert_count, hidden_size, top_k: HipMoEExecutor(expert_count, hidden_size,
                                                                                         top_k)
    runner = types.ModuleType("vm_gpu_plug_runner")
    runner.run_layer = torch_runner
    runner.FallbackExecutor = FallbackExecutor
    sys.modules["vm_gpu_plug_builder"] = builder
    sys.modules["vm_gpu_plug_runner"] = runner
    yield
    del sys.modules["vm_gpu_plug_builder"], sys.modules["vm_gpu_plug_runner"]


@pytest.mark.parametrize("target", ["veymoe.executor:HipMoEExecutor", "vm_gpu_plug_builder",
                                    "vm_gpu_plug_runner:run_layer"])
def test_custom_executor_arm_validates_and_times(device, target):
    result = bench.run_custom_executor(target, SEED, calls=20)
    print(f"[plugin] {result}", flush=True)
    assert "skipped" not in result, result
    assert result["within_tolerance"], result
    assert result["builtin_us_per_call"] > 0 and result["custom_us_per_call"] > 0
    if target != "vm_gpu_plug_runner:run_layer":   # the same kernels as the built-in arm
        assert result["max_abs"] == 0.0, result


def test_custom_executor_fallback_is_skipped_not_timed(device):
    result = bench.run_custom_executor("vm_gpu_plug_runner:FallbackExecutor", SEED, calls=20)
    assert result["skipped"].startswith("reference fallback"), result
    assert "custom_us_per_call" not in result and "builtin_us_per_call" not in result


def test_custom_executor_that_cannot_load_is_skipped(device):
    result = bench.run_custom_executor("vm_gpu_plug_missing:run", SEED, calls=20)
    assert result["skipped"].startswith("ModuleNotFoundError"), result
