"""Executor argument contracts (models/flashnext/tests/unit/test_metal_runtime.py:19-155),
host side only: every check here fails before any kernel could run."""
import os
from types import SimpleNamespace
from unittest import mock

import numpy as np
import pytest

from veymoe.executor import HipMoEExecutor, probe_capabilities, weighted_combine


@pytest.mark.parametrize("kwargs", [
    {"expert_count": 0, "hidden_size": 2, "top_k": 1},
    {"expert_count": 2, "hidden_size": 0, "top_k": 1},
    {"expert_count": 2, "hidden_size": 2, "top_k": 0},
    {"expert_count": 513, "hidden_size": 2, "top_k": 1},
    {"expert_count": 2, "hidden_size": 2, "top_k": 11},
])
def test_constructor_rejects_bad_dimensions(kwargs):
    with pytest.raises(ValueError):
        HipMoEExecutor(**kwargs)


def test_constructor_rejects_top_k_larger_than_expert_count():
    with pytest.raises(ValueError):
        HipMoEExecutor(expert_count=2, hidden_size=2, top_k=3)


def test_constructor_bounds():
    with pytest.raises(ValueError):
        HipMoEExecutor(2, 32, 1, max_tokens=9)
    with pytest.raises(ValueError):
        HipMoEExecutor(2, 32, 1, max_width=16385)
    with pytest.raises(ValueError):
        HipMoEExecutor(2, 32, 1, group_size=64)


def test_combine_rejects_incompatible_route_shapes():
    with pytest.raises(ValueError):
        weighted_combine(np.zeros((2, 3, 2), np.float32), np.zeros((2, 2), np.int32), np.ones((2, 1), np.float32))


def test_combine_rejects_an_expert_index_out_of_range():
    with pytest.raises(ValueError):
        weighted_combine(np.zeros((2, 3, 2), np.float32), np.array([[0, 3]], np.int32), np.ones((1, 2), np.float32))


def test_execute_rejects_a_malformed_q4_projection_pack():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    bad = (np.zeros((2, 4, 3), np.uint32), np.zeros((2, 4, 1), np.float32), np.zeros((2, 4, 1), np.float32))
    valid = (np.zeros((2, 4, 4), np.uint32), np.zeros((2, 4, 1), np.float32), np.zeros((2, 4, 1), np.float32))
    projections = {"gate_proj": bad, "up_proj": valid,
                   "down_proj": (np.zeros((2, 32, 4), np.uint32), np.zeros((2, 32, 1), np.float32),
                                 np.zeros((2, 32, 1), np.float32))}
    with pytest.raises(ValueError, match="weight shape"):
        executor.execute(np.zeros((1, 32), np.float32), np.zeros((1, 1), np.int32), projections)


def test_execute_rejects_a_route_with_another_token_count():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    with pytest.raises(ValueError, match="same token count"):
        executor.execute(np.zeros((2, 32), np.float32), np.zeros((1, 1), np.int32), {})


def test_execute_rejects_shared_forms():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    x, routes = np.zeros((1, 32), np.float32), np.zeros((1, 1), np.int32)
    with pytest.raises(ValueError, match="together"):
        executor.execute(x, routes, {}, shared=np.zeros((1, 32)))
    with pytest.raises(ValueError, match="not both"):
        executor.execute(x, routes, {}, shared_y=np.zeros((1, 32)), shared=np.zeros((1, 32)),
                         shared_gate=np.zeros((1, 1)))
    with pytest.raises(ValueError, match="stream pack"):
        executor.execute(x, routes, {}, stream_pack=np.zeros(4))


def test_execute_rejects_weights_that_are_not_packed_words():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    proj = (np.zeros((2, 4, 4), np.float32), np.zeros((2, 4, 1), np.float32), np.zeros((2, 4, 1), np.float32))
    down = (np.zeros((2, 32, 4), np.uint32), np.zeros((2, 32, 1)), np.zeros((2, 32, 1)))
    with pytest.raises(TypeError, match="uint32"):
        executor.execute(np.zeros((1, 32), np.float32), np.zeros((1, 1), np.int32),
                         {"gate_proj": proj, "up_proj": proj, "down_proj": down})


def test_unavailable_backend_raises_instead_of_falling_back():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    proj = (np.zeros((2, 32, 4), np.uint32), np.zeros((2, 32, 1)), np.zeros((2, 32, 1)))
    down = (np.zeros((2, 32, 4), np.uint32), np.zeros((2, 32, 1)), np.zeros((2, 32, 1)))
    with pytest.raises(RuntimeError, match="custom MoE is unavailable"):
        executor.execute(np.zeros((1, 32), np.float32), np.zeros((1, 1), np.int32),
                         {"gate_proj": proj, "up_proj": proj, "down_proj": down})
    assert executor.last_path == "none"


def test_capabilities_report_unavailable_backend():
    caps = probe_capabilities(SimpleNamespace(available=False, supports_custom_moe=False))
    assert not caps.available and not caps.supports_custom_moe


def test_capabilities_enable_executor_only_when_supported():
    backend = SimpleNamespace(available=True, supports_custom_moe=True)
    executor = HipMoEExecutor(expert_count=2, hidden_size=2, top_k=1, backend=backend)
    assert executor.capabilities.supports_custom_moe


def test_unsupported_backend_fails_before_execution():
    backend = SimpleNamespace(available=True, supports_custom_moe=False)
    executor = HipMoEExecutor(expert_count=2, hidden_size=2, top_k=1, backend=backend)
    with pytest.raises(RuntimeError, match="custom MoE"):
        executor.execute(np.zeros((1, 2), np.float32), np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32))


def test_up_swiglu_fusion_flag_defaults_off_and_reads_the_environment():
    with mock.patch.dict(os.environ, {}, clear=False):
        os.environ.pop("FLASHNEXT_FUSED_UP_SWIGLU", None)
        assert not HipMoEExecutor(2, 32, 1).fused_up_swiglu
        assert HipMoEExecutor(2, 32, 1, fused_up_swiglu=True).fused_up_swiglu
        os.environ["FLASHNEXT_FUSED_UP_SWIGLU"] = "1"
        assert HipMoEExecutor(2, 32, 1).fused_up_swiglu


def test_probe_without_gpu_reports_reason():
    caps = probe_capabilities()
    import torch

    if not torch.cuda.is_available():
        assert not caps.available and caps.reason
