"""The --custom-executor plug-in convention of the benchmark harness
(bench_runtime_layer.py:86-227 of the reference), on the CPU with stand-in
executors: name discovery, signature-driven calls, output normalisation and
load failures."""
import sys
import types

import pytest

from veymoe import plugin

CONTEXT = {"x": "X", "packs": "P", "indices": "I", "group_size": 32, "bits": 4, "mode": "affine", "top_k": 2,
           "scores": "S", "hidden_size": 8, "expert_count": 2}


def _module(name, **attrs):
    mod = types.ModuleType(name)
    for key, value in attrs.items():
        setattr(mod, key, value)
    sys.modules[name] = mod
    return mod


def test_bare_module_entry_names_in_reference_order():
    _module("vm_plug_a", run=lambda x: ("run", x), build_executor=lambda packs: ("built", packs))
    assert plugin.load_target("vm_plug_a")(CONTEXT["packs"]) == ("built", "P")
    _module("vm_plug_b", run=lambda x: ("run", x))
    assert plugin.load_target("vm_plug_b")("X") == ("run", "X")
    _module("vm_plug_c", helper=1)
    with pytest.raises(AttributeError):
        plugin.load_target("vm_plug_c")


def test_module_attribute_and_load_failures():
    _module("vm_plug_d", my_runner=lambda x, indices: (x, indices))
    target, reason = plugin.load_custom_executor("vm_plug_d:my_runner")
    assert reason is None and target("a", "b") == ("a", "b")
    assert plugin.load_custom_executor(None) == (None, "not requested")
    target, reason = plugin.load_custom_executor("vm_plug_missing_module:x")
    assert target is None and reason.startswith("ModuleNotFoundError")
    target, reason = plugin.load_custom_executor("vm_plug_d:absent")
    assert target is None and reason.startswith("AttributeError")


def test_builders_classes_and_runners():
    class Executor:
        def __init__(self, expert_count, hidden_size, top_k):
            self.shape = (expert_count, hidden_size, top_k)

        def execute(self, x, indices, scores=None):
            return {"output": (x, indices, scores, self.shape)}

    runner = plugin.runner_from_target(Executor, CONTEXT)
    assert runner.shape == (2, 8, 2)
    out = plugin.normalise_output(plugin.run_custom(runner, CONTEXT))
    assert out == ("X", "I", "S", (2, 8, 2))

    def builder(packs, group_size, bits, mode):
        return lambda x, rhs_indices=None: (x, packs, group_size, bits, mode, rhs_indices)

    runner = plugin.runner_from_target(builder, CONTEXT)
    assert plugin.run_custom(runner, dict(CONTEXT, rhs_indices="R")) == ("X", "P", 32, 4, "affine", "R")

    def direct(x, indices, **rest):           # a runner: takes x / indices, receives every other name
        return (x, indices, sorted(rest))

    assert plugin.runner_from_target(direct, CONTEXT) is direct
    assert plugin.run_custom(direct, CONTEXT)[2] == sorted(k for k in CONTEXT if k not in ("x", "indices"))

    mod = _module("vm_plug_e", create_executor=lambda top_k: (lambda x: (x, top_k)))
    assert plugin.run_custom(plugin.runner_from_target(mod, CONTEXT), CONTEXT) == ("X", 2)


def test_missing_required_argument_and_output_forms():
    def needs_more(x, packs, indices, group_size, bits, mode, scale):
        return x

    with pytest.raises(TypeError):
        plugin.invoke(needs_more, CONTEXT)
    assert plugin.normalise_output(("only",)) == "only"
    assert plugin.normalise_output({"y": 3}) == 3
    with pytest.raises(TypeError):
        plugin.normalise_output((1, 2))


def test_fallback_paths_are_not_native():
    class Fell:
        last_path = "reference"

    class Native:
        last_path = "hip"

    assert not plugin.uses_native_path(Fell())
    assert plugin.uses_native_path(Native())
    assert plugin.uses_native_path(object())
