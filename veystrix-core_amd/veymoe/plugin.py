"""The benchmark harness's custom-executor plug-in convention.

The reference's layer benchmark takes ``--custom-executor module:attr``
(models/flashnext/tests/bench/bench_runtime_layer.py:11-25, 86-225) and finds
an executor in what it names:

* ``module:attr`` names the target; a bare ``module`` is searched for
  ``build_executor``, ``create_executor``, ``MetalMoEExecutor``,
  ``Executor``, ``execute``, ``run`` in that order (:86-98);
* a module, class, builder or runner becomes a runner: builders and classes
  are called with the context names their signature asks for, objects with
  ``execute``/``run`` and callables that take ``x``/``inputs``/``indices``/
  ``rhs_indices``/``route`` are runners already (:148-172);
* a runner is called with the context names its signature asks for (:110-145);
  the executor of this package takes its flattened production call instead
  (the reference does the same for ``MetalMoEExecutor``, :175-203), and an
  output with one axis more than the scores is combined with them;
* a runner that reports a fallback (``last_path`` other than the native one)
  is not timed (:206-213); an output may be an array, a one-item tuple or a
  mapping with ``output``/``out``/``y``/``result`` (:216-227).

The context carries the reference's aliases (:383-409): the activations, the
packed projections of the routed experts only (a compact bank, so ``routes``
are local indices ``0..k-1`` and the checkpoint ids travel as
``expert_ids``), the scores, the quantisation arguments and the shapes.
Tensors are torch tensors on the GPU.
"""
from __future__ import annotations

import importlib
import inspect
from typing import Any, Callable, Dict, Optional, Tuple

ENTRY_NAMES = ("build_executor", "create_executor", "MetalMoEExecutor", "Executor", "execute", "run")
RUNNER_NAMES = {"x", "inputs", "indices", "rhs_indices", "route"}
NATIVE_PATHS = (None, "hip", "custom-metal")


def load_target(spec: str):
    """``module:attribute``, or the first entry name a bare module defines."""
    module_name, separator, attribute = spec.partition(":")
    module = importlib.import_module(module_name)
    if separator:
        return getattr(module, attribute)
    for name in ENTRY_NAMES:
        if hasattr(module, name):
            return getattr(module, name)
    raise AttributeError(f"{spec} has no executor builder or runner attribute")


def load_custom_executor(spec: Optional[str]) -> Tuple[Any, Optional[str]]:
    """(target, None), or (None, reason) when nothing was asked for or it cannot load."""
    if not spec:
        return None, "not requested"
    try:
        return load_target(spec), None
    except (ImportError, ModuleNotFoundError, AttributeError, OSError) as exc:
        return None, f"{type(exc).__name__}: {exc}"


def invoke(fn: Callable[..., Any], values: Dict[str, Any]) -> Any:
    """Call ``fn`` with the context entries its signature names (all of them
    when it takes ``**kwargs``); a required name the context lacks raises."""
    try:
        signature = inspect.signature(fn)
    except (TypeError, ValueError):
        return fn(values["x"], values["packs"], values["indices"], values["group_size"], values["bits"],
                  values["mode"])
    params = list(signature.parameters.values())
    if any(p.kind == inspect.Parameter.VAR_KEYWORD for p in params):
        kwargs = dict(values)
    else:
        kwargs = {p.name: values[p.name] for p in params
                  if p.kind in (inspect.Parameter.POSITIONAL_OR_KEYWORD, inspect.Parameter.KEYWORD_ONLY)
                  and p.name in values}
    positional = []
    for p in params:
        if p.kind != inspect.Parameter.POSITIONAL_ONLY:
            continue
        if p.name not in values:
            if p.default is inspect.Parameter.empty:
                raise TypeError(f"custom executor needs unsupported argument {p.name!r}")
            continue
        positional.append(values[p.name])
    return fn(*positional, **kwargs)


def runner_from_target(target, context: Dict[str, Any]):
    """A runner from a module, builder, class or callable."""
    if inspect.ismodule(target):
        for name in ENTRY_NAMES[:4]:
            if hasattr(target, name):
                return runner_from_target(getattr(target, name), context)
        for name in ("execute", "run"):
            if hasattr(target, name):
                return getattr(target, name)
        raise TypeError("custom module has no executor entry point")
    if inspect.isclass(target):
        return invoke(target, context)
    for name in ("build_executor", "create_executor"):
        if hasattr(target, name):
            return invoke(getattr(target, name), context)
    if hasattr(target, "execute") or hasattr(target, "run"):
        return target
    if callable(target):
        if set(inspect.signature(target).parameters) & RUNNER_NAMES:
            return target
        return invoke(target, context)
    raise TypeError(f"custom target is not callable: {target!r}")


def _combine_per_slot(result, scores):
    if result.dim() == scores.dim() + 1:
        return (result.float() * scores.float()[..., None]).sum(dim=-2).to(result.dtype)
    return result


def run_custom(runner, context: Dict[str, Any]):
    """Run an executor object or function on the context."""
    if type(runner).__name__ in ("HipMoEExecutor", "MetalMoEExecutor"):
        x = context["x"]
        k = context["top_k"]
        scores = context["scores"].reshape(-1, k)
        result = runner.execute(x.reshape(-1, x.shape[-1]), context["routes"].reshape(-1, k),
                                context["packs"], scores=scores)
        return _combine_per_slot(result, scores)
    if hasattr(runner, "execute"):
        return invoke(runner.execute, context)
    if hasattr(runner, "run"):
        return invoke(runner.run, context)
    return invoke(runner, context)


def uses_native_path(runner) -> bool:
    """False when the runner reports that it fell back to a reference path."""
    return getattr(runner, "last_path", None) in NATIVE_PATHS


def normalise_output(output):
    if isinstance(output, dict):
        for key in ("output", "out", "y", "result"):
            if key in output:
                return output[key]
    if isinstance(output, (tuple, list)):
        if len(output) != 1:
            raise TypeError("custom executor must return one output array")
        return output[0]
    return output


def make_context(x, packs, routes, expert_ids, scores, *, hidden_size: int, top_k: int, group_size: int = 32,
                 bits: int = 4, mode: str = "affine", expert_outputs=None) -> Dict[str, Any]:
    """The reference's context aliases (bench_runtime_layer.py:383-409)."""
    return {
        "x": x, "inputs": x, "hidden_states": x,
        "packs": packs, "weights": packs, "expert_weights": packs, "projections": packs,
        "gate": packs["gate_proj"], "up": packs["up_proj"], "down": packs["down_proj"],
        "gate_proj": packs["gate_proj"], "up_proj": packs["up_proj"], "down_proj": packs["down_proj"],
        "indices": routes, "rhs_indices": routes, "expert_indices": routes,
        "route": expert_ids, "expert_ids": expert_ids,
        "scores": scores, "gating_scores": scores,
        "routes": routes, "route_indices": routes,
        "expert_outputs": expert_outputs, "expert_values": expert_outputs,
        "group_size": group_size, "bits": bits, "mode": mode, "activation": "swiglu",
        "expert_count": len(expert_ids), "hidden_size": hidden_size, "top_k": top_k,
    }


__all__ = ["ENTRY_NAMES", "invoke", "load_custom_executor", "load_target", "make_context", "normalise_output",
           "run_custom", "runner_from_target", "uses_native_path"]
