"""StepGraph host-side refusals (no GPU): a graph records exact top-k
routing, so it cannot stand in for layers whose calls adapt their routing
(adaptive_topk.py:76-262) or report it to a route observer (:240-253)."""
from types import SimpleNamespace

import pytest

from veymoe import adaptive
from veymoe.graph import StepGraph


@pytest.fixture(autouse=True)
def _reset():
    yield
    adaptive.set_threshold(1.0)
    adaptive.set_layer_thresholds()
    adaptive.set_route_observer()


def _layers(n):
    return [SimpleNamespace(_flashnext_layer_id=i) for i in range(n)]


def test_build_refuses_an_adaptive_layer():
    adaptive.set_layer_thresholds({2: 0.7})
    with pytest.raises(RuntimeError, match="layer 2"):
        StepGraph(_layers(3))


def test_build_refuses_a_global_threshold_below_one():
    adaptive.set_threshold(0.9)
    with pytest.raises(RuntimeError, match="threshold"):
        StepGraph(_layers(1))


def test_build_refuses_a_route_observer():
    adaptive.set_route_observer(lambda *a: None)
    with pytest.raises(RuntimeError, match="observer"):
        StepGraph(_layers(2))


def test_threshold_of_another_layer_is_no_reason_to_refuse():
    adaptive.set_layer_thresholds({5: 0.5})
    with pytest.raises(AttributeError):   # gets past the routing check to the layer checks
        StepGraph(_layers(2))
