"""Adaptive top-k routing on the host (models/flashnext/adaptive_topk.py:76-235,
the rule at :44-51, configuration at :296-431).

At a threshold below 1.0 each row keeps, in descending gate order, the fewest
of its top-k experts whose share of the row's top-k gate mass reaches the
threshold, and at least the minimum keep.  Two optional steps change which
slots stay:
  * cache-aware swap: a kept expert that is not resident trades places with a
    resident dropped one whose gate is within ``epsilon`` below it, cheapest
    kept expert first, each dropped expert serving once (``swap_row``); only
    for calls of at most ``max_rows`` rows;
  * resident masks: per layer, a dropped slot whose expert is in the layer's
    resident set stays enabled.
Dropped slots then take the row's first expert with score 0, and the scores
renormalise over the kept mass: normalizer = topk_mass + blend * (kept_mass -
topk_mass), every step rounded in bf16.

The reference syncs the scores to the host for this and computes it in
Python; so does ``MoELayer`` here: a router-only call writes the routes and
the gates, ``plan`` rewrites the routes, and an experts-only call uses them.
The default threshold 1.0 leaves routing untouched and never comes here.
"""
from __future__ import annotations

from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

_threshold = 1.0
_layer_thresholds: Dict[int, float] = {}
_min_keep = 1
_layer_min_keeps: Dict[int, int] = {}
_swap_resident: Optional[Callable[[int, int], bool]] = None
_swap_epsilon = 0.02
_swap_max_rows = 4
_resident_experts: Dict[int, set] = {}
_observer: Optional[Callable] = None
_observer_max_rows: Optional[int] = None
_last_keeps: Dict[int, Tuple[int, ...]] = {}
_keep_sum = 0
_keep_count = 0


def set_threshold(value: float) -> None:
    global _threshold
    _threshold = float(value)


def set_layer_thresholds(values=None) -> None:
    _layer_thresholds.clear()
    if values:
        _layer_thresholds.update({int(k): float(v) for k, v in values.items()})


def set_min_keep(value: int, layer_values=None) -> None:
    global _min_keep
    _min_keep = max(1, int(value))
    _layer_min_keeps.clear()
    if layer_values:
        _layer_min_keeps.update({int(k): max(1, int(v)) for k, v in layer_values.items()})


def set_swap_resident(predicate=None, epsilon: Optional[float] = None, max_rows: Optional[int] = None) -> None:
    """``predicate(layer, expert) -> bool`` reports residency; None restores exact routing."""
    global _swap_resident, _swap_epsilon, _swap_max_rows
    _swap_resident = predicate
    if epsilon is not None:
        _swap_epsilon = float(epsilon)
    if max_rows is not None:
        _swap_max_rows = int(max_rows)


def set_resident_experts(values=None) -> None:
    _resident_experts.clear()
    if values:
        _resident_experts.update({int(layer): {int(e) for e in experts} for layer, experts in values.items()})


def set_route_observer(observer=None, max_rows: Optional[int] = None) -> None:
    """``observer(layer, expert_rows, weight_rows, keeps)`` sees each call's
    routing before the swap, for at most ``max_rows`` rows (None: all)."""
    global _observer, _observer_max_rows
    _observer = observer
    _observer_max_rows = None if max_rows is None else int(max_rows)


def threshold_for(layer: Optional[int]) -> float:
    return _layer_thresholds.get(layer, _threshold)


def observing() -> bool:
    """A route observer is set: it sees every call's routes, at threshold 1.0
    too (adaptive_topk.py:240-253)."""
    return _observer is not None


def observe_exact(layer: Optional[int], inds: np.ndarray, gates: np.ndarray) -> None:
    """Threshold 1.0 with an observer: every row keeps all k slots."""
    if _observer is None or layer is None:
        return
    rows, k = np.asarray(inds).shape
    n = rows if _observer_max_rows is None else min(rows, _observer_max_rows)
    _observer(layer, np.asarray(inds)[:n].tolist(), np.asarray(gates)[:n].tolist(), [k] * n)


def record_exact(layer: Optional[int], rows: int, k: int) -> None:
    """A call at threshold 1.0 keeps all k slots of every row; the keep
    statistics count it (adaptive_topk.py:236-239)."""
    global _keep_sum, _keep_count
    if layer is None:
        return
    _last_keeps[layer] = (k,) * rows
    _keep_sum += rows * k
    _keep_count += rows


def last_keeps() -> Dict[int, Tuple[int, ...]]:
    return dict(_last_keeps)


def reset_keep_stats() -> None:
    global _keep_sum, _keep_count
    _keep_sum = 0
    _keep_count = 0


def mean_keeps() -> float:
    return _keep_sum / _keep_count if _keep_count else 0.0


def keep_for_mass(weights: Sequence[float], threshold: float) -> int:
    """Slots kept: the first position (1-based) at which the running share of
    the row's total reaches the threshold; all of them if it never does."""
    total = float(sum(weights))
    share = 0.0
    for position, weight in enumerate(weights):
        share += weight / total
        if share >= threshold:
            return position + 1
    return len(weights)


def swap_row(experts: List[int], weights: List[float], keep: int, resident: Callable[[int], bool],
             epsilon: float) -> Tuple[List[int], List[float]]:
    """Kept experts that are not resident exchange places with resident dropped
    ones whose weight is at most ``epsilon`` lower: the lightest kept expert
    first, each taking the heaviest qualifying dropped expert not yet taken.
    Returns the input lists themselves when nothing moves."""
    spare = [p for p in range(keep, len(experts)) if resident(experts[p])]
    cold = [p for p in range(keep) if not resident(experts[p])]
    if not spare or not cold:
        return experts, weights
    experts, weights = list(experts), list(weights)
    taken = set()
    for p in sorted(cold, key=lambda q: weights[q]):
        best = None
        for c in spare:
            if c not in taken and weights[p] - weights[c] <= epsilon and (best is None or weights[c] > weights[best]):
                best = c
        if best is None:
            continue
        taken.add(best)
        experts[p], experts[best] = experts[best], experts[p]
        weights[p], weights[best] = weights[best], weights[p]
    return experts, weights


def _bf16(values) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(values, dtype=np.float32)))


def plan(layer: Optional[int], inds: np.ndarray, gates: np.ndarray, blend: float = 1.0,
         bf16: bool = True) -> Tuple[np.ndarray, np.ndarray, List[int], int]:
    """Routes of one call at the layer's threshold.

    ``inds`` [rows, k] and ``gates`` [rows, k]: the selected experts and their
    softmax gates.  Returns (experts [rows, k] int32, renormalised scores
    [rows, k] as float32 with every step rounded in bf16 when ``bf16``, the
    enabled slots per row, the width: one past the last enabled slot of any
    row).  Slots past a row's keep that no resident mask enables take the
    row's first expert and score 0.  All k slots are returned: the reference
    trims them to the width, and the slots beyond it add nothing to the
    combine."""
    global _keep_sum, _keep_count
    threshold = threshold_for(layer)
    inds = np.asarray(inds, dtype=np.int64)
    gates = np.asarray(gates, dtype=np.float32)
    rows, k = inds.shape
    order = np.argsort(-gates, axis=1, kind="stable")
    inds = np.take_along_axis(inds, order, axis=1)
    gates = np.take_along_axis(gates, order, axis=1)
    minimum = max(1, min(k, _layer_min_keeps.get(layer, _min_keep)))
    expert_rows = inds.tolist()
    weight_rows = gates.tolist()
    keeps = [max(minimum, keep_for_mass(w, threshold)) for w in weight_rows]
    if _observer is not None and layer is not None:
        n = rows if _observer_max_rows is None else min(rows, _observer_max_rows)
        _observer(layer, expert_rows[:n], weight_rows[:n], keeps[:n])
    if _swap_resident is not None and layer is not None and rows <= _swap_max_rows:
        swapped = [swap_row(e, w, keep, lambda x: _swap_resident(layer, x), _swap_epsilon)
                   for e, w, keep in zip(expert_rows, weight_rows, keeps)]
        expert_rows = [e for e, _ in swapped]
        weight_rows = [w for _, w in swapped]
    resident = _resident_experts.get(layer)
    masks = [[p < keep or (resident is not None and e in resident) for p, e in enumerate(row)]
             for row, keep in zip(expert_rows, keeps)]
    effective = [sum(m) for m in masks]
    width = max(p + 1 for mask in masks for p, on in enumerate(mask) if on)
    if layer is not None:
        _last_keeps[layer] = tuple(effective)
        _keep_sum += sum(effective)
        _keep_count += len(effective)
    out_inds = np.array([[e if m else row[0] for e, m in zip(row, mask)] for row, mask in zip(expert_rows, masks)],
                        dtype=np.int32).reshape(rows, k)
    kept = np.array([[w if m else 0.0 for w, m in zip(row, mask)] for row, mask in zip(weight_rows, masks)],
                    dtype=np.float32).reshape(rows, k)
    rnd = _bf16 if bf16 else (lambda v: np.asarray(v, dtype=np.float32))
    topk_mass = rnd(gates.astype(np.float64).sum(axis=1, keepdims=True))
    kept_mass = rnd(kept.astype(np.float64).sum(axis=1, keepdims=True))
    diff = rnd(kept_mass - topk_mass)
    # blend is a scalar of the scores' type (compiled.py:111)
    normalizer = rnd(topk_mass + rnd(rnd(np.float32(blend)) * diff))
    scores = rnd(kept.astype(np.float64) / normalizer.astype(np.float64))
    return out_inds, scores, effective, width
