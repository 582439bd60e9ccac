"""CPU oracle of the routed-expert MoE layer.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports, calls or
links this module; only ``tests/``, ``__graft_entry__.smoke()`` and the CPU
baseline leg of ``bench.py`` use it, and only as the checker.

It restates, in NumPy with float64 accumulation, the semantics of the
reference's MLX quantized MoE path (joyboyreturns/Veystrix-Core):

  * Q4/G32 affine projection: ``_numpy_projection``
    (models/flashnext/metal_runtime.py:997-1029), the float64-accumulating
    NumPy reference the reference keeps for its executor:
    ``y[o] = sum_g s[o,g] * sum_{k in g} x_k q[o,k] + b[o,g] * sum_{k in g} x_k``
    with nibble k at bits ``4*(k&7)`` of word ``k>>3`` (:1022).
  * Router: ``_router_plain`` + ``_renorm_plain`` (models/flashnext/compiled.py:61-71,
    adaptive_topk.py:59-65,257-262): bf16 Linear, precise softmax (fp32 inside,
    bf16 out), top-k, ``scores / (topk_mass + blend*(selected_mass-topk_mass))``.
  * SwiGLU: the bf16 op-by-op sigmoid sequence of the fused up kernel
    (metal_runtime.py:267-285): |g|, exp, 1+e, 1/(1+e), select/1-x, g*sig, *u,
    each step rounded to bf16.
  * Fused down + combine (metal_runtime.py:291-336):
    ``combined = sum_j fp32(bf16(down_j)) * fp32(score_j)`` in fp32 in slot
    order (contraction off), ``y = bf16(fp32(bf16(combined)) + fp32(shared_y))``
    or with shared parts ``bf16(fp32(shared)*fp32(shared_gate))``.
  * Generic combine of the prefill path (adaptive_topk.py:275-278,
    compiled.py:77-79): ``(y*scores[...,None]).sum(-2) + shared_gate*shared`` in
    bf16 element ops.
  * ``weighted_combine`` (metal_runtime.py:145-191).

Two modes:
  ``"bf16"``  rounds to bf16 at the reference's rounding points listed above;
  ``"f32"``   no intermediate rounding (the "fp32 accumulation oracle"); the
              weights, scales, biases and router weight are still bf16 data.

Pinning (tests/test_oracle.py): the weighted_combine known-answer test of
test_metal_runtime.py:222-263; the bf16 bit round trip of
test_swiglu_contract.py:21-23; an exhaustive 65,536-pattern SwiGLU scan against
float64 mathematics; brute-force pure-Python loops (oracle/ref_loops.py, a
restatement of ``_numpy_projection``'s loop nest) on tiny shapes; closed-form
projection cases (zero nibbles, zero scale, all-15 nibbles, one-hot inputs);
softmax/top-k against a full sort with the stated tie rule.

Tie rule for top-k (MLX ``argpartition`` leaves it unspecified, so it is
"parity unpinned" against MLX itself): gates descending, then expert index
ascending; the selection is returned in that order.
"""
from __future__ import annotations

import numpy as np

GROUP_SIZE = 32
BITS = 4

# --------------------------------------------------------------------------
# bfloat16 as uint16 bit patterns (models/flashnext/store.py:26-41 carries BF16
# as "<u2" and reinterprets it).


def bf16_bits_to_f32(bits) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(values) -> np.ndarray:
    """Round float32 to the nearest bf16, ties to even; NaN stays NaN."""
    values = np.asarray(values, dtype=np.float32)
    u = values.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(values)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16r(values) -> np.ndarray:
    """Round to bf16 and return the value as float32.

    float64 input is first rounded to float32, as a float32 kernel that stores
    a bf16 would do."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(values).astype(np.float32)))


def _round(values, mode):
    if mode == "bf16":
        return bf16r(values)
    return np.asarray(values).astype(np.float32)


# --------------------------------------------------------------------------
# Q4/G32 affine projection (metal_runtime.py:997-1029).


def unpack_nibbles(packed) -> np.ndarray:
    """uint32 [..., n/8] -> uint8 [..., n]; nibble k = (w[k>>3] >> 4*(k&7)) & 15."""
    packed = np.asarray(packed, dtype=np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    nib = (packed[..., :, None] >> shifts) & np.uint32(15)
    return nib.reshape(*packed.shape[:-1], packed.shape[-1] * 8).astype(np.uint8)


def dequantize(packed, scales_bits, biases_bits, group_size=GROUP_SIZE) -> np.ndarray:
    """Dense float64 weights ``scale*q + bias`` of one or more experts."""
    q = unpack_nibbles(packed).astype(np.float64)
    s = bf16_bits_to_f32(scales_bits).astype(np.float64)
    b = bf16_bits_to_f32(biases_bits).astype(np.float64)
    shape = q.shape
    groups = shape[-1] // group_size
    q = q.reshape(*shape[:-1], groups, group_size)
    return (q * s[..., None] + b[..., None]).reshape(shape)


def q4_project(x, packed, scales_bits, biases_bits, group_size=GROUP_SIZE) -> np.ndarray:
    """Project rows ``x [n, in]`` through one expert ``[out, in/8]``.

    Same grouping as ``_numpy_projection``: per group, ``s*sum(x*q) + b*sum(x)``,
    accumulated in float64.  Returns float64 ``[n, out]``."""
    x = np.asarray(x, dtype=np.float64)
    q = unpack_nibbles(packed).astype(np.float64)
    out_width, in_width = q.shape
    if x.shape[-1] != in_width or in_width % group_size:
        raise ValueError("input width does not match the packed projection")
    groups = in_width // group_size
    qg = q.reshape(out_width, groups, group_size)
    xg = x.reshape(x.shape[0], groups, group_size)
    qsum = np.einsum("ngk,ogk->nog", xg, qg)            # sum x*q per group
    xsum = xg.sum(axis=-1)                              # sum x per group
    s = bf16_bits_to_f32(scales_bits).astype(np.float64)
    b = bf16_bits_to_f32(biases_bits).astype(np.float64)
    return (qsum * s[None] + xsum[:, None, :] * b[None]).sum(axis=-1)


def qmm_project(x, packed, scales_bits, biases_bits, group_size=GROUP_SIZE, weight_mode="bf16") -> np.ndarray:
    """Matrix form of the projection used for more than 8 rows.

    The reference runs those rows through ``mx.gather_qmm`` (expert_cache.py:
    806-829; MLX 0.32.2, uv.lock:655), whose matrix kernels dequantise a tile
    of weights into threadgroup memory in the activation type before the
    multiply.  Restated: ``w = round(scale*q + bias)`` once per weight (bf16
    mode), then ``x @ w.T`` accumulated in float64.  Returns float64 [n, out]."""
    w = _round(dequantize(packed, scales_bits, biases_bits, group_size), weight_mode)
    return np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T


# --------------------------------------------------------------------------
# Activations.


def sigmoid(g, mode):
    """MLX's stable sigmoid sequence (metal_runtime.py:277-283), rounded per step in bf16 mode.

    exp is evaluated in float64 and rounded to float32 first (a correctly
    rounded float32 exp) before the bf16 rounding."""
    g = np.asarray(g, dtype=np.float32)
    mag = np.abs(g)
    with np.errstate(over="ignore"):
        e = _round(np.exp(mag.astype(np.float64)).astype(np.float32), mode)
    den = _round(np.float32(1) + e, mode)
    with np.errstate(divide="ignore"):
        small = _round(np.float32(1) / den, mode)
    big = _round(np.float32(1) - small, mode)
    return np.where(g < 0, small, big).astype(np.float32)


def silu(g, mode):
    g = np.asarray(g, dtype=np.float32)
    return _round(g * sigmoid(g, mode), mode)


def swiglu(gate, up, mode):
    """``silu(gate) * up`` (mlx-vlm swiglu; metal_runtime.py:284)."""
    return _round(silu(gate, mode) * np.asarray(up, dtype=np.float32), mode)


# --------------------------------------------------------------------------
# Router (compiled.py:61-71, adaptive_topk.py:59-65,257-262).


def router_logits(x, weight_bits, mode, logit_bias=None):
    """bf16 Linear without bias: float64 accumulation, output rounded."""
    w = bf16_bits_to_f32(weight_bits).astype(np.float64)
    logits = np.asarray(x, dtype=np.float64) @ w.T
    if logit_bias is not None:
        logits = logits + np.asarray(logit_bias, dtype=np.float32).astype(np.float64)
    return _round(logits, mode)


def softmax(logits, mode):
    """Precise softmax: computed in float64 here, float32 in the reference,
    output rounded to the activation type."""
    z = np.asarray(logits, dtype=np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return _round(e / e.sum(axis=-1, keepdims=True), mode)


def topk(gates, k):
    """Indices of the k largest gates per row, by (gate desc, index asc)."""
    gates = np.asarray(gates, dtype=np.float32)
    rows, experts = gates.shape
    idx = np.arange(experts)
    out = np.empty((rows, k), dtype=np.int32)
    for r in range(rows):
        order = np.lexsort((idx, -gates[r].astype(np.float64)))
        out[r] = order[:k]
    return out


def renorm(scores, mode, blend=1.0, topk_mass=None):
    """``scores / (topk_mass + blend*(selected_mass - topk_mass))``.

    With the full top-k selected, selected_mass == topk_mass, so the result is
    ``scores / sum(scores)``; every step is rounded in bf16 mode, blend
    included: compiled.py:111 makes it ``mx.array(blend, scores.dtype)``, and
    the plain form (adaptive_topk.py:260-261) multiplies a bf16 array by a
    Python float, which MLX casts to the array's type."""
    scores = np.asarray(scores, dtype=np.float32)
    selected = _round(scores.astype(np.float64).sum(axis=-1, keepdims=True), mode)
    mass = selected if topk_mass is None else topk_mass
    diff = _round(selected - mass, mode)
    normalizer = _round(mass + _round(_round(np.float32(blend), mode) * diff, mode), mode)
    return _round(scores.astype(np.float64) / normalizer.astype(np.float64), mode)


def route(x, router_bits, k, mode, logit_bias=None, blend=1.0):
    """Returns (inds [T,k] int32, renormalised scores [T,k], gates [T,E])."""
    logits = router_logits(x, router_bits, mode, logit_bias)
    gates = softmax(logits, mode)
    inds = topk(gates, k)
    scores = np.take_along_axis(gates, inds, axis=-1)
    return inds, renorm(scores, mode, blend), gates


def keep_for_mass(weights, threshold):
    """adaptive_topk.py:44-51: the first 1-based position at which the running
    sum of weight / total reaches ``threshold``; len(weights) otherwise."""
    total = sum(weights)
    running = 0.0
    for i in range(len(weights)):
        running += weights[i] / total
        if running >= threshold:
            return i + 1
    return len(weights)


def swap_row(experts, weights, keep, resident, epsilon):
    """adaptive_topk.py:397-431: each cold kept slot, lightest first, swaps
    with the heaviest resident dropped slot within ``epsilon`` below it that
    no earlier slot took."""
    spare = [i for i in range(keep, len(experts)) if resident(experts[i])]
    cold = [i for i in range(keep) if not resident(experts[i])]
    if not spare or not cold:
        return list(experts), list(weights)
    experts, weights = list(experts), list(weights)
    used = []
    for i in sorted(cold, key=lambda j: weights[j]):
        choice = -1
        for j in spare:
            if j in used or weights[i] - weights[j] > epsilon:
                continue
            if choice < 0 or weights[j] > weights[choice]:
                choice = j
        if choice >= 0:
            used.append(choice)
            experts[i], experts[choice] = experts[choice], experts[i]
            weights[i], weights[choice] = weights[choice], weights[i]
    return experts, weights


def adaptive_routes(inds, gates_k, threshold, mode, min_keep=1, blend=1.0, resident=None, swap=None,
                    epsilon=0.02):
    """The adaptive top-k of adaptive_topk.py:76-235 and the renorm of :257-262.

    ``inds``/``gates_k`` [T, k]: the top-k experts and their (rounded) gates.
    Rows are ordered by gate descending; keep = max(min(k, min_keep), the mass
    rule); ``swap(expert) -> bool`` enables the cache-aware swap; ``resident``
    (a set) keeps dropped slots of resident experts.  Disabled slots take the
    row's first expert and score 0; the result is cut to the widest row.
    Returns (inds [T, width], scores [T, width], keeps)."""
    inds = np.asarray(inds)
    gates_k = np.asarray(gates_k, dtype=np.float32)
    t, k = inds.shape
    expert_rows, weight_rows, keeps = [], [], []
    floor = max(1, min(k, min_keep))
    for r in range(t):
        order = sorted(range(k), key=lambda j: -float(gates_k[r, j]))
        e = [int(inds[r, j]) for j in order]
        w = [float(gates_k[r, j]) for j in order]
        keep = max(floor, keep_for_mass(w, threshold))
        if swap is not None:
            e, w = swap_row(e, w, keep, swap, epsilon)
        expert_rows.append(e)
        weight_rows.append(w)
        keeps.append(keep)
    enabled = [[j < keeps[r] or (resident is not None and expert_rows[r][j] in resident) for j in range(k)]
               for r in range(t)]
    width = max(j + 1 for r in range(t) for j in range(k) if enabled[r][j])
    out_inds = np.array([[expert_rows[r][j] if enabled[r][j] else expert_rows[r][0] for j in range(width)]
                         for r in range(t)], dtype=np.int32)
    kept = np.array([[weight_rows[r][j] if enabled[r][j] else 0.0 for j in range(width)] for r in range(t)],
                    dtype=np.float32)
    topk_mass = _round(gates_k.astype(np.float64).sum(axis=-1, keepdims=True), mode)
    return out_inds, renorm(kept, mode, blend, topk_mass), [sum(row) for row in enabled]


# --------------------------------------------------------------------------
# Experts and combine.


def expert_forward(x, gate, up, down, mode, group_size=GROUP_SIZE, qmm=False):
    """One expert on rows x: (gate_out, up_out, act, down_out), each rounded.
    ``qmm`` selects the matrix form (weights rounded to the activation type)."""
    if qmm:
        project = lambda rows, proj: qmm_project(rows, *proj, group_size=group_size, weight_mode=mode)  # noqa: E731
    else:
        project = lambda rows, proj: q4_project(rows, *proj, group_size=group_size)  # noqa: E731
    g = _round(project(x, gate), mode)
    u = _round(project(x, up), mode)
    a = swiglu(g, u, mode)
    d = _round(project(a, down), mode)
    return g, u, a, d


def _take_expert(proj, e):
    # works for dense [E, ...] arrays and for lazily generated expert banks
    return tuple(np.asarray(part[int(e)]) for part in proj)


def weighted_combine(expert_outputs, routes, scores):
    """metal_runtime.py:145-191: normal form ``outputs[..., slots, hidden]``
    or, when outputs hold every expert, selection by ``routes`` first."""
    outputs = np.asarray(expert_outputs)
    routes = np.asarray(routes)
    scores = np.asarray(scores)
    if outputs.ndim < 2 or routes.ndim == 0:
        raise ValueError("expert_outputs and routes need at least one dimension")
    if scores.shape != routes.shape:
        raise ValueError("routes and scores must have identical shapes")
    slots = routes.shape[-1]
    if outputs.shape[:-1] == routes.shape:
        selected = outputs
    elif outputs.ndim == routes.ndim + 1 and outputs.shape[-2] >= slots:
        if routes.size and (routes.min() < 0 or routes.max() >= outputs.shape[-2]):
            raise ValueError("routes contain an expert outside expert_outputs")
        selected = np.take_along_axis(outputs, np.expand_dims(routes, -1), axis=-2)
    else:
        raise ValueError(
            f"expert_outputs shape {outputs.shape} does not match routes {routes.shape}")
    return (selected * scores[..., None]).sum(axis=-2)


def fused_combine(down_out, scores, mode, shared_y=None, shared=None, shared_gate=None):
    """Fused down + combine epilogue (metal_runtime.py:299-335).

    down_out [T,k,H] already rounded; scores [T,k]; combined in float32 in
    slot order with the product rounded before the add (contract off)."""
    down_out = np.asarray(down_out, dtype=np.float32)
    scores = np.asarray(scores, dtype=np.float32)
    tokens, slots, hidden = down_out.shape
    combined = np.zeros((tokens, hidden), dtype=np.float32)
    for j in range(slots):
        combined = (combined + (down_out[:, j, :] * scores[:, j:j + 1]).astype(np.float32)).astype(np.float32)
    routed = _round(combined, mode)
    if shared_y is not None:
        return _round(routed + np.asarray(shared_y, dtype=np.float32), mode)
    if shared is not None:
        comp = _round(np.asarray(shared, dtype=np.float32)
                      * np.asarray(shared_gate, dtype=np.float32).reshape(tokens, 1), mode)
        return _round(routed + comp, mode)
    return routed


def generic_combine(down_out, scores, mode, shared_term=None):
    """adaptive_topk.py:277-278: ``(y*scores[...,None]).sum(-2) + shared``.

    Element products rounded, the slot sum accumulated in float32 and rounded
    once, then the shared term added and rounded."""
    down_out = np.asarray(down_out, dtype=np.float32)
    scores = np.asarray(scores, dtype=np.float32)
    prod = _round(down_out * scores[..., None], mode)
    acc = np.zeros(prod.shape[:1] + prod.shape[2:], dtype=np.float32)
    for j in range(prod.shape[1]):
        acc = (acc + prod[:, j, :]).astype(np.float32)
    y = _round(acc, mode)
    if shared_term is not None:
        y = _round(y + np.asarray(shared_term, dtype=np.float32), mode)
    return y


def execute(x, routes, projections, mode, scores=None, shared_y=None, shared=None,
            shared_gate=None, group_size=GROUP_SIZE, activation=None, qmm=False):
    """MetalMoEExecutor.execute semantics on dense projections.

    routes [T,k] are expert indices into the dense arrays.  Returns
    (gate_out, up_out, act, down_out [T,k,H], output) where ``output`` is the
    fused combine when scores are given, else ``down_out``."""
    x = np.asarray(x, dtype=np.float32)
    routes = np.asarray(routes)
    tokens, slots = routes.shape
    gate, up, down = (projections[name] for name in ("gate_proj", "up_proj", "down_proj"))
    inter = np.asarray(gate[0][int(routes[0, 0])]).shape[0]
    hidden = x.shape[1]
    g_out = np.zeros((tokens, slots, inter), np.float32)
    u_out = np.zeros_like(g_out)
    act = np.zeros_like(g_out)
    d_out = np.zeros((tokens, slots, hidden), np.float32)
    for t in range(tokens):
        for j in range(slots):
            e = int(routes[t, j])
            if activation is None:
                g, u, a, d = expert_forward(x[t:t + 1], _take_expert(gate, e), _take_expert(up, e),
                                            _take_expert(down, e), mode, group_size, qmm)
                g_out[t, j], u_out[t, j], act[t, j] = g[0], u[0], a[0]
            else:
                a = np.asarray(activation, np.float32)[t, j][None]
                act[t, j] = a[0]
                d = _round(q4_project(a, *_take_expert(down, e), group_size=group_size), mode)
            d_out[t, j] = d[0]
    if scores is None:
        return g_out, u_out, act, d_out, d_out
    out = fused_combine(d_out, scores, mode, shared_y, shared, shared_gate)
    return g_out, u_out, act, d_out, out


# --------------------------------------------------------------------------
# The whole layer (adaptive_topk._moe_call at threshold 1.0).


def shared_expert(x, layer, mode, group_size=GROUP_SIZE, qmm=False):
    """(shared [T,H], shared_gate [T,1]) for the layer's shared expert, or (None, None)."""
    if layer.get("shared_gate_proj") is None:
        return None, None
    sg = _take_expert(layer["shared_gate_proj"], 0)
    su = _take_expert(layer["shared_up_proj"], 0)
    sd = _take_expert(layer["shared_down_proj"], 0)
    _, _, _, shared = expert_forward(x, sg, su, sd, mode, group_size, qmm)
    seg = _take_expert(layer["shared_expert_gate"], 0)
    logit = _round(q4_project(x, *seg, group_size=group_size), mode)
    return shared, sigmoid(logit, mode)


def decode_combine(layer_id):
    """The combine a decode call (rows <= 8) of layer ``layer_id`` takes.

    ``StreamingSwitchGLU.metal_combines_scores`` is False for layer 0
    (expert_cache.py:1434-1443), so the reference's layer 0 decodes through
    the generic combine of adaptive_topk.py:275-278 and every other layer
    through the fused one (:289-293)."""
    return "generic" if layer_id == 0 else "fused"


def moe_layer(x, layer, mode, path="decode", group_size=GROUP_SIZE, qmm=None, combine=None, adaptive=None):
    """One MoE layer.  ``layer`` holds numpy arrays (see veymoe.synth).

    path "decode": rows <= 8, vector-form projections, and the combine of
    ``decode_combine(layer["layer_id"])``: fused shared_y combine
    (adaptive_topk.py:289-293), or the generic one for layer 0;
    path "prefill": generic combine (adaptive_topk.py:275-278), matrix-form
    projections (gather_qmm, weights rounded) unless ``qmm`` says otherwise.
    ``combine`` ("fused"/"generic") overrides the rule.  ``adaptive``: keyword
    arguments of ``adaptive_routes`` (threshold, min_keep, ...) applied to the
    top-k before the experts.
    Returns dict(inds, scores, gates, output, down, shared, shared_gate)."""
    x = np.asarray(x, dtype=np.float32)
    if qmm is None:
        qmm = path != "decode"
    if combine is None:
        combine = decode_combine(layer.get("layer_id")) if path == "decode" else "generic"
    k = int(layer["top_k"])
    inds, scores, gates = route(x, layer["router"], k, mode, layer.get("router_bias"))
    if adaptive is not None:
        inds, scores, _ = adaptive_routes(inds, np.take_along_axis(gates, inds, axis=-1), mode=mode, **adaptive)
        k = inds.shape[1]
    shared, shared_gate = shared_expert(x, layer, mode, group_size, qmm)
    projections = {name: layer[name] for name in ("gate_proj", "up_proj", "down_proj")}
    tokens = x.shape[0]
    hidden = x.shape[1]
    down = np.zeros((tokens, k, hidden), np.float32)
    for e in np.unique(inds):
        rows, cols = np.nonzero(inds == e)
        _, _, _, d = expert_forward(x[rows], _take_expert(projections["gate_proj"], e),
                                    _take_expert(projections["up_proj"], e),
                                    _take_expert(projections["down_proj"], e), mode, group_size, qmm)
        down[rows, cols] = d
    shared_y = None
    if shared is not None:
        shared_y = _round(shared_gate * shared, mode)
    if combine == "fused":
        out = fused_combine(down, scores, mode, shared_y=shared_y)
    else:
        out = generic_combine(down, scores, mode, shared_y)
    return dict(inds=inds, scores=scores, gates=gates, output=out, down=down,
                shared=shared, shared_gate=shared_gate)


def max_abs_rel(actual, expected) -> float:
    """max |actual - expected| / max |expected| (0 when both are zero)."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    scale = float(np.abs(expected).max()) if expected.size else 0.0
    err = float(np.abs(actual - expected).max()) if expected.size else 0.0
    if scale == 0.0:
        return err
    return err / scale
