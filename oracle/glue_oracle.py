"""CPU oracle of the decoder glue around the MoE call.

TEST INFRASTRUCTURE ONLY (see oracle/moe_oracle.py): the product never
imports this module.

Each decoder layer of the reference runs its MoE branch inside a
hyper-connection: the hidden state holds ``hc`` streams of ``H`` values; the
branch input is a mix of the normalised streams, and the branch output is
injected back into every stream with a per-stream weight.

* ``rms_norm``   patch_rmsnorm.py:108-135 (``_rms_norm``): cast to float32,
  mean of squares over the whole row or over groups of ``group_size``
  (:111-117), ``y * rsqrt(mean + eps)``, times the float32 gain (the weight
  itself for one-centered checkpoints, ``1 + weight`` otherwise, :62-66),
  cast back.  float32 steps; the mean is summed in float64 and rounded to
  float32 (the reference's reduction order is not visible).
* ``hyper_mix``  qwen4_verifier.py:20-33 (``_hyper``): ``normed =
  hc_norm(hidden)``; ``mix = sigmoid(W_up . silu(W_down . normed / hc))``;
  ``mixed = mean over streams of mix * normed``; injection weights
  ``2 * sigmoid(W_inj . normed / hc)``.  Every op rounds to bf16 as MLX's
  bf16 arrays do; the quantized linears are the vector form (q4_project);
  sigmoid/silu are moe_oracle's restatement of MLX's sequence.  The stream
  mean is MLX's ``sum * (1/N)`` in the array dtype, the sum accumulated in
  float32 in stream order.
* ``inject``     compile_glue.py:32-35 (``_inject``): ``hidden +
  (branch[..., None, :] * weights[..., None]).reshape(hidden.shape)``, each op
  rounded.
"""
from __future__ import annotations

import numpy as np

from . import moe_oracle as mo


def _r(values, mode):
    return mo.bf16r(values) if mode == "bf16" else np.asarray(values, dtype=np.float32)


def rms_norm(x, weight, eps, group_size=0, one_centered=True, mode="bf16"):
    """x [..., n] (values of the activation dtype), weight [n] -> [..., n]."""
    x = np.asarray(x, dtype=np.float32)
    n = x.shape[-1]
    gs = n if not group_size else int(group_size)
    if n % gs:
        raise ValueError("group_size must divide the row")
    y = x.reshape(*x.shape[:-1], n // gs, gs)
    w = np.asarray(weight, dtype=np.float32).reshape(n // gs, gs)
    gain = w if one_centered else (np.float32(1) + w).astype(np.float32)
    mean = (np.square(y.astype(np.float64)).sum(axis=-1, keepdims=True) / gs).astype(np.float32)
    inv = (1.0 / np.sqrt((mean + np.float32(eps)).astype(np.float32).astype(np.float64))).astype(np.float32)
    y = (y * inv).astype(np.float32)
    y = (y * gain).astype(np.float32)
    return _r(y.reshape(x.shape), mode)


def linear(x, proj, mode):
    """A Q4/G32 quantized Linear (weight [out, in/8], scales, biases) on rows x."""
    w, s, b = proj
    return _r(mo.q4_project(np.asarray(x, dtype=np.float32), w, s, b), mode)


def hyper_mix(hidden, norm_weight, down, up, inj, hc, eps, group_size=0, one_centered=True, mode="bf16"):
    """(mixed [T, H], weights [T, hc], normed [T, hc*H]) of hidden [T, hc*H]."""
    hidden = np.asarray(hidden, dtype=np.float32)
    T, n = hidden.shape
    H = n // hc
    normed = rms_norm(hidden, norm_weight, eps, group_size, one_centered, mode)
    a = _r(linear(normed, down, mode) / np.float32(hc), mode)
    d = mo.silu(a, mode)
    mix = mo.sigmoid(linear(d, up, mode), mode)
    prod = _r(mix.reshape(T, hc, H) * normed.reshape(T, hc, H), mode)
    total = np.zeros((T, H), dtype=np.float32)
    for j in range(hc):
        total = (total + prod[:, j]).astype(np.float32)
    mixed = _r(_r(total, mode) * _r(np.float32(1.0 / hc), mode), mode)
    g = _r(linear(normed, inj, mode) / np.float32(hc), mode)
    weights = _r(np.float32(2) * mo.sigmoid(g, mode), mode)
    return mixed, weights, normed


def inject(hidden, branch, weights, mode="bf16"):
    """hidden [T, hc*H], branch [T, H], weights [T, hc] -> [T, hc*H]."""
    hidden = np.asarray(hidden, dtype=np.float32)
    branch = np.asarray(branch, dtype=np.float32)
    weights = np.asarray(weights, dtype=np.float32)
    T, hc = weights.shape
    injection = _r(branch[:, None, :] * weights[:, :, None], mode)
    return _r(hidden + injection.reshape(T, -1), mode)


__all__ = ["hyper_mix", "inject", "linear", "rms_norm"]
