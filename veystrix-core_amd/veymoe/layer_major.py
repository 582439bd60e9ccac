"""Layer-major (windowed) prefill through the MoE layers.

Counterpart of the reference's layer-major prefill (models/flashnext/layer_major.py:1-27,
118-128, 155-211).  Chunk-major order runs every chunk through every layer in
turn, so each chunk re-reads the experts it routes; a window of several chunks
run layer-major reads each layer's experts once for all of them:

    chunk 1 -> layers 0..L-1, chunk 2 -> layers 0..L-1, ...     (chunk-major)
    layer 0 -> chunks 1..n,   layer 1 -> chunks 1..n,   ...     (layer-major)

Here a layer of a window is ONE grouped call over all the window's rows (the
device sort groups every chunk's rows of an expert into the same tiles), so an
expert's records are read from HBM once per window and the row count per
expert grows with the window, which raises the MFMA work per weight byte.

Exactness: every output row of the MoE layer depends on its own input row only
(router logits, top-k, expert rows and combine are per row, and each MFMA
output element accumulates the same K sequence whatever rows share its tile),
so a window gives the chunk-major bits whenever every chunk takes the grouped
path.  A trailing chunk of at most ``TINY_CHUNK_TOKENS`` rows would take the
decode path instead; like the reference (``peel_tail``) it runs chunk-major
after the window.
"""
from __future__ import annotations

from typing import Callable, List, Optional, Sequence, Tuple

import torch

DEFAULT_WINDOW_TOKENS = 8192
MIN_WINDOW_TOKENS = 1024
MAX_WINDOW_TOKENS = 32768
TINY_CHUNK_TOKENS = 8   # rows <= this take the decode path (the reference's custom-kernel bound)

Span = Tuple[int, int]


def plan_windows(spans: Sequence[Span], offset: int, window: int, required=(), anchors=()) -> List[List[Span]]:
    """Group chunk spans (relative ``(start, end)``) into windows of whole chunks.

    A window holds at most ``window`` tokens unless one chunk alone is larger.
    It is cut at a ``required`` absolute position (the end of the system
    prompt) that falls on one of its chunk ends; otherwise, when more chunks
    follow, at the last ``anchors`` position in its second half; otherwise at
    the last chunk that fits."""
    spans = [(int(a), int(b)) for a, b in spans]
    required = {int(p) for p in required}
    anchors = {int(p) for p in anchors}
    windows: List[List[Span]] = []
    i = 0
    while i < len(spans):
        first = spans[i][0]
        limit = first + int(window)
        last = i
        while last + 1 < len(spans) and spans[last + 1][1] <= limit:
            last += 1
        cut = next((k for k in range(i, last + 1) if offset + spans[k][1] in required), None)
        if cut is None and last + 1 < len(spans):
            half = first + int(window) // 2
            preferred = [k for k in range(i, last + 1) if offset + spans[k][1] in anchors and spans[k][1] > half]
            cut = preferred[-1] if preferred else None
        last = last if cut is None else cut
        windows.append(spans[i:last + 1])
        i = last + 1
    return windows


def peel_tail(group: Sequence[Span]) -> Tuple[List[Span], Optional[Span]]:
    """(spans run layer-major, trailing tiny span or None): only a window of
    more than one chunk whose last chunk has at most TINY_CHUNK_TOKENS rows is
    split."""
    group = list(group)
    if len(group) > 1 and group[-1][1] - group[-1][0] <= TINY_CHUNK_TOKENS:
        return group[:-1], group[-1]
    return group, None


# ------------------------------------------------------------ cost model ---

def expert_pass_bytes(experts: int, layers: int, expert_bytes: int) -> int:
    """Bytes of one pass over every expert of ``layers`` layers."""
    return int(experts) * int(layers) * int(expert_bytes)


def chunk_major_bytes(tokens: int, chunk: int, layers: int, experts_read_per_layer: float, expert_bytes: int) -> int:
    """Expert bytes of chunk-major order: every chunk reads its routed experts in every layer."""
    chunks = -(-int(tokens) // int(chunk))
    return int(chunks * layers * experts_read_per_layer * expert_bytes)


def layer_major_bytes(tokens: int, window: int, layers: int, experts: int, expert_bytes: int) -> int:
    """Expert bytes of layer-major order: every window reads each layer's experts once."""
    return -(-int(tokens) // int(window)) * expert_pass_bytes(experts, layers, expert_bytes)


# -------------------------------------------------------------- execution ---

Glue = Optional[Callable[[int, torch.Tensor, torch.Tensor], torch.Tensor]]


def _next_input(glue: Glue, index: int, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return y if glue is None else glue(index, x, y)


def run_chunk_major(layers: Sequence, chunks: Sequence[torch.Tensor], glue: Glue = None) -> List[torch.Tensor]:
    """The reference order: each chunk [rows, hidden] through every layer.
    ``glue(i, x, y)`` maps layer i's input and MoE output to layer i+1's
    input (the decoder work around the MoE block: residual, norms, attention);
    by default the output is the next input."""
    outs = []
    for x in chunks:
        for i, layer in enumerate(layers):
            x = _next_input(glue, i, x, layer(x))
        outs.append(x)
    return outs


def run_window(layers: Sequence, chunks: Sequence[torch.Tensor], glue: Glue = None) -> List[torch.Tensor]:
    """One window layer-major: per layer, one call over the rows of every
    chunk (each expert read once for the window); a trailing tiny chunk runs
    chunk-major afterwards.  Returns the per-chunk outputs."""
    spans, start = [], 0
    for c in chunks:
        spans.append((start, start + c.shape[0]))
        start += c.shape[0]
    body, tail = peel_tail(spans)
    outs: List[torch.Tensor] = []
    if body:
        x = torch.cat([chunks[k] for k in range(len(body))])
        for i, layer in enumerate(layers):
            x = _next_input(glue, i, x, layer(x))
        outs = list(torch.split(x, [b - a for a, b in body]))
    if tail is not None:
        outs += run_chunk_major(layers, [chunks[-1]], glue)
    return outs


def run_prefill(layers: Sequence, chunks: Sequence[torch.Tensor], window: int = DEFAULT_WINDOW_TOKENS,
                glue: Glue = None) -> List[torch.Tensor]:
    """Every chunk through every layer, windows planned with ``plan_windows``
    and each window run layer-major."""
    if not MIN_WINDOW_TOKENS <= int(window) <= MAX_WINDOW_TOKENS:
        raise ValueError(f"window must be between {MIN_WINDOW_TOKENS} and {MAX_WINDOW_TOKENS} tokens")
    spans, start = [], 0
    for c in chunks:
        spans.append((start, start + c.shape[0]))
        start += c.shape[0]
    index = {span: k for k, span in enumerate(spans)}
    outs: List[torch.Tensor] = []
    for group in plan_windows(spans, 0, window):
        outs += run_window(layers, [chunks[index[s]] for s in group], glue)
    return outs


__all__ = ["DEFAULT_WINDOW_TOKENS", "MAX_WINDOW_TOKENS", "MIN_WINDOW_TOKENS", "TINY_CHUNK_TOKENS",
           "chunk_major_bytes", "expert_pass_bytes", "layer_major_bytes", "peel_tail", "plan_windows",
           "run_chunk_major", "run_prefill", "run_window"]
