"""Layer-major prefill windows on the CPU: window planning and the expert-byte
cost model against the reference's own cases
(models/flashnext/tests/unit/test_layer_major.py:60-128), and the
window/chunk-major orchestration on a row-wise stand-in layer."""
import pytest
import torch

from veymoe import layer_major as lm


def spans_of(sizes):
    out, position = [], 0
    for size in sizes:
        out.append((position, position + size))
        position += size
    return out


def test_windows_hold_whole_chunks_within_the_limit():
    spans = spans_of([2048] * 10)
    windows = lm.plan_windows(spans, 0, 8192)
    assert [len(w) for w in windows] == [4, 4, 2]
    assert [s for w in windows for s in w] == spans


def test_a_chunk_larger_than_the_window_still_runs_alone():
    assert [len(w) for w in lm.plan_windows(spans_of([3000, 3000]), 0, 1024)] == [1, 1]


def test_window_ends_at_the_required_system_boundary():
    spans = spans_of([2048, 2048, 1349, 2048, 2048])
    windows = lm.plan_windows(spans, 0, 8192, required=(5445,))
    assert windows[0][-1][1] == 5445
    assert [s for w in windows for s in w] == spans


def test_required_position_is_offset_aware():
    spans = spans_of([2048, 2048, 2048])
    assert lm.plan_windows(spans, 1000, 8192, required=(1000 + 2048,))[0] == spans[:1]


def test_anchors_in_the_second_half_only():
    spans = spans_of([2048] * 6)
    assert lm.plan_windows(spans, 0, 8192, anchors=(6144,))[0][-1][1] == 6144
    assert lm.plan_windows(spans, 0, 8192, anchors=(2048,))[0][-1][1] == 8192
    assert lm.plan_windows([], 0, 8192) == []


def test_cost_model_matches_the_reference_figures():
    record = 3_072_000                                # 48 layers, 512 experts of hidden 2560 / inter 640
    assert lm.expert_pass_bytes(512, 48, record) / 1e9 == pytest.approx(75.5, abs=0.1)
    chunk = lm.chunk_major_bytes(16384, 2048, 48, 400, record)
    window = lm.layer_major_bytes(16384, 8192, 48, 512, record)
    assert chunk / 1e9 == pytest.approx(472.4, abs=1.0)
    assert window / 1e9 == pytest.approx(151.0, abs=1.0)
    assert chunk / window > 3.0


def test_peel_tail():
    assert lm.peel_tail(spans_of([100, 100, 8])) == (spans_of([100, 100]), (200, 208))
    assert lm.peel_tail(spans_of([100, 100, 9])) == (spans_of([100, 100, 9]), None)
    assert lm.peel_tail(spans_of([5])) == (spans_of([5]), None)


def test_window_and_chunk_major_orders_agree_on_a_rowwise_layer():
    g = torch.Generator().manual_seed(0)
    layers = [lambda x, a=a: torch.tanh(x * a + 0.25) for a in (0.5, 1.5, -0.75)]
    glue = lambda i, x, y: x + 0.5 * y
    chunks = [torch.randn((n, 16), generator=g) for n in (40, 17, 33, 3)]
    ref = lm.run_chunk_major(layers, chunks, glue)
    got = lm.run_window(layers, chunks, glue)
    assert len(got) == 4 and all(torch.equal(a, b) for a, b in zip(got, ref))
    planned = lm.run_prefill(layers, chunks * 20, window=1024, glue=glue)
    assert all(torch.equal(a, b) for a, b in zip(planned, lm.run_chunk_major(layers, chunks * 20, glue)))
    with pytest.raises(ValueError):
        lm.run_prefill(layers, chunks, window=512)
