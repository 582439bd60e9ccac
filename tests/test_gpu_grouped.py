"""GPU parity of the grouped path (more than 8 rows): router GEMM, device
token-by-expert sort, MFMA grouped gate/up/down and the combines, against the
oracle.

The router logits of the grouped path come from an MFMA GEMM with fp32
accumulation, the oracle's from float64; a logit that sits on a bf16 rounding
boundary can round the other way, which can swap two experts whose gates tie
within one bf16 step.  Index sets are therefore required to match exactly
except on tokens whose oracle gates at ranks k-1 and k are within one bf16
step (a near tie, counted and bounded), and outputs are compared on the tokens
whose index sets match.

The matrix-form kernels round every dequantised weight to bf16 before the
MFMA, as the reference's gather_qmm matrix kernels stage weights in the
activation type; they are compared elementwise with the oracle's matrix form
(moe_oracle.qmm_project) and, at the layer tolerance (max-abs-rel 2e-2), with
the vector-form oracle that keeps the weights unrounded.
"""
import numpy as np
import pytest
import torch

from gpu_util import bf16_device, host, packs, to_device, ulp_diff_bf16
from oracle import moe_oracle as mo
from veymoe import assemble, synth
from veymoe.grouped import COMBINE_FUSED, COMBINE_GENERIC, COMBINE_NONE, grouped_experts
from veymoe.layer import HipSwitchGLU
from veymoe.layout import RecordLayout, pack_record
from veymoe.pool import ExpertPool

pytestmark = pytest.mark.gpu


def _near_tie(gates_row, k):
    order = np.sort(mo.f32_to_bf16_bits(np.asarray(gates_row, np.float32)).astype(np.int64))[::-1]
    return order[k - 1] - order[k] <= 1


def _check_selection(inds, ref, k, max_near_ties, label=""):
    """Rows whose index sets differ must be near ties; returns the matching
    rows.  The number of differing rows seen is printed (pytest -s / -v
    output) next to the bound, so a run shows what it found."""
    same = np.array([set(a) == set(b) for a, b in zip(inds.tolist(), ref["inds"].tolist())])
    for t in np.nonzero(~same)[0]:
        assert _near_tie(ref["gates"][t], k), (t, inds[t], ref["inds"][t])
    print(f"[selection] {label} rows {len(same)}: index sets differing from the oracle "
          f"{int((~same).sum())} (near ties; bound {max_near_ties})", flush=True)
    assert (~same).sum() <= max_near_ties, int((~same).sum())
    return same


def _layer_ref(spec, seed, x_np, rows, qmm=True):
    layer_np = synth.numpy_layer(spec, seed)
    return mo.moe_layer(x_np[rows], layer_np, "bf16", path="prefill", qmm=qmm)


def _close_qmm(actual, expected, message):
    """Against the matrix-form oracle the remaining differences are bf16
    rounding-boundary flips of intermediate values (fp32 against float64
    accumulation): each at most one bf16 step at the scale of the output,
    and rare."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    scale = float(np.abs(expected).max())
    np.testing.assert_allclose(actual, expected, rtol=2e-2, atol=2.0 ** -7 * scale, err_msg=message)
    assert mo.max_abs_rel(actual, expected) <= 2.0 ** -7, (message, mo.max_abs_rel(actual, expected))
    far = ulp_diff_bf16(actual, expected) > 1
    assert far.mean() < 2e-3, (message, far.mean())


def _assert_layer(actual, spec, seed, x_np, rows, same, ref, message):
    """Elementwise against the matrix-form oracle, max-abs-rel 2e-2 against
    the vector-form oracle."""
    _close_qmm(actual[same], ref["output"][same], message)
    vec = _layer_ref(spec, seed, x_np, rows, qmm=False)
    assert mo.max_abs_rel(actual[same], vec["output"][same]) <= 2e-2, message


@pytest.mark.parametrize("tokens", [9, 40, 130])
def test_grouped_layer_small(device, tokens):
    spec = synth.CONFIGS["decode_small"]
    seed = 300 + tokens
    layer = assemble.build_layer(spec, seed, device, dense=True)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, tokens))
    y = layer(bf16_device(x_np, device))
    torch.cuda.synchronize()
    rows = np.arange(tokens)
    ref = _layer_ref(spec, seed, x_np, rows)
    same = _check_selection(layer.last_inds.cpu().numpy(), ref, spec.top_k, max(1, tokens // 20), f"T={tokens}")
    _assert_layer(host(y), spec, seed, x_np, rows, same, ref, f"grouped layer T={tokens}")


@pytest.mark.parametrize("tokens", [130, 300])
def test_grouped_layer_narrow_hidden_with_shared_expert(device, tokens):
    """Hidden 256 with a shared expert: at 130 rows one more group of the
    sorted GEMMs, at 300 rows on the side stream, whose rows and sigmoid gates
    the combine reads back.
    At this width a token's 32 combine threads share a wave with another
    token's, so the combine takes its per-lane loads (wider layers read a
    token's indices, scores and gate through scalar loads)."""
    spec = synth.LayerSpec("narrow_shared", 256, 128, 64, 4, 128, 1)
    seed = 320 + tokens
    layer = assemble.build_layer(spec, seed, device, dense=True)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, tokens))
    y = layer(bf16_device(x_np, device))
    torch.cuda.synchronize()
    rows = np.arange(tokens)
    ref = _layer_ref(spec, seed, x_np, rows)
    same = _check_selection(layer.last_inds.cpu().numpy(), ref, spec.top_k, max(1, tokens // 20), f"T={tokens}")
    _assert_layer(host(y), spec, seed, x_np, rows, same, ref, f"narrow grouped layer T={tokens}")


def test_grouped_layer_tile_heights_agree(device):
    """768, 1024 and 4096 tokens over 64 experts top-4: 48, 64 and 256 rows
    per expert on average.  A call whose experts average more rows than one
    tile of the usual height holds takes 96-row tiles: neither GEMM at 768
    tokens, the down GEMM at 1024 (above its 48), both at 4096 (several row
    tiles per group).  Each call is checked against the oracle on a sample,
    and a row's result does not depend on its tile, so the first 768 rows of
    every call are equal bit for bit."""
    spec = synth.CONFIGS["decode_small"]
    seed = 311
    layer = assemble.build_layer(spec, seed, device, dense=True)
    x_all = mo.bf16_bits_to_f32(synth.tokens(spec, seed, 4096))
    first = None
    for tokens in (768, 1024, 4096):
        x_np = x_all[:tokens]
        y = layer(bf16_device(x_np, device))
        torch.cuda.synchronize()
        sample = np.random.default_rng(tokens).choice(tokens, 48, replace=False)
        ref = _layer_ref(spec, seed, x_np, sample)
        inds = layer.last_inds.cpu().numpy()[sample]
        same = _check_selection(inds, ref, spec.top_k, 3, f"T={tokens} over 64 experts")
        _assert_layer(host(y)[sample], spec, seed, x_np, sample, same, ref, f"grouped layer T={tokens} (sample)")
        if first is None:
            first = y[:768].clone()
        else:
            assert torch.equal(first.view(torch.int16), y[:768].view(torch.int16)), tokens


@pytest.mark.parametrize("hidden,experts,tokens,zipf", [(4096, 128, 300, None), (4096, 128, 8256, None),
                                                         (1024, 512, 4096, None), (2048, 512, 1000, 1.1),
                                                         (1024, 96, 300, None)],
                         ids=["k4096-8stage", "k4096-4stage", "k1024-4stage", "k2048-bias", "chunked-e96"])
def test_router_gemm_instances(device, hidden, experts, tokens, zipf):
    """The router GEMM of calls above 64 rows at the K and ring depths the
    prefill shapes do not reach (K = 4096 with eight and four stages, K = 1024
    with four), with a router bias (the log-Zipf popularity of the
    synthetic layers), and at 96 experts, which the ring does not take (the
    chunked GEMM computes those logits): the experts chosen per row equal the decode router's,
    which sums every logit in another order, except on near ties (bounded,
    and checked against the oracle's gates); at 300 rows the whole layer is
    compared with the oracle."""
    from veymoe.router import router_topk

    spec = synth.LayerSpec(f"router_k{hidden}", hidden, 256, experts, 6, 0, tokens, zipf_s=zipf)
    seed = 340 + hidden // 1024 + experts
    layer = assemble.build_layer(spec, seed, device, dense=True)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, tokens))
    x = bf16_device(x_np, device)
    y = layer(x)
    grouped = layer.last_inds.sort(dim=1).values
    bias = layer.gate.bias.float() if layer.gate.bias is not None else None
    decode, _ = router_topk(x, layer.gate.weight, spec.top_k, logit_bias=bias)
    decode = decode.sort(dim=1).values
    torch.cuda.synchronize()
    differ = np.nonzero(~(grouped == decode).all(dim=1).cpu().numpy())[0]
    print(f"[selection] router GEMM K={hidden} E={experts} T={tokens}: {len(differ)} rows differ from the "
          f"decode router", flush=True)
    if len(differ):
        layer_np = synth.numpy_layer(spec, seed)
        _, _, gates = mo.route(x_np[differ], layer_np["router"], spec.top_k, "bf16", layer_np.get("router_bias"))
        for i in range(len(differ)):
            assert _near_tie(gates[i], spec.top_k), int(differ[i])
    assert len(differ) <= max(1, tokens // 1000)
    if tokens <= 512:
        rows = np.arange(tokens)
        ref = _layer_ref(spec, seed, x_np, rows)
        same = _check_selection(layer.last_inds.cpu().numpy(), ref, spec.top_k, max(1, tokens // 20),
                                f"K={hidden} T={tokens}")
        _assert_layer(host(y), spec, seed, x_np, rows, same, ref, f"layer K={hidden} T={tokens}")


def test_grouped_batched_config_pool(device):
    """The full-size layer with Zipf(1.1) routing at 32 tokens, experts in a
    pool behind a permuted slot table, shared expert included."""
    spec = synth.CONFIGS["batched"]
    seed = 320
    pool = ExpertPool(spec.layout, spec.experts + 8, layers=1, experts=spec.experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, 32))
    y = layer(bf16_device(x_np, device))
    torch.cuda.synchronize()
    rows = np.arange(32)
    ref = _layer_ref(spec, seed, x_np, rows)
    same = _check_selection(layer.last_inds.cpu().numpy(), ref, spec.top_k, 2, "batched T=32")
    _assert_layer(host(y), spec, seed, x_np, rows, same, ref, "batched layer")
    distinct = len(np.unique(ref["inds"]))
    assert 40 <= distinct <= 320, distinct


def test_grouped_prefill_matches_decode_rows(device):
    """At the full prefill shape (2048 tokens, 512 experts top-10 + shared):
    256 rows spread over the call against the oracle, and the first 8 rows
    against the decode kernels run on those 8 rows alone.

    The grouped router is an MFMA GEMM and the decode router a v_dot2
    reduction: both accumulate in fp32, in different orders, so a logit on a
    bf16 rounding boundary can round differently and swap two experts whose
    gates tie within one bf16 step.  The number of such rows is printed."""
    spec = synth.CONFIGS["prefill"]
    seed = 330
    pool = ExpertPool(spec.layout, spec.experts, layers=1, experts=spec.experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, 2048))
    x = bf16_device(x_np, device)
    y = layer(x)
    inds_all = layer.last_inds.clone()
    y8 = layer(x[:8].contiguous())
    torch.cuda.synchronize()
    agree = (inds_all[:8].sort(dim=1).values == layer.last_inds.sort(dim=1).values).all(dim=1).cpu().numpy()
    print(f"[selection] prefill rows 0..7: grouped and decode routers agree on {int(agree.sum())} of 8", flush=True)
    assert int(agree.sum()) >= 7
    # matrix form + generic combine against vector form + fused combine: the layer tolerance
    assert mo.max_abs_rel(host(y)[:8][agree], host(y8)[agree]) <= 2e-2
    sample = np.linspace(0, 2047, 256).astype(np.int64)
    ref = _layer_ref(spec, seed, x_np, sample)
    same = _check_selection(inds_all.cpu().numpy()[sample], ref, spec.top_k, 3, "prefill T=2048 (256 rows)")
    _assert_layer(host(y)[sample], spec, seed, x_np, sample, same, ref, "prefill sample vs oracle")


def test_grouped_router_against_the_decode_router_over_8192_rows(device):
    """The rate at which the grouped (MFMA) router and the decode (v_dot2)
    router pick different expert sets for the same token, over 8192 tokens
    at the full prefill shape: the layer in 2048-row calls (MFMA router)
    against vm_router_topk, which sums every logit in the decode order at
    any row count.  Calls of up to 64 rows route with the decode router, so
    only calls above that can differ; the differing rows must be near ties
    and their count is printed."""
    from veymoe.router import router_topk

    spec = synth.CONFIGS["prefill"]
    seed = 331
    pool = ExpertPool(spec.layout, spec.experts, layers=1, experts=spec.experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    rows = 8192
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, rows))
    x = bf16_device(x_np, device)
    grouped = []
    for c in range(0, rows, 2048):
        layer(x[c:c + 2048].contiguous())
        grouped.append(layer.last_inds.clone())
    grouped = torch.cat(grouped).sort(dim=1).values
    bias = layer.gate.bias.float() if layer.gate.bias is not None else None
    decode, _ = router_topk(x, layer.gate.weight, spec.top_k, logit_bias=bias)
    decode = decode.sort(dim=1).values
    torch.cuda.synchronize()
    differ = np.nonzero(~(grouped == decode).all(dim=1).cpu().numpy())[0]
    print(f"[selection] grouped vs decode router over {rows} rows: {len(differ)} rows differ "
          f"({len(differ) / rows:.2e})", flush=True)
    if len(differ):
        layer_np = synth.numpy_layer(spec, seed)
        _, _, gates = mo.route(x_np[differ], layer_np["router"], spec.top_k, "bf16", layer_np["router_bias"])
        for i in range(len(differ)):
            assert _near_tie(gates[i], spec.top_k), int(differ[i])
    assert len(differ) <= rows // 1000


def _switch(np_packs, hidden, inter, experts, device):
    return HipSwitchGLU(hidden, inter, experts, projections=to_device(np_packs, device))


@pytest.mark.parametrize("mode", [COMBINE_NONE, COMBINE_GENERIC, COMBINE_FUSED])
@pytest.mark.parametrize("tokens,crowd,hidden,inter", [(150, 100, 256, 128), (60, 40, 256, 256), (24, 17, 4096, 512)],
                         ids=["64-row-tiles", "16-row-tiles", "16-row-tiles-k4096"])
def test_grouped_experts_modes(device, mode, tokens, crowd, hidden, inter):
    """150 tokens run the 64-row tile GEMM; calls of up to 64 rows whose
    hidden and intermediate sizes have an instance run the 16-row tile
    kernels (K = 256 both ways; K = 4096 for gate/up with 512 for down, the
    largest instance).  One expert takes `crowd` rows, so it spans two
    (three, two) tiles."""
    experts, k = 12, 3
    np_packs = packs(41, hidden, inter, experts)
    rng = np.random.default_rng(42)
    inds = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)]).astype(np.int32)
    inds[:crowd, 0] = 5                     # expert 5: several row tiles
    scores = mo.bf16r(rng.uniform(0.05, 0.6, (tokens, k)).astype(np.float32))
    x_np = mo.bf16r(rng.normal(size=(tokens, hidden)).astype(np.float32))
    shared_y = mo.bf16r(rng.normal(0, 0.1, (tokens, hidden)).astype(np.float32))
    switch = _switch(np_packs, hidden, inter, experts, device)
    out = grouped_experts(switch, bf16_device(x_np, device), torch.tensor(inds, device=device),
                          bf16_device(scores, device), bf16_device(shared_y, device), mode)
    torch.cuda.synchronize()
    _, _, _, d_out, _ = mo.execute(x_np, inds, np_packs, "bf16", qmm=True)
    if mode == COMBINE_NONE:
        _close_qmm(host(out), d_out, "per-slot rows")
    elif mode == COMBINE_GENERIC:
        _close_qmm(host(out), mo.generic_combine(d_out, scores, "bf16", shared_y), "generic combine")
    else:
        _close_qmm(host(out), mo.fused_combine(d_out, scores, "bf16", shared_y=shared_y), "fused combine")


def test_grouped_invalid_expert_id_contributes_nothing(device):
    hidden, inter, experts, tokens, k = 128, 64, 6, 12, 2
    np_packs = packs(51, hidden, inter, experts)
    rng = np.random.default_rng(52)
    inds = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)]).astype(np.int32)
    inds[3, 1] = 99                          # outside 0..experts-1
    x_np = mo.bf16r(rng.normal(size=(tokens, hidden)).astype(np.float32))
    switch = _switch(np_packs, hidden, inter, experts, device)
    out = grouped_experts(switch, bf16_device(x_np, device), torch.tensor(inds, device=device))
    torch.cuda.synchronize()
    assert float(out[3, 1].abs().max()) == 0.0
    ok = np.ones(tokens * k, bool)
    ok[3 * k + 1] = False
    inds_ok = inds.copy()
    inds_ok[3, 1] = 0
    _, _, _, d_out, _ = mo.execute(x_np, inds_ok, np_packs, "bf16", qmm=True)
    _close_qmm(host(out).reshape(-1, hidden)[ok], d_out.reshape(-1, hidden)[ok], "valid rows")


def test_grouped_pool_matches_dense_bitwise(device):
    """The same experts through a pool + permuted slot table give the same bits."""
    hidden, inter, experts, tokens, k = 256, 128, 16, 70, 4
    np_packs = packs(61, hidden, inter, experts)
    rng = np.random.default_rng(62)
    inds = torch.tensor(np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)]).astype(np.int32),
                        device=device)
    x = bf16_device(rng.normal(size=(tokens, hidden)).astype(np.float32), device)
    dense = _switch(np_packs, hidden, inter, experts, device)
    layout = RecordLayout(hidden, inter)
    pool = ExpertPool(layout, experts + 5, layers=1, experts=experts, device=device)
    slots = rng.permutation(experts + 5)[:experts]
    for e in range(experts):
        parts = {(name, part): np_packs[name][i][e] for name in np_packs
                 for i, part in enumerate(("weight", "scales", "biases"))}
        pool.record(int(slots[e])).copy_(torch.from_numpy(pack_record(parts, layout)))
    pool.place_all(0, slots)
    pooled = HipSwitchGLU(hidden, inter, experts, pool=pool, layer_id=0)
    a = grouped_experts(dense, x, inds)
    b = grouped_experts(pooled, x, inds)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_pooled_switch_above_the_decode_bound_takes_one_lru_pass(device):
    """A pool-backed HipSwitchGLU called with more than 8 rows assigns and
    fills once per call: pool and switch hit/miss counts, slot table and free
    list follow the reference's LRU (expert_pool.py:123-159) fed the same
    routed ids, and the per-slot outputs equal the dense expert block's."""
    from oracle import pool_oracle
    from veymoe.pool import HostRecordStore

    spec = synth.LayerSpec("sw_pool", 256, 128, 96, 4, 0, 12)
    seed = 404
    store = HostRecordStore(spec.layout, spec.experts)
    for e in range(spec.experts):
        store.put(0, e, synth.expert_record(spec, seed, 0, e))
    pool = ExpertPool(spec.layout, 48, layers=1, experts=spec.experts, device=device)
    pooled = HipSwitchGLU(spec.hidden, spec.inter, spec.experts, pool=pool, layer_id=0, host_store=store)
    layer_np = synth.numpy_layer(spec, seed, materialise=True)
    dense = HipSwitchGLU(spec.hidden, spec.inter, spec.experts, layer_id=0,
                         projections={n: assemble.projection(*layer_np[n], device)
                                      for n in ("gate_proj", "up_proj", "down_proj")})
    ref = pool_oracle.LruSlots(48)
    rng = np.random.default_rng(5)
    for step in range(6):
        rows = 9 + 3 * step
        # each call routes within a window of 40 experts (fits the pool), moving by 17 per call
        window = (17 * step + np.arange(40)) % spec.experts
        inds = np.stack([rng.choice(window, spec.top_k, replace=False) for _ in range(rows)]).astype(np.int32)
        x = assemble.tokens_tensor(spec, seed, device, rows, stream=50 + step)
        got = pooled(x[None], torch.tensor(inds[None], device=device))
        want = dense(x[None], torch.tensor(inds[None], device=device))
        torch.cuda.synchronize()
        assert got.shape == (1, rows, spec.top_k, spec.hidden)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        routed = inds.reshape(-1).tolist()
        _, misses = ref.assign(0, routed)
        hits = len(routed) - len(misses)
        assert (pool.hits, pool.misses) == (ref.hits, ref.misses), step
        assert pooled.misses == ref.misses, step
        assert list(pool._slot_of.items()) == list(ref.slot_of.items()), step
        assert pool._free == ref.free, step
        assert hits >= 0
    assert ref.misses > 48                      # evictions happened
