"""The C ABI library: it loads, exports every declared symbol, its struct
layouts agree with the ctypes mirror, and its argument checks reject bad
calls before touching a device (no GPU needed)."""
import ctypes
import os
import re
import subprocess

import pytest

from veymoe import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "veymoe.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|uint64_t)\s+(vm_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES)
    assert lib.vm_abi_version() == 3


def test_struct_layouts_match_the_header(tmp_path):
    structs = {
        "VmQ4Proj": _lib.VmQ4Proj, "VmPoolView": _lib.VmPoolView, "VmMoeArgs": _lib.VmMoeArgs,
        "VmRouterArgs": _lib.VmRouterArgs, "VmLayerArgs": _lib.VmLayerArgs, "VmGroupedArgs": _lib.VmGroupedArgs,
        "VmDeviceLru": _lib.VmDeviceLru, "VmHyperArgs": _lib.VmHyperArgs,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', 'int main(void) {']
    for name, cls in structs.items():
        lines.append(f'printf("{name} size %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{name}.{field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    c_values = dict(line.rsplit(" ", 1) for line in out if line)
    for name, cls in structs.items():
        assert int(c_values[f"{name} size"]) == ctypes.sizeof(cls), name
        for field, _ in cls._fields_:
            assert int(c_values[f"{name}.{field}"]) == getattr(cls, field).offset, (name, field)


def _exec_args(**kw):
    a = _lib.VmMoeArgs()
    a.x = 256
    a.routes = 512
    a.output = 768
    a.gate = _lib.VmQ4Proj(1024, 1040, 1056)
    a.up = _lib.VmQ4Proj(1024, 1040, 1056)
    a.down = _lib.VmQ4Proj(1024, 1040, 1056)
    a.tokens, a.slots, a.hidden_size, a.inter_size = 1, 2, 64, 64
    a.expert_count, a.group_size = 4, 32
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code,message", [
    ("group_size", 64, _lib.VM_EUNSUPPORTED, "group_size"),
    ("tokens", 0, _lib.VM_EINVAL, "tokens"),
    ("slots", 11, _lib.VM_EINVAL, "slots"),
    ("hidden_size", 48, _lib.VM_EINVAL, "group aligned"),
    ("act_dtype", 7, _lib.VM_EINVAL, "dtype"),
    ("x", None, _lib.VM_EINVAL, "required"),
    ("shared", 2048, _lib.VM_EINVAL, "together"),
])
def test_execute_rejects_bad_arguments_without_a_device(field, value, code, message):
    a = _exec_args(**{field: value})
    rc = _lib.lib().vm_moe_execute(ctypes.byref(a), None)
    assert rc == code
    assert message in _lib.last_error()


def test_execute_needs_workspace():
    a = _exec_args(scores=4096, workspace=None, workspace_bytes=0)
    assert _lib.lib().vm_moe_execute(ctypes.byref(a), None) == _lib.VM_EWORKSPACE


def test_router_and_layer_bounds():
    lib = _lib.lib()
    r = _lib.VmRouterArgs()
    r.tokens, r.hidden_size, r.expert_count, r.top_k = 1, 64, 513, 4
    assert lib.vm_router_topk(ctypes.byref(r), None) == _lib.VM_EINVAL
    r.expert_count, r.top_k = 4, 5
    assert lib.vm_router_topk(ctypes.byref(r), None) == _lib.VM_EINVAL
    assert "top_k cannot exceed" in _lib.last_error()
    layer = _lib.VmLayerArgs()
    layer.tokens, layer.hidden_size, layer.expert_count, layer.top_k = 9, 64, 8, 2
    layer.inter_size, layer.group_size = 64, 32
    assert lib.vm_moe_layer(ctypes.byref(layer), None) == _lib.VM_EINVAL


def _lru_call(**kw):
    """vm_moe_layer_lru on fake pointers: every case must fail validation."""
    a = _lib.VmLayerArgs()
    a.x, a.output, a.router_weight = 256, 512, 768
    a.tokens, a.hidden_size, a.inter_size, a.expert_count, a.top_k, a.group_size = 1, 64, 64, 8, 2, 32
    a.pool.base, a.pool.record_stride, a.pool.records = 4096, 4096, 16
    lru = _lib.VmDeviceLru()
    lru.slot_table, lru.slot_owner, lru.lru_order, lru.counters, lru.host_row = 1024, 1056, 1088, 1120, 1152
    lru.host_store, lru.host_stride, lru.host_records = 8192, 4096, 8
    lru.layers, lru.layer, lru.slots, lru.order_len = 2, 0, 16, 16
    for k, v in kw.items():
        target = lru if hasattr(lru, k) and k not in ("slot_table",) and not hasattr(a, k) else a
        setattr(target, k, v)
    return _lib.lib().vm_moe_layer_lru(ctypes.byref(a), ctypes.byref(lru), None)


@pytest.mark.parametrize("field,value,code,message", [
    ("tokens", 9, _lib.VM_EUNSUPPORTED, "decode calls"),
    ("phases", 1, _lib.VM_EINVAL, "phases"),
    ("host_store", None, _lib.VM_EINVAL, "state pointers"),
    ("layer", 2, _lib.VM_EINVAL, "outside"),
    ("slots", 15, _lib.VM_EINVAL, "must equal the pool records"),
    ("lru_order", None, _lib.VM_EINVAL, "state pointers"),
    ("order_len", 17, _lib.VM_EINVAL, "exceeds the slots"),
    ("order_len", 1, _lib.VM_EINVAL, "queued slots"),
])
def test_layer_lru_rejects_bad_arguments_without_a_device(field, value, code, message):
    assert _lru_call(**{field: value}) == code
    assert message in _lib.last_error()


def test_pool_stage_checks_indices_before_copying():
    lib = _lib.lib()
    src = (ctypes.c_int64 * 1)(5)
    dst = (ctypes.c_int64 * 1)(0)
    rc = lib.vm_pool_stage(4096, 4096, 4096, 2, 8192, 4096, 4, 4096, src, dst, 1, None)
    assert rc == _lib.VM_EINVAL and "src_index" in _lib.last_error()
    src[0], dst[0] = 0, 2
    rc = lib.vm_pool_stage(4096, 4096, 4096, 2, 8192, 4096, 4, 4096, src, dst, 1, None)
    assert rc == _lib.VM_EINVAL and "dst_slot" in _lib.last_error()
    assert lib.vm_pool_stage(None, 0, 0, 0, None, 0, 0, 0, src, dst, 0, None) == _lib.VM_OK


def test_library_has_no_cpu_fallback_symbols():
    """The product library holds only GPU entry points: every compute call
    takes a stream and runs HIP kernels."""
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert {n for n in exported if n.startswith("vm_")} == set(_declared())


def _hyper_call(**kw):
    """vm_hyper_mix on fake pointers: every case must fail validation."""
    a = _lib.VmHyperArgs()
    a.hidden, a.norm_weight, a.mixed, a.weights, a.workspace = 256, 512, 768, 1024, 4096
    for proj, base in (("mix_down", 8192), ("mix_up", 16384), ("inject", 24576)):
        q = getattr(a, proj)
        q.weight, q.scales, q.biases = base, base + 2048, base + 4096
    a.tokens, a.hidden_size, a.hc_count, a.lowrank, a.norm_group, a.one_centered = 1, 256, 4, 32, 0, 1
    a.workspace_bytes = 1 << 20
    a.eps = 1e-6
    for k, v in kw.items():
        setattr(a, k, v)
    return _lib.lib().vm_hyper_mix(ctypes.byref(a), None)


@pytest.mark.parametrize("field,value,code,message", [
    ("hc_count", 0, _lib.VM_EINVAL, "hc_count"),
    ("hc_count", 9, _lib.VM_EINVAL, "hc_count"),
    ("hidden_size", 4100, _lib.VM_EUNSUPPORTED, "multiple of 64"),
    ("lowrank", 48, _lib.VM_EUNSUPPORTED, "lowrank"),
    ("norm_group", 96, _lib.VM_EUNSUPPORTED, "norm_group"),
    ("mixed", None, _lib.VM_EINVAL, "required"),
    ("hidden", 258, _lib.VM_EINVAL, "aligned"),
    ("workspace_bytes", 16, _lib.VM_EWORKSPACE, "workspace"),
    ("tokens", 70000, _lib.VM_EUNSUPPORTED, "65535"),
])
def test_hyper_mix_rejects_bad_arguments_without_a_device(field, value, code, message):
    assert _hyper_call(**{field: value}) == code
    assert message in _lib.last_error()


def test_hyper_mix_workspace_size():
    lib = _lib.lib()
    # normed [T, n] bf16 then d [T, lowrank] bf16, each 256-byte aligned
    assert lib.vm_hyper_mix_workspace(1, 4, 2048, 32, 0) == 8192 * 2 + 256
    assert lib.vm_hyper_mix_workspace(3, 4, 2048, 32, 1) == 3 * 8192 * 4 + 512


def test_layer_injection_is_validated_without_a_device():
    a = _lib.VmLayerArgs()
    a.x, a.output, a.router_weight = 256, 512, 768
    a.tokens, a.hidden_size, a.inter_size, a.expert_count, a.top_k, a.group_size = 1, 64, 64, 8, 2, 32
    a.gate.weight = a.up.weight = a.down.weight = 4096
    a.gate.scales = a.up.scales = a.down.scales = 8192
    a.gate.biases = a.up.biases = a.down.biases = 8192
    a.inject_out = 16384
    assert _lib.lib().vm_moe_layer(ctypes.byref(a), None) == _lib.VM_EINVAL
    assert "inject_hidden" in _lib.last_error()
    a.inject_hidden, a.inject_weights, a.hc_count = 16384, 20480, 9
    assert _lib.lib().vm_moe_layer(ctypes.byref(a), None) == _lib.VM_EINVAL
    assert "hc_count" in _lib.last_error()


def test_static_layer_refuses_calls_above_its_scratch_without_a_device():
    text = open(HEADER).read()
    assert re.search(r"#define VM_STATIC_SCRATCH_BYTES \(4ull << 20\)", text)
    assert _lib.VM_STATIC_SCRATCH_BYTES == 4 << 20
    lib = _lib.lib()
    a = _lib.VmLayerArgs()
    a.x, a.output, a.router_weight = 256, 512, 768
    a.tokens, a.hidden_size, a.inter_size, a.expert_count, a.top_k, a.group_size = 2048, 2048, 512, 512, 10, 32
    a.gate.weight = a.up.weight = a.down.weight = 4096
    a.gate.scales = a.up.scales = a.down.scales = 8192
    a.gate.biases = a.up.biases = a.down.biases = 8192
    need = lib.vm_moe_layer_workspace(2048, 10, 2048, 512, 0, 512, 0)
    assert need > _lib.VM_STATIC_SCRATCH_BYTES
    assert lib.vm_moe_layer_static(ctypes.byref(a), None) == _lib.VM_EWORKSPACE
    assert "static" in _lib.last_error() and str(need) in _lib.last_error()
    a.tokens = 8   # a decode call fits; the argument checks still come first
    assert lib.vm_moe_layer_workspace(8, 10, 2048, 512, 0, 512, 0) <= _lib.VM_STATIC_SCRATCH_BYTES
    a.router_weight = 770
    assert lib.vm_moe_layer_static(ctypes.byref(a), None) == _lib.VM_EINVAL


def test_decode_workspace_reserves_hand_off_words_for_one_token_bf16_only():
    """fp32 calls above the decode bound take one decode workspace per chunk
    of 8 rows.  Laid out by hand at 8 rows, hidden 2048, top-10 of 512, inter
    512 with a shared expert (offsets 256-aligned): logits 8*512*4 = 16384 B,
    activations 8*11*512*4 = 180224 B, sigmoid 32 -> 256, indices, scores and
    route words 320 -> 512 each, the LRU fill list 4 + 8*80 = 644 -> 768, after
    a 256-byte head: 199424 B, with no hand-off words (those serve one-token
    bf16 calls only).  2048 fp32 rows: 256 such chunks, 48.7 MiB."""
    lib = _lib.lib()
    per = lib.vm_moe_layer_workspace(8, 10, 2048, 512, 512, 512, 1)
    assert per == 199424
    assert lib.vm_moe_layer_workspace(2048, 10, 2048, 512, 512, 512, 1) == 256 * 199424
    # one token: fp32 by the same hand layout (logits 2048, activations
    # 22528, the rest 256 each, fill list 768) is 26624 B; bf16 (activations
    # 11264) 15360 B, plus the two-launch pipeline's hand-off words (at least
    # one 32-bit word per routed activation) when the library carries it
    assert lib.vm_moe_layer_workspace(1, 10, 2048, 512, 512, 512, 1) == 26624
    one = lib.vm_moe_layer_workspace(1, 10, 2048, 512, 512, 512, 0)
    if _lib.lib_built_with_fused_pipelines():
        assert one >= 15360 + 10 * 512 * 4
    else:
        assert one == 15360


def test_default_build_carries_the_default_pipeline_only():
    """The one-token pipelines 1 and 2 (measured slower) are compiled only
    with -DVM_FUSED_PIPELINES=1; the shipped build refuses them."""
    lib = _lib.lib()
    if _lib.lib_built_with_fused_pipelines():
        pytest.skip("this library was built with the one-token pipelines")
    assert lib.vm_decode_pipeline(-1) == 0
    assert lib.vm_decode_pipeline(1) == _lib.VM_EUNSUPPORTED
    assert "VM_FUSED_PIPELINES" in _lib.last_error()
    assert lib.vm_decode_pipeline(0) == 0
