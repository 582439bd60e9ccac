"""Checkpoint loading on the CPU: the safetensors reader and writer against the
``safetensors`` library (the format's own implementation), expert records
against the synthetic packer, and the slab pack file against the reference's
own test case (models/flashnext/tests/unit/test_slab_pack.py:65-96)."""
import os
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from veymoe import checkpoint as ck
from veymoe import synth
from veymoe.layout import HEADER, PARTS, RecordLayout
from veymoe.pool import HostRecordStore

SPEC = synth.LayerSpec("ckpt", 256, 128, 48, 4, 128, 1)
SEED = 31


def _export(tmp_path, layers=(0,), shards=2, spec=SPEC):
    """Synthetic layers written as a sharded checkpoint with an index."""
    tensors = {}
    for layer in layers:
        tensors.update(ck.layer_tensors(synth.numpy_layer(spec, SEED, layer, materialise=True), layer))
    names = sorted(tensors)
    weight_map = {}
    for s in range(shards):
        shard = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = {n: tensors[n] for n in names[s::shards]}
        ck.write_safetensors(str(tmp_path / shard), part)
        weight_map.update({n: shard for n in part})
    ck.write_index(str(tmp_path), weight_map)
    return tensors


def test_written_shards_read_back_with_the_safetensors_library(tmp_path):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 16, (5, 7), dtype=np.uint16)
    words = rng.integers(0, 2 ** 32, (3, 4), dtype=np.uint32)
    floats = rng.normal(size=(6,)).astype(np.float32)
    path = str(tmp_path / "a.safetensors")
    ck.write_safetensors(path, {"b": ("BF16", bits), "w": ("U32", words), "f": ("F32", floats)}, {"format": "mlx"})
    with safe_open(path, framework="pt") as f:
        assert f.metadata() == {"format": "mlx"}
        assert torch.equal(f.get_tensor("b").view(torch.int16), torch.from_numpy(bits.view(np.int16)))
        assert torch.equal(f.get_tensor("f"), torch.from_numpy(floats))
    with safe_open(path, framework="np") as f:
        np.testing.assert_array_equal(f.get_tensor("w"), words)
    store = ck.SafetensorsStore(str(tmp_path))
    np.testing.assert_array_equal(store.tensor("b"), bits)
    np.testing.assert_array_equal(store.rows("w", [2, 0]), words[[2, 0]])
    assert store.refs["b"].row_bytes == 14 and store.dtype("w") == "U32"


def test_library_written_shards_read_with_the_store(tmp_path):
    g = torch.Generator().manual_seed(1)
    bf = torch.randn((4, 32), generator=g).to(torch.bfloat16)
    i32 = torch.randint(-2 ** 31, 2 ** 31 - 1, (3, 8), dtype=torch.int32, generator=g)
    save_file({"x.scales": bf, "x.weight": i32}, str(tmp_path / "model.safetensors"))
    store = ck.SafetensorsStore(str(tmp_path))
    assert store.dtype("x.scales") == "BF16" and store.shape("x.scales") == (4, 32)
    np.testing.assert_array_equal(store.tensor("x.scales").view(np.int16), bf.view(torch.int16).numpy())
    np.testing.assert_array_equal(store.tensor("x.weight").view(np.int32), i32.numpy())


def test_expert_records_equal_the_synthetic_packer(tmp_path):
    _export(tmp_path, layers=(0, 3))
    store = ck.SafetensorsStore(str(tmp_path))
    assert ck.layer_dims(store, 3) == (SPEC.experts, SPEC.hidden, SPEC.inter)
    layout = SPEC.layout
    for layer in (0, 3):
        for expert in (0, 17, SPEC.experts - 1):
            got = ck.pack_expert(store, layer, expert, layout)
            np.testing.assert_array_equal(got, synth.expert_record(SPEC, SEED, layer, expert))
    host = HostRecordStore(layout, 2 * SPEC.experts, pin=False)
    assert ck.fill_host_store(store, host, [0, 3], chunk=7) == 2 * SPEC.experts
    for layer, expert in ((0, 5), (3, 40)):
        np.testing.assert_array_equal(host.buffer[host.row(layer, expert)].numpy(),
                                      synth.expert_record(SPEC, SEED, layer, expert))


def test_wrong_dtypes_and_shapes_are_refused(tmp_path):
    tensors = _export(tmp_path, shards=1)
    name = ck.expert_tensor(0, "up_proj", "scales")
    dtype, arr = tensors[name]
    tensors[name] = ("F16", arr)                     # same bytes, wrong dtype
    ck.write_safetensors(str(tmp_path / "model-00001-of-00001.safetensors"), tensors)
    store = ck.SafetensorsStore(str(tmp_path))
    with pytest.raises(ValueError, match="dtype F16, expected BF16"):
        ck.layer_dims(store, 0)
    with pytest.raises(ValueError, match="Row dtype mismatch"):
        ck.pack_expert(store, 0, 1, SPEC.layout)
    tensors[name] = ("BF16", arr[:, :, :2])          # truncated rows
    ck.write_safetensors(str(tmp_path / "model-00001-of-00001.safetensors"), tensors)
    store = ck.SafetensorsStore(str(tmp_path))
    with pytest.raises(ValueError, match="shape"):
        ck.layer_dims(store, 0)
    with pytest.raises(ValueError, match="Row size mismatch"):
        ck.pack_expert(store, 0, 1, SPEC.layout)


def test_corrupt_shards_are_refused(tmp_path):
    path = tmp_path / "model.safetensors"
    ck.write_safetensors(str(path), {"a": ("U32", np.zeros((4, 4), np.uint32))})
    data = path.read_bytes()
    path.write_bytes(data[:-8])                      # data shorter than the header says
    with pytest.raises(ValueError, match="inconsistent"):
        ck.SafetensorsStore(str(tmp_path))
    path.write_bytes(struct.pack("<Q", ck.HEADER_LIMIT + 1) + data[8:])
    with pytest.raises(ValueError, match="exceeds"):
        ck.SafetensorsStore(str(tmp_path))


def test_slab_pack_matches_the_reference_case(tmp_path):
    """test_slab_pack.py:65-96 of the reference: allocation {5: [10, 20],
    11: [30, 40]} -> 4 records in sorted-layer order, layer 5 from slot 0,
    layer 11 from slot 2, the gate weight of (5, 10) first after the header."""
    _export(tmp_path, layers=(5, 11))
    store = ck.SafetensorsStore(str(tmp_path))
    layout = SPEC.layout
    out = str(tmp_path / "test_slab.bin")
    total = ck.write_slab_pack(store, {11: [30, 40], 5: [10, 20]}, out, layout, model_hash=b"abcdefgh")
    assert total == ck.PACK_HEADER_SIZE + 4 * layout.record_stride == os.path.getsize(out)
    pack = ck.SlabPackFile(out, layout, expected_model_hash=b"abcdefgh")
    assert pack.expert_count == 4
    assert pack.layer_to_base_slot == {5: 0, 11: 2}
    assert pack.layer_expert_to_slot == {(5, 10): 0, (5, 20): 1, (11, 30): 2, (11, 40): 3}
    raw = open(out, "rb").read()
    gate_w = store.rows(ck.expert_tensor(5, "gate_proj", "weight"), [10])
    start = ck.PACK_HEADER_SIZE + layout.offset("gate_proj", "weight")
    assert raw[start:start + gate_w.nbytes] == gate_w.tobytes()
    assert struct.unpack_from("<IIIII", raw, 0) == (0x4D4F4553, 1, 4, layout.record_stride, 4096)
    np.testing.assert_array_equal(pack.record(11, 40), synth.expert_record(SPEC, SEED, 11, 40))
    host = pack.to_host_store(HostRecordStore(layout, 4, pin=False))
    np.testing.assert_array_equal(host.buffer[host.row(5, 20)].numpy(), synth.expert_record(SPEC, SEED, 5, 20))
    with pytest.raises(ValueError, match="model identity"):
        ck.SlabPackFile(out, layout, expected_model_hash=b"zzzzzzzz")
    with pytest.raises(ValueError, match="record stride"):
        ck.SlabPackFile(out, RecordLayout(512, 128))


def test_slab_pack_header_checks(tmp_path):
    layout = SPEC.layout
    path = tmp_path / "p.bin"
    header = bytearray(4096)
    struct.pack_into("<IIIII8sI", header, 0, 0x4D4F4553, 1, 1, layout.record_stride, 4096, b"\0" * 8, 0)
    struct.pack_into("<HHI", header, 32, 0, 0, 0)
    path.write_bytes(bytes(header) + bytes(layout.record_stride))
    assert ck.SlabPackFile(str(path), layout).expert_count == 1
    path.write_bytes(bytes(header) + bytes(layout.record_stride - 1))
    with pytest.raises(ValueError, match="Invalid slab pack size"):
        ck.SlabPackFile(str(path), layout)
    bad = bytearray(header)
    struct.pack_into("<I", bad, 0, 0x12345678)
    path.write_bytes(bytes(bad) + bytes(layout.record_stride))
    with pytest.raises(ValueError, match="Invalid slab pack header"):
        ck.SlabPackFile(str(path), layout)
    bad = bytearray(header)
    struct.pack_into("<HHI", bad, 32, 0, 0, 3)
    path.write_bytes(bytes(bad) + bytes(layout.record_stride))
    with pytest.raises(ValueError, match="directory slot 3"):
        ck.SlabPackFile(str(path), layout)
    path.write_bytes(bytes(100))
    with pytest.raises(ValueError, match="truncated"):
        ck.SlabPackFile(str(path), layout)
    assert HEADER == ck.PACK_HEADER_SIZE
    assert [layout.offset(*k) for k in PARTS] == layout.part_offsets()
