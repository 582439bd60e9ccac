"""Checkpoint loading: safetensors shards -> expert records -> host store / pool.

Counterpart of the reference's on-disk side of the expert path:

* ``SafetensorsStore`` reads the shard headers of a checkpoint directory (the
  ``model.safetensors.index.json`` weight map, else every ``*.safetensors``
  file) into ``TensorRef`` entries (shard, dtype, shape, data start, row bytes)
  and serves rows through read-only memory maps, as ``SafeTensorStore`` does
  (models/flashnext/store.py:108-117, 221-236, 238-262).  bf16 travels as its
  uint16 bit pattern (store.py:26-41).
* ``pack_expert`` assembles the nine rows of one routed expert into a record
  at the ``RecordLayout`` part offsets, with the dtype and size checks of
  ``build_slab_pack`` (models/flashnext/slab_pack.py:300-338).
* ``fill_host_store`` / ``fill_pool`` move records into pinned host memory (the
  source of miss fills) or straight into pool slots; ``load_layer`` builds a
  ``MoELayer`` from the router, shared expert and shared gate tensors of one
  layer (the tensor families of models/flashnext/preflight.py:66-74).
* ``write_slab_pack`` / ``SlabPackFile`` write and read the reference's slab
  pack file (slab_pack.py:1-24, 240-344, 514-612): a 4 KiB header ("MOES",
  version, expert count, record stride, header size, model hash, layout id,
  then (layer u16, expert u16, slot u32) directory entries) followed by the
  records, with the hidden and intermediate sizes as parameters.
* ``write_safetensors`` writes a shard in the safetensors format (header
  length, JSON header, data), for exporting synthetic layers as checkpoints.

Tensor names follow the MLX checkpoint: ``{prefix}.switch_mlp.{gate,up,down}_proj
.{weight,scales,biases}`` stacked over experts, ``{prefix}.gate.weight`` (the
router, bf16), ``{prefix}.shared_expert.{proj}.{part}`` and
``{prefix}.shared_expert_gate.{part}``, where ``prefix`` is
``language_model.model.layers.{layer}.mlp`` by default.
"""
from __future__ import annotations

import json
import os
import struct
from typing import Dict, Iterable, Mapping, Optional, Sequence, Tuple

import numpy as np
import torch

from .layout import HEADER, PART_NAMES, PARTS, PROJECTIONS, RecordLayout

# safetensors dtype -> numpy read dtype (bf16 as raw uint16 bits)
DTYPES: Dict[str, np.dtype] = {
    "F32": np.dtype("<f4"), "F16": np.dtype("<f2"), "BF16": np.dtype("<u2"), "U32": np.dtype("<u4"),
    "I32": np.dtype("<i4"), "I64": np.dtype("<i8"), "U64": np.dtype("<u8"), "F64": np.dtype("<f8"),
    "U16": np.dtype("<u2"), "I16": np.dtype("<i2"), "U8": np.dtype("u1"), "I8": np.dtype("i1"),
    "BOOL": np.dtype("?"),
}
HEADER_LIMIT = 100 * 1024 * 1024  # largest shard header accepted (preflight.py:45)
DEFAULT_PREFIX = "language_model.model.layers.{layer}.mlp"

# slab pack file (slab_pack.py:43-53)
PACK_MAGIC = 0x4D4F4553  # "MOES"
PACK_VERSION = 1         # Q4/G32 records, layout id 0
PACK_HEADER_SIZE = 4096
PACK_DIRECTORY_OFFSET = 32
PACK_ENTRY_SIZE = 8
PACK_MAX_ENTRIES = (PACK_HEADER_SIZE - PACK_DIRECTORY_OFFSET) // PACK_ENTRY_SIZE


class TensorRef:
    """Where one tensor lives: shard file, dtype, shape, first data byte."""
    __slots__ = ("shard", "dtype", "shape", "start", "row_bytes")

    def __init__(self, shard: str, dtype: str, shape: Sequence[int], start: int):
        if dtype not in DTYPES:
            raise ValueError(f"unsupported safetensors dtype {dtype}")
        self.shard = shard
        self.dtype = dtype
        self.shape = tuple(int(s) for s in shape)
        self.start = int(start)
        trailing = int(np.prod(self.shape[1:])) if len(self.shape) > 1 else 1
        self.row_bytes = trailing * DTYPES[dtype].itemsize

    @property
    def nbytes(self) -> int:
        return int(np.prod(self.shape)) * DTYPES[self.dtype].itemsize if self.shape else DTYPES[self.dtype].itemsize


def read_header(path: str) -> Tuple[dict, int]:
    """(header dict, first data byte) of one safetensors shard."""
    with open(path, "rb") as handle:
        raw = handle.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path} is not a safetensors file (truncated header length)")
        length = struct.unpack("<Q", raw)[0]
        if length > HEADER_LIMIT:
            raise ValueError(f"{path}: safetensors header of {length} bytes exceeds {HEADER_LIMIT}")
        text = handle.read(length)
        if len(text) != length:
            raise ValueError(f"{path}: truncated safetensors header")
    return json.loads(text), 8 + length


class SafetensorsStore:
    """Memory-mapped, read-only view over the shards of one checkpoint."""

    def __init__(self, model_dir: str):
        self.dir = os.path.expanduser(model_dir)
        self.refs: Dict[str, TensorRef] = {}
        self._views: Dict[str, np.ndarray] = {}
        index = os.path.join(self.dir, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as handle:
                shards = sorted(set(json.load(handle)["weight_map"].values()))
        else:
            shards = sorted(f for f in os.listdir(self.dir) if f.endswith(".safetensors"))
        if not shards:
            raise ValueError(f"no safetensors shards in {self.dir}")
        for shard in shards:
            self.add_shard(shard)

    def add_shard(self, shard: str) -> None:
        path = os.path.join(self.dir, shard)
        header, data_start = read_header(path)
        size = os.path.getsize(path)
        for name, meta in header.items():
            if name == "__metadata__":
                continue
            begin, end = meta["data_offsets"]
            ref = TensorRef(shard, meta["dtype"], meta["shape"], data_start + begin)
            if end - begin != ref.nbytes or data_start + end > size:
                raise ValueError(f"{shard}: tensor {name} has inconsistent data offsets")
            self.refs[name] = ref

    def __contains__(self, name: str) -> bool:
        return name in self.refs

    def shape(self, name: str) -> Tuple[int, ...]:
        return self.refs[name].shape

    def dtype(self, name: str) -> str:
        return self.refs[name].dtype

    def view(self, name: str) -> np.ndarray:
        """The whole tensor as a read-only memory map (bf16 as uint16)."""
        view = self._views.get(name)
        if view is None:
            ref = self.refs[name]
            view = np.memmap(os.path.join(self.dir, ref.shard), dtype=DTYPES[ref.dtype], mode="r",
                             offset=ref.start, shape=ref.shape)
            self._views[name] = view
        return view

    def rows(self, name: str, indices: Iterable[int]) -> np.ndarray:
        """Rows of the leading axis, gathered into a new array."""
        return np.ascontiguousarray(self.view(name)[np.asarray(list(indices), dtype=np.int64)])

    def tensor(self, name: str) -> np.ndarray:
        """The whole tensor, copied out of the map."""
        return np.array(self.view(name))


# ---------------------------------------------------------------- names ---

def layer_prefix(layer: int, prefix: str = DEFAULT_PREFIX) -> str:
    return prefix.format(layer=int(layer))


def expert_tensor(layer: int, proj: str, part: str, prefix: str = DEFAULT_PREFIX) -> str:
    return f"{layer_prefix(layer, prefix)}.switch_mlp.{proj}.{part}"


def layer_dims(store: SafetensorsStore, layer: int, prefix: str = DEFAULT_PREFIX,
               group_size: int = 32) -> Tuple[int, int, int]:
    """(experts, hidden, intermediate) of one layer's stacked expert tensors,
    after the shape and dtype checks of validate_slab_allocation
    (slab_pack.py:412-460)."""
    gate = store.shape(expert_tensor(layer, "gate_proj", "weight", prefix))
    if len(gate) != 3:
        raise ValueError(f"layer {layer}: expert weights must be [experts, out, in/8]")
    experts, inter, hidden = gate[0], gate[1], gate[2] * 8
    layout = RecordLayout(hidden, inter, group_size)
    for proj, part in PARTS:
        name = expert_tensor(layer, proj, part, prefix)
        want = (experts, *layout.shape(proj, part))
        if store.shape(name) != want:
            raise ValueError(f"{name}: shape {store.shape(name)} does not match {want}")
        dtype = "U32" if part == "weight" else "BF16"
        if store.dtype(name) != dtype:
            raise ValueError(f"{name}: dtype {store.dtype(name)}, expected {dtype}")
    return experts, hidden, inter


# -------------------------------------------------------------- records ---

def pack_expert(store: SafetensorsStore, layer: int, expert: int, layout: RecordLayout,
                out: Optional[np.ndarray] = None, prefix: str = DEFAULT_PREFIX) -> np.ndarray:
    """One routed expert's nine rows as a record of ``layout.record_stride``
    bytes (zero padding after the last part)."""
    if out is None:
        out = np.zeros(layout.record_stride, dtype=np.uint8)
    elif out.size < layout.record_stride:
        raise ValueError("record buffer is smaller than the record stride")
    for proj, part in PARTS:
        name = expert_tensor(layer, proj, part, prefix)
        row = store.rows(name, [expert])[0]
        expected_dtype = np.dtype(np.uint32 if part == "weight" else np.uint16)
        if row.dtype != expected_dtype:
            raise ValueError(f"Row dtype mismatch for {name}: got {row.dtype}, expected {expected_dtype}")
        raw = row.view(np.uint8).reshape(-1)
        rows, cols = layout.shape(proj, part)
        if raw.size != rows * cols * expected_dtype.itemsize:
            raise ValueError(f"Row size mismatch for {name}: got {raw.size} bytes, "
                             f"expected {rows * cols * expected_dtype.itemsize}")
        start = layout.offset(proj, part)
        out[start:start + raw.size] = raw
    out[layout.record_bytes:layout.record_stride] = 0
    return out


def _records(store, layout, layer, experts, prefix, chunk):
    """Yield (experts chunk, records [n, stride] uint8) gathered part by part:
    one fancy-indexed read of every part per chunk instead of nine per expert."""
    experts = [int(e) for e in experts]
    for start in range(0, len(experts), chunk):
        sel = experts[start:start + chunk]
        records = np.zeros((len(sel), layout.record_stride), dtype=np.uint8)
        for proj, part in PARTS:
            rows = store.rows(expert_tensor(layer, proj, part, prefix), sel)
            raw = rows.reshape(len(sel), -1).view(np.uint8)
            off = layout.offset(proj, part)
            records[:, off:off + raw.shape[1]] = raw
        yield sel, records


def fill_host_store(store: SafetensorsStore, host_store, layers: Iterable[int],
                    experts: Optional[Iterable[int]] = None, prefix: str = DEFAULT_PREFIX,
                    chunk: int = 64) -> int:
    """Put the records of every (layer, expert) into a ``HostRecordStore``
    (pinned host memory, the source of miss fills).  Returns records written."""
    layout = host_store.layout
    count = 0
    for layer in layers:
        n_experts, hidden, inter = layer_dims(store, layer, prefix, layout.group_size)
        if (hidden, inter) != (layout.hidden, layout.inter):
            raise ValueError(f"layer {layer} is {hidden}/{inter}, the store holds {layout.hidden}/{layout.inter}")
        todo = range(n_experts) if experts is None else experts
        for sel, records in _records(store, layout, layer, todo, prefix, chunk):
            for expert, record in zip(sel, records):
                host_store.put(layer, expert, record)
                count += 1
    return count


def fill_pool(store: SafetensorsStore, pool, layer: int, slots: Optional[Sequence[int]] = None,
              prefix: str = DEFAULT_PREFIX, chunk: int = 64) -> np.ndarray:
    """Write every expert of ``layer`` into pool slots (``slots[e]``, default the
    lowest free slots) and map them: a resident layer, no LRU traffic."""
    n_experts, hidden, inter = layer_dims(store, layer, prefix, pool.layout.group_size)
    if (hidden, inter) != (pool.layout.hidden, pool.layout.inter):
        raise ValueError(f"layer {layer} is {hidden}/{inter}, the pool holds "
                         f"{pool.layout.hidden}/{pool.layout.inter}")
    if slots is None:
        slots = sorted(pool._free)[:n_experts]
    slots = np.asarray(slots, dtype=np.int64)
    if slots.size != n_experts:
        raise ValueError(f"layer {layer} needs {n_experts} free slots")
    staging = torch.empty((chunk, pool.layout.record_stride), dtype=torch.uint8, pin_memory=True)
    for sel, records in _records(store, pool.layout, layer, range(n_experts), prefix, chunk):
        staging[:len(sel)].copy_(torch.from_numpy(records))
        for i, expert in enumerate(sel):
            pool.record(int(slots[expert])).copy_(staging[i], non_blocking=False)
    pool.place_all(layer, slots)
    pool.sync_tables()
    return slots


def _bf16_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def _projection(store, base: str, device, lead: bool):
    from .executor import Q4G32Projection

    parts = []
    for part in PART_NAMES:
        arr = store.tensor(f"{base}.{part}")
        if lead and arr.ndim == 2:
            arr = arr[None]
        if part == "weight":
            if arr.dtype != np.uint32:
                raise ValueError(f"{base}.weight must be U32")
            parts.append(torch.from_numpy(np.ascontiguousarray(arr).view(np.int32)).to(device))
        else:
            if store.dtype(f"{base}.{part}") != "BF16":
                raise ValueError(f"{base}.{part} must be BF16")
            parts.append(_bf16_tensor(arr, device))
    return Q4G32Projection(*parts)


def load_layer(store: SafetensorsStore, layer: int, top_k: int, device, *, pool=None, host_store=None,
               resident: bool = False, dense: bool = False, prefix: str = DEFAULT_PREFIX,
               router_bias: Optional[np.ndarray] = None):
    """A ``MoELayer`` for one checkpoint layer: the router (``gate.weight``),
    the shared expert and its gate when present, and routed experts that are
    dense device arrays (``dense``), resident pool records (``resident``) or
    pool records filled on demand from ``host_store``."""
    from .layer import HipSwitchGLU, MoELayer, QuantizedMLP, RouterLinear

    n_experts, hidden, inter = layer_dims(store, layer, prefix)
    base = layer_prefix(layer, prefix)
    router = store.tensor(f"{base}.gate.weight")
    if store.dtype(f"{base}.gate.weight") != "BF16" or router.shape != (n_experts, hidden):
        raise ValueError(f"{base}.gate.weight must be BF16 [{n_experts}, {hidden}]")
    bias = None if router_bias is None else torch.from_numpy(np.asarray(router_bias, np.float32)).to(device)
    gate = RouterLinear(_bf16_tensor(router, device), bias)
    if dense:
        projections = {proj: _projection(store, f"{base}.switch_mlp.{proj}", device, False) for proj in PROJECTIONS}
        switch = HipSwitchGLU(hidden, inter, n_experts, projections=projections, layer_id=layer)
    else:
        if pool is None:
            raise ValueError("a pool-backed layer needs an ExpertPool")
        if resident:
            fill_pool(store, pool, layer, prefix=prefix)
        elif host_store is None:
            raise ValueError("a non-resident pool layer needs a host record store")
        switch = HipSwitchGLU(hidden, inter, n_experts, pool=pool, layer_id=layer, host_store=host_store)
    shared = shared_gate = None
    if f"{base}.shared_expert.gate_proj.weight" in store:
        shared = QuantizedMLP(*(_projection(store, f"{base}.shared_expert.{proj}", device, True)
                                for proj in PROJECTIONS))
        shared_gate = _projection(store, f"{base}.shared_expert_gate", device, True)
    return MoELayer(gate, switch, top_k, shared_expert=shared, shared_expert_gate=shared_gate, layer_id=layer)


# ---------------------------------------------------------- safetensors ---

def write_safetensors(path: str, tensors: Mapping[str, Tuple[str, np.ndarray]],
                      metadata: Optional[Mapping[str, str]] = None) -> None:
    """Write ``{name: (dtype, array)}`` as one safetensors file (bf16 given as
    uint16 bit patterns).  Data in name order, 8-byte aligned header."""
    header, blobs, offset = {}, [], 0
    for name in sorted(tensors):
        dtype, array = tensors[name]
        array = np.ascontiguousarray(array)
        if array.dtype.itemsize != DTYPES[dtype].itemsize:
            raise ValueError(f"{name}: {array.dtype} does not hold {dtype}")
        raw = array.tobytes()
        header[name] = {"dtype": dtype, "shape": list(array.shape), "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    if metadata:
        header["__metadata__"] = dict(metadata)
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as handle:
        handle.write(struct.pack("<Q", len(text)))
        handle.write(text)
        for blob in blobs:
            handle.write(blob)


def write_index(model_dir: str, weight_map: Mapping[str, str]) -> None:
    with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as handle:
        json.dump({"metadata": {}, "weight_map": dict(sorted(weight_map.items()))}, handle)


def layer_tensors(layer_np: Mapping, layer: int, prefix: str = DEFAULT_PREFIX) -> Dict[str, Tuple[str, np.ndarray]]:
    """The checkpoint tensors of one layer given in the oracle's layer form
    (``synth.numpy_layer(..., materialise=True)``)."""
    base = layer_prefix(layer, prefix)
    out = {f"{base}.gate.weight": ("BF16", np.asarray(layer_np["router"], np.uint16))}
    for proj in PROJECTIONS:
        for part, arr in zip(PART_NAMES, layer_np[proj]):
            out[f"{base}.switch_mlp.{proj}.{part}"] = ("U32" if part == "weight" else "BF16", np.asarray(arr))
    if "shared_gate_proj" in layer_np:
        for proj in PROJECTIONS:
            for part, arr in zip(PART_NAMES, layer_np[f"shared_{proj}"]):
                out[f"{base}.shared_expert.{proj}.{part}"] = ("U32" if part == "weight" else "BF16", np.asarray(arr)[0])
        for part, arr in zip(PART_NAMES, layer_np["shared_expert_gate"]):
            out[f"{base}.shared_expert_gate.{part}"] = ("U32" if part == "weight" else "BF16", np.asarray(arr)[0])
    return out


# ------------------------------------------------------------ slab pack ---

def write_slab_pack(store: SafetensorsStore, allocation: Mapping[int, Sequence[int]], path: str,
                    layout: RecordLayout, model_hash: bytes = b"\x00" * 8, prefix: str = DEFAULT_PREFIX) -> int:
    """The reference's slab pack: header, directory of (layer, expert, slot) in
    sorted-layer order, then one record per entry.  Returns the file size."""
    ordered = [(layer, int(expert)) for layer in sorted(allocation) for expert in allocation[layer]]
    if len(ordered) > PACK_MAX_ENTRIES:
        raise ValueError(f"Slab pack directory requires {len(ordered)} entries, but the {PACK_HEADER_SIZE}-byte "
                         f"header supports only {PACK_MAX_ENTRIES}")
    if layout.record_stride >= 2 ** 32:
        raise ValueError("record stride does not fit the pack header")
    header = bytearray(PACK_HEADER_SIZE)
    struct.pack_into("<IIIII8sI", header, 0, PACK_MAGIC, PACK_VERSION, len(ordered), layout.record_stride,
                     PACK_HEADER_SIZE, bytes(model_hash)[:8].ljust(8, b"\x00"), 0)
    for slot, (layer, expert) in enumerate(ordered):
        struct.pack_into("<HHI", header, PACK_DIRECTORY_OFFSET + slot * PACK_ENTRY_SIZE, layer, expert, slot)
    tmp = f"{path}.tmp"
    record = np.zeros(layout.record_stride, dtype=np.uint8)
    with open(tmp, "wb") as handle:
        handle.write(header)
        for layer, expert in ordered:
            handle.write(pack_expert(store, layer, expert, layout, record, prefix).tobytes())
    os.replace(tmp, path)
    return PACK_HEADER_SIZE + len(ordered) * layout.record_stride


class SlabPackFile:
    """A slab pack opened read-only: header checks, directory, record views."""

    def __init__(self, path: str, layout: RecordLayout, expected_model_hash: Optional[bytes] = None):
        self.path = path
        self.layout = layout
        size = os.path.getsize(path)
        if size < PACK_HEADER_SIZE:
            raise ValueError(f"Slab pack {path} is truncated: got {size} bytes, expected at least {PACK_HEADER_SIZE}")
        with open(path, "rb") as handle:
            header = handle.read(PACK_HEADER_SIZE)
        magic, version, count, stride, header_size, model_hash, reserved = struct.unpack_from("<IIIII8sI", header, 0)
        if magic != PACK_MAGIC:
            raise ValueError(f"Invalid slab pack header in {path}")
        if version != PACK_VERSION or reserved != 0:
            raise ValueError(f"Slab pack layout version {version} does not match expected {PACK_VERSION} in {path}")
        if stride != layout.record_stride:
            raise ValueError(f"Unsupported record stride {stride} in {path}")
        if header_size != PACK_HEADER_SIZE:
            raise ValueError(f"Unsupported header size {header_size} in {path}, expected {PACK_HEADER_SIZE}")
        if expected_model_hash is not None and model_hash != bytes(expected_model_hash)[:8].ljust(8, b"\x00"):
            raise ValueError(f"Slab pack model identity does not match checkpoint in {path}")
        if count > PACK_MAX_ENTRIES:
            raise ValueError(f"Slab pack directory has {count} entries in {path}, but the {PACK_HEADER_SIZE}-byte "
                             f"header supports only {PACK_MAX_ENTRIES}")
        if size != PACK_HEADER_SIZE + count * stride:
            raise ValueError(f"Invalid slab pack size in {path}: got {size} bytes, expected "
                             f"{PACK_HEADER_SIZE + count * stride} from header")
        self.model_hash = model_hash
        self.expert_count = count
        self.layer_to_base_slot: Dict[int, int] = {}
        self.layer_expert_to_slot: Dict[Tuple[int, int], int] = {}
        seen = set()
        for i in range(count):
            layer, expert, slot = struct.unpack_from("<HHI", header, PACK_DIRECTORY_OFFSET + i * PACK_ENTRY_SIZE)
            if slot >= count:
                raise ValueError(f"Invalid slab pack directory slot {slot} in {path}: expected a value below {count}")
            if slot in seen:
                raise ValueError(f"Duplicate slab pack directory slot {slot} in {path}")
            if (layer, expert) in self.layer_expert_to_slot:
                raise ValueError(f"Duplicate slab pack directory expert {(layer, expert)} in {path}")
            seen.add(slot)
            self.layer_to_base_slot.setdefault(layer, slot)
            self.layer_expert_to_slot[(layer, expert)] = slot
        self.records = np.memmap(path, dtype=np.uint8, mode="r", offset=PACK_HEADER_SIZE, shape=(count, stride)) \
            if count else np.zeros((0, stride), dtype=np.uint8)

    def record(self, layer: int, expert: int) -> np.ndarray:
        return self.records[self.layer_expert_to_slot[(int(layer), int(expert))]]

    def to_host_store(self, host_store=None):
        """Copy every record into a pinned ``HostRecordStore`` (row = pack slot)."""
        from .pool import HostRecordStore

        if host_store is None:
            host_store = HostRecordStore(self.layout, max(1, self.expert_count))
        if host_store.capacity < self.expert_count or host_store.layout.record_stride != self.layout.record_stride:
            raise ValueError("host record store cannot hold this pack")
        chunk = 64
        for start in range(0, self.expert_count, chunk):
            end = min(self.expert_count, start + chunk)
            host_store.buffer[start:end].copy_(torch.from_numpy(np.array(self.records[start:end])))
        for key, slot in self.layer_expert_to_slot.items():
            host_store.alias(*key, slot)
        return host_store


__all__ = ["DEFAULT_PREFIX", "SafetensorsStore", "SlabPackFile", "TensorRef", "expert_tensor", "fill_host_store",
           "fill_pool", "layer_dims", "layer_tensors", "load_layer", "pack_expert", "read_header", "write_index",
           "write_safetensors", "write_slab_pack"]
