"""GGUF v3 reader and packed-expert tensor mapping for the MoE layer.

Host-side: the file is memory-mapped and parsed with ``struct``; tensor bytes
are handed out as zero-copy numpy views of the mapping, and
``moe_layer_from_gguf`` copies a layer's router, packed experts and shared
expert to the GPU once and builds an ``ops.MoELayer`` over them.

Follows the reference reader ``crates/gguf/src/lib.rs``:
- header, metadata and tensor directory: ``GgufFile::open`` (lib.rs:164-294);
- metadata values (13 types, arrays nested at most 8 deep, arrays longer than
  1024 values parsed but not kept): ``read_metadata_value`` (lib.rs:1654-1730);
- ``general.alignment`` (default 32, a multiple of 8): ``metadata_alignment``
  (lib.rs:1821-1832); key rules: ``validate_metadata_key`` (lib.rs:1903-1915);
- a tensor's storage range ends where the next tensor (by offset) or the file
  begins: ``assign_storage_byte_lengths`` (lib.rs:1854-1875);
- layer tensor names: ``crates/model/src/index.rs:417-429``; packed expert
  dims ``[in, out, experts]``: ``crates/model/src/moe_ffn.rs:2385-2410``.
Errors raise ``GGUFError`` where the reference returns ``Error::gguf``.
"""

from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"GGUF"
VERSION = 3
DEFAULT_ALIGNMENT = 32
MAX_TENSOR_DIMS = 4
MAX_KEY_BYTES = 0xFFFF
MAX_TENSOR_NAME_BYTES = 64
MAX_STORED_ARRAY_VALUES = 1024
MAX_METADATA_DEPTH = 8

# ggml tensor type codes and (values per block, bytes per block)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = (
    0, 1, 8, 10, 11, 12, 14, 30)
_BLOCK_NAMES = {10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 14: "Q6_K", 8: "Q8_0"}
BLOCKS = {
    0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
    9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
    15: (256, 292), 30: (1, 2),
}
# metadata value types
(MT_U8, MT_I8, MT_U16, MT_I16, MT_U32, MT_I32, MT_F32, MT_BOOL, MT_STRING, MT_ARRAY, MT_U64,
 MT_I64, MT_F64) = range(13)
_SCALAR = {MT_U8: "<B", MT_I8: "<b", MT_U16: "<H", MT_I16: "<h", MT_U32: "<I", MT_I32: "<i",
           MT_F32: "<f", MT_U64: "<Q", MT_I64: "<q", MT_F64: "<d"}


class GGUFError(ValueError):
    pass


@dataclass
class TensorInfo:
    name: str
    dims: tuple          # ggml order: dims[0] is the row width (fastest)
    ty: int
    relative_offset: int
    absolute_offset: int = 0
    storage_byte_len: int = 0

    @property
    def elements(self) -> int:
        return int(np.prod(self.dims, dtype=np.uint64))

    @property
    def nbytes(self) -> int:
        """Bytes the tensor's blocks occupy (rows of dims[0] values)."""
        if self.ty not in BLOCKS:
            raise GGUFError(f"GGUF tensor {self.name} has unsupported type {self.ty}")
        per, size = BLOCKS[self.ty]
        # block_count_for_quant_block (crates/gguf/src/lib.rs:1877-1900): rows
        # must be whole blocks (first dimension), then the element count
        if per > 1:
            if not self.dims:
                raise GGUFError(f"GGUF tensor {self.name} has no dimensions")
            kind = _BLOCK_NAMES.get(self.ty, f"type {self.ty}")
            if self.dims[0] % per:
                raise GGUFError(f"GGUF tensor {self.name} first dimension {self.dims[0]} is not "
                                f"divisible by {kind} block size {per}")
            if self.elements % per:
                raise GGUFError(f"GGUF tensor {self.name} element count {self.elements} is not "
                                f"divisible by {kind} block size {per}")
        return self.elements // per * size


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n):
        if n < 0 or self.pos + n > len(self.buf):
            raise GGUFError("GGUF file ends inside its header")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def scalar(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self, limit=None):
        n = self.scalar("<Q")
        if limit is not None and n > limit:
            raise GGUFError(f"GGUF string of {n} bytes exceeds the {limit}-byte limit")
        try:
            return bytes(self.take(n)).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError("GGUF string is not valid UTF-8") from e

    def value_type(self):
        t = self.scalar("<I")
        if t > MT_F64:
            raise GGUFError(f"unknown GGUF metadata value type {t}")
        return t

    def value(self, t, store=True, depth=0):
        if depth > MAX_METADATA_DEPTH:
            raise GGUFError("GGUF metadata array nesting is too deep")
        if t in _SCALAR:
            return self.scalar(_SCALAR[t])
        if t == MT_BOOL:
            v = self.scalar("<B")
            if v > 1:
                raise GGUFError(f"invalid GGUF bool value {v}; expected 0 or 1")
            return bool(v)
        if t == MT_STRING:
            if not store:  # skipped unchecked, as skip_string (lib.rs:1741-1746)
                self.take(self.scalar("<Q"))
                return ""
            return self.string()
        et = self.value_type()
        n = self.scalar("<Q")
        keep = store and n <= MAX_STORED_ARRAY_VALUES
        vals = [self.value(et, keep, depth + 1) for _ in range(n)]
        return GGUFArray(et, n, vals if keep else None)


@dataclass
class GGUFArray:
    """A metadata array; ``values`` is None when it held more than 1024 values."""
    element_type: int
    length: int
    values: list | None = field(default=None)


def _check_key(key):
    if not key.isascii():
        raise GGUFError(f"GGUF metadata key {key!r} must be ASCII")
    if not key or key.startswith(".") or key.endswith(".") or ".." in key:
        raise GGUFError(f"GGUF metadata key {key!r} must be hierarchical")


class GGUFFile:
    """A parsed GGUF v3 file, memory-mapped read-only."""

    def __init__(self, path):
        self.path = str(path)
        with open(self.path, "rb") as f:
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse()
        except Exception:
            self.close()  # unmapped now, or once the traceback's views are gone
            raise

    def _parse(self):
        self.file_size = len(self._map)
        r = _Reader(memoryview(self._map))
        if bytes(r.take(4)) != MAGIC:
            raise GGUFError("not a GGUF file (bad magic)")
        self.version = r.scalar("<I")
        if self.version != VERSION:
            raise GGUFError(f"unsupported GGUF version {self.version}; expected {VERSION}")
        self.tensor_count = r.scalar("<Q")
        self.metadata_kv_count = r.scalar("<Q")
        self.metadata = {}
        self.metadata_types = {}
        for _ in range(self.metadata_kv_count):
            key = r.string(MAX_KEY_BYTES)
            _check_key(key)
            t = r.value_type()
            val = r.value(t)
            if key in self.metadata:
                raise GGUFError(f"duplicate GGUF metadata key {key}")
            self.metadata[key] = val
            self.metadata_types[key] = t
        # metadata_alignment (lib.rs:1821-1840): only an unsigned integer value
        # counts; any other type falls back to the default
        al = DEFAULT_ALIGNMENT
        if self.metadata_types.get("general.alignment") in (MT_U8, MT_U16, MT_U32, MT_U64):
            al = self.metadata["general.alignment"]
        if al < 8 or al % 8:
            raise GGUFError(f"GGUF general.alignment must be a multiple of 8 and at least 8, "
                            f"got {al}")
        self.alignment = al
        self.tensors = {}
        for _ in range(self.tensor_count):
            name = r.string(MAX_TENSOR_NAME_BYTES)
            nd = r.scalar("<I")
            if nd == 0:
                raise GGUFError(f"GGUF tensor {name} must have at least one dimension")
            if nd > MAX_TENSOR_DIMS:
                raise GGUFError(f"GGUF tensor {name} has {nd} dimensions; max supported is "
                                f"{MAX_TENSOR_DIMS}")
            dims = tuple(r.scalar("<Q") for _ in range(nd))
            if 0 in dims:
                raise GGUFError(f"GGUF tensor {name} contains a zero dimension")
            ty = r.scalar("<I")
            off = r.scalar("<Q")
            if off % al:
                raise GGUFError(f"GGUF tensor {name} relative offset {off} is not aligned to {al}")
            if name in self.tensors:
                raise GGUFError(f"duplicate GGUF tensor {name}")
            self.tensors[name] = TensorInfo(name, dims, ty, off)
        self.tensor_data_offset = -(-r.pos // al) * al
        for t in self.tensors.values():
            t.absolute_offset = self.tensor_data_offset + t.relative_offset
            if t.absolute_offset > self.file_size:
                raise GGUFError(f"GGUF tensor {t.name} absolute offset {t.absolute_offset} "
                                f"exceeds file size {self.file_size}")
        by_off = sorted(self.tensors.values(), key=lambda t: t.absolute_offset)
        for i, t in enumerate(by_off):
            end = by_off[i + 1].absolute_offset if i + 1 < len(by_off) else self.file_size
            if end <= t.absolute_offset:
                raise GGUFError(f"GGUF tensor {t.name} has invalid storage range "
                                f"[{t.absolute_offset}..{end})")
            t.storage_byte_len = end - t.absolute_offset

    def close(self):
        """Unmaps the file; while views from ``tensor_bytes`` are alive the
        mapping stays open and is released with the last of them."""
        try:
            self._map.close()
        except BufferError:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor(self, name) -> TensorInfo:
        try:
            return self.tensors[name]
        except KeyError:
            raise GGUFError(f"missing GGUF tensor {name}") from None

    def tensor_bytes(self, name) -> np.ndarray:
        """The tensor's blocks as a zero-copy uint8 view of the mapping."""
        t = self.tensor(name)
        n = t.nbytes
        if n > t.storage_byte_len:
            raise GGUFError(f"GGUF tensor {name} needs {n} bytes but its storage range holds "
                            f"{t.storage_byte_len}")
        return np.frombuffer(self._map, dtype=np.uint8, count=n, offset=t.absolute_offset)


# ---------------------------------------------------------------- MoE layer

@dataclass
class PackedExperts:
    """One layer's routed experts: gate/up dims [H, I, E], down [I, H, E]."""
    gate: TensorInfo
    up: TensorInfo
    down: TensorInfo
    hidden: int
    intermediate: int
    experts: int


def _q(t: TensorInfo):
    if t.ty not in (GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0):
        raise GGUFError(f"GGUF tensor {t.name} has type {t.ty}; the MoE kernels take "
                        "Q2_K/Q3_K/Q4_K/Q6_K/Q8_0")
    return t.ty


_SHARED_GU = {GGML_Q8_0, GGML_Q2_K, GGML_Q3_K, GGML_Q4_K}
_SHARED_DOWN = _SHARED_GU | {GGML_Q6_K}


def packed_experts(g: GGUFFile, layer: int) -> PackedExperts:
    """``blk.{layer}.ffn_{gate,up,down}_exps.weight`` (index.rs:426-428) with
    their dims checked against each other (moe_ffn.rs:2385-2410)."""
    p = f"blk.{layer}"
    gate, up, down = (g.tensor(f"{p}.ffn_{m}_exps.weight") for m in ("gate", "up", "down"))
    for t in (gate, up, down):
        if len(t.dims) != 3:
            raise GGUFError(f"GGUF tensor {t.name} must have 3 dims [in, out, experts], "
                            f"has {len(t.dims)}")
        _q(t)
    H, I, E = gate.dims
    if up.dims != gate.dims or up.ty != gate.ty:
        raise GGUFError(f"{up.name} dims/type {up.dims}/{up.ty} differ from {gate.name} "
                        f"{gate.dims}/{gate.ty}")
    if down.dims != (I, H, E):
        raise GGUFError(f"{down.name} dims {down.dims}; expected {(I, H, E)}")
    return PackedExperts(gate, up, down, int(H), int(I), int(E))


def moe_layer_from_gguf(g: GGUFFile, layer: int, *, top_k: int, score_fn: int,
                        norm_topk_prob: bool, routed_scaling_factor: float,
                        device="cuda", max_tokens=1):
    """An ``ops.MoELayer`` over layer ``layer``'s tensors, copied to ``device``:
    router ``ffn_gate_inp.weight`` (f32 [H, E]), optional correction bias
    ``exp_probs_b.bias`` (f32 [E]), packed experts, optional shared
    expert ``ffn_{gate,up,down}_shexp.weight`` (index.rs:417-429): Q8_0, or a
    K-quant gate/up (Laguna XS: Q4_K) with a K-quant or Q8_0 down."""
    import torch

    from . import ops

    px = packed_experts(g, layer)
    H, I, E = px.hidden, px.intermediate, px.experts
    p = f"blk.{layer}"

    def dev(name):
        return torch.from_numpy(g.tensor_bytes(name).copy()).to(device)

    rt = g.tensor(f"{p}.ffn_gate_inp.weight")
    if rt.ty != GGML_F32 or rt.dims != (H, E):
        raise GGUFError(f"{rt.name} must be f32 [{H}, {E}], is type {rt.ty} dims {rt.dims}")
    router = dev(rt.name).view(torch.float32).view(E, H)
    bias = None
    bn = f"{p}.exp_probs_b.bias"
    if bn in g.tensors:
        bt = g.tensors[bn]
        if bt.ty != GGML_F32 or bt.dims != (E,):
            raise GGUFError(f"{bn} must be f32 [{E}], is type {bt.ty} dims {bt.dims}")
        bias = dev(bn).view(torch.float32)
    shared = {}
    Is = 0
    if f"{p}.ffn_gate_shexp.weight" in g.tensors:
        sg, su, sd = (g.tensor(f"{p}.ffn_{m}_shexp.weight") for m in ("gate", "up", "down"))
        Is = int(sg.dims[1])
        # Q8_0 (GLM, Laguna S) or Laguna XS's Q4_K gate/up with a K-quant down
        # (crates/model/src/laguna/gguf_model.rs:829-849)
        for t, want, kinds in ((sg, (H, Is), _SHARED_GU), (su, (H, Is), _SHARED_GU),
                               (sd, (Is, H), _SHARED_DOWN)):
            if t.ty not in kinds or t.dims != want:
                raise GGUFError(f"{t.name} must be {list(want)} of type {sorted(kinds)}, is type "
                                f"{t.ty} dims {list(t.dims)}")
        if su.ty != sg.ty:
            raise GGUFError(f"{su.name} type {su.ty} differs from {sg.name} type {sg.ty}")
        shared = dict(shared_gate=dev(sg.name), shared_up=dev(su.name), shared_down=dev(sd.name),
                      shared_quant=sg.ty, shared_down_quant=sd.ty)
    return ops.MoELayer(
        hidden=H, experts=E, intermediate=I, top_k=top_k, quant=px.gate.ty,
        down_quant=px.down.ty, score_fn=score_fn, norm_topk_prob=norm_topk_prob,
        routed_scaling_factor=routed_scaling_factor, router=router, router_bias=bias,
        gate=dev(px.gate.name), up=dev(px.up.name), down=dev(px.down.name),
        shared_intermediate=Is, max_tokens=max_tokens, **shared)


# ------------------------------------------------------------------ writer

def _pack_value(t, v):
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == MT_BOOL:
        return struct.pack("<B", int(v))
    if t == MT_STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    et, vals = v
    return struct.pack("<IQ", et, len(vals)) + b"".join(_pack_value(et, x) for x in vals)


def write_gguf(path, metadata, tensors, alignment=DEFAULT_ALIGNMENT):
    """Writes a GGUF v3 file. ``metadata``: list of (key, type, value), an
    array value being (element type, list); ``tensors``: list of (name, dims,
    ggml type, bytes). Tensor data is laid out in list order, each start
    aligned to ``alignment``."""
    head = [MAGIC, struct.pack("<IQQ", VERSION, len(tensors), len(metadata))]
    for key, t, v in metadata:
        kb = key.encode("utf-8")
        head += [struct.pack("<Q", len(kb)), kb, struct.pack("<I", t), _pack_value(t, v)]
    off = 0
    offsets = []
    for name, dims, ty, data in tensors:
        nb = name.encode("utf-8")
        head += [struct.pack("<Q", len(nb)), nb, struct.pack("<I", len(dims)),
                 struct.pack(f"<{len(dims)}Q", *dims), struct.pack("<IQ", ty, off)]
        offsets.append(off)
        off = -(-(off + len(data)) // alignment) * alignment
    h = b"".join(head)
    h += b"\0" * (-len(h) % alignment)
    with open(path, "wb") as f:
        f.write(h)
        for (name, dims, ty, data), o in zip(tensors, offsets):
            f.seek(len(h) + o)
            f.write(bytes(data))
