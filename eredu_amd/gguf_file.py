"""GGUF container I/O and streaming load onto the GPU.

``GgufReader`` parses a GGUF header the way eredu-gguf's ``Reader`` does
(eredu-gguf/src/reader.rs:616-790): magic ``GGUF`` (little-endian) or
``FUGG`` (big-endian), versions 1-3 (u32 counts in v1, u64 after), typed
metadata with nested arrays, ``general.alignment`` (u32/u64, a power of two,
default 32), tensor descriptors whose data starts at the aligned end of the
header, each offset aligned, shapes divisible by the GGML block, ranges
inside the file and not overlapping.  ``write_gguf`` is the deterministic
writer of eredu-gguf/src/writer.rs (test inputs, conversion output).

``stream_convert`` streams a checkpoint onto the GPU (the role of
eredu-gguf/src/catalog.rs:435-660's converted-tensor iteration): the
raw blocks of each tensor go file -> pinned host buffer -> HBM on a copy
stream while the previous tensor is converted on the compute stream (two
pinned staging buffers, ordered by events), so file reads, PCIe copies and
conversion overlap.  Tensors are routed as eredu routes them
(eredu-gguf/src/convert.rs:125-140): little-endian Q4_K / Q5_K / Q6_K /
Q5_1 / Q8_0 stay in their blocks (executed by the native linear), Q4_0,
Q4_1, Q5_0, Q2_K, Q3_K and big-endian blocks are expanded to the MLX affine
triple by ``eq_gguf_convert_affine``, dense tensors are copied as they are.  ``stream_convert_affine`` expands every
quantized tensor (the explicit convert_affine of portable backends).
"""
from __future__ import annotations

import dataclasses
import io
import os
import struct
from typing import BinaryIO, Dict, Iterable, List, Optional, Sequence, Tuple, Union

from ._native import EreduError

DEFAULT_ALIGNMENT = 32

# GGML type code -> (values per block, bytes per block), eredu-gguf/src/format.rs:368-400
BLOCK_GEOMETRY: Dict[int, Tuple[int, int]] = {
    0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
    2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
    16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110),
    22: (256, 82), 23: (256, 136), 29: (256, 56), 39: (32, 17),
}
F32, F16, BF16, Q4_0, Q8_0, Q4_K = 0, 1, 30, 2, 8, 12

# metadata value type codes (GGUF spec): scalar struct formats
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 10: "Q", 11: "q", 12: "d"}
T_BOOL, T_STRING, T_ARRAY = 7, 8, 9


@dataclasses.dataclass(frozen=True)
class MetadataValue:
    """A typed metadata value: ``type`` is the GGUF code; arrays carry
    ``elem_type`` and a tuple of values (nested arrays as MetadataValue)."""

    type: int
    value: object
    elem_type: Optional[int] = None

    @staticmethod
    def array(elem_type: int, values: Sequence) -> "MetadataValue":
        return MetadataValue(T_ARRAY, tuple(values), elem_type)


@dataclasses.dataclass(frozen=True)
class TensorInfo:
    name: str
    dimensions: Tuple[int, ...]  # GGUF order: innermost first
    ggml_type: int
    relative_offset: int
    data_offset: int
    byte_len: int

    @property
    def mlx_shape(self) -> Tuple[int, ...]:
        return tuple(reversed(self.dimensions))


def _geometry(name: str, ggml_type: int) -> Tuple[int, int]:
    if ggml_type not in BLOCK_GEOMETRY:
        raise EreduError(f"tensor {name!r}: unsupported GGML type {ggml_type}")
    return BLOCK_GEOMETRY[ggml_type]


def _align_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


class _Parser:
    def __init__(self, f: BinaryIO, size: int):
        self.f, self.size, self.e, self.version = f, size, "<", 0

    def exact(self, n: int) -> bytes:
        if n < 0 or self.f.tell() + n > self.size:
            raise EreduError(f"truncated GGUF at offset {self.f.tell()} (need {n} bytes)")
        b = self.f.read(n)
        if len(b) != n:
            raise EreduError(f"truncated GGUF at offset {self.f.tell()}")
        return b

    def scalar(self, fmt: str):
        return struct.unpack(self.e + fmt, self.exact(struct.calcsize(fmt)))[0]

    def count(self) -> int:
        return self.scalar("I" if self.version == 1 else "Q")

    def string(self) -> str:
        n = self.count()
        try:
            return self.exact(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise EreduError(f"invalid UTF-8 string at offset {self.f.tell()}") from e

    def value(self, ty: int, depth: int = 0):
        if ty in _SCALAR:
            return MetadataValue(ty, self.scalar(_SCALAR[ty]))
        if ty == T_BOOL:
            b = self.scalar("B")
            if b > 1:
                raise EreduError(f"invalid boolean {b}")
            return MetadataValue(ty, bool(b))
        if ty == T_STRING:
            return MetadataValue(ty, self.string())
        if ty == T_ARRAY:
            if depth > 8:
                raise EreduError("metadata nesting too deep")
            et = self.scalar("I")
            n = self.count()
            if n > self.size:
                raise EreduError(f"metadata array of {n} elements exceeds the file")
            vals = [self.value(et, depth + 1) for _ in range(n)]
            return MetadataValue.array(et, [v if et == T_ARRAY else v.value for v in vals])
        raise EreduError(f"unsupported metadata type {ty}")


class GgufReader:
    """Validated GGUF header and payload access (eredu-gguf/src/reader.rs:600-840)."""

    def __init__(self, source: Union[str, bytes, BinaryIO]):
        if isinstance(source, (bytes, bytearray)):
            self._f: BinaryIO = io.BytesIO(bytes(source))
        elif isinstance(source, str):
            self._f = open(source, "rb")
        else:
            self._f = source
        f = self._f
        f.seek(0, os.SEEK_END)
        size = f.tell()
        f.seek(0)
        p = _Parser(f, size)
        magic = p.exact(4)
        if magic == b"GGUF":
            p.e, self.endian = "<", "little"
        elif magic == b"FUGG":
            p.e, self.endian = ">", "big"
        else:
            raise EreduError(f"invalid magic {magic!r}")
        self.version = p.version = p.scalar("I")
        if not 1 <= self.version <= 3:
            raise EreduError(f"unsupported GGUF version {self.version}")
        n_tensors, n_meta = p.count(), p.count()
        if n_tensors > size or n_meta > size:
            raise EreduError("tensor or metadata count exceeds the file")
        self.metadata: Dict[str, MetadataValue] = {}
        for _ in range(n_meta):
            key = p.string()
            if len(key) > 65535 or not key.isascii():
                raise EreduError(f"metadata key {key!r}: keys must be ASCII and at most 65535 bytes")
            v = p.value(p.scalar("I"))
            if key in self.metadata:
                raise EreduError(f"duplicate metadata key {key!r}")
            self.metadata[key] = v
        a = self.metadata.get("general.alignment")
        if a is None:
            self.alignment = DEFAULT_ALIGNMENT
        elif a.type in (4, 10):
            self.alignment = int(a.value)
        else:
            raise EreduError("general.alignment must be uint32 or uint64")
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise EreduError(f"invalid alignment {self.alignment}")
        raw = []
        names = set()
        for _ in range(n_tensors):
            name = p.string()
            if not name:
                raise EreduError("empty tensor name")
            if name in names:
                raise EreduError(f"duplicate tensor {name!r}")
            names.add(name)
            rank = p.scalar("I")
            if rank > 8:
                raise EreduError(f"tensor {name!r}: rank {rank} exceeds 8")
            dims = tuple(p.count() for _ in range(rank))
            raw.append((name, dims, p.scalar("I"), p.scalar("Q")))
        data_start = _align_up(f.tell(), self.alignment)
        if n_tensors and data_start > size:
            raise EreduError("tensor data starts beyond end of file")
        self.tensors: List[TensorInfo] = []
        for name, dims, ty, rel in raw:
            if rel % self.alignment:
                raise EreduError(f"tensor {name!r}: relative offset {rel} is not aligned to {self.alignment}")
            elements = 1
            for d in dims:
                elements *= d
            block, nbytes = _geometry(name, ty)
            if elements and ((dims[0] if dims else 1) % block or elements % block):
                raise EreduError(f"tensor {name!r}: shape {list(dims)} is not divisible by block size {block}")
            byte_len = elements // block * nbytes
            off = data_start + rel
            if off + byte_len > size:
                raise EreduError(f"tensor {name!r}: data range {off}..{off + byte_len} exceeds file size {size}")
            self.tensors.append(TensorInfo(name, dims, ty, rel, off, byte_len))
        ranges = sorted((t.data_offset, t.data_offset + t.byte_len, t.name) for t in self.tensors if t.byte_len)
        for (a0, a1, an), (b0, b1, bn) in zip(ranges, ranges[1:]):
            if a1 > b0:
                raise EreduError(f"tensor {bn!r}: data overlaps tensor {an!r}")

    def tensor(self, name: str) -> TensorInfo:
        for t in self.tensors:
            if t.name == name:
                return t
        raise EreduError(f"tensor {name!r} is not present")

    def read_raw(self, t: TensorInfo, out=None):
        """The tensor's payload bytes (into ``out``, a writable buffer of at
        least byte_len bytes, when given)."""
        self._f.seek(t.data_offset)
        if out is None:
            return self._f.read(t.byte_len)
        view = memoryview(out).cast("B")[: t.byte_len]
        got = self._f.readinto(view)
        if got != t.byte_len:
            raise EreduError(f"tensor {t.name!r}: short read")
        return view

    def close(self):
        self._f.close()


class _Enc:
    def __init__(self, out: BinaryIO, e: str, version: int):
        self.out, self.e, self.version = out, e, version

    def scalar(self, fmt, v):
        self.out.write(struct.pack(self.e + fmt, v))

    def count(self, n):
        self.scalar("I" if self.version == 1 else "Q", n)

    def string(self, s: str):
        b = s.encode("utf-8")
        self.count(len(b))
        self.out.write(b)

    def value(self, v: MetadataValue):
        if v.type in _SCALAR:
            self.scalar(_SCALAR[v.type], v.value)
        elif v.type == T_BOOL:
            self.scalar("B", 1 if v.value else 0)
        elif v.type == T_STRING:
            self.string(v.value)
        elif v.type == T_ARRAY:
            self.scalar("I", v.elem_type)
            self.count(len(v.value))
            for x in v.value:
                self.value(x if v.elem_type == T_ARRAY else MetadataValue(v.elem_type, x))
        else:
            raise EreduError(f"unsupported metadata type {v.type}")


def write_gguf(out: BinaryIO, metadata: Dict[str, MetadataValue],
               tensors: Iterable[Tuple[str, Sequence[int], int, bytes]], version: int = 3,
               endian: str = "little", alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Deterministic GGUF writer (eredu-gguf/src/writer.rs:50-200): keys in
    sorted order, ``general.alignment`` added when it is not the default,
    tensor payloads at aligned offsets.  ``tensors``: (name, GGUF dimensions,
    GGML type, payload bytes, already in the file's byte order)."""
    if not 1 <= version <= 3:
        raise EreduError(f"unsupported GGUF version {version}")
    if alignment <= 0 or alignment & (alignment - 1):
        raise EreduError(f"invalid alignment {alignment}")
    meta = dict(metadata)
    a = meta.get("general.alignment")
    if a is None:
        if alignment != DEFAULT_ALIGNMENT:
            meta["general.alignment"] = MetadataValue(4 if alignment < 2**32 else 10, alignment)
    elif a.type not in (4, 10) or a.value != alignment:
        raise EreduError("general.alignment does not match writer alignment")
    tensors = list(tensors)
    names, offsets, nxt = set(), [], 0
    for name, dims, ty, data in tensors:
        if not name:
            raise EreduError("empty tensor name")
        if name in names:
            raise EreduError(f"duplicate tensor {name!r}")
        names.add(name)
        elements = 1
        for d in dims:
            elements *= d
        block, nbytes = _geometry(name, ty)
        if elements and ((dims[0] if dims else 1) % block or elements % block):
            raise EreduError(f"tensor {name!r}: shape is not divisible by block size {block}")
        if elements // block * nbytes != len(data):
            raise EreduError(f"tensor {name!r}: payload has {len(data)} bytes, expected {elements // block * nbytes}")
        nxt = _align_up(nxt, alignment)
        offsets.append(nxt)
        nxt += len(data)
    e = "<" if endian == "little" else ">"
    out.write(b"GGUF" if endian == "little" else b"FUGG")
    enc = _Enc(out, e, version)
    enc.scalar("I", version)
    enc.count(len(tensors))
    enc.count(len(meta))
    for k in sorted(meta):
        if len(k) > 65535 or not k.isascii():
            raise EreduError(f"metadata key {k!r} must be ASCII and at most 65535 bytes")
        enc.string(k)
        enc.scalar("I", meta[k].type)
        enc.value(meta[k])
    for (name, dims, ty, _), off in zip(tensors, offsets):
        enc.string(name)
        enc.scalar("I", len(dims))
        for d in dims:
            enc.count(d)
        enc.scalar("I", ty)
        enc.scalar("Q", off)
    start = out.tell()
    data_start = _align_up(start, alignment)
    if tensors:
        out.write(b"\0" * (data_start - start))
    for (name, dims, ty, data), off in zip(tensors, offsets):
        pos = out.tell() - data_start
        out.write(b"\0" * (off - pos))
        out.write(data)


def stream_convert(path: str, names: Optional[Sequence[str]] = None, staging_bytes: int = 256 << 20):
    """Loads a GGUF file's tensors into HBM, converting each on the GPU as it
    arrives the way eredu loads a checkpoint (eredu-gguf/src/convert.rs:276-313
    routed by conversion_kind, :125-140; safemlx/src/ops/gguf.rs:421-528):

    * dense F32 / F16 / BF16 (and the integer dense types) -> ``gguf.DenseTensor``,
    * little-endian Q4_K / Q5_K / Q6_K / Q5_1 / Q8_0 -> ``gguf.NativeTensor``
      (blocks kept as stored, executed by the native linear),
    * MXFP4 (type 39) -> ``gguf.MxFp4Tensor`` (E2M1 codes + E8M0 scale bytes),
    * Q4_0, Q4_1, Q5_0, Q2_K, Q3_K, and big-endian blocks of the native
      types -> ``gguf.AffineTensor``.

    Returns {name: tensor}.  Two pinned staging buffers of ``staging_bytes``
    alternate: while tensor i is copied to the device and converted, tensor
    i + 1 is read from the file into the other buffer; events order each
    buffer's reuse after its copy.  A tensor larger than a buffer goes
    through in buffer-sized pieces."""
    from . import gguf as G

    return _stream(path, names, staging_bytes, lambda desc, raw, endian: G.convert(desc, raw, endian), True)


def stream_convert_affine(path: str, names: Optional[Sequence[str]] = None, staging_bytes: int = 256 << 20):
    """stream_convert with every quantized tensor of an affine type (Q4_0,
    Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K) expanded to the MLX
    affine triple (the explicit eredu_gguf::convert_affine, convert.rs:318-564,
    which portable backends use); dense tensors as in stream_convert.  Returns
    {name: AffineTensor | torch.Tensor (dense)}."""
    from . import gguf as G

    def conv(desc, raw, endian):
        if G.conversion_kind(desc.ggml_type, endian).kind == "dense":
            return G.convert(desc, raw, endian).array
        return G.convert_affine(desc, raw, endian)

    return _stream(path, names, staging_bytes, conv)


def _stream(path: str, names: Optional[Sequence[str]], staging_bytes: int, conv, mxfp4: bool = False):
    import torch

    from . import gguf as G

    reader = GgufReader(path)
    endian = G.Endian.Big if reader.endian == "big" else G.Endian.Little
    wanted = [t for t in reader.tensors if names is None or t.name in set(names)]
    if names is not None:
        missing = set(names) - {t.name for t in wanted}
        if missing:
            raise EreduError(f"tensors not present: {sorted(missing)}")
    for t in wanted:  # refuse before anything is read
        ty = G.ggml_type_from_code(t.ggml_type)
        kind = G.conversion_kind(ty, endian)
        if kind.kind != "dense" and not ty.has_device_kernels() and not (mxfp4 and kind.kind == "mxfp4"):
            raise EreduError(f"tensor {t.name!r}: GGML type {t.ggml_type} has no device conversion")
    dev = torch.device("cuda")
    copy_stream = torch.cuda.Stream()
    compute = torch.cuda.current_stream()
    cap = max(staging_bytes, 1)
    pinned = [torch.empty(cap, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    freed = [torch.cuda.Event(), torch.cuda.Event()]
    for ev in freed:
        ev.record(copy_stream)
    out: Dict[str, object] = {}
    slot = 0
    try:
        for t in wanted:
            # allocated on the copy stream that fills it; record_stream below
            # keeps the allocator from handing it to a later copy while the
            # conversion on the compute stream still reads it
            with torch.cuda.stream(copy_stream):
                raw_dev = torch.empty(t.byte_len, dtype=torch.uint8, device=dev)
            done = 0
            while done < t.byte_len:
                n = min(cap, t.byte_len - done)
                freed[slot].synchronize()  # the buffer's previous copy has finished
                reader._f.seek(t.data_offset + done)
                got = reader._f.readinto(memoryview(pinned[slot].numpy())[:n])
                if got != n:
                    raise EreduError(f"tensor {t.name!r}: short read")
                with torch.cuda.stream(copy_stream):
                    raw_dev[done:done + n].copy_(pinned[slot][:n], non_blocking=True)
                    freed[slot].record(copy_stream)
                done += n
                slot ^= 1
            compute.wait_stream(copy_stream)
            raw_dev.record_stream(compute)
            desc = G.TensorDescriptor(t.name, list(t.dimensions), G.ggml_type_from_code(t.ggml_type), t.byte_len)
            out[t.name] = conv(desc, raw_dev, endian)
        torch.cuda.synchronize()
    finally:
        reader.close()
    return out
