"""GGUF container reader/writer (CPU), after eredu-gguf/tests/container.rs:
every metadata type in versions 1-3 and both byte orders, alignment, the
metadata-only file, deterministic output, every raw type's checked size,
truncations as errors, and the header validations of reader.rs:616-790."""
import io
import struct

import pytest

from eredu_amd import EreduError
from eredu_amd import gguf_file as F

M = F.MetadataValue


def metadata():
    return {
        "a.u8": M(0, 255), "b.i8": M(1, -3), "c.u16": M(2, 500), "d.i16": M(3, -500), "e.u32": M(4, 90000),
        "f.i32": M(5, -90000), "g.f32": M(6, 1.25), "h.bool": M(7, True), "i.string": M(8, "héllo"),
        "j.u64": M(10, 2**32 + 1), "k.i64": M(11, -9_000_000_000), "l.f64": M(12, -2.5),
        "m.array": M.array(3, [-1, 0, 2]),
        "n.nested": M.array(9, [M.array(8, ["x"]), M.array(8, ["y", "z"])]),
        "o.empty": M.array(0, []), "p.au8": M.array(0, [0, 255]), "q.ai8": M.array(1, [-1, 2]),
        "r.au16": M.array(2, [1, 500]), "s.au32": M.array(4, [1, 90000]), "t.ai32": M.array(5, [-1, 90000]),
        "u.af32": M.array(6, [-1.5, 2.25]), "v.abool": M.array(7, [False, True]),
        "w.au64": M.array(10, [1, 2**64 - 1]), "x.ai64": M.array(11, [-(2**63), 1]),
        "y.af64": M.array(12, [-1.5, 2.25]),
    }


def file(version, endian, alignment):
    dense = struct.pack("<f" if endian == "little" else ">f", 1.5)
    out = io.BytesIO()
    F.write_gguf(out, metadata(), [("dense", [1], F.F32, dense), ("zero", [0], F.F16, b""),
                                   ("raw.weight", [64], F.Q4_0, bytes(36))],
                 version=version, endian=endian, alignment=alignment)
    return out.getvalue()


@pytest.mark.parametrize("version", [1, 2, 3])
@pytest.mark.parametrize("endian", ["little", "big"])
def test_versions_endian_metadata_dense_and_alignment(version, endian):
    r = F.GgufReader(file(version, endian, 64))
    assert r.version == version and r.endian == endian and r.alignment == 64
    expected = metadata()
    expected["general.alignment"] = M(4, 64)
    assert r.metadata == expected
    assert len(r.tensors) == 3 and all(t.data_offset % 64 == 0 for t in r.tensors)
    assert r.read_raw(r.tensors[0]) == struct.pack("<f" if endian == "little" else ">f", 1.5)
    assert r.tensors[2].byte_len == 36 and r.tensors[1].byte_len == 0


def test_metadata_only_file_needs_no_tensor_padding():
    r = F.GgufReader(b"GGUF" + struct.pack("<IQQ", 3, 0, 0))
    assert r.tensors == [] and r.metadata == {}


def test_deterministic_and_raw_quantized_roundtrip():
    a, b = file(3, "little", 32), file(3, "little", 32)
    assert a == b
    r = F.GgufReader(a)
    assert r.read_raw(r.tensors[2]) == bytes(36)


def test_every_supported_raw_type_has_checked_size():
    for ty in (F.Q4_0, 3, 6, 7, F.Q8_0, 10, 11, F.Q4_K, 13, 14):
        block, nbytes = F.BLOCK_GEOMETRY[ty]
        data = bytes(range(nbytes % 256)) + bytes(nbytes - nbytes % 256)
        out = io.BytesIO()
        F.write_gguf(out, {}, [("x.weight", [block], ty, data)])
        r = F.GgufReader(out.getvalue())
        assert r.read_raw(r.tensors[0]) == data


def test_all_truncations_are_errors():
    bytes_ = file(3, "little", 32)
    for n in range(len(bytes_)):
        with pytest.raises(EreduError):
            F.GgufReader(bytes_[:n])


def _header(n_tensors, meta=b"", n_meta=0, tensors=b""):
    return b"GGUF" + struct.pack("<IQQ", 3, n_tensors, n_meta) + meta + tensors


def _tensor(name, dims, ty, off):
    nb = name.encode()
    return struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)) + b"".join(
        struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)


def test_header_validations():
    with pytest.raises(EreduError, match="magic"):
        F.GgufReader(b"GGUX" + bytes(20))
    with pytest.raises(EreduError, match="version"):
        F.GgufReader(b"GGUF" + struct.pack("<IQQ", 4, 0, 0))
    body = _tensor("a", [32], F.Q4_0, 0) + _tensor("a", [32], F.Q4_0, 32)
    with pytest.raises(EreduError, match="duplicate tensor"):
        F.GgufReader(_header(2, tensors=body) + bytes(200))
    with pytest.raises(EreduError, match="not aligned"):
        F.GgufReader(_header(1, tensors=_tensor("a", [32], F.Q4_0, 8)) + bytes(200))
    with pytest.raises(EreduError, match="divisible by block"):
        F.GgufReader(_header(1, tensors=_tensor("a", [48], F.Q4_0, 0)) + bytes(200))
    with pytest.raises(EreduError, match="exceeds file size"):
        F.GgufReader(_header(1, tensors=_tensor("a", [32 * 100], F.Q4_0, 0)) + bytes(64))
    body = _tensor("a", [64], F.Q4_0, 0) + _tensor("b", [32], F.Q4_0, 32)  # a is 36 bytes: overlaps b
    with pytest.raises(EreduError, match="overlaps"):
        F.GgufReader(_header(2, tensors=body) + bytes(200))
    with pytest.raises(EreduError, match="unsupported GGML type"):
        F.GgufReader(_header(1, tensors=_tensor("a", [32], 99, 0)) + bytes(200))
    key = b"general.alignment"
    meta = struct.pack("<Q", len(key)) + key + struct.pack("<II", 4, 48)
    with pytest.raises(EreduError, match="invalid alignment"):
        F.GgufReader(_header(0, meta, 1))
    meta = struct.pack("<Q", len(key)) + key + struct.pack("<I", 8) + struct.pack("<Q", 2) + b"32"
    with pytest.raises(EreduError, match="uint32 or uint64"):
        F.GgufReader(_header(0, meta, 1))


def test_writer_validations():
    with pytest.raises(EreduError, match="payload"):
        F.write_gguf(io.BytesIO(), {}, [("a", [32], F.Q4_0, bytes(17))])
    with pytest.raises(EreduError, match="alignment"):
        F.write_gguf(io.BytesIO(), {"general.alignment": M(4, 64)}, [], alignment=32)
    with pytest.raises(EreduError, match="version"):
        F.write_gguf(io.BytesIO(), {}, [], version=4)
