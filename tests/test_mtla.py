""""MTLA" binary model files of the C ABI (BinaryModelLoader, Model.swift:401-679), host-only.
Files are built byte by byte here with `struct` and checksummed with `zlib.crc32` (the same
reflected 0xEDB88320 CRC-32), independently of the library's writer; the cases follow the
reference's ModelLoaderTests.swift."""
import struct
import zlib

import numpy as np
import pytest

from metalaudio_amd import nn

RNG = np.random.default_rng(33)
MAGIC = 0x4D544C41


def entries(tensors):
    """Entry bytes for name -> array, in the order given."""
    out = b""
    for name, a in tensors.items():
        a = np.asarray(a, np.float32)
        nb = name.encode() if isinstance(name, str) else name
        out += struct.pack("<4I", len(nb), a.ndim, 0, a.nbytes) + nb
        out += struct.pack(f"<{a.ndim}I", *a.shape) + a.tobytes()
    return out


def v2(tensors, count=None, body=None):
    body = entries(tensors) if body is None else body
    n = len(tensors) if count is None else count
    return struct.pack("<5I", MAGIC, 2, n, zlib.crc32(body), 0) + body


def test_crc32_matches_zlib_on_known_answer(tmp_path):
    # The standard CRC-32 check value: crc32("123456789") = 0xCBF43926.
    assert zlib.crc32(b"123456789") == 0xCBF43926
    w = {"x": np.array([1.0, 2.0], np.float32)}
    # The library's writer stores the checksum zlib computes over the entries.
    p = tmp_path / "m.bin"
    nn.BinaryModelFile.save(w, p)
    assert struct.unpack_from("<I", p.read_bytes(), 12)[0] == zlib.crc32(entries(w))


def test_save_writes_the_reference_layout_byte_for_byte(tmp_path):
    """save (Model.swift:625-679): version 2, tensors sorted by name, CRC over the entries."""
    t = {"zeta": RNG.standard_normal((2, 3)).astype(np.float32),
         "alpha": RNG.standard_normal(5).astype(np.float32),
         "mid.é": RNG.standard_normal((1, 2, 2)).astype(np.float32)}
    p = tmp_path / "m.bin"
    nn.BinaryModelFile.save(t, p)
    ordered = {k: t[k] for k in sorted(t, key=lambda s: s.encode())}
    assert p.read_bytes() == v2(ordered)


def test_round_trip_multiple_tensors(tmp_path):
    t = {"conv.weight": RNG.standard_normal((8, 4, 3)).astype(np.float32),
         "conv.bias": RNG.standard_normal(8).astype(np.float32),
         "empty": np.zeros((0, 5), np.float32),
         "scalar_like": np.array([3.5], np.float32)}
    p = tmp_path / "m.bin"
    nn.BinaryModelFile.save(t, p)
    m = nn.BinaryModelFile(p)
    assert m.names == sorted(t)
    for k, v in t.items():
        got = m.load_tensor(k)
        assert got.shape == v.shape
        np.testing.assert_array_equal(got, v)


def test_empty_dict_round_trip(tmp_path):
    p = tmp_path / "e.bin"
    nn.BinaryModelFile.save({}, p)
    assert p.read_bytes() == struct.pack("<5I", MAGIC, 2, 0, zlib.crc32(b""), 0)
    assert nn.BinaryModelFile(p).names == []


def test_reads_handcrafted_v2_and_legacy_v1(tmp_path):
    a = np.array([1.0, 2.0], np.float32)
    p = tmp_path / "v2.bin"
    p.write_bytes(v2({"test": a}))
    np.testing.assert_array_equal(nn.BinaryModelFile(p).load_tensor("test"), a)
    # testLoadLegacyV1File: 16-byte header (magic, 1, count, reserved), no checksum.
    p1 = tmp_path / "v1.bin"
    p1.write_bytes(struct.pack("<4I", MAGIC, 1, 1, 0) + entries({"test": a}))
    np.testing.assert_array_equal(nn.BinaryModelFile(p1).load_tensor("test"), a)


def bad_file(case, tmp_path):
    a = np.array([1.0, 2.0], np.float32)
    p = tmp_path / "bad.bin"
    if case == "missing":
        return tmp_path / "absent.bin"
    if case == "magic":
        p.write_bytes(struct.pack("<5I", 0x12345678, 2, 0, 0, 0))
    elif case == "too_small":
        p.write_bytes(struct.pack("<2I", MAGIC, 2))
    elif case == "v2_header_short":
        p.write_bytes(struct.pack("<4I", MAGIC, 2, 0, 0))
    elif case == "version":
        p.write_bytes(struct.pack("<5I", MAGIC, 99, 0, 0, 0))
    elif case == "checksum":
        raw = bytearray(v2({"test": a}))
        raw[25] ^= 0xFF
        p.write_bytes(bytes(raw))
    elif case == "trunc_entry_header":
        body = struct.pack("<2I", 4, 1)
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "trunc_data":
        body = entries({"test": a})[:-4]
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "bad_utf8":
        body = struct.pack("<4I", 4, 1, 0, 8) + bytes([0xFF, 0xFE, 0xFF, 0xFE])
        body += struct.pack("<I", 2) + a.tobytes()
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "size_mismatch":
        body = struct.pack("<4I", 4, 1, 0, 12) + b"test" + struct.pack("<I", 2) + a.tobytes()
        body += b"\x00" * 4
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "long_name":
        name = b"n" * 1024
        body = struct.pack("<4I", len(name), 1, 0, 8) + name + struct.pack("<I", 2) + a.tobytes()
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "rank":
        body = struct.pack("<4I", 1, 17, 0, 4) + b"t" + struct.pack("<17I", *([1] * 17))
        body += a[:1].tobytes()
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "overflow":
        body = struct.pack("<4I", 1, 3, 0, 0) + b"t" + struct.pack("<3I", 0xFFFFFFFF, 0xFFFFFFFF,
                                                                   0xFFFFFFFF)
        p.write_bytes(v2({}, count=1, body=body))
    elif case == "count_over":
        p.write_bytes(v2({"test": a}, count=2))
    return p


@pytest.mark.parametrize("case,code", [
    ("missing", 13), ("magic", 14), ("too_small", 14), ("v2_header_short", 14), ("version", 14),
    ("checksum", 14), ("trunc_entry_header", 14), ("trunc_data", 14), ("bad_utf8", 14),
    ("size_mismatch", 14), ("long_name", 14), ("rank", 1), ("overflow", 14), ("count_over", 14),
])
def test_error_paths(tmp_path, case, code):
    """ModelLoaderError cases (Model.swift:369-399, 466-622)."""
    with pytest.raises(nn.MNNError) as e:
        nn.BinaryModelFile(bad_file(case, tmp_path))
    assert e.value.code == code


def test_name_of_1023_bytes_is_accepted(tmp_path):
    name = "n" * 1023
    a = np.array([4.0], np.float32)
    p = tmp_path / "n.bin"
    p.write_bytes(v2({name: a}))
    m = nn.BinaryModelFile(p)
    assert m.names == [name]
    np.testing.assert_array_equal(m.load_tensor(name), a)


def test_missing_tensor_and_wrong_count(tmp_path):
    p = tmp_path / "m.bin"
    p.write_bytes(v2({"t": np.arange(4, dtype=np.float32)}))
    m = nn.BinaryModelFile(p)
    with pytest.raises(nn.MNNError) as e:
        m.load_tensor("u")
    assert e.value.code == 15
    import ctypes as C
    from metalaudio_amd._lib import check, lib
    out = np.empty(3, np.float32)
    with pytest.raises(nn.MNNError) as e:
        check(lib().mnn_mtla_read_f32(m.handle, b"t", out.ctypes.data_as(C.POINTER(C.c_float)), 3))
    assert e.value.code == 2
