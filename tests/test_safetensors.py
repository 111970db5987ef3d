"""SafeTensors reader of the C ABI (SafeTensorsLoader.swift:41-660), host-only: handcrafted files
and files written by the `safetensors` package, conversions, metadata and every error path of the
reference's LoaderError."""
import json
import struct

import numpy as np
import pytest

from metalaudio_amd import nn

RNG = np.random.default_rng(21)


def write_st(path, tensors, metadata=None, header_override=None, pad_data=b""):
    """tensors: name -> (dtype string, shape, raw bytes). Offsets follow the order given."""
    header, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata is not None:
        header["__metadata__"] = metadata
    h = header_override if header_override is not None else json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs) + pad_data)
    return path


def test_reads_every_dtype(tmp_path):
    f32 = RNG.standard_normal((3, 4)).astype(np.float32)
    f16 = np.array([0.0, -0.0, 1.5, -2.25, 6.1e-5, 5.96e-8, 65504.0, 1e-7], np.float16)
    bf = RNG.standard_normal(6).astype(np.float32)
    bf16_bits = (bf.view(np.uint32) >> 16).astype(np.uint16)
    i64 = np.array([-3, 0, 7, 1 << 40], np.int64)
    i32 = np.array([-5, 9], np.int32)
    i16 = np.array([-300, 12], np.int16)
    i8 = np.array([-128, 127], np.int8)
    u8 = np.array([0, 255], np.uint8)
    bl = np.array([0, 1, 2], np.uint8)
    p = write_st(tmp_path / "all.safetensors", {
        "a.f32": ("F32", f32.shape, f32.tobytes()), "b.f16": ("F16", f16.shape, f16.tobytes()),
        "c.bf16": ("BF16", bf.shape, bf16_bits.tobytes()), "d.i64": ("I64", i64.shape, i64.tobytes()),
        "e.i32": ("I32", i32.shape, i32.tobytes()), "f.i16": ("I16", i16.shape, i16.tobytes()),
        "g.i8": ("I8", i8.shape, i8.tobytes()), "h.u8": ("U8", u8.shape, u8.tobytes()),
        "i.bool": ("BOOL", bl.shape, bl.tobytes())}, metadata={"format": "pt", "note": "xé"})
    st = nn.SafeTensors(p)
    assert st.available_tensors == sorted(["a.f32", "b.f16", "c.bf16", "d.i64", "e.i32", "f.i16",
                                           "g.i8", "h.u8", "i.bool"])
    assert st.tensor_info("a.f32") == ("F32", (3, 4), 12)
    np.testing.assert_array_equal(st.load_tensor("a.f32"), f32)
    np.testing.assert_array_equal(st.load_tensor("b.f16"), f16.astype(np.float32))
    np.testing.assert_array_equal(st.load_tensor("c.bf16"),
                                  (bf16_bits.astype(np.uint32) << 16).view(np.float32))
    np.testing.assert_array_equal(st.load_tensor("d.i64"), i64.astype(np.float32))
    np.testing.assert_array_equal(st.load_tensor("e.i32"), i32.astype(np.float32))
    np.testing.assert_array_equal(st.load_tensor("f.i16"), i16.astype(np.float32))
    np.testing.assert_array_equal(st.load_tensor("g.i8"), i8.astype(np.float32))
    np.testing.assert_array_equal(st.load_tensor("h.u8"), u8.astype(np.float32))
    np.testing.assert_array_equal(st.load_tensor("i.bool"), [0.0, 1.0, 1.0])
    assert st.metadata("format") == "pt" and st.metadata("note") == "xé"
    with pytest.raises(nn.MNNError) as e:
        st.metadata("absent")
    assert e.value.code == 15


def test_half_conversion_is_exact_for_every_finite_half(tmp_path):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    h = bits.view(np.float16)
    keep = np.isfinite(h)
    p = write_st(tmp_path / "h.safetensors", {"h": ("F16", (int(keep.sum()),),
                                                   h[keep].tobytes())})
    np.testing.assert_array_equal(nn.SafeTensors(p).load_tensor("h"), h[keep].astype(np.float32))


def test_matches_the_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    t = {"enc.0.conv.weight": RNG.standard_normal((48, 2, 8)).astype(np.float32),
         "enc.0.conv.bias": RNG.standard_normal(48).astype(np.float32),
         "enc.0.norm.weight": np.ones(48, np.float16)}
    save_file(t, str(tmp_path / "m.safetensors"), metadata={"k": "v"})
    st = nn.SafeTensors(tmp_path / "m.safetensors")
    assert st.available_tensors == sorted(t)
    for k, v in t.items():
        np.testing.assert_array_equal(st.load_tensor(k), v.astype(np.float32))
        assert st.tensor_info(k)[1] == v.shape
    assert st.metadata("k") == "v"


def test_skips_malformed_entries_and_unknown_dtypes(tmp_path):
    good = np.arange(4, dtype=np.float32)
    hdr = {"good": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]},
           "bad_dtype": {"dtype": "C64", "shape": [1], "data_offsets": [0, 8]},
           "no_offsets": {"dtype": "F32", "shape": [1]},
           "neg": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}
    p = write_st(tmp_path / "s.safetensors", {"good": ("F32", (4,), good.tobytes())},
                 header_override=json.dumps(hdr).encode())
    st = nn.SafeTensors(p)
    assert st.available_tensors == ["good"]
    np.testing.assert_array_equal(st.load_tensor("good"), good)


@pytest.mark.parametrize("case,code", [
    ("missing", 13), ("short", 14), ("too_large", 14), ("truncated_header", 14), ("bad_json", 14),
    ("not_utf8", 14), ("offset_oob", 14), ("reversed", 14), ("ragged", 14), ("nan", 1), ("inf", 1),
    ("not_found", 15), ("count", 2),
])
def test_error_paths(tmp_path, case, code):
    """LoaderError cases (SafeTensorsLoader.swift:95-128) and the NaN/Inf check
    (validateWeights, :624-658)."""
    p = tmp_path / "e.safetensors"
    ok = np.arange(4, dtype=np.float32)
    name = "t"
    if case == "missing":
        p = tmp_path / "absent.safetensors"
    elif case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "too_large":
        p.write_bytes(struct.pack("<Q", 200 * 1024 * 1024) + b"{}")
    elif case == "truncated_header":
        p.write_bytes(struct.pack("<Q", 100) + b"{}")
    elif case == "bad_json":
        write_st(p, {}, header_override=b'{"t": {"dtype": "F32",')
    elif case == "not_utf8":
        write_st(p, {}, header_override=b'{"\xff": 1}')
    elif case == "offset_oob":
        write_st(p, {"t": ("F32", (4,), ok.tobytes())},
                 header_override=json.dumps({"t": {"dtype": "F32", "shape": [4],
                                                   "data_offsets": [0, 64]}}).encode())
    elif case == "reversed":  # end < begin: INVALID_FILE, not a huge allocation
        write_st(p, {"t": ("F32", (4,), ok.tobytes())},
                 header_override=json.dumps({"t": {"dtype": "F32", "shape": [4],
                                                   "data_offsets": [16, 0]}}).encode())
    elif case == "ragged":
        write_st(p, {"t": ("F32", (1,), b"\x00\x00\x80")})
    elif case in ("nan", "inf"):
        bad = ok.copy()
        bad[2] = np.nan if case == "nan" else np.inf
        write_st(p, {"t": ("F32", (4,), bad.tobytes())})
    elif case in ("not_found", "count"):
        write_st(p, {"t": ("F32", (4,), ok.tobytes())})
        name = "u" if case == "not_found" else "t"
    with pytest.raises(nn.MNNError) as e:
        st = nn.SafeTensors(p)
        if case == "count":
            out = np.empty(3, np.float32)
            from metalaudio_amd._lib import check, lib
            import ctypes as C
            check(lib().mnn_safetensors_read_f32(st.handle, b"t",
                                                 out.ctypes.data_as(C.POINTER(C.c_float)), 3))
        st.load_tensor(name)
    assert e.value.code == code
