"""GGUF reading through the C ABI (rt_hip_gguf_*), no GPU needed.

Restates the reference's reader tests (tests/test_gguf.cpp:69-140: header,
metadata and tensor-info round trip; bad magic and version; type sizes) on
files written by tests/gguf_writer.py, plus what a mapped reader must
survive: every truncation of a valid file and corrupt counts or lengths
fail with RT_HIP_E_FORMAT, never a crash or an out-of-range read.
"""
import struct

import numpy as np
import pytest

from conftest import load_package
from gguf_writer import (ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, T_BF16, T_F16, T_F32, T_Q4_0, T_Q4_K,
                         T_Q5_K, T_Q6_K, T_Q8_0, U8, U16, U32, U64, GgufWriter)

E_ARG, E_SHAPE, E_UNSUPPORTED, E_FORMAT = 1, 2, 6, 7


@pytest.fixture(scope="module")
def rt():
    return load_package().rt_hip


def _open_status(rt, path):
    lib = rt.library()
    import ctypes as C
    h = C.c_void_p()
    st = lib.status("rt_hip_gguf_open", str(path).encode(), C.byref(h))
    if st == 0:
        lib.lib.rt_hip_gguf_close(h)
    return st, lib.lib.rt_hip_last_error().decode()


def test_header_metadata_and_tensor_info_round_trip(rt, tmp_path):
    """test_gguf.cpp:69-108: a gemma3-style header with one F32 [3, 2] tensor."""
    vals = np.arange(6, dtype=np.float32) * 0.5 - 1.0
    w = (GgufWriter()
         .add("general.architecture", STR, "gemma3")
         .add("general.file_type", U32, 15)
         .add("gemma3.attention.layer_norm_rms_epsilon", F32, 1e-6)
         .add("tokenizer.ggml.tokens", ARR, (STR, ["<s>", "hello", "world"]))
         .add_tensor("w", [3, 2], T_F32, vals.tobytes()))
    f = rt.GgufFile(w.write(str(tmp_path / "a.gguf")))
    assert len(f) == 1
    assert f.meta_str("general.architecture") == "gemma3"
    assert f.meta_u64("general.file_type") == 15
    assert f.meta_f32("gemma3.attention.layer_norm_rms_epsilon") == np.float32(1e-6)
    assert f.meta_array_len("tokenizer.ggml.tokens") == 3
    assert f.meta_str("tokenizer.ggml.tokens", 1) == "hello"
    assert f.find("w") == 0 and f.find("nope") == -1
    info = f.info(0)
    assert info["name"] == "w" and info["dims"] == [3, 2] and info["type"] == T_F32
    assert info["n_elements"] == 6 and info["bytes"] == 24
    assert np.array_equal(f.read(0).view(np.float32), vals)
    assert f.linear_shape(0) == (2, 3)  # GGUF [in, out] -> weight [out, in]
    f.close()


def test_every_metadata_type(rt, tmp_path):
    w = (GgufWriter()
         .add("u8", U8, 250).add("i8", I8, -5).add("u16", U16, 65000).add("i16", I16, -30000)
         .add("u32", U32, 4000000000).add("i32", I32, -7).add("f32", F32, 2.5).add("b", BOOL, True)
         .add("u64", U64, 1 << 60).add("i64", I64, -(1 << 40)).add("f64", F64, 0.125)
         .add("nested", ARR, (ARR, [(I32, [1, 2]), (I32, [3])]))
         .add("empty", ARR, (U8, [])))
    f = rt.GgufFile(w.write(str(tmp_path / "m.gguf")))
    # the reference's as_u64 set (gguf.cpp:104-112): u8, u16, u32, u64, i32, i64
    assert f.meta_u64("u8") == 250 and f.meta_u64("u16") == 65000 and f.meta_u64("u32") == 4000000000
    assert f.meta_u64("i32") == (-7) % (1 << 64) and f.meta_u64("i64") == (-(1 << 40)) % (1 << 64)
    assert f.meta_u64("u64") == 1 << 60
    assert f.meta_f32("f32") == 2.5 and f.meta_f32("f64") == 0.125
    assert f.meta_array_len("nested") == 2 and f.meta_array_len("empty") == 0
    lib = rt.library()
    import ctypes as C
    v = C.c_uint64()
    for key in (b"i8", b"i16", b"b", b"f32", b"nested"):
        assert lib.status("rt_hip_gguf_meta_u64", f.h, key, -1, C.byref(v)) == E_UNSUPPORTED, key
    assert lib.status("rt_hip_gguf_meta_u64", f.h, b"missing", -1, C.byref(v)) == E_ARG
    assert lib.status("rt_hip_gguf_meta_u64", f.h, b"nested", 5, C.byref(v)) == E_ARG
    f.close()


def test_rejects_bad_magic_and_version(rt, tmp_path):
    """test_gguf.cpp:110-123."""
    w = GgufWriter().add("general.architecture", STR, "x")
    st, msg = _open_status(rt, w.write(str(tmp_path / "bad.gguf"), magic=b"GGUX"))
    assert st == E_FORMAT and "not a GGUF file" in msg
    for v in (1, 4):
        st, msg = _open_status(rt, w.write(str(tmp_path / f"v{v}.gguf"), version=v))
        assert st == E_FORMAT and "unsupported GGUF version" in msg
    assert _open_status(rt, w.write(str(tmp_path / "v2.gguf"), version=2))[0] == 0
    st, msg = _open_status(rt, tmp_path / "absent.gguf")
    assert st == E_FORMAT and "cannot open" in msg


def test_type_sizes(rt):
    """test_gguf.cpp:125-139 (gguf_byte_size)."""
    tb = rt.library().lib.rt_hip_gguf_type_bytes
    assert tb(T_F32, 10) == 40 and tb(T_F16, 10) == 20 and tb(T_BF16, 10) == 20
    assert tb(T_Q4_0, 32) == 18 and tb(T_Q8_0, 32) == 34
    assert tb(T_Q4_K, 256) == 144 and tb(T_Q5_K, 256) == 176 and tb(T_Q6_K, 256) == 210
    assert tb(T_Q4_K, 257) == 288
    assert tb(9999, 32) == -1 and tb(3, 32) == -1  # unknown / unsized types


def test_alignment_and_offsets(rt, tmp_path):
    a = np.arange(5, dtype=np.float32)
    b = np.arange(7, dtype=np.float32) + 100
    for align in (32, 64, 256):
        w = (GgufWriter(alignment=align).add("general.alignment", U32, align)
             .add_tensor("a", [5], T_F32, a.tobytes()).add_tensor("b", [7], T_F32, b.tobytes()))
        f = rt.GgufFile(w.write(str(tmp_path / f"al{align}.gguf")))
        ia, ib = f.info(0), f.info(1)
        assert ia["file_offset"] % align == 0 and ib["file_offset"] % align == 0
        assert np.array_equal(f.read(0).view(np.float32), a)
        assert np.array_equal(f.read(1).view(np.float32), b)
        assert f.linear_shape(0) == (1, 5)
        f.close()


def test_every_truncation_fails_cleanly(rt, tmp_path):
    q4k = np.random.default_rng(0).integers(0, 256, size=2 * 144, dtype=np.uint8)
    w = (GgufWriter().add("general.architecture", STR, "llama")
         .add("tokens", ARR, (STR, ["a", "bb", "ccc"]))
         .add_tensor("blk.0.ffn_up.weight", [256, 2], T_Q4_K, q4k.tobytes()))
    data = w.to_bytes()
    assert _open_status(rt, w.write(str(tmp_path / "full.gguf")))[0] == 0
    p = tmp_path / "cut.gguf"
    for n in range(0, len(data)):
        p.write_bytes(data[:n])
        st, _ = _open_status(rt, p)
        assert st == E_FORMAT, n


def test_corrupt_counts_and_lengths(rt, tmp_path):
    good = GgufWriter().add("k", STR, "v").to_bytes()
    p = tmp_path / "c.gguf"
    # n_kv far beyond the file
    p.write_bytes(good[:16] + struct.pack("<Q", 1 << 40) + good[24:])
    assert _open_status(rt, p)[0] == E_FORMAT
    # a key length beyond the file
    p.write_bytes(good[:24] + struct.pack("<Q", 1 << 50) + good[32:])
    assert _open_status(rt, p)[0] == E_FORMAT
    # an unknown value type
    bad = bytearray(good)
    key_end = 24 + 8 + 1
    bad[key_end:key_end + 4] = struct.pack("<I", 77)
    p.write_bytes(bytes(bad))
    assert _open_status(rt, p)[0] == E_FORMAT
    # a tensor whose data lies past the end of the file
    w = GgufWriter().add_tensor("t", [1024], T_F32, np.zeros(1024, np.float32).tobytes())
    p.write_bytes(w.to_bytes()[:-16])
    st, msg = _open_status(rt, p)
    assert st == E_FORMAT and "past the end" in msg
    # rank 0 and rank 5
    for rank in (0, 5):
        w = GgufWriter().add_tensor("t", [2] * rank, T_F32, b"")
        p.write_bytes(w.to_bytes())
        assert _open_status(rt, p)[0] == E_FORMAT, rank


def test_unsized_types_and_linear_shape_errors(rt, tmp_path):
    w = (GgufWriter().add_tensor("q5_1", [32], 7, b"\0" * 24)
         .add_tensor("cube", [2, 2, 2], T_F32, np.zeros(8, np.float32).tobytes()))
    f = rt.GgufFile(w.write(str(tmp_path / "u.gguf")))
    assert f.info(0)["bytes"] == -1 and f.info(0)["file_offset"] == -1
    lib = rt.library()
    import ctypes as C
    buf = (C.c_uint8 * 64)()
    assert lib.status("rt_hip_gguf_read_tensor", f.h, 0, buf, 24) == E_UNSUPPORTED
    assert lib.status("rt_hip_gguf_read_tensor", f.h, 1, buf, 16) == E_ARG  # wrong size
    r, c = C.c_int64(), C.c_int64()
    assert lib.status("rt_hip_gguf_linear_shape", f.h, 1, C.byref(r), C.byref(c)) == E_SHAPE
    assert lib.status("rt_hip_gguf_tensor_info", f.h, 9, None) == E_ARG
    f.close()
