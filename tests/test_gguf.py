"""GGUF ingest (include/rxq4_gguf.h) on the CPU: files written by
tests/gguf_writer.py from the GGUF specification are parsed back field for
field; broken files (every truncation point, wrong magic/version/endianness,
bad types, shapes, offsets, alignment, duplicates, random corruption) return
an error status and never crash.  The device copy is tested in
tests/test_gpu_gguf.py.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import rxq4
from rxq4 import gguf
from tests import gguf_writer as gw
from tests import util

META = [
    ("general.architecture", gw.STRING, "qwen3"),
    ("general.alignment", gw.UINT32, 64),
    ("t.u8", gw.UINT8, 250), ("t.i8", gw.INT8, -5), ("t.u16", gw.UINT16, 65000),
    ("t.i16", gw.INT16, -30000), ("t.u32", gw.UINT32, 4_000_000_000), ("t.i32", gw.INT32, -7),
    ("t.f32", gw.FLOAT32, 1.5), ("t.bool", gw.BOOL, True), ("t.u64", gw.UINT64, 2**62),
    ("t.i64", gw.INT64, -2**40), ("t.f64", gw.FLOAT64, -0.125), ("t.empty", gw.STRING, ""),
    ("t.utf8", gw.STRING, "ünïcødé"),
    ("t.arr_i32", gw.ARRAY, [1, -2, 3], gw.INT32),
    ("t.arr_f32", gw.ARRAY, [0.5, 2.0], gw.FLOAT32),
    ("t.arr_str", gw.ARRAY, ["a", "", "bc", "Ω"], gw.STRING),
    ("t.arr_none", gw.ARRAY, [], gw.UINT8),
]


def model_tensors():
    """A Q4_K [300 x 512], a Q6_K [7 x 256] (odd byte count), an F32 norm
    vector and an F16 matrix, in that order."""
    r = util.rng(800)
    q4 = util.weights(801, 300, 512)
    from tests import kquant_blocks as kb
    q6 = kb.random_blocks(14, util.rng(802), 7, 256)
    norm = r.standard_normal(512).astype(np.float32)
    h = r.standard_normal((3, 64)).astype(np.float16)
    return [("blk.0.ffn_up.weight", 12, (512, 300), q4.tobytes()),
            ("blk.0.attn_v.weight", 14, (256, 7), q6.tobytes()),
            ("blk.0.attn_norm.weight", 0, (512,), gw.f32_tensor(norm)),
            ("token_embd.weight", 1, (64, 3), h.tobytes())]


def test_round_trip(tmp_path):
    tens = model_tensors()
    path = tmp_path / "m.gguf"
    gw.write(path, META, tens, alignment=64)
    with gguf.GGUFFile(path) as f:
        assert f.version == 3 and f.alignment == 64
        m = f.metadata
        assert m["general.architecture"] == "qwen3"
        assert (m["t.u8"], m["t.i8"], m["t.u16"], m["t.i16"]) == (250, -5, 65000, -30000)
        assert (m["t.u32"], m["t.i32"], m["t.u64"], m["t.i64"]) == (4_000_000_000, -7, 2**62, -2**40)
        assert m["t.f32"] == 1.5 and m["t.f64"] == -0.125 and m["t.bool"] is True
        assert m["t.empty"] == "" and m["t.utf8"] == "ünïcødé"
        assert m["t.arr_i32"].tolist() == [1, -2, 3] and m["t.arr_i32"].dtype == np.int32
        assert m["t.arr_f32"].tolist() == [0.5, 2.0]
        assert m["t.arr_str"] == ["a", "", "bc", "Ω"]
        assert m["t.arr_none"].size == 0
        assert list(f.tensors) == [t[0] for t in tens]
        for name, gtype, ne, raw in tens:
            t = f.tensors[name]
            assert (t.ggml_type, t.shape, t.nbytes) == (gtype, ne, len(raw))
            assert t.offset % 64 == 0 and t.host % 64 == 0
            assert f.host_array(name).tobytes() == raw
        q4 = f.tensors["blk.0.ffn_up.weight"]
        assert (q4.row_length, q4.rows) == (512, 300)
        last = tens[-1]
        assert f.data_bytes == f.tensors[last[0]].offset + len(last[3])
        L = gguf.lib()
        assert L.rxq4_gguf_find_tensor(f._h, b"blk.0.attn_v.weight") == 1
        assert L.rxq4_gguf_find_tensor(f._h, b"missing") == -1
        assert L.rxq4_gguf_find_kv(f._h, b"t.f64") == 12


def test_version2_default_alignment_and_empty(tmp_path):
    path = tmp_path / "v2.gguf"
    gw.write(path, [("a", gw.UINT32, 1)], [("w", 12, (256, 2), bytes(288))], version=2)
    with gguf.GGUFFile(path) as f:
        assert f.version == 2 and f.alignment == 32
        assert f.tensors["w"].nbytes == 288
    empty = tmp_path / "e.gguf"
    gw.write(empty, [], [])
    with gguf.GGUFFile(empty) as f:
        assert f.tensors == {} and f.metadata == {} and f.data_bytes == 0


def test_block_geometry():
    assert gguf.block_geometry(12) == (256, 144)
    assert gguf.block_geometry(13) == (256, 176)
    assert gguf.block_geometry(14) == (256, 210)
    assert gguf.block_geometry(0) == (1, 4) and gguf.block_geometry(30) == (1, 2)
    assert gguf.block_geometry(8) == (32, 34)
    for t in (4, 5, 31, 32, 33, 36, -1, 1000):
        assert gguf.block_geometry(t) == (0, 0)


def _open_status(path) -> int:
    try:
        gguf.GGUFFile(path).close()
        return rxq4.SUCCESS
    except rxq4.RxQ4Error as e:
        return e.status


BAD = {
    "magic": dict(magic=b"GGML"),
    "v1": dict(version=1),
    "big_endian": dict(version=3 << 24),
    "v4": dict(version=4),
    "offset_unaligned": dict(offsets=[8]),
    "offset_past_end": dict(offsets=[1 << 20]),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_broken_header_fields(tmp_path, case):
    path = tmp_path / "b.gguf"
    gw.write(path, [], [("w", 12, (256, 1), bytes(144))], **BAD[case])
    want = rxq4.UNSUPPORTED_MODEL if case in ("v1", "big_endian", "v4") else rxq4.INVALID_ARGUMENT
    assert _open_status(path) == want


@pytest.mark.parametrize("tensors,kvs,status", [
    ([("w", 77, (256, 1), bytes(144))], [], rxq4.UNSUPPORTED_QUANT_FORMAT),    # unknown type
    ([("w", 12, (100, 1), bytes(144))], [], rxq4.INVALID_ARGUMENT),            # partial block
    ([("w", 0, (1, 1, 1, 1, 1), bytes(4))], [], rxq4.INVALID_ARGUMENT),        # 5 dims
    ([("w", 0, (), b"")], [], rxq4.INVALID_ARGUMENT),                          # 0 dims
    ([("w", 0, (4,), bytes(16)), ("w", 0, (4,), bytes(16))], [], rxq4.INVALID_ARGUMENT),
    ([("w", 0, (1 << 40, 1 << 30), b"")], [], rxq4.INVALID_ARGUMENT),         # too large
    ([], [("general.alignment", gw.UINT32, 48)], rxq4.INVALID_ARGUMENT),      # not a power of 2
    ([], [("general.alignment", gw.UINT64, 32)], rxq4.INVALID_ARGUMENT),      # wrong type
    ([], [("k", gw.UINT8, 1), ("k", gw.UINT8, 2)], rxq4.INVALID_ARGUMENT),    # duplicate key
    ([], [("k", 13, 0)], rxq4.INVALID_ARGUMENT),                              # unknown kv type
])
def test_broken_contents(tmp_path, tensors, kvs, status):
    path = tmp_path / "c.gguf"
    b = gw.build([kv for kv in kvs if kv[1] != 13], tensors,
                 alignment=48 if any(kv[2] == 48 for kv in kvs) else 32)
    if any(kv[1] == 13 for kv in kvs):  # an unknown value type, written by hand
        b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw.gstr("k") + struct.pack("<IB", 13, 0)
    path.write_bytes(b)
    assert _open_status(path) == status


def test_every_truncation_fails_cleanly(tmp_path):
    tens = model_tensors()[1:3]
    full = gw.build(META, tens)
    path = tmp_path / "t.gguf"
    path.write_bytes(full)
    assert _open_status(path) == rxq4.SUCCESS
    last_end = len(full)
    cuts = list(range(0, 600)) + list(range(600, last_end, 97)) + [last_end - 1]
    for n in cuts:
        path.write_bytes(full[:n])
        assert _open_status(path) != rxq4.SUCCESS, n


def test_random_corruption_never_crashes(tmp_path):
    full = bytearray(gw.build(META, model_tensors()[1:3]))
    r = np.random.default_rng(5)
    path = tmp_path / "r.gguf"
    head = 900  # metadata and tensor infos
    for _ in range(400):
        b = bytearray(full)
        for pos in r.integers(0, head, size=r.integers(1, 4)):
            b[pos] = int(r.integers(0, 256))
        path.write_bytes(bytes(b))
        _open_status(path)  # any status; the process must survive
    # huge counts are rejected before anything is sized by them
    b = bytearray(full)
    b[8:16] = struct.pack("<Q", 1 << 60)
    path.write_bytes(bytes(b))
    assert _open_status(path) == rxq4.INVALID_ARGUMENT


def test_missing_file_and_bad_calls(tmp_path):
    assert _open_status(tmp_path / "nope.gguf") == rxq4.INVALID_ARGUMENT
    L = gguf.lib()
    assert L.rxq4_gguf_tensor_info(None, 0, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_gguf_upload(None, None, 0, None) == rxq4.INVALID_ARGUMENT
    path = tmp_path / "s.gguf"
    gw.write(path, [("s", gw.STRING, "x"), ("a", gw.ARRAY, ["p", "q"], gw.STRING)], [])
    with gguf.GGUFFile(path) as f:
        v = gguf.c_int64()
        assert L.rxq4_gguf_kv_int(f._h, 0, gguf.ctypes.byref(v)) == rxq4.INVALID_ARGUMENT
        assert L.rxq4_gguf_kv_int(f._h, 5, gguf.ctypes.byref(v)) == rxq4.INVALID_ARGUMENT
        ptrs = (gguf.c_void_p * 2)()
        lens = (gguf.c_uint64 * 2)()
        assert L.rxq4_gguf_kv_array_strs(f._h, 1, 1, 2, ptrs, lens) == rxq4.INVALID_ARGUMENT
        assert L.rxq4_gguf_kv_array_strs(f._h, 1, 1, 1, ptrs, lens) == rxq4.SUCCESS
        assert gguf.ctypes.string_at(ptrs[0], lens[0]) == b"q"
