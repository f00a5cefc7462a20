"""GGUF reader / writer / slicer (CPU).  The parser must not repeat
gguf_parser.h's faults: missing block sizes for Q8_0 / Q2_K / Q3_K (wrong
per-expert strides), wrong metadata skip sizes (bool 8, uint64 1, int64 and
float64 not skipped) and a hard-wired 32-byte data alignment."""
import struct

import numpy as np
import pytest

from winmoe_amd import gguf
from winmoe_amd.gguf import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, STRING, UINT8, UINT16, UINT32,
                             UINT64, GGUFError, GGUFFile, Value, expert_slice, tensor_nbytes, write_gguf)


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def test_hand_built_file(tmp_path):
    """A file assembled byte by byte here (not by write_gguf): a bool, a uint64,
    an int64 and a float64 before the key that follows them, an array of
    strings, a Q8_0 tensor and an F32 tensor after the 32-byte-aligned header."""
    kv = [
        ("a.flag", struct.pack("<I", BOOL) + struct.pack("<?", True)),
        ("a.big", struct.pack("<I", UINT64) + struct.pack("<Q", 2 ** 40 + 7)),
        ("a.neg", struct.pack("<I", INT64) + struct.pack("<q", -5)),
        ("a.pi", struct.pack("<I", FLOAT64) + struct.pack("<d", 3.25)),
        ("a.names", struct.pack("<I", ARRAY) + struct.pack("<IQ", STRING, 2) + _s("x") + _s("yz")),
        ("general.architecture", struct.pack("<I", STRING) + _s("winmoe")),
    ]
    q8 = bytes(range(34)) * 4               # 4 Q8_0 blocks: [64, 2]
    f32 = struct.pack("<3f", 1.0, -2.0, 0.5)
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(kv))
    for k, v in kv:
        head += _s(k) + v
    head += _s("t.q8") + struct.pack("<I", 2) + struct.pack("<QQ", 64, 2) + struct.pack("<IQ", 8, 0)
    head += _s("t.f32") + struct.pack("<I", 1) + struct.pack("<Q", 3) + struct.pack("<IQ", 0, 160)
    pad = (-len(head)) % 32
    body = q8 + b"\0" * (160 - len(q8)) + f32
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + b"\0" * pad + body)

    g = GGUFFile(str(p))
    assert g.kv["a.flag"] is True
    assert g.kv["a.big"] == 2 ** 40 + 7
    assert g.kv["a.neg"] == -5
    assert g.kv["a.pi"] == 3.25
    assert g.kv["a.names"] == ["x", "yz"]
    assert g.arch() == "winmoe"
    t = g.find("t.q8")
    assert t.dims == (64, 2) and t.ggml_type == 8 and t.nbytes == 136
    assert bytes(g.data("t.q8")) == q8
    assert np.frombuffer(bytes(g.data("t.f32")), np.float32).tolist() == [1.0, -2.0, 0.5]
    assert g.find("absent") is None


@pytest.mark.parametrize("gt,be,bb", [(8, 32, 34), (10, 256, 84), (11, 256, 110), (12, 256, 144), (13, 256, 176),
                                      (14, 256, 210), (0, 1, 4), (1, 1, 2), (30, 1, 2)])
def test_block_sizes(gt, be, bb):
    assert tensor_nbytes((be * 3, 5), gt) == 15 * bb
    with pytest.raises(GGUFError):
        tensor_nbytes((be * 3 + 1, 5), gt) if be > 1 else tensor_nbytes((1, 1), 999)


def _all_values():
    return {
        "u8": Value(UINT8, 200), "i8": Value(INT8, -100), "u16": Value(UINT16, 60000), "i16": Value(INT16, -30000),
        "u32": Value(UINT32, 4000000000), "i32": Value(INT32, -2000000000), "f32": Value(FLOAT32, 0.5),
        "b": Value(BOOL, False), "s": Value(STRING, "héllo"), "u64": Value(UINT64, 2 ** 63 + 1),
        "i64": Value(INT64, -(2 ** 62)), "f64": Value(FLOAT64, -1.5e300),
        "arr_i32": Value(ARRAY, [1, -2, 3], INT32),
        "arr_nested": Value(ARRAY, [Value(ARRAY, [1, 2], UINT8), Value(ARRAY, ["a"], STRING)], ARRAY),
        "after": Value(UINT32, 7),
    }


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    tensors = []
    for name, dims, gt in [("a", (64, 3), 8), ("b", (256, 2, 3), 10), ("c", (512,), 11), ("d", (256, 4), 14),
                           ("e", (7,), 0), ("f", (256, 1), 12)]:
        n = tensor_nbytes(dims, gt)
        tensors.append((name, dims, gt, rng.integers(0, 256, n, dtype=np.uint8).tobytes()))
    p = str(tmp_path / "rt.gguf")
    write_gguf(p, _all_values(), tensors, alignment=alignment)
    g = GGUFFile(p)
    assert g.alignment == alignment
    for k, v in _all_values().items():
        if k == "arr_nested":
            got = g.kv_typed[k]
            assert [x.value for x in got.value] == [[1, 2], ["a"]]
        elif v.type == FLOAT32:
            assert g.kv[k] == pytest.approx(v.value)
        else:
            assert g.kv[k] == v.value, k
        assert g.kv_typed[k].type == v.type
    for name, dims, gt, data in tensors:
        t = g.find(name)
        assert t.dims == tuple(dims) and t.ggml_type == gt and t.offset % alignment == 0
        assert bytes(g.data(name)) == data
    # the data section starts on the alignment boundary
    assert g._data_start[0] % alignment == 0


def test_expert_slices(tmp_path):
    """Per-expert stride = nbytes / E for a stacked Q8_0 / Q2_K tensor (the
    reference's parser gets n*4 bytes for these types)."""
    H, I, E = 256, 8, 5
    rng = np.random.default_rng(1)
    per = {}
    tensors = []
    for name, gt in [("blk.0.ffn_gate_exps.weight", 8), ("blk.0.ffn_down_exps.weight", 10)]:
        dims = (H, I, E) if "gate" in name else (256, H // 32, E)
        experts = [rng.integers(0, 256, tensor_nbytes(dims[:2], gt), dtype=np.uint8).tobytes() for _ in range(E)]
        per[name] = experts
        tensors.append((name, dims, gt, b"".join(experts)))
    p = str(tmp_path / "ex.gguf")
    write_gguf(p, {"general.architecture": "winmoe"}, tensors)
    g = GGUFFile(p)
    for name, experts in per.items():
        assert g.find(name).nbytes == sum(len(x) for x in experts)
        for e in range(E):
            assert bytes(expert_slice(g, name, e)) == experts[e]
    with pytest.raises(IndexError):
        expert_slice(g, "blk.0.ffn_gate_exps.weight", E)


def test_split_shards(tmp_path):
    rng = np.random.default_rng(2)
    a = rng.integers(0, 256, 34 * 2, dtype=np.uint8).tobytes()
    b = rng.integers(0, 256, 84, dtype=np.uint8).tobytes()
    base = str(tmp_path / "m")
    write_gguf(f"{base}-00001-of-00002.gguf", {"split.no": Value(UINT16, 0), "split.count": Value(UINT16, 2),
                                              "general.architecture": "winmoe"}, [("x", (64,), 8, a)])
    write_gguf(f"{base}-00002-of-00002.gguf", {"split.no": Value(UINT16, 1), "split.count": Value(UINT16, 2)},
               [("y", (256,), 10, b)])
    g = GGUFFile(f"{base}-00001-of-00002.gguf")
    assert bytes(g.data("x")) == a and bytes(g.data("y")) == b
    assert g.find("y").shard == 1 and g.arch() == "winmoe"


def test_errors(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML" + b"\0" * 28)
    with pytest.raises(GGUFError):
        GGUFFile(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    with pytest.raises(GGUFError):
        GGUFFile(str(p))
    good = str(tmp_path / "g.gguf")
    write_gguf(good, {"k": "v"}, [("t", (64,), 8, bytes(68))])
    raw = open(good, "rb").read()
    p.write_bytes(raw[:-10])                       # tensor runs past the end
    with pytest.raises(GGUFError):
        GGUFFile(str(p))
    p.write_bytes(raw[:20])                        # header cut short
    with pytest.raises(GGUFError):
        GGUFFile(str(p))
    # a tensor offset off the alignment
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + _s("t") + struct.pack("<IQIQ", 1, 64, 8, 8)
    p.write_bytes(head + b"\0" * ((-len(head)) % 32) + bytes(128))
    with pytest.raises(GGUFError):
        GGUFFile(str(p))
    with pytest.raises(GGUFError):
        write_gguf(str(p), {}, [("t", (64,), 8, bytes(10))])
