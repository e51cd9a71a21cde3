"""GGUF reader (q27h_gguf_* through the C ABI) against the CPU oracle (oracle/gguf_oracle.py), and the oracle
pinned by a hand-assembled known-answer file. CPU only: parsing never touches the GPU.

The reference ships no GGUF fixtures (its model file is not part of the repository); files here are built by
tests/gguf_writer.py from the public GGUF layout, plus byte-level edits for every error path the reference
reports (src/gguf.cpp:113-194), and every prefix of a valid file (truncation at each byte).
"""
import os
import struct

import numpy as np
import pytest

import gguf_writer as W
from oracle import gguf_oracle as O


@pytest.fixture(scope="module")
def G(q27):
    return q27.gguf


def write(tmp_path, data: bytes, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


# ---------------------------------------------------------------- known answer (pins the oracle)
def known_answer_bytes():
    b = struct.pack("<IIQQ", 0x46554747, 3, 1, 2)                           # 24 bytes
    b += struct.pack("<Q", 20) + b"general.architecture" + struct.pack("<I", 8) + struct.pack("<Q", 6) + b"qwen35"
    b += struct.pack("<Q", 18) + b"qwen35.block_count" + struct.pack("<I", 4) + struct.pack("<I", 65)
    b += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2) + struct.pack("<QQ", 4, 2) + struct.pack("<IQ", 0, 0)
    assert len(b) == 24 + 46 + 34 + 41 == 145
    b += b"\0" * (160 - 145)                                                   # data section at 160 (32-aligned)
    b += np.arange(8, dtype=np.float32).tobytes()
    return b


def test_oracle_known_answer():
    kv, ts, start = O.parse(known_answer_bytes())
    assert start == 160
    assert kv == {b"general.architecture": (O.STRING, b"qwen35"), b"qwen35.block_count": (O.INT, 65)}
    assert ts == [dict(name=b"t", n_dims=2, ne=(4, 2, 1, 1), type=0, offset=0, nbytes=32, data_off=160)]


def test_library_known_answer(G, tmp_path):
    with G.GGUF(write(tmp_path, known_answer_bytes())) as g:
        assert g.keys() == ["general.architecture", "qwen35.block_count"]
        assert g.get_str("general.architecture") == "qwen35"
        assert g.get_int("qwen35.block_count") == 65
        assert g.get_float("qwen35.block_count") == 65.0
        t = g.tensor("t")
        assert (t.name, t.type, t.n_dims, t.ne, t.offset, t.nbytes) == ("t", 0, 2, (4, 2, 1, 1), 0, 32)
        assert t.rows() == 2 and t.row_bytes() == 16
        assert np.array_equal(t.array().view(np.float32), np.arange(8, dtype=np.float32))


# ---------------------------------------------------------------- round trips, library == oracle
def rich_file(alignment=32, seed=0):
    r = np.random.default_rng(seed)
    kv = [("general.architecture", W.STR, "qwen35"),
          ("u8", W.U8, 255), ("i8", W.I8, -128), ("u16", W.U16, 65535), ("i16", W.I16, -32768),
          ("u32", W.U32, 4294967295), ("i32", W.I32, -2147483648), ("f32", W.F32, 1e-6), ("bool", W.BOOL, 1),
          ("u64", W.U64, (1 << 64) - 5), ("i64", W.I64, -(1 << 62)), ("f64", W.F64, 1e300),
          ("one", W.ARR, [7], W.I32), ("ints", W.ARR, [1, -2, 3], W.I64), ("bools", W.ARR, [1, 0, 1], W.BOOL),
          ("floats", W.ARR, [0.5, -2.25], W.F32), ("doubles", W.ARR, [1e-300], W.F64),
          ("tokens", W.ARR, ["<s>", "", "héllo", "a" * 300], W.STR), ("empty", W.ARR, [], W.U32),
          ("unicode.ключ", W.STR, "значение")]
    if alignment != 32:
        kv.append(("general.alignment", W.U32, alignment))
    tensors = []
    for i, (typ, (bb, bs)) in enumerate(sorted(O.BLOCK.items())):
        ne = (bs * 2, 3) if bs > 1 else (5, 3, 2)
        nb = (ne[0] // bs) * bb * int(np.prod(ne[1:]))
        tensors.append((f"blk.{i}.w", typ, ne, r.integers(0, 256, nb, dtype=np.uint8).tobytes()))
    tensors.append(("scalar", 0, (1,), struct.pack("<f", 3.5)))
    tensors.append(("4d", 1, (2, 2, 2, 2), bytes(range(32))))
    return W.build(kv, tensors, alignment=alignment), kv, tensors


def assert_same(g, data: bytes):
    kv, ts, _ = O.parse(data)
    assert g.keys() == [k.decode() for k in kv]
    for k, (kind, v) in kv.items():
        gv = g.kv(k.decode())
        assert gv.kind == kind, k
        if kind in (O.INT, O.BOOL):
            assert gv.i == v
        elif kind == O.FLOAT:
            assert gv.f == v
        elif kind == O.STRING:
            assert gv.s == v.decode()
        elif kind == O.ARR_INT:
            assert list(gv.ai) == v
        elif kind == O.ARR_FLOAT:
            assert list(gv.af) == v
        else:
            assert list(gv.as_) == [x.decode() for x in v]
    got = g.tensors()
    assert len(got) == len(ts)
    for t, o in zip(got, ts):
        assert (t.name.encode(), t.n_dims, t.ne, t.type, t.offset, t.nbytes) == (
            o["name"], o["n_dims"], o["ne"], o["type"], o["offset"], o["nbytes"])
        assert bytes(t.array()) == data[o["data_off"]:o["data_off"] + o["nbytes"]]


@pytest.mark.parametrize("alignment", [32, 64, 4096, 1])
def test_round_trip_matches_oracle(G, tmp_path, alignment):
    data, kv, tensors = rich_file(alignment)
    with G.GGUF(write(tmp_path, data)) as g:
        assert_same(g, data)
        assert g.get_int("u64") == -5                      # u64 kept in int64 (src/gguf.cpp:96)
        assert g.get_int("one") == 7                       # single-element int array (src/gguf.cpp:206)
        assert g.get_float("f32") == np.float32(1e-6)
        assert g.kv("bool").kind == 2 and g.get_int("bool") == 1
        assert g.get_str("unicode.ключ") == "значение"
        for name, typ, ne, blob in tensors:
            t = g.tensor(name)
            assert t.type == typ and bytes(t.array()) == blob
            assert t.data % min(alignment, 4096) == 0 or alignment == 1


def test_type_tables(G):
    for typ, (bb, bs) in O.BLOCK.items():
        assert G.gtype_block_bytes(typ) == bb and G.gtype_block_size(typ) == bs
    assert G.gtype_name(22) == "IQ2_S" and G.gtype_name(29) == "IQ1_M" and G.gtype_name(8) == "?"
    with pytest.raises(Exception, match="unknown ggml type 8"):
        G.gtype_block_bytes(8)  # Q8_0 is not a type of this engine's files


def test_accessor_errors(G, tmp_path, q27):
    data, _, _ = rich_file()
    with G.GGUF(write(tmp_path, data)) as g:
        with pytest.raises(q27.Q27Error, match="missing key nope") as e:
            g.kv("nope")
        assert e.value.code == -7
        assert not g.has("nope") and g.has("u8")
        with pytest.raises(q27.Q27Error, match="missing tensor nope"):
            g.tensor("nope")
        assert g.find("nope") is None
        with pytest.raises(q27.Q27Error, match="key is not an int: ints"):
            g.get_int("ints")
        with pytest.raises(q27.Q27Error, match="key is not a float: general.architecture"):
            g.get_float("general.architecture")
        with pytest.raises(q27.Q27Error, match="key is not a string: u8"):
            g.get_str("u8")
    with pytest.raises(q27.Q27Error, match="cannot open") as e:
        G.GGUF(str(tmp_path / "absent.gguf"))
    assert e.value.code == -6


def test_repeated_key_and_name_keep_the_last(G, tmp_path):
    data = W.build([("k", W.U32, 1), ("k", W.U32, 2)],
                   [("t", 0, (1,), b"\1\0\0\0"), ("t", 0, (2,), b"\2\0\0\0\3\0\0\0")])
    with G.GGUF(write(tmp_path, data)) as g:
        assert g.get_int("k") == 2 and g.keys() == ["k"]
        assert g.tensor("t").ne[0] == 2 and len(g.tensors()) == 2
        assert_same(g, data)


# ---------------------------------------------------------------- every error path, same message as the oracle
def _err_cases():
    ok, _, _ = rich_file()
    small = W.build([("a", W.U32, 1)], [("t", 0, (4,), bytes(16))])
    nested = bytearray(W.build([("a", W.ARR, [], W.ARR)], []) + bytes(32))
    nested[24 + 9 + 8:24 + 9 + 16] = struct.pack("<Q", 1)  # one element of array type: "gguf: bad value type 9"
    cases = {
        "bad magic": b"GGUG" + ok[4:],
        "version 2": ok[:4] + struct.pack("<I", 2) + ok[8:],
        "n_dims 0": W.build([], [("t", 0, (), b"")]),
        "n_dims 5": W.build([], [("t", 0, (1, 1, 1, 1, 1), b"\0" * 4)]),
        "unknown type": W.build([], [("t", 8, (32,), b"\0" * 34)]),
        "nested array": nested,
        "bad value type": small[:24 + 9] + struct.pack("<I", 13) + small[24 + 13:],
        "out of file": small[:-1],
        "huge counts": struct.pack("<IIQQ", 0x46554747, 3, 1 << 60, 1 << 60),
        "huge string": struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1 << 62),
        "absurd shape": W.build([], [("t", 12, (256 << 40, 1 << 40, 1 << 40, 1 << 40), b"")]),
        "wrapping shape": W.build([], [("t", 0, (1 << 62, 4), b"")]),
        "zero alignment": W.build([("general.alignment", W.U32, 0)], []),
        "alignment string": W.build([("general.alignment", W.STR, "x")], []),
    }
    return cases


@pytest.mark.parametrize("case", sorted(_err_cases()))
def test_malformed_files(G, tmp_path, q27, case):
    data = _err_cases()[case]
    path = write(tmp_path, data)
    try:
        O.parse(data, path)
        want = None
    except (O.GGUFError, ZeroDivisionError) as e:
        want = str(e)
    with pytest.raises(q27.Q27Error) as e:
        G.GGUF(path)
    assert e.value.code == -5
    if case == "zero alignment":  # the reference divides by zero here
        assert "general.alignment is 0" in str(e.value)
    elif case == "huge string":
        assert "truncated string" in str(e.value)
    else:
        assert want is not None and want in str(e.value), (want, str(e.value))


def test_every_prefix_of_a_file(G, tmp_path, q27):
    """Truncated at every byte: the library either parses exactly what the oracle parses or reports the oracle's
    error; it never reads outside the mapping."""
    data = W.build([("general.architecture", W.STR, "qwen35"), ("v", W.ARR, [1, 2], W.U16),
                    ("s", W.ARR, ["ab", "c"], W.STR)], [("a", 12, (256, 1), bytes(144)), ("b", 0, (3,), bytes(12))])
    p = str(tmp_path / "pre.gguf")
    for n in range(len(data) + 1):
        pre = data[:n]
        with open(p, "wb") as f:
            f.write(pre)
        try:
            O.parse(pre, p)
            want = None
        except O.GGUFError as e:
            want = str(e)
        if want is None:
            with G.GGUF(p) as g:
                assert_same(g, pre)
        else:
            with pytest.raises(q27.Q27Error) as e:
                G.GGUF(p)
            assert want in str(e.value), (n, want, str(e.value))
    os.remove(p)


def test_cpp_dropin_reads_a_file(tmp_path):
    """include/q27/gguf.h (the reference's GGUF class) compiled into a program, linked with the library, run."""
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    data, _, tensors = rich_file(64)
    path = write(tmp_path, data)
    src = tmp_path / "dump.cpp"
    src.write_text(r"""
#include <cstdio>
#include "q27/gguf.h"
int main(int argc, char** argv) {
  q27::GGUF g(argv[1]);
  std::printf("%s %lld %g %zu\n", g.get_str("general.architecture").c_str(), (long long)g.get_int("u64"),
              g.get_float("f64"), g.kv("tokens").as.size());
  for (const auto& t : g.tensors()) {
    unsigned sum = 0;
    for (uint64_t i = 0; i < t.nbytes; i++) sum = sum * 31 + t.data[i];
    std::printf("%s %s %lld %llu %u\n", t.name.c_str(), q27::gtype_name(t.type), (long long)t.row_bytes(),
                (unsigned long long)t.nbytes, sum);
  }
  try { g.tensor("nope"); } catch (const std::exception& e) { std::printf("%s\n", e.what()); }
  try { q27::GGUF bad(argv[0]); } catch (const std::exception& e) { std::printf("%.17s\n", e.what()); }
}
""")
    exe = tmp_path / "dump"
    lib = os.path.join(root, "qwen27-engine_amd", "lib")
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{root}/include", str(src), f"-L{lib}", "-lq27h",
                    f"-Wl,-rpath,{lib}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe), path], capture_output=True, text=True, check=True).stdout.splitlines()
    assert out[0] == "qwen35 -5 1e+300 4"
    for line, (name, typ, ne, blob) in zip(out[1:], tensors):
        h = 0
        for b in blob:
            h = (h * 31 + b) & 0xFFFFFFFF
        bb, bs = O.BLOCK[typ]
        assert line.split() == [name, {0: "F32", 1: "F16", 30: "BF16"}.get(typ, line.split()[1]),
                                str(ne[0] // bs * bb), str(len(blob)), str(h)]
    assert out[-2] == "missing tensor nope"
    assert out[-1] == "not a GGUF file: "
