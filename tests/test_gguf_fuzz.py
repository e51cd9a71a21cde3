"""Fuzz of the GGUF parser on the CPU: the library's reader (csrc/gguf.hip, host code) compiled with
AddressSanitizer and UndefinedBehaviorSanitizer into a small driver, run over a few thousand mutated files (bit flips,
random bytes, corrupted length and count fields, truncations). Every file must parse to exactly what the oracle
(oracle/gguf_oracle.py) parses -- same tensor and key counts and the same tensor bytes -- or fail with the oracle's
message, and the sanitizers must stay silent. Skipped when g++ or the sanitizer runtimes are unavailable."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import gguf_writer as W
from oracle import gguf_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "qwen27-engine_amd", "csrc")

DRIVER = r"""
#include <cstdio>
#include "q27h.h"
int main(int argc, char** argv) {
  for (int i = 1; i < argc; i++) {
    q27h_gguf* g = nullptr;
    if (q27h_gguf_open(argv[i], &g) != Q27H_OK) {  // the message in hex: names in it may hold any byte
      std::printf("ERR ");
      for (const char* c = q27h_last_error(); *c; c++) std::printf("%02x", (unsigned char)*c);
      std::printf("\n");
      continue;
    }
    const long long nt = q27h_gguf_n_tensors(g), nk = q27h_gguf_n_kv(g);
    unsigned sum = 0;
    for (long long t = 0; t < nt; t++) {
      q27h_gtensor x;
      q27h_gguf_tensor(g, t, &x);
      for (unsigned long long b = 0; b < x.nbytes; b++) sum = sum * 31u + x.data[b];
    }
    for (long long k = 0; k < nk; k++) {
      q27h_gvalue v;
      const char* key; size_t kn;
      if (q27h_gguf_key(g, k, &key, &kn) != Q27H_OK || q27h_gguf_kv_at(g, k, &v) != Q27H_OK) return 2;
      for (size_t c = 0; c < kn; c++) sum = sum * 31u + (unsigned char)key[c];
      for (unsigned long long j = 0; v.kind == Q27H_GV_ARR_STRING && j < v.n; j++) {
        const char* s; size_t n;
        if (q27h_gguf_kv_str_at(g, k, j, &s, &n) != Q27H_OK) return 2;
        for (size_t c = 0; c < n; c++) sum = sum * 31u + (unsigned char)s[c];
      }
    }
    std::printf("OK %lld %lld %u\n", nt, nk, sum);
    q27h_gguf_close(g);
  }
}
"""


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("fuzz")
    (d / "drv.cpp").write_text(DRIVER)
    exe = d / "drv"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-fno-omit-frame-pointer", "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                        f"-I{ROOT}/include", f"-I{CSRC}", os.path.join(CSRC, "gguf.hip"), os.path.join(CSRC, "status.hip"),
                        str(d / "drv.cpp"), "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("sanitizer build unavailable: " + r.stderr[-300:])
    return str(exe), d


def expected(data: bytes, path: str):
    try:
        kv, ts, _ = O.parse(data, path)
    except O.GGUFError as e:
        return ("ERR", str(e))
    except ZeroDivisionError:
        return ("ERR", "gguf: general.alignment is 0")
    h = 0
    for t in ts:
        for b in data[t["data_off"]:t["data_off"] + t["nbytes"]]:
            h = (h * 31 + b) & 0xFFFFFFFF
    for k, (kind, v) in kv.items():
        for b in k:
            h = (h * 31 + b) & 0xFFFFFFFF
        if kind == O.ARR_STRING:
            for s in v:
                for b in s:
                    h = (h * 31 + b) & 0xFFFFFFFF
    return ("OK", f"{len(ts)} {len(kv)} {h}")


def seeds():
    yield W.build([("general.architecture", W.STR, "qwen35"), ("n", W.U32, 65), ("f", W.F32, 0.5),
                   ("toks", W.ARR, ["a", "bc", ""], W.STR), ("ids", W.ARR, [1, 2, 3], W.I32)],
                  [("blk.0.w", 12, (256, 2), bytes(range(256)) * 1 + bytes(32)), ("b", 0, (3,), bytes(12)),
                   ("c", 22, (256,), bytes(82))])
    yield W.build([("general.alignment", W.U32, 64), ("x", W.ARR, [0.25], W.F64)],
                  [("t", 1, (2, 2, 2), bytes(16)), ("u", 30, (5,), bytes(10))], alignment=64)


def mutations(data: bytes, r, n):
    b = len(data)
    for i in range(n):
        d = bytearray(data)
        kind = i % 5
        if kind == 0:                       # flip 1..4 bits
            for _ in range(r.integers(1, 5)):
                p = r.integers(0, b)
                d[p] ^= 1 << r.integers(0, 8)
        elif kind == 1:                     # random bytes in the header / directory
            for _ in range(r.integers(1, 4)):
                d[r.integers(0, min(b, 200))] = r.integers(0, 256)
        elif kind == 2:                     # a length / count field made huge, tiny or off by a little
            p = int(r.integers(0, max(1, min(b, 200) - 8)))
            vals = [0, 1, 2 ** 32, 2 ** 63, 2 ** 64 - 1, int(r.integers(0, 1 << 20))]
            v = vals[int(r.integers(0, len(vals)))]
            d[p:p + 8] = struct.pack("<Q", v)
        elif kind == 3:                     # truncation
            d = d[:r.integers(0, b)]
        else:                               # a u32 type / n_dims field replaced
            p = int(r.integers(0, max(1, min(b, 200) - 4)))
            d[p:p + 4] = struct.pack("<I", int(r.integers(0, 40)))
        yield bytes(d)


def test_mutated_files_match_oracle_under_sanitizers(driver):
    exe, d = driver
    r = np.random.default_rng(2024)
    files, want = [], []
    for si, seed in enumerate(seeds()):
        for j, m in enumerate(mutations(seed, r, 1500)):
            p = str(d / f"m{si}_{j}.gguf")
            with open(p, "wb") as f:
                f.write(m)
            files.append(p)
            want.append(expected(m, p))
    got = []
    for i in range(0, len(files), 500):
        res = subprocess.run([exe] + files[i:i + 500], capture_output=True, text=True, timeout=300)
        assert res.returncode == 0, res.stderr[-2000:]
        assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr[-2000:]
        got += res.stdout.splitlines()
    assert len(got) == len(files)
    bad = []
    for f, g, (status, text) in zip(files, got, want):
        if status == "OK":
            ok = g == f"OK {text}"
        else:
            # the C ABI's message is a C string: a name with a NUL byte in it ends there
            ok = g.startswith("ERR ") and text.split("\x00")[0] in bytes.fromhex(g[4:]).decode("utf-8", "replace")
        if not ok:
            bad.append((os.path.basename(f), g, status, text))
    assert not bad, bad[:5]
    assert sum(1 for s, _ in want if s == "OK") > 50  # some mutations still parse (the comparison is not vacuous)
