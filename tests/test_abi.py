"""The C ABI on the host (no GPU needed): the library loads, exports every symbol include/q27h.h declares, and
rejects the shapes and arguments the reference launchers reject (src/ops.cu:699,704,724,734; src/prefill.cu:518)
before anything is enqueued. Also compiles the C++ drop-in header q27/ops.h against the ABI."""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "q27h.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(q27h_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(q27):
    L = q27.lib()
    syms = declared_symbols()
    assert len(syms) >= 27
    for s in syms:
        assert hasattr(L, s), s
    assert L.q27h_abi_version() == 1


def test_python_binding_covers_the_abi(q27):
    from qwen27_engine_amd import _lib  # loaded by the q27 fixture

    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_kv_cache_bytes(q27):
    # src/attn.cu:890-892: q8 -> nkvh * n_ctx * (256 + 16); f16 -> nkvh * n_ctx * 512
    assert q27.ops.kv_cache_bytes(4, 180224, True) == 4 * 180224 * 272
    assert q27.ops.kv_cache_bytes(4, 180224, False) == 4 * 180224 * 512
    assert q27.ops.kv_cache_bytes(2, 1, True) == 544


FAKE = 1 << 20  # an aligned non-null address: the calls below must fail before any use of it


@pytest.mark.parametrize("call,code,needle", [
    (lambda o: o.rmsnorm_q8(FAKE, FAKE, FAKE, FAKE, FAKE, 4096, 4, 1e-6, 0), -1, "n must be 5120"),
    (lambda o: o.sum_norm_q8(FAKE, FAKE, 5120, 4, FAKE, FAKE, 1e-6, FAKE, FAKE, FAKE, 0), -2, "cross-card"),
    (lambda o: o.sum_norm_q8(FAKE, FAKE, 5000, 4, None, FAKE, 1e-6, FAKE, FAKE, FAKE, 0), -1, "5120"),
    (lambda o: o.sum_norm_rows(FAKE, FAKE, 5120, 8, FAKE, FAKE, 1e-6, None, FAKE, FAKE, FAKE, 0), -2, "cross-card"),
    (lambda o: o.add_norm_rows(FAKE, FAKE, None, 1024, 8, FAKE, 1e-6, None, FAKE, FAKE, FAKE, 0), -1, "5120"),
    (lambda o: o.swiglu_q8(FAKE, FAKE, FAKE, FAKE, 100, 0), -1, "n % 32"),
    (lambda o: o.quantize_q8_1(FAKE, FAKE, FAKE, 100, 2, 0), -1, "multiple of 32"),
    (lambda o: o.gdn_conv_l2(FAKE, FAKE, FAKE, FAKE, FAKE, 10240, 4, True, 32, 1e-6, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 47, 0),
     -1, "bad shape"),
    (lambda o: o.gdn_conv_l2(FAKE, FAKE, FAKE, FAKE, FAKE, 10240, 5, True, 32, 1e-6, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 0),
     -1, "T must be <= 4"),
    (lambda o: o.gdn_conv_prefill(FAKE, FAKE, FAKE, FAKE, FAKE, 10200, 64, 32, 1e-6, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 0),
     -1, "bad shape"),
    (lambda o: o.gdn_step(FAKE, FAKE, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 5, 0.088, True, 0), -1, "T must be <= 4"),
    (lambda o: o.gdn_step(FAKE, FAKE, FAKE, 10242, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 2048, 0.088, False, 0, True), -1,
     "bad shape"),
    (lambda o: o.gdn_step(FAKE, FAKE + 8, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 4, 0.088, True, 0), -4,
     "alignment"),
    (lambda o: o.gdn_step_chunked(FAKE, FAKE, FAKE, 10242, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 2048, 0.088, 0), -1,
     "bad shape"),
    (lambda o: o.gdn_step_chunked(FAKE, FAKE, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 65535 * 32 + 1, 0.088, 0), -1,
     "T too large"),
    (lambda o: o.gdn_step_chunked(FAKE, FAKE + 8, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 2048, 0.088, 0), -4,
     "alignment"),
    (lambda o: o.gdn_step_chunked(FAKE, FAKE, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, None, 48, 16, 2048, 0.088, 0), -4,
     "null pointer"),
    # o may not share memory with the rows, gates or planes it is staged beside (here o lies inside the q rows)
    (lambda o: o.gdn_step_chunked(FAKE, FAKE + 4096, FAKE + 8192, 10240, 1 << 30, (1 << 30) + (1 << 24), 1 << 31,
                                  FAKE, FAKE + 65536, 48, 16, 2048, 0.088, 0), -4, "overlaps"),
    (lambda o: o.gdn_step_chunked(FAKE, FAKE + 4096, FAKE + 8192, 10240, 1 << 30, (1 << 30) + (1 << 24), 1 << 31,
                                  FAKE, (1 << 31) + (1 << 20), 48, 16, 2048, 0.088, 0), -4, "overlaps"),
    (lambda o: o.to_q8_wire(FAKE, None, True, FAKE, 4096, 4, 0, 16), -1, "n must be 5120"),
    (lambda o: o.to_q8_wire(FAKE, None, True, FAKE, 5120, 4, 0, 24), -1, "qb must be 16 or 32"),
    (lambda o: o.add_norm_rows_q8(FAKE, FAKE, FAKE, 5120, 4, FAKE, 1e-6, None, FAKE, FAKE, None, 0, 0), -1,
     "qb must be 16 or 32"),
    (lambda o: o.add_norm_rows_q8(FAKE, FAKE, FAKE + 8, 5120, 4, FAKE, 1e-6, None, FAKE, FAKE, None, 0, 16), -4,
     "alignment"),
    (lambda o: o.to_bf16(FAKE, FAKE, 5, 0), -1, "even"),
    (lambda o: o.get_rows_q4_k(FAKE, 2880, FAKE, 4, FAKE, 5000, 0), -1, "multiple of 256"),
    (lambda o: o.get_rows_q8_0(FAKE, 100, FAKE, 4, FAKE, 5120, 0), -1, "row_bytes"),
    (lambda o: o.rmsnorm_q8(FAKE + 4, FAKE, None, FAKE, FAKE, 5120, 4, 1e-6, 0), -4, "alignment"),
    (lambda o: o.attn_prep(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 1e-6, 0.6, 24, 4, 0, True, 0), -1, "bad shape"),
    (lambda o: o.gemv_bf16_pair(FAKE, FAKE, FAKE, FAKE, FAKE, 48, 5121, 4, 0), -1, "K % 8"),
    (lambda o: o.gemv_bf16_pair(FAKE, FAKE + 2, FAKE, FAKE, FAKE, 48, 5120, 4, 0), -4, "alignment"),
    (lambda o: o.gemv_bf16_pair(FAKE, FAKE, None, FAKE, FAKE, 48, 5120, 4, 0), -4, "null pointer"),
    (lambda o: o.gated_rmsnorm_q8(FAKE + 4, FAKE, FAKE, FAKE, FAKE, 48, 1e-6, 0), -4, "alignment"),
])
def test_rejected_before_launch(q27, call, code, needle):
    with pytest.raises(q27.Q27Error) as ei:
        call(q27.ops)
    assert ei.value.code == code
    assert needle in str(ei.value)


def test_empty_inputs_are_no_ops(q27):
    # zero rows / tokens enqueue nothing (and so need no device)
    q27.ops.rmsnorm_q8(FAKE, FAKE, None, FAKE, FAKE, 5120, 0, 1e-6, 0)
    q27.ops.swiglu_q8(FAKE, FAKE, FAKE, FAKE, 0, 0)
    q27.ops.gated_rmsnorm_q8(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 1e-6, 0)
    q27.ops.get_rows_iq2_s(FAKE, 1640, FAKE, 0, FAKE, 5120, 0)
    q27.ops.attn_prep(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 1e-6, 0.6, 24, 4, 16, True, 0)
    q27.ops.gdn_step(FAKE, FAKE, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 0, 0.088, True, 0)
    q27.ops.gdn_step_chunked(FAKE, FAKE, FAKE, 10240, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 0, 0.088, 0)


def test_cpp_dropin_header_compiles(tmp_path):
    """include/q27/ops.h re-exposes the reference signatures; a caller written against src/ops.h compiles."""
    src = tmp_path / "caller.cpp"
    src.write_text(r'''
#include "q27/ops.h"
#include "q27/prefill.h"
#include "q27/qmat.h"
void step(float* x, const float* part, const float* w, float* h, int8_t* xq, float* xd, float* xs, hipStream_t s,
          const float* g, const float* u, const uint8_t* emb, const int* ids, int* plane) {
  q27::rmsnorm_q8(x, w, h, xq, xd, 5120, 4, 1e-6f, s);
  q27::sum_norm_q8(x, part, 5120, 4, nullptr, w, 1e-6f, h, xq, xd, s);
  q27::swiglu_q8(g, u, xq, xd, 4 * 17408, s);
  q27::sum_norm_rows(x, part, 5120, 2048, nullptr, w, 1e-6f, nullptr, xq, xd, xs, s);
  q27::quantize_q8_1(x, xq, xd, 6144, 2048, s, xs);
  q27::get_rows_iq2_s(emb, 1640, ids, 4, x, 5120, s);
  q27::gdn_flip_plane(plane, s);
  if (q27::wire_q8()) {
    q27::to_q8_wire(part, h, false, (uint8_t*)xq, 5120, 2048, s);  // src/prefill.h:38
    q27::add_norm_rows_q8(x, (const uint8_t*)xq, (const uint8_t*)xq, 5120, 2048, w, 1e-6f, nullptr, xq, xd, xs, s);
  } else {
    q27::to_bf16(part, (__hip_bfloat16*)h, 5120, s);
  }
  q27::gdn_step(x, x + 2048, x + 4096, 10240, g, u, h, plane, h, 48, 16, 4, 0.0884f, true, s);         // decode
  q27::gdn_step(x, x + 2048, x + 4096, 10240, g, u, h, plane, h, 48, 16, 2048, 0.0884f, false, s, true);  // prefill
  (void)q27::kv_cache_bytes(4, 180224, true);
}
void decode_gemv(const void* raw, const int8_t* xq, const float* xd, float* y, hipStream_t s) {
  q27::QMat m = q27::qmat_upload_raw(q27::GType::IQ3_S, 17408, 5120, raw, s);  // src/qmat.h:34 (device half)
  q27::qgemv(m, xq, xd, y, 4, s);                                                // src/qmat.h:44-46
  q27::qmat_free(m);
  (void)q27::qmat_supported(q27::GType::IQ1_M);
}
void load_gguf(const char* path, void* scratch, size_t scratch_bytes, hipStream_t s) {
  q27::GGUF g(path);                                                   // src/gguf.h:46
  const q27::GTensor& t = g.tensor("blk.0.ffn_up.weight");
  q27::QMat m = q27::qmat_upload(t, 0, (int)t.ne[1], scratch, scratch_bytes, s);  // src/qmat.h:34
  (void)g.get_int("qwen35.block_count");
  (void)g.get_float("qwen35.rope.freq_base");
  (void)g.get_str("general.architecture");
  (void)q27::gtype_name(t.type);
  q27::qmat_free(m);
}
''')
    inc = os.path.join(ROOT, "include")
    r = subprocess.run(["/opt/rocm/llvm/bin/clang++", "-std=c++17", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__", f"-I{inc}", "-I/opt/rocm/include",
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_qgemv_rejects_before_enqueue(q27):
    L = q27.lib()
    assert L.q27h_qgemv(8, 64, 256, FAKE, FAKE, FAKE, FAKE, 1, None) == -2  # Q8_0: not a GEMV type
    assert "not supported" in L.q27h_last_error().decode()
    assert L.q27h_qgemv(12, 60, 256, FAKE, FAKE, FAKE, FAKE, 1, None) == -1  # N % 8
    assert L.q27h_qgemv(12, 64, 300, FAKE, FAKE, FAKE, FAKE, 1, None) == -1  # K % 256
    assert L.q27h_qgemv(12, 64, 256, FAKE, FAKE, FAKE, FAKE, 5, None) == -1  # ncols
    assert L.q27h_qgemv(12, 64, 256, FAKE + 16, FAKE, FAKE, FAKE, 1, None) == -4  # buf alignment
    # the fused form: the same checks, and at most 40960 activations in LDS
    assert L.q27h_qgemv_f32(8, 64, 256, FAKE, FAKE, FAKE, 1, None) == -2
    assert L.q27h_qgemv_f32(12, 64, 300, FAKE, FAKE, FAKE, 1, None) == -1
    assert L.q27h_qgemv_f32(12, 64, 256, FAKE, FAKE, FAKE, 0, None) == -1
    assert L.q27h_qgemv_f32(12, 64, 17408, FAKE, FAKE, FAKE, 4, None) == -1  # 69632 activations
    assert L.q27h_qgemv_f32(12, 64, 256, FAKE + 16, FAKE, FAKE, 1, None) == -4
    assert L.q27h_qmat_repack(14, 64, 256, FAKE, FAKE + 8, None) == -4
    assert L.q27h_qmat_repack(21, 64, 250, FAKE, FAKE, None) == -1
    # bytes: fields then scales, each 256-byte aligned (Q4_K 128 + 16 per chunk, 32 per (tile, block)); ntb at K = 512
    ntb = (64 // 8) * (512 // 256)
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert L.q27h_qmat_bytes(12, 64, 1024) == al(2 * ntb * 8 * 128) + al(2 * ntb * 8 * 16) + al(2 * ntb * 32)
    assert L.q27h_qmat_bytes(23, 64, 1024) == al(2 * ntb * 8 * 128) + al(2 * ntb * 8 * 8) + al(2 * ntb * 16)
    # fields wider than 16 bytes per chunk pad a tile's blocks to a multiple of 4 (K = 512: 2 blocks -> 4)
    assert L.q27h_qmat_bytes(12, 64, 512) == al(2 * ntb * 8 * 128) + al(ntb * 8 * 16) + al(ntb * 32)
    assert L.q27h_qmat_bytes(8, 64, 512) == 0


def test_gdn_prefill_exact_switch(q27):
    """The process-wide prefill choice of gdn_step is a host setting: it returns the previous value."""
    prev = q27.ops.gdn_prefill_exact(True)
    try:
        assert q27.ops.gdn_prefill_exact(False) is True
        assert q27.ops.gdn_prefill_exact(False) is False
    finally:
        q27.ops.gdn_prefill_exact(prev)
