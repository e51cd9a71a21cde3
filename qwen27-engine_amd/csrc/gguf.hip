// GGUF (version 3) reader and the staged host -> HBM copy that feeds the weight upload (src/gguf.h, src/gguf.cpp,
// src/qmat.h:34 of the reference engine).
//
// The file is memory-mapped read-only; the header, the key / value table and the tensor directory are parsed once
// into host structures, and tensor data pointers point into the mapping (data section aligned to
// general.alignment, default 32). Malformed files are rejected with the reference's messages; every length read
// from the file is bounds-checked against the mapping before use.
//
// Upload: the reference copies each tensor with one cudaMemcpyAsync from the pageable mapping, which the driver
// stages through its own small pinned buffers on the calling thread. Here the rows are split into 16 MiB chunks;
// several host threads fill a chunk into one of six pinned staging buffers (allocated once per process, reused)
// -- with pread from the file (q27h_gguf_upload_rows) or memcpy from any host range (q27h_copy_h2d_staged) -- and
// its DMA to HBM is enqueued on the caller's stream while the next chunk is being filled.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <functional>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <thread>
#include <vector>

#include "q27h_internal.h"

namespace q27h {
namespace {

// GGUF metadata value types (gguf_type of the GGUF specification).
enum : uint32_t { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

struct Value {
  int kind = Q27H_GV_INT;
  int64_t i = 0;
  double f = 0;
  std::string s;
  std::vector<int64_t> ai;
  std::vector<double> af;
  std::vector<std::string> as;
};

struct Tensor {
  std::string name;
  uint32_t type = 0;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0, nbytes = 0;
  const uint8_t* data = nullptr;
};

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  template <class T>
  T get() {
    if ((size_t)(end - p) < sizeof(T)) throw std::runtime_error("gguf: truncated file");
    T v;
    std::memcpy(&v, p, sizeof(T));
    p += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (n > (uint64_t)(end - p)) throw std::runtime_error("gguf: truncated string");
    std::string s((const char*)p, n);
    p += n;
    return s;
  }
};

// One scalar of type t: integers (and bools) into i (returns true), floats into f (returns false).
bool scalar(Cursor& c, uint32_t t, int64_t& i, double& f) {
  switch (t) {
    case kU8: i = c.get<uint8_t>(); return true;
    case kI8: i = c.get<int8_t>(); return true;
    case kU16: i = c.get<uint16_t>(); return true;
    case kI16: i = c.get<int16_t>(); return true;
    case kU32: i = c.get<uint32_t>(); return true;
    case kI32: i = c.get<int32_t>(); return true;
    case kU64: i = (int64_t)c.get<uint64_t>(); return true;
    case kI64: i = c.get<int64_t>(); return true;
    case kBool: i = c.get<uint8_t>(); return true;
    case kF32: f = c.get<float>(); return false;
    case kF64: f = c.get<double>(); return false;
    default: throw std::runtime_error("gguf: bad value type " + std::to_string(t));
  }
}

}  // namespace
}  // namespace q27h

// The opaque handle of the C ABI.
struct q27h_gguf {
  std::string path;
  const uint8_t* base = nullptr;
  uint64_t size = 0;
  int fd = -1;
  std::map<std::string, q27h::Value> kv;
  std::vector<std::string> keys;  // file order
  std::vector<q27h::Tensor> tensors;
  std::map<std::string, int64_t> index;

  ~q27h_gguf() {
    if (base) munmap((void*)base, size);
    if (fd >= 0) close(fd);
  }

  void parse() {
    using namespace q27h;
    Cursor c{base, base + size};
    if (c.get<uint32_t>() != 0x46554747u) throw std::runtime_error("not a GGUF file: " + path);
    const uint32_t version = c.get<uint32_t>();
    if (version != 3) throw std::runtime_error("GGUF version " + std::to_string(version) + " not supported");
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    for (uint64_t k = 0; k < n_kv; k++) {
      std::string key = c.str();
      const uint32_t t = c.get<uint32_t>();
      Value v;
      if (t == kStr) {
        v.kind = Q27H_GV_STRING;
        v.s = c.str();
      } else if (t == kArr) {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        // elements are appended as read (nothing reserved from n): a corrupt count ends at the mapping's end
        if (et == kStr) {
          v.kind = Q27H_GV_ARR_STRING;
          for (uint64_t j = 0; j < n; j++) v.as.push_back(c.str());
        } else {
          int64_t iv = 0;
          double fv = 0;
          for (uint64_t j = 0; j < n; j++) {
            if (scalar(c, et, iv, fv)) v.ai.push_back(iv);
            else v.af.push_back(fv);
          }
          v.kind = (et == kF32 || et == kF64) ? Q27H_GV_ARR_FLOAT : Q27H_GV_ARR_INT;
        }
      } else {
        const bool isint = scalar(c, t, v.i, v.f);
        v.kind = isint ? (t == kBool ? Q27H_GV_BOOL : Q27H_GV_INT) : Q27H_GV_FLOAT;
      }
      if (!kv.count(key)) keys.push_back(key);
      kv[key] = std::move(v);  // a repeated key keeps its last value
    }
    // entries are appended as they are read (nothing is reserved from the counts in the header): a corrupt count
    // ends in "gguf: truncated file" at the end of the mapping instead of a huge allocation
    for (uint64_t k = 0; k < n_tensors; k++) {
      Tensor& t = tensors.emplace_back();
      t.name = c.str();
      t.n_dims = (int)c.get<uint32_t>();
      if (t.n_dims < 1 || t.n_dims > 4) throw std::runtime_error("bad n_dims for " + t.name);
      for (int d = 0; d < t.n_dims; d++) t.ne[d] = (int64_t)c.get<uint64_t>();
      t.type = c.get<uint32_t>();
      t.offset = c.get<uint64_t>();
      const int bb = q27h_gtype_block_bytes((int)t.type), bs = q27h_gtype_block_size((int)t.type);
      if (bb == 0) throw std::runtime_error("unknown ggml type " + std::to_string(t.type));
      // element count and size in unsigned 128-bit arithmetic, saturated: an absurd shape cannot wrap around into
      // a small size and fails the "tensor out of file" check below
      unsigned __int128 n = 1;
      for (int d = 0; d < 4; d++) {
        n *= (uint64_t)t.ne[d];
        if (n > ~uint64_t(0)) n = ~uint64_t(0);
      }
      const unsigned __int128 nb = n / (unsigned)bs * (unsigned)bb;
      t.nbytes = nb > ~uint64_t(0) ? ~uint64_t(0) : (uint64_t)nb;
      index[t.name] = (int64_t)k;  // a repeated name finds its last entry
    }
    uint64_t align = 32;
    if (auto it = kv.find("general.alignment"); it != kv.end()) {
      const Value& a = it->second;
      if (a.kind == Q27H_GV_INT || a.kind == Q27H_GV_BOOL) align = (uint64_t)a.i;
      else if (a.kind == Q27H_GV_ARR_INT && a.ai.size() == 1) align = (uint64_t)a.ai[0];
      else throw std::runtime_error("key is not an int: general.alignment");
      if (align == 0) throw std::runtime_error("gguf: general.alignment is 0");
    }
    uint64_t data_start = (uint64_t)(c.p - base);
    data_start = (data_start + align - 1) / align * align;
    for (auto& t : tensors) {
      if (data_start > size || t.offset > size - data_start || t.nbytes > size - data_start - t.offset)
        throw std::runtime_error("tensor out of file: " + t.name);
      t.data = base + data_start + t.offset;
    }
  }
};

using namespace q27h;

namespace {

template <class F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    return fail(Q27H_ERR_FORMAT, e.what());
  }
}

const Value* find_kv(const q27h_gguf* g, const char* key) {
  auto it = g->kv.find(key);
  return it == g->kv.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" int q27h_gtype_block_bytes(int type) {
  switch (type) {
    case 0: return 4;     // F32
    case 1: return 2;     // F16
    case 30: return 2;    // BF16
    case 10: return 84;   // Q2_K
    case 12: return 144;  // Q4_K
    case 14: return 210;  // Q6_K
    case 16: return 66;   // IQ2_XXS
    case 17: return 74;   // IQ2_XS
    case 18: return 98;   // IQ3_XXS
    case 21: return 110;  // IQ3_S
    case 22: return 82;   // IQ2_S
    case 23: return 136;  // IQ4_XS
    case 29: return 56;   // IQ1_M
    default: return 0;
  }
}

extern "C" int q27h_gtype_block_size(int type) {
  if (q27h_gtype_block_bytes(type) == 0) return 0;
  return (type == 0 || type == 1 || type == 30) ? 1 : 256;
}

extern "C" const char* q27h_gtype_name(int type) {
  switch (type) {
    case 0: return "F32";
    case 1: return "F16";
    case 10: return "Q2_K";
    case 12: return "Q4_K";
    case 14: return "Q6_K";
    case 16: return "IQ2_XXS";
    case 17: return "IQ2_XS";
    case 18: return "IQ3_XXS";
    case 21: return "IQ3_S";
    case 22: return "IQ2_S";
    case 23: return "IQ4_XS";
    case 29: return "IQ1_M";
    case 30: return "BF16";
    default: return "?";
  }
}

extern "C" int q27h_gguf_open(const char* path, q27h_gguf** out) {
  if (!path || !out) return fail(Q27H_ERR_ARG, "gguf_open: null pointer");
  *out = nullptr;
  auto* g = new q27h_gguf;
  g->path = path;
  g->fd = open(path, O_RDONLY);
  if (g->fd < 0) {
    delete g;
    return fail(Q27H_ERR_IO, std::string("cannot open ") + path);
  }
  struct stat st;
  if (fstat(g->fd, &st) != 0) {
    delete g;
    return fail(Q27H_ERR_IO, std::string("cannot stat ") + path);
  }
  g->size = (uint64_t)st.st_size;
  if (g->size > 0) {
    void* p = mmap(nullptr, g->size, PROT_READ, MAP_SHARED, g->fd, 0);
    if (p == MAP_FAILED) {
      delete g;
      return fail(Q27H_ERR_IO, std::string("cannot mmap ") + path);
    }
    g->base = (const uint8_t*)p;
  }
  const int rc = guarded([&] {
    g->parse();
    return Q27H_OK;
  });
  if (rc != Q27H_OK) {
    delete g;
    return rc;
  }
  *out = g;
  return Q27H_OK;
}

extern "C" void q27h_gguf_close(q27h_gguf* g) { delete g; }

extern "C" int64_t q27h_gguf_n_tensors(const q27h_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

extern "C" int64_t q27h_gguf_find(const q27h_gguf* g, const char* name) {
  if (!g || !name) return -1;
  auto it = g->index.find(name);
  return it == g->index.end() ? -1 : it->second;
}

extern "C" int q27h_gguf_tensor(const q27h_gguf* g, int64_t i, q27h_gtensor* out) {
  if (!g || !out) return fail(Q27H_ERR_ARG, "gguf_tensor: null pointer");
  if (i < 0 || i >= (int64_t)g->tensors.size()) return fail(Q27H_ERR_NOT_FOUND, "gguf_tensor: index out of range");
  const Tensor& t = g->tensors[i];
  out->name = t.name.c_str();
  out->name_len = t.name.size();
  out->type = (int)t.type;
  out->n_dims = t.n_dims;
  for (int d = 0; d < 4; d++) out->ne[d] = t.ne[d];
  out->offset = t.offset;
  out->nbytes = t.nbytes;
  out->data = t.data;
  return Q27H_OK;
}

extern "C" int64_t q27h_gguf_n_kv(const q27h_gguf* g) { return g ? (int64_t)g->keys.size() : 0; }

extern "C" int q27h_gguf_key(const q27h_gguf* g, int64_t i, const char** s, size_t* len) {
  if (!g || !s || !len) return fail(Q27H_ERR_ARG, "gguf_key: null pointer");
  if (i < 0 || i >= (int64_t)g->keys.size()) return fail(Q27H_ERR_NOT_FOUND, "gguf_key: index out of range");
  *s = g->keys[i].c_str();
  *len = g->keys[i].size();
  return Q27H_OK;
}

namespace {
int fill_value(const Value& v, q27h_gvalue* out) {
  out->kind = v.kind;
  out->i = v.i;
  out->f = v.f;
  out->s = v.s.c_str();
  out->s_len = v.s.size();
  out->n = v.kind == Q27H_GV_ARR_INT ? v.ai.size()
           : v.kind == Q27H_GV_ARR_FLOAT ? v.af.size()
           : v.kind == Q27H_GV_ARR_STRING ? v.as.size() : 0;
  out->ai = v.ai.empty() ? nullptr : v.ai.data();
  out->af = v.af.empty() ? nullptr : v.af.data();
  return Q27H_OK;
}
}  // namespace

extern "C" int q27h_gguf_kv(const q27h_gguf* g, const char* key, q27h_gvalue* out) {
  if (!g || !key || !out) return fail(Q27H_ERR_ARG, "gguf_kv: null pointer");
  const Value* v = find_kv(g, key);
  if (!v) return fail(Q27H_ERR_NOT_FOUND, std::string("missing key ") + key);
  return fill_value(*v, out);
}

extern "C" int q27h_gguf_kv_at(const q27h_gguf* g, int64_t i, q27h_gvalue* out) {
  if (!g || !out) return fail(Q27H_ERR_ARG, "gguf_kv_at: null pointer");
  if (i < 0 || i >= (int64_t)g->keys.size()) return fail(Q27H_ERR_NOT_FOUND, "gguf_kv_at: index out of range");
  return fill_value(g->kv.at(g->keys[i]), out);
}

extern "C" int q27h_gguf_kv_str_at(const q27h_gguf* g, int64_t i, uint64_t j, const char** s, size_t* len) {
  if (!g || !s || !len) return fail(Q27H_ERR_ARG, "gguf_kv_str_at: null pointer");
  if (i < 0 || i >= (int64_t)g->keys.size()) return fail(Q27H_ERR_NOT_FOUND, "gguf_kv_str_at: index out of range");
  const Value& v = g->kv.at(g->keys[i]);
  if (v.kind != Q27H_GV_ARR_STRING) return fail(Q27H_ERR_FORMAT, "key is not a string array: " + g->keys[i]);
  if (j >= v.as.size()) return fail(Q27H_ERR_NOT_FOUND, "index out of range for " + g->keys[i]);
  *s = v.as[j].c_str();
  *len = v.as[j].size();
  return Q27H_OK;
}

// ---------------------------------------------------------------- staged host -> device copy
namespace {

// Chunk size, buffer count and smallest per-thread slice: measured on 1.07 GB of 38 MB tensors read from the page
// cache, 16 MiB x 6 gives 52.8 GB/s (92% of a pinned 1 GiB DMA, 57.6 GB/s); 32 MiB x 4: 42.5, 8 MiB x 8: 51.0,
// 4 MiB x 16: 46.4 (shorter chunks fill the pipeline sooner at each tensor, longer ones pay less per chunk).
#ifndef Q27H_STAGE_MB
#define Q27H_STAGE_MB 16
#endif
#ifndef Q27H_STAGE_BUFS
#define Q27H_STAGE_BUFS 6
#endif
#ifndef Q27H_SLICE_KB
#define Q27H_SLICE_KB 1024
#endif
constexpr int kStageBufs = Q27H_STAGE_BUFS;
constexpr size_t kStageBytes = size_t(Q27H_STAGE_MB) << 20;

struct Staging {
  std::mutex mu;
  int device = -1;
  void* buf[kStageBufs] = {};
  hipEvent_t done[kStageBufs] = {};
  bool ready = false;
};
Staging g_stage;

int stage_init(int device) {
  if (g_stage.ready && g_stage.device == device) return Q27H_OK;
  if (g_stage.ready) {  // the buffers are pinned for all devices; only the events belong to the old one
    for (auto& e : g_stage.done) {
      (void)hipEventSynchronize(e);
      (void)hipEventDestroy(e);
    }
  } else {
    for (auto& b : g_stage.buf)
      if (hipHostMalloc(&b, kStageBytes, hipHostMallocPortable) != hipSuccess)
        return fail(Q27H_ERR_HIP, "copy_h2d_staged: hipHostMalloc of the staging buffers failed");
  }
  for (auto& e : g_stage.done)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
      return fail(Q27H_ERR_HIP, "copy_h2d_staged: hipEventCreate failed");
  g_stage.device = device;
  g_stage.ready = true;
  return Q27H_OK;
}

#ifndef MADV_POPULATE_READ
#define MADV_POPULATE_READ 22
#endif

// Persistent host workers for the staging fills (created on first use, parked between jobs): spawning threads per
// chunk costs a fifth of the chunk's copy time. Jobs are serialised by the staging mutex.
class Workers {
 public:
  static constexpr int kMax = 16;
  // Runs f(i) for i in [0, n) on n threads (the caller is thread 0, n <= kMax); returns when all are done.
  void run(int n, const std::function<void(int)>& f) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      while ((int)threads_.size() < n - 1) {
        const int id = (int)threads_.size() + 1;
        threads_.emplace_back([this, id] { loop(id); });
      }
      job_ = &f;
      active_ = n - 1;
      pending_ = n - 1;
      gen_++;
    }
    cv_.notify_all();
    f(0);
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [&] { return pending_ == 0; });
    job_ = nullptr;
  }
  ~Workers() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : threads_) t.join();
  }

 private:
  void loop(int id) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int)>* job = nullptr;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
        if (id > active_) continue;  // not part of this job
        job = job_;
      }
      (*job)(id);
      std::lock_guard<std::mutex> lk(mu_);
      if (--pending_ == 0) done_cv_.notify_all();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  std::vector<std::thread> threads_;
  const std::function<void(int)>* job_ = nullptr;
  uint64_t gen_ = 0;
  int active_ = 0, pending_ = 0;
  bool stop_ = false;
};
Workers g_workers;

// Fills n bytes of dst with up to `threads` host threads (slices of at least 2 MiB); part(dst, off, len) copies one
// slice and returns false on failure.
template <class Part>
bool par_fill(uint8_t* dst, size_t n, int threads, const Part& part) {
  const size_t min_slice = size_t(Q27H_SLICE_KB) << 10;
  const int nt = (int)std::max<size_t>(1, std::min<size_t>((size_t)std::min(threads, Workers::kMax), n / min_slice));
  if (nt == 1) return part(dst, 0, n);
  const size_t slice = (n + nt - 1) / nt;
  char ok[Workers::kMax];
  g_workers.run(nt, [&](int i) {
    const size_t a = std::min(n, i * slice), b = std::min(n, a + slice);
    ok[i] = part(dst, a, b - a);
  });
  return std::all_of(ok, ok + nt, [](char c) { return c != 0; });
}

// One slice of a memory copy. The source's page-table entries are populated in one system call first
// (MADV_POPULATE_READ; ignored where unsupported): taking a page fault per 4 KiB page of a file mapping costs more
// than the copy itself.
bool copy_part(uint8_t* dst, const uint8_t* src, size_t off, size_t len) {
  const uintptr_t a = (uintptr_t)(src + off) & ~uintptr_t(4095), b = (uintptr_t)(src + off + len);
  (void)madvise((void*)a, b - a, MADV_POPULATE_READ);
  std::memcpy(dst + off, src + off, len);
  return true;
}

// One slice read from a file descriptor (pread from the page cache straight into the staging buffer).
bool read_part(int fd, uint64_t file_off, uint8_t* dst, size_t off, size_t len) {
  while (len > 0) {
    const ssize_t r = pread(fd, dst + off, len, (off_t)(file_off + off));
    if (r <= 0) return false;
    off += (size_t)r;
    len -= (size_t)r;
  }
  return true;
}

// The staging loop: chunk i is filled by fill(buffer, offset, bytes) into pinned buffer i % 4 once that buffer's
// previous DMA has drained, then DMA'd to dst + offset on stream st.
template <class Fill>
int staged(uint8_t* dst, size_t bytes, hipStream_t st, const char* what, const Fill& fill) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(Q27H_ERR_HIP, std::string(what) + ": no device");
  if (int rc = stage_init(device); rc != Q27H_OK) return rc;
  for (size_t off = 0, i = 0; off < bytes; off += kStageBytes, i++) {
    const int b = (int)(i % kStageBufs);
    const size_t n = std::min(kStageBytes, bytes - off);
    // the buffer's previous DMA (recorded at its last use, possibly in an earlier call) must have drained
    if (hipEventSynchronize(g_stage.done[b]) != hipSuccess) return fail(Q27H_ERR_HIP, std::string(what) + ": event wait failed");
    if (!fill((uint8_t*)g_stage.buf[b], off, n)) return fail(Q27H_ERR_IO, std::string(what) + ": read failed");
    if (hipMemcpyAsync(dst + off, g_stage.buf[b], n, hipMemcpyHostToDevice, st) != hipSuccess)
      return fail(Q27H_ERR_HIP, std::string(what) + ": hipMemcpyAsync failed");
    if (hipEventRecord(g_stage.done[b], st) != hipSuccess) return fail(Q27H_ERR_HIP, std::string(what) + ": event record failed");
  }
  return Q27H_OK;
}

int default_threads(int threads) {
  return threads > 0 ? threads : (int)std::min(8u, std::max(1u, std::thread::hardware_concurrency()));
}

}  // namespace

extern "C" int q27h_copy_h2d_staged(void* dst, const void* src, size_t bytes, int threads, q27h_stream_t s) {
  if (bytes == 0) return Q27H_OK;
  if (!dst || !src) return fail(Q27H_ERR_ARG, "copy_h2d_staged: null pointer");
  threads = default_threads(threads);
  std::lock_guard<std::mutex> lock(g_stage.mu);
  const auto* in = (const uint8_t*)src;
  return staged((uint8_t*)dst, bytes, stream_of(s), "copy_h2d_staged", [&](uint8_t* buf, size_t off, size_t n) {
    return par_fill(buf, n, threads, [&](uint8_t* d, size_t o, size_t len) { return copy_part(d, in + off, o, len); });
  });
}

extern "C" int q27h_gguf_upload_rows(const q27h_gguf* g, int64_t tensor, int64_t row0, int64_t nrows, void* dst,
                                     int threads, q27h_stream_t s) {
  if (!g || !dst) return fail(Q27H_ERR_ARG, "gguf_upload_rows: null pointer");
  if (tensor < 0 || tensor >= (int64_t)g->tensors.size()) return fail(Q27H_ERR_NOT_FOUND, "gguf_upload_rows: index out of range");
  const Tensor& t = g->tensors[tensor];
  const int bb = q27h_gtype_block_bytes((int)t.type), bs = q27h_gtype_block_size((int)t.type);
  const uint64_t row_bytes = (uint64_t)(t.ne[0] / bs) * (uint64_t)bb;
  const int64_t rows = t.ne[1] * t.ne[2] * t.ne[3];
  if (row0 < 0 || nrows < 0 || row0 > rows || nrows > rows - row0)
    return fail(Q27H_ERR_SHAPE, "gguf_upload_rows: rows outside " + t.name);
  const size_t bytes = (size_t)nrows * row_bytes;
  if (bytes == 0) return Q27H_OK;
  const uint64_t file_off = (uint64_t)(t.data - g->base) + (uint64_t)row0 * row_bytes;
  threads = default_threads(threads);
  std::lock_guard<std::mutex> lock(g_stage.mu);
  return staged((uint8_t*)dst, bytes, stream_of(s), "gguf_upload_rows", [&](uint8_t* buf, size_t off, size_t n) {
    return par_fill(buf, n, threads,
                    [&](uint8_t* d, size_t o, size_t len) { return read_part(g->fd, file_off + off, d, o, len); });
  });
}
