// runtime.cpp -- the C-ABI of libwgx (include/wgx.h): contexts, owned device
// buffers, validated launch records, replay through a captured HIP graph.
//
// Mirrors WgpuExecutionContext (src/context.ts:17-390): buffers are owned by
// the context (storageBuffer / #ownedBuffers, context.ts:43-45,86-92),
// recordShader only validates and appends a command (context.ts:158-161,
// 201-205), submit replays the whole list in order (context.ts:323-370), sync
// waits (context.ts:377-380), reset drops the list (context.ts:386-389).
//
// MI355X-specific choices:
//  * one HIP stream per context; the command list is captured once into a
//    hipGraph and replayed with a single hipGraphLaunch per submit (re-captured
//    only when the list changes), so a ~300-launch program costs one submit;
//  * every tensor a record names must lie inside a buffer this context owns,
//    and its byte extent is checked against that buffer, so no recorded launch
//    can address memory outside the inputs and outputs it was given;
//  * implicit-im2col launches get their per-k {offset, tap} table built on
//    the host at record time (it depends only on shapes) and kept in a
//    context-owned device buffer.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"

using namespace wgx;

namespace {

struct Buf {
  uint64_t size;
  uint32_t usage;
  uint64_t serial;      // allocation number, so a recycled address is not mistaken for it
  const void* owner;    // the context that allocated it (freed with that context)
};

// (buffer base, allocation serial) pairs a command reads or writes
using Uses = std::vector<std::pair<uintptr_t, uint64_t>>;

// An LDS-patch convolution as recorded: what a paired launch needs, and the
// byte ranges it reads and writes (to tell whether two are independent).
struct ConvRec {
  ConvLdsDesc d;
  int cus;
  std::vector<std::pair<uintptr_t, uint64_t>> reads;  // (address, bytes)
  std::pair<uintptr_t, uint64_t> write;
};

struct Cmd {
  std::function<hipError_t(hipStream_t)> fn;
  std::string name;
  Uses uses;
  std::shared_ptr<ConvRec> conv;  // set for LDS-patch convolutions
};

bool ranges_overlap(const std::pair<uintptr_t, uint64_t>& a, const std::pair<uintptr_t, uint64_t>& b) {
  return a.first < b.first + b.second && b.first < a.first + a.second;
}

// Two recorded convolutions can run in one launch when neither writes what
// the other reads or writes.
bool independent(const ConvRec& a, const ConvRec& b) {
  if (ranges_overlap(a.write, b.write)) return false;
  for (const auto& r : b.reads)
    if (ranges_overlap(a.write, r)) return false;
  for (const auto& r : a.reads)
    if (ranges_overlap(b.write, r)) return false;
  return true;
}

// What every context on one device shares: the buffer registry and the queue
// (a single HIP stream), like a GPUDevice and its queue.
struct DeviceState {
  int device = -1;
  bool has_dev = false;
  hipStream_t stream = nullptr;
  std::string arch = "host";
  std::map<uintptr_t, Buf> bufs;
  uint64_t next_serial = 1;
  int refs = 0;
};

int elsize(int dt) {
  switch (dt) {
    case WGX_FLOAT32:
    case WGX_INT32:
      return 4;
    case WGX_FLOAT16:
    case WGX_BFLOAT16:
      return 2;
    case WGX_INT8:
    case WGX_UINT8:
    case WGX_BOOL:
      return 1;
    case WGX_FLOAT64:
    case WGX_INT64:
      return 8;
    default:
      return 0;
  }
}

const char* dtname(int dt) {
  switch (dt) {
    case WGX_FLOAT32: return "float32";
    case WGX_FLOAT16: return "float16";
    case WGX_BFLOAT16: return "bfloat16";
    case WGX_INT32: return "int32";
    case WGX_INT8: return "int8";
    case WGX_UINT8: return "uint8";
    case WGX_BOOL: return "bool";
    case WGX_FLOAT64: return "float64";
    case WGX_INT64: return "int64";
    default: return "?";
  }
}

bool is_float_gemm_dtype(int dt) {
  return dt == WGX_FLOAT32 || dt == WGX_FLOAT16 || dt == WGX_BFLOAT16;
}

long long numel(const wgx_tensor* t) {
  long long n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
  return n;
}

}  // namespace

struct wgx_ctx {
  DeviceState* d = nullptr;
  bool destroyed = false;
  Uses cur_uses;  // buffers named by the record call in progress
  std::vector<Cmd> cmds;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool graph_valid = false;
  int graph_mode = 1;
  std::string err;
  std::string last_kernel;
  int paired = 0;  // paired launches the last submit issued
  // the last command, when it is a mergeable max-pool (or a chain of them):
  // stride 1, padding K/2 ("same" size), dilation 1, square odd window
  struct PoolChain {
    int cmd = -1;  // index in cmds
    int dt, BC, H, W, P, n;
    const void* x;
    void* y[3];
    int32_t* idx[3];  // indices outputs (null: none)
    size_t bytes;     // of x and of every values output
  } pool;

  int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    err = buf;
    return code;
  }
  int hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? WGX_ERR_OOM : WGX_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
  }
  void invalidate() {
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    exec = nullptr;
    graph = nullptr;
    graph_valid = false;
  }
  // The owned buffer containing [p, p+bytes), or nullptr.
  const Buf* find(const void* p, uint64_t bytes, uint64_t* off = nullptr,
                  uintptr_t* base = nullptr) const {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = d->bufs.upper_bound(a);
    if (it == d->bufs.begin()) return nullptr;
    --it;
    const uint64_t o = a - it->first;
    if (o > it->second.size || bytes > it->second.size - o) return nullptr;
    if (off) *off = o;
    if (base) *base = it->first;
    return &it->second;
  }
  // find() that also notes the buffer as used by the record in progress
  const Buf* use(const void* p, uint64_t bytes) {
    uintptr_t base = 0;
    const Buf* b = find(p, bytes, nullptr, &base);
    if (b) cur_uses.emplace_back(base, b->serial);
    return b;
  }
  int check(const wgx_tensor* t, const char* what) {
    if (!t) return fail(WGX_ERR_INVALID, "%s: tensor is NULL", what);
    if (elsize(t->dtype) == 0) return fail(WGX_ERR_INVALID, "%s: unknown dtype %d", what, t->dtype);
    if (t->ndim < 0 || t->ndim > WGX_MAX_NDIM)
      return fail(WGX_ERR_INVALID, "%s: rank %d exceeds maximum rank of %d", what, t->ndim,
                  WGX_MAX_NDIM);
    for (int i = 0; i < t->ndim; ++i)
      if (t->shape[i] <= 0)
        return fail(WGX_ERR_INVALID, "%s: dimensions must be positive integers", what);
    const uint64_t bytes = (uint64_t)numel(t) * elsize(t->dtype);
    if (!use(t->data, bytes))
      return fail(WGX_ERR_INVALID, "%s: %llu bytes at %p are not inside a buffer of this context",
                  what, (unsigned long long)bytes, t->data);
    return WGX_OK;
  }
  hipStream_t dry() const { return d->has_dev ? describe_only() : name_only(); }
  int push(std::function<hipError_t(hipStream_t)> fn, const std::string& name) {
    last_kernel = name;
    cmds.push_back({std::move(fn), name, cur_uses});
    invalidate();
    return WGX_OK;
  }
  // Every buffer the recorded commands use must still be the allocation they
  // were recorded against.
  int check_uses() {
    for (const Cmd& cmd : cmds)
      for (const auto& u : cmd.uses) {
        auto it = d->bufs.find(u.first);
        if (it == d->bufs.end() || it->second.serial != u.second)
          return fail(WGX_ERR_INVALID, "submit: '%s' uses a destroyed buffer", cmd.name.c_str());
      }
    return WGX_OK;
  }
  void* owned_alloc(uint64_t bytes) {
    void* p = nullptr;
    if (d->has_dev) {
      if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
      // Zero-fill on the context's own stream and wait for it: the stream is
      // non-blocking, so a fill on the null stream would not be ordered with
      // the uploads and launches that follow on it (a late fill could land on
      // top of uploaded data).
      if (hipMemsetAsync(p, 0, bytes, d->stream) != hipSuccess || hipStreamSynchronize(d->stream) != hipSuccess) {
        hipFree(p);
        return nullptr;
      }
    } else {
      p = aligned_alloc(256, (bytes + 255) / 256 * 256);
      if (p) memset(p, 0, bytes);
    }
    if (p) d->bufs[reinterpret_cast<uintptr_t>(p)] = {bytes, 0, d->next_serial++, this};
    return p;
  }
  void release(uintptr_t base) {
    if (d->has_dev)
      hipFree(reinterpret_cast<void*>(base));
    else
      free(reinterpret_cast<void*>(base));
    d->bufs.erase(base);
  }
};

#define CTX_GUARD(c)                                                              \
  do {                                                                            \
    if (!(c)) return WGX_ERR_INVALID;                                             \
    if ((c)->destroyed) return (c)->fail(WGX_ERR_DESTROYED, "WgpuExecutionContext is destroyed"); \
    if ((c)->d->has_dev) hipSetDevice((c)->d->device);                            \
    (c)->cur_uses.clear();                                                        \
  } while (0)

extern "C" {

int wgx_ctx_create(int device, wgx_ctx** out) {
  if (!out) return WGX_ERR_INVALID;
  *out = nullptr;
  DeviceState* ds = new DeviceState();
  ds->device = device;
  if (device >= 0) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device >= n) {
      delete ds;
      return WGX_ERR_NO_DEVICE;
    }
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&ds->stream, hipStreamNonBlocking) != hipSuccess) {
      delete ds;
      return WGX_ERR_HIP;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
      std::string a = prop.gcnArchName;
      ds->arch = a.substr(0, a.find(':'));
    }
    ds->has_dev = true;
    // the no-allocation entry point's scratch address, looked up once per
    // device with the device current (a failure is kept and reported by
    // wgx_mm_noalloc; nothing else depends on it)
    void* scratch_ptr = nullptr;
    noalloc_scratch(device, &scratch_ptr);
  }
  wgx_ctx* c = new wgx_ctx();
  c->d = ds;
  ds->refs = 1;
  *out = c;
  return WGX_OK;
}

int wgx_ctx_create_shared(wgx_ctx* parent, wgx_ctx** out) {
  if (!parent || !out) return WGX_ERR_INVALID;
  *out = nullptr;
  if (parent->destroyed) return parent->fail(WGX_ERR_DESTROYED, "WgpuExecutionContext is destroyed");
  wgx_ctx* c = new wgx_ctx();
  c->d = parent->d;
  c->d->refs++;
  *out = c;
  return WGX_OK;
}

void wgx_ctx_destroy(wgx_ctx* c) {
  if (!c) return;
  DeviceState* ds = c->d;
  if (ds->has_dev) {
    hipSetDevice(ds->device);
    hipStreamSynchronize(ds->stream);
  }
  c->invalidate();
  std::vector<uintptr_t> mine;
  for (auto& kv : ds->bufs)
    if (kv.second.owner == c) mine.push_back(kv.first);
  for (uintptr_t b : mine) c->release(b);
  if (--ds->refs == 0) {
    std::vector<uintptr_t> rest;
    for (auto& kv : ds->bufs) rest.push_back(kv.first);
    for (uintptr_t b : rest) c->release(b);
    if (ds->has_dev && ds->stream) hipStreamDestroy(ds->stream);
    delete ds;
  }
  delete c;
}

int wgx_free(wgx_ctx* c, void* ptr) {
  CTX_GUARD(c);
  auto it = c->d->bufs.find(reinterpret_cast<uintptr_t>(ptr));
  if (it == c->d->bufs.end()) return c->fail(WGX_ERR_INVALID, "free: %p is not a buffer of this device", ptr);
  if (c->d->has_dev) {
    hipError_t e = hipStreamSynchronize(c->d->stream);
    if (e != hipSuccess) return c->hip_fail(e, "free");
  }
  c->release(it->first);
  return WGX_OK;
}

const char* wgx_last_error(const wgx_ctx* c) { return c ? c->err.c_str() : "null context"; }
int wgx_ctx_has_device(const wgx_ctx* c) { return c && c->d->has_dev ? 1 : 0; }
const char* wgx_ctx_arch(const wgx_ctx* c) { return c ? c->d->arch.c_str() : ""; }
void* wgx_ctx_stream(const wgx_ctx* c) { return c ? (void*)c->d->stream : nullptr; }
const char* wgx_last_kernel(const wgx_ctx* c) { return c ? c->last_kernel.c_str() : ""; }
int wgx_paired_launches(const wgx_ctx* c) { return c ? c->paired : 0; }
int wgx_command_count(const wgx_ctx* c) { return c ? (int)c->cmds.size() : 0; }

int wgx_alloc(wgx_ctx* c, uint64_t bytes, uint32_t usage, void** out) {
  CTX_GUARD(c);
  if (!out) return c->fail(WGX_ERR_INVALID, "alloc: out is NULL");
  const uint64_t sz = bytes < 4 ? 4 : (bytes + 3) / 4 * 4;
  void* p = c->owned_alloc(sz);
  if (!p) return c->fail(WGX_ERR_OOM, "alloc: could not allocate %llu bytes", (unsigned long long)sz);
  c->d->bufs[reinterpret_cast<uintptr_t>(p)].usage = usage;
  *out = p;
  return WGX_OK;
}

int wgx_buffer_info(const wgx_ctx* c, const void* ptr, uint64_t* base_offset, uint64_t* size,
                    uint32_t* usage) {
  if (!c) return WGX_ERR_INVALID;
  uint64_t off = 0;
  const Buf* b = c->find(ptr, 0, &off);
  if (!b) return WGX_ERR_INVALID;
  if (base_offset) *base_offset = off;
  if (size) *size = b->size;
  if (usage) *usage = b->usage;
  return WGX_OK;
}

int wgx_write(wgx_ctx* c, void* dst, const void* src, uint64_t bytes) {
  CTX_GUARD(c);
  if (bytes == 0) return WGX_OK;
  if (!c->find(dst, bytes)) return c->fail(WGX_ERR_INVALID, "write: destination range is not an owned buffer");
  if (!c->d->has_dev) {
    memcpy(dst, src, bytes);
    return WGX_OK;
  }
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->d->stream);
  return e == hipSuccess ? WGX_OK : c->hip_fail(e, "write");
}

int wgx_read(wgx_ctx* c, const void* src, void* dst, uint64_t bytes) {
  CTX_GUARD(c);
  if (bytes == 0) return WGX_OK;
  if (!c->find(src, bytes)) return c->fail(WGX_ERR_INVALID, "read: source range is not an owned buffer");
  if (!c->d->has_dev) {
    memcpy(dst, src, bytes);
    return WGX_OK;
  }
  hipError_t e = hipStreamSynchronize(c->d->stream);
  if (e == hipSuccess) e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
  return e == hipSuccess ? WGX_OK : c->hip_fail(e, "read");
}

int wgx_record_copy(wgx_ctx* c, void* dst, const void* src, uint64_t bytes) {
  CTX_GUARD(c);
  if (!c->use(src, bytes)) return c->fail(WGX_ERR_INVALID, "copy: source range is not an owned buffer");
  if (!c->use(dst, bytes)) return c->fail(WGX_ERR_INVALID, "copy: destination range is not an owned buffer");
  if (bytes == 0 || src == dst) {
    c->last_kernel = "copy_elided";
    return WGX_OK;
  }
  return c->push([=](hipStream_t s) { return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s); },
                 "copy_d2d");
}

// ------------------------------------------------------------------ GEMM family

// float32 runs on the matrix cores (v_mfma_f32_32x32x2_f32, twice the rate
// of unpacked vector FMA) when its operands are 16-byte vectors, else on the
// LDS-blocked vector-FMA kernel; WGX_F32_VECTOR_FMA=1 forces the latter.
static bool f32_on_mfma() {
  static int v = -1;
  if (v < 0) v = getenv("WGX_F32_VECTOR_FMA") ? 0 : 1;
  return v == 1;
}

// Compute units of the context's device (256 on MI355X; host-only contexts
// assume that).
static int device_cu_count(wgx_ctx* c) {
  int cus = 0;
  if (!c->d->has_dev ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->d->device) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

static int record_gemm(wgx_ctx* c, GemmDesc d) {
  std::string name;
  bool mfma = d.dtype != WGX_FLOAT32;
  hipError_t e = hipSuccess;
  d.splits = 1;
  if (d.dtype == WGX_FLOAT32 && f32_on_mfma()) {
    e = launch_gemm_mfma(d, c->dry(), &name);
    if (e == hipSuccess) mfma = true;
    else if (e != hipErrorNotSupported) return c->hip_fail(e, "kernel set-up");
  }
  if (mfma) {
    // split-K: the partial-sum workspace is owned by the context
    size_t ws_bytes = 0;
    const int splits = gemm_split_plan(d, &ws_bytes);
    if (splits > 1) {
      d.ws = static_cast<float*>(c->owned_alloc(ws_bytes));
      if (!d.ws) return c->fail(WGX_ERR_OOM, "gemm: split-K workspace allocation failed");
      d.splits = splits;
    }
    // a [K, N] B that the large-tile kernel reads as [N, K]: its staging copy
    const size_t bt_bytes = gemm_stage_b_bytes(d);
    if (bt_bytes > 0) {
      d.bt = c->owned_alloc(bt_bytes);
      if (!d.bt) return c->fail(WGX_ERR_OOM, "gemm: [N,K] staging workspace allocation failed");
    }
  }
  if (!mfma) e = launch_gemm_f32(d, c->dry(), &name);
  else e = launch_gemm_mfma(d, c->dry(), &name);
  if (e != hipSuccess) return c->hip_fail(e, "kernel set-up");
  if (!mfma) return c->push([d](hipStream_t s) { return launch_gemm_f32(d, s, nullptr); }, name);
  return c->push([d](hipStream_t s) { return launch_gemm_mfma(d, s, nullptr); }, name);
}

// Validates an mm / addmm and fills its GEMM description (shared by the
// recorded and the no-allocation entry points).
static int mm_desc(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, const wgx_tensor* bias,
                   const wgx_tensor* out, float alpha, float beta, uint32_t flags, GemmDesc* dp) {
  int r;
  if ((r = c->check(a, "mm: in1")) || (r = c->check(b, "mm: in2")) || (r = c->check(out, "mm: out")))
    return r;
  if (bias && (r = c->check(bias, "mm: bias"))) return r;
  if (!is_float_gemm_dtype(a->dtype) || b->dtype != a->dtype || out->dtype != a->dtype ||
      (bias && bias->dtype != a->dtype))
    return c->fail(WGX_ERR_INVALID, "mm: tensors must have matching float32, float16 or bfloat16 dtype");
  if (a->ndim != 2 || b->ndim != 2 || out->ndim != 2)
    return c->fail(WGX_ERR_INVALID, "mm: tensors must be 2D matrices");
  const bool tb = flags & WGX_MM_TRANS_B;
  const long long M = a->shape[0], K = a->shape[1];
  const long long K2 = tb ? b->shape[1] : b->shape[0];
  const long long N = tb ? b->shape[0] : b->shape[1];
  if (K != K2) return c->fail(WGX_ERR_INVALID, "mm: inner dimensions must match (%lld != %lld)", K, K2);
  if (out->shape[0] != M || out->shape[1] != N)
    return c->fail(WGX_ERR_INVALID, "mm: output shape [%lld, %lld] != expected [%lld, %lld]",
                   (long long)out->shape[0], (long long)out->shape[1], M, N);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || M * K > INT32_MAX || K * N > INT32_MAX || M * N > INT32_MAX)
    return c->fail(WGX_ERR_INVALID, "mm: matrices above 2^31 elements are not supported");
  GemmDesc d{};
  d.dtype = a->dtype;
  d.batch = 1;
  d.M = (int)M;
  d.N = (int)N;
  d.K = (int)K;
  d.A = a->data;
  d.lda = K;
  d.B = b->data;
  d.ldb = tb ? K : N;
  d.bmode = tb ? B_NK : B_KN;
  d.C = out->data;
  d.ldc = N;
  d.alpha = alpha;
  d.beta = beta;
  if (bias) {
    const long long bn = numel(bias);
    const bool per_col = bn == N && (bias->ndim == 1 || (bias->ndim == 2 && bias->shape[0] == 1));
    const bool per_row = bn == M && bias->ndim == 2 && bias->shape[1] == 1 && N != 1;
    if (per_col) d.bias_mode = BIAS_COL;
    else if (per_row) d.bias_mode = BIAS_ROW;
    else return c->fail(WGX_ERR_INVALID, "addmm: bias must broadcast as [N], [1,N] or [M,1]");
    d.bias = bias->data;
  }
  *dp = d;
  return WGX_OK;
}

int wgx_record_mm(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, const wgx_tensor* bias,
                  const wgx_tensor* out, float alpha, float beta, uint32_t flags) {
  CTX_GUARD(c);
  GemmDesc d{};
  if (int r = mm_desc(c, a, b, bias, out, alpha, beta, flags, &d)) return r;
  return record_gemm(c, d);
}

int wgx_mm_noalloc(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, const wgx_tensor* bias,
                   const wgx_tensor* out, float alpha, float beta, uint32_t flags) {
  CTX_GUARD(c);
  GemmDesc d{};
  if (int r = mm_desc(c, a, b, bias, out, alpha, beta, flags, &d)) return r;
  if (!c->d->has_dev) return c->fail(WGX_ERR_NO_DEVICE, "mm_noalloc: host-only context has no device");
  // the same kernel choice as record_gemm, with the workspace carved out of
  // the fixed per-device scratch array instead of context-owned memory
  std::string name;
  bool mfma = d.dtype != WGX_FLOAT32;
  hipError_t e = hipSuccess;
  d.splits = 1;
  if (d.dtype == WGX_FLOAT32 && f32_on_mfma()) {
    e = launch_gemm_mfma(d, describe_only(), &name);
    if (e == hipSuccess) mfma = true;
    else if (e != hipErrorNotSupported) return c->hip_fail(e, "mm_noalloc: kernel set-up");
  }
  if (mfma) {
    size_t ws_bytes = 0;
    const int splits = gemm_split_plan(d, &ws_bytes);
    const size_t bt_bytes = gemm_stage_b_bytes(d);
    const size_t ws_span = (ws_bytes + 255) / 256 * 256;
    if (ws_span + bt_bytes > WGX_NOALLOC_SCRATCH_BYTES)
      return c->fail(WGX_ERR_INVALID,
                     "mm_noalloc: this GEMM needs %llu bytes of workspace; the fixed scratch holds %u",
                     (unsigned long long)(ws_span + bt_bytes), (unsigned)WGX_NOALLOC_SCRATCH_BYTES);
    if (ws_span + bt_bytes > 0) {
      void* base = nullptr;
      e = noalloc_scratch(c->d->device, &base);
      if (e != hipSuccess) return c->hip_fail(e, "mm_noalloc: scratch address");
      // every split-K range writes all of its partial sums and the staging
      // pass writes the whole [N, K] copy before they are read, so nothing
      // left by an earlier call is ever read and nothing needs clearing
      if (splits > 1) {
        d.splits = splits;
        d.ws = static_cast<float*>(base);
      }
      if (bt_bytes > 0) d.bt = static_cast<char*>(base) + ws_span;
    }
    e = launch_gemm_mfma(d, describe_only(), &name);  // one-time kernel set-up (LDS limits)
    if (e == hipSuccess) e = launch_gemm_mfma(d, c->d->stream, nullptr);
  } else {
    e = launch_gemm_f32(d, describe_only(), &name);
    if (e == hipSuccess) e = launch_gemm_f32(d, c->d->stream, nullptr);
  }
  if (e != hipSuccess) return c->hip_fail(e, "mm_noalloc");
  c->last_kernel = name;
  return WGX_OK;
}

int wgx_record_bmm(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, const wgx_tensor* out,
                   uint32_t flags) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(a, "bmm: a")) || (r = c->check(b, "bmm: b")) || (r = c->check(out, "bmm: out")))
    return r;
  if (!is_float_gemm_dtype(a->dtype) || b->dtype != a->dtype || out->dtype != a->dtype)
    return c->fail(WGX_ERR_INVALID, "bmm: tensors must have matching float32, float16 or bfloat16 dtype");
  if (a->ndim != 3 || b->ndim != 3 || out->ndim != 3)
    return c->fail(WGX_ERR_INVALID, "bmm: inputs and output must be 3D");
  const bool tb = flags & WGX_MM_TRANS_B;
  const long long B = a->shape[0], M = a->shape[1], K = a->shape[2];
  const long long K2 = tb ? b->shape[2] : b->shape[1];
  const long long N = tb ? b->shape[1] : b->shape[2];
  if (b->shape[0] != B || K2 != K) return c->fail(WGX_ERR_INVALID, "bmm: batch/K mismatch between a and b");
  if (out->shape[0] != B || out->shape[1] != M || out->shape[2] != N)
    return c->fail(WGX_ERR_INVALID, "bmm: output shape != [%lld, %lld, %lld]", B, M, N);
  if (B > 65535) return c->fail(WGX_ERR_INVALID, "bmm: batch above 65535 is not supported");
  if (M * K > INT32_MAX || K * N > INT32_MAX || M * N > INT32_MAX)
    return c->fail(WGX_ERR_INVALID, "bmm: matrices above 2^31 elements are not supported");
  GemmDesc d{};
  d.dtype = a->dtype;
  d.batch = (int)B;
  d.M = (int)M;
  d.N = (int)N;
  d.K = (int)K;
  d.A = a->data;
  d.lda = K;
  d.sA = M * K;
  d.B = b->data;
  d.ldb = tb ? K : N;
  d.sB = K * N;
  d.bmode = tb ? B_NK : B_KN;
  d.C = out->data;
  d.ldc = N;
  d.sC = M * N;
  d.alpha = 1.0f;
  d.beta = 1.0f;
  return record_gemm(c, d);
}

// ------------------------------------------------------------------ convolution

// res (checked by the caller): an output-shaped tensor added after the
// epilogue, y = rcs * y + rrs * res; depthwise convolutions only.
static int record_conv(wgx_ctx* c, const wgx_tensor* in, const wgx_tensor* weight, const wgx_tensor* bias,
                       const wgx_conv_args* args, const wgx_tensor* res, float rcs, float rrs,
                       const wgx_tensor* out) {
  int r;
  if (!args) return c->fail(WGX_ERR_INVALID, "convolution: args is NULL");
  if ((r = c->check(in, "convolution: input")) || (r = c->check(weight, "convolution: weight")) ||
      (r = c->check(out, "convolution: output")))
    return r;
  if (bias && (r = c->check(bias, "convolution: bias"))) return r;
  const int dt = in->dtype;
  // bfloat16 is this library's addition (every convolution kernel here is
  // instantiated for it); the reference takes float32 and float16
  if ((dt != WGX_FLOAT32 && dt != WGX_FLOAT16 && dt != WGX_BFLOAT16) || weight->dtype != dt || out->dtype != dt)
    return c->fail(WGX_ERR_INVALID, "convolution: Tensors must have matching float32, float16 or bfloat16 dtype");
  if (bias && bias->dtype != dt) return c->fail(WGX_ERR_INVALID, "convolution: bias dtype must match input dtype");
  if (in->ndim != 4 || weight->ndim != 4 || out->ndim != 4)
    return c->fail(WGX_ERR_INVALID, "convolution: expected 4D tensors for input, weight, and output");
  const int sH = args->stride[0], sW = args->stride[1], pH = args->padding[0], pW = args->padding[1];
  const int dH = args->dilation[0], dW = args->dilation[1];
  const int opH = args->output_padding[0], opW = args->output_padding[1];
  const int groups = args->groups;
  if (sH <= 0 || sW <= 0 || dH <= 0 || dW <= 0 || pH < 0 || pW < 0 || groups <= 0)
    return c->fail(WGX_ERR_INVALID, "convolution: stride, dilation and groups must be positive, padding non-negative");
  const long long B = in->shape[0], IC = in->shape[1], IH = in->shape[2], IW = in->shape[3];
  const long long KH = weight->shape[2], KW = weight->shape[3];
  long long OC;
  if (IC % groups) return c->fail(WGX_ERR_INVALID, "convolution: IC (%lld) not divisible by groups (%d)", IC, groups);
  if (args->transposed) {
    OC = weight->shape[1] * groups;
    if (weight->shape[0] != IC)
      return c->fail(WGX_ERR_INVALID, "convolution: weight dim0 !== IC (%lld != %lld)", (long long)weight->shape[0], IC);
    if (opH >= sH || opW >= sW) return c->fail(WGX_ERR_INVALID, "convolution: output_padding >= stride");
    if (opH < 0 || opW < 0) return c->fail(WGX_ERR_INVALID, "convolution: negative output_padding");
    const long long eoh = (IH - 1) * sH - 2LL * pH + (long long)dH * (KH - 1) + opH + 1;
    const long long eow = (IW - 1) * sW - 2LL * pW + (long long)dW * (KW - 1) + opW + 1;
    if (out->shape[2] != eoh || out->shape[3] != eow)
      return c->fail(WGX_ERR_INVALID, "convolution: expected output spatial [%lld, %lld]", eoh, eow);
  } else {
    OC = weight->shape[0];
    if (opH != 0 || opW != 0)
      return c->fail(WGX_ERR_INVALID, "convolution: non-zero output_padding unsupported for non-transposed conv");
    if (weight->shape[1] * groups != IC)
      return c->fail(WGX_ERR_INVALID, "convolution: weight in-ch (%lld) != IC/groups (%lld)",
                     (long long)weight->shape[1], IC / groups);
    const long long ohn = IH + 2LL * pH - (long long)dH * (KH - 1) - 1;
    const long long own = IW + 2LL * pW - (long long)dW * (KW - 1) - 1;
    if (ohn < 0 || own < 0) return c->fail(WGX_ERR_INVALID, "convolution: invalid geometry (kernel larger than input)");
    const long long eoh = ohn / sH + 1, eow = own / sW + 1;
    if (out->shape[2] != eoh || out->shape[3] != eow)
      return c->fail(WGX_ERR_INVALID, "convolution: expected output spatial [%lld, %lld]", eoh, eow);
  }
  if (OC % groups) return c->fail(WGX_ERR_INVALID, "convolution: OC not divisible by groups");
  if (out->shape[0] != B || out->shape[1] != OC)
    return c->fail(WGX_ERR_INVALID, "convolution: expected output [%lld, %lld, ...]", B, OC);
  if (bias && numel(bias) != OC) return c->fail(WGX_ERR_INVALID, "convolution: bias must have OC elements");
  const long long OH = out->shape[2], OW = out->shape[3];
  if (B * IC * IH * IW > INT32_MAX || B * OC * OH * OW > INT32_MAX || numel(weight) > INT32_MAX)
    return c->fail(WGX_ERR_INVALID, "convolution: tensors above 2^31 elements are not supported");
  const int has_clamp = args->has_clamp ? 1 : 0;
  if (args->activation != WGX_ACT_NONE && args->activation != WGX_ACT_SILU)
    return c->fail(WGX_ERR_INVALID, "convolution: unknown activation %d", (int)args->activation);
  const int act = args->activation;
  const float cmin = args->clamp_min, cmax = args->clamp_max;

  const bool depthwise = !args->transposed && groups == OC && IC == OC && weight->shape[1] == 1;
  std::string name;
  hipError_t e;
  if (depthwise) {
    DwDesc d{};
    d.dtype = dt;
    d.B = (int)B;
    d.C = (int)IC;
    d.IH = (int)IH;
    d.IW = (int)IW;
    d.OH = (int)OH;
    d.OW = (int)OW;
    d.KH = (int)KH;
    d.KW = (int)KW;
    d.sH = sH;
    d.sW = sW;
    d.pH = pH;
    d.pW = pW;
    d.dH = dH;
    d.dW = dW;
    d.x = in->data;
    d.w = weight->data;
    d.bias = bias ? bias->data : nullptr;
    d.y = out->data;
    d.has_clamp = has_clamp;
    d.act = act;
    d.cmin = cmin;
    d.cmax = cmax;
    d.res = res ? res->data : nullptr;
    d.res_conv_scale = rcs;
    d.res_scale = rrs;
    e = launch_depthwise(d, c->dry(), &name);
    if (e == hipSuccess) return c->push([d](hipStream_t s) { return launch_depthwise(d, s, nullptr); }, name);
    // bands too wide for LDS: fall through to the direct kernel
  }
  // dense 3x3 convolutions over a multiple of 8 (float32) or 16 input channels: the
  // LDS-patch implicit GEMM (no per-element address work), the one dense
  // kernel with the residual epilogue
  if (!args->transposed && groups == 1 && dH == 1 && dW == 1) {
    ConvLdsDesc ld{};
    ld.dtype = dt;
    ld.B = (int)B;
    ld.IC = (int)IC;
    ld.IH = (int)IH;
    ld.IW = (int)IW;
    ld.OC = (int)OC;
    ld.OH = (int)OH;
    ld.OW = (int)OW;
    ld.KH = (int)KH;
    ld.KW = (int)KW;
    ld.sH = sH;
    ld.sW = sW;
    ld.pH = pH;
    ld.pW = pW;
    ld.x = in->data;
    ld.w = weight->data;
    ld.bias = bias ? bias->data : nullptr;
    ld.y = out->data;
    ld.act = act;
    ld.has_clamp = has_clamp;
    ld.cmin = cmin;
    ld.cmax = cmax;
    ld.res = res ? res->data : nullptr;
    ld.res_conv_scale = rcs;
    ld.res_scale = rrs;
    if (conv_lds_applies(ld)) {
      const int cus = device_cu_count(c);
      if (conv_lds_wants_prepass(ld, cus)) {
        ld.wpre = c->owned_alloc((uint64_t)numel(weight) * elsize(weight->dtype));
        if (!ld.wpre) return c->fail(WGX_ERR_OOM, "convolution: pre-ordered weight workspace allocation failed");
      }
      e = launch_conv_lds(ld, cus, c->dry(), &name);
      if (e == hipSuccess) {
        const int pr = c->push([ld, cus](hipStream_t s) { return launch_conv_lds(ld, cus, s, nullptr); }, name);
        auto rec = std::make_shared<ConvRec>();
        rec->d = ld;
        rec->cus = cus;
        auto range = [](const wgx_tensor* t) {
          return std::make_pair(reinterpret_cast<uintptr_t>(t->data), (uint64_t)numel(t) * elsize(t->dtype));
        };
        rec->reads.push_back(range(in));
        rec->reads.push_back(range(weight));
        if (bias) rec->reads.push_back(range(bias));
        if (res) rec->reads.push_back(range(res));
        rec->write = range(out);
        c->cmds.back().conv = rec;
        return pr;
      }
      if (e != hipErrorInvalidValue) return c->hip_fail(e, "kernel set-up");
      // a configuration whose LDS does not fit, or a many-tile float16 shape
      // that the GEMM kernels below run faster
    }
  }
  if (res)
    return c->fail(WGX_ERR_INVALID,
                   "convolution: a residual is supported on depthwise convolutions and on the dense 3x3 "
                   "convolutions the LDS-patch kernel takes");
  const ConvGeom geom{(int)IH, (int)IW, (int)OW, sH, sW, pH, pW, (int)KH, (int)KW, dH, dW};
  // A 1x1 convolution is a plain GEMM with the input plane as its [IC, H*W]
  // operand -- unless it has fewer 64 x 64 output tiles than CUs: then it
  // goes through the im2col form (a one-tap table) to the wave-split kernel,
  // which splits K over the waves of each tile (measured on the YOLO-N 640
  // frame, whose 1x1 convolutions at 80x80 and below have 28-200 tiles:
  // 527 -> 481 us).
  // The GEMM's im2col mode is built for float32 and float16 only: a bfloat16
  // 1x1 convolution always takes the plain [IC, H*W] form, other bfloat16
  // convolutions that the LDS-patch kernel does not take the direct kernel.
  const long long pw_tiles = (OC + 63) / 64 * ((OH * OW + 63) / 64) * B;
  const bool pointwise = KH == 1 && KW == 1 && sH == 1 && sW == 1 && pH == 0 && pW == 0 &&
                         (pw_tiles >= device_cu_count(c) || dt == WGX_BFLOAT16);
  // a few taps per output channel in a spatial kernel (network stems, K =
  // IC*KH*KW <= 32, KH*KW > 1): the direct small-tap kernel, not a GEMM with a
  // 1-2 step K loop ([1,3,640,640]*[16,3,3,3] s2: 14.7 against 28.4 us).  A
  // 1x1 convolution with few channels stays on the wave-split GEMM:
  // [1,32,80,80]*[32,32,1,1] 4.3 us there against 23.4 on the small-tap
  // kernel, [1,16,40,40]*[4,16,1,1] 4.4 against 8.2.
  const char* st_env = getenv("WGX_SMALL_TAPS");  // "0": never the small-tap kernel
  const bool small_taps = !args->transposed && groups == 1 && !pointwise && KH * KW > 1 && IC * KH * KW <= 32 &&
                          OC <= 64 && !(st_env && strcmp(st_env, "0") == 0);
  const bool gemm_ok = !args->transposed && groups == 1 && !small_taps &&
                       (pointwise || (dt != WGX_BFLOAT16 && conv_ktab_fits((int)(IC * KH * KW), (int)IC, geom)));
  if (gemm_ok) {
    GemmDesc d{};
    d.dtype = dt;
    d.batch = (int)B;
    d.M = (int)OC;
    d.N = (int)(OH * OW);
    d.K = (int)(IC * KH * KW);
    d.A = weight->data;
    d.lda = d.K;
    d.sA = 0;
    d.B = in->data;
    d.sB = IC * IH * IW;
    d.C = out->data;
    d.ldc = OH * OW;
    d.sC = OC * OH * OW;
    d.bias = bias ? bias->data : nullptr;
    d.bias_mode = BIAS_ROW;
    d.alpha = 1.0f;
    d.beta = 1.0f;
    d.has_clamp = has_clamp;
    d.act = act;
    d.cmin = cmin;
    d.cmax = cmax;
    d.g = geom;
    if (pointwise) {
      d.bmode = B_KN;  // x[b] is already the [IC, H*W] operand
      d.ldb = IH * IW;
    } else {
      d.bmode = B_CONV;
      const int rows = conv_ktab_rows(d.K);
      std::vector<uint32_t> tab(rows);
      conv_fill_ktab(tab.data(), d.K, (int)IC, d.g);
      void* dev = c->owned_alloc(sizeof(uint32_t) * rows);
      if (!dev) return c->fail(WGX_ERR_OOM, "convolution: im2col table allocation failed");
      if (c->d->has_dev) {
        e = hipMemcpy(dev, tab.data(), sizeof(uint32_t) * rows, hipMemcpyHostToDevice);
        if (e != hipSuccess) return c->hip_fail(e, "convolution: im2col table upload");
      } else {
        memcpy(dev, tab.data(), sizeof(uint32_t) * rows);
      }
      d.ktab = static_cast<const uint32_t*>(dev);
    }
    return record_gemm(c, d);
  }
  DirectConvDesc d{};
  d.dtype = dt;
  d.transposed = args->transposed ? 1 : 0;
  d.B = (int)B;
  d.IC = (int)IC;
  d.IH = (int)IH;
  d.IW = (int)IW;
  d.OC = (int)OC;
  d.OH = (int)OH;
  d.OW = (int)OW;
  d.KH = (int)KH;
  d.KW = (int)KW;
  d.sH = sH;
  d.sW = sW;
  d.pH = pH;
  d.pW = pW;
  d.dH = dH;
  d.dW = dW;
  d.groups = groups;
  d.x = in->data;
  d.w = weight->data;
  d.bias = bias ? bias->data : nullptr;
  d.y = out->data;
  d.has_clamp = has_clamp;
  d.act = act;
  d.cmin = cmin;
  d.cmax = cmax;
  e = launch_direct_conv(d, c->dry(), &name);
  if (e != hipSuccess) return c->hip_fail(e, "kernel set-up");
  return c->push([d](hipStream_t s) { return launch_direct_conv(d, s, nullptr); }, name);
}

int wgx_record_conv2d(wgx_ctx* c, const wgx_tensor* in, const wgx_tensor* weight,
                      const wgx_tensor* bias, const wgx_conv_args* args, const wgx_tensor* out) {
  CTX_GUARD(c);
  return record_conv(c, in, weight, bias, args, nullptr, 1.0f, 0.0f, out);
}

int wgx_record_conv2d_residual(wgx_ctx* c, const wgx_tensor* in, const wgx_tensor* weight,
                               const wgx_tensor* bias, const wgx_conv_args* args,
                               const wgx_tensor* residual, float conv_scale, float residual_scale,
                               const wgx_tensor* out) {
  CTX_GUARD(c);
  int r;
  if (!residual) return c->fail(WGX_ERR_INVALID, "convolution: residual is NULL");
  if ((r = c->check(residual, "convolution: residual")) || (r = c->check(out, "convolution: output"))) return r;
  if (residual->dtype != out->dtype || residual->ndim != out->ndim)
    return c->fail(WGX_ERR_INVALID, "convolution: residual must match the output's dtype and shape");
  for (int i = 0; i < out->ndim; ++i)
    if (residual->shape[i] != out->shape[i])
      return c->fail(WGX_ERR_INVALID, "convolution: residual must match the output's dtype and shape");
  // element i of the output reads element i of the residual: the same
  // memory is fine, a shifted overlap is not
  const uintptr_t rb = reinterpret_cast<uintptr_t>(residual->data), ob = reinterpret_cast<uintptr_t>(out->data);
  const uintptr_t bytes = (uintptr_t)numel(out) * elsize(out->dtype);
  if (rb != ob && rb < ob + bytes && ob < rb + bytes)
    return c->fail(WGX_ERR_INVALID, "convolution: residual partly overlaps the output");
  return record_conv(c, in, weight, bias, args, residual, conv_scale, residual_scale, out);
}

// ------------------------------------------------------------------ simple ops

static int float_dt(int dt) { return dt == WGX_FLOAT32 || dt == WGX_FLOAT16 || dt == WGX_BFLOAT16; }

static int record_binary(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, const wgx_tensor* out,
                         float alpha, int op, const char* opname) {
  int r;
  if ((r = c->check(a, opname)) || (r = c->check(b, opname)) || (r = c->check(out, opname))) return r;
  if (!float_dt(a->dtype) || b->dtype != a->dtype || out->dtype != a->dtype)
    return c->fail(WGX_ERR_INVALID, "%s: tensors must have matching float dtype", opname);
  if (a->ndim > out->ndim || b->ndim > out->ndim)
    return c->fail(WGX_ERR_INVALID, "%s: input rank exceeds output rank", opname);
  BcastDesc d{};
  d.dtype = a->dtype;
  d.ndim = out->ndim;
  d.numel = numel(out);
  d.a = a->data;
  d.b = b->data;
  d.out = out->data;
  d.alpha = alpha;
  d.op = op;
  long long sa = 1, sb = 1;
  for (int k = out->ndim - 1; k >= 0; --k) {
    const int ka = k - (out->ndim - a->ndim), kb = k - (out->ndim - b->ndim);
    const long long da = ka >= 0 ? a->shape[ka] : 1, db = kb >= 0 ? b->shape[kb] : 1;
    const long long o = out->shape[k];
    if ((da != o && da != 1) || (db != o && db != 1))
      return c->fail(WGX_ERR_INVALID, "%s: shapes do not broadcast to the output", opname);
    d.out_shape[k] = o;
    d.a_stride[k] = da == 1 ? 0 : sa;
    d.b_stride[k] = db == 1 ? 0 : sb;
    sa *= da;
    sb *= db;
  }
  std::string name;
  launch_binary(d, c->dry(), &name);
  return c->push([d](hipStream_t s) { return launch_binary(d, s, nullptr); }, name);
}

int wgx_record_add(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, float alpha, int subtract,
                   const wgx_tensor* out) {
  CTX_GUARD(c);
  return record_binary(c, a, b, out, subtract ? -alpha : alpha, 0, subtract ? "sub" : "add");
}

int wgx_record_mul(wgx_ctx* c, const wgx_tensor* a, const wgx_tensor* b, const wgx_tensor* out) {
  CTX_GUARD(c);
  return record_binary(c, a, b, out, 1.0f, 1, "mul");
}

int wgx_record_unary(wgx_ctx* c, int op, const wgx_tensor* in, const wgx_tensor* out) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(in, "unary: in")) || (r = c->check(out, "unary: out"))) return r;
  if (op < 0 || op > 3) return c->fail(WGX_ERR_INVALID, "unary: unknown op %d", op);
  if (!float_dt(in->dtype) || out->dtype != in->dtype || numel(in) != numel(out))
    return c->fail(WGX_ERR_INVALID, "unary: input and output must have the same float dtype and size");
  const int dt = in->dtype;
  const long long n = numel(in);
  const void* x = in->data;
  void* y = out->data;
  std::string name;
  launch_unary(op, dt, n, x, y, c->dry(), &name);
  return c->push([=](hipStream_t s) { return launch_unary(op, dt, n, x, y, s, nullptr); }, name);
}

static int norm_dim(int dim, int ndim) { return dim < 0 ? dim + ndim : dim; }

int wgx_record_cat(wgx_ctx* c, const wgx_tensor* inputs, int n_inputs, int dim, const wgx_tensor* out) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(out, "cat: out"))) return r;
  if (n_inputs <= 0 || !inputs) return c->fail(WGX_ERR_INVALID, "cat: no inputs");
  const int d = norm_dim(dim, out->ndim);
  if (d < 0 || d >= out->ndim) return c->fail(WGX_ERR_INVALID, "cat: dim out of range");
  long long total = 0;
  for (int i = 0; i < n_inputs; ++i) {
    const wgx_tensor* t = &inputs[i];
    if ((r = c->check(t, "cat: input"))) return r;
    if (t->dtype != out->dtype || t->ndim != out->ndim)
      return c->fail(WGX_ERR_INVALID, "cat: inputs must match the output dtype and rank");
    for (int k = 0; k < out->ndim; ++k)
      if (k != d && t->shape[k] != out->shape[k])
        return c->fail(WGX_ERR_INVALID, "cat: input %d shape mismatch at dim %d", i, k);
    total += t->shape[d];
  }
  if (total != out->shape[d]) return c->fail(WGX_ERR_INVALID, "cat: sizes along dim do not add up");
  long long outer = 1, inner = 1;
  for (int k = 0; k < d; ++k) outer *= out->shape[k];
  for (int k = d + 1; k < out->ndim; ++k) inner *= out->shape[k];
  const int es = elsize(out->dtype);
  long long off = 0;
  for (int i = 0; i < n_inputs; ++i) {
    const long long is = inputs[i].shape[d] * inner, os = out->shape[d] * inner, doff = off * inner;
    const void* src = inputs[i].data;
    void* dst = out->data;
    std::string name;
    launch_slab_copy(es, outer, is, os, doff, 0, src, dst, false, c->dry(), &name);
    c->push([=](hipStream_t s) { return launch_slab_copy(es, outer, is, os, doff, 0, src, dst, false, s, nullptr); },
            name);
    off += inputs[i].shape[d];
  }
  return WGX_OK;
}

int wgx_record_split(wgx_ctx* c, const wgx_tensor* in, int dim, const wgx_tensor* outputs, int n_outputs) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(in, "split: in"))) return r;
  if (n_outputs <= 0 || !outputs) return c->fail(WGX_ERR_INVALID, "split: no outputs");
  const int d = norm_dim(dim, in->ndim);
  if (d < 0 || d >= in->ndim) return c->fail(WGX_ERR_INVALID, "split: dim out of range");
  long long total = 0;
  for (int i = 0; i < n_outputs; ++i) {
    const wgx_tensor* t = &outputs[i];
    if ((r = c->check(t, "split: output"))) return r;
    if (t->dtype != in->dtype || t->ndim != in->ndim)
      return c->fail(WGX_ERR_INVALID, "split: outputs must match the input dtype and rank");
    for (int k = 0; k < in->ndim; ++k)
      if (k != d && t->shape[k] != in->shape[k])
        return c->fail(WGX_ERR_INVALID, "split: output %d shape mismatch at dim %d", i, k);
    total += t->shape[d];
  }
  if (total != in->shape[d]) return c->fail(WGX_ERR_INVALID, "split: sizes along dim do not add up");
  long long outer = 1, inner = 1;
  for (int k = 0; k < d; ++k) outer *= in->shape[k];
  for (int k = d + 1; k < in->ndim; ++k) inner *= in->shape[k];
  const int es = elsize(in->dtype);
  long long off = 0;
  for (int i = 0; i < n_outputs; ++i) {
    const long long is = in->shape[d] * inner, os = outputs[i].shape[d] * inner, soff = off * inner;
    const void* src = in->data;
    void* dst = outputs[i].data;
    std::string name;
    launch_slab_copy(es, outer, is, os, 0, soff, src, dst, true, c->dry(), &name);
    c->push([=](hipStream_t s) { return launch_slab_copy(es, outer, is, os, 0, soff, src, dst, true, s, nullptr); },
            name);
    off += outputs[i].shape[d];
  }
  return WGX_OK;
}

int wgx_record_upsample_nearest2d(wgx_ctx* c, const wgx_tensor* in, const wgx_tensor* out) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(in, "upsample: in")) || (r = c->check(out, "upsample: out"))) return r;
  if (!float_dt(in->dtype) || out->dtype != in->dtype || in->ndim != 4 || out->ndim != 4 ||
      in->shape[0] != out->shape[0] || in->shape[1] != out->shape[1])
    return c->fail(WGX_ERR_INVALID, "upsample: expected 4D float tensors with matching N, C");
  const int dt = in->dtype;
  const int BC = (int)(in->shape[0] * in->shape[1]);
  const int IH = (int)in->shape[2], IW = (int)in->shape[3], OH = (int)out->shape[2], OW = (int)out->shape[3];
  const void* x = in->data;
  void* y = out->data;
  std::string name;
  launch_upsample_nearest(dt, BC, IH, IW, OH, OW, x, y, c->dry(), &name);
  return c->push([=](hipStream_t s) { return launch_upsample_nearest(dt, BC, IH, IW, OH, OW, x, y, s, nullptr); },
                 name);
}

int wgx_record_max_pool2d(wgx_ctx* c, const wgx_tensor* in, const int32_t kernel[2], const int32_t stride[2],
                          const int32_t padding[2], const int32_t dilation[2], int ceil_mode, const wgx_tensor* out,
                          const wgx_tensor* indices) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(in, "max_pool2d: in")) || (r = c->check(out, "max_pool2d: out"))) return r;
  if (indices && (r = c->check(indices, "max_pool2d: indices"))) return r;
  if (!float_dt(in->dtype) || out->dtype != in->dtype || in->ndim != 4 || out->ndim != 4)
    return c->fail(WGX_ERR_INVALID, "max_pool2d: expected 4D float tensors");
  if (!kernel || !stride || !padding || !dilation)
    return c->fail(WGX_ERR_INVALID, "max_pool2d: kernel, stride, padding and dilation are required");
  const int KH = kernel[0], KW = kernel[1], sH = stride[0], sW = stride[1], pH = padding[0], pW = padding[1];
  const int dH = dilation[0], dW = dilation[1];
  if (KH <= 0 || KW <= 0 || sH <= 0 || sW <= 0 || dH <= 0 || dW <= 0 || pH < 0 || pW < 0)
    return c->fail(WGX_ERR_INVALID, "max_pool2d: invalid kernel/stride/padding/dilation");
  const long long IH = in->shape[2], IW = in->shape[3];
  // floor or ceil of the window count, at least 0 (max-pool-2d/index.ts:73-78)
  auto count = [&](long long num, int s) {
    const long long q = ceil_mode ? (num >= 0 ? (num + s - 1) / s : -((-num) / s)) : (num >= 0 ? num / s : -((-num + s - 1) / s));
    return q + 1 < 0 ? 0LL : q + 1;
  };
  const long long eoh = count(IH + 2LL * pH - ((long long)dH * (KH - 1) + 1), sH);
  const long long eow = count(IW + 2LL * pW - ((long long)dW * (KW - 1) + 1), sW);
  if (out->shape[0] != in->shape[0] || out->shape[1] != in->shape[1] || out->shape[2] != eoh || out->shape[3] != eow)
    return c->fail(WGX_ERR_INVALID, "max_pool2d: expected output spatial [%lld, %lld]", eoh, eow);
  if (indices) {
    if (indices->dtype != WGX_INT32) return c->fail(WGX_ERR_INVALID, "max_pool2d: indices output must be int32");
    if (indices->ndim != 4)
      return c->fail(WGX_ERR_INVALID, "max_pool2d: indices output must have the values' shape");
    for (int k = 0; k < 4; ++k)
      if (indices->shape[k] != out->shape[k])
        return c->fail(WGX_ERR_INVALID, "max_pool2d: indices output must have the values' shape");
  }
  const int dt = in->dtype;
  const int BC = (int)(in->shape[0] * in->shape[1]);
  const void* x = in->data;
  void* y = out->data;
  int32_t* ix = indices ? static_cast<int32_t*>(indices->data) : nullptr;
  const int ih = (int)IH, iw = (int)IW, oh = (int)eoh, ow = (int)eow;
  std::string name;
  // Consecutive records of the same "same-size" pool, each pooling the
  // previous output (the SPPF block of YOLO-style detectors), fold into the
  // previous command: one launch writes the 2 or 3 levels.  The folded
  // launch reads x once, up front, per plane, and then writes every level,
  // so each output must be disjoint from x and from every other output
  // (index outputs may also be the very same memory: a lane writes the
  // levels of a pixel in order, so the last level's index stays, as after
  // separate launches).
  const bool same = KH == KW && (KH & 1) && sH == 1 && sW == 1 && pH == KH / 2 && pW == KW / 2 && dH == 1 &&
                    dW == 1 && oh == ih && ow == iw && max_pool_chain_lds(ih, iw, KH / 2) <= 64 * 1024;
  const size_t bytes = (size_t)BC * ih * iw * elsize(dt), ibytes = (size_t)BC * ih * iw * 4;
  auto disjoint = [](const void* a, size_t na, const void* b, size_t nb) {
    const char *pa = static_cast<const char*>(a), *pb = static_cast<const char*>(b);
    return !a || !b || pa + na <= pb || pb + nb <= pa;
  };
  auto& pc = c->pool;
  if (same && pc.cmd >= 0 && pc.cmd == (int)c->cmds.size() - 1 && pc.n < 3 && pc.y[pc.n - 1] == x &&
      pc.dt == dt && pc.BC == BC && pc.H == ih && pc.W == iw && pc.P == KH / 2) {
    bool ok = disjoint(y, bytes, pc.x, bytes) && disjoint(ix, ibytes, pc.x, bytes) && disjoint(ix, ibytes, y, bytes);
    for (int k = 0; k < pc.n; ++k) {
      ok = ok && disjoint(y, bytes, pc.y[k], bytes) && disjoint(y, bytes, pc.idx[k], ibytes) &&
           disjoint(ix, ibytes, pc.y[k], bytes) && (ix == pc.idx[k] || disjoint(ix, ibytes, pc.idx[k], ibytes));
    }
    if (ok) {
      pc.y[pc.n] = y;
      pc.idx[pc.n] = ix;
      pc.n++;
      const auto q = pc;
      launch_max_pool_chain(dt, BC, ih, iw, q.P, q.n, q.x, q.y, q.idx, c->dry(), &name);
      Cmd& last = c->cmds.back();
      last.fn = [q](hipStream_t s) {
        return launch_max_pool_chain(q.dt, q.BC, q.H, q.W, q.P, q.n, q.x, q.y, q.idx, s, nullptr);
      };
      last.name = name;
      for (const auto& u : c->cur_uses) last.uses.push_back(u);
      c->last_kernel = name;
      c->invalidate();
      return WGX_OK;
    }
  }
  launch_max_pool(dt, BC, ih, iw, oh, ow, KH, KW, sH, sW, pH, pW, dH, dW, x, y, ix, c->dry(), &name);
  const int r2 = c->push([=](hipStream_t s) {
    return launch_max_pool(dt, BC, ih, iw, oh, ow, KH, KW, sH, sW, pH, pW, dH, dW, x, y, ix, s, nullptr);
  }, name);
  if (r2 == WGX_OK && same && disjoint(x, bytes, y, bytes) && disjoint(x, bytes, ix, ibytes) &&
      disjoint(y, bytes, ix, ibytes)) {
    pc.cmd = (int)c->cmds.size() - 1;
    pc.dt = dt;
    pc.BC = BC;
    pc.H = ih;
    pc.W = iw;
    pc.P = KH / 2;
    pc.n = 1;
    pc.x = x;
    pc.y[0] = y;
    pc.y[1] = pc.y[2] = nullptr;
    pc.idx[0] = ix;
    pc.idx[1] = pc.idx[2] = nullptr;
    pc.bytes = bytes;
  }
  return r2;
}

int wgx_record_permute(wgx_ctx* c, const wgx_tensor* in, const int32_t* dims, int n_dims, const wgx_tensor* out) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(in, "permute: in")) || (r = c->check(out, "permute: out"))) return r;
  if (out->dtype != in->dtype) return c->fail(WGX_ERR_INVALID, "permute: input and output dtypes differ");
  const int rank = in->ndim;
  if (out->ndim != rank) return c->fail(WGX_ERR_INVALID, "permute: output rank != input rank");
  if (n_dims != rank || (rank > 0 && !dims))
    return c->fail(WGX_ERR_INVALID, "permute: dims count (%d) != input rank (%d)", n_dims, rank);
  PermuteDesc d{};
  d.elsize = elsize(in->dtype);
  d.ndim = rank;
  unsigned seen = 0;
  for (int k = 0; k < rank; ++k) {
    int p = dims[k] < 0 ? dims[k] + rank : dims[k];
    if (p < 0 || p >= rank || (seen >> p & 1u)) return c->fail(WGX_ERR_INVALID, "permute: invalid permute dims");
    seen |= 1u << p;
    d.perm[k] = p;
    d.in_shape[k] = in->shape[k];
  }
  for (int k = 0; k < rank; ++k)
    if (out->shape[k] != in->shape[d.perm[k]])
      return c->fail(WGX_ERR_INVALID, "permute: output shape does not match permuted input shape");
  d.x = in->data;
  d.y = out->data;
  const uintptr_t xb = reinterpret_cast<uintptr_t>(in->data), yb = reinterpret_cast<uintptr_t>(out->data);
  const uintptr_t nb = (uintptr_t)numel(in) * d.elsize;
  if (xb < yb + nb && yb < xb + nb) return c->fail(WGX_ERR_INVALID, "permute: output overlaps the input");
  std::string name;
  launch_permute(d, c->dry(), &name);
  return c->push([d](hipStream_t s) { return launch_permute(d, s, nullptr); }, name);
}

int wgx_record_softmax(wgx_ctx* c, const wgx_tensor* in, int dim, const wgx_tensor* out) {
  CTX_GUARD(c);
  int r;
  if ((r = c->check(in, "softmax: in")) || (r = c->check(out, "softmax: out"))) return r;
  if (!float_dt(in->dtype) || out->dtype != in->dtype)
    return c->fail(WGX_ERR_INVALID, "softmax: Tensors must have matching float dtype");
  if (in->ndim == 0) return c->fail(WGX_ERR_INVALID, "softmax: scalar input unsupported");
  if (numel(in) != numel(out)) return c->fail(WGX_ERR_INVALID, "softmax: input/output numel mismatch");
  const int d = norm_dim(dim, in->ndim);
  if (d < 0 || d >= in->ndim) return c->fail(WGX_ERR_INVALID, "softmax: dim out of range");
  long long outer = 1, inner = 1;
  for (int k = 0; k < d; ++k) outer *= in->shape[k];
  for (int k = d + 1; k < in->ndim; ++k) inner *= in->shape[k];
  const long long rr = in->shape[d];
  const int dt = in->dtype;
  const void* x = in->data;
  void* y = out->data;
  // a line is read twice (max/sum, then the outputs): the output may be the
  // input itself, but must not overlap it otherwise
  const uintptr_t xb = reinterpret_cast<uintptr_t>(x), yb = reinterpret_cast<uintptr_t>(y);
  const uintptr_t nb = (uintptr_t)numel(in) * elsize(dt);
  if (xb != yb && xb < yb + nb && yb < xb + nb)
    return c->fail(WGX_ERR_INVALID, "softmax: output partly overlaps the input");
  std::string name;
  launch_softmax(dt, outer, rr, inner, x, y, c->dry(), &name);
  return c->push([=](hipStream_t s) { return launch_softmax(dt, outer, rr, inner, x, y, s, nullptr); }, name);
}

// ------------------------------------------------------------------ execution

// Issues the recorded commands on the context's stream in order; two
// adjacent independent LDS-patch convolutions that both take the float32
// batch-1 configuration go out as one paired launch.
static int issue_all(wgx_ctx* c) {
  const size_t n = c->cmds.size();
  c->paired = 0;
  for (size_t i = 0; i < n; ++i) {
    const Cmd& cmd = c->cmds[i];
    if (cmd.conv && i + 1 < n && c->cmds[i + 1].conv && independent(*cmd.conv, *c->cmds[i + 1].conv)) {
      const hipError_t e = launch_conv_lds_pair(cmd.conv->d, c->cmds[i + 1].conv->d, cmd.conv->cus, c->d->stream);
      if (e == hipSuccess) {
        ++c->paired;
        ++i;
        continue;
      }
      if (e != hipErrorNotSupported) return c->hip_fail(e, cmd.name.c_str());
    }
    const hipError_t e = cmd.fn(c->d->stream);
    if (e != hipSuccess) return c->hip_fail(e, cmd.name.c_str());
  }
  return WGX_OK;
}

static int run_eager(wgx_ctx* c) { return issue_all(c); }

// Command lists shorter than this run as direct launches even in graph
// mode: one graph launch of a single kernel node costs more than the launch
// it replaces (the paired float32 headline step: 31.9 us per submit through
// a graph, 26.8 us issued directly).  WGX_GRAPH_MIN=n moves the threshold.
static size_t graph_min_cmds() {
  const char* e = getenv("WGX_GRAPH_MIN");  // read per submit: a test may change it
  return e ? (size_t)std::max(0L, strtol(e, nullptr, 10)) : 3;
}

int wgx_submit(wgx_ctx* c) {
  CTX_GUARD(c);
  if (c->cmds.empty()) return WGX_OK;
  if (!c->d->has_dev) return c->fail(WGX_ERR_NO_DEVICE, "submit: host-only context has no device");
  if (int r = c->check_uses()) return r;
  if (!c->graph_mode || c->cmds.size() < graph_min_cmds()) return run_eager(c);
  if (!c->graph_valid) {
    hipError_t e = hipStreamBeginCapture(c->d->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return c->hip_fail(e, "submit: begin capture");
    const int r = issue_all(c);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(c->d->stream, &g);
    if (r != WGX_OK) {
      if (g) hipGraphDestroy(g);
      return r;
    }
    if (e2 != hipSuccess) return c->hip_fail(e2, "submit: end capture");
    c->graph = g;
    e = hipGraphInstantiate(&c->exec, c->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      c->invalidate();
      return c->hip_fail(e, "submit: graph instantiate");
    }
    c->graph_valid = true;
  }
  hipError_t e = hipGraphLaunch(c->exec, c->d->stream);
  return e == hipSuccess ? WGX_OK : c->hip_fail(e, "submit: graph launch");
}

int wgx_sync(wgx_ctx* c) {
  CTX_GUARD(c);
  if (!c->d->has_dev) return WGX_OK;
  hipError_t e = hipStreamSynchronize(c->d->stream);
  return e == hipSuccess ? WGX_OK : c->hip_fail(e, "sync");
}

}  // extern "C"

struct wgx_fence {
  int device = -1;
  hipEvent_t ev = nullptr;  // null: nothing to wait for (host-only context)
  std::string err;
};

extern "C" {

int wgx_fence_record(wgx_ctx* c, wgx_fence** out) {
  CTX_GUARD(c);
  if (!out) return c->fail(WGX_ERR_INVALID, "sync: out is NULL");
  *out = nullptr;
  wgx_fence* f = new wgx_fence();
  if (c->d->has_dev) {
    f->device = c->d->device;
    hipError_t e = hipEventCreateWithFlags(&f->ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(f->ev, c->d->stream);
    if (e != hipSuccess) {
      if (f->ev) hipEventDestroy(f->ev);
      delete f;
      return c->hip_fail(e, "sync");
    }
  }
  *out = f;
  return WGX_OK;
}

int wgx_fence_wait(wgx_fence* f) {
  if (!f) return WGX_ERR_INVALID;
  if (!f->ev) return WGX_OK;
  hipSetDevice(f->device);
  const hipError_t e = hipEventSynchronize(f->ev);
  if (e == hipSuccess) return WGX_OK;
  f->err = std::string("sync: ") + hipGetErrorString(e);
  return WGX_ERR_HIP;
}

const char* wgx_fence_error(const wgx_fence* f) { return f ? f->err.c_str() : "null fence"; }

void wgx_fence_destroy(wgx_fence* f) {
  if (!f) return;
  if (f->ev) {
    hipSetDevice(f->device);
    hipEventDestroy(f->ev);
  }
  delete f;
}

int wgx_reset(wgx_ctx* c) {
  CTX_GUARD(c);
  c->cmds.clear();
  c->pool.cmd = -1;
  c->invalidate();
  return WGX_OK;
}

int wgx_set_graph_mode(wgx_ctx* c, int enabled) {
  CTX_GUARD(c);
  c->graph_mode = enabled ? 1 : 0;
  c->invalidate();
  return WGX_OK;
}

int wgx_time_submits(wgx_ctx* c, int reps, float* ms_per_submit) {
  CTX_GUARD(c);
  if (!c->d->has_dev) return c->fail(WGX_ERR_NO_DEVICE, "time: host-only context has no device");
  if (reps <= 0 || !ms_per_submit) return c->fail(WGX_ERR_INVALID, "time: reps must be positive");
  hipEvent_t a, b;
  hipError_t e = hipEventCreate(&a);
  if (e != hipSuccess) return c->hip_fail(e, "time: event");
  e = hipEventCreate(&b);
  if (e != hipSuccess) {
    hipEventDestroy(a);
    return c->hip_fail(e, "time: event");
  }
  int r = WGX_OK;
  e = hipEventRecord(a, c->d->stream);
  for (int i = 0; i < reps && e == hipSuccess && r == WGX_OK; ++i) r = wgx_submit(c);
  if (e == hipSuccess && r == WGX_OK) e = hipEventRecord(b, c->d->stream);
  if (e == hipSuccess && r == WGX_OK) e = hipEventSynchronize(b);
  float ms = 0.f;
  if (e == hipSuccess && r == WGX_OK) e = hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (r != WGX_OK) return r;
  if (e != hipSuccess) return c->hip_fail(e, "time");
  *ms_per_submit = ms / reps;
  return WGX_OK;
}

}  // extern "C"
