// addon.cc -- N-API binding of libwgx (include/wgx.h) for the Node host layer.
//
// The JS side (index.js) keeps the reference's API (src/context.ts,
// src/tensor.ts, src/shader.ts, src/program.ts); this addon is the thin
// JS <-> C-ABI bridge it calls.  Handles are N-API externals wrapping a
// wgx_ctx*; device addresses cross as JS numbers (GPU virtual addresses fit
// in 53 bits); tensors cross as {ptr, dtype, shape}.  Every non-zero status
// becomes a thrown Error carrying wgx_last_error().
#define NAPI_VERSION 6
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "wgx.h"

namespace {

#define NAPI_CALL(env, call)                                   \
  do {                                                         \
    if ((call) != napi_ok) {                                   \
      napi_throw_error((env), nullptr, "napi call failed: " #call); \
      return nullptr;                                          \
    }                                                          \
  } while (0)

struct Args {
  size_t argc = 12;
  napi_value argv[12];
};

bool get_args(napi_env env, napi_callback_info info, Args& a, size_t need) {
  if (napi_get_cb_info(env, info, &a.argc, a.argv, nullptr, nullptr) != napi_ok) return false;
  if (a.argc < need) {
    napi_throw_type_error(env, nullptr, "wgx: too few arguments");
    return false;
  }
  return true;
}

wgx_ctx* handle(napi_env env, napi_value v) {
  void* p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "wgx: expected a context handle");
    return nullptr;
  }
  return static_cast<wgx_ctx*>(p);
}

double num(napi_env env, napi_value v) {
  double d = 0;
  napi_get_value_double(env, v, &d);
  return d;
}

int32_t i32(napi_env env, napi_value v) {
  int32_t x = 0;
  napi_get_value_int32(env, v, &x);
  return x;
}

bool is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t == napi_null || t == napi_undefined;
}

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value make_num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

// Throws for a non-zero status; returns true when the call succeeded.
bool ok(napi_env env, wgx_ctx* c, int status) {
  if (status == 0) return true;
  std::string msg = c ? wgx_last_error(c) : "wgx error";
  if (msg.empty()) msg = "wgx error " + std::to_string(status);
  napi_throw_error(env, nullptr, msg.c_str());
  return false;
}

napi_value prop(napi_env env, napi_value obj, const char* name) {
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  return v;
}

bool to_tensor(napi_env env, napi_value obj, wgx_tensor& t) {
  memset(&t, 0, sizeof t);
  t.data = reinterpret_cast<void*>(static_cast<uintptr_t>(num(env, prop(env, obj, "ptr"))));
  t.dtype = i32(env, prop(env, obj, "dtype"));
  napi_value shape = prop(env, obj, "shape");
  uint32_t n = 0;
  napi_get_array_length(env, shape, &n);
  if (n > WGX_MAX_NDIM) {
    napi_throw_range_error(env, nullptr, "wgx: tensor rank exceeds 8");
    return false;
  }
  t.ndim = (int32_t)n;
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, shape, i, &e);
    t.shape[i] = (int64_t)num(env, e);
  }
  return true;
}

void pair2(napi_env env, napi_value arr, int32_t out[2]) {
  napi_value e;
  napi_get_element(env, arr, 0, &e);
  out[0] = i32(env, e);
  napi_get_element(env, arr, 1, &e);
  out[1] = i32(env, e);
}

void finalize_noop(napi_env, void*, void*) {}

// ------------------------------------------------------------------ contexts

napi_value ctx_create(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = nullptr;
  const int st = wgx_ctx_create(i32(env, a.argv[0]), &c);
  if (st != 0) {
    napi_throw_error(env, nullptr, st == WGX_ERR_NO_DEVICE ? "No suitable GPU adapter found"
                                                          : "wgx: device initialisation failed");
    return nullptr;
  }
  napi_value v;
  NAPI_CALL(env, napi_create_external(env, c, finalize_noop, nullptr, &v));
  return v;
}

napi_value ctx_create_shared(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* p = handle(env, a.argv[0]);
  if (!p) return nullptr;
  wgx_ctx* c = nullptr;
  if (!ok(env, p, wgx_ctx_create_shared(p, &c))) return nullptr;
  napi_value v;
  NAPI_CALL(env, napi_create_external(env, c, finalize_noop, nullptr, &v));
  return v;
}

napi_value ctx_destroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (c) wgx_ctx_destroy(c);
  return undefined(env);
}

napi_value ctx_info(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  napi_value o, v;
  napi_create_object(env, &o);
  napi_get_boolean(env, wgx_ctx_has_device(c) != 0, &v);
  napi_set_named_property(env, o, "hasDevice", v);
  napi_create_string_utf8(env, wgx_ctx_arch(c), NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, o, "arch", v);
  napi_create_string_utf8(env, wgx_last_kernel(c), NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, o, "lastKernel", v);
  napi_create_int32(env, wgx_command_count(c), &v);
  napi_set_named_property(env, o, "commandCount", v);
  return o;
}

// ------------------------------------------------------------------ buffers

napi_value alloc(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  void* p = nullptr;
  if (!ok(env, c, wgx_alloc(c, (uint64_t)num(env, a.argv[1]), (uint32_t)num(env, a.argv[2]), &p)))
    return nullptr;
  return make_num(env, (double)reinterpret_cast<uintptr_t>(p));
}

napi_value free_buf(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  void* p = reinterpret_cast<void*>(static_cast<uintptr_t>(num(env, a.argv[1])));
  if (!ok(env, c, wgx_free(c, p))) return nullptr;
  return undefined(env);
}

// write(h, ptr, arrayBuffer, byteOffset, byteLength)
napi_value write(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  void* data = nullptr;
  size_t len = 0;
  NAPI_CALL(env, napi_get_arraybuffer_info(env, a.argv[2], &data, &len));
  const size_t off = (size_t)num(env, a.argv[3]), n = (size_t)num(env, a.argv[4]);
  if (off + n > len) {
    napi_throw_range_error(env, nullptr, "wgx: write range outside the source buffer");
    return nullptr;
  }
  void* dst = reinterpret_cast<void*>(static_cast<uintptr_t>(num(env, a.argv[1])));
  if (!ok(env, c, wgx_write(c, dst, static_cast<char*>(data) + off, n))) return nullptr;
  return undefined(env);
}

// read(h, ptr, byteLength) -> ArrayBuffer
napi_value read(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  const size_t n = (size_t)num(env, a.argv[2]);
  void* out = nullptr;
  napi_value ab;
  NAPI_CALL(env, napi_create_arraybuffer(env, n, &out, &ab));
  const void* src = reinterpret_cast<const void*>(static_cast<uintptr_t>(num(env, a.argv[1])));
  if (!ok(env, c, wgx_read(c, src, out, n))) return nullptr;
  return ab;
}

// ------------------------------------------------------------------ records

napi_value record_copy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  void* dst = reinterpret_cast<void*>(static_cast<uintptr_t>(num(env, a.argv[1])));
  const void* src = reinterpret_cast<const void*>(static_cast<uintptr_t>(num(env, a.argv[2])));
  if (!ok(env, c, wgx_record_copy(c, dst, src, (uint64_t)num(env, a.argv[3])))) return nullptr;
  return undefined(env);
}

// recordMm(h, a, b, bias|null, out, alpha, beta, flags)
napi_value record_mm(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 8)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor ta, tb, tbias, to;
  if (!to_tensor(env, a.argv[1], ta) || !to_tensor(env, a.argv[2], tb) || !to_tensor(env, a.argv[4], to))
    return nullptr;
  const bool has_bias = !is_nullish(env, a.argv[3]);
  if (has_bias && !to_tensor(env, a.argv[3], tbias)) return nullptr;
  if (!ok(env, c, wgx_record_mm(c, &ta, &tb, has_bias ? &tbias : nullptr, &to, (float)num(env, a.argv[5]),
                                (float)num(env, a.argv[6]), (uint32_t)num(env, a.argv[7]))))
    return nullptr;
  return undefined(env);
}

napi_value record_bmm(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor ta, tb, to;
  if (!to_tensor(env, a.argv[1], ta) || !to_tensor(env, a.argv[2], tb) || !to_tensor(env, a.argv[3], to))
    return nullptr;
  if (!ok(env, c, wgx_record_bmm(c, &ta, &tb, &to, (uint32_t)num(env, a.argv[4])))) return nullptr;
  return undefined(env);
}

// recordConv2d(h, in, weight, bias|null, args, out)
napi_value record_conv2d(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 6)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor tin, tw, tb, to;
  if (!to_tensor(env, a.argv[1], tin) || !to_tensor(env, a.argv[2], tw) || !to_tensor(env, a.argv[5], to))
    return nullptr;
  const bool has_bias = !is_nullish(env, a.argv[3]);
  if (has_bias && !to_tensor(env, a.argv[3], tb)) return nullptr;
  napi_value o = a.argv[4];
  wgx_conv_args ca;
  memset(&ca, 0, sizeof ca);
  pair2(env, prop(env, o, "stride"), ca.stride);
  pair2(env, prop(env, o, "padding"), ca.padding);
  pair2(env, prop(env, o, "dilation"), ca.dilation);
  pair2(env, prop(env, o, "outputPadding"), ca.output_padding);
  ca.transposed = i32(env, prop(env, o, "transposed"));
  ca.groups = i32(env, prop(env, o, "groups"));
  ca.has_clamp = i32(env, prop(env, o, "hasClamp"));
  ca.clamp_min = (float)num(env, prop(env, o, "clampMin"));
  ca.clamp_max = (float)num(env, prop(env, o, "clampMax"));
  ca.activation = i32(env, prop(env, o, "activation"));  // absent: 0, no activation
  napi_value rv = prop(env, o, "residual");  // absent / null: no residual
  if (!is_nullish(env, rv)) {
    wgx_tensor tr;
    if (!to_tensor(env, rv, tr)) return nullptr;
    if (!ok(env, c, wgx_record_conv2d_residual(c, &tin, &tw, has_bias ? &tb : nullptr, &ca, &tr,
                                               (float)num(env, prop(env, o, "convScale")),
                                               (float)num(env, prop(env, o, "residualScale")), &to)))
      return nullptr;
    return undefined(env);
  }
  if (!ok(env, c, wgx_record_conv2d(c, &tin, &tw, has_bias ? &tb : nullptr, &ca, &to))) return nullptr;
  return undefined(env);
}

// recordAdd(h, a, b, alpha, subtract, out)
napi_value record_add(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 6)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, y, o;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor(env, a.argv[2], y) || !to_tensor(env, a.argv[5], o))
    return nullptr;
  if (!ok(env, c, wgx_record_add(c, &x, &y, (float)num(env, a.argv[3]), i32(env, a.argv[4]), &o))) return nullptr;
  return undefined(env);
}

napi_value record_mul(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, y, o;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor(env, a.argv[2], y) || !to_tensor(env, a.argv[3], o))
    return nullptr;
  if (!ok(env, c, wgx_record_mul(c, &x, &y, &o))) return nullptr;
  return undefined(env);
}

// recordUnary(h, op, in, out)
napi_value record_unary(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, o;
  if (!to_tensor(env, a.argv[2], x) || !to_tensor(env, a.argv[3], o)) return nullptr;
  if (!ok(env, c, wgx_record_unary(c, i32(env, a.argv[1]), &x, &o))) return nullptr;
  return undefined(env);
}

bool to_tensor_list(napi_env env, napi_value arr, std::vector<wgx_tensor>& out) {
  uint32_t n = 0;
  napi_get_array_length(env, arr, &n);
  out.resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, arr, i, &e);
    if (!to_tensor(env, e, out[i])) return false;
  }
  return true;
}

// recordCat(h, [tensors], dim, out)
napi_value record_cat(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  std::vector<wgx_tensor> ins;
  wgx_tensor o;
  if (!to_tensor_list(env, a.argv[1], ins) || !to_tensor(env, a.argv[3], o)) return nullptr;
  if (!ok(env, c, wgx_record_cat(c, ins.data(), (int)ins.size(), i32(env, a.argv[2]), &o))) return nullptr;
  return undefined(env);
}

// recordSplit(h, in, dim, [outs])
napi_value record_split(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x;
  std::vector<wgx_tensor> outs;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor_list(env, a.argv[3], outs)) return nullptr;
  if (!ok(env, c, wgx_record_split(c, &x, i32(env, a.argv[2]), outs.data(), (int)outs.size()))) return nullptr;
  return undefined(env);
}

napi_value record_upsample(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, o;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor(env, a.argv[2], o)) return nullptr;
  if (!ok(env, c, wgx_record_upsample_nearest2d(c, &x, &o))) return nullptr;
  return undefined(env);
}

// recordMaxPool2d(h, in, kernel, stride, padding, dilation, ceilMode, values, indices|null)
napi_value record_max_pool(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 9)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, o, ix;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor(env, a.argv[7], o)) return nullptr;
  const bool has_idx = !is_nullish(env, a.argv[8]);
  if (has_idx && !to_tensor(env, a.argv[8], ix)) return nullptr;
  int32_t k[2], s[2], p[2], d[2];
  pair2(env, a.argv[2], k);
  pair2(env, a.argv[3], s);
  pair2(env, a.argv[4], p);
  pair2(env, a.argv[5], d);
  if (!ok(env, c, wgx_record_max_pool2d(c, &x, k, s, p, d, i32(env, a.argv[6]), &o, has_idx ? &ix : nullptr)))
    return nullptr;
  return undefined(env);
}

// recordPermute(h, in, dims, out)
napi_value record_permute(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, o;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor(env, a.argv[3], o)) return nullptr;
  uint32_t n = 0;
  napi_get_array_length(env, a.argv[2], &n);
  if (n > WGX_MAX_NDIM) {
    napi_throw_range_error(env, nullptr, "wgx: permute dims exceed rank 8");
    return nullptr;
  }
  int32_t dims[WGX_MAX_NDIM] = {0};
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, a.argv[2], i, &e);
    dims[i] = i32(env, e);
  }
  if (!ok(env, c, wgx_record_permute(c, &x, dims, (int)n, &o))) return nullptr;
  return undefined(env);
}

// recordSoftmax(h, in, dim, out)
napi_value record_softmax(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_tensor x, o;
  if (!to_tensor(env, a.argv[1], x) || !to_tensor(env, a.argv[3], o)) return nullptr;
  if (!ok(env, c, wgx_record_softmax(c, &x, i32(env, a.argv[2]), &o))) return nullptr;
  return undefined(env);
}

// ------------------------------------------------------------------ execution

napi_value submit(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c || !ok(env, c, wgx_submit(c))) return nullptr;
  return undefined(env);
}

napi_value sync(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c || !ok(env, c, wgx_sync(c))) return nullptr;
  return undefined(env);
}

// syncAsync(h) -> Promise: sync() / queue.onSubmittedWorkDone()
// (src/context.ts:377-380).  A fence is recorded on the queue here, on the
// JS thread; a libuv worker waits for it (the wait touches only the fence,
// never the context, so recording may go on meanwhile) and the promise
// settles back on the JS thread.
struct SyncWork {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  wgx_fence* fence = nullptr;
  int status = 0;
};

void sync_execute(napi_env, void* data) {
  SyncWork* w = static_cast<SyncWork*>(data);
  w->status = wgx_fence_wait(w->fence);
}

void sync_complete(napi_env env, napi_status st, void* data) {
  SyncWork* w = static_cast<SyncWork*>(data);
  if (st == napi_ok && w->status == 0) {
    napi_resolve_deferred(env, w->deferred, undefined(env));
  } else {
    std::string msg = st == napi_ok ? wgx_fence_error(w->fence) : "sync: cancelled";
    napi_value m, err;
    napi_create_string_utf8(env, msg.c_str(), NAPI_AUTO_LENGTH, &m);
    napi_create_error(env, nullptr, m, &err);
    napi_reject_deferred(env, w->deferred, err);
  }
  wgx_fence_destroy(w->fence);
  napi_delete_async_work(env, w->work);
  delete w;
}

napi_value sync_async(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c) return nullptr;
  wgx_fence* f = nullptr;
  if (!ok(env, c, wgx_fence_record(c, &f))) return nullptr;
  SyncWork* w = new SyncWork();
  w->fence = f;
  napi_value promise, name;
  if (napi_create_promise(env, &w->deferred, &promise) != napi_ok ||
      napi_create_string_utf8(env, "wgx_sync", NAPI_AUTO_LENGTH, &name) != napi_ok ||
      napi_create_async_work(env, nullptr, name, sync_execute, sync_complete, w, &w->work) != napi_ok ||
      napi_queue_async_work(env, w->work) != napi_ok) {
    wgx_fence_destroy(f);
    delete w;
    napi_throw_error(env, nullptr, "wgx: could not queue the sync");
    return nullptr;
  }
  return promise;
}

napi_value reset(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c || !ok(env, c, wgx_reset(c))) return nullptr;
  return undefined(env);
}

napi_value set_graph_mode(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  if (!c || !ok(env, c, wgx_set_graph_mode(c, i32(env, a.argv[1])))) return nullptr;
  return undefined(env);
}

napi_value time_submits(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  wgx_ctx* c = handle(env, a.argv[0]);
  float ms = 0.f;
  if (!c || !ok(env, c, wgx_time_submits(c, i32(env, a.argv[1]), &ms))) return nullptr;
  return make_num(env, ms);
}

napi_value init(napi_env env, napi_value exports) {
  struct Fn {
    const char* name;
    napi_callback cb;
  } fns[] = {{"ctxCreate", ctx_create},       {"ctxCreateShared", ctx_create_shared},
             {"ctxDestroy", ctx_destroy},     {"ctxInfo", ctx_info},
             {"alloc", alloc},                {"free", free_buf},
             {"write", write},                {"read", read},
             {"recordCopy", record_copy},     {"recordMm", record_mm},
             {"recordBmm", record_bmm},       {"recordConv2d", record_conv2d},
             {"recordAdd", record_add},       {"recordMul", record_mul},
             {"recordUnary", record_unary},   {"recordCat", record_cat},
             {"recordSplit", record_split},   {"recordUpsampleNearest2d", record_upsample},
             {"recordMaxPool2d", record_max_pool}, {"recordPermute", record_permute},
             {"recordSoftmax", record_softmax}, {"submit", submit},
             {"sync", sync},                  {"syncAsync", sync_async},
             {"reset", reset},
             {"setGraphMode", set_graph_mode}, {"timeSubmits", time_submits}};
  for (const Fn& f : fns) {
    napi_value v;
    NAPI_CALL(env, napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &v));
    NAPI_CALL(env, napi_set_named_property(env, exports, f.name, v));
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
