/*
 * wgx.h -- C-ABI of libwgx, the MI355X (gfx950) execution library behind the
 * wgpu-executorch Shader / WgpuExecutionContext API for the GEMM-shaped hot
 * path: aten.mm / aten.addmm / aten.bmm, aten.convolution (implicit-im2col
 * GEMM, 1x1, depthwise, grouped and transposed fallbacks) and
 * et_vk.conv_with_clamp, plus the simple ops a YOLO-style program chain needs.
 *
 * Plain C types only: device pointers, sizes, small POD structs.  No C++
 * exception crosses this boundary; every call returns a wgx_status and the
 * message of the last failure is available from wgx_last_error().
 *
 * Model (mirrors the reference's record/submit split, src/context.ts:17-390):
 *   - a context owns every buffer it allocated; all contexts of one device
 *     share that device's single HIP stream (GPUDevice.queue);
 *   - wgx_record_* validate and append a launch record, nothing runs yet;
 *   - wgx_submit replays the recorded list in order (as one HIP graph,
 *     re-captured only when the list changed), wgx_sync waits for it;
 *   - wgx_write / wgx_read are stream-ordered with submitted work.
 * A context created on device -1 is a host-only validation context: buffers
 * live in host memory, records are validated and kept, and wgx_submit fails
 * with WGX_ERR_NO_DEVICE.  It lets the shape/argument logic be tested without
 * a GPU.
 */
#ifndef WGX_H
#define WGX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Maximum tensor rank.  Replaces MAX_NDIM, src/tensor.ts:23. */
#define WGX_MAX_NDIM 8

/* Element types.  Replaces DType / DTYPE_BYTESIZE, src/tensor.ts:4-30
 * (bfloat16 is an addition of this library). */
typedef enum {
  WGX_FLOAT32 = 0,
  WGX_FLOAT16 = 1,
  WGX_INT32 = 2,
  WGX_INT8 = 3,
  WGX_UINT8 = 4,
  WGX_BOOL = 5,
  WGX_FLOAT64 = 6,
  WGX_INT64 = 7,
  WGX_BFLOAT16 = 8
} wgx_dtype;

typedef enum {
  WGX_OK = 0,
  WGX_ERR_INVALID = 1,   /* bad argument, shape or dtype                     */
  WGX_ERR_HIP = 2,       /* a HIP runtime call failed                        */
  WGX_ERR_DESTROYED = 3, /* context already destroyed                        */
  WGX_ERR_NO_DEVICE = 4, /* host-only context asked to execute               */
  WGX_ERR_OOM = 5        /* device allocation failed                         */
} wgx_status;

/* Buffer usage bits, the subset of GPUBufferUsage the reference checks
 * (src/context.ts:9-11, src/tensor.ts:68-70,118-120). */
#define WGX_USAGE_COPY_SRC 0x4u
#define WGX_USAGE_COPY_DST 0x8u
#define WGX_USAGE_STORAGE 0x80u

/* A non-owning tensor view: device pointer + dtype + row-major contiguous
 * shape.  Replaces Tensor's (dtype, shape, buffer) triple, src/tensor.ts:43-101. */
typedef struct {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[WGX_MAX_NDIM];
} wgx_tensor;

/* aten.convolution.default scalar arguments (src/shaders/convolution/
 * index.ts:33-44) plus the clamp of et_vk.conv_with_clamp.default
 * (src/shaders/conv-with-clamp/index.ts:33-46).  Two-element lists are given
 * already expanded (parseHw, src/shaders/convolution/index.ts:46-50).
 * `activation` has no counterpart in the reference's operators: it lets a
 * program runner fold a following elementwise activation into the
 * convolution's epilogue (conv -> sigmoid -> mul is SiLU); it is applied
 * after the bias and before the clamp, in float32, before the one rounding. */
#define WGX_ACT_NONE 0
#define WGX_ACT_SILU 1
typedef struct {
  int32_t stride[2];
  int32_t padding[2];
  int32_t dilation[2];
  int32_t output_padding[2];
  int32_t transposed;
  int32_t groups;
  int32_t has_clamp;
  float clamp_min;
  float clamp_max;
  int32_t activation; /* WGX_ACT_NONE or WGX_ACT_SILU */
} wgx_conv_args;

typedef struct wgx_ctx wgx_ctx;

/* ---------------------------------------------------------------- context */

/* new WgpuExecutionContext(device) (src/context.ts:28-30).  device >= 0 is a
 * HIP device ordinal; -1 makes a host-only validation context. */
int wgx_ctx_create(int device, wgx_ctx** out);
/* A further context on the same device as `parent`: it shares the parent's
 * buffer registry and queue (one HIP stream per device, so work submitted
 * from any context runs in submission order, like GPUDevice.queue) and has
 * its own command list.  This is how several WgpuExecutionContexts are
 * created over one GPUDevice (src/context.ts:28-30). */
int wgx_ctx_create_shared(wgx_ctx* parent, wgx_ctx** out);
/* destroy() (src/context.ts:61-72): frees every buffer this context
 * allocated and the handle; the device state goes with the last context. */
void wgx_ctx_destroy(wgx_ctx* ctx);
/* Message of the most recent failure on this context ("" if none). */
const char* wgx_last_error(const wgx_ctx* ctx);
/* 1 if the context executes on a GPU, 0 for a host-only context. */
int wgx_ctx_has_device(const wgx_ctx* ctx);
/* Name of the device architecture ("gfx950"), or "host". */
const char* wgx_ctx_arch(const wgx_ctx* ctx);
/* The HIP stream (hipStream_t) all of this context's work runs on. */
void* wgx_ctx_stream(const wgx_ctx* ctx);

/* ---------------------------------------------------------------- buffers */

/* storageBuffer(size) (src/context.ts:86-92): a context-owned buffer of at
 * least max(4, round_up(bytes, 4)) bytes, 256-byte aligned, zero-filled. */
int wgx_alloc(wgx_ctx* ctx, uint64_t bytes, uint32_t usage, void** out);
/* GPUBuffer.destroy(): frees the buffer whose base address is ptr (any
 * context of the device may free it).  A later submit of a command recorded
 * against it fails with WGX_ERR_INVALID instead of touching freed memory. */
int wgx_free(wgx_ctx* ctx, void* ptr);
/* Size and usage of the owned buffer that contains ptr (0 / error if none). */
int wgx_buffer_info(const wgx_ctx* ctx, const void* ptr, uint64_t* base_offset,
                    uint64_t* size, uint32_t* usage);
/* Tensor.setData (src/tensor.ts:115-135): stream-ordered host-to-device copy. */
int wgx_write(wgx_ctx* ctx, void* dst, const void* src, uint64_t bytes);
/* Tensor.getData (src/tensor.ts:142-158): waits for submitted work, then
 * copies device-to-host. */
int wgx_read(wgx_ctx* ctx, const void* src, void* dst, uint64_t bytes);

/* ---------------------------------------------------------------- recording */

/* copy(src, dst) (src/context.ts:172-192): deferred device copy of bytes. */
int wgx_record_copy(wgx_ctx* ctx, void* dst, const void* src, uint64_t bytes);

/* aten.mm.default [in1, in2, out] (src/shaders/mm/index.ts:32-93), and with a
 * bias aten.addmm.default (absent from the reference, which would compose
 * mm + add, src/shaders/add/index.ts:99-128):
 *   out = beta * bias + alpha * (a @ b)
 * a [M,K]; b [K,N], or [N,K] when flags has WGX_MM_TRANS_B (nn.Linear
 * weight layout); bias [N] or [1,N] or NULL; out [M,N].  float32, float16 or
 * bfloat16, all the same dtype; float16/bfloat16 accumulate in float32. */
#define WGX_MM_TRANS_B 0x1u
int wgx_record_mm(wgx_ctx* ctx, const wgx_tensor* a, const wgx_tensor* b,
                  const wgx_tensor* bias, const wgx_tensor* out, float alpha, float beta,
                  uint32_t flags);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc): the wgx_record_mm GEMM (same arguments, same kernels,
 * same results) launched at once on the context's stream instead of being
 * recorded, with its workspace -- the [N, K] copy of a 16-bit [K, N] B that
 * the large-tile kernel reads, and split-K partial sums -- taken from one
 * fixed device array of WGX_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends.  It calls no hipMalloc / hipFree (nor any allocating
 * routine); a GEMM whose workspace exceeds the array fails with
 * WGX_ERR_INVALID before anything is launched.  Every call on a GPU shares
 * that GPU's array: calls from contexts of one device are ordered on its
 * single stream, but calls that overlap on one GPU from different device
 * states (separately created contexts) race on it.  Host-only contexts fail
 * with WGX_ERR_NO_DEVICE. */
#define WGX_NOALLOC_SCRATCH_BYTES (8u << 20)
int wgx_mm_noalloc(wgx_ctx* ctx, const wgx_tensor* a, const wgx_tensor* b,
                   const wgx_tensor* bias, const wgx_tensor* out, float alpha, float beta,
                   uint32_t flags);

/* aten.bmm.default [a, b, out] (src/shaders/bmm/index.ts:27-96):
 * a [B,M,K] @ b [B,K,N] (or [B,N,K] with WGX_MM_TRANS_B) -> out [B,M,N]. */
int wgx_record_bmm(wgx_ctx* ctx, const wgx_tensor* a, const wgx_tensor* b,
                   const wgx_tensor* out, uint32_t flags);

/* aten.convolution.default (src/shaders/convolution/index.ts:58-310) and
 * et_vk.conv_with_clamp.default (args->has_clamp).  in NCHW [B,IC,IH,IW];
 * weight OIHW [OC,IC/groups,KH,KW] (transposed: [IC,OC/groups,KH,KW]); bias
 * [OC] or NULL; out NCHW.  Output spatial size must match the reference
 * formula (index.ts:112-139). */
int wgx_record_conv2d(wgx_ctx* ctx, const wgx_tensor* in, const wgx_tensor* weight,
                      const wgx_tensor* bias, const wgx_conv_args* args,
                      const wgx_tensor* out);
/* The same convolution with an output-shaped tensor added in its epilogue:
 * out = conv_scale * conv(in) + residual_scale * residual, where conv(in) is
 * the full result above (bias, activation, clamp), rounded once.  No
 * counterpart in the reference: recordProgram folds
 * aten.add.Tensor(a, b, alpha) into the convolution that produces a or b
 * with it (src/shaders/add/index.ts:33-129: out = a + alpha * b).  Depthwise
 * convolutions, and dense 3x3 convolutions (stride 1 or 2, dilation 1, a
 * multiple of 8 float32 or 16 16-bit input channels) that the LDS-patch
 * kernel takes; WGX_ERR_INVALID for the rest.  residual may be the output
 * itself but must not partly overlap it. */
int wgx_record_conv2d_residual(wgx_ctx* ctx, const wgx_tensor* in, const wgx_tensor* weight,
                               const wgx_tensor* bias, const wgx_conv_args* args,
                               const wgx_tensor* residual, float conv_scale,
                               float residual_scale, const wgx_tensor* out);

/* Elementwise / data-movement ops a YOLO-style program chain needs (simple,
 * bandwidth-bound kernels; not the optimisation target). */
/* aten.add.Tensor / aten.sub.Tensor with alpha and broadcasting
 * (src/shaders/add/index.ts:33-129): out = a + alpha * b (sub: a - alpha*b). */
int wgx_record_add(wgx_ctx* ctx, const wgx_tensor* a, const wgx_tensor* b, float alpha,
                   int subtract, const wgx_tensor* out);
/* aten.mul.Tensor with broadcasting. */
int wgx_record_mul(wgx_ctx* ctx, const wgx_tensor* a, const wgx_tensor* b,
                   const wgx_tensor* out);
/* Unary activations: 0 sigmoid, 1 relu, 2 hardswish, 3 silu. */
#define WGX_UNARY_SIGMOID 0
#define WGX_UNARY_RELU 1
#define WGX_UNARY_HARDSWISH 2
#define WGX_UNARY_SILU 3
int wgx_record_unary(wgx_ctx* ctx, int op, const wgx_tensor* in, const wgx_tensor* out);
/* aten.cat.default along dim (negative dims count from the end). */
int wgx_record_cat(wgx_ctx* ctx, const wgx_tensor* inputs, int n_inputs, int dim,
                   const wgx_tensor* out);
/* aten.split_with_sizes_copy.default along dim into n_outputs tensors. */
int wgx_record_split(wgx_ctx* ctx, const wgx_tensor* in, int dim, const wgx_tensor* outputs,
                     int n_outputs);
/* aten.upsample_nearest2d.vec, integer-or-fractional scale from the shapes. */
int wgx_record_upsample_nearest2d(wgx_ctx* ctx, const wgx_tensor* in, const wgx_tensor* out);
/* aten.max_pool2d_with_indices.default [in, kernel_size, stride, padding,
 * dilation, ceil_mode, [values, indices]] (src/shaders/max-pool-2d/
 * index.ts:41-106): values[b,c,oh,ow] is the first strictly greatest element
 * of the window in row-major order (cells outside the image are skipped;
 * the initial value is -65504 for float16, -3.4e38 otherwise) and
 * indices[b,c,oh,ow] its flat position ih * IW + iw in the plane (0 when no
 * element beats the initial value).  indices is int32 of the values' shape,
 * or NULL to skip it.  The output size is floor (ceil with ceil_mode) of
 * (I + 2p - d(K-1) - 1) / s, plus 1, at least 0 (index.ts:75-78). */
int wgx_record_max_pool2d(wgx_ctx* ctx, const wgx_tensor* in, const int32_t kernel[2],
                          const int32_t stride[2], const int32_t padding[2],
                          const int32_t dilation[2], int ceil_mode, const wgx_tensor* out,
                          const wgx_tensor* indices);
/* aten.permute_copy.default [in, dims, out] (src/shaders/permute/
 * index.ts:33-99): out dim k is input dim dims[k] (negative dims count from
 * the end); any dtype, out of the permuted shape. */
int wgx_record_permute(wgx_ctx* ctx, const wgx_tensor* in, const int32_t* dims, int n_dims,
                       const wgx_tensor* out);
/* aten._softmax.default [in, dim, half_to_float, out] (src/shaders/softmax/
 * index.ts:62-125): out = exp(x - max) / sum(exp(x - max)) along dim
 * (negative counts from the end), float32 arithmetic for every dtype;
 * out has the input's dtype and element count. */
int wgx_record_softmax(wgx_ctx* ctx, const wgx_tensor* in, int dim, const wgx_tensor* out);

/* ---------------------------------------------------------------- execution */

/* submit() (src/context.ts:323-370): replay every recorded command in order.
 * No-op when nothing is recorded. */
int wgx_submit(wgx_ctx* ctx);
/* sync() (src/context.ts:377-380): wait for all submitted work. */
int wgx_sync(wgx_ctx* ctx);
/* The pieces of an asynchronous sync() (src/context.ts:377-380: a Promise
 * that settles when the work submitted so far is done), for hosts that wait
 * off their main thread.  wgx_fence_record marks the queue's current end
 * (call it from the thread that records and submits); wgx_fence_wait blocks
 * until the queue has passed that mark and may run on any thread, also while
 * the context records or after it was destroyed, because it touches only the
 * fence; wgx_fence_error gives the reason of a failed wait; the owner frees
 * the fence with wgx_fence_destroy.  A host-only context's fence is always
 * passed. */
typedef struct wgx_fence wgx_fence;
int wgx_fence_record(wgx_ctx* ctx, wgx_fence** out);
int wgx_fence_wait(wgx_fence* fence);
const char* wgx_fence_error(const wgx_fence* fence);
void wgx_fence_destroy(wgx_fence* fence);
/* reset() (src/context.ts:386-389): drop recorded commands, keep buffers. */
int wgx_reset(wgx_ctx* ctx);
/* Number of recorded commands. */
int wgx_command_count(const wgx_ctx* ctx);
/* 1 (default) replays through a captured HIP graph, 0 launches eagerly. */
int wgx_set_graph_mode(wgx_ctx* ctx, int enabled);
/* Submits the recorded list `reps` times back to back and returns the mean
 * device time per submit in *ms_per_submit, measured with HIP events
 * recorded on the context's stream around the whole run. */
int wgx_time_submits(wgx_ctx* ctx, int reps, float* ms_per_submit);

/* Name of the kernel the last wgx_record_* call selected (for tests/profiling). */
const char* wgx_last_kernel(const wgx_ctx* ctx);
/* Number of paired launches the last wgx_submit issued: two adjacent
 * recorded convolutions that read and write disjoint memory and both take
 * the float32 batch-1 LDS-patch configuration run as one launch (set
 * WGX_MERGE=0 to keep them apart).  No counterpart in the reference, which
 * runs every dispatch of a pass on its own; for tests and profiling. */
int wgx_paired_launches(const wgx_ctx* ctx);

#ifdef __cplusplus
}
#endif

#endif /* WGX_H */
