// internal.h -- shared declarations between the runtime and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "wgx.h"

namespace wgx {

// Epilogue activation of a convolution: v = act(acc + bias), then clamp.
// SiLU is x * sigmoid(x) = x / (1 + e^-x), in float32 before the one
// rounding to the storage type.
__device__ __forceinline__ float apply_act(int act, float x) {
  // x * (1 / (1 + e^-x)) with the hardware reciprocal (1 ulp), not an IEEE
  // division (about a dozen instructions); -0 for large negative x (the
  // denominator overflows to inf), NaN propagates
  return act == WGX_ACT_SILU ? x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)) : x;
}

// Passing this stream to a launch_* function selects the kernel, fills *name
// and performs one-time kernel set-up (LDS attributes) without launching.
inline hipStream_t describe_only() { return reinterpret_cast<hipStream_t>(~uintptr_t(0)); }
// Like describe_only() but with no HIP call at all (host-only contexts).
inline hipStream_t name_only() { return reinterpret_cast<hipStream_t>(~uintptr_t(1)); }
inline bool is_dry(hipStream_t s) { return s == describe_only() || s == name_only(); }

// One GEMM-shaped launch: C[b] = epilogue(A[b] (M x K) * B[b] (K x N)).
//   A: row-major, k-contiguous, leading dim lda, batch stride sA (0 = shared).
//   B: bmode NK  -> row-major [N,K] (k-contiguous), leading dim ldb
//      bmode KN  -> row-major [K,N] (n-contiguous), leading dim ldb
//      bmode CONV-> implicit im2col of an NCHW input (see ConvGeom): element
//                   (k, n) = x[b][ktab[k].off + colbase(n)] when tap ktab[k].tap
//                   is inside the image for output pixel n, else 0.
//   C: row-major, leading dim ldc, batch stride sC.
//   epilogue: v = alpha*acc + beta*bias (bias per column n, or per row m),
//             optional clamp, rounded once to the storage dtype.
enum BMode { B_NK = 0, B_KN = 1, B_CONV = 2 };
enum BiasMode { BIAS_NONE = 0, BIAS_COL = 1, BIAS_ROW = 2 };

struct ConvGeom {
  int IH, IW, OW, sH, sW, pH, pW, KH, KW, dH, dW;
};

struct GemmDesc {
  int dtype;  // WGX_FLOAT32 / WGX_FLOAT16 / WGX_BFLOAT16
  int batch, M, N, K;
  const void* A;
  long long lda, sA;
  const void* B;
  long long ldb, sB;
  void* C;
  long long ldc, sC;
  const void* bias;
  int bias_mode;
  float alpha, beta;
  int has_clamp;
  int act;  // WGX_ACT_*: applied after the bias, before the clamp
  float cmin, cmax;
  int bmode;
  ConvGeom g;
  const uint32_t* ktab;  // device table for B_CONV: Kpad entries (off << 6) | tap
  // split-K (set from gemm_split_plan): splits > 1 divides K into that many
  // contiguous ranges; ws holds their fp32 partial sums, [splits][batch][M][N]
  int splits;
  float* ws;
  // [N, K] copy of a 16-bit [K, N] B for the large-tile kernel
  // (gemm_stage_b_bytes > 0): batch * N * K elements
  void* bt;
};

// Split-K plan for an MFMA launch: how many K ranges (1 = none) and the
// workspace size the launch then needs.
int gemm_split_plan(const GemmDesc& d, size_t* ws_bytes);
// Bytes of the [N, K] staging workspace the launch needs for its [K, N] B
// (0: B is read in place).
size_t gemm_stage_b_bytes(const GemmDesc& d);

// Table rows needed for a B_CONV launch (K rounded up to the largest K tile).
int conv_ktab_rows(int K);
// Fills a host table for B_CONV: entry k = (ic*IH*IW + kh*dH*IW + kw*dW) << 6 | (kh*KW+kw);
// padding entries get tap 63 (never inside the image).
void conv_fill_ktab(uint32_t* tab, int K, int IC, const ConvGeom& g);
// The packed table applies: KH*KW <= 63, offsets < 2^26, table <= 32 KB.
bool conv_ktab_fits(int K, int IC, const ConvGeom& g);

hipError_t launch_gemm_mfma(const GemmDesc& d, hipStream_t s, std::string* name);
// Device address of the fixed WGX_NOALLOC_SCRATCH_BYTES workspace on
// `device` (noalloc.hip), looked up once per device and cached.
hipError_t noalloc_scratch(int device, void** out);
hipError_t launch_gemm_f32(const GemmDesc& d, hipStream_t s, std::string* name);

// Dense KxK convolution with each wave's input patch in LDS (conv_lds.hip):
// groups 1, dilation 1, IC a multiple of 8 (float32) or 16 (16-bit data),
// 3x3 at stride 1 or 2.
struct ConvLdsDesc {
  int dtype;
  int B, IC, IH, IW, OC, OH, OW, KH, KW, sH, sW, pH, pW;
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int act;  // WGX_ACT_*: applied after the bias, before the clamp
  int has_clamp;
  float cmin, cmax;
  // optional residual of the output's shape, added after the clamp:
  // y = res_conv_scale * y + res_scale * res (null: none)
  const void* res;
  float res_conv_scale, res_scale;
  // workspace for the pre-ordered weights (OC * IC * KH * KW elements) when
  // conv_lds_wants_prepass says the configuration uses them, else null
  void* wpre;
};
bool conv_lds_applies(const ConvLdsDesc& d);
bool conv_lds_wants_prepass(const ConvLdsDesc& d, int cus);
// cus: compute units of the device (the configuration depends on it)
hipError_t launch_conv_lds(const ConvLdsDesc& d, int cus, hipStream_t s, std::string* name);
// Two independent convolutions in one launch where both take the float32
// batch-1 configuration; hipErrorNotSupported (nothing launched) otherwise.
hipError_t launch_conv_lds_pair(const ConvLdsDesc& a, const ConvLdsDesc& b, int cus, hipStream_t s);

struct DwDesc {
  int dtype;
  int B, C, IH, IW, OH, OW, KH, KW, sH, sW, pH, pW, dH, dW;
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int has_clamp;
  int act;  // WGX_ACT_*: applied after the bias, before the clamp
  float cmin, cmax;
  // optional residual of the output's shape, added after the clamp:
  // y = res_conv_scale * y + res_scale * res (null: none)
  const void* res;
  float res_conv_scale, res_scale;
};
hipError_t launch_depthwise(const DwDesc& d, hipStream_t s, std::string* name);

struct DirectConvDesc {
  int dtype;
  int transposed;
  int B, IC, IH, IW, OC, OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, groups;
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int has_clamp;
  int act;  // WGX_ACT_*: applied after the bias, before the clamp
  float cmin, cmax;
};
hipError_t launch_direct_conv(const DirectConvDesc& d, hipStream_t s, std::string* name);
// Dense convolutions with at most 32 taps per output channel and at most 64
// output channels: launch_direct_conv runs them on its small-tap kernel.
bool small_tap_conv(const DirectConvDesc& d);

// Elementwise family (eltwise.hip).
struct BcastDesc {
  int dtype;
  int ndim;
  long long numel;
  long long out_shape[WGX_MAX_NDIM];
  long long a_stride[WGX_MAX_NDIM];  // 0 on broadcast dims
  long long b_stride[WGX_MAX_NDIM];
  const void* a;
  const void* b;
  void* out;
  float alpha;
  int op;  // 0 add (a + alpha*b), 1 mul
};
hipError_t launch_binary(const BcastDesc& d, hipStream_t s, std::string* name);
hipError_t launch_unary(int op, int dtype, long long n, const void* x, void* y, hipStream_t s,
                        std::string* name);
// Copies a [outer, inner_src] strided block into dst at a column offset:
// dst[o*inner_dst + off + i] = src[o*inner_src + i], elements of elsize bytes.
hipError_t launch_slab_copy(int elsize, long long outer, long long inner_src,
                            long long inner_dst, long long dst_off, long long src_off,
                            const void* src, void* dst, bool gather, hipStream_t s,
                            std::string* name);
hipError_t launch_upsample_nearest(int dtype, int BC, int IH, int IW, int OH, int OW,
                                   const void* x, void* y, hipStream_t s, std::string* name);
// n = 2 or 3 chained K x K max-pools (K = 2P + 1, stride 1, padding P,
// dilation 1) of one [BC, H, W] map in one pass: y1 = pool(x), y2 =
// pool(y1), y3 = pool(y2), each with its int32 indices into the plane it
// pooled (idx[k] may be null).  One block per plane, max_pool_chain_lds
// bytes of LDS (at most 64 KB).
size_t max_pool_chain_lds(int H, int W, int P);
hipError_t launch_max_pool_chain(int dtype, int BC, int H, int W, int P, int n, const void* x, void* const y[3],
                                 int32_t* const idx[3], hipStream_t s, std::string* name);
// max_pool2d_with_indices: values y and, when idx is not null, the int32
// flat index ih * IW + iw of each window's first strictly greatest element.
hipError_t launch_max_pool(int dtype, int BC, int IH, int IW, int OH, int OW, int KH, int KW,
                           int sH, int sW, int pH, int pW, int dH, int dW, const void* x,
                           void* y, int32_t* idx, hipStream_t s, std::string* name);

// permute_copy of a contiguous tensor: out dim k is input dim perm[k].
// out_shape / src_stride are filled by launch_permute.
struct PermuteDesc {
  int elsize;
  int ndim;
  int perm[WGX_MAX_NDIM];
  long long in_shape[WGX_MAX_NDIM];
  long long out_shape[WGX_MAX_NDIM];
  long long src_stride[WGX_MAX_NDIM];
  const void* x;
  void* y;
};
hipError_t launch_permute(const PermuteDesc& d, hipStream_t s, std::string* name);
// softmax of a contiguous [outer, r, inner] view along r.
hipError_t launch_softmax(int dtype, long long outer, long long r, long long inner, const void* x, void* y,
                          hipStream_t s, std::string* name);

}  // namespace wgx
