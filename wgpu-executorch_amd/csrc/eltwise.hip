// eltwise.hip -- the simple, bandwidth-bound ops a YOLO-style program chain
// needs around the GEMM-shaped hot path: broadcast add/sub/mul
// (src/shaders/add/index.ts:33-129, add-broadcast*.wgsl.ts), unary activations
// (sigmoid/relu/hardswish), cat / split_with_sizes as strided slab copies,
// nearest upsample and max-pool.  One lane per output element, float32
// arithmetic, one rounding to the storage type.  Not an optimisation target.
#include <math.h>
#include <stdio.h>

#include "internal.h"

namespace wgx {
namespace {

template <int DT>
__device__ __forceinline__ float ldv(const void* p, long long i) {
  if constexpr (DT == WGX_FLOAT32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == WGX_FLOAT16)
    return (float)static_cast<const _Float16*>(p)[i];
  else
    return __uint_as_float((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
}

template <int DT>
__device__ __forceinline__ void stv(void* p, long long i, float v) {
  if constexpr (DT == WGX_FLOAT32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == WGX_FLOAT16)
    static_cast<_Float16*>(p)[i] = (_Float16)v;
  else {
    uint32_t u = __float_as_uint(v);
    uint16_t h = ((u & 0x7fffffffu) > 0x7f800000u) ? (uint16_t)((u >> 16) | 0x40u)
                                                   : (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    static_cast<uint16_t*>(p)[i] = h;
  }
}

inline unsigned blocks_for(long long n) { return (unsigned)((n + 255) / 256); }

template <int DT>
__global__ __launch_bounds__(256) void k_binary(BcastDesc d) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= d.numel) return;
  long long rem = i, ia = 0, ib = 0;
  for (int k = d.ndim - 1; k >= 0; --k) {
    const long long c = rem % d.out_shape[k];
    rem /= d.out_shape[k];
    ia += c * d.a_stride[k];
    ib += c * d.b_stride[k];
  }
  const float a = ldv<DT>(d.a, ia), b = ldv<DT>(d.b, ib);
  stv<DT>(d.out, i, d.op == 0 ? a + d.alpha * b : a * b);
}

template <int DT>
__global__ __launch_bounds__(256) void k_unary(int op, long long n, const void* x, void* y) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = ldv<DT>(x, i);
  float r;
  if (op == WGX_UNARY_SIGMOID) r = 1.0f / (1.0f + __expf(-v));
  else if (op == WGX_UNARY_RELU) r = fmaxf(v, 0.0f);
  else if (op == WGX_UNARY_HARDSWISH) r = v * fminf(fmaxf(v + 3.0f, 0.0f), 6.0f) / 6.0f;
  else r = v / (1.0f + __expf(-v));
  stv<DT>(y, i, r);
}

template <typename E>
__global__ __launch_bounds__(256) void k_slab(long long outer, long long inner_src,
                                              long long inner_dst, long long dst_off,
                                              long long src_off, const E* src, E* dst,
                                              bool gather) {
  // gather == false (cat):   dst[o][dst_off + i] = src[o][i],          i < inner_src
  // gather == true  (split): dst[o][i]           = src[o][src_off + i], i < inner_dst
  const long long inner = gather ? inner_dst : inner_src;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= outer * inner) return;
  const long long o = i / inner, j = i % inner;
  if (gather)
    dst[o * inner_dst + j] = src[o * inner_src + src_off + j];
  else
    dst[o * inner_dst + dst_off + j] = src[o * inner_src + j];
}

template <int DT>
__global__ __launch_bounds__(256) void k_upsample(int BC, int IH, int IW, int OH, int OW,
                                                  const void* x, void* y) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)BC * OH * OW) return;
  const int ow = (int)(i % OW), oh = (int)((i / OW) % OH);
  const long long pl = i / ((long long)OH * OW);
  // nearest: src = floor(dst * in / out), PyTorch's legacy 'nearest' rule
  const int ih = min((int)(((long long)oh * IH) / OH), IH - 1);
  const int iw = min((int)(((long long)ow * IW) / OW), IW - 1);
  stv<DT>(y, i, ldv<DT>(x, (pl * IH + ih) * IW + iw));
}

template <int DT>
__global__ __launch_bounds__(256) void k_maxpool(int BC, int IH, int IW, int OH, int OW, int KH,
                                                 int KW, int sH, int sW, int pH, int pW, int dH,
                                                 int dW, const void* x, void* y) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)BC * OH * OW) return;
  const int ow = (int)(i % OW), oh = (int)((i / OW) % OH);
  const long long pl = i / ((long long)OH * OW);
  float m = -INFINITY;
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * sH - pH + kh * dH;
    if (ih < 0 || ih >= IH) continue;
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = ow * sW - pW + kw * dW;
      if (iw < 0 || iw >= IW) continue;
      m = fmaxf(m, ldv<DT>(x, (pl * IH + ih) * IW + iw));
    }
  }
  stv<DT>(y, i, m);
}

// A chain of n (2 or 3) max-pools of one K x K window, stride 1, padding
// P = K/2, dilation 1, each pooling the previous one's output: pooling a
// pooled map again is a pool of the larger window 2K-1 (then 3K-2) over the
// first input, the borders padded with -inf either way.  One block per plane:
// the plane with a -inf border of R = nP in LDS, row maxima of radius P, 2P
// and 3P (clipped to R), then column maxima of the same radii: output k is
// the Chebyshev window of radius kP.
template <int DT>
__global__ __launch_bounds__(256) void k_maxpool_chain(int H, int W, int P, int n, const void* x, void* y1,
                                                       void* y2, void* y3) {
  extern __shared__ float sm[];
  const int R = n * P, PH = H + 2 * R, PW = W + 2 * R;
  float* xs = sm;             // [PH][PW]
  float* hr = sm + PH * PW;   // [3][PH][W]
  const long long plane = blockIdx.x;
  const long long base = plane * H * W;
  for (int i = threadIdx.x; i < PH * PW; i += 256) {
    const int r = i / PW - R, c = i % PW - R;
    xs[i] = (r >= 0 && r < H && c >= 0 && c < W) ? ldv<DT>(x, base + (long long)r * W + c) : -INFINITY;
  }
  __syncthreads();
  const int r1 = P, r2 = min(2 * P, R), r3 = min(3 * P, R);
  for (int i = threadIdx.x; i < PH * W; i += 256) {
    const int r = i / W, c = i % W;
    const float* row = xs + r * PW + c + R;
    float m1 = -INFINITY, m2 = -INFINITY, m3 = -INFINITY;
    for (int d = -r3; d <= r3; ++d) {
      const float v = row[d];
      const int ad = d < 0 ? -d : d;
      m3 = fmaxf(m3, v);
      if (ad <= r2) m2 = fmaxf(m2, v);
      if (ad <= r1) m1 = fmaxf(m1, v);
    }
    hr[i] = m1;
    hr[PH * W + i] = m2;
    hr[2 * PH * W + i] = m3;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < H * W; i += 256) {
    const int oh = i / W, ow = i % W;
    const float* c0 = hr + (oh + R) * W + ow;
    float a1 = -INFINITY, a2 = -INFINITY, a3 = -INFINITY;
    for (int d = -r1; d <= r1; ++d) a1 = fmaxf(a1, c0[d * W]);
    for (int d = -r2; d <= r2; ++d) a2 = fmaxf(a2, c0[PH * W + d * W]);
    for (int d = -r3; d <= r3; ++d) a3 = fmaxf(a3, c0[2 * PH * W + d * W]);
    stv<DT>(y1, base + i, a1);
    stv<DT>(y2, base + i, a2);
    if (n == 3) stv<DT>(y3, base + i, a3);
  }
}

}  // namespace

size_t max_pool_chain_lds(int H, int W, int P, int n) {
  const long long R = (long long)n * P, PH = H + 2 * R, PW = W + 2 * R;
  return (size_t)(PH * PW + 3 * PH * W) * sizeof(float);
}

hipError_t launch_max_pool_chain(int dtype, int BC, int H, int W, int P, int n, const void* x, void* y1, void* y2,
                                 void* y3, hipStream_t s, std::string* name) {
  if (name) *name = n == 2 ? "max_pool2d_chain2" : "max_pool2d_chain3";
  const size_t lds = max_pool_chain_lds(H, W, P, n);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  if (BC == 0 || is_dry(s)) return hipSuccess;
  if (dtype == WGX_FLOAT16)
    hipLaunchKernelGGL(k_maxpool_chain<WGX_FLOAT16>, dim3(BC), dim3(256), lds, s, H, W, P, n, x, y1, y2, y3);
  else if (dtype == WGX_BFLOAT16)
    hipLaunchKernelGGL(k_maxpool_chain<WGX_BFLOAT16>, dim3(BC), dim3(256), lds, s, H, W, P, n, x, y1, y2, y3);
  else
    hipLaunchKernelGGL(k_maxpool_chain<WGX_FLOAT32>, dim3(BC), dim3(256), lds, s, H, W, P, n, x, y1, y2, y3);
  return hipGetLastError();
}

hipError_t launch_binary(const BcastDesc& d, hipStream_t s, std::string* name) {
  if (name) *name = d.op == 0 ? "binary_add" : "binary_mul";
  if (d.numel == 0 || is_dry(s)) return hipSuccess;
  if (d.dtype == WGX_FLOAT16)
    hipLaunchKernelGGL(k_binary<WGX_FLOAT16>, dim3(blocks_for(d.numel)), dim3(256), 0, s, d);
  else if (d.dtype == WGX_BFLOAT16)
    hipLaunchKernelGGL(k_binary<WGX_BFLOAT16>, dim3(blocks_for(d.numel)), dim3(256), 0, s, d);
  else
    hipLaunchKernelGGL(k_binary<WGX_FLOAT32>, dim3(blocks_for(d.numel)), dim3(256), 0, s, d);
  return hipGetLastError();
}

hipError_t launch_unary(int op, int dtype, long long n, const void* x, void* y, hipStream_t s,
                        std::string* name) {
  static const char* names[] = {"unary_sigmoid", "unary_relu", "unary_hardswish", "unary_silu"};
  if (name) *name = names[op & 3];
  if (n == 0 || is_dry(s)) return hipSuccess;
  if (dtype == WGX_FLOAT16)
    hipLaunchKernelGGL(k_unary<WGX_FLOAT16>, dim3(blocks_for(n)), dim3(256), 0, s, op, n, x, y);
  else if (dtype == WGX_BFLOAT16)
    hipLaunchKernelGGL(k_unary<WGX_BFLOAT16>, dim3(blocks_for(n)), dim3(256), 0, s, op, n, x, y);
  else
    hipLaunchKernelGGL(k_unary<WGX_FLOAT32>, dim3(blocks_for(n)), dim3(256), 0, s, op, n, x, y);
  return hipGetLastError();
}

hipError_t launch_slab_copy(int elsize, long long outer, long long inner_src, long long inner_dst,
                            long long dst_off, long long src_off, const void* src, void* dst,
                            bool gather, hipStream_t s, std::string* name) {
  if (name) *name = gather ? "slab_gather" : "slab_scatter";
  const long long n = outer * (gather ? inner_dst : inner_src);
  if (n == 0 || is_dry(s)) return hipSuccess;
  const dim3 g(blocks_for(n));
  switch (elsize) {
    case 1:
      hipLaunchKernelGGL(k_slab<uint8_t>, g, dim3(256), 0, s, outer, inner_src, inner_dst, dst_off,
                         src_off, (const uint8_t*)src, (uint8_t*)dst, gather);
      break;
    case 2:
      hipLaunchKernelGGL(k_slab<uint16_t>, g, dim3(256), 0, s, outer, inner_src, inner_dst, dst_off,
                         src_off, (const uint16_t*)src, (uint16_t*)dst, gather);
      break;
    case 4:
      hipLaunchKernelGGL(k_slab<uint32_t>, g, dim3(256), 0, s, outer, inner_src, inner_dst, dst_off,
                         src_off, (const uint32_t*)src, (uint32_t*)dst, gather);
      break;
    default:
      hipLaunchKernelGGL(k_slab<uint64_t>, g, dim3(256), 0, s, outer, inner_src, inner_dst, dst_off,
                         src_off, (const uint64_t*)src, (uint64_t*)dst, gather);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_upsample_nearest(int dtype, int BC, int IH, int IW, int OH, int OW,
                                   const void* x, void* y, hipStream_t s, std::string* name) {
  if (name) *name = "upsample_nearest2d";
  const long long n = (long long)BC * OH * OW;
  if (n == 0 || is_dry(s)) return hipSuccess;
  if (dtype == WGX_FLOAT16)
    hipLaunchKernelGGL(k_upsample<WGX_FLOAT16>, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW,
                       OH, OW, x, y);
  else if (dtype == WGX_BFLOAT16)
    hipLaunchKernelGGL(k_upsample<WGX_BFLOAT16>, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW,
                       OH, OW, x, y);
  else
    hipLaunchKernelGGL(k_upsample<WGX_FLOAT32>, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW,
                       OH, OW, x, y);
  return hipGetLastError();
}

hipError_t launch_max_pool(int dtype, int BC, int IH, int IW, int OH, int OW, int KH, int KW,
                           int sH, int sW, int pH, int pW, int dH, int dW, const void* x, void* y,
                           hipStream_t s, std::string* name) {
  if (name) *name = "max_pool2d";
  const long long n = (long long)BC * OH * OW;
  if (n == 0 || is_dry(s)) return hipSuccess;
  if (dtype == WGX_FLOAT16)
    hipLaunchKernelGGL(k_maxpool<WGX_FLOAT16>, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW,
                       OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, x, y);
  else if (dtype == WGX_BFLOAT16)
    hipLaunchKernelGGL(k_maxpool<WGX_BFLOAT16>, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW,
                       OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, x, y);
  else
    hipLaunchKernelGGL(k_maxpool<WGX_FLOAT32>, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW,
                       OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, x, y);
  return hipGetLastError();
}

}  // namespace wgx
