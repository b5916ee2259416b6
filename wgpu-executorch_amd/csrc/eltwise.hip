// eltwise.hip -- the simple, bandwidth-bound ops a YOLO-style program chain
// needs around the GEMM-shaped hot path: broadcast add/sub/mul
// (src/shaders/add/index.ts:33-129, add-broadcast*.wgsl.ts), unary activations
// (sigmoid/relu/hardswish), cat / split_with_sizes as strided slab copies,
// nearest upsample, max-pool with indices, permute_copy and softmax.  One
// lane per output element (a wave per row for softmax), float32 arithmetic,
// one rounding to the storage type.  Not an optimisation target.
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

// v rounded to the storage type and back (what a load of the stored value gives)
template <int DT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (DT == WGX_FLOAT32) return v;
  else if constexpr (DT == WGX_FLOAT16)
    return (float)(_Float16)v;
  else {
    const uint32_t u = __float_as_uint(v);
    const uint32_t h = ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    return __uint_as_float(h << 16);
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

// Initial value of a max-pool window: the most negative finite value of
// the reference's arithmetic type (-65504 in f16, -3.4e38 in f32), so an
// element wins only if it is strictly greater (NaN and -inf never do), and a
// window with no element inside the image yields that value with index 0
// (src/shaders/max-pool-2d/max-pool-2d-spatial.wgsl.ts:52-79).
template <int DT>
__device__ __forceinline__ float pool_floor() {
  return DT == WGX_FLOAT16 ? -65504.0f : -3.4e38f;
}

// One output per lane: the first strictly greatest element of the window in
// row-major (kh outer, kw inner) order; its flat index ih * IW + iw within
// the plane goes to idx when idx is not null.
template <int DT>
__global__ __launch_bounds__(256) void k_maxpool(int BC, int IH, int IW, int OH, int OW, int KH,
                                                 int KW, int sH, int sW, int pH, int pW, int dH,
                                                 int dW, const void* x, void* y, int32_t* idx) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)BC * OH * OW) return;
  const int ow = (int)(i % OW), oh = (int)((i / OW) % OH);
  const long long pl = i / ((long long)OH * OW);
  float m = pool_floor<DT>();
  int at = 0;
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * sH - pH + kh * dH;
    if (ih < 0 || ih >= IH) continue;
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = ow * sW - pW + kw * dW;
      if (iw < 0 || iw >= IW) continue;
      const float v = ldv<DT>(x, (pl * IH + ih) * IW + iw);
      if (v > m) {
        m = v;
        at = ih * IW + iw;
      }
    }
  }
  stv<DT>(y, i, m);
  if (idx) idx[i] = at;
}

// A chain of n (2 or 3) max-pools of one K x K window (K = 2P + 1), stride
// 1, padding P, dilation 1, each pooling the previous one's output (the SPPF
// block of YOLO-style detectors), in one launch.  One block per plane: the
// plane sits in LDS with a border of P cells holding -inf (an element that
// never wins, as the reference skips cells outside the image); each level
// pools the previous level's LDS image into the other buffer, with the same
// first-strictly-greatest rule and initial value as k_maxpool, and writes its
// values (and indices into the previous level's plane) straight out.  Every
// level maps pixel i to the same lane, so a lane writes level 1, 2, 3 of a
// pixel in that order: index outputs that share memory end as level n's, as
// after n separate launches.
template <int DT>
__global__ __launch_bounds__(256) void k_maxpool_chain(int H, int W, int P, int n, const void* x, void* y1,
                                                       void* y2, void* y3, int32_t* i1, int32_t* i2,
                                                       int32_t* i3) {
  extern __shared__ float sm[];
  const int PW = W + 2 * P, PH = H + 2 * P, K = 2 * P + 1;
  float* a = sm;            // [PH][PW], the level being pooled
  float* b = sm + PH * PW;  // [PH][PW], the level being written
  const long long base = (long long)blockIdx.x * H * W;
  for (int i = threadIdx.x; i < PH * PW; i += 256) {
    const int r = i / PW - P, c = i % PW - P;
    a[i] = (r >= 0 && r < H && c >= 0 && c < W) ? ldv<DT>(x, base + (long long)r * W + c) : -INFINITY;
    b[i] = -INFINITY;
  }
  __syncthreads();
  void* ys[3] = {y1, y2, y3};
  int32_t* is[3] = {i1, i2, i3};
  for (int l = 0; l < n; ++l) {
    for (int i = threadIdx.x; i < H * W; i += 256) {
      const int oh = i / W, ow = i % W;
      float m = pool_floor<DT>();
      int at = 0;
      for (int kh = 0; kh < K; ++kh) {
        const float* row = a + (oh + kh) * PW + ow;
        for (int kw = 0; kw < K; ++kw) {
          const float v = row[kw];
          if (v > m) {
            m = v;
            at = (oh + kh - P) * W + ow + kw - P;
          }
        }
      }
      // the stored value, rounded to the storage type, is the next level's input
      stv<DT>(ys[l], base + i, m);
      b[(oh + P) * PW + ow + P] = rnd<DT>(m);
      if (is[l]) is[l][base + i] = at;
    }
    __syncthreads();
    float* t = a;
    a = b;
    b = t;
  }
}

// permute_copy, general form: out element i (row-major over out_shape)
// reads the input element whose coordinate along input dim perm[k] is out
// coordinate k (src/shaders/permute/permute.wgsl.ts).
template <typename E>
__global__ __launch_bounds__(256) void k_permute(PermuteDesc d, long long n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  long long rem = i, src = 0;
  for (int k = d.ndim - 1; k >= 0; --k) {
    const long long c = rem % d.out_shape[k];
    rem /= d.out_shape[k];
    src += c * d.src_stride[k];
  }
  static_cast<E*>(d.y)[i] = static_cast<const E*>(d.x)[src];
}

// Batched transpose [batch, R, C] -> [batch, C, R] (a permutation that swaps
// the last two dimensions): a 64 x 64 tile per block, read along rows and
// written along columns of the input, both coalesced, through LDS (one
// padding column so the column reads hit distinct banks).
template <typename E>
__global__ __launch_bounds__(256) void k_transpose(long long R, long long C, const E* x, E* y) {
  __shared__ E t[64][65];
  const long long off = (long long)blockIdx.z * R * C;
  const long long r0 = (long long)blockIdx.y * 64, c0 = (long long)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const long long r = r0 + i, c = c0 + tx;
    if (r < R && c < C) t[i][tx] = x[off + r * C + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const long long c = c0 + i, r = r0 + tx;
    if (c < C && r < R) y[off + c * R + r] = t[tx][i];
  }
}

// Softmax of one contiguous row per wave64 (inner extent 1): each lane keeps
// a running maximum and a sum of exponentials rescaled to it over its
// strided share of the row, the lanes combine their (max, sum) pairs by
// butterfly shuffles, then every element is written as exp(x - max) / sum.
// float32 throughout (the reference's f16 kernels accumulate in f16,
// src/shaders/softmax/softmax-last-dim-f16.wgsl.ts:34-48).
__device__ __forceinline__ void softmax_merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  s = s * __expf(m - mm) + s2 * __expf(m2 - mm);
  m = mm;
}

template <int DT>
__global__ __launch_bounds__(256) void k_softmax_rows(long long rows, long long r, const void* x, void* y) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const long long base = row * r;
  float m = -3.4e38f, s = 0.0f;
  for (long long j = lane; j < r; j += 64) {
    const float v = ldv<DT>(x, base + j);
    if (v > m) {
      s *= __expf(m - v);
      m = v;
    }
    s += __expf(v - m);
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    softmax_merge(m, s, m2, s2);
  }
  const float inv = 1.0f / s;
  for (long long j = lane; j < r; j += 64) stv<DT>(y, base + j, __expf(ldv<DT>(x, base + j) - m) * inv);
}

// Softmax along a dimension with inner extent > 1: one lane per (outer,
// inner) line, consecutive lanes on consecutive inner positions, so each
// step of the line walk is one coalesced row of the wave.
template <int DT>
__global__ __launch_bounds__(256) void k_softmax_strided(long long outer, long long r, long long inner,
                                                         const void* x, void* y) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const long long o = t / inner, in = t % inner;
  const long long base = o * r * inner + in;
  float m = -3.4e38f, s = 0.0f;
  for (long long j = 0; j < r; ++j) {
    const float v = ldv<DT>(x, base + j * inner);
    if (v > m) {
      s *= __expf(m - v);
      m = v;
    }
    s += __expf(v - m);
  }
  const float inv = 1.0f / s;
  for (long long j = 0; j < r; ++j) stv<DT>(y, base + j * inner, __expf(ldv<DT>(x, base + j * inner) - m) * inv);
}

}  // namespace

size_t max_pool_chain_lds(int H, int W, int P) {
  const long long PH = H + 2LL * P, PW = W + 2LL * P;
  return (size_t)(2 * PH * PW) * sizeof(float);
}

hipError_t launch_max_pool_chain(int dtype, int BC, int H, int W, int P, int n, const void* x, void* const y[3],
                                 int32_t* const idx[3], hipStream_t s, std::string* name) {
  if (name) *name = n == 2 ? "max_pool2d_chain2" : "max_pool2d_chain3";
  const size_t lds = max_pool_chain_lds(H, W, P);
  if (lds > 64 * 1024 || n < 2 || n > 3) return hipErrorInvalidValue;
  if (BC == 0 || is_dry(s)) return hipSuccess;
  auto k = dtype == WGX_FLOAT16 ? k_maxpool_chain<WGX_FLOAT16>
           : dtype == WGX_BFLOAT16 ? k_maxpool_chain<WGX_BFLOAT16> : k_maxpool_chain<WGX_FLOAT32>;
  hipLaunchKernelGGL(k, dim3(BC), dim3(256), lds, s, H, W, P, n, x, y[0], y[1], y[2], idx[0], idx[1], idx[2]);
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
                           int32_t* idx, hipStream_t s, std::string* name) {
  if (name) *name = "max_pool2d";
  const long long n = (long long)BC * OH * OW;
  if (n == 0 || is_dry(s)) return hipSuccess;
  auto k = dtype == WGX_FLOAT16 ? k_maxpool<WGX_FLOAT16>
           : dtype == WGX_BFLOAT16 ? k_maxpool<WGX_BFLOAT16> : k_maxpool<WGX_FLOAT32>;
  hipLaunchKernelGGL(k, dim3(blocks_for(n)), dim3(256), 0, s, BC, IH, IW, OH, OW, KH, KW, sH, sW, pH, pW,
                     dH, dW, x, y, idx);
  return hipGetLastError();
}

hipError_t launch_permute(const PermuteDesc& d, hipStream_t s, std::string* name) {
  // the last two dimensions swapped, the others kept: a batched transpose
  bool swap2 = d.ndim >= 2 && d.perm[d.ndim - 1] == d.ndim - 2 && d.perm[d.ndim - 2] == d.ndim - 1;
  for (int k = 0; k + 2 < d.ndim; ++k) swap2 = swap2 && d.perm[k] == k;
  long long batch = 1;
  for (int k = 0; k + 2 < d.ndim; ++k) batch *= d.in_shape[k];
  const long long R = swap2 ? d.in_shape[d.ndim - 2] : 0, C = swap2 ? d.in_shape[d.ndim - 1] : 0;
  swap2 = swap2 && batch <= 65535 && (R + 63) / 64 <= 65535;
  if (name) *name = swap2 ? "permute_transpose" : "permute_gather";
  long long n = 1;
  for (int k = 0; k < d.ndim; ++k) n *= d.in_shape[k];
  if (n == 0 || is_dry(s)) return hipSuccess;
  if (swap2) {
    const dim3 g((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64), (unsigned)batch);
    switch (d.elsize) {
      case 1: hipLaunchKernelGGL(k_transpose<uint8_t>, g, dim3(256), 0, s, R, C, (const uint8_t*)d.x, (uint8_t*)d.y); break;
      case 2: hipLaunchKernelGGL(k_transpose<uint16_t>, g, dim3(256), 0, s, R, C, (const uint16_t*)d.x, (uint16_t*)d.y); break;
      case 4: hipLaunchKernelGGL(k_transpose<uint32_t>, g, dim3(256), 0, s, R, C, (const uint32_t*)d.x, (uint32_t*)d.y); break;
      default: hipLaunchKernelGGL(k_transpose<uint64_t>, g, dim3(256), 0, s, R, C, (const uint64_t*)d.x, (uint64_t*)d.y); break;
    }
    return hipGetLastError();
  }
  PermuteDesc q = d;
  // out dim k reads input dim perm[k]: its input stride
  long long st[WGX_MAX_NDIM], acc = 1;
  for (int k = d.ndim - 1; k >= 0; --k) {
    st[k] = acc;
    acc *= d.in_shape[k];
  }
  for (int k = 0; k < d.ndim; ++k) {
    q.out_shape[k] = d.in_shape[d.perm[k]];
    q.src_stride[k] = st[d.perm[k]];
  }
  const dim3 g(blocks_for(n));
  switch (d.elsize) {
    case 1: hipLaunchKernelGGL(k_permute<uint8_t>, g, dim3(256), 0, s, q, n); break;
    case 2: hipLaunchKernelGGL(k_permute<uint16_t>, g, dim3(256), 0, s, q, n); break;
    case 4: hipLaunchKernelGGL(k_permute<uint32_t>, g, dim3(256), 0, s, q, n); break;
    default: hipLaunchKernelGGL(k_permute<uint64_t>, g, dim3(256), 0, s, q, n); break;
  }
  return hipGetLastError();
}

hipError_t launch_softmax(int dtype, long long outer, long long r, long long inner, const void* x, void* y,
                          hipStream_t s, std::string* name) {
  if (name) *name = inner == 1 ? "softmax_rows" : "softmax_strided";
  if (outer * r * inner == 0 || is_dry(s)) return hipSuccess;
  if (inner == 1) {
    auto k = dtype == WGX_FLOAT16 ? k_softmax_rows<WGX_FLOAT16>
             : dtype == WGX_BFLOAT16 ? k_softmax_rows<WGX_BFLOAT16> : k_softmax_rows<WGX_FLOAT32>;
    hipLaunchKernelGGL(k, dim3((unsigned)((outer + 3) / 4)), dim3(256), 0, s, outer, r, x, y);
  } else {
    auto k = dtype == WGX_FLOAT16 ? k_softmax_strided<WGX_FLOAT16>
             : dtype == WGX_BFLOAT16 ? k_softmax_strided<WGX_BFLOAT16> : k_softmax_strided<WGX_FLOAT32>;
    hipLaunchKernelGGL(k, dim3(blocks_for(outer * inner)), dim3(256), 0, s, outer, r, inner, x, y);
  }
  return hipGetLastError();
}

}  // namespace wgx
