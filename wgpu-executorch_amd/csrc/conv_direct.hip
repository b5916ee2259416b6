// conv_direct.hip -- the correctness fallbacks of aten.convolution: grouped
// convolution with 1 < groups (not depthwise) and transposed convolution.
//
// Reference: conv2d.wgsl.ts:44-89 (direct, one thread per output, general
// groups) and conv-transpose2d.wgsl.ts:48-99 (gather form), selected by
// src/shaders/convolution/index.ts:213-222.  Neither is on a benchmarked
// configuration; these kernels exist so the convolution entry point accepts
// everything the reference accepts.  One lane per output element, float32
// accumulation (bias first, then input channels and taps in the reference's
// order), one rounding to the storage type.
#include <math.h>
#include <stdio.h>

#include "internal.h"

namespace wgx {
namespace {

struct DcParams {
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int B, IC, IH, IW, OC, OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, groups;
  int has_clamp;
  int act;
  float cmin, cmax;
  long long total;
};

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

template <int DT, bool TRANSPOSED>
__global__ __launch_bounds__(256) void k_direct(DcParams p) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total) return;
  const int ow = (int)(i % p.OW);
  const int oh = (int)((i / p.OW) % p.OH);
  const int oc = (int)((i / ((long long)p.OW * p.OH)) % p.OC);
  const int b = (int)(i / ((long long)p.OW * p.OH * p.OC));
  const int icpg = p.IC / p.groups, ocpg = p.OC / p.groups;
  const int g = oc / ocpg;
  float acc = p.bias ? ldv<DT>(p.bias, oc) : 0.0f;
  if constexpr (!TRANSPOSED) {
    for (int icg = 0; icg < icpg; ++icg) {
      const int ic = g * icpg + icg;
      for (int kh = 0; kh < p.KH; ++kh) {
        const int ih = oh * p.sH - p.pH + kh * p.dH;
        if (ih < 0 || ih >= p.IH) continue;
        for (int kw = 0; kw < p.KW; ++kw) {
          const int iw = ow * p.sW - p.pW + kw * p.dW;
          if (iw < 0 || iw >= p.IW) continue;
          acc += ldv<DT>(p.x, (((long long)b * p.IC + ic) * p.IH + ih) * p.IW + iw) *
                 ldv<DT>(p.w, (((long long)oc * icpg + icg) * p.KH + kh) * p.KW + kw);
        }
      }
    }
  } else {
    const int oc_in_g = oc % ocpg;
    for (int kh = 0; kh < p.KH; ++kh) {
      const int nh = oh + p.pH - kh * p.dH;
      if (nh < 0 || nh % p.sH != 0) continue;
      const int ih = nh / p.sH;
      if (ih >= p.IH) continue;
      for (int kw = 0; kw < p.KW; ++kw) {
        const int nw = ow + p.pW - kw * p.dW;
        if (nw < 0 || nw % p.sW != 0) continue;
        const int iw = nw / p.sW;
        if (iw >= p.IW) continue;
        for (int icg = 0; icg < icpg; ++icg) {
          const int ic = g * icpg + icg;
          acc += ldv<DT>(p.x, (((long long)b * p.IC + ic) * p.IH + ih) * p.IW + iw) *
                 ldv<DT>(p.w, (((long long)ic * ocpg + oc_in_g) * p.KH + kh) * p.KW + kw);
        }
      }
    }
  }
  acc = apply_act(p.act, acc);
  if (p.has_clamp) acc = fminf(fmaxf(acc, p.cmin), p.cmax);
  stv<DT>(p.y, i, acc);
}

// Dense convolutions with few taps per output channel (IC * KH * KW <= 32,
// OC <= OCB): the network stems, e.g. [1,3,640,640] * [16,3,3,3] s2.  As a
// GEMM their K is too short for the matrix cores and their weight rows are
// not 16-byte vectors (K = 27), so the GEMM path falls back to element loads
// (28 us for that stem on MI355X).  Here one lane computes every output
// channel of one output pixel: the weights sit in LDS as fp32 [tap][OCB]
// (zero past OC) and are read as broadcast float4s, the lane's input window
// is read once per tap (zero outside the image), and each output channel is
// one coalesced store across the wave's consecutive pixels.  fp32
// accumulation, bias first, taps in the reference's order (ic, kh, kw).
template <int DT, int OCB>
__global__ __launch_bounds__(256) void k_conv_small(DcParams p) {
  constexpr int MAXT = 32;
  __shared__ __attribute__((aligned(16))) float ws[MAXT * OCB];
  __shared__ __attribute__((aligned(16))) float bs[OCB];
  const int T = p.IC * p.KH * p.KW;
  for (int i = threadIdx.x; i < MAXT * OCB; i += 256) {
    const int t = i / OCB, oc = i - t * OCB;
    ws[i] = (t < T && oc < p.OC) ? ldv<DT>(p.w, (long long)oc * T + t) : 0.0f;
  }
  for (int i = threadIdx.x; i < OCB; i += 256) bs[i] = (p.bias && i < p.OC) ? ldv<DT>(p.bias, i) : 0.0f;
  __syncthreads();
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total) return;
  const int ow = (int)(i % p.OW);
  const int oh = (int)((i / p.OW) % p.OH);
  const int b = (int)(i / ((long long)p.OW * p.OH));
  float acc[OCB];
#pragma unroll
  for (int oc = 0; oc < OCB; ++oc) acc[oc] = bs[oc];
  int t = 0;
  for (int ic = 0; ic < p.IC; ++ic)
    for (int kh = 0; kh < p.KH; ++kh) {
      const int ih = oh * p.sH - p.pH + kh * p.dH;
      for (int kw = 0; kw < p.KW; ++kw, ++t) {
        const int iw = ow * p.sW - p.pW + kw * p.dW;
        const bool in = ih >= 0 && ih < p.IH && iw >= 0 && iw < p.IW;
        const float xv = in ? ldv<DT>(p.x, (((long long)b * p.IC + ic) * p.IH + ih) * p.IW + iw) : 0.0f;
        const float4* wr = reinterpret_cast<const float4*>(ws + t * OCB);
#pragma unroll
        for (int q = 0; q < OCB / 4; ++q) {
          const float4 w4 = wr[q];
          acc[4 * q] += w4.x * xv;
          acc[4 * q + 1] += w4.y * xv;
          acc[4 * q + 2] += w4.z * xv;
          acc[4 * q + 3] += w4.w * xv;
        }
      }
    }
  const long long plane = (long long)p.OH * p.OW;
  const long long ybase = (long long)b * p.OC * plane + (long long)oh * p.OW + ow;
#pragma unroll
  for (int oc = 0; oc < OCB; ++oc) {
    if (oc < p.OC) {
      float v = apply_act(p.act, acc[oc]);
      if (p.has_clamp) v = fminf(fmaxf(v, p.cmin), p.cmax);
      stv<DT>(p.y, ybase + oc * plane, v);
    }
  }
}

template <int DT>
hipError_t go_small(const DcParams& p, int ocb, hipStream_t s) {
  if (is_dry(s) || p.total == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((p.total + 255) / 256);
  if (ocb == 16) hipLaunchKernelGGL((k_conv_small<DT, 16>), dim3(blocks), dim3(256), 0, s, p);
  else if (ocb == 32) hipLaunchKernelGGL((k_conv_small<DT, 32>), dim3(blocks), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((k_conv_small<DT, 64>), dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int DT>
hipError_t go(const DcParams& p, bool transposed, hipStream_t s) {
  if (is_dry(s) || p.total == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((p.total + 255) / 256);
  if (transposed)
    hipLaunchKernelGGL((k_direct<DT, true>), dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((k_direct<DT, false>), dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace

bool small_tap_conv(const DirectConvDesc& d) {
  return !d.transposed && d.groups == 1 && d.IC * d.KH * d.KW <= 32 && d.OC <= 64;
}

hipError_t launch_direct_conv(const DirectConvDesc& d, hipStream_t s, std::string* name) {
  DcParams p;
  p.x = d.x;
  p.w = d.w;
  p.bias = d.bias;
  p.y = d.y;
  p.B = d.B;
  p.IC = d.IC;
  p.IH = d.IH;
  p.IW = d.IW;
  p.OC = d.OC;
  p.OH = d.OH;
  p.OW = d.OW;
  p.KH = d.KH;
  p.KW = d.KW;
  p.sH = d.sH;
  p.sW = d.sW;
  p.pH = d.pH;
  p.pW = d.pW;
  p.dH = d.dH;
  p.dW = d.dW;
  p.groups = d.groups;
  p.has_clamp = d.has_clamp;
  p.act = d.act;
  p.cmin = d.cmin;
  p.cmax = d.cmax;
  if (small_tap_conv(d)) {
    p.total = (long long)d.B * d.OH * d.OW;
    const int ocb = d.OC <= 16 ? 16 : (d.OC <= 32 ? 32 : 64);
    if (name) *name = "conv_small_taps_oc" + std::to_string(ocb);
    if (p.total >= (1LL << 31) * 256LL) return hipErrorInvalidValue;
    if (d.dtype == WGX_FLOAT16) return go_small<WGX_FLOAT16>(p, ocb, s);
    if (d.dtype == WGX_BFLOAT16) return go_small<WGX_BFLOAT16>(p, ocb, s);
    return go_small<WGX_FLOAT32>(p, ocb, s);
  }
  p.total = (long long)d.B * d.OC * d.OH * d.OW;
  if (name) *name = d.transposed ? "conv_transpose_direct" : "conv_grouped_direct";
  if (d.dtype == WGX_FLOAT16) return go<WGX_FLOAT16>(p, d.transposed, s);
  if (d.dtype == WGX_BFLOAT16) return go<WGX_BFLOAT16>(p, d.transposed, s);
  return go<WGX_FLOAT32>(p, d.transposed, s);
}

}  // namespace wgx
