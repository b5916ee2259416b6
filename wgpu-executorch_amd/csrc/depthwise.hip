// depthwise.hip -- depthwise conv2d (groups == IC == OC, weight [C,1,KH,KW]),
// NCHW, float16 / bfloat16 / float32 storage, float32 arithmetic.
//
// Serves the depthwise branch of aten.convolution (src/shaders/convolution/
// index.ts:194-221: conv2d-depthwise-3x3*.wgsl.ts for 3x3 s1 p1 d1 and
// conv2d-depthwise*.wgsl.ts for any other kernel <= 7x7).  One kernel covers
// both: the work is HBM-bound (about 2 flop per byte), so the design goal is
// to move every input and output byte once, with full-width coalesced accesses.
//
// A block owns a band of output rows of one plane (or several whole planes when
// a plane has fewer outputs than the block has lanes).  It streams the input
// rows the band needs into LDS once -- zero-filled outside the image, so the
// stencil loop has no bounds tests -- then each lane produces outputs along a
// row (consecutive lanes -> consecutive ow, so the stores coalesce).  Accumulation:
// bias first, then taps kh-outer / kw-inner (the reference's order,
// conv2d-depthwise.wgsl.ts:228-268), in float32, rounded once.
#include <math.h>
#include <stdio.h>

#include "internal.h"

namespace wgx {
namespace {

constexpr int NT = 256;

struct DwParams {
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int C, IH, IW, OH, OW, KH, KW, sH, sW, pH, pW, dH, dW;
  int toh;      // output rows per band
  int bands;    // bands per plane
  int ppb;      // planes per block (bands == 1 when ppb > 1)
  int nplanes;  // B * C
  int in_rows;  // LDS rows per band
  int lw;       // LDS row width
  int has_clamp;
  float cmin, cmax;
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

template <int DT, int KH_, int KW_>
__global__ __launch_bounds__(NT) void k_depthwise(DwParams p) {
  extern __shared__ float lds[];
  const int KH = KH_ ? KH_ : p.KH;
  const int KW = KW_ ? KW_ : p.KW;
  const int khw = KH * KW;
  const int tid = threadIdx.x;
  int plane0, band;
  if (p.ppb > 1) {
    plane0 = blockIdx.x * p.ppb;
    band = 0;
  } else {
    plane0 = blockIdx.x / p.bands;
    band = blockIdx.x % p.bands;
  }
  const int nloc = min(p.ppb, p.nplanes - plane0);
  const int oh0 = band * p.toh;
  const int ih_base = oh0 * p.sH - p.pH;
  const int plane_in = p.in_rows * p.lw;
  float* wl = lds + p.ppb * plane_in;  // [ppb][khw] weights, then [ppb] bias

  // weights and bias of the planes this block owns
  for (int i = tid; i < nloc * (khw + 1); i += NT) {
    const int pp = i / (khw + 1), j = i % (khw + 1);
    const int c = (plane0 + pp) % p.C;
    float v;
    if (j < khw) v = ldv<DT>(p.w, (long long)c * khw + j);
    else v = p.bias ? ldv<DT>(p.bias, c) : 0.0f;
    wl[pp * (khw + 1) + j] = v;
  }

  // input band -> LDS, zero outside the image (LDS column j is iw = j - pW)
  const int total_in = nloc * plane_in;
  for (int i = tid; i < total_in; i += NT) {
    const int pp = i / plane_in, rem = i % plane_in;
    const int r = rem / p.lw, col = rem % p.lw;
    const int ih = ih_base + r, iw = col - p.pW;
    float v = 0.0f;
    if (ih >= 0 && ih < p.IH && iw >= 0 && iw < p.IW)
      v = ldv<DT>(p.x, ((long long)(plane0 + pp) * p.IH + ih) * p.IW + iw);
    lds[i] = v;
  }
  __syncthreads();

  const int rows_here = min(p.toh, p.OH - oh0);
  const int total_out = nloc * rows_here * p.OW;
  for (int i = tid; i < total_out; i += NT) {
    const int pp = i / (rows_here * p.OW), rem = i % (rows_here * p.OW);
    const int orow = rem / p.OW, ow = rem % p.OW;
    const float* src = lds + pp * plane_in + (orow * p.sH) * p.lw + ow * p.sW;
    const float* wp = wl + pp * (khw + 1);
    float acc = wp[khw];
    if constexpr (KH_ > 0) {
#pragma unroll
      for (int kh = 0; kh < KH_; ++kh)
#pragma unroll
        for (int kw = 0; kw < KW_; ++kw)
          acc += src[kh * p.dH * p.lw + kw * p.dW] * wp[kh * KW_ + kw];
    } else {
      for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw) acc += src[kh * p.dH * p.lw + kw * p.dW] * wp[kh * KW + kw];
    }
    if (p.has_clamp) acc = fminf(fmaxf(acc, p.cmin), p.cmax);
    stv<DT>(p.y, ((long long)(plane0 + pp) * p.OH + oh0 + orow) * p.OW + ow, acc);
  }
}

template <int DT>
hipError_t launch_dt(const DwParams& p, int blocks, size_t lds, hipStream_t s, std::string* name) {
  char buf[64];
  auto go = [&](auto fn, const char* tag) {
    if (name) {
      snprintf(buf, sizeof buf, "depthwise_%s_%s", DT == WGX_FLOAT32 ? "f32" : DT == WGX_FLOAT16 ? "f16" : "bf16", tag);
      *name = buf;
    }
    if (lds > 64 * 1024 && s != name_only()) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    if (is_dry(s)) return hipSuccess;
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(NT), lds, s, p);
    return hipGetLastError();
  };
  if (p.KH == 3 && p.KW == 3) return go(k_depthwise<DT, 3, 3>, "3x3");
  if (p.KH == 5 && p.KW == 5) return go(k_depthwise<DT, 5, 5>, "5x5");
  return go(k_depthwise<DT, 0, 0>, "kxk");
}

}  // namespace

hipError_t launch_depthwise(const DwDesc& d, hipStream_t s, std::string* name) {
  DwParams p;
  p.x = d.x;
  p.w = d.w;
  p.bias = d.bias;
  p.y = d.y;
  p.C = d.C;
  p.IH = d.IH;
  p.IW = d.IW;
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
  p.has_clamp = d.has_clamp;
  p.cmin = d.cmin;
  p.cmax = d.cmax;
  p.nplanes = d.B * d.C;
  // LDS row width: every column any output touches, iw in [-pW, (OW-1)sW - pW + (KW-1)dW].
  p.lw = (d.OW - 1) * d.sW + (d.KW - 1) * d.dW + 1;
  const int plane_out = d.OH * d.OW;
  const int khw = d.KH * d.KW;
  if (plane_out < NT) {
    p.ppb = NT / plane_out < 16 ? NT / plane_out : 16;
    if (p.ppb < 1) p.ppb = 1;
    p.toh = d.OH;
    p.bands = 1;
  } else {
    p.ppb = 1;
    // about 4 outputs per lane per band, at least one row
    int toh = (4 * NT + d.OW - 1) / d.OW;
    if (toh > d.OH) toh = d.OH;
    if (toh < 1) toh = 1;
    p.toh = toh;
    p.bands = (d.OH + toh - 1) / toh;
  }
  p.in_rows = (p.toh - 1) * d.sH + (d.KH - 1) * d.dH + 1;
  const size_t lds = sizeof(float) * ((size_t)p.ppb * p.in_rows * p.lw + (size_t)p.ppb * (khw + 1));
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const int blocks = p.ppb > 1 ? (p.nplanes + p.ppb - 1) / p.ppb : p.nplanes * p.bands;
  if (d.dtype == WGX_FLOAT16) return launch_dt<WGX_FLOAT16>(p, blocks, lds, s, name);
  if (d.dtype == WGX_BFLOAT16) return launch_dt<WGX_BFLOAT16>(p, blocks, lds, s, name);
  return launch_dt<WGX_FLOAT32>(p, blocks, lds, s, name);
}

}  // namespace wgx
