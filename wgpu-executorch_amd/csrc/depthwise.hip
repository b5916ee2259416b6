// depthwise.hip -- depthwise conv2d (groups == IC == OC, weight [C,1,KH,KW]),
// NCHW, float16 / bfloat16 / float32 storage, float32 arithmetic.
//
// Serves the depthwise branch of aten.convolution (src/shaders/convolution/
// index.ts:194-221: conv2d-depthwise-3x3*.wgsl.ts for 3x3 s1 p1 d1 and
// conv2d-depthwise*.wgsl.ts for any other kernel <= 7x7).  The work is
// HBM-bound (about 2 flop per byte for 3x3 stride 1), so the design goal is to
// move every input and output byte once, in full-width coalesced accesses,
// while keeping the per-output instruction count well under what the vector
// ALUs can issue at HBM speed (about 20 per output for fp16 3x3).
//
// Three kernels, tried in this order:
//  * k_dw_reg<K, S, OV, R> (fp16; K x K with K in {3, 5}, stride S in {1, 2}
//    in both dimensions, "same" padding P = K/2, dilation 1, even widths): no
//    LDS at all.  Each lane walks a band of R output rows down a column strip
//    of OV outputs, holding every input row of the band in registers (packed
//    halves), with the halo columns taken from the neighbouring lanes.  Tap
//    pairs are v_dot2_f32_f16, odd taps v_fma_mix_f32: fp32 accumulation
//    without unpacking the input.
//  * k_dw_fast<DT, K, S, OV>: the same kernel family for any width and for
//    float32.  A block owns ppb whole planes, or a band of output rows of one
//    large plane.  The input rows it needs form one contiguous range of
//    memory; the block reads it with 16-byte vector loads (aligned chunks of
//    the flat range, so any plane width works) and writes it, converted to
//    fp32, into an LDS tile with a zero border -- the stencil loop then has no
//    bounds tests.  Each lane produces OV consecutive outputs of one row from
//    float4 reads of its input window and writes them with one vector store;
//    consecutive lanes own consecutive output segments, so stores coalesce.
//  * k_depthwise<DT, KH, KW>: any kernel size, stride, padding and dilation
//    (element-wise staging through LDS).  Correct for every shape the
//    convolution driver accepts; used where the two above do not apply.
// All three accumulate in fp32 in the reference's order: bias, then taps
// kh-outer / kw-inner (conv2d-depthwise.wgsl.ts:56-128), rounded once.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

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
  int act;
  float cmin, cmax;
  const void* res;  // residual (output-shaped) or null: y = rcs * y + rrs * res
  float rcs, rrs;
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
__device__ __forceinline__ uint32_t to_bits(float v) {
  if constexpr (DT == WGX_FLOAT32) return __float_as_uint(v);
  else if constexpr (DT == WGX_FLOAT16)
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  else {
    const uint32_t u = __float_as_uint(v);
    return ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
}

template <int DT>
__device__ __forceinline__ void stv(void* p, long long i, float v) {
  if constexpr (DT == WGX_FLOAT32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = (uint16_t)to_bits<DT>(v);
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
    acc = apply_act(p.act, acc);
    if (p.has_clamp) acc = fminf(fmaxf(acc, p.cmin), p.cmax);
    const long long yi = ((long long)(plane0 + pp) * p.OH + oh0 + orow) * p.OW + ow;
    if (p.res) acc = p.rcs * acc + p.rrs * ldv<DT>(p.res, yi);
    stv<DT>(p.y, yi, acc);
  }
}

// ------------------------------------------------------------ fast family
// n / d for 0 <= n < 2^31 by a multiply-high and a shift (m, l from
// make_fastdiv: l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1).
struct FastDiv {
  uint32_t m, l;
};
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) { return (__umulhi(n, f.m) + n) >> f.l; }
FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const unsigned long long m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return {(uint32_t)m, l};
}

struct DwFast {
  const char* xa;    // x rounded down to 16 bytes
  uint32_t lead0;    // elements of xa before x
  unsigned long long x_end;  // bytes from xa to the end of x
  const void* w;
  const void* bias;
  void* y;
  int C, IH, IW, OH, OW;
  int multi;  // 1: blocks of whole planes; 0: bands of one plane
  int ppb, nplanes, toh, bands, segs;
  int LW, LR, PLANE;  // LDS tile: row pitch, rows and plane stride in floats
  FastDiv fd_plane;  // IH * IW
  FastDiv fd_iw;     // IW
  FastDiv fd_items;  // OH * segs (items of one whole plane)
  FastDiv fd_segs;   // segs
  int has_clamp;
  int act;
  float cmin, cmax;
  const void* res;  // residual (output-shaped) or null: y = rcs * y + rrs * res
  float rcs, rrs;
};

__device__ __forceinline__ void unpack(const uint4& v, float* f, std::integral_constant<int, WGX_FLOAT32>) {
  f[0] = __uint_as_float(v.x);
  f[1] = __uint_as_float(v.y);
  f[2] = __uint_as_float(v.z);
  f[3] = __uint_as_float(v.w);
}
__device__ __forceinline__ void unpack(const uint4& v, float* f, std::integral_constant<int, WGX_FLOAT16>) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xffffu));
    f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
  }
}
__device__ __forceinline__ void unpack(const uint4& v, float* f, std::integral_constant<int, WGX_BFLOAT16>) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

template <int DT, int K, int S, int OV>
__global__ __launch_bounds__(NT) void k_dw_fast(DwFast p) {
  constexpr int ES = DT == WGX_FLOAT32 ? 4 : 2;
  constexpr int EPC = 16 / ES;               // elements per 16-byte chunk
  constexpr int P = K / 2;                   // "same" padding
  constexpr int KK = K * K;
  constexpr int WST = (KK + 1 + 3) / 4 * 4;  // LDS floats per plane: taps, bias, pad
  constexpr int WN = (OV - 1) * S + K;       // input window of one kernel row
  constexpr int NW4 = (WN + 3) / 4;          // ... read as float4s
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x;

  int plane0, oh0, nloc, rows_here, rofs;
  uint32_t nq;             // input elements this block stages
  unsigned long long g0;   // first of them (flat index into x)
  if (p.multi) {
    plane0 = blockIdx.x * p.ppb;
    nloc = min(p.ppb, p.nplanes - plane0);
    oh0 = 0;
    rows_here = p.OH;
    rofs = P;  // LDS row of ih = 0
    g0 = (unsigned long long)plane0 * p.IH * p.IW;
    nq = (uint32_t)(nloc * p.IH * p.IW);
  } else {
    plane0 = blockIdx.x / p.bands;
    const int band = blockIdx.x - plane0 * p.bands;
    nloc = 1;
    oh0 = band * p.toh;
    rows_here = min(p.toh, p.OH - oh0);
    const int ih_lo = oh0 * S - P;
    const int r_s = max(ih_lo, 0), r_e = min(ih_lo + p.LR, p.IH);
    rofs = r_s - ih_lo;
    g0 = ((unsigned long long)plane0 * p.IH + r_s) * p.IW;
    nq = r_e > r_s ? (uint32_t)((r_e - r_s) * p.IW) : 0u;
  }
  const int rows_st = p.multi ? p.IH : 0;  // staged rows per plane (multi only)
  float* tile = lds;
  float* wl = lds + p.ppb * p.PLANE;

  // 1. zero the tile (its border is the zero padding); weights and bias
  {
    const int n4 = nloc * p.PLANE / 4;
    float4* t4 = reinterpret_cast<float4*>(tile);
    for (int i = tid; i < n4; i += NT) t4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = tid; i < nloc * WST; i += NT) {
      const int pp = i / WST, j = i - pp * WST;
      const int c = (plane0 + pp) % p.C;
      float v = 0.0f;
      if (j < KK) v = ldv<DT>(p.w, (long long)c * KK + j);
      else if (j == KK && p.bias) v = ldv<DT>(p.bias, c);
      wl[i] = v;
    }
  }
  __syncthreads();

  // 2. stage the input: 16-byte chunks of the flat range [g0, g0 + nq),
  //    chunk k of the block starts at byte cb0 + 16 k from xa
  if (nq > 0) {
    const unsigned long long byte_lo = (g0 + p.lead0) * ES;
    const unsigned long long cb0 = byte_lo & ~15ull;
    const uint32_t lead = (uint32_t)(byte_lo - cb0) / ES;  // elements before g0 in chunk 0
    const uint32_t nck = (uint32_t)((byte_lo + (unsigned long long)nq * ES - cb0 + 15) / 16);
    const unsigned long long left = p.x_end - cb0;
    const uint32_t rec = left > 0x7fffffffull ? 0x7fffffffu : (uint32_t)left;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p.xa + cb0), 0, (int)rec,
                                                                        0x00020000);
    const uint32_t plane_in = (uint32_t)(p.IH * p.IW);
    for (uint32_t base = 0; base < nck; base += 4 * NT) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t k = base + u * NT + tid;
        // whole chunks inside x: one vector load; the tail chunk of x (which
        // may end mid-chunk at the end of its allocation) goes element-wise
        if (k < nck && 16u * k + 16u <= rec) {
          const auto r = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(16u * k), 0, 0);
          v[u] = make_uint4(r[0], r[1], r[2], r[3]);
        } else if (k < nck) {
          uint32_t e[EPC];
#pragma unroll
          for (int j = 0; j < EPC; ++j) {
            const uint32_t off = 16u * k + ES * j;
            e[j] = off + ES <= rec ? (ES == 4 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0)
                                              : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0))
                                   : 0u;
          }
          if constexpr (ES == 4) v[u] = make_uint4(e[0], e[1], e[2], e[3]);
          else
            v[u] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t k = base + u * NT + tid;
        if (k >= nck) break;
        float f[EPC];
        unpack(v[u], f, std::integral_constant<int, DT>{});
        const uint32_t j0 = k == 0 ? lead : 0u;
        const uint32_t q0 = k * EPC + j0 - lead;  // first element of the chunk inside the range
        uint32_t pp = p.multi ? fdiv(q0, p.fd_plane) : 0u;
        const uint32_t rem = q0 - pp * plane_in;
        uint32_t r = fdiv(rem, p.fd_iw);
        uint32_t col = rem - r * p.IW;
        uint32_t li = pp * p.PLANE + (r + rofs) * p.LW + P + col;
        if (j0 == 0 && q0 + EPC <= nq && col + EPC <= (uint32_t)p.IW) {
#pragma unroll
          for (int j = 0; j < EPC; ++j) tile[li + j] = f[j];
        } else {
#pragma unroll
          for (int j = 0; j < EPC; ++j) {
            const uint32_t q = q0 + (uint32_t)j - j0;
            if ((uint32_t)j >= j0 && q < nq) {
              tile[li] = f[j];
              ++li;
              if (++col == (uint32_t)p.IW) {
                col = 0;
                li += p.LW - p.IW;
                if (++r == (uint32_t)rows_st) {  // next plane (whole-plane blocks)
                  r = 0;
                  li += p.PLANE - rows_st * p.LW;
                }
              }
            }
          }
        }
      }
    }
  }
  __syncthreads();

  // 3. outputs: item = (plane, output row, segment of OV columns) (one instantiation
  //    per clamp / residual: no per-output selects)
  auto outputs = [&]<bool CL, bool RS>() {
    const uint32_t items_pp = (uint32_t)(rows_here * p.segs);
    const uint32_t items = (uint32_t)nloc * items_pp;
    for (uint32_t i = tid; i < items; i += NT) {
      const uint32_t pp = p.multi ? fdiv(i, p.fd_items) : 0u;
      const uint32_t rem = i - pp * items_pp;
      const uint32_t orow = fdiv(rem, p.fd_segs);
      const int ow0 = (int)(rem - orow * p.segs) * OV;
      const float* src = tile + pp * p.PLANE + orow * S * p.LW + ow0 * S;
      const float* wp = wl + pp * WST;
      float wv[WST];
  #pragma unroll
      for (int q = 0; q < WST / 4; ++q) {
        const float4 t = reinterpret_cast<const float4*>(wp)[q];
        wv[4 * q] = t.x;
        wv[4 * q + 1] = t.y;
        wv[4 * q + 2] = t.z;
        wv[4 * q + 3] = t.w;
      }
      float acc[OV];
  #pragma unroll
      for (int o = 0; o < OV; ++o) acc[o] = wv[KK];
  #pragma unroll
      for (int kh = 0; kh < K; ++kh) {
        float win[NW4 * 4];
  #pragma unroll
        for (int q = 0; q < NW4; ++q) {
          const float4 t = reinterpret_cast<const float4*>(src + kh * p.LW)[q];
          win[4 * q] = t.x;
          win[4 * q + 1] = t.y;
          win[4 * q + 2] = t.z;
          win[4 * q + 3] = t.w;
        }
  #pragma unroll
        for (int kw = 0; kw < K; ++kw)
  #pragma unroll
          for (int o = 0; o < OV; ++o) acc[o] = fmaf(win[o * S + kw], wv[kh * K + kw], acc[o]);
      }
      const long long yo = ((long long)(plane0 + pp) * p.OH + oh0 + orow) * p.OW + ow0;
      uint32_t h[OV];
  #pragma unroll
      for (int o = 0; o < OV; ++o) {
        float v = acc[o];
        v = apply_act(p.act, v);
        if constexpr (CL) v = fminf(fmaxf(v, p.cmin), p.cmax);
        if (RS && ow0 + o < p.OW) v = p.rcs * v + p.rrs * ldv<DT>(p.res, yo + o);
        h[o] = to_bits<DT>(v);
      }
      char* yp = static_cast<char*>(p.y) + yo * ES;
      const uintptr_t ya = reinterpret_cast<uintptr_t>(yp);
      if (ow0 + OV <= p.OW && (ya & 15) == 0 && (OV * ES) % 16 == 0) {
  #pragma unroll
        for (int q = 0; q < OV * ES / 16; ++q) {
          uint4 t;
          if constexpr (ES == 4) t = make_uint4(h[4 * q], h[4 * q + 1], h[4 * q + 2], h[4 * q + 3]);
          else
            t = make_uint4(h[8 * q] | (h[8 * q + 1] << 16), h[8 * q + 2] | (h[8 * q + 3] << 16),
                           h[8 * q + 4] | (h[8 * q + 5] << 16), h[8 * q + 6] | (h[8 * q + 7] << 16));
          using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
          __builtin_nontemporal_store(u32x4{t.x, t.y, t.z, t.w}, reinterpret_cast<u32x4*>(yp) + q);
        }
      } else if (ow0 + OV <= p.OW && (ya & 7) == 0 && OV * ES == 8) {
        uint2 t;
        if constexpr (ES == 4) t = make_uint2(h[0], h[1]);
        else t = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
        __builtin_nontemporal_store(u32x2{t.x, t.y}, reinterpret_cast<u32x2*>(yp));
      } else {
  #pragma unroll
        for (int o = 0; o < OV; ++o) {
          if (ow0 + o < p.OW) {
            if constexpr (ES == 4) reinterpret_cast<uint32_t*>(yp)[o] = h[o];
            else reinterpret_cast<uint16_t*>(yp)[o] = (uint16_t)h[o];
          }
        }
      }
    }
  };
  if (p.has_clamp) {
    if (p.res) outputs.template operator()<true, true>();
    else outputs.template operator()<true, false>();
  } else {
    if (p.res) outputs.template operator()<false, true>();
    else outputs.template operator()<false, false>();
  }
}

// ------------------------------------------------------------ register family
// fp16, K x K, stride S, same padding, even widths: no LDS tile at all.  One
// wave owns a band of R output rows of pw planes; lane (plane slot, segment)
// owns OV consecutive output columns of its plane.  The lane reads its own
// S*OV-column chunk of every input row the band needs (all rows issued up
// front: (R-1)*S + K loads in flight per lane), takes the halo columns on
// either side from the neighbouring lanes' chunks (ds_bpermute; the image
// border is zero), and accumulates each input row into the up-to-ceil(K/S)
// output rows it feeds.  Rows above or below the image are loads at an
// out-of-range offset, which read as zero.
//
// The input stays packed (two halves per dword) from load to multiply: a tap
// pair whose first element sits at an even window position is one
// v_dot2_f32_f16 against the packed weight pair, a tap left over is one
// v_fma_mix_f32 on its half of the dword.  Both accumulate in fp32, and the
// taps of a row are added in kw order (bias, then kh-outer / kw-inner).
struct DwReg {
  const char* x;
  uint16_t* y;
  const uint16_t* w;
  const uint16_t* bias;
  int C, IH, IW, OH, OW;
  int segs, pw, bands, nplanes;
  long long units;
  unsigned long long x_bytes, y_bytes;
  int has_clamp;
  int act;
  float cmin, cmax;
  const void* res;  // residual (output-shaped) or null: y = rcs * y + rrs * res
  float rcs, rrs;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
// Cache policy of this kernel's output stores: default.  One store
// instruction writes pw short row pieces in different planes; with the
// non-temporal bit these partial lines bypass L2 write-combining and the
// kernel runs at less than half the speed (measured on MI355X), whereas the
// LDS-tiled kernel, whose lanes write one contiguous run, gains from it.
constexpr int kStoreNT = 0;
__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
__device__ __forceinline__ float lo_f(uint32_t d) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(d & 0xffffu)); }
__device__ __forceinline__ float hi_f(uint32_t d) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(d >> 16)); }
__device__ __forceinline__ float dot2(uint32_t x, uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, x), __builtin_bit_cast(half2_t, w), acc, false);
}
__device__ __forceinline__ uint32_t lane_from(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}

template <int K, int S, int OV, int R>
__global__ __launch_bounds__(64) void k_dw_reg(DwReg p) {
  constexpr int P = K / 2;
  constexpr int CW = S * OV;           // own chunk: input columns [S*ow0, S*ow0 + CW)
  constexpr int CD = CW / 2;           // ... as dwords
  constexpr int HLP = (P + 1) & ~1;    // left halo columns, rounded up to whole dwords
  constexpr int LD = HLP / 2;          // window dwords left of the own chunk
  constexpr int MAXE = (OV - 1) * S + HLP - P + K - 1;  // last window column a tap reads
  constexpr int WD = MAXE / 2 + 1;     // window dwords
  constexpr int RD = WD - LD - CD;     // window dwords right of the own chunk
  constexpr int NR = (R - 1) * S + K;  // input rows of the band
  constexpr int NP = (K - 1) / 2;      // tap pairs per kernel row
  static_assert(LD <= CD && RD <= CD && CD % 2 == 0, "window shape");
  using rsrc_t = __amdgpu_buffer_rsrc_t;
  constexpr uint32_t OOB = 0x80000000u;

  // Blocks are dealt to the 8 XCDs round-robin; renumber them so each XCD
  // runs a contiguous run of units, i.e. all bands of a plane group on one
  // XCD at about the same time: the halo rows a band shares with its
  // neighbours are then L2 hits instead of second HBM reads.
  const long long G = p.units, b = blockIdx.x;
  long long unit = b;
  if (G >= 8) {
    const long long xcd = b & 7, base = G >> 3, rem = G & 7;
    unit = xcd * base + (xcd < rem ? xcd : rem) + (b >> 3);
  }
  const int lane = threadIdx.x;
  const int pg = (int)(unit / p.bands), band = (int)(unit - (long long)pg * p.bands);
  const int ps = lane / p.segs, seg = lane - ps * p.segs;
  const int plane = pg * p.pw + ps;
  const bool active = ps < p.pw && plane < p.nplanes;
  const int oh0 = band * R;
  const int col0 = seg * CW;
  const int lim = p.IW - col0;  // valid input columns in the own chunk

  // this wave's planes as buffer ranges (offsets stay far below 2^31)
  const unsigned long long xb0 = (unsigned long long)pg * p.pw * p.IH * p.IW * 2;
  const unsigned long long yb0 = (unsigned long long)pg * p.pw * p.OH * p.OW * 2;
  const unsigned long long xl = p.x_bytes - xb0, yl = p.y_bytes - yb0;
  const rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p.x) + xb0, 0,
                                                      (int)(xl > 0x7fffffffull ? 0x7fffffffull : xl), 0x00020000);
  const rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<char*>(p.y) + yb0, 0,
                                                      (int)(yl > 0x7fffffffull ? 0x7fffffffull : yl), 0x00020000);

  // 1. every input row of the band: one (or two) vector loads per row; the
  //    last segment of a row that ends mid-chunk loads only its valid dwords.
  //    When the width is a multiple of 4 columns every lane loads 8-byte
  //    pieces (a piece past the row end at an out-of-range offset, which
  //    reads zero): the whole wave takes one path instead of the vector path
  //    and the element path one after the other ([256,512,20,20] 5x5 s2:
  //    60.8 -> 52.1 us).
  uint32_t raw[NR][CD];
  const bool pieces = (p.IW % CW) != 0 && (p.IW & 3) == 0;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int ih = oh0 * S - P + j;
    const bool rok = active && ih >= 0 && ih < p.IH;
    const uint32_t off = (uint32_t)(((ps * p.IH + ih) * p.IW + col0) * 2);
    if (pieces) {
#pragma unroll
      for (int q = 0; q < CD; q += 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rx, (int)(rok && 2 * q < lim ? off + 4 * q : OOB), 0, 0);
        raw[j][q] = v[0];
        raw[j][q + 1] = v[1];
      }
    } else if (lim >= CW) {
#pragma unroll
      for (int q = 0; q + 4 <= CD; q += 4) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(rok ? off + 4 * q : OOB), 0, 0);
        raw[j][q] = v[0];
        raw[j][q + 1] = v[1];
        raw[j][q + 2] = v[2];
        raw[j][q + 3] = v[3];
      }
      if constexpr (CD % 4 == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rx, (int)(rok ? off + 4 * (CD - 2) : OOB), 0, 0);
        raw[j][CD - 2] = v[0];
        raw[j][CD - 1] = v[1];
      }
    } else {
#pragma unroll
      for (int d = 0; d < CD; ++d)
        raw[j][d] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rx, (int)(rok && 2 * d < lim ? off + 4 * d : OOB), 0, 0);
    }
  }

  // 1b. the residual's output rows (the same offsets as the stores below),
  //     issued now so their latency hides under the stencil
  constexpr int OD = OV / 2;
  uint32_t rres[R][OD];
  const int nvalid = active ? min(OV, p.OW - seg * OV) : 0;
  if (p.res) {
    const rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(static_cast<const char*>(p.res)) + yb0, 0,
                                                        (int)(yl > 0x7fffffffull ? 0x7fffffffull : yl), 0x00020000);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int oh = oh0 + r;
      const uint32_t off = (uint32_t)(((ps * p.OH + oh) * p.OW + seg * OV) * 2);
      const bool rok = oh < p.OH;
      if (nvalid == OV) {
        if constexpr (OV == 8) {
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(rr, (int)(rok ? off : OOB), 0, 0);
#pragma unroll
          for (int d = 0; d < 4; ++d) rres[r][d] = v[d];
        } else {
          const auto v = __builtin_amdgcn_raw_buffer_load_b64(rr, (int)(rok ? off : OOB), 0, 0);
          rres[r][0] = v[0];
          rres[r][1] = v[1];
        }
      } else {
#pragma unroll
        for (int d = 0; d < OD; ++d) {
          const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rr, (int)(rok && 2 * d < nvalid ? off + 4 * d : OOB), 0, 0);
          const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rr, (int)(rok && 2 * d + 1 < nvalid ? off + 4 * d + 2 : OOB), 0, 0);
          rres[r][d] = lo | (hi << 16);
        }
      }
    }
  }

  // 2. weights of this lane's plane: packed pairs (w[kw], w[kw+1]) starting at
  //    even and at odd kw, and the two taps that can be left over, in fp32
  uint32_t wpe[K][NP], wpo[K][NP];
  float wfirst[K], wlast[K], bias = 0.0f;
  {
    const int c = active ? plane % p.C : 0;
    uint32_t wr[K * K];
#pragma unroll
    for (int t = 0; t < K * K; ++t) wr[t] = p.w[c * K * K + t];
#pragma unroll
    for (int kh = 0; kh < K; ++kh) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        wpe[kh][q] = wr[kh * K + 2 * q] | (wr[kh * K + 2 * q + 1] << 16);
        wpo[kh][q] = wr[kh * K + 2 * q + 1] | (wr[kh * K + 2 * q + 2] << 16);
      }
      wfirst[kh] = h2f(wr[kh * K]);
      wlast[kh] = h2f(wr[kh * K + K - 1]);
    }
    if (p.bias) bias = h2f(p.bias[c]);
  }
  float acc[R][OV];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int o = 0; o < OV; ++o) acc[r][o] = bias;

  // 3. rows in order; window dword i holds input columns col0 - HLP + 2i, +1
  const bool has_left = seg > 0, has_right = seg + 1 < p.segs;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    uint32_t win[WD];
#pragma unroll
    for (int d = 0; d < CD; ++d) win[LD + d] = raw[j][d];
#pragma unroll
    for (int h = 0; h < LD; ++h) {
      const uint32_t v = lane_from(raw[j][CD - LD + h], lane - 1);
      win[h] = has_left ? v : 0u;
    }
#pragma unroll
    for (int h = 0; h < RD; ++h) {
      const uint32_t v = lane_from(raw[j][h], lane + 1);
      win[LD + CD + h] = has_right ? v : 0u;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int kh = j - r * S;  // compile-time after unrolling
      if (kh >= 0 && kh < K) {
#pragma unroll
        for (int o = 0; o < OV; ++o) {
          const int e0 = HLP + o * S - P;  // window column of tap kw = 0
          float a = acc[r][o];
          if ((e0 & 1) == 0) {
#pragma unroll
            for (int q = 0; q < NP; ++q) a = dot2(win[e0 / 2 + q], wpe[kh][q], a);
            a = fmaf(lo_f(win[(e0 + K - 1) / 2]), wlast[kh], a);
          } else {
            a = fmaf(hi_f(win[(e0 - 1) / 2]), wfirst[kh], a);
#pragma unroll
            for (int q = 0; q < NP; ++q) a = dot2(win[(e0 + 1) / 2 + q], wpo[kh][q], a);
          }
          acc[r][o] = a;
        }
      }
    }
  }

  // 4. stores: OV halves per output row, one vector store when whole (one
  //    instantiation per clamp / residual: no per-output selects)
  if (!active) return;
  auto stores = [&]<bool CL, bool RS>() {
  #pragma unroll
    for (int r = 0; r < R; ++r) {
      const int oh = oh0 + r;
      if (oh >= p.OH) break;
      uint32_t h[OV];
  #pragma unroll
      for (int o = 0; o < OV; ++o) {
        float v = acc[r][o];
        v = apply_act(p.act, v);
        if constexpr (CL) v = fminf(fmaxf(v, p.cmin), p.cmax);
        if constexpr (RS) v = p.rcs * v + p.rrs * ((o & 1) ? hi_f(rres[r][o / 2]) : lo_f(rres[r][o / 2]));
        h[o] = __builtin_bit_cast(uint16_t, (_Float16)v);
      }
      const uint32_t off = (uint32_t)(((ps * p.OH + oh) * p.OW + seg * OV) * 2);
      if (nvalid == OV) {
        if constexpr (OV == 8) {
          using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
          const u32x4 v = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
          __builtin_amdgcn_raw_buffer_store_b128(v, ry, (int)off, 0, kStoreNT);
        } else {
          using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
          const u32x2 v = {h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
          __builtin_amdgcn_raw_buffer_store_b64(v, ry, (int)off, 0, kStoreNT);
        }
      } else {
  #pragma unroll
        for (int o = 0; o < OV; ++o)
          if (o < nvalid) __builtin_amdgcn_raw_buffer_store_b16((unsigned short)h[o], ry, (int)(off + 2 * o), 0, kStoreNT);
      }
    }
  };
  if (p.has_clamp) {
    if (p.res) stores.template operator()<true, true>();
    else stores.template operator()<true, false>();
  } else {
    if (p.res) stores.template operator()<false, true>();
    else stores.template operator()<false, false>();
  }
}

// Plans the register kernel; false when d is outside its family.
bool plan_reg(const DwDesc& d, DwReg& p, int& ov, int& R, long long& blocks) {
  const int K = d.KH;
  if (d.dtype != WGX_FLOAT16 || d.KW != K || (K != 3 && K != 5) || d.sH != d.sW || (d.sH != 1 && d.sH != 2) ||
      d.pH != K / 2 || d.pW != K / 2 || d.dH != 1 || d.dW != 1)
    return false;
  if ((d.IW & 1) || (d.OW & 1) || (reinterpret_cast<uintptr_t>(d.x) & 3) || (reinterpret_cast<uintptr_t>(d.y) & 3) ||
      (reinterpret_cast<uintptr_t>(d.res) & 3) ||
      (d.w && (reinterpret_cast<uintptr_t>(d.w) & 1)))
    return false;
  const int S = d.sH;
  ov = ((d.OW + 3) / 4 * 4 < (d.OW + 7) / 8 * 8) ? 4 : 8;
  if (S == 2 && K == 5 && ov == 8) ov = 4;  // keeps the row window in registers
  const int segs = (d.OW + ov - 1) / ov;
  if (segs > 64) return false;
  const long long nplanes = (long long)d.B * d.C;
  p.segs = segs;
  p.pw = 64 / segs;
  const long long groups = (nplanes + p.pw - 1) / p.pw;
  // Band height: the fewest dead rows in the last band, ties to the taller
  // band (fewer halo rows read twice); 4 when the grid would leave CUs idle.
  R = 4;
  if (groups * ((d.OH + 7) / 8) >= 2048) {
    int best = 1 << 30;
    for (int r : {8, 5, 4}) {
      const int rows = (d.OH + r - 1) / r * r;  // output rows computed, dead ones included
      if (rows < best) {
        best = rows;
        R = r;
      }
    }
  }
  p.bands = (d.OH + R - 1) / R;
  p.units = groups * p.bands;
  // a wave's planes must stay addressable with 31-bit buffer offsets
  if ((long long)p.pw * d.IH * d.IW * 2 >= (1LL << 30) || p.units >= (1LL << 31)) return false;
  p.x = static_cast<const char*>(d.x);
  p.y = static_cast<uint16_t*>(d.y);
  p.w = static_cast<const uint16_t*>(d.w);
  p.bias = static_cast<const uint16_t*>(d.bias);
  p.C = d.C;
  p.IH = d.IH;
  p.IW = d.IW;
  p.OH = d.OH;
  p.OW = d.OW;
  p.nplanes = (int)nplanes;
  p.x_bytes = (unsigned long long)nplanes * d.IH * d.IW * 2;
  p.y_bytes = (unsigned long long)nplanes * d.OH * d.OW * 2;
  p.has_clamp = d.has_clamp;
  p.act = d.act;
  p.cmin = d.cmin;
  p.cmax = d.cmax;
  p.res = d.res;
  p.rcs = d.res_conv_scale;
  p.rrs = d.res_scale;
  blocks = p.units;
  return true;
}

template <int K, int S, int OV, int R>
hipError_t launch_reg(const DwReg& p, long long blocks, hipStream_t s, std::string* name) {
  if (name) {
    char buf[64];
    snprintf(buf, sizeof buf, "depthwise_f16_%dx%ds%d_r%dv%d", K, K, S, R, OV);
    *name = buf;
  }
  if (is_dry(s)) return hipSuccess;
  hipLaunchKernelGGL((k_dw_reg<K, S, OV, R>), dim3((unsigned)blocks), dim3(64), 0, s, p);
  return hipGetLastError();
}

template <int K, int S, int OV>
hipError_t launch_reg_r(const DwReg& p, int R, long long blocks, hipStream_t s, std::string* name) {
  if (R == 8) return launch_reg<K, S, OV, 8>(p, blocks, s, name);
  if (R == 5) return launch_reg<K, S, OV, 5>(p, blocks, s, name);
  return launch_reg<K, S, OV, 4>(p, blocks, s, name);
}

hipError_t launch_reg_any(const DwReg& p, int K, int S, int ov, int R, long long blocks, hipStream_t s,
                          std::string* name) {
  if (K == 3 && S == 1) return ov == 8 ? launch_reg_r<3, 1, 8>(p, R, blocks, s, name) : launch_reg_r<3, 1, 4>(p, R, blocks, s, name);
  if (K == 3 && S == 2) return ov == 8 ? launch_reg_r<3, 2, 8>(p, R, blocks, s, name) : launch_reg_r<3, 2, 4>(p, R, blocks, s, name);
  if (K == 5 && S == 1) return ov == 8 ? launch_reg_r<5, 1, 8>(p, R, blocks, s, name) : launch_reg_r<5, 1, 4>(p, R, blocks, s, name);
  return launch_reg_r<5, 2, 4>(p, R, blocks, s, name);
}

constexpr int kFastLds = 40 * 1024;  // LDS budget of one block (4 blocks per CU)

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

template <int DT, int K, int S, int OV>
hipError_t launch_fast(const DwFast& p, int blocks, size_t lds, hipStream_t s, std::string* name) {
  if (name) {
    char buf[64];
    snprintf(buf, sizeof buf, "depthwise_%s_%dx%ds%d_v%d", DT == WGX_FLOAT32 ? "f32" : DT == WGX_FLOAT16 ? "f16" : "bf16",
             K, K, S, OV);
    *name = buf;
  }
  if (is_dry(s)) return hipSuccess;
  hipLaunchKernelGGL((k_dw_fast<DT, K, S, OV>), dim3(blocks), dim3(NT), lds, s, p);
  return hipGetLastError();
}

template <int DT, int K, int S>
hipError_t launch_fast_ov(const DwFast& p, int ov, int blocks, size_t lds, hipStream_t s, std::string* name) {
  return ov == 8 ? launch_fast<DT, K, S, 8>(p, blocks, lds, s, name) : launch_fast<DT, K, S, 4>(p, blocks, lds, s, name);
}

template <int DT>
hipError_t launch_fast_dt(const DwFast& p, int K, int S, int ov, int blocks, size_t lds, hipStream_t s,
                          std::string* name) {
  if (K == 3) return S == 1 ? launch_fast_ov<DT, 3, 1>(p, ov, blocks, lds, s, name)
                            : launch_fast_ov<DT, 3, 2>(p, ov, blocks, lds, s, name);
  return S == 1 ? launch_fast_ov<DT, 5, 1>(p, ov, blocks, lds, s, name)
                : launch_fast_ov<DT, 5, 2>(p, ov, blocks, lds, s, name);
}

// Plans the fast kernel for d; false when the shape is outside its family or
// its LDS tile does not fit.
bool plan_fast(const DwDesc& d, DwFast& p, int& ov, int& blocks, size_t& lds) {
  const int K = d.KH;
  if (d.KW != K || (K != 3 && K != 5) || d.sH != d.sW || (d.sH != 1 && d.sH != 2) || d.pH != K / 2 ||
      d.pW != K / 2 || d.dH != 1 || d.dW != 1)
    return false;
  const int S = d.sH, P = K / 2;
  const int es = d.dtype == WGX_FLOAT32 ? 4 : 2;
  // output segment per lane: 8, or 4 where that wastes fewer lanes on the row end
  ov = ((d.OW + 3) / 4 * 4 < (d.OW + 7) / 8 * 8) ? 4 : 8;
  const int segs = (d.OW + ov - 1) / ov;
  const int nw4 = ((ov - 1) * S + K + 3) / 4;
  const int wst = (K * K + 1 + 3) / 4 * 4;
  int LW = (segs - 1) * ov * S + 4 * nw4;
  if (LW < P + d.IW) LW = P + d.IW;
  LW = (LW + 3) / 4 * 4;
  const long long nplanes = (long long)d.B * d.C;
  const long long lr_full = std::max((long long)(d.OH - 1) * S + K, (long long)d.IH + P);
  const long long plane_bytes = lr_full * LW * 4 + wst * 4;
  p.multi = plane_bytes <= kFastLds;
  if (p.multi) {
    int ppb = (768 + d.OH * segs - 1) / (d.OH * segs);
    ppb = std::min<long long>(ppb, kFastLds / plane_bytes);
    ppb = std::min<long long>(ppb, std::max<long long>(1, nplanes / 512));  // >= 2 blocks per CU
    p.ppb = std::max(ppb, 1);
    p.toh = d.OH;
    p.bands = 1;
    p.LR = (int)lr_full;
    blocks = (int)((nplanes + p.ppb - 1) / p.ppb);
  } else {
    p.ppb = 1;
    const int rows_fit = (kFastLds / 4 - wst) / LW;  // LDS rows of one band
    const int toh_lds = (rows_fit - K) / S + 1;
    if (rows_fit < K || toh_lds < 1) return false;
    int toh = std::min(d.OH, std::max(1, (1024 + segs - 1) / segs));
    toh = std::min(toh, toh_lds);
    p.toh = toh;
    p.bands = (d.OH + toh - 1) / toh;
    p.LR = (toh - 1) * S + K;
    if (nplanes * p.bands > INT32_MAX) return false;
    blocks = (int)(nplanes * p.bands);
  }
  p.PLANE = p.LR * LW;
  p.LW = LW;
  p.segs = segs;
  p.nplanes = (int)nplanes;
  lds = ((size_t)p.ppb * p.PLANE + (size_t)p.ppb * wst) * 4;
  if (lds > 64 * 1024) return false;
  const uintptr_t xv = reinterpret_cast<uintptr_t>(d.x);
  p.xa = reinterpret_cast<const char*>(xv & ~uintptr_t(15));
  p.lead0 = (uint32_t)((xv & 15) / es);
  p.x_end = (xv & 15) + (unsigned long long)nplanes * d.IH * d.IW * es;
  p.w = d.w;
  p.bias = d.bias;
  p.y = d.y;
  p.C = d.C;
  p.IH = d.IH;
  p.IW = d.IW;
  p.OH = d.OH;
  p.OW = d.OW;
  p.fd_plane = make_fastdiv((uint32_t)(d.IH * d.IW));
  p.fd_iw = make_fastdiv((uint32_t)d.IW);
  p.fd_items = make_fastdiv((uint32_t)(d.OH * segs));
  p.fd_segs = make_fastdiv((uint32_t)segs);
  p.has_clamp = d.has_clamp;
  p.act = d.act;
  p.cmin = d.cmin;
  p.cmax = d.cmax;
  p.res = d.res;
  p.rcs = d.res_conv_scale;
  p.rrs = d.res_scale;
  return (long long)p.ppb * d.IH * d.IW < (1LL << 30);
}

int dw_device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

}  // namespace

hipError_t launch_depthwise(const DwDesc& d, hipStream_t s, std::string* name) {
  {
    DwFast f;
    int ov = 8, blocks = 0;
    size_t lds = 0;
    // WGX_DW_KERNEL=reg|lds|generic narrows the choice (A/B timing of the
    // variants, and tests of the register kernel on small shapes); a kernel
    // that does not apply falls through to the next one
    const char* only = getenv("WGX_DW_KERNEL");
    const bool force_reg = only && only[0] == 'r';
    const bool allow_reg = !only || force_reg, allow_lds = !only || force_reg || only[0] == 'l';
    DwReg rp;
    int rov = 8, R = 4;
    long long rblocks = 0;
    // The register kernel runs one wave per unit: with fewer units than two
    // per CU on small planes (batch-1 maps of at most 40 columns) the
    // LDS-tiled kernel's 256-lane blocks fill the chip better (measured on
    // MI355X: [1,256,40,40] 3x3 4.1 vs 4.7 us, [1,512,20,20] 5x5 s2 4.4 vs
    // 5.6 us, [1,64,40,40] 3x3 3.9 vs 4.8 us); on large planes it loses
    // ([1,16,160,160] 8.5 vs 5.0 us), and at batch 256 the register kernel
    // is ahead on both configurations (107 vs 123 us, 56 vs 78 us).
    const bool reg_ok = allow_reg && plan_reg(d, rp, rov, R, rblocks);
    const bool fast_ok = allow_lds && plan_fast(d, f, ov, blocks, lds);
    if (reg_ok && (force_reg || !fast_ok || d.OW > 40 || rblocks >= 2LL * dw_device_cus()))
      return launch_reg_any(rp, d.KH, d.sH, rov, R, rblocks, s, name);
    if (fast_ok) {
      const int K = d.KH, S = d.sH;
      if (d.dtype == WGX_FLOAT16) return launch_fast_dt<WGX_FLOAT16>(f, K, S, ov, blocks, lds, s, name);
      if (d.dtype == WGX_BFLOAT16) return launch_fast_dt<WGX_BFLOAT16>(f, K, S, ov, blocks, lds, s, name);
      return launch_fast_dt<WGX_FLOAT32>(f, K, S, ov, blocks, lds, s, name);
    }
  }
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
  p.act = d.act;
  p.cmin = d.cmin;
  p.cmax = d.cmax;
  p.res = d.res;
  p.rcs = d.res_conv_scale;
  p.rrs = d.res_scale;
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
