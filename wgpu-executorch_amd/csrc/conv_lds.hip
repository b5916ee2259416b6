// conv_lds.hip -- dense KxK convolution (groups 1, dilation 1, input channels
// a multiple of 8 for float32, 16 for 16-bit data) as an implicit GEMM on the
// gfx950 matrix cores, with each
// wave's input patch in LDS and no per-element address arithmetic.
//
// Serves the dense branch of aten.convolution / et_vk.conv_with_clamp
// (src/shaders/convolution/index.ts:168-238: the tile64 / tile32 / gemm
// implicit-im2col variants; conv-with-clamp/index.ts:60-319) for float16,
// bfloat16 and float32 NCHW tensors with OIHW weights:
//   y[b,oc,oh,ow] = bias[oc] + sum_{ic,kh,kw} w[oc,ic,kh,kw] * x[b,ic,oh*s-p+kh,ow*s-p+kw]
// (zero outside the image), fp32 accumulation, then SiLU / clamp, one rounding.
//
// GEMM view: M = OC (the A operand, weight rows), N = output pixels (B, the
// im2col columns), K = IC*KH*KW.  Each wave owns TM x TN MFMA tiles of 32 x 32:
// TM*32 output channels by a region of 4*TN x 8 output pixels (each 32-pixel
// MFMA column block is a 4 x 8 rectangle, so a region's input footprint is a
// small 2-D patch rather than a row strip).
//
// K is walked in chunks of 2*CPL input channels (CPL = 8 for 16-bit data, 4
// for float32).  Within a chunk the K order is arranged so that both operands
// need no address work:
//   * lanes 0-31 take the chunk's first CPL channels and lanes 32-63 the
//     next CPL; each lane half walks its CPL channels x T taps (T = KH*KW) in
//     the natural (ic, kh, kw) order, 16 bytes at a time;
//   * A: those CPL*T k of a weight row are contiguous in OIHW memory, so every
//     A fragment is ONE 16-byte buffer load at a loop-invariant lane offset
//     plus a compile-time step offset;
//   * B: the chunk's input patch (2*CPL channels x PH x PW, zero outside the
//     image) sits in the wave's own LDS; the element a lane needs for k =
//     (channel, kh, kw) of its output pixel is at
//         pixel_base(lane) + (channel * PH * PW + kh * PW + kw) * ES
//     where the second term is a compile-time constant per (step, element):
//     one ds_read with an immediate offset per element.
// Both operands see the same k order, so the GEMM computes the convolution.
// The patch of the next chunk is loaded (lane-strided, one buffer load per
// element at precomputed lane offsets, the chunk selected by the descriptor
// base) while the current chunk is multiplied.  Each wave has its own patch,
// so the K loop has no barrier.
//
// Few output tiles (batch-1 maps): the W waves of a block share one tile and
// take chunks w, w+W, ...; their partial sums meet in LDS and are added in
// wave order (fixed, so the result does not depend on timing).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "internal.h"

namespace wgx {
namespace {

using f32x16 = float __attribute__((ext_vector_type(16)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr uint32_t OOB = 0x80000000u;

__device__ __forceinline__ rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
// The scalar offset (soff) is added to the lane's offset by the load itself:
// per-element constants cost no vector instruction.
__device__ __forceinline__ uint4 ld16(rsrc_t r, uint32_t off, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
template <int ES>
__device__ __forceinline__ uint32_t ld_el(rsrc_t r, uint32_t off, uint32_t soff) {
  if constexpr (ES == 4) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, 0);
  else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, (int)soff, 0);
}

struct CParams {
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int IC, IH, IW, OC, OH, OW, pH, pW;
  long long sx, sy;  // elements per input / output image
  int tiles_m, tiles_w, tiles_h, ntiles;
  int nchunks;  // IC / 16
  int W;        // waves per block sharing one tile
  int act, has_clamp;
  float cmin, cmax;
  const void* res;  // output-shaped residual or null: y = rcs * y + rrs * res
  float rcs, rrs;
  // waves of a block that share one input patch, each on its own output-
  // channel tile of the same pixels (the channel-last kernel on pre-ordered
  // weights with row segments; 1 otherwise)
  int share;
};

template <int DT>
__device__ __forceinline__ f32x16 mma(uint4 b, uint4 a, f32x16 c) {
  if constexpr (DT == WGX_FLOAT32) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.x), __uint_as_float(a.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.y), __uint_as_float(a.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.z), __uint_as_float(a.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.w), __uint_as_float(a.w), c, 0, 0, 0);
    return c;
  } else if constexpr (DT == WGX_BFLOAT16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b), __builtin_bit_cast(bf16x8, a),
                                                   c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, b), __builtin_bit_cast(f16x8, a), c,
                                                  0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ float to_f(uint32_t h) {
  if constexpr (DT == WGX_FLOAT32) return __uint_as_float(h);
  else if constexpr (DT == WGX_BFLOAT16) return __uint_as_float(h << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT>
__device__ __forceinline__ uint32_t from_f(float v) {
  if constexpr (DT == WGX_FLOAT32) return __float_as_uint(v);
  else if constexpr (DT == WGX_BFLOAT16) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  } else {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

// Geometry of one wave's region and its patch.  In LDS a channel's patch
// plane (PH x PW, row-major) is padded to whole blocks of 64 elements: patch
// element (channel, block, lane) sits at (channel * PHWP + block * 64 + lane),
// so each lane's load targets for every channel differ only by constants.
template <int DT, int KH, int KW, int S, int TN, bool RV = false>
struct Geo {
  static constexpr int ES = DT == WGX_FLOAT32 ? 4 : 2;
  static constexpr int EPC = 16 / ES;            // k per lane per 16-byte fragment
  static constexpr int T = KH * KW;
  // channels per lane half (a chunk is 2*CPL channels): 4 for float32, whose
  // fragments hold 4 k, so a chunk is 8 channels and a wave of a batch-1
  // launch gets more of them to pipeline; 8 for 16-bit data
  static constexpr int CPL = ES == 4 ? 4 : 8;
  static constexpr int STEPS = CPL * T / EPC;    // fragments per chunk per lane half
  static constexpr int RH = 4 * TN, RW = 8;      // output pixels of the region
  static constexpr int PH = (RH - 1) * S + KH;   // input rows / columns it reads
  static constexpr int PW = (RW - 1) * S + KW;
  static constexpr int PHW = PH * PW;
  static constexpr int NBLK = (PHW + 63) / 64;   // 64-element blocks per channel plane
  // Row-segment form (RV: float32, image width a multiple of 4): the patch is
  // loaded as 16-byte row segments on the image's 4-column grid, so a row
  // holds PWR >= PW + 3 columns (the region's first column sits 0-3 columns
  // into it); NRS segments per channel, NPASS passes of 64 lanes.
  static constexpr int PWR = (PW + 3 + 3) / 4 * 4;
  static constexpr int NSEG = PWR / 4;
  static constexpr int NRS = PH * NSEG;
  static constexpr int NPASS = (NRS + 63) / 64;
  static constexpr int PHWP = RV ? PH * PWR : NBLK * 64;  // a channel's plane in LDS (elements)
  static constexpr int ROWP = RV ? PWR : PW;              // its row pitch
  static constexpr int LDS_WAVE = 2 * CPL * PHWP * ES;  // bytes of a wave's patch
  // A fragments kept in flight ahead of the one being multiplied
  static constexpr int PF = ES == 4 ? STEPS / 3 : STEPS;
  static_assert(STEPS % PF == 0, "the prefetch ring wraps at chunk ends");
  // Interleaved lane halves (the weight loads): element e of fragment s in
  // lane half h is chunk k = 2*EPC*s + EPC*h + e (channel k / T, tap k % T),
  // so the two halves of a fragment are neighbouring 16-byte pieces of one
  // weight row, which the address unit takes as one run.  koff(k): LDS byte
  // offset of chunk k from the lane's pixel base; the upper half adds
  // dhalf(t) to the lower half's koff for a lower-half tap t (the same for
  // every channel).
  static constexpr int koff(int k) {
    const int ch = k / T, tap = k % T;
    return (ch * PHWP + (tap / KW) * ROWP + (tap % KW)) * ES;
  }
  static constexpr int dhalf(int t) { return koff(t + EPC) - koff(t); }
};

// Epilogue shared by the convolution kernels: acc[i][j][4g + e] is output
// channel m0 + i*32 + (lane % 32), region row 4j + g, region column
// 4*(lane / 32) + e.  With W > 1 waves per block the partial sums of the
// block's waves meet in LDS and are added in wave order, then bias,
// activation and clamp, one rounding, 8- or 16-byte stores.
// CL / RS: the launch clamps / adds a residual (one instantiation each, so
// the per-element code carries no selects for what the launch does not do).
template <int DT, int TM, int TN, bool CL, bool RS, int CW>
__device__ __forceinline__ void conv_epilogue_t(const CParams& p, f32x16 (&acc)[TM][TN], char* lds, int W, int wave,
                                                int lane, int m0, int oh0, int ow0, int z, const float (&brow)[TM]) {
  constexpr int ES = DT == WGX_FLOAT32 ? 4 : 2;
  constexpr int NG = TM * TN * 4;
  const int fr = lane & 31, fc = lane >> 5;
  float* part = reinterpret_cast<float*>(lds);
  if (W > 1) {
    __syncthreads();  // every wave is done with its patch
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          reinterpret_cast<float4*>(part)[(wave * NG + (i * TN + j) * 4 + g) * 64 + lane] =
              make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
    __syncthreads();
  }
  char* yimg = static_cast<char*>(p.y) + (long long)z * p.sy * ES;
  static_assert(ES == 2 || CW == 8, "float32 regions are 8 columns wide");
  if constexpr (ES == 2) {
    // 16-bit: lane (fr, fc) holds pixels 8g + 4fc .. 8g + 4fc + 3 of the
    // 32-pixel block (groups g = 2gp and 2gp + 1) of output channel fr;
    // v_permlane32_swap trades the upper half-wave's group 2gp for the lower
    // half-wave's group 2gp + 1, so lane fr then holds all 8 pixels of group
    // 2gp and lane fr + 32 those of group 2gp + 1, and each lane writes one
    // 16-byte piece (CW = 8: rows 2gp and 2gp + 1; CW = 16: the two halves of
    // one 32-byte row, which the address unit merges)
    const bool vec8 = (p.OW & 7) == 0 && ((reinterpret_cast<uintptr_t>(p.y) | reinterpret_cast<uintptr_t>(p.res)) & 15) == 0;
    const bool vec4 = (p.OW & 3) == 0;
    auto store_rows = [&](int i, int j, int gp, const float4& a, const float4& b) {
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
      float v[8];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(av[d]), __float_as_uint(bv[d]), false, false);
        v[d] = __uint_as_float(r[0]);
        v[4 + d] = __uint_as_float(r[1]);
      }
      constexpr int RB = 32 / CW;
      const int px = 8 * (2 * gp + fc);  // the group's first pixel in the block
      const int oc = m0 + i * 32 + fr, oh = oh0 + RB * j + px / CW, ow = ow0 + px % CW;
      if (oc >= p.OC || oh >= p.OH || ow >= p.OW) return;
      float bias = 0.0f;
#pragma unroll
      for (int ii = 0; ii < TM; ++ii)
        if (ii == i) bias = brow[ii];
      const long long eo = (long long)oc * p.OH * p.OW + (long long)oh * p.OW + ow;
      uint16_t* dst = reinterpret_cast<uint16_t*>(yimg) + eo;
      const bool full = ow + 7 < p.OW;
      // the residual's elements at the output's positions, read by the lane
      // that writes them (a residual that is the output itself is fine)
      uint32_t rr[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
      if constexpr (RS) {
        const uint16_t* rp = static_cast<const uint16_t*>(p.res) + (long long)z * p.sy + eo;
        if (vec8 && full) {
          const uint4 t = *reinterpret_cast<const uint4*>(rp);
          const uint32_t tw[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
          for (int d = 0; d < 4; ++d) rr[2 * d] = tw[d] & 0xffffu, rr[2 * d + 1] = tw[d] >> 16;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (ow + e < p.OW) rr[e] = rp[e];
        }
      }
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = apply_act(p.act, v[e] + bias);
        if constexpr (CL) x = fminf(fmaxf(x, p.cmin), p.cmax);
        if constexpr (RS) x = p.rcs * x + p.rrs * to_f<DT>(rr[e]);
        h[e] = from_f<DT>(x);
      }
      if (vec8 && full) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
      } else if (vec4) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        if (ow + 4 < p.OW) *reinterpret_cast<uint2*>(dst + 4) = make_uint2(h[4] | (h[5] << 16), h[6] | (h[7] << 16));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (ow + e < p.OW) dst[e] = (uint16_t)h[e];
      }
    };
    auto grp = [&](const f32x16& x, int g) { return make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]); };
    if (W == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int gp = 0; gp < 2; ++gp) store_rows(i, j, gp, grp(acc[i][j], 2 * gp), grp(acc[i][j], 2 * gp + 1));
    } else {
      auto sum = [&](int q) {
        float4 v = reinterpret_cast<const float4*>(part)[q * 64 + lane];
        for (int w = 1; w < W; ++w) {
          const float4 u = reinterpret_cast<const float4*>(part)[(w * NG + q) * 64 + lane];
          v.x += u.x;
          v.y += u.y;
          v.z += u.z;
          v.w += u.w;
        }
        return v;
      };
      // group pairs (2 qp, 2 qp + 1) over the waves
      for (int qp = wave; qp < NG / 2; qp += W) {
        const int i = qp / (TN * 2), j = (qp >> 1) % TN, gp = qp & 1;
        store_rows(i, j, gp, sum(2 * qp), sum(2 * qp + 1));
      }
    }
    return;
  }
  const bool vec = (p.OW & 3) == 0;
  auto store_group = [&](int q, float4 v) {
    const int i = q / (TN * 4), j = (q >> 2) % TN, g = q & 3;
    const int oc = m0 + i * 32 + fr, oh = oh0 + 4 * j + g, ow = ow0 + 4 * fc;
    if (oc >= p.OC || oh >= p.OH || ow >= p.OW) return;
    float bias = 0.0f;
#pragma unroll
    for (int ii = 0; ii < TM; ++ii)
      if (ii == i) bias = brow[ii];
    float vv[4] = {v.x + bias, v.y + bias, v.z + bias, v.w + bias};
    const long long eo = (long long)oc * p.OH * p.OW + (long long)oh * p.OW + ow;
    char* dst = yimg + eo * ES;
    // the residual's elements at the output's positions, read by the lane
    // that writes them (a residual that is the output itself is fine)
    uint32_t rr[4] = {0u, 0u, 0u, 0u};
    if constexpr (RS) {
      const char* rsrc_p = static_cast<const char*>(p.res) + ((long long)z * p.sy + eo) * ES;
      if (vec && ow + 3 < p.OW) {
        if constexpr (ES == 4) {
          const uint4 t = *reinterpret_cast<const uint4*>(rsrc_p);
          rr[0] = t.x, rr[1] = t.y, rr[2] = t.z, rr[3] = t.w;
        } else {
          const uint2 t = *reinterpret_cast<const uint2*>(rsrc_p);
          rr[0] = t.x & 0xffffu, rr[1] = t.x >> 16, rr[2] = t.y & 0xffffu, rr[3] = t.y >> 16;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (ow + e < p.OW)
            rr[e] = ES == 4 ? reinterpret_cast<const uint32_t*>(rsrc_p)[e] : reinterpret_cast<const uint16_t*>(rsrc_p)[e];
      }
    }
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = apply_act(p.act, vv[e]);
      if constexpr (CL) x = fminf(fmaxf(x, p.cmin), p.cmax);
      if constexpr (RS) x = p.rcs * x + p.rrs * to_f<DT>(rr[e]);
      h[e] = from_f<DT>(x);
    }
    if (vec && ow + 3 < p.OW) {
      if constexpr (ES == 4) *reinterpret_cast<uint4*>(dst) = make_uint4(h[0], h[1], h[2], h[3]);
      else *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (ow + e < p.OW) {
          if constexpr (ES == 4) reinterpret_cast<uint32_t*>(dst)[e] = h[e];
          else reinterpret_cast<uint16_t*>(dst)[e] = (uint16_t)h[e];
        }
    }
  };
  if (W == 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          store_group((i * TN + j) * 4 + g,
                      make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]));
  } else {
    for (int q = wave; q < NG; q += W) {
      float4 v = reinterpret_cast<const float4*>(part)[q * 64 + lane];
      for (int w = 1; w < W; ++w) {
        const float4 u = reinterpret_cast<const float4*>(part)[(w * NG + q) * 64 + lane];
        v.x += u.x;
        v.y += u.y;
        v.z += u.z;
        v.w += u.w;
      }
      store_group(q, v);
    }
  }
}

template <int DT, int TM, int TN, int CW = 8>
__device__ __forceinline__ void conv_epilogue(const CParams& p, f32x16 (&acc)[TM][TN], char* lds, int W, int wave,
                                              int lane, int m0, int oh0, int ow0, int z, const float (&brow)[TM]) {
  if (p.has_clamp) {
    if (p.res) conv_epilogue_t<DT, TM, TN, true, true, CW>(p, acc, lds, W, wave, lane, m0, oh0, ow0, z, brow);
    else conv_epilogue_t<DT, TM, TN, true, false, CW>(p, acc, lds, W, wave, lane, m0, oh0, ow0, z, brow);
  } else {
    if (p.res) conv_epilogue_t<DT, TM, TN, false, true, CW>(p, acc, lds, W, wave, lane, m0, oh0, ow0, z, brow);
    else conv_epilogue_t<DT, TM, TN, false, false, CW>(p, acc, lds, W, wave, lane, m0, oh0, ow0, z, brow);
  }
}

// One tile of the channel-major LDS-patch convolution: block blk of nblk
// (the launch's whole grid, or one convolution's share of a paired launch).
template <int DT, int KH, int KW, int S, int TM, int TN, bool RV>
__device__ __forceinline__ void conv_lds_tile(const CParams& p, int blk, int nblk) {
  using G = Geo<DT, KH, KW, S, TN, RV>;
  static_assert(!RV || DT == WGX_FLOAT32, "row segments are 4 float32 pixels");
  constexpr int ES = G::ES, T = G::T, STEPS = G::STEPS, NBLK = G::NBLK, PF = G::PF;
  extern __shared__ uint4 lds_u4[];
  char* lds = reinterpret_cast<char*>(lds_u4);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = p.W;
  const int fr = lane & 31, fc = lane >> 5;
  // XCD-aware numbering (block ids are dealt round-robin to the 8 XCDs):
  // XCD x gets a contiguous run of tiles; output-channel tiles vary fastest,
  // so the tiles of one pixel region (one input patch) meet in one L2
  const int Gn = nblk;
  const int rb = (Gn & 7) == 0 ? (blk & 7) * (Gn >> 3) + (blk >> 3) : blk;
  int t = rb;
  const int tm = t % p.tiles_m;
  t /= p.tiles_m;
  const int tw = t % p.tiles_w;
  t /= p.tiles_w;
  const int th = t % p.tiles_h;
  const int z = t / p.tiles_h;
  const int m0 = tm * TM * 32, oh0 = th * G::RH, ow0 = tw * G::RW;
  const int K = p.IC * T;

  // A: lane offset of its weight row's 16-byte run (this lane half's 8
  // channels of the chunk); rows past OC read zero
  uint32_t va[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int oc = m0 + i * 32 + fr;
    va[i] = oc < p.OC ? (uint32_t)(oc * K * ES + fc * 16) : OOB;
  }
  // patch block e of a channel: this lane's (row, column) of the patch
  // and its input offset in channel 0 of the chunk (OOB outside the image or
  // past the plane)
  const int ih0 = oh0 * S - p.pH, iw0 = ow0 * S - p.pW;
  const int plane = p.IH * p.IW;
  constexpr int NVP = RV ? G::NPASS : NBLK;
  uint32_t vp[NVP];
  // RV: segment pass e covers row segment q = 64e + lane (row q / NSEG,
  // columns a0 + 4 (q % NSEG) + 0..3 of the image, a0 = iw0 rounded down to
  // a multiple of 4: with the width a multiple of 4 a segment is wholly
  // inside or wholly outside the image); vw: its LDS byte offset, -1 past
  // the patch
  const int a0 = iw0 - (((iw0 % 4) + 4) % 4), dl = RV ? iw0 - a0 : 0;
  int vw[RV ? G::NPASS : 1];
#pragma unroll
  for (int e = 0; e < NVP; ++e) {
    const int q = e * 64 + lane;
    if constexpr (RV) {
      const int pr = q / G::NSEG, sg = q - pr * G::NSEG;
      const int ih = ih0 + pr, col = a0 + 4 * sg;
      vp[e] = (q < G::NRS && ih >= 0 && ih < p.IH && col >= 0 && col + 4 <= p.IW) ? (uint32_t)(ih * p.IW + col) * ES
                                                                                    : OOB;
      vw[e] = q < G::NRS ? q * 16 : -1;
    } else {
      const int pr = q / G::PW, pc = q - pr * G::PW;
      const int ih = ih0 + pr, iw = iw0 + pc;
      vp[e] = (q < G::PHW && ih >= 0 && ih < p.IH && iw >= 0 && iw < p.IW) ? (uint32_t)(ih * p.IW + iw) * ES : OOB;
    }
  }
  char* wl = lds + wave * G::LDS_WAVE;
  // B: the lane's output pixel in each 4 x 8 block of the region
  // the lane's bias per row block, fetched now, off the epilogue's path
  float brow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int oc = m0 + i * 32 + fr;
    brow[i] = (p.bias && oc < p.OC)
                  ? to_f<DT>(ES == 4 ? reinterpret_cast<const uint32_t*>(p.bias)[oc]
                                     : (uint32_t)reinterpret_cast<const uint16_t*>(p.bias)[oc])
                  : 0.0f;
  }
  // per region block j and lower-half tap t: the lane's B base (its pixel,
  // plus what the upper lane half adds for that tap; see Geo::koff)
  int vb[TN][T];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int v0 = (((4 * j + (fr >> 3)) * S) * G::ROWP + (fr & 7) * S + dl) * ES;
#pragma unroll
    for (int t = 0; t < T; ++t) vb[j][t] = v0 + (fc ? G::dhalf(t) : 0);
  }

  const char* ximg = static_cast<const char*>(p.x) + (long long)z * p.sx * ES;
  const char* wbase = static_cast<const char*>(p.w);
  constexpr int CH = 2 * G::CPL;  // channels per chunk
  const uint32_t chunk_x = (uint32_t)(CH * plane * ES), chunk_w = (uint32_t)(CH * T * ES);
  const uint32_t wbytes = (uint32_t)((long long)p.OC * K * ES);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // the chunk's patch in registers: CH channels x NBLK blocks (16-bit
  // elements two channels to a register)
  constexpr int NPV = RV ? 1 : (ES == 4 ? CH * NBLK : CH / 2 * NBLK);
  uint32_t pv[NPV];
  uint4 ps[RV ? G::NPASS : 1][RV ? CH : 1];  // RV: the row segments
  const uint32_t cplane = (uint32_t)(plane * ES);
  auto load_patch = [&](int c) {
    const rsrc_t rx = rsrc(ximg + (long long)c * chunk_x, chunk_x);
    if constexpr (RV) {
#pragma unroll
      for (int e = 0; e < G::NPASS; ++e)
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) ps[e][ch] = ld16(rx, vp[e], ch * cplane);
      return;
    }
#pragma unroll
    for (int e = 0; e < NBLK; ++e)
#pragma unroll
      for (int ch = 0; ch < CH; ch += (ES == 4 ? 1 : 2)) {
        if constexpr (ES == 4) {
          pv[ch * NBLK + e] = ld_el<4>(rx, vp[e], ch * cplane);
        } else {
          const uint32_t lo = ld_el<2>(rx, vp[e], ch * cplane), hi = ld_el<2>(rx, vp[e], (ch + 1) * cplane);
          pv[(ch >> 1) * NBLK + e] = lo | (hi << 16);
        }
      }
  };
  auto store_patch = [&]() {
    if constexpr (RV) {
#pragma unroll
      for (int e = 0; e < G::NPASS; ++e)
        if (vw[e] >= 0) {
#pragma unroll
          for (int ch = 0; ch < CH; ++ch)
            *reinterpret_cast<uint4*>(wl + ch * G::PHWP * ES + vw[e]) = ps[e][ch];
        }
      return;
    }
#pragma unroll
    for (int e = 0; e < NBLK; ++e)
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        char* dst = wl + (ch * G::PHWP + e * 64 + lane) * ES;
        if constexpr (ES == 4) *reinterpret_cast<uint32_t*>(dst) = pv[ch * NBLK + e];
        else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)(pv[(ch >> 1) * NBLK + e] >> (16 * (ch & 1)));
      }
  };

  // A fragments run PF steps ahead of the multiply, across chunk ends: a[s %
  // PF] holds step s of the current chunk, and once it is consumed the slot
  // takes step s + PF (of this chunk, or of the wave's next chunk)
  auto wrsrc = [&](int cc) { return rsrc(wbase + (long long)cc * chunk_w, wbytes - (uint32_t)cc * chunk_w); };
  uint4 a[PF][TM];
  int c = wave;
  if (c < p.nchunks) {
    load_patch(c);
    const rsrc_t rw0 = wrsrc(c);
#pragma unroll
    for (int s = 0; s < PF; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i) a[s][i] = ld16(rw0, va[i], (uint32_t)(s * 32));
  }
  for (; c < p.nchunks; c += W) {
    const bool more = c + W < p.nchunks;
    const rsrc_t rw = wrsrc(c);
    const rsrc_t rn = wrsrc(more ? c + W : c);
    // the patch -> LDS (the previous chunk's reads came first: a wave's LDS
    // operations run in order)
    store_patch();
    asm volatile("" ::: "memory");
    if (more) load_patch(c + W);
    // B fragments of step s + 1 are read from LDS while step s multiplies
    // (two register sets; the scheduling barriers keep the compiler from
    // sinking the reads next to their first use)
    auto read_b = [&](uint4* bf, int s) {
      // element e of fragment s: chunk k = 2*EPC*s + e (lower half; the
      // upper half's k + EPC through the lane's base for tap k % T)
      auto ld = [&](int j, int e) -> const char* {
        const int k = 2 * G::EPC * s + e;
        return wl + vb[j][k % T] + G::koff(k);
      };
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (ES == 4) {
          bf[j].x = *reinterpret_cast<const uint32_t*>(ld(j, 0));
          bf[j].y = *reinterpret_cast<const uint32_t*>(ld(j, 1));
          bf[j].z = *reinterpret_cast<const uint32_t*>(ld(j, 2));
          bf[j].w = *reinterpret_cast<const uint32_t*>(ld(j, 3));
        } else {
          const uint32_t h0 = *reinterpret_cast<const uint16_t*>(ld(j, 0));
          const uint32_t h1 = *reinterpret_cast<const uint16_t*>(ld(j, 1));
          const uint32_t h2 = *reinterpret_cast<const uint16_t*>(ld(j, 2));
          const uint32_t h3 = *reinterpret_cast<const uint16_t*>(ld(j, 3));
          const uint32_t h4 = *reinterpret_cast<const uint16_t*>(ld(j, 4));
          const uint32_t h5 = *reinterpret_cast<const uint16_t*>(ld(j, 5));
          const uint32_t h6 = *reinterpret_cast<const uint16_t*>(ld(j, 6));
          const uint32_t h7 = *reinterpret_cast<const uint16_t*>(ld(j, 7));
          bf[j] = make_uint4(h0 | (h1 << 16), h2 | (h3 << 16), h4 | (h5 << 16), h6 | (h7 << 16));
        }
      }
    };
    uint4 bb[2][TN];
    read_b(bb[0], 0);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      uint4 af[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = a[s % PF][i];
      if (s + PF < STEPS) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[s % PF][i] = ld16(rw, va[i], (uint32_t)((s + PF) * 32));
      } else if (more) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[s % PF][i] = ld16(rn, va[i], (uint32_t)((s + PF - STEPS) * 32));
      }
      if (s + 1 < STEPS) read_b(bb[(s + 1) & 1], s + 1);
      __builtin_amdgcn_sched_barrier(0);
      const uint4* b = bb[s & 1];
      if constexpr (ES == 4) {
        // the four k of a fragment, each over every accumulator in turn, so
        // consecutive MFMAs never wait on each other's results
        const float* bf = reinterpret_cast<const float*>(b);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[j * 4 + e],
                                                              __uint_as_float(reinterpret_cast<const uint32_t*>(&af[i])[e]),
                                                              acc[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int i = 0; i < TM; ++i) acc[i][j] = mma<DT>(b[j], af[i], acc[i][j]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::: "memory");
  }

  conv_epilogue<DT, TM, TN>(p, acc, lds, W, wave, lane, m0, oh0, ow0, z, brow);
}

template <int DT, int KH, int KW, int S, int TM, int TN, bool RV>
__global__ __launch_bounds__(512) void k_conv_lds(CParams p) {
  conv_lds_tile<DT, KH, KW, S, TM, TN, RV>(p, blockIdx.x, gridDim.x);
}

// Two independent float32 batch-1 convolutions (32 x (32 TN) tiles, 4 waves
// per block) in one launch: blocks [0, na) run a's tiles, the rest b's, so the
// start-up loads of one and the reduction and stores of the other overlap
// on the same CUs instead of following each other.
template <int SA, bool RVA, int SB, bool RVB, int TNA, int TNB>
__global__ __launch_bounds__(256) void k_conv_lds_pair(CParams pa, CParams pb, int na) {
  if ((int)blockIdx.x < na)
    conv_lds_tile<WGX_FLOAT32, 3, 3, SA, 1, TNA, RVA>(pa, blockIdx.x, na);
  else
    conv_lds_tile<WGX_FLOAT32, 3, 3, SB, 1, TNB, RVB>(pb, blockIdx.x - na, gridDim.x - na);
}


// ------------------------------------------------------------ 16-bit form
// float16 / bfloat16 with a channel-last patch.  Within a chunk of 16 input
// channels the K order is (tap, channel): step t is tap (kh, kw) = (t / KW,
// t % KW), lanes 0-31 taking the chunk's channels 0-7 of it and lanes 32-63
// channels 8-15.  Then
//   * B: a patch pixel holds its 16 channels in 32 contiguous bytes, so a
//     lane's B fragment (8 channels of one tap at its output pixel) is ONE
//     16-byte ds_read at a lane base plus a compile-time tap offset (the
//     channel-major form above needs one 2-byte ds_read per element);
//   * A: a lane's 8 channels x T taps are still 8T contiguous elements of its
//     OIHW weight row (T 16-byte loads per chunk); the fragment of tap t
//     (elements c*T + t, c = 0..7) is assembled from them in registers.
// LDS: patch row r starts at r * PW * 32 + (r / S) * 16 bytes; in it column c
// sits at slot c (S == 1), or (c & 1) * CE + c / 2 (S == 2: the even columns,
// then the odd ones), 32 bytes a slot.  The 16-byte stagger between the rows
// that consecutive 8-lane groups read and the column split at stride 2 put
// the 16 lanes of one LDS cycle on different banks.
// CW: output columns of the region, 8 (32-pixel blocks of 4 rows x 8) or 16
// (blocks of 2 rows x 16: longer patch rows and 32-byte output row pieces)
template <int KH, int KW, int S, int TN, int CW = 8>
struct GeoCL {
  static constexpr int T = KH * KW;
  static constexpr int RB = 32 / CW;  // rows of a 32-pixel block
  static constexpr int RH = RB * TN, RW = CW;
  static constexpr int PH = (RH - 1) * S + KH, PW = (RW - 1) * S + KW;
  static constexpr int PHW = PH * PW;
  static constexpr int NBLK = (PHW + 63) / 64;  // patch pixels per lane
  static constexpr int CE = (PW + 1) / 2;      // even columns (S == 2)
  static constexpr int slot(int c) { return S == 1 ? c : (c & 1) * CE + (c >> 1); }
  static constexpr int row(int r) { return r * PW * 32 + (r / S) * 16; }
  static constexpr int LDS_WAVE = row(PH);     // bytes of a wave's patch
  // tap t relative to the lane's pixel (patch row a*S, column b*S): rows
  // a*S + kh start row(kh) after row a*S (r / S steps by kh / S), and column
  // b*S + kw sits slot(kw) after slot b*S
  static constexpr int toff(int t) { return row(t / KW) + slot(t % KW) * 32; }
  // row-segment staging: 8-column segments of one channel (16 bytes), at
  // most NSEG per patch row (the first one starts up to 7 columns left of
  // the patch), one task per (row, segment, half of the chunk's channels)
  static constexpr int NSEG = (PW + 7 + 7) / 8;
  static constexpr int NTASK = PH * NSEG * 2;
  static constexpr int NPASS = (NTASK + 63) / 64;
};

// RV: the patch loaded as 16-byte row segments (images whose width is a
// multiple of 8 columns): a lane loads one segment of each of 8 channels and
// turns the 8 x 8 block channel-last in registers, 16 bytes per pixel, in
// place of one 2-byte load per pixel and channel.
// PRE: the weights come pre-ordered [chunk][tap][OC][16 channels] (written
// by k_w_tapmajor), so a fragment is one 16-byte load and a row block's 32
// rows are contiguous; they stream RING taps
// ahead of the multiplies instead of a whole chunk ahead, which frees the
// registers of the chunk-ahead copy and its rebuild.
template <int DT, int KH, int KW, int S, int TM, int TN, bool RV, bool PRE = false, int CW = 8, bool SH = false>
__global__ __launch_bounds__(TM * TN >= 4 ? 256 : 512)
__attribute__((amdgpu_waves_per_eu(PRE && TM * TN == 4 ? 2 : 1))) void k_conv_cl(CParams p) {
  using G = GeoCL<KH, KW, S, TN, CW>;
  constexpr int T = G::T, NBLK = G::NBLK;
  constexpr int RING = 3;
  // the next chunk's tap t + RING - T takes the slot tap t just left
  static_assert(T % RING == 0, "the weight ring must divide the tap count");
  constexpr int NL = T;  // 16-byte weight loads per row block per chunk (8 channels x T taps)
  extern __shared__ uint4 lds_u4[];
  char* lds = reinterpret_cast<char*>(lds_u4);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = p.W;
  const int fr = lane & 31, fc = lane >> 5;
  // SHW > 1 (pre-ordered weights, row segments, W = 1): the block's waves take
  // output-channel tiles tmb*SHW + wave of one pixel tile and load one shared
  // patch between them, each wave a contiguous share of its segment tasks
  // (SH: built for a shared patch, p.share >= 2, so a wave's share of the
  // segment tasks fits fewer passes)
  const int SHW = (PRE && RV && SH) ? p.share : 1;
  const int sw = SHW > 1 ? wave : 0;
  // XCD-aware numbering, output-channel tiles fastest (as in k_conv_lds)
  const int Gn = gridDim.x;
  const int rb = (Gn & 7) == 0 ? (blockIdx.x & 7) * (Gn >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int mtb = (p.tiles_m + SHW - 1) / SHW;
  int t0 = rb;
  const int tm = (t0 % mtb) * SHW + sw;
  t0 /= mtb;
  const int tw = t0 % p.tiles_w;
  t0 /= p.tiles_w;
  const int th = t0 % p.tiles_h;
  const int z = t0 / p.tiles_h;
  const int m0 = tm * TM * 32, oh0 = th * G::RH, ow0 = tw * G::RW;
  const int K = p.IC * T;

  // A: lane offset of its weight row's run (this lane half's 8 channels of
  // the chunk x T taps); rows past OC read zero
  // (PRE: of its fragment of tap 0 in chunk 0; chunk c, tap t lie (c*T + t)
  // * OC * 32 bytes further)
  uint32_t va[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int oc = m0 + i * 32 + fr;
    va[i] = oc < p.OC ? (PRE ? (uint32_t)(oc * 32 + fc * 16) : (uint32_t)(oc * K + fc * 8 * T) * 2) : OOB;
  }
  // patch pixel q = e*64 + lane: its input offset in channel 0 of the chunk
  // (OOB outside the image) and its LDS slot (-1 past the patch)
  const int ih0 = oh0 * S - p.pH, iw0 = ow0 * S - p.pW;
  const int plane = p.IH * p.IW;
  constexpr int NP = RV ? 1 : NBLK;
  uint32_t vp[NP];
  int vw[NP];
  if constexpr (!RV) {
#pragma unroll
    for (int e = 0; e < NBLK; ++e) {
      const int q = e * 64 + lane;
      const int pr = q / G::PW, pc = q - pr * G::PW;
      const int ih = ih0 + pr, iw = iw0 + pc;
      vp[e] = (q < G::PHW && ih >= 0 && ih < p.IH && iw >= 0 && iw < p.IW) ? (uint32_t)(ih * p.IW + iw) * 2 : OOB;
      vw[e] = q < G::PHW ? G::row(pr) + G::slot(pc) * 32 : -1;
    }
  }
  // RV task q = e*64 + lane: segment g = q % NSEG at image column a0 + 8g
  // (a0: iw0 rounded down to a multiple of 8, so a segment lies wholly
  // inside or outside the image), channel half h = (q / NSEG) & 1, patch row
  // r = q / (2 NSEG).  Segments vary fastest: neighbouring lanes load
  // neighbouring 16 bytes of one channel row, which the address unit takes
  // as one run (neighbours in different channel planes cost it one cycle
  // pair each).  sp: its input offset in channel 0 of the chunk (OOB
  // outside), sr: LDS offset of its row and channel half (-1: no task), sg:
  // the patch column of its first pixel
  constexpr int NS = RV ? (SH ? ((G::NTASK + 1) / 2 + 63) / 64 : G::NPASS) : 1;
  uint32_t sp[NS];
  int sr[NS], sg[NS];
  // tasks per wave: all of them, or a contiguous share of a shared patch
  const int qpw = (G::NTASK + SHW - 1) / SHW;
  if constexpr (RV) {
    const int a0 = iw0 - (((iw0 % 8) + 8) % 8), dl = iw0 - a0;
#pragma unroll
    for (int e = 0; e < NS; ++e) {
      const int ql = e * 64 + lane, q = sw * qpw + ql, rh = q / G::NSEG, g = q - rh * G::NSEG;
      const int h = rh & 1, r = rh >> 1;
      const int ih = ih0 + r, s0 = a0 + 8 * g;
      const bool ok = ql < qpw && q < G::NTASK;
      sp[e] = (ok && ih >= 0 && ih < p.IH && s0 >= 0 && s0 < p.IW)
                  ? (uint32_t)((ih * p.IW + s0) * 2 + h * 8 * plane * 2)
                  : OOB;
      sr[e] = ok ? G::row(r) + h * 16 : -1;
      sg[e] = 8 * g - dl;
    }
  }
  // a wave's own patch, or (shared) two patch buffers taken in turn by
  // consecutive chunks
  char* const wl0 = lds + (SHW > 1 ? 0 : wave * G::LDS_WAVE);
  char* wl = wl0;
  float brow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int oc = m0 + i * 32 + fr;
    brow[i] = (p.bias && oc < p.OC) ? to_f<DT>((uint32_t)reinterpret_cast<const uint16_t*>(p.bias)[oc]) : 0.0f;
  }
  // B: the lane's output pixel (row RB*j + fr/CW, column fr%CW of the region)
  int vb[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) vb[j] = G::row((G::RB * j + fr / CW) * S) + (fr % CW) * 32 + fc * 16;

  const char* ximg = static_cast<const char*>(p.x) + (long long)z * p.sx * 2;
  const char* wbase = static_cast<const char*>(p.w);
  const uint32_t chunk_x = (uint32_t)(16 * plane * 2), chunk_w = (uint32_t)(16 * T * 2);
  const uint32_t wbytes = (uint32_t)((long long)p.OC * K * 2);
  const uint32_t cplane = (uint32_t)(plane * 2);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // the chunk's patch pixels in registers, channels 2m and 2m+1 in pv[e][m]
  // (RV: segment e of channel ch in ps[e][ch], pixels 2d and 2d+1 in dword d)
  uint32_t pv[RV ? 1 : NBLK][8];
  uint4 ps[NS][RV ? 8 : 1];
  auto load_patch = [&](int c) {
    const rsrc_t rx = rsrc(ximg + (long long)c * chunk_x, chunk_x);
    if constexpr (RV) {
#pragma unroll
      for (int e = 0; e < NS; ++e)
        if (e * 64 < qpw) {
#pragma unroll
          for (int ch = 0; ch < 8; ++ch) ps[e][ch] = ld16(rx, sp[e], ch * cplane);
        }
    } else {
#pragma unroll
      for (int e = 0; e < NBLK; ++e)
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const uint32_t lo = ld_el<2>(rx, vp[e], 2 * m * cplane), hi = ld_el<2>(rx, vp[e], (2 * m + 1) * cplane);
          pv[e][m] = lo | (hi << 16);
        }
    }
  };
  auto store_patch = [&]() {
    if constexpr (RV) {
      auto dw = [](const uint4& v, int d) { return d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w; };
#pragma unroll
      for (int e = 0; e < NS; ++e)
        if (sr[e] >= 0) {
#pragma unroll
          for (int px = 0; px < 8; ++px) {
            const int col = sg[e] + px;
            if (col < 0 || col >= G::PW) continue;
            uint32_t m4[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const uint32_t a = dw(ps[e][2 * m], px >> 1), b = dw(ps[e][2 * m + 1], px >> 1);
              m4[m] = (px & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
            }
            *reinterpret_cast<uint4*>(wl + sr[e] + G::slot(col) * 32) = make_uint4(m4[0], m4[1], m4[2], m4[3]);
          }
        }
    } else {
#pragma unroll
      for (int e = 0; e < NBLK; ++e)
        if (vw[e] >= 0) {
          *reinterpret_cast<uint4*>(wl + vw[e]) = make_uint4(pv[e][0], pv[e][1], pv[e][2], pv[e][3]);
          *reinterpret_cast<uint4*>(wl + vw[e] + 16) = make_uint4(pv[e][4], pv[e][5], pv[e][6], pv[e][7]);
        }
    }
  };
  // the lane's raw weight run of the next chunk (element c*T + t: channel c,
  // tap t) and the fragments of the current one
  uint4 ra[PRE ? 1 : TM][PRE ? 1 : NL];
  // PRE: tap t of chunk c into ring slot t % RING
  uint4 ar[PRE ? RING : 1][TM];
  const rsrc_t rwp = rsrc(wbase, wbytes);
  auto load_tap = [&](int c, int t) {
#pragma unroll
    for (int i = 0; i < TM; ++i) ar[t % RING][i] = ld16(rwp, va[i], (uint32_t)((c * T + t) * p.OC * 32));
  };
  auto load_a = [&](int c) {
    const rsrc_t rw = rsrc(wbase + (long long)c * chunk_w, wbytes - (uint32_t)c * chunk_w);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int s = 0; s < NL; ++s) ra[i][s] = ld16(rw, va[i], (uint32_t)(s * 16));
  };
  uint4 af[PRE ? 1 : T][TM];
  auto build_a = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      uint32_t w[4 * NL];
#pragma unroll
      for (int s = 0; s < NL; ++s) {
        w[4 * s] = ra[i][s].x;
        w[4 * s + 1] = ra[i][s].y;
        w[4 * s + 2] = ra[i][s].z;
        w[4 * s + 3] = ra[i][s].w;
      }
      auto h = [&](int q) -> uint32_t { return (q & 1) ? (w[q >> 1] >> 16) : (w[q >> 1] & 0xffffu); };
#pragma unroll
      for (int t = 0; t < T; ++t)
        af[t][i] = make_uint4(h(t) | (h(T + t) << 16), h(2 * T + t) | (h(3 * T + t) << 16),
                              h(4 * T + t) | (h(5 * T + t) << 16), h(6 * T + t) | (h(7 * T + t) << 16));
    }
  };

  int c = SHW > 1 ? 0 : wave;
  if (c < p.nchunks) {
    load_patch(c);
    if constexpr (PRE) {
#pragma unroll
      for (int t = 0; t < RING; ++t) load_tap(c, t);
    } else {
      load_a(c);
    }
  }
  for (int it = 0; c < p.nchunks; c += W, ++it) {
    const bool more = c + W < p.nchunks;
    // the patch -> LDS (the previous chunk's reads came first: a wave's LDS
    // operations run in order), the weights -> fragments, then the next
    // chunk's loads go out behind this chunk's multiplies
    if (SHW > 1) wl = wl0 + (it & 1) * G::LDS_WAVE;
    store_patch();
    if constexpr (!PRE) build_a();
    // shared patch: every wave's share is in LDS before any wave reads it
    // (the buffer written here was last read two chunks ago, before every
    // wave reached the previous chunk's barrier)
    if (SHW > 1) __syncthreads();
    asm volatile("" ::: "memory");
    if (more) {
      load_patch(c + W);
      if constexpr (!PRE) load_a(c + W);
    }
    auto read_b = [&](uint4* bf, int t) {
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const uint4*>(wl + vb[j] + G::toff(t));
    };
    uint4 bb[2][TN];
    read_b(bb[0], 0);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (t + 1 < T) read_b(bb[(t + 1) & 1], t + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = mma<DT>(bb[t & 1][j], PRE ? ar[t % RING][i] : af[PRE ? 0 : t][i], acc[i][j]);
      if constexpr (PRE) {
        // the slot just read takes tap t + RING (of the next chunk past the last tap)
        if (t + RING < T) load_tap(c, t + RING);
        else if (more) load_tap(c + W, t + RING - T);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::: "memory");
  }

  conv_epilogue<DT, TM, TN, CW>(p, acc, lds, W, wave, lane, m0, oh0, ow0, z, brow);
}

// 16-bit weights [OC][IC][T] -> [IC/16][T][OC][16]: for chunk q and tap t
// the 16 channels of consecutive output channels are consecutive 32-byte
// pieces, so the 32 rows of a weight fragment load are 1 KB of contiguous
// memory (the channel-last kernel's PRE form)
__global__ __launch_bounds__(256) void k_w_tapmajor(const uint16_t* __restrict__ w, uint16_t* __restrict__ wp,
                                                    long long n, int OC, int IC, int T) {
  for (long long d = (long long)blockIdx.x * 256 + threadIdx.x; d < n; d += (long long)gridDim.x * 256) {
    const int cc = (int)(d & 15);
    const long long rest = d >> 4;
    const int oc = (int)(rest % OC);
    const long long qt = rest / OC;
    const int t = (int)(qt % T), q = (int)(qt / T);
    wp[d] = w[((long long)oc * IC + q * 16 + cc) * T + t];
  }
}

struct Cfg {
  int tm, tn, w;
  bool cl;  // 16-bit data: the channel-last kernel (else the channel-major one)
  bool rv;  // float32: the patch loaded as 16-byte row segments
  int cw = 8;  // output columns of a region (16: the channel-last tile on pre-ordered weights)
};

template <bool CL, bool RV, int DT, int KH, int KW, int S, int TM, int TN>
hipError_t launch_t(const CParams& p, size_t lds, unsigned grid, int w, hipStream_t s) {
  void (*fn)(CParams);
  if constexpr (CL) fn = k_conv_cl<DT, KH, KW, S, TM, TN, RV>;
  else fn = k_conv_lds<DT, KH, KW, S, TM, TN, RV>;
  // the channel-last kernel's larger tiles are built for at most 256 threads
  if (CL && TM * TN >= 4 && w > 4) return hipErrorInvalidValue;
  static bool attr_set = false;
  if (!attr_set && s != name_only()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  if (is_dry(s)) return hipSuccess;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * w), lds, s, p);
  return hipGetLastError();
}

template <bool CL, bool RV, int DT, int KH, int KW, int S, int TM, int TN>
hipError_t launch_cfg(const CParams& p, const Cfg& c, unsigned grid, hipStream_t s) {
  const size_t wave_patch =
      CL ? (size_t)GeoCL<KH, KW, S, TN>::LDS_WAVE : (size_t)Geo<DT, KH, KW, S, TN, RV>::LDS_WAVE;
  const size_t patch = (size_t)c.w * wave_patch;
  const size_t part = c.w > 1 ? (size_t)c.w * TM * TN * 4 * 64 * 16 : 0;
  const size_t lds = patch > part ? patch : part;
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  return launch_t<CL, RV, DT, KH, KW, S, TM, TN>(p, lds, grid, c.w, s);
}

// Instantiated tiles (TM x TN): 32 x 32 up to 64 x 128 (stride 1) and 64 x
// 64 (stride 2, whose patches are four times larger).
template <bool CL, bool RV, int DT, int KH, int KW, int S>
hipError_t launch_geo(const CParams& p, const Cfg& c, unsigned grid, hipStream_t s) {
  if (c.tm == 1 && c.tn == 1) return launch_cfg<CL, RV, DT, KH, KW, S, 1, 1>(p, c, grid, s);
  if (c.tm == 1 && c.tn == 2) return launch_cfg<CL, RV, DT, KH, KW, S, 1, 2>(p, c, grid, s);
  if (c.tm == 2 && c.tn == 1) return launch_cfg<CL, RV, DT, KH, KW, S, 2, 1>(p, c, grid, s);
  if (c.tm == 2 && c.tn == 2) return launch_cfg<CL, RV, DT, KH, KW, S, 2, 2>(p, c, grid, s);
  if constexpr (S == 1)
    if (c.tm == 2 && c.tn == 4) return launch_cfg<CL, RV, DT, KH, KW, S, 2, 4>(p, c, grid, s);
  return hipErrorInvalidValue;
}

template <int DT>
hipError_t launch_dt(const CParams& p, const Cfg& c, int S, unsigned grid, hipStream_t s) {
  if constexpr (DT == WGX_FLOAT32) {
    if (c.rv)
      return S == 1 ? launch_geo<false, true, DT, 3, 3, 1>(p, c, grid, s) : launch_geo<false, true, DT, 3, 3, 2>(p, c, grid, s);
    return S == 1 ? launch_geo<false, false, DT, 3, 3, 1>(p, c, grid, s) : launch_geo<false, false, DT, 3, 3, 2>(p, c, grid, s);
  } else {
    if (c.cl && c.rv)
      return S == 1 ? launch_geo<true, true, DT, 3, 3, 1>(p, c, grid, s) : launch_geo<true, true, DT, 3, 3, 2>(p, c, grid, s);
    if (c.cl) return S == 1 ? launch_geo<true, false, DT, 3, 3, 1>(p, c, grid, s) : launch_geo<true, false, DT, 3, 3, 2>(p, c, grid, s);
    return S == 1 ? launch_geo<false, false, DT, 3, 3, 1>(p, c, grid, s) : launch_geo<false, false, DT, 3, 3, 2>(p, c, grid, s);
  }
}

// LDS bytes of a channel-last block of W waves: their patches, or the
// partial sums of their reduction, whichever is larger.
template <int S, int TM, int TN, int CW = 8>
size_t cl_block_lds(int W) {
  const size_t patch = (size_t)W * GeoCL<3, 3, S, TN, CW>::LDS_WAVE;
  const size_t part = W > 1 ? (size_t)W * TM * TN * 4 * 64 * 16 : 0;
  return patch > part ? patch : part;
}

// The channel-last tile on pre-ordered weights: the reorder pass into wpre,
// then the kernel reading them, in blocks of W waves.
template <int DT, bool RV, int TM, int TN, int S, int CW = 8, bool SH = false>
hipError_t launch_cl_pre(const CParams& p, const void* w, void* wpre, unsigned grid, int W, hipStream_t s) {
  // a shared patch: two buffers for the block (W is 1 then)
  const size_t lds = p.share > 1 ? 2 * (size_t)GeoCL<3, 3, S, TN, CW>::LDS_WAVE : cl_block_lds<S, TM, TN, CW>(W);
  const int nw = p.share > 1 ? p.share : W;
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  if (is_dry(s)) return hipSuccess;
  auto fn = k_conv_cl<DT, 3, 3, S, TM, TN, RV, true, CW, SH>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const long long n = (long long)p.OC * p.IC * 9;
  const unsigned rgrid = (unsigned)std::min<long long>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(k_w_tapmajor, dim3(rgrid), dim3(256), 0, s, static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(wpre), n, p.OC, p.IC, 9);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  CParams q = p;
  q.w = wpre;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * nw), lds, s, q);
  return hipGetLastError();
}

// A shared patch (p.share >= 2, row segments only) takes the kernel built
// for it: a wave's share of the segment tasks fits fewer passes.
template <int DT, bool RV, int TM, int TN, int S, int CW = 8>
hipError_t launch_cl_pre_sh(const CParams& p, const void* w, void* wpre, unsigned grid, int W, hipStream_t s) {
  if constexpr (RV)
    if (p.share > 1) return launch_cl_pre<DT, RV, TM, TN, S, CW, true>(p, w, wpre, grid, W, s);
  return launch_cl_pre<DT, RV, TM, TN, S, CW, false>(p, w, wpre, grid, W, s);
}

// The tiles that run on pre-ordered weights: 64 x 64 one-wave (either
// stride) and 64 x 128 one-wave (stride 1).  The batch-1 split-chunk tiles
// keep the raw weights: on them the kernel gains (32 x 64 s1 [1,64,80,80]
// -> 128: 7.6 us, 64 x 32 s2 [1,128,80,80] -> 256: 8.5 us), but the reorder
// launch (4.4 us) costs more than that in a graph of batch-1 launches
// (10.0 / 11.5 us against 9.1 / 12.5 us amortised; [1,256,20,20] -> 256:
// 17.7 against 12.4 us).
bool pre_form(const Cfg& c, int S) {
  return c.cl && c.tm == 2 && c.w == 1 && (c.tn == 2 || (c.tn == 4 && S == 1));
}

template <int DT>
hipError_t launch_pre_dt(const CParams& p, const Cfg& c, int S, const void* w, void* wpre, unsigned grid,
                         hipStream_t s) {
  if (c.cw == 16) {  // row segments only (the caller keeps 8 columns otherwise)
    if (c.tm == 2 && c.tn == 2 && S == 2) return launch_cl_pre_sh<DT, true, 2, 2, 2, 16>(p, w, wpre, grid, c.w, s);
    if (c.tm == 2 && c.tn == 2 && S == 1) return launch_cl_pre_sh<DT, true, 2, 2, 1, 16>(p, w, wpre, grid, c.w, s);
    return hipErrorInvalidValue;
  }
  if (c.tm == 2 && c.tn == 2 && S == 2)
    return c.rv ? launch_cl_pre_sh<DT, true, 2, 2, 2>(p, w, wpre, grid, c.w, s)
                : launch_cl_pre_sh<DT, false, 2, 2, 2>(p, w, wpre, grid, c.w, s);
  if (c.tm == 2 && c.tn == 2)
    return c.rv ? launch_cl_pre_sh<DT, true, 2, 2, 1>(p, w, wpre, grid, c.w, s)
                : launch_cl_pre_sh<DT, false, 2, 2, 1>(p, w, wpre, grid, c.w, s);
  if (c.tm == 2 && c.tn == 4 && S == 1)
    return c.rv ? launch_cl_pre_sh<DT, true, 2, 4, 1>(p, w, wpre, grid, c.w, s)
                : launch_cl_pre_sh<DT, false, 2, 4, 1>(p, w, wpre, grid, c.w, s);
  return hipErrorInvalidValue;
}

// Input channels per chunk: 8 for float32 (the channel-major kernel's lane
// halves take 4 each), 16 for 16-bit data (8 per lane half, both kernels).
int chunk_channels(int dtype) { return dtype == WGX_FLOAT32 ? 8 : 16; }

long long tile_count(const ConvLdsDesc& d, const Cfg& c) {
  const int rh = 32 / c.cw * c.tn;  // output rows of a region
  return (long long)d.B * ((d.OC + 32 * c.tm - 1) / (32 * c.tm)) * ((d.OH + rh - 1) / rh) *
         ((d.OW + c.cw - 1) / c.cw);
}

// The configuration for a shape, from sweeps of the 3x3 maps [1,64,80,80] ->
// 128 (stride 1) and [1,128,80,80] -> 256 (stride 2) at batch 1 and 64:
//  - few output tiles (under two per SIMD at 64 x 64: batch-1 maps): a 32 x
//    64 tile (64 x 32 for 16-bit data at stride 2, whose patch is larger) and
//    W waves per block splitting its chunks of input channels, W up to the chunk
//    count and 8 while the waves stay below four per SIMD;
//  - many tiles: 64 x 64, one wave per tile, for float32; for 16-bit data at
//    stride 1 on images whose rows are whole 16-byte segments, the 64 x 128
//    channel-last tile; for other 16-bit shapes the LDS-staged GEMM
//    (gemm_mfma's conv form) is faster, and choose() returns tm = 0: the
//    kernel does not apply.
// WGX_CONV_LDS=TMxTNwW forces a configuration.
Cfg choose(const ConvLdsDesc& d, int cus) {
  const long long simds = 4LL * cus;
  const bool cl = d.dtype != WGX_FLOAT32 && !(getenv("WGX_CONV_CL") && strcmp(getenv("WGX_CONV_CL"), "0") == 0);
  // many tiles, 16-bit: the channel-last kernel with row-segment patch loads
  // at stride 1 while a 64 x 128 tiling still gives every SIMD a wave ([16,64,80,80]
  // -> 128: 60.9 us, [64,64,80,80]: 199 us, [8,32,160,160] -> 64: 45.9 us,
  // against 68.9 / 222 / 64.5 us for the LDS-staged GEMM); otherwise the GEMM
  // ([16,128,40,40] -> 256: 46.7 us against 56.8 for 32 x 64 one-wave tiles)
  // With pre-ordered weights (WGX_CONV_PRE, default on) the 64 x 64 tile
  // fits three waves per SIMD and wins at both strides while it gives every
  // SIMD a wave: [64,64,80,80] 151 us (64 x 128: 213), [8,32,160,160] 39.1
  // (50.0), [16,128,40,40] -> 256 37.7 (GEMM 47.1), stride 2
  // [64,128,80,80] -> 256 181 (GEMM 211), [16,128,80,80] 52.4 (57.8).
  // bfloat16 has no im2col GEMM and keeps the 64 x 64 tile where float16
  // would take the GEMM.
  auto many16 = [&]() {
    const bool seg = cl && d.IW % 8 == 0 && (reinterpret_cast<uintptr_t>(d.x) & 15) == 0 &&
                     !(getenv("WGX_CONV_RV") && strcmp(getenv("WGX_CONV_RV"), "0") == 0);
    const bool pre = !(getenv("WGX_CONV_PRE") && strcmp(getenv("WGX_CONV_PRE"), "0") == 0);
    Cfg m{2, 4, 1, cl};
    if (pre) {
      // the 64 x 64 tile, at either stride, while it gives every SIMD a wave
      m.tn = 2;
      // 16-column regions at stride 1 on widths that fill them (WGX_CONV_CW=8
      // keeps 8): [64,64,80,80] -> 128 123.8 -> 110.7 us, [8,32,160,160] -> 64
      // 30.6 -> 28.1; at stride 2 they tie (129.5 / 129.6 us), at width 40
      // they lose a little (33.1 -> 33.6: a third of the last region empty)
      const bool cw8 = getenv("WGX_CONV_CW") && strcmp(getenv("WGX_CONV_CW"), "8") == 0;
      if (d.sH == 1 && d.OW % 16 == 0 && !cw8) m.cw = 16;
      if (!(seg && tile_count(d, m) >= simds)) m.tm = 0;
    } else if (!(seg && d.sH == 1 && tile_count(d, m) >= simds)) {
      m.tm = 0;
    }
    // no bfloat16 im2col GEMM: the 64 x 64 one-wave tile
    if (m.tm == 0 && d.dtype == WGX_BFLOAT16) m = Cfg{2, 2, 1, cl};
    return m;
  };
  Cfg c{2, 2, 1, cl};
  if (tile_count(d, c) < 2 * simds) {
    if (d.dtype != WGX_FLOAT32 && d.sH == 2) c = Cfg{2, 1, 1, cl};
    else c = Cfg{1, 2, 1, cl};
    const long long tiles = tile_count(d, c);
    int w = 1;
    // each wave keeps at least 16 input channels (two float32 chunks, one
    // 16-bit chunk): [1,64,80,80] float32 16.8 us at 4 waves, 17.3 at 8
    while (w < 8 && w * 32 <= d.IC && tiles * w * 2 <= 4 * simds) w *= 2;
    c.w = w;
    // one wave per tile because the tiles are many (not because the input
    // has a single 16-channel chunk): the many-tile choice
    if (d.dtype != WGX_FLOAT32 && w == 1 && d.IC >= 32 && tiles * 2 > 4 * simds) c = many16();
  } else if (d.dtype != WGX_FLOAT32) {
    c = many16();
  }
  if (const char* e = getenv("WGX_CONV_LDS")) {
    // TMxTNwW, or TMxTNwWc16 for 16-column regions (kept on the pre-ordered
    // 64 x 64 tile only)
    int tm = 0, tn = 0, ww = 0, cwv = 8;
    if (sscanf(e, "%dx%dw%dc%d", &tm, &tn, &ww, &cwv) >= 3 && tm >= 1 && tm <= 2 && tn >= 1 && tn <= 4 && ww >= 1 &&
        ww <= 8) {
      c = Cfg{tm, tn, ww, cl};
      c.cw = cwv == 16 ? 16 : 8;
    }
  }
  return c;
}

// The kernel parameters of d under configuration c.
CParams make_params(const ConvLdsDesc& d, const Cfg& c) {
  CParams p{};
  p.x = d.x;
  p.w = d.w;
  p.bias = d.bias;
  p.y = d.y;
  p.IC = d.IC;
  p.IH = d.IH;
  p.IW = d.IW;
  p.OC = d.OC;
  p.OH = d.OH;
  p.OW = d.OW;
  p.pH = d.pH;
  p.pW = d.pW;
  p.sx = (long long)d.IC * d.IH * d.IW;
  p.sy = (long long)d.OC * d.OH * d.OW;
  p.tiles_m = (d.OC + 32 * c.tm - 1) / (32 * c.tm);
  p.tiles_h = (d.OH + 32 / c.cw * c.tn - 1) / (32 / c.cw * c.tn);
  p.tiles_w = (d.OW + c.cw - 1) / c.cw;
  p.ntiles = d.B * p.tiles_m * p.tiles_h * p.tiles_w;
  p.share = 1;
  p.nchunks = d.IC / chunk_channels(d.dtype);
  p.W = c.w;
  p.act = d.act;
  p.has_clamp = d.has_clamp;
  p.cmin = d.cmin;
  p.cmax = d.cmax;
  p.res = d.res;
  p.rcs = d.res_conv_scale;
  p.rrs = d.res_scale;
  return p;
}

// Images whose rows are whole 16-byte segments on a 16-byte base (float32: a
// multiple of 4 columns, 16-bit: of 8) load the patch as row segments;
// WGX_CONV_RV=0 keeps the element loads.
// (the channel-last 64 x 32 tile on raw weights spills 2 registers with row
// segments and still gains: [1,128,80,80] -> 256 stride 2 12.7 -> 11.7 us,
// [1,128,40,40] -> 256 12.0 -> 10.7)
bool use_rv(const ConvLdsDesc& d, const Cfg& c) {
  const bool rv_off = getenv("WGX_CONV_RV") && strcmp(getenv("WGX_CONV_RV"), "0") == 0;
  return d.IW % (d.dtype == WGX_FLOAT32 ? 4 : 8) == 0 && (reinterpret_cast<uintptr_t>(d.x) & 15) == 0 &&
         (d.dtype == WGX_FLOAT32 || c.cl) && !rv_off;
}

template <int SA, bool RVA, int SB, bool RVB, int TNA, int TNB>
hipError_t launch_pair_t(const CParams& pa, const CParams& pb, hipStream_t s) {
  auto fn = k_conv_lds_pair<SA, RVA, SB, RVB, TNA, TNB>;
  const size_t w = (size_t)pa.W;  // both parts run W waves per block
  const size_t la = w * Geo<WGX_FLOAT32, 3, 3, SA, TNA, RVA>::LDS_WAVE;
  const size_t lb = w * Geo<WGX_FLOAT32, 3, 3, SB, TNB, RVB>::LDS_WAVE;
  const size_t part = w > 1 ? w * 1 * 2 * 4 * 64 * 16 : 0;  // the waves' partial sums
  const size_t lds = std::max(std::max(la, lb), part);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(fn, dim3((unsigned)(pa.ntiles + pb.ntiles)), dim3(64 * (unsigned)w), lds, s, pa, pb, pa.ntiles);
  return hipGetLastError();
}

// (at most one part runs 32 x 32 tiles: TNA == 1 takes TNB == 2 only)
template <int SA, bool RVA, int TNA>
hipError_t launch_pair_b(const CParams& pa, const CParams& pb, int sb, bool rvb, int tnb, hipStream_t s) {
  if constexpr (TNA == 2) {
    if (tnb == 1) {
      if (sb == 1)
        return rvb ? launch_pair_t<SA, RVA, 1, true, 2, 1>(pa, pb, s) : launch_pair_t<SA, RVA, 1, false, 2, 1>(pa, pb, s);
      return rvb ? launch_pair_t<SA, RVA, 2, true, 2, 1>(pa, pb, s) : launch_pair_t<SA, RVA, 2, false, 2, 1>(pa, pb, s);
    }
  }
  if (tnb != 2) return hipErrorInvalidValue;
  if (sb == 1)
    return rvb ? launch_pair_t<SA, RVA, 1, true, TNA, 2>(pa, pb, s) : launch_pair_t<SA, RVA, 1, false, TNA, 2>(pa, pb, s);
  return rvb ? launch_pair_t<SA, RVA, 2, true, TNA, 2>(pa, pb, s) : launch_pair_t<SA, RVA, 2, false, TNA, 2>(pa, pb, s);
}

}  // namespace

bool conv_lds_applies(const ConvLdsDesc& d) {
  if (getenv("WGX_CONV_LDS") && strcmp(getenv("WGX_CONV_LDS"), "off") == 0) return false;
  if (d.dtype != WGX_FLOAT16 && d.dtype != WGX_FLOAT32 && d.dtype != WGX_BFLOAT16) return false;
  if (d.IC % chunk_channels(d.dtype) != 0 || d.IC <= 0 || d.OC <= 0) return false;
  const bool geo = (d.KH == 3 && d.KW == 3 && d.sH == d.sW && (d.sH == 1 || d.sH == 2));
  if (!geo) return false;
  const int es = d.dtype == WGX_FLOAT32 ? 4 : 2;
  // 32-bit buffer offsets: one input image and the whole weight tensor
  if ((long long)d.IC * d.IH * d.IW * es >= (1LL << 31)) return false;
  if ((long long)d.OC * d.IC * d.KH * d.KW * es >= (1LL << 31)) return false;
  return true;
}

// The channel-last tiles of pre_form (the batched 16-bit choice) run on
// weights pre-ordered by a small pass into a workspace of OC * IC * 9
// elements (WGX_CONV_PRE=0: on the raw weights).
bool conv_lds_wants_prepass(const ConvLdsDesc& d, int cus) {
  if (getenv("WGX_CONV_PRE") && strcmp(getenv("WGX_CONV_PRE"), "0") == 0) return false;
  if (!conv_lds_applies(d) || d.dtype == WGX_FLOAT32 || d.KH != 3 || d.KW != 3) return false;
  return pre_form(choose(d, cus), d.sH);
}

hipError_t launch_conv_lds(const ConvLdsDesc& d, int cus, hipStream_t s, std::string* name) {
  if (!conv_lds_applies(d)) return hipErrorNotSupported;
  Cfg c = choose(d, cus);
  if (c.tm == 0) return hipErrorInvalidValue;  // the caller takes another kernel
  const bool pre = d.wpre && pre_form(c, d.sH);
  c.rv = use_rv(d, c);
  if (!(pre && c.rv && c.tm == 2 && c.tn == 2)) c.cw = 8;
  CParams p = make_params(d, c);
  if (pre && c.rv && c.w == 1) {
    // the output-channel tiles of one pixel tile share its patch, in blocks
    // of the largest of 4, 3, 2 waves that divides their count
    // (WGX_CONV_SHARE=0: a patch per wave)
    const char* e = getenv("WGX_CONV_SHARE");
    if (!(e && strcmp(e, "0") == 0))
      for (int g = 4; g >= 2; --g)
        if (p.tiles_m % g == 0) {
          p.share = g;
          p.ntiles /= g;
          break;
        }
  }
  if (name) {
    char buf[96];
    snprintf(buf, sizeof buf, "conv_%s_%s_%dx%ds%d_%dx%dw%d%s%s", c.cl ? "cl" : "lds",
             d.dtype == WGX_FLOAT32 ? "f32" : (d.dtype == WGX_BFLOAT16 ? "bf16" : "f16"), d.KH, d.KW, d.sH,
             32 * c.tm, 32 * c.tn, c.w, c.cw == 16 ? "c16" : "", pre ? "_pre" : "");
    *name = buf;
  }
  if (p.ntiles == 0) return hipSuccess;
  const unsigned grid = (unsigned)p.ntiles;
  if (pre) {
    if (d.dtype == WGX_BFLOAT16) return launch_pre_dt<WGX_BFLOAT16>(p, c, d.sH, d.w, d.wpre, grid, s);
    return launch_pre_dt<WGX_FLOAT16>(p, c, d.sH, d.w, d.wpre, grid, s);
  }
  if (d.dtype == WGX_FLOAT32) return launch_dt<WGX_FLOAT32>(p, c, d.sH, grid, s);
  if (d.dtype == WGX_BFLOAT16) return launch_dt<WGX_BFLOAT16>(p, c, d.sH, grid, s);
  return launch_dt<WGX_FLOAT16>(p, c, d.sH, grid, s);
}

// Two independent float32 convolutions that both take the batch-1 32 x 64
// configuration, in one launch of 4-wave blocks (k_conv_lds_pair; the part
// with more input channels on 32 x 32 tiles); the partial sums of a tile are
// added in the order of its 4 waves.  Not
// supported (hipErrorNotSupported, nothing launched) for anything else, with
// a forced configuration (WGX_CONV_LDS) or with WGX_MERGE=0.
hipError_t launch_conv_lds_pair(const ConvLdsDesc& a, const ConvLdsDesc& b, int cus, hipStream_t s) {
  const char* m = getenv("WGX_MERGE");
  if ((m && strcmp(m, "0") == 0) || getenv("WGX_CONV_LDS")) return hipErrorNotSupported;
  if (a.dtype != WGX_FLOAT32 || b.dtype != WGX_FLOAT32 || !conv_lds_applies(a) || !conv_lds_applies(b))
    return hipErrorNotSupported;
  Cfg ca = choose(a, cus), cb = choose(b, cus);
  if (ca.tm != 1 || ca.tn != 2 || cb.tm != 1 || cb.tn != 2) return hipErrorNotSupported;
  // 4 waves per block for both (headline step, paired: 32 us at 4 waves,
  // 40 at 2, 55 at 1; 35.5 us as two launches)
  ca.w = cb.w = 4;
  // the part with more input channels (more chunks per wave) on 32 x 32
  // tiles, so its blocks carry about the other part's work and the CUs finish
  // together (headline step 26.0 -> 25.4 us)
  if (b.IC > a.IC)
    cb.tn = 1;
  else if (a.IC > b.IC)
    ca.tn = 1;
  ca.rv = use_rv(a, ca);
  cb.rv = use_rv(b, cb);
  const CParams pa = make_params(a, ca), pb = make_params(b, cb);
  if (pa.ntiles == 0 || pb.ntiles == 0 || (long long)pa.ntiles + pb.ntiles >= (1LL << 31)) return hipErrorNotSupported;
  if (is_dry(s)) return hipSuccess;
  if (ca.tn == 1) {
    if (a.sH == 1)
      return ca.rv ? launch_pair_b<1, true, 1>(pa, pb, b.sH, cb.rv, cb.tn, s)
                   : launch_pair_b<1, false, 1>(pa, pb, b.sH, cb.rv, cb.tn, s);
    return ca.rv ? launch_pair_b<2, true, 1>(pa, pb, b.sH, cb.rv, cb.tn, s)
                 : launch_pair_b<2, false, 1>(pa, pb, b.sH, cb.rv, cb.tn, s);
  }
  if (a.sH == 1)
    return ca.rv ? launch_pair_b<1, true, 2>(pa, pb, b.sH, cb.rv, cb.tn, s)
                 : launch_pair_b<1, false, 2>(pa, pb, b.sH, cb.rv, cb.tn, s);
  return ca.rv ? launch_pair_b<2, true, 2>(pa, pb, b.sH, cb.rv, cb.tn, s)
               : launch_pair_b<2, false, 2>(pa, pb, b.sH, cb.rv, cb.tn, s);
}

}  // namespace wgx
