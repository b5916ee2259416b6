// gemm_mfma.hip -- fp16 / bf16 GEMM and implicit-im2col convolution on gfx950
// matrix cores (v_mfma_f32_32x32x16_{f16,bf16}), fp32 accumulation.
//
// Serves aten.mm / aten.addmm / aten.bmm (src/shaders/mm/index.ts:32-93,
// src/shaders/bmm/index.ts:27-96) and the groups == 1 branch of
// aten.convolution (src/shaders/convolution/index.ts:171-238: 1x1 and dense
// KxK, any stride / padding / dilation) for float16 and bfloat16.
//
// Block: 256 threads = 4 wave64s in a 2x2 layout; block tile BM x BN, K tile
// BK = 64.  Each wave owns a (BM/2) x (BN/2) sub-tile made of 32x32 MFMA
// tiles.  A and B tiles are staged in LDS k-contiguous ([row][k], 144-byte
// row pitch: 16 B of padding keeps the 16-byte fragment reads and writes free
// of bank conflicts), double-buffered: the global loads of tile t+1 are in
// flight while tile t is multiplied, one barrier per K tile.
//
// B operand forms (see internal.h):
//   B_NK   16-byte vector loads of k-contiguous rows (W^T / nn.Linear layout).
//   B_KN   n-contiguous rows: each lane owns one column n and a run of k,
//          issues 2-byte loads that are coalesced across lanes, packs them
//          and writes 16-byte k-runs into LDS (the transpose happens in the
//          register file, nothing is materialised).
//   B_CONV implicit im2col of an NCHW input, same lane mapping as B_KN.  The
//          (ic, kh, kw) decode of every k is a per-launch table {offset, tap}
//          read with scalar loads (the k run is wave-uniform); each lane
//          holds its output pixel's base offset and a 64-bit mask of the
//          kernel taps that land inside the image, so padding costs one bit
//          test and out-of-image taps are never loaded.
// Epilogue: alpha*acc + beta*bias (per column for addmm, per row for conv),
// optional clamp (conv_with_clamp), one rounding to the storage type, staged
// through LDS so every lane stores 16 contiguous bytes.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

#include "internal.h"

namespace wgx {
namespace {

using f32x16 = float __attribute__((ext_vector_type(16)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));

constexpr int BK = 64;
constexpr int RS = BK + 8;  // LDS row pitch in 16-bit elements
constexpr int NT = 256;

struct KParams {
  const uint16_t* A;
  const uint16_t* B;
  uint16_t* C;
  const uint16_t* bias;
  const int2* ktab;
  int M, N, K;
  long long lda, ldb, ldc, sA, sB, sC;
  int bias_mode;
  float alpha, beta;
  int has_clamp;
  float cmin, cmax;
  ConvGeom g;
  int tiles_n;
};

template <bool BF>
__device__ __forceinline__ f32x16 mfma(uint4 a, uint4 b, f32x16 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool BF>
__device__ __forceinline__ float ld_f32(uint16_t h) {
  if constexpr (BF) return __uint_as_float((uint32_t)h << 16);
  else return (float)__builtin_bit_cast(_Float16, h);
}

template <bool BF>
__device__ __forceinline__ uint16_t st_bits(float v) {
  if constexpr (BF) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

template <int BM, int BN, int BMODE, bool AVEC, bool BVEC, bool BF>
__global__ __launch_bounds__(NT) void k_gemm(KParams p) {
  extern __shared__ uint4 smem_u4[];
  uint16_t* smem = reinterpret_cast<uint16_t*>(smem_u4);
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * RS;
  constexpr int CA = BM * BK / 8 / NT;  // 16-byte A chunks per thread
  constexpr int CBV = BN * BK / 8 / NT; // 16-byte B chunks per thread (B_NK)
  constexpr int KR = BK * BN / NT;      // k run per lane (B_KN / B_CONV)
  static_assert(CA >= 1 && (BMODE != B_NK || CBV >= 1), "tile too small");
  static_assert(BMODE == B_NK || (BN >= 64 && KR % 8 == 0), "column loader needs BN >= 64");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const uint16_t* __restrict__ A = p.A + (long long)blockIdx.z * p.sA;
  const uint16_t* __restrict__ Bp = p.B + (long long)blockIdx.z * p.sB;
  const int M = p.M, N = p.N, K = p.K;

  // ---------------------------------------------------------- per-lane column state
  const int nl = tid % BN;           // B_KN / B_CONV: this lane's column in the tile
  const int krun = tid / BN;         // wave-uniform since BN >= 64
  const int gn_col = n0 + nl;
  int colbase = 0;
  unsigned long long cmask = 0ull;
  if constexpr (BMODE == B_CONV) {
    if (gn_col < N) {
      const ConvGeom& g = p.g;
      const int oh = gn_col / g.OW, ow = gn_col - oh * g.OW;
      const int ih0 = oh * g.sH - g.pH, iw0 = ow * g.sW - g.pW;
      colbase = ih0 * g.IW + iw0;
      for (int kh = 0; kh < g.KH; ++kh) {
        const int ih = ih0 + kh * g.dH;
        if (ih < 0 || ih >= g.IH) continue;
        for (int kw = 0; kw < g.KW; ++kw) {
          const int iw = iw0 + kw * g.dW;
          if (iw >= 0 && iw < g.IW) cmask |= 1ull << (kh * g.KW + kw);
        }
      }
    }
  }

  // ---------------------------------------------------------- global -> registers
  uint4 ra[CA];
  uint4 rbv[BMODE == B_NK ? CBV : 1];
  uint32_t rbs[BMODE == B_NK ? 1 : KR / 2];

  auto load_rows = [&](const uint16_t* __restrict__ src, long long ld, int r0, int rlim,
                       int k0, auto vec_tag, uint4* dst, int nchunk) {
    constexpr bool VEC = decltype(vec_tag)::value;
#pragma unroll
    for (int i = 0; i < nchunk; ++i) {
      const int c = tid + i * NT;
      const int row = c >> 3, kc = c & 7;
      const int gr = r0 + row, gk = k0 + kc * 8;
      if constexpr (VEC) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (gr < rlim && gk < K) v = *reinterpret_cast<const uint4*>(src + gr * ld + gk);
        dst[i] = v;
      } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          h[e] = (gr < rlim && gk + e < K) ? (uint32_t)src[gr * ld + gk + e] : 0u;
        dst[i] = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]),
                            pack2(h[6], h[7]));
      }
    }
  };

  auto load_tile = [&](int k0) {
    load_rows(A, p.lda, m0, M, k0, std::integral_constant<bool, AVEC>{}, ra, CA);
    if constexpr (BMODE == B_NK) {
      load_rows(Bp, p.ldb, n0, N, k0, std::integral_constant<bool, BVEC>{}, rbv, CBV);
    } else if constexpr (BMODE == B_KN) {
      const int kb = k0 + krun * KR;
#pragma unroll
      for (int e = 0; e < KR; e += 2) {
        uint32_t lo = 0, hi = 0;
        if (gn_col < N) {
          if (kb + e < K) lo = Bp[(long long)(kb + e) * p.ldb + gn_col];
          if (kb + e + 1 < K) hi = Bp[(long long)(kb + e + 1) * p.ldb + gn_col];
        }
        rbs[e / 2] = pack2(lo, hi);
      }
    } else {
      const int kb = __builtin_amdgcn_readfirstlane(k0 + krun * KR);
      const int2* __restrict__ tab = p.ktab + kb;
#pragma unroll
      for (int e = 0; e < KR; e += 2) {
        const int2 t0 = tab[e], t1 = tab[e + 1];
        uint32_t lo = 0, hi = 0;
        if ((cmask >> t0.y) & 1ull) lo = Bp[colbase + t0.x];
        if ((cmask >> t1.y) & 1ull) hi = Bp[colbase + t1.x];
        rbs[e / 2] = pack2(lo, hi);
      }
    }
  };

  auto store_tile = [&](int stage) {
    uint16_t* sa = smem + stage * STAGE;
    uint16_t* sb = sa + BM * RS;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<uint4*>(sa + (c >> 3) * RS + (c & 7) * 8) = ra[i];
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < CBV; ++i) {
        const int c = tid + i * NT;
        *reinterpret_cast<uint4*>(sb + (c >> 3) * RS + (c & 7) * 8) = rbv[i];
      }
    } else {
#pragma unroll
      for (int q = 0; q < KR / 8; ++q)
        *reinterpret_cast<uint4*>(sb + nl * RS + krun * KR + q * 8) =
            make_uint4(rbs[4 * q], rbs[4 * q + 1], rbs[4 * q + 2], rbs[4 * q + 3]);
    }
  };

  // ---------------------------------------------------------- main loop
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int frow = lane & 31;
  const int fk = (lane >> 5) * 8;
  for (int t = 0; t < KT; ++t) {
    const int cur = t & 1;
    if (t + 1 < KT) load_tile((t + 1) * BK);
    const uint16_t* sa = smem + cur * STAGE;
    const uint16_t* sb = sa + BM * RS;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      uint4 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const uint4*>(sa + (wm * WM + i * 32 + frow) * RS + kk * 16 + fk);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const uint4*>(sb + (wn * WN + j * 32 + frow) * RS + kk * 16 + fk);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma<BF>(af[i], bfr[j], acc[i][j]);
    }
    if (t + 1 < KT) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------- epilogue via LDS
  constexpr int CS = BN + 8;
  static_assert(BM * CS <= 2 * STAGE, "C staging must fit in the A/B buffers");
  uint16_t* cs = smem;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // v_mfma_f32_32x32x16 result layout: lane holds column lane%32, rows
        // 8*(r/4) + 4*(lane/32) + r%4 of the 32x32 tile.
        const int row = wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = wn * WN + j * 32 + frow;
        float v = p.alpha * acc[i][j][r];
        if (p.bias_mode == BIAS_COL) {
          const int gn = n0 + col;
          if (gn < N) v += p.beta * ld_f32<BF>(p.bias[gn]);
        } else if (p.bias_mode == BIAS_ROW) {
          const int gm = m0 + row;
          if (gm < M) v += p.beta * ld_f32<BF>(p.bias[gm]);
        }
        if (p.has_clamp) v = fminf(fmaxf(v, p.cmin), p.cmax);
        cs[row * CS + col] = st_bits<BF>(v);
      }
  __syncthreads();

  uint16_t* __restrict__ C = p.C + (long long)blockIdx.z * p.sC;
  const bool cvec = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  constexpr int CC = BM * BN / 8 / NT;
#pragma unroll
  for (int i = 0; i < CC; ++i) {
    const int c = tid + i * NT;
    const int row = c / (BN / 8), cc = c % (BN / 8);
    const int gm = m0 + row, gn = n0 + cc * 8;
    if (gm >= M) continue;
    const uint16_t* srow = cs + row * CS + cc * 8;
    if (cvec && gn + 8 <= N) {
      *reinterpret_cast<uint4*>(C + gm * p.ldc + gn) = *reinterpret_cast<const uint4*>(srow);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (gn + e < N) C[gm * p.ldc + gn + e] = srow[e];
    }
  }
}

template <int BM, int BN, int BMODE, bool AVEC, bool BVEC, bool BF>
hipError_t launch_one(const KParams& kp, int batch, hipStream_t s) {
  auto fn = k_gemm<BM, BN, BMODE, AVEC, BVEC, BF>;
  const size_t lds = (size_t)2 * (BM + BN) * RS * sizeof(uint16_t);
  static bool attr_set = false;
  if (!attr_set && s != name_only()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  if (is_dry(s)) return hipSuccess;
  const int tiles_m = (kp.M + BM - 1) / BM;
  dim3 grid(tiles_m * kp.tiles_n, 1, batch);
  hipLaunchKernelGGL(fn, grid, dim3(NT), lds, s, kp);
  return hipGetLastError();
}

struct Tile {
  int bm, bn;
};

// Picks the block tile: fewest "rounds" over 256 CUs, weighted by tile area
// and a per-tile efficiency penalty for small tiles (operand reuse).
Tile choose_tile(int M, int N, int batch, bool avec, int bmode) {
  if (!avec) return {64, 64};
  static const Tile cands[] = {{256, 256}, {256, 128}, {128, 128}, {128, 64}, {64, 64}};
  const char* force = getenv("WGX_MFMA_TILE");
  if (force) {
    int bm = 0, bn = 0;
    if (sscanf(force, "%dx%d", &bm, &bn) == 2)
      for (const Tile& t : cands)
        if (t.bm == bm && t.bn == bn) return t;
  }
  double best = 1e300;
  Tile bt = {64, 64};
  for (const Tile& t : cands) {
    const long long tiles = (long long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    const double rounds = ceil((double)tiles / 256.0);
    const double eff = 1.0 + 48.0 / t.bm + 48.0 / t.bn;  // smaller tiles re-read more
    const double cost = rounds * t.bm * t.bn * eff;
    if (cost < best) {
      best = cost;
      bt = t;
    }
  }
  return bt;
}

template <int BMODE, bool AVEC, bool BVEC, bool BF>
hipError_t dispatch_tile(const Tile& t, const KParams& kp, int batch, hipStream_t s) {
  if (t.bm == 256 && t.bn == 256) return launch_one<256, 256, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 256 && t.bn == 128) return launch_one<256, 128, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 128) return launch_one<128, 128, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 64) return launch_one<128, 64, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  return launch_one<64, 64, BMODE, AVEC, BVEC, BF>(kp, batch, s);
}

}  // namespace

hipError_t launch_gemm_mfma(const GemmDesc& d, hipStream_t s, std::string* name) {
  KParams kp;
  kp.A = static_cast<const uint16_t*>(d.A);
  kp.B = static_cast<const uint16_t*>(d.B);
  kp.C = static_cast<uint16_t*>(d.C);
  kp.bias = static_cast<const uint16_t*>(d.bias);
  kp.ktab = d.ktab;
  kp.M = d.M;
  kp.N = d.N;
  kp.K = d.K;
  kp.lda = d.lda;
  kp.ldb = d.ldb;
  kp.ldc = d.ldc;
  kp.sA = d.sA;
  kp.sB = d.sB;
  kp.sC = d.sC;
  kp.bias_mode = d.bias ? d.bias_mode : BIAS_NONE;
  kp.alpha = d.alpha;
  kp.beta = d.beta;
  kp.has_clamp = d.has_clamp;
  kp.cmin = d.cmin;
  kp.cmax = d.cmax;
  kp.g = d.g;
  const bool bf = d.dtype == WGX_BFLOAT16;
  const bool avec = (d.K % 8 == 0) && (d.lda % 8 == 0) && (d.sA % 8 == 0) &&
                    ((reinterpret_cast<uintptr_t>(d.A) & 15) == 0);
  const bool bvec = (d.K % 8 == 0) && (d.ldb % 8 == 0) && (d.sB % 8 == 0) &&
                    ((reinterpret_cast<uintptr_t>(d.B) & 15) == 0);
  Tile t = choose_tile(d.M, d.N, d.batch, avec, d.bmode);
  if (d.bmode == B_NK && !bvec) t = {64, 64};
  kp.tiles_n = (d.N + t.bn - 1) / t.bn;
  if (name) {
    char buf[96];
    static const char* modes[] = {"nk", "kn", "conv"};
    snprintf(buf, sizeof buf, "gemm_mfma_%s_%dx%d_%s%s", bf ? "bf16" : "f16", t.bm, t.bn,
             modes[d.bmode], avec ? "" : "_scalarA");
    *name = buf;
  }
  if (!bf) {
    if (d.bmode == B_NK) {
      if (!bvec) return launch_one<64, 64, B_NK, false, false, false>(kp, d.batch, s);
      if (avec) return dispatch_tile<B_NK, true, true, false>(t, kp, d.batch, s);
      return launch_one<64, 64, B_NK, false, true, false>(kp, d.batch, s);
    }
    if (d.bmode == B_KN) {
      if (avec) return dispatch_tile<B_KN, true, false, false>(t, kp, d.batch, s);
      return launch_one<64, 64, B_KN, false, false, false>(kp, d.batch, s);
    }
    if (avec) return dispatch_tile<B_CONV, true, false, false>(t, kp, d.batch, s);
    return launch_one<64, 64, B_CONV, false, false, false>(kp, d.batch, s);
  }
  if (d.bmode == B_NK) {
    if (!bvec) return launch_one<64, 64, B_NK, false, false, true>(kp, d.batch, s);
    if (avec) return dispatch_tile<B_NK, true, true, true>(t, kp, d.batch, s);
    return launch_one<64, 64, B_NK, false, true, true>(kp, d.batch, s);
  }
  if (d.bmode == B_KN) {
    if (avec) return dispatch_tile<B_KN, true, false, true>(t, kp, d.batch, s);
    return launch_one<64, 64, B_KN, false, false, true>(kp, d.batch, s);
  }
  return hipErrorInvalidValue;  // bf16 convolution is not offered
}

int conv_ktab_rows(int K) { return (K + BK - 1) / BK * BK; }

void conv_fill_ktab(int2* tab, int K, int IC, const ConvGeom& g) {
  const int khw = g.KH * g.KW;
  const int rows = conv_ktab_rows(K);
  for (int k = 0; k < rows; ++k) {
    if (k < K) {
      const int ic = k / khw, tap = k % khw, kh = tap / g.KW, kw = tap % g.KW;
      tab[k].x = ic * g.IH * g.IW + kh * g.dH * g.IW + kw * g.dW;
      tab[k].y = tap;
    } else {
      tab[k].x = 0;
      tab[k].y = 63;
    }
  }
  (void)IC;
}

}  // namespace wgx
