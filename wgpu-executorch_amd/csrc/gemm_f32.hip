// gemm_f32.hip -- float32 GEMM and implicit-im2col convolution on the vector
// FMA path (v_fma_f32) with LDS blocking.
//
// Serves aten.mm / aten.addmm / aten.bmm in float32 (src/shaders/mm/
// index.ts:32-93, src/shaders/bmm/index.ts:27-96) and the groups == 1 branch of
// aten.convolution in float32 (src/shaders/convolution/index.ts:171-238).
//
// Block: 256 threads, block tile BM x BN, K tile 16, each thread a TM x TN
// register tile.  LDS holds A transposed ([k][m]) and B as [k][n] so each
// thread reads its TM rows and TN columns as contiguous vectors; two LDS
// stages, the next K tile's global loads are issued before the current tile's
// FMAs.  B forms match gemm_mfma.hip: B_NK (rows of k), B_KN (rows of n, vector
// loads), B_CONV (implicit im2col through the per-k {offset, tap} table and a
// per-lane tap mask).  Each output is accumulated in k order with fused
// multiply-adds and rounded once.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "internal.h"

namespace wgx {
namespace {

constexpr int BK = 16;
constexpr int NT = 256;

struct KParams {
  const float* A;
  const float* B;
  float* C;
  const float* bias;
  const uint32_t* ktab;
  int M, N, K;
  long long lda, ldb, ldc, sA, sB, sC;
  int bias_mode;
  float alpha, beta;
  int has_clamp;
  int act;
  float cmin, cmax;
  ConvGeom g;
  int tiles_n;
};

template <int BM, int BN, int TM, int TN, int BMODE, bool AVEC, bool BVEC>
__global__ __launch_bounds__(NT) void k_sgemm(KParams p) {
  static_assert((BM / TM) * (BN / TN) == NT, "thread layout");
  constexpr int PA = BM + 4, PB = BN + 4;
  __shared__ float sA[2][BK][PA];
  __shared__ float sB[2][BK][PB];
  extern __shared__ uint32_t ktab_lds[];  // B_CONV: the per-k table, (offset << 6) | tap
  constexpr int TX = BN / TN;
  constexpr int ACH = BM * BK / 4;  // 4-float A chunks per tile
  constexpr int BCH = BN * BK / 4;  // 4-float B chunks per tile

  const int tid = threadIdx.x;
  const int tx = tid % TX, ty = tid / TX;
  const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const float* __restrict__ A = p.A + (long long)blockIdx.z * p.sA;
  const float* __restrict__ Bp = p.B + (long long)blockIdx.z * p.sB;
  const int M = p.M, N = p.N, K = p.K;

  // B_CONV lane mapping: column nl, k run krun*KRc .. +KRc.
  constexpr int KRc = BK * BN / NT >= 1 ? BK * BN / NT : 1;
  const int nl = tid % BN, krun = tid / BN;
  const int gcol = n0 + nl;
  int colbase = 0;
  unsigned long long cmask = 0ull;
  if constexpr (BMODE == B_CONV) {
    if (gcol < N && krun * KRc < BK) {
      const ConvGeom& g = p.g;
      const int oh = gcol / g.OW, ow = gcol - oh * g.OW;
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

  constexpr int NA = (ACH + NT - 1) / NT;
  constexpr int NB = (BMODE == B_CONV) ? 1 : (BCH + NT - 1) / NT;
  float4 ra[NA];
  float4 rb[NB];
  float rc[BMODE == B_CONV ? KRc : 1];

  // rows of 4 consecutive k (A, and B in the B_NK form)
  // Loads are unconditional from clamped in-bounds addresses, zeroed after
  // with a select, so a tile's loads are all in flight together.
  auto load_krows = [&](const float* __restrict__ src, long long ld, int r0, int rlim, int k0,
                        bool vec, float4* dst, int nch, int total) {
#pragma unroll
    for (int i = 0; i < nch; ++i) {
      const int c = tid + i * NT;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (c < total) {
        const int row = c / (BK / 4), kq = c % (BK / 4);
        const int gr = r0 + row, gk = k0 + kq * 4;
        const float* s = src + (long long)(gr < rlim ? gr : rlim - 1) * ld;
        if (vec) {
          const bool ok = gr < rlim && gk < K;
          const float4 t = *reinterpret_cast<const float4*>(s + (ok ? gk : 0));
          v = ok ? t : v;
        } else {
          float t[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool ok = gr < rlim && gk + e < K;
            const float x = s[ok ? gk + e : 0];
            t[e] = ok ? x : 0.f;
          }
          v = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
      dst[i] = v;
    }
  };

  auto load_tile = [&](int k0) {
    load_krows(A, p.lda, m0, M, k0, AVEC, ra, NA, ACH);
    if constexpr (BMODE == B_NK) {
      load_krows(Bp, p.ldb, n0, N, k0, BVEC, rb, NB, BCH);
    } else if constexpr (BMODE == B_KN) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int c = tid + i * NT;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < BCH) {
          const int kr = c / (BN / 4), nq = c % (BN / 4);
          const int gk = k0 + kr, gn = n0 + nq * 4;
          const float* s = Bp + (long long)(gk < K ? gk : K - 1) * p.ldb;
          if (BVEC) {
            const bool ok = gk < K && gn < N;
            const float4 t = *reinterpret_cast<const float4*>(s + (ok ? gn : 0));
            v = ok ? t : v;
          } else {
            float t[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool ok = gk < K && gn + e < N;
              const float x = s[ok ? gn + e : 0];
              t[e] = ok ? x : 0.f;
            }
            v = make_float4(t[0], t[1], t[2], t[3]);
          }
        }
        rb[i] = v;
      }
    } else {
      const int kb = k0 + krun * KRc;
      uint32_t ent[KRc];
#pragma unroll
      for (int e = 0; e < KRc; ++e) ent[e] = ktab_lds[kb + e];
      float t[KRc];
#pragma unroll
      for (int e = 0; e < KRc; ++e) {
        const bool ok = (cmask >> (ent[e] & 63u)) & 1ull;
        t[e] = Bp[ok ? colbase + (int)(ent[e] >> 6) : 0];
      }
#pragma unroll
      for (int e = 0; e < KRc; ++e) rc[e] = ((cmask >> (ent[e] & 63u)) & 1ull) ? t[e] : 0.f;
    }
  };

  auto store_tile = [&](int st) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = tid + i * NT;
      if (c < ACH) {
        const int row = c / (BK / 4), kq = c % (BK / 4);
        sA[st][kq * 4 + 0][row] = ra[i].x;
        sA[st][kq * 4 + 1][row] = ra[i].y;
        sA[st][kq * 4 + 2][row] = ra[i].z;
        sA[st][kq * 4 + 3][row] = ra[i].w;
      }
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int c = tid + i * NT;
        if (c < BCH) {
          const int row = c / (BK / 4), kq = c % (BK / 4);
          sB[st][kq * 4 + 0][row] = rb[i].x;
          sB[st][kq * 4 + 1][row] = rb[i].y;
          sB[st][kq * 4 + 2][row] = rb[i].z;
          sB[st][kq * 4 + 3][row] = rb[i].w;
        }
      }
    } else if constexpr (BMODE == B_KN) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int c = tid + i * NT;
        if (c < BCH) {
          const int kr = c / (BN / 4), nq = c % (BN / 4);
          *reinterpret_cast<float4*>(&sB[st][kr][nq * 4]) = rb[i];
        }
      }
    } else {
      if (krun * KRc < BK) {
#pragma unroll
        for (int e = 0; e < KRc; ++e) sB[st][krun * KRc + e][nl] = rc[e];
      }
    }
  };

  float acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = 0.f;

  const int KT = (K + BK - 1) / BK;
  if constexpr (BMODE == B_CONV) {
    const int rows = (K + 63) / 64 * 64;
    for (int i = tid; i < rows; i += NT) ktab_lds[i] = p.ktab[i];
    __syncthreads();
  }
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int t = 0; t < KT; ++t) {
    const int cur = t & 1;
    if (t + 1 < KT) load_tile((t + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; i += 2) {
        const float2 v = *reinterpret_cast<const float2*>(&sA[cur][kk][ty * TM + i]);
        a[i] = v.x;
        a[i + 1] = v.y;
      }
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const float2 v = *reinterpret_cast<const float2*>(&sB[cur][kk][tx * TN + j]);
        b[j] = v.x;
        b[j + 1] = v.y;
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    if (t + 1 < KT) store_tile(cur ^ 1);
    __syncthreads();
  }

  float* __restrict__ C = p.C + (long long)blockIdx.z * p.sC;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int gm = m0 + ty * TM + i;
    if (gm >= M) continue;
    float rowb = 0.f;
    if (p.bias_mode == BIAS_ROW) rowb = p.beta * p.bias[gm];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int gn = n0 + tx * TN + j;
      if (gn >= N) continue;
      float v = p.alpha * acc[i][j] + rowb;
      if (p.bias_mode == BIAS_COL) v += p.beta * p.bias[gn];
      v = apply_act(p.act, v);
      if (p.has_clamp) v = fminf(fmaxf(v, p.cmin), p.cmax);
      C[gm * p.ldc + gn] = v;
    }
  }
}

template <int BM, int BN, int TM, int TN, int BMODE, bool AVEC, bool BVEC>
hipError_t launch_one(const KParams& kp, int batch, hipStream_t s) {
  const size_t lds = BMODE == B_CONV ? (size_t)conv_ktab_rows(kp.K) * sizeof(uint32_t) : 0;
  if (is_dry(s)) return hipSuccess;
  const int tiles_m = (kp.M + BM - 1) / BM;
  dim3 grid(tiles_m * kp.tiles_n, 1, batch);
  hipLaunchKernelGGL((k_sgemm<BM, BN, TM, TN, BMODE, AVEC, BVEC>), grid, dim3(NT), lds, s, kp);
  return hipGetLastError();
}

template <int BMODE, bool AVEC, bool BVEC>
hipError_t by_tile(int t, const KParams& kp, int batch, hipStream_t s) {
  if (t == 128) return launch_one<128, 128, 8, 8, BMODE, AVEC, BVEC>(kp, batch, s);
  if (t == 64) return launch_one<64, 64, 4, 4, BMODE, AVEC, BVEC>(kp, batch, s);
  return launch_one<32, 64, 2, 4, BMODE, AVEC, BVEC>(kp, batch, s);
}

}  // namespace

hipError_t launch_gemm_f32(const GemmDesc& d, hipStream_t s, std::string* name) {
  KParams kp;
  kp.A = static_cast<const float*>(d.A);
  kp.B = static_cast<const float*>(d.B);
  kp.C = static_cast<float*>(d.C);
  kp.bias = static_cast<const float*>(d.bias);
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
  kp.act = d.act;
  kp.cmin = d.cmin;
  kp.cmax = d.cmax;
  kp.g = d.g;
  const bool avec = (d.K % 4 == 0) && (d.lda % 4 == 0) && (d.sA % 4 == 0) &&
                    ((reinterpret_cast<uintptr_t>(d.A) & 15) == 0);
  bool bvec;
  if (d.bmode == B_NK)
    bvec = (d.K % 4 == 0) && (d.ldb % 4 == 0) && (d.sB % 4 == 0) &&
           ((reinterpret_cast<uintptr_t>(d.B) & 15) == 0);
  else
    bvec = (d.N % 4 == 0) && (d.ldb % 4 == 0) && (d.sB % 4 == 0) &&
           ((reinterpret_cast<uintptr_t>(d.B) & 15) == 0);

  // Tile: the largest of 128/64/32 rows that still gives >= 256 blocks.
  int tile = 32;
  const char* force = getenv("WGX_F32_TILE");
  if (force) {
    tile = atoi(force);
  } else {
    for (int t : {128, 64}) {
      const long long blocks =
          (long long)((d.M + t - 1) / t) * ((d.N + (t == 32 ? 64 : t) - 1) / (t == 32 ? 64 : t)) *
          d.batch;
      if (blocks >= 256) {
        tile = t;
        break;
      }
    }
  }
  if (tile != 128 && tile != 64) tile = 32;
  const int bn = tile == 32 ? 64 : tile;
  kp.tiles_n = (d.N + bn - 1) / bn;
  if (name) {
    char buf[96];
    static const char* modes[] = {"nk", "kn", "conv"};
    snprintf(buf, sizeof buf, "gemm_f32_%dx%d_%s", tile, bn, modes[d.bmode]);
    *name = buf;
  }
  if (d.bmode == B_NK) {
    if (avec && bvec) return by_tile<B_NK, true, true>(tile, kp, d.batch, s);
    return by_tile<B_NK, false, false>(tile, kp, d.batch, s);
  }
  if (d.bmode == B_KN) {
    if (avec && bvec) return by_tile<B_KN, true, true>(tile, kp, d.batch, s);
    if (avec) return by_tile<B_KN, true, false>(tile, kp, d.batch, s);
    return by_tile<B_KN, false, false>(tile, kp, d.batch, s);
  }
  if (avec) return by_tile<B_CONV, true, false>(tile, kp, d.batch, s);
  return by_tile<B_CONV, false, false>(tile, kp, d.batch, s);
}

}  // namespace wgx
