// gemm_mfma.hip -- fp16 / bf16 GEMM and implicit-im2col convolution on gfx950
// matrix cores (v_mfma_f32_32x32x16_{f16,bf16}), fp32 accumulation.
//
// Serves aten.mm / aten.addmm / aten.bmm (src/shaders/mm/index.ts:32-93,
// src/shaders/bmm/index.ts:27-96) and the groups == 1 branch of
// aten.convolution (src/shaders/convolution/index.ts:171-238: 1x1 and dense
// KxK, any stride / padding / dilation) for float16 and bfloat16.
//
// Block: WGM x WGN wave64s (4 or 8 waves); block tile BM x BN, K tile BK = 64.
// Each wave owns a (BM/WGM) x (BN/WGN) sub-tile made of 32x32 MFMA tiles (the
// large tiles run 8 waves = 2 per SIMD, each with a 64x128 sub-tile, so every
// LDS fragment feeds several MFMAs and one wave's loads overlap the other's
// MFMAs).  Tiles are assigned XCD-aware: consecutive block ids go to
// different XCDs, so each XCD gets a contiguous run of tiles that share A
// rows in its own L2.  A and B tiles are staged in LDS k-contiguous ([row][k], 144-byte
// row pitch: 16 B of padding keeps the 16-byte fragment reads and writes free
// of bank conflicts), double-buffered: the global loads of tile t+1 are in
// flight while tile t is multiplied, one barrier per K tile.
//
// B operand forms (see internal.h):
//   B_NK   16-byte vector loads of k-contiguous rows (W^T / nn.Linear layout).
//   B_KN   n-contiguous rows: each lane loads a 4(k) x 8(n) block as four
//          16-byte row segments, transposes it in registers and writes eight
//          8-byte k-runs into LDS (nothing is materialised).  Shapes whose
//          rows are not 16-byte aligned use a per-column 2-byte loader.
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

struct KParams {
  const uint16_t* A;
  const uint16_t* B;
  uint16_t* C;
  const uint16_t* bias;
  const uint32_t* ktab;
  int M, N, K;
  long long lda, ldb, ldc, sA, sB, sC;
  int bias_mode;
  float alpha, beta;
  int has_clamp;
  float cmin, cmax;
  ConvGeom g;
  int tiles_n;
  int batch;
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

// One persistent block walks tiles blockIdx', blockIdx'+G, ... (G = grid size;
// blockIdx' is the XCD-aware renumbering).  Per tile: K slices of BK = 64 go
// through two LDS stages, the global loads of slice t+1 are in flight while
// slice t is multiplied.  Before a tile's epilogue the block already issues
// the next tile's first slice, so the epilogue's output stores drain while
// the next tile starts.
//
// The MFMA is issued with the operands swapped (B fragment first): the
// accumulator then holds C^T, i.e. each lane owns 4 consecutive columns of one
// output row per register group, which the epilogue packs into 8-byte LDS
// writes before the coalesced 16-byte global stores.
template <int BM, int BN, int WGM, int WGN, int BMODE, bool AVEC, bool BVEC, bool BF>
__global__ __launch_bounds__(WGM * WGN * 64)
__attribute__((amdgpu_waves_per_eu(BM * BN <= 64 * 64 ? 4 : 2))) void k_gemm(KParams p) {
  extern __shared__ uint4 smem_u4[];
  uint16_t* smem = reinterpret_cast<uint16_t*>(smem_u4);
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * RS;
  constexpr int CA = BM * BK / 8 / NT;  // 16-byte A chunks per thread
  constexpr int CBV = BN * BK / 8 / NT; // 16-byte B chunks per thread (B_NK)
  constexpr int KR = BK * BN / NT;      // k run per lane (column loaders)
  constexpr bool KNV = BMODE == B_KN && BVEC;  // 4x8 block transpose loader
  constexpr int NKB = KNV ? 2 * BN / NT : 1;   // 4x8 blocks per thread
  constexpr int RBV = BMODE == B_NK ? CBV : (KNV ? 4 * NKB : 1);
  constexpr int RBS = (BMODE == B_NK || KNV) ? 1 : KR / 2;
  static_assert(TM >= 1 && TN >= 1 && CA >= 1 && (BMODE != B_NK || CBV >= 1), "tile too small");
  static_assert(BMODE == B_NK || KNV || (BN >= 64 && KR % 8 == 0), "column loader needs BN >= 64");
  static_assert(!KNV || (2 * BN) % NT == 0, "4x8 block loader needs 2*BN divisible by threads");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int M = p.M, N = p.N, K = p.K;
  const int KT = (K + BK - 1) / BK;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_mn = tiles_m * p.tiles_n;
  const int ntiles = tiles_mn * p.batch;
  // XCD-aware numbering: block ids are dealt round-robin to the 8 XCDs; give
  // XCD x a contiguous run of logical tiles so tiles that share A rows meet in
  // the same L2.
  const int G = gridDim.x;
  const int rb = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;

  // ------------------------------------------------ per-tile load state
  const int nl = tid % BN;    // column loaders: this lane's column in the tile
  const int krun = tid / BN;  // wave-uniform since BN >= 64
  struct LoadState {
    const uint16_t* A;
    const uint16_t* B;
    int m0, n0, gn_col, colbase;
    unsigned long long cmask;
  };
  auto tile_state = [&](int tile) {
    LoadState s;
    const int z = tile / tiles_mn, r = tile % tiles_mn;
    s.m0 = (r / p.tiles_n) * BM;
    s.n0 = (r % p.tiles_n) * BN;
    s.A = p.A + (long long)z * p.sA;
    s.B = p.B + (long long)z * p.sB;
    s.gn_col = s.n0 + nl;
    s.colbase = 0;
    s.cmask = 0ull;
    if constexpr (BMODE == B_CONV) {
      if (s.gn_col < N) {
        const ConvGeom& g = p.g;
        const int oh = s.gn_col / g.OW, ow = s.gn_col - oh * g.OW;
        const int ih0 = oh * g.sH - g.pH, iw0 = ow * g.sW - g.pW;
        s.colbase = ih0 * g.IW + iw0;
        for (int kh = 0; kh < g.KH; ++kh) {
          const int ih = ih0 + kh * g.dH;
          if (ih < 0 || ih >= g.IH) continue;
          for (int kw = 0; kw < g.KW; ++kw) {
            const int iw = iw0 + kw * g.dW;
            if (iw >= 0 && iw < g.IW) s.cmask |= 1ull << (kh * g.KW + kw);
          }
        }
      }
    }
    return s;
  };

  // ------------------------------------------------ global -> registers
  struct Regs {
    uint4 a[CA];
    uint4 bv[RBV];
    uint32_t bs[RBS];
  };
  Regs R0;

  // Every global load below is unconditional and reads an in-bounds address
  // (out-of-range rows / k are clamped, out-of-image taps read element 0);
  // the value is zeroed afterwards with a select, so all of a slice's loads
  // are in flight at once instead of each waiting behind the previous one.
  auto load_rows = [&](const uint16_t* __restrict__ src, long long ld, int r0, int rlim,
                       int k0, auto vec_tag, uint4* dst, int nchunk) {
    constexpr bool VEC = decltype(vec_tag)::value;
#pragma unroll
    for (int i = 0; i < nchunk; ++i) {
      const int c = tid + i * NT;
      const int row = c >> 3, kc = c & 7;
      const int gr = r0 + row, gk = k0 + kc * 8;
      const int grc = gr < rlim ? gr : rlim - 1;
      if constexpr (VEC) {
        const bool ok = gr < rlim && gk < K;
        const uint4 v = *reinterpret_cast<const uint4*>(src + (long long)grc * ld + (ok ? gk : 0));
        dst[i] = ok ? v : make_uint4(0, 0, 0, 0);
      } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool ok = gr < rlim && gk + e < K;
          const uint32_t v = src[(long long)grc * ld + (ok ? gk + e : 0)];
          h[e] = ok ? v : 0u;
        }
        dst[i] = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]),
                            pack2(h[6], h[7]));
      }
    }
  };

  const uint32_t* ktab_lds = reinterpret_cast<const uint32_t*>(smem + 2 * STAGE);
  auto load_slice = [&](const LoadState& st, int k0, Regs& R) {
    load_rows(st.A, p.lda, st.m0, M, k0, std::integral_constant<bool, AVEC>{}, R.a, CA);
    if constexpr (BMODE == B_NK) {
      load_rows(st.B, p.ldb, st.n0, N, k0, std::integral_constant<bool, BVEC>{}, R.bv, CBV);
    } else if constexpr (KNV) {
      // 4 k-rows x 8 columns per block, four 16-byte loads
#pragma unroll
      for (int i = 0; i < NKB; ++i) {
        const int c = tid + i * NT;
        const int kg = c & 15, ng = c >> 4;
        const int gn = st.n0 + ng * 8;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int gk = k0 + kg * 4 + j;
          const bool ok = gk < K && gn < N;
          const uint4 v = *reinterpret_cast<const uint4*>(
              st.B + (long long)(gk < K ? gk : K - 1) * p.ldb + (ok ? gn : 0));
          R.bv[4 * i + j] = ok ? v : make_uint4(0, 0, 0, 0);
        }
      }
    } else if constexpr (BMODE == B_KN) {
      const int kb = k0 + krun * KR;
      const int gnc = st.gn_col < N ? st.gn_col : N - 1;
      uint32_t v[KR];
#pragma unroll
      for (int e = 0; e < KR; ++e) {
        const int kk = kb + e < K ? kb + e : K - 1;
        v[e] = st.B[(long long)kk * p.ldb + gnc];
      }
#pragma unroll
      for (int e = 0; e < KR; e += 2) {
        const uint32_t lo = (st.gn_col < N && kb + e < K) ? v[e] : 0u;
        const uint32_t hi = (st.gn_col < N && kb + e + 1 < K) ? v[e + 1] : 0u;
        R.bs[e / 2] = pack2(lo, hi);
      }
    } else {
      // im2col: per-k entries (offset << 6) | tap, staged in LDS
      const uint32_t* tl = ktab_lds + k0 + krun * KR;
      uint32_t ent[KR];
#pragma unroll
      for (int q = 0; q < KR; q += 4) {
        const uint4 e4 = *reinterpret_cast<const uint4*>(tl + q);
        ent[q] = e4.x;
        ent[q + 1] = e4.y;
        ent[q + 2] = e4.z;
        ent[q + 3] = e4.w;
      }
      uint32_t v[KR];
#pragma unroll
      for (int e = 0; e < KR; ++e) {
        const bool ok = (st.cmask >> (ent[e] & 63u)) & 1ull;
        v[e] = st.B[ok ? st.colbase + (int)(ent[e] >> 6) : 0];
      }
#pragma unroll
      for (int e = 0; e < KR; e += 2) {
        const uint32_t lo = ((st.cmask >> (ent[e] & 63u)) & 1ull) ? v[e] : 0u;
        const uint32_t hi = ((st.cmask >> (ent[e + 1] & 63u)) & 1ull) ? v[e + 1] : 0u;
        R.bs[e / 2] = pack2(lo, hi);
      }
    }
  };

  auto store_slice = [&](int stage, const Regs& R) {
    uint16_t* sa = smem + stage * STAGE;
    uint16_t* sb = sa + BM * RS;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<uint4*>(sa + (c >> 3) * RS + (c & 7) * 8) = R.a[i];
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < CBV; ++i) {
        const int c = tid + i * NT;
        *reinterpret_cast<uint4*>(sb + (c >> 3) * RS + (c & 7) * 8) = R.bv[i];
      }
    } else if constexpr (KNV) {
      // transpose the 4x8 block: column e gets (row0[e], row1[e], row2[e], row3[e])
#pragma unroll
      for (int i = 0; i < NKB; ++i) {
        const int c = tid + i * NT;
        const int kg = c & 15, ng = c >> 4;
        const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 0]);
        const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 1]);
        const uint32_t* r2 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 2]);
        const uint32_t* r3 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 3]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = e >> 1;
          uint2 col;
          if (e & 1) {
            col.x = (r0[d] >> 16) | (r1[d] & 0xffff0000u);
            col.y = (r2[d] >> 16) | (r3[d] & 0xffff0000u);
          } else {
            col.x = (r0[d] & 0xffffu) | (r1[d] << 16);
            col.y = (r2[d] & 0xffffu) | (r3[d] << 16);
          }
          *reinterpret_cast<uint2*>(sb + (ng * 8 + e) * RS + kg * 4) = col;
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < KR / 8; ++q)
        *reinterpret_cast<uint4*>(sb + nl * RS + krun * KR + q * 8) =
            make_uint4(R.bs[4 * q], R.bs[4 * q + 1], R.bs[4 * q + 2], R.bs[4 * q + 3]);
    }
  };

  f32x16 acc[TM][TN];
  const int frow = lane & 31;
  const int fk = (lane >> 5) * 8;
  auto compute_slice = [&](int stage) {
    const uint16_t* sa = smem + stage * STAGE;
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
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma<BF>(bfr[j], af[i], acc[i][j]);
    }
  };

  if constexpr (BMODE == B_CONV) {
    uint32_t* tw = reinterpret_cast<uint32_t*>(smem + 2 * STAGE);
    for (int i = tid; i < KT * BK; i += NT) tw[i] = p.ktab[i];
    __syncthreads();
  }

  int tile = rb;
  if (tile >= ntiles) return;
  LoadState cur = tile_state(tile);
  load_slice(cur, 0, R0);

  constexpr int CS = BN + 8;
  static_assert(BM * CS <= 2 * STAGE, "C staging must fit in the A/B buffers");

  while (true) {
    __syncthreads();  // the previous tile's epilogue is done with LDS
    store_slice(0, R0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int t = 0; t < KT; ++t) {
      if (t + 1 < KT) load_slice(cur, (t + 1) * BK, R0);
      compute_slice(t & 1);
      if (t + 1 < KT) store_slice((t + 1) & 1, R0);
      __syncthreads();
    }

    // the next tile's first slice goes out before this tile's epilogue
    const int m0 = cur.m0, n0 = cur.n0;
    const int z = tile / tiles_mn;
    const int next = tile + G;
    if (next < ntiles) {
      cur = tile_state(next);
      load_slice(cur, 0, R0);
    }

    // ------------------------------------------------ epilogue via LDS
    // acc[i][j] holds C^T: lane owns row m = i*32 + lane%32 and, per register
    // group g, the 4 columns n = j*32 + 8g + 4*(lane/32) + (0..3).
    uint16_t* cs = smem;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = wm * WM + i * 32 + frow;
      const int gm = m0 + row;
      float rowb = 0.0f;
      if (p.bias_mode == BIAS_ROW && gm < M) rowb = p.beta * ld_f32<BF>(p.bias[gm]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = wn * WN + j * 32 + 8 * g + 4 * (lane >> 5);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = p.alpha * acc[i][j][4 * g + e] + rowb;
            if (p.bias_mode == BIAS_COL) {
              const int gn = n0 + col + e;
              if (gn < N) x += p.beta * ld_f32<BF>(p.bias[gn]);
            }
            if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
            v[e] = x;
          }
          *reinterpret_cast<uint2*>(cs + row * CS + col) =
              make_uint2(pack2(st_bits<BF>(v[0]), st_bits<BF>(v[1])),
                         pack2(st_bits<BF>(v[2]), st_bits<BF>(v[3])));
        }
    }
    __syncthreads();

    uint16_t* __restrict__ C = p.C + (long long)z * p.sC;
    const bool cvec = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0) &&
                      ((p.sC & 7) == 0);
    constexpr int CC = BM * BN / 8 / NT;
#pragma unroll
    for (int i = 0; i < CC; ++i) {
      const int c = tid + i * NT;
      const int row = c / (BN / 8), cc = c % (BN / 8);
      const int gm = m0 + row, gn = n0 + cc * 8;
      if (gm >= M) continue;
      const uint16_t* srow = cs + row * CS + cc * 8;
      if (cvec && gn + 8 <= N) {
        *reinterpret_cast<uint4*>(C + (long long)gm * p.ldc + gn) = *reinterpret_cast<const uint4*>(srow);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (gn + e < N) C[(long long)gm * p.ldc + gn + e] = srow[e];
      }
    }
    if (next >= ntiles) break;
    tile = next;
  }
}

int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

template <int BM, int BN, int WGM, int WGN, int BMODE, bool AVEC, bool BVEC, bool BF>
hipError_t launch_one(const KParams& kp, int batch, hipStream_t s) {
  auto fn = k_gemm<BM, BN, WGM, WGN, BMODE, AVEC, BVEC, BF>;
  const size_t stages = (size_t)2 * (BM + BN) * RS * sizeof(uint16_t);
  const size_t lds =
      stages + (BMODE == B_CONV ? (size_t)conv_ktab_rows(kp.K) * sizeof(uint32_t) : 0);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  static bool attr_set = false;
  if (!attr_set && s != name_only()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  if (is_dry(s)) return hipSuccess;
  // persistent grid: as many blocks as fit on the device at once, capped by the tile count
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                   WGM * WGN * 64, lds) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const long long ntiles = (long long)((kp.M + BM - 1) / BM) * kp.tiles_n * batch;
  long long grid = (long long)device_cus() * per_cu;
  if (grid > ntiles) grid = ntiles;
  KParams k2 = kp;
  k2.batch = batch;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WGM * WGN * 64), lds, s, k2);
  return hipGetLastError();
}

struct Tile {
  int bm, bn, wgm, wgn;
};

constexpr Tile kTiles[] = {{256, 128, 4, 2}, {128, 256, 2, 4}, {128, 128, 2, 2}, {128, 64, 2, 2},
                           {64, 64, 2, 2}};

size_t tile_lds(const Tile& t, int bmode, int K) {
  return (size_t)2 * (t.bm + t.bn) * RS * 2 + (bmode == B_CONV ? (size_t)conv_ktab_rows(K) * 4 : 0);
}

// Picks the block tile: fewest rounds over the 256 CUs (a block of 8 waves
// fills a CU, two 4-wave blocks share one), weighted by tile area and a
// per-tile efficiency penalty for small tiles (less operand reuse).
Tile choose_tile(int M, int N, int K, int batch, bool avec, int bmode) {
  if (!avec) return {64, 64, 2, 2};
  const char* force = getenv("WGX_MFMA_TILE");
  if (force) {
    int bm = 0, bn = 0;
    if (sscanf(force, "%dx%d", &bm, &bn) == 2)
      for (const Tile& t : kTiles)
        if (t.bm == bm && t.bn == bn && tile_lds(t, bmode, K) <= 160 * 1024) return t;
  }
  double best = 1e300;
  Tile bt = {64, 64, 2, 2};
  for (const Tile& t : kTiles) {
    if (tile_lds(t, bmode, K) > 160 * 1024) continue;
    const long long tiles = (long long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    const int per_cu = t.wgm * t.wgn == 8 ? 1 : 2;
    const double rounds = ceil((double)tiles / (256.0 * per_cu));
    const double eff = 1.0 + 64.0 / t.bm + 64.0 / t.bn;
    const double cost = rounds * t.bm * t.bn * per_cu * eff;
    if (cost < best) {
      best = cost;
      bt = t;
    }
  }
  return bt;
}

template <int BMODE, bool AVEC, bool BVEC, bool BF>
hipError_t dispatch_tile(const Tile& t, const KParams& kp, int batch, hipStream_t s) {
  // the 4x8 KN block loader needs 2*BN divisible by the thread count
  constexpr bool KN = BMODE == B_KN;
  if (t.bm == 256 && t.bn == 128) return launch_one<256, 128, 4, 2, BMODE, AVEC, (KN ? false : BVEC), BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 256) return launch_one<128, 256, 2, 4, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 128) return launch_one<128, 128, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 64) return launch_one<128, 64, 2, 2, BMODE, AVEC, (KN ? false : BVEC), BF>(kp, batch, s);
  return launch_one<64, 64, 2, 2, BMODE, AVEC, (KN ? false : BVEC), BF>(kp, batch, s);
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
  const auto aligned16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  const bool avec = (d.K % 8 == 0) && (d.lda % 8 == 0) && (d.sA % 8 == 0) && aligned16(d.A);
  bool bvec;
  if (d.bmode == B_NK)
    bvec = (d.K % 8 == 0) && (d.ldb % 8 == 0) && (d.sB % 8 == 0) && aligned16(d.B);
  else if (d.bmode == B_KN)
    bvec = (d.N % 8 == 0) && (d.ldb % 8 == 0) && (d.sB % 8 == 0) && aligned16(d.B);
  else
    bvec = false;
  Tile t = choose_tile(d.M, d.N, d.K, d.batch, avec, d.bmode);
  if (d.bmode == B_NK && !bvec) t = {64, 64, 2, 2};
  if (d.bmode == B_KN && !bvec && !(t.bm == 128 && t.bn == 128)) t = {64, 64, 2, 2};
  kp.tiles_n = (d.N + t.bn - 1) / t.bn;
  const bool knv = d.bmode == B_KN && bvec && (2 * t.bn) % (t.wgm * t.wgn * 64) == 0;
  if (name) {
    char buf[96];
    static const char* modes[] = {"nk", "kn", "conv"};
    snprintf(buf, sizeof buf, "gemm_mfma_%s_%dx%d_%s%s%s", bf ? "bf16" : "f16", t.bm, t.bn,
             modes[d.bmode], d.bmode == B_KN ? (knv ? "4x8" : "col") : "", avec ? "" : "_scalarA");
    *name = buf;
  }
  if (bf && d.bmode == B_CONV) return hipErrorInvalidValue;  // bf16 convolution is not offered
  if (!avec) {
    if (d.bmode == B_NK)
      return bf ? (bvec ? launch_one<64, 64, 2, 2, B_NK, false, true, true>(kp, d.batch, s)
                        : launch_one<64, 64, 2, 2, B_NK, false, false, true>(kp, d.batch, s))
                : (bvec ? launch_one<64, 64, 2, 2, B_NK, false, true, false>(kp, d.batch, s)
                        : launch_one<64, 64, 2, 2, B_NK, false, false, false>(kp, d.batch, s));
    if (d.bmode == B_KN)
      return bf ? launch_one<64, 64, 2, 2, B_KN, false, false, true>(kp, d.batch, s)
                : launch_one<64, 64, 2, 2, B_KN, false, false, false>(kp, d.batch, s);
    return launch_one<64, 64, 2, 2, B_CONV, false, false, false>(kp, d.batch, s);
  }
  if (d.bmode == B_NK) {
    if (!bvec)
      return bf ? launch_one<64, 64, 2, 2, B_NK, true, false, true>(kp, d.batch, s)
                : launch_one<64, 64, 2, 2, B_NK, true, false, false>(kp, d.batch, s);
    return bf ? dispatch_tile<B_NK, true, true, true>(t, kp, d.batch, s)
              : dispatch_tile<B_NK, true, true, false>(t, kp, d.batch, s);
  }
  if (d.bmode == B_KN) {
    if (!bvec) {
      if (t.bm == 128)
        return bf ? launch_one<128, 128, 2, 2, B_KN, true, false, true>(kp, d.batch, s)
                  : launch_one<128, 128, 2, 2, B_KN, true, false, false>(kp, d.batch, s);
      return bf ? launch_one<64, 64, 2, 2, B_KN, true, false, true>(kp, d.batch, s)
                : launch_one<64, 64, 2, 2, B_KN, true, false, false>(kp, d.batch, s);
    }
    return bf ? dispatch_tile<B_KN, true, true, true>(t, kp, d.batch, s)
              : dispatch_tile<B_KN, true, true, false>(t, kp, d.batch, s);
  }
  return dispatch_tile<B_CONV, true, false, false>(t, kp, d.batch, s);
}

int conv_ktab_rows(int K) { return (K + BK - 1) / BK * BK; }

void conv_fill_ktab(uint32_t* tab, int K, int IC, const ConvGeom& g) {
  const int khw = g.KH * g.KW;
  const int rows = conv_ktab_rows(K);
  for (int k = 0; k < rows; ++k) {
    if (k < K) {
      const int ic = k / khw, tap = k % khw, kh = tap / g.KW, kw = tap % g.KW;
      const uint32_t off = (uint32_t)(ic * g.IH * g.IW + kh * g.dH * g.IW + kw * g.dW);
      tab[k] = (off << 6) | (uint32_t)tap;
    } else {
      tab[k] = 63u;  // tap 63 is never inside the image (KH*KW <= 63)
    }
  }
  (void)IC;
}

bool conv_ktab_fits(int K, int IC, const ConvGeom& g) {
  const long long maxoff = (long long)IC * g.IH * g.IW + (long long)g.KH * g.dH * g.IW + (long long)g.KW * g.dW;
  return g.KH * g.KW <= 63 && maxoff < (1LL << 26) && (long long)conv_ktab_rows(K) * 4 <= 32 * 1024;
}

}  // namespace wgx
