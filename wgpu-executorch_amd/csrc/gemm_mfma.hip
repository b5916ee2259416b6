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
#include <string.h>

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
  int act;
  float cmin, cmax;
  ConvGeom g;
  int tiles_n;
  int gm;            // m-tiles per group of the tile order
  uint32_t b_bytes;  // B_CONV: bytes of one input image
  int batch;
  int splits, kchunk;  // split-K: K ranges per tile, K slices per range
  float* ws;           // split-K partial sums, [splits][batch][M][N]
  int nt_store;        // large-tile kernel: non-temporal output stores
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

// Buffer descriptors for raw buffer loads (word 3 = 0x00020000: the gfx9
// raw-buffer format).  An offset at or past the range reads as zero.
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr uint32_t OOB = 0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 ld_b128(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t ld_b16(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ void st_b128(uint4 v, rsrc_t r, uint32_t off) {
  using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
  const u32x4 d = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(d, r, (int)off, 0, 0);
}
__device__ __forceinline__ void st_b16(uint32_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b16((unsigned short)v, r, (int)off, 0, 0);
}

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
__attribute__((amdgpu_waves_per_eu((BM / WGM / 32) * (BN / WGN / 32) >= 8 ? 1 : 2))) void k_gemm(KParams p) {
  extern __shared__ uint4 smem_u4[];
  uint16_t* smem = reinterpret_cast<uint16_t*>(smem_u4);
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * RS;
  constexpr int BMAX = BM > BN ? BM : BN;  // bias floats parked in LDS
  constexpr int CA = BM * BK / 8 / NT;  // 16-byte A chunks per thread
  constexpr int CBV = BN * BK / 8 / NT; // 16-byte B chunks per thread (B_NK)
  constexpr int KR = BK * BN / NT;      // k run per lane (column loaders)
  constexpr bool KNV = BMODE == B_KN && BVEC;  // 4x8 block transpose loader
  constexpr int NKB = KNV ? (2 * BN + NT - 1) / NT : 1;  // 4x8 blocks per thread
  constexpr int RBV = BMODE == B_NK ? CBV : (KNV ? 4 * NKB : 1);
  constexpr int RBS = (BMODE == B_NK || KNV) ? 1 : KR / 2;
  static_assert(TM >= 1 && TN >= 1 && CA >= 1 && (BMODE != B_NK || CBV >= 1), "tile too small");
  static_assert(BMODE == B_NK || KNV || (BN >= 64 && KR % 8 == 0), "column loader needs BN >= 64");
  static_assert(!KNV || (2 * BN) % 64 == 0, "4x8 block loader keeps whole waves busy or idle");

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
  // Operands are read with raw buffer loads.  Each tile gets buffer
  // descriptors whose range ends where the operand's valid data ends, and a
  // masked element (k or n past the edge, an out-of-image tap) is given the
  // offset OOB, which the hardware range check turns into a zero.  So every
  // load is unconditional and branch-free, and the loads of a slice are all
  // in flight together.
  struct LoadState {
    rsrc_t ra, rb;
    int m0, n0, z, gn_col, colbase;
    unsigned long long cmask;
    uint32_t bias_h;  // this thread's bias element of the tile (raw bits)
  };
  auto tile_state = [&](int tile) {
    LoadState s;
    // grouped order: p.gm m-tiles walked first, then n, so a run of
    // consecutive tiles (one XCD's share) covers a compact rectangle
    const int z = tile / tiles_mn, r = tile % tiles_mn;
    const int gsz = p.gm * p.tiles_n;
    const int grp = r / gsz, rr = r - grp * gsz;
    const int gmh = min(p.gm, tiles_m - grp * p.gm);
    s.m0 = (grp * p.gm + rr % gmh) * BM;
    s.n0 = (rr / gmh) * BN;
    s.z = z;
    const int mrows = min(BM, M - s.m0);
    s.ra = make_rsrc(p.A + (long long)z * p.sA + (long long)s.m0 * p.lda,
                     (uint32_t)((mrows - 1) * p.lda + K) * 2u);
    if constexpr (BMODE == B_NK) {
      const int nrows = min(BN, N - s.n0);
      s.rb = make_rsrc(p.B + (long long)z * p.sB + (long long)s.n0 * p.ldb,
                       (uint32_t)((nrows - 1) * p.ldb + K) * 2u);
    } else if constexpr (BMODE == B_CONV) {
      s.rb = make_rsrc(p.B + (long long)z * p.sB, p.b_bytes);
    } else {
      s.rb = make_rsrc(p.B, 0u);  // B_KN: rebuilt per slice (see load_slice)
    }
    // bias: thread t < BN (per column) or < BM (per row) fetches element t
    // of the tile; it is parked in LDS when the tile starts
    s.bias_h = 0u;
    if (p.bias_mode != BIAS_NONE) {
      const bool col = p.bias_mode == BIAS_COL;
      const int lim = col ? N : M, b0 = col ? s.n0 : s.m0, cnt = col ? BN : BM;
      const rsrc_t rbias = make_rsrc(p.bias, (uint32_t)lim * 2u);
      s.bias_h = ld_b16(rbias, (tid < cnt && b0 + tid < lim) ? (uint32_t)(b0 + tid) * 2u : OOB);
    }
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

  // k-contiguous rows (A, and B in the B_NK form): 8 lanes cover one row's
  // 64 k of the slice; rows past the tile's valid rows fall outside the
  // descriptor's range.
  auto load_rows = [&](rsrc_t rs, long long ld, int k0, auto vec_tag, uint4* dst, int nchunk) {
    constexpr bool VEC = decltype(vec_tag)::value;
#pragma unroll
    for (int i = 0; i < nchunk; ++i) {
      const int c = tid + i * NT;
      const int row = c >> 3, kc = c & 7;
      const int gk = k0 + kc * 8;
      const uint32_t base = (uint32_t)(row * ld + gk) * 2u;
      if constexpr (VEC) {
        dst[i] = ld_b128(rs, gk < K ? base : OOB);
      } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = ld_b16(rs, gk + e < K ? base + 2u * e : OOB);
        dst[i] = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]),
                            pack2(h[6], h[7]));
      }
    }
  };

  float* bias_lds = reinterpret_cast<float*>(smem + 2 * STAGE);
  const uint32_t* ktab_lds = reinterpret_cast<const uint32_t*>(smem + 2 * STAGE + 2 * BMAX);
  auto load_slice = [&](const LoadState& st, int k0, Regs& R) {
    load_rows(st.ra, p.lda, k0, std::integral_constant<bool, AVEC>{}, R.a, CA);
    if constexpr (BMODE == B_NK) {
      load_rows(st.rb, p.ldb, k0, std::integral_constant<bool, BVEC>{}, R.bv, CBV);
    } else if constexpr (BMODE == B_KN) {
      // rows of n: the descriptor starts at (k0, n0) and ends after the last
      // valid element of the slice's last valid row
      const int krows = min(BK, K - k0);  // <= 0 past K: every load reads zero
      const int kb0 = krows > 0 ? k0 : 0;
      const rsrc_t rs = make_rsrc(p.B + (long long)st.z * p.sB + (long long)kb0 * p.ldb + st.n0,
                                  krows > 0 ? (uint32_t)((krows - 1) * p.ldb + (N - st.n0)) * 2u : 0u);
      if constexpr (KNV) {
        // 4 k-rows x 8 columns per block, four 16-byte loads
#pragma unroll
        for (int i = 0; i < NKB; ++i) {
          const int c = tid + i * NT;
          if (2 * BN % NT != 0 && c >= 2 * BN) break;  // wave-uniform
          const int kg = c & 15, ng = c >> 4;
          const bool nok = st.n0 + ng * 8 < N;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int kr = kg * 4 + j;
            R.bv[4 * i + j] = ld_b128(rs, (nok && kr < krows) ? (uint32_t)(kr * p.ldb + ng * 8) * 2u : OOB);
          }
        }
      } else {
        const int kb = krun * KR;
        const bool nok = st.gn_col < N;
        uint32_t v[KR];
#pragma unroll
        for (int e = 0; e < KR; ++e)
          v[e] = ld_b16(rs, (nok && kb + e < krows) ? (uint32_t)((kb + e) * p.ldb + nl) * 2u : OOB);
#pragma unroll
        for (int e = 0; e < KR; e += 2) R.bs[e / 2] = pack2(v[e], v[e + 1]);
      }
    } else {
      // im2col: per-k entries (offset << 6) | tap, staged in LDS; a slice
      // past K reads the first table rows and masks every tap
      const bool live = k0 < K;
      const unsigned long long lmask = live ? st.cmask : 0ull;
      const uint32_t* tl = ktab_lds + (live ? k0 : 0) + krun * KR;
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
        const bool ok = (lmask >> (ent[e] & 63u)) & 1ull;
        v[e] = ld_b16(st.rb, ok ? (uint32_t)(st.colbase + (int)(ent[e] >> 6)) * 2u : OOB);
      }
#pragma unroll
      for (int e = 0; e < KR; e += 2) R.bs[e / 2] = pack2(v[e], v[e + 1]);
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
        if (2 * BN % NT != 0 && c >= 2 * BN) break;  // wave-uniform
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
  // Fragments are software-pipelined: the LDS reads for k step kk+1 are
  // issued before the MFMAs of step kk, so their latency hides behind them.
  auto compute_slice = [&](int stage) {
    const uint16_t* sa = smem + stage * STAGE;
    const uint16_t* sb = sa + BM * RS;
    uint4 af[2][TM], bfr[2][TN];
    auto frags = [&](int kk, uint4* a, uint4* b) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const uint4*>(sa + (wm * WM + i * 32 + frow) * RS + kk * 16 + fk);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const uint4*>(sb + (wn * WN + j * 32 + frow) * RS + kk * 16 + fk);
    };
    frags(0, af[0], bfr[0]);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) frags(kk + 1, af[(kk + 1) & 1], bfr[(kk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma<BF>(bfr[kk & 1][j], af[kk & 1][i], acc[i][j]);
    }
  };

  if constexpr (BMODE == B_CONV) {
    uint32_t* tw = reinterpret_cast<uint32_t*>(smem + 2 * STAGE + 2 * BMAX);
    for (int i = tid; i < KT * BK; i += NT) tw[i] = p.ktab[i];
    __syncthreads();
  }

  // Slice s of a tile lives in register set R[s % 2] between its global
  // load and its LDS store: the loads run two K slices ahead of the MFMAs.
  Regs R1;
  int tile = rb;
  if (tile >= ntiles) return;
  LoadState cur = tile_state(tile);
  load_slice(cur, 0, R0);
  load_slice(cur, BK, R1);

  constexpr int CS = BN + 8;
  static_assert(BM * CS <= 2 * STAGE, "C staging must fit in the A/B buffers");

  // One K step: slice t+1 (held in Rn) goes to LDS, slice t+3 is requested
  // into the freed registers, slice t is multiplied.  The stage written here
  // was last read in step t-1, which ended with a barrier.  Nothing in a
  // step is conditional: a slice at or past K loads as zeros (its offsets are
  // out of range), so the compiler can count outstanding loads exactly and
  // wait only for the slice being stored.
  auto step = [&](int t, Regs& Rn) {
    store_slice((t + 1) & 1, Rn);
    load_slice(cur, (t + 3) * BK, Rn);
    compute_slice(t & 1);
#ifdef WGX_INTERLEAVE
    // Spread the slice's LDS writes and global loads between its MFMAs
    // (they were issued first in program order) so the matrix pipe keeps
    // being fed while they go out.
#pragma unroll
    for (int q = 0; q < TM * TN * (BK / 16); ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // one LDS write
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
    }
#endif
    __syncthreads();
  };

  while (true) {
    __syncthreads();  // the previous tile's epilogue is done with LDS
    store_slice(0, R0);
    if (p.bias_mode != BIAS_NONE && tid < BMAX) bias_lds[tid] = p.beta * ld_f32<BF>((uint16_t)cur.bias_h);
    load_slice(cur, 2 * BK, R0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    __syncthreads();

    // slice s is held in R[s % 2]
    if (KT & 1) {
      step(0, R1);
      for (int t = 1; t < KT; t += 2) {
        step(t, R0);
        step(t + 1, R1);
      }
    } else {
      for (int t = 0; t < KT; t += 2) {
        step(t, R1);
        step(t + 1, R0);
      }
    }

    // the next tile's first two slices go out before this tile's epilogue
    const int m0 = cur.m0, n0 = cur.n0;
    const int z = tile / tiles_mn;
    const int next = tile + G;
    if (next < ntiles) {
      cur = tile_state(next);
      load_slice(cur, 0, R0);
      load_slice(cur, BK, R1);
    }

    // ------------------------------------------------ epilogue via LDS
    // acc[i][j] holds C^T: lane owns row m = i*32 + lane%32 and, per register
    // group g, the 4 columns n = j*32 + 8g + 4*(lane/32) + (0..3).
    uint16_t* cs = smem;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = wm * WM + i * 32 + frow;
      const float rowb = p.bias_mode == BIAS_ROW ? bias_lds[row] : 0.0f;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = wn * WN + j * 32 + 8 * g + 4 * (lane >> 5);
          float4 bc = make_float4(0.f, 0.f, 0.f, 0.f);
          if (p.bias_mode == BIAS_COL) bc = *reinterpret_cast<const float4*>(bias_lds + col);
          const float bb[4] = {bc.x, bc.y, bc.z, bc.w};
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = p.alpha * acc[i][j][4 * g + e] + rowb + bb[e];
            x = apply_act(p.act, x);
            if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
            v[e] = x;
          }
          *reinterpret_cast<uint2*>(cs + row * CS + col) =
              make_uint2(pack2(st_bits<BF>(v[0]), st_bits<BF>(v[1])),
                         pack2(st_bits<BF>(v[2]), st_bits<BF>(v[3])));
        }
    }
    __syncthreads();

    // Stores through a descriptor whose range ends after the tile's last valid
    // row; columns past N get the offset OOB, which the hardware drops.
    const int mrows = min(BM, M - m0);
    const rsrc_t rc = make_rsrc(p.C + (long long)z * p.sC + (long long)m0 * p.ldc + n0,
                                (uint32_t)((mrows - 1) * p.ldc + (N - n0)) * 2u);
    const bool cvec = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0) &&
                      ((p.sC & 7) == 0) && ((N & 7) == 0);
    constexpr int CC = BM * BN / 8 / NT;
#pragma unroll
    for (int i = 0; i < CC; ++i) {
      const int c = tid + i * NT;
      const int row = c / (BN / 8), cc = c % (BN / 8);
      const uint4 cv = *reinterpret_cast<const uint4*>(cs + row * CS + cc * 8);
      const int gn = n0 + cc * 8;
      const uint32_t off = (uint32_t)(row * p.ldc + cc * 8) * 2u;
      if (cvec) {
        st_b128(cv, rc, gn < N ? off : OOB);
      } else {
        const uint32_t w[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          st_b16((w[e >> 1] >> (16 * (e & 1))) & 0xffffu, rc, gn + e < N ? off + 2u * e : OOB);
      }
    }
    if (next >= ntiles) break;
    tile = next;
  }
}

// ============================================================ pipelined kernel
// The main kernel for 16-byte-aligned A.  A (and B in the B_NK form) stream
// from global memory straight into LDS with buffer_load ... lds (LDS-DMA: no
// registers in between), through three LDS stages: while slice t is
// multiplied, slices t+1 and t+2 are in flight.  Each stage is its own
// __shared__ array, so the compiler can tell that reading stage t does not
// touch the stages being filled and inserts no wait for them; the kernel
// waits explicitly (vmcnt) for exactly the slice it needs next.  B in the
// B_KN / B_CONV forms (a transpose or a gather) goes through registers, one
// slice ahead.  Tiles in LDS are [rows][64] 16-bit elements, 128-byte rows,
// with the 16-byte chunk c of row r stored at chunk c ^ (r & 7): the eight
// rows a fragment read touches per cycle then hit eight different bank
// groups.  The epilogue writes C straight from the accumulators (each lane
// owns 4 consecutive columns of a row per register group), so the next
// tile's first slices can be in flight during it.
typedef __attribute__((address_space(3))) void lds_void;

// One LDS-DMA load: 16 bytes per lane from buffer offset voff into LDS at
// lds_wave_base + 16 * lane.  Written as inline asm so the compiler does not
// track it: every wait for these loads is the explicit wait_vm<> below, and
// the compiler does not add a conservative vmcnt(0) before each LDS read.
// The "memory" clobber keeps LDS accesses from moving across it.  One wait
// state separates the M0 write from the instruction that reads M0.
__device__ __forceinline__ void dma16(rsrc_t r, const uint16_t* lds_wave_base, uint32_t voff) {
  const uint32_t la = (uint32_t)(uintptr_t)lds_wave_base;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(la), "v"(voff), "s"(r) : "memory", "m0");
}
// The same with the slice's k offset in the instruction's scalar offset, so a
// lane's vector offset stays fixed for a whole tile (no per-slice VALU work).
__device__ __forceinline__ void dma16s(rsrc_t r, const void* lds_wave_base, uint32_t voff, uint32_t soff) {
  const uint32_t la = (uint32_t)(uintptr_t)lds_wave_base;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(la), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
__device__ __forceinline__ void st_b64(uint2 v, rsrc_t r, uint32_t off) {
  using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
  const u32x2 d = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(d, r, (int)off, 0, 0);
}
// s_waitcnt vmcnt(n) with lgkmcnt / expcnt left unconstrained (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}
// gfx950 LDS serves a 128-bit read 16 lanes (256 bytes, 64 banks) at a time;
// 16 consecutive rows are 8 row pairs sharing a 256-byte bank period, so the
// swizzle keys on the pair index: chunk c of row r is stored at c ^ ((r/2) % 8).
// Returns a byte offset into a [rows][128 B] tile.
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Element types of the pipelined kernel.
enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

__device__ __forceinline__ uint32_t ld_b32(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ void st_b32(uint32_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, (int)off, 0, 0);
}

template <int DT>
__device__ __forceinline__ float to_f32(uint32_t bits) {
  if constexpr (DT == DT_F32) return __uint_as_float(bits);
  else if constexpr (DT == DT_BF16) return __uint_as_float(bits << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// One 16-byte fragment pair's worth of MFMAs: for 16-bit types one
// v_mfma_f32_32x32x16 (8 k per lane); for fp32 four v_mfma_f32_32x32x2_f32,
// component e of each lane's 4 consecutive k.  A and B fragments use the same
// lane->k mapping, so any pairing of k across the four is a valid sum.
template <int DT>
__device__ __forceinline__ f32x16 mfma_frag(uint4 b, uint4 a, f32x16 c) {
  if constexpr (DT == DT_F32) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.x), __uint_as_float(a.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.y), __uint_as_float(a.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.z), __uint_as_float(a.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b.w), __uint_as_float(a.w), c, 0, 0, 0);
    return c;
  } else {
    return mfma<DT == DT_BF16>(b, a, c);
  }
}

template <int BM, int BN, int WGM, int WGN, int BMODE, bool BVEC, int DT, int NS>
__global__ __launch_bounds__(WGM * WGN * 64)
__attribute__((amdgpu_waves_per_eu((BM / WGM / 32) * (BN / WGN / 32) >= 8 ? 1 : 2))) void k_gemm3(KParams p) {
  constexpr int NT = WGM * WGN * 64, NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int ES = DT == DT_F32 ? 4 : 2;  // element bytes
  constexpr int EPC = 16 / ES;              // elements per 16-byte chunk
  constexpr int BK = 128 / ES;              // k per slice: one 128-byte row
  constexpr int BMAX = BM > BN ? BM : BN;
  constexpr bool BDMA = BMODE == B_NK;
  constexpr int CHA = BM * 8 / NT;             // A: DMA instructions per thread per slice
  constexpr int CHB = BDMA ? BN * 8 / NT : 0;  // B (B_NK): same
  constexpr int DMAS = CHA + CHB;              // DMA loads per thread per slice
  constexpr bool KNV = BMODE == B_KN && BVEC;
  constexpr int KGS = BK / 4;                  // 4-k groups per slice (transpose loader)
  constexpr int NKB = KNV ? (2 * BN + NT - 1) / NT : 1;  // 4 k x EPC n blocks per thread
  constexpr int KR = BK * BN / NT;             // column loaders (B_KN scalar / B_CONV)
  constexpr int RBV = KNV ? 4 * NKB : 1;
  constexpr int RBS = (BDMA || KNV) ? 1 : KR;
  static_assert(TM >= 1 && TN >= 1 && CHA >= 1 && (BM * 8) % NT == 0, "tile shape");
  static_assert(!BDMA || (BN * 8) % NT == 0, "B tile shape");
  static_assert(BDMA || KNV || (BN >= 64 && KR % EPC == 0), "column loader needs BN >= 64");
  static_assert(NS == 3 || NS == 4, "stages");
  static_assert((NS - 2) * DMAS < 64, "vmcnt");

  __shared__ __attribute__((aligned(1024))) uint16_t sA0[BM * 64], sA1[BM * 64], sA2[BM * 64];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[BN * 64], sB1[BN * 64], sB2[BN * 64];
  __shared__ __attribute__((aligned(1024))) uint16_t sA3[NS > 3 ? BM * 64 : 8], sB3[NS > 3 ? BN * 64 : 8];
  __shared__ __attribute__((aligned(16))) float sbias[2][BMAX];
  extern __shared__ uint32_t ktab_lds[];  // B_CONV: per-k (offset << 6) | tap

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int M = p.M, N = p.N, K = p.K;
  const int KT = (K + BK - 1) / BK;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_mn = tiles_m * p.tiles_n;
  const int ntiles = tiles_mn * p.batch;
  const int S = p.splits;      // K ranges per tile (split-K)
  const int nunits = ntiles * S;
  const int G = gridDim.x;
  const int rb = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const char* Ab = reinterpret_cast<const char*>(p.A);
  const char* Bb = reinterpret_cast<const char*>(p.B);
  char* Cb = reinterpret_cast<char*>(p.C);

  if constexpr (BMODE == B_CONV) {
    for (int i = tid; i < KT * BK; i += NT) ktab_lds[i] = p.ktab[i];
    __syncthreads();
  }

  auto stA = [&](auto s) -> char* {
    if constexpr (decltype(s)::value == 0) return reinterpret_cast<char*>(sA0);
    else if constexpr (decltype(s)::value == 1) return reinterpret_cast<char*>(sA1);
    else if constexpr (decltype(s)::value == 2) return reinterpret_cast<char*>(sA2);
    else return reinterpret_cast<char*>(sA3);
  };
  auto stB = [&](auto s) -> char* {
    if constexpr (decltype(s)::value == 0) return reinterpret_cast<char*>(sB0);
    else if constexpr (decltype(s)::value == 1) return reinterpret_cast<char*>(sB1);
    else if constexpr (decltype(s)::value == 2) return reinterpret_cast<char*>(sB2);
    else return reinterpret_cast<char*>(sB3);
  };

  struct TileState {
    rsrc_t ra, rb;
    int m0, n0, z, gn_col, colbase;
    int tile, sp, kbase, kts;  // output tile, K range, its first k and slice count
    unsigned long long cmask;
    uint32_t bias_h;
    // byte offset of this lane's 16-byte DMA chunk at k = 0 (OOB for rows past
    // the operand's edge); a slice adds k0 * ES as the scalar offset
    uint32_t va[CHA], vb[CHB > 0 ? CHB : 1];
  };
  const int nl = tid % BN;
  const int krun = tid / BN;
  auto tile_state = [&](int unit) {
    TileState s;
    const int tile = unit / S;
    s.tile = tile;
    s.sp = unit - tile * S;
    s.kbase = s.sp * p.kchunk * BK;
    s.kts = min(p.kchunk, KT - s.sp * p.kchunk);
    const int z = tile / tiles_mn, r = tile % tiles_mn;
    const int gsz = p.gm * p.tiles_n;
    const int grp = r / gsz, rr = r - grp * gsz;
    const int gmh = min(p.gm, tiles_m - grp * p.gm);
    s.m0 = (grp * p.gm + rr % gmh) * BM;
    s.n0 = (rr / gmh) * BN;
    s.z = z;
    const int mrows = min(BM, M - s.m0);
    s.ra = make_rsrc(Ab + ((long long)z * p.sA + (long long)s.m0 * p.lda) * ES,
                     (uint32_t)((mrows - 1) * p.lda + K) * ES);
    if constexpr (BMODE == B_NK) {
      const int nrows = min(BN, N - s.n0);
      s.rb = make_rsrc(Bb + ((long long)z * p.sB + (long long)s.n0 * p.ldb) * ES,
                       (uint32_t)((nrows - 1) * p.ldb + K) * ES);
    } else if constexpr (BMODE == B_CONV) {
      s.rb = make_rsrc(Bb + (long long)z * p.sB * ES, p.b_bytes);
    } else {
      s.rb = make_rsrc(p.B, 0u);
    }
    s.bias_h = 0u;
    if (p.bias_mode != BIAS_NONE) {
      const bool col = p.bias_mode == BIAS_COL;
      const int lim = col ? N : M, b0 = col ? s.n0 : s.m0, cnt = col ? BN : BM;
      const rsrc_t rbias = make_rsrc(p.bias, (uint32_t)lim * ES);
      const uint32_t off = (tid < cnt && b0 + tid < lim) ? (uint32_t)(b0 + tid) * ES : OOB;
      s.bias_h = ES == 4 ? ld_b32(rbias, off) : ld_b16(rbias, off);
    }
#pragma unroll
    for (int i = 0; i < CHA; ++i) {
      const int row = (i * NW + wave) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ ((row >> 1) & 7);
      s.va[i] = row < mrows ? (uint32_t)(((long long)row * p.lda + chunk * EPC) * ES) : OOB;
    }
    if constexpr (BDMA) {
      const int nrows = min(BN, N - s.n0);
#pragma unroll
      for (int i = 0; i < CHB; ++i) {
        const int row = (i * NW + wave) * 8 + (lane >> 3);
        const int chunk = (lane & 7) ^ ((row >> 1) & 7);
        s.vb[i] = row < nrows ? (uint32_t)(((long long)row * p.ldb + chunk * EPC) * ES) : OOB;
      }
    }
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

  // ---------------------------------------------------------- loads
  // DMA lane mapping: instruction i of wave w fills LDS chunks
  // (i*NW + w)*64 + lane, i.e. row (i*NW + w)*8 + lane/8, stored chunk lane%8,
  // which holds logical chunk (lane%8) ^ ((row/2)%8) (see swz).
  auto dma_rows = [&](rsrc_t rs, long long ld, int k0, char* dst, auto ch_tag) {
    constexpr int CH = decltype(ch_tag)::value;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int row = (i * NW + wave) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ ((row >> 1) & 7);
      const uint32_t off = (uint32_t)(row * ld + k0 + chunk * EPC) * ES;
      dma16(rs, reinterpret_cast<const uint16_t*>(dst + (i * NW + wave) * 1024),
            k0 + chunk * EPC < K ? off : OOB);
    }
  };
  // One slice (k0 = first k) of A, and of B in the B_NK form, into stage dst.
  // A slice that reaches past K takes the masked form above (every chunk
  // past K reads zero); a whole slice uses the tile's fixed lane offsets.
  auto dma_slice = [&](const TileState& st, int k0, char* da, char* db) {
    if (k0 + BK <= K) {
      const uint32_t so = (uint32_t)k0 * ES;
#pragma unroll
      for (int i = 0; i < CHA; ++i) dma16s(st.ra, da + (i * NW + wave) * 1024, st.va[i], so);
      if constexpr (BDMA) {
#pragma unroll
        for (int i = 0; i < CHB; ++i) dma16s(st.rb, db + (i * NW + wave) * 1024, st.vb[i], so);
      }
    } else {
      dma_rows(st.ra, p.lda, k0, da, std::integral_constant<int, CHA>{});
      if constexpr (BDMA) dma_rows(st.rb, p.ldb, k0, db, std::integral_constant<int, CHB>{});
    }
  };
  struct BRegs {
    uint4 bv[RBV];
    uint32_t bs[RBS];
  };
  // register-staged B (B_KN / B_CONV): global -> registers, one element per
  // bs[] entry (16-bit values zero-extended)
  auto load_b = [&](const TileState& st, int k0, BRegs& R) {
    if constexpr (BMODE == B_KN) {
      const int krows = min(BK, K - k0);  // <= 0 past K: every load reads zero
      const int kb0 = krows > 0 ? k0 : 0;
      const rsrc_t rs = make_rsrc(Bb + ((long long)st.z * p.sB + (long long)kb0 * p.ldb + st.n0) * ES,
                                  krows > 0 ? (uint32_t)((krows - 1) * p.ldb + (N - st.n0)) * ES : 0u);
      if constexpr (KNV) {
#pragma unroll
        for (int i = 0; i < NKB; ++i) {
          const int c = tid + i * NT;
          if (2 * BN % NT != 0 && c >= 2 * BN) break;  // wave-uniform
          const int kg = c % KGS, ng = c / KGS;
          const bool nok = st.n0 + ng * EPC < N;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int kr = kg * 4 + j;
            R.bv[4 * i + j] = ld_b128(rs, (nok && kr < krows) ? (uint32_t)(kr * p.ldb + ng * EPC) * ES : OOB);
          }
        }
      } else {
        const int kb = krun * KR;
        const bool nok = st.gn_col < N;
#pragma unroll
        for (int e = 0; e < KR; ++e) {
          const uint32_t off = (nok && kb + e < krows) ? (uint32_t)((kb + e) * p.ldb + nl) * ES : OOB;
          R.bs[e] = ES == 4 ? ld_b32(rs, off) : ld_b16(rs, off);
        }
      }
    } else if constexpr (BMODE == B_CONV) {
      const bool live = k0 < K;
      const unsigned long long lmask = live ? st.cmask : 0ull;
      const uint32_t* tl = ktab_lds + (live ? k0 : 0) + krun * KR;
      uint32_t ent[KR];
#pragma unroll
      for (int q = 0; q < KR; q += 4) {
        const uint4 e4 = *reinterpret_cast<const uint4*>(tl + q);
        ent[q] = e4.x;
        ent[q + 1] = e4.y;
        ent[q + 2] = e4.z;
        ent[q + 3] = e4.w;
      }
#pragma unroll
      for (int e = 0; e < KR; ++e) {
        const bool ok = (lmask >> (ent[e] & 63u)) & 1ull;
        const uint32_t off = ok ? (uint32_t)(st.colbase + (int)(ent[e] >> 6)) * ES : OOB;
        R.bs[e] = ES == 4 ? ld_b32(st.rb, off) : ld_b16(st.rb, off);
      }
    }
  };
  // registers -> LDS (swizzled [n][k] layout)
  auto store_b = [&](char* sb, const BRegs& R) {
    if constexpr (KNV) {
#pragma unroll
      for (int i = 0; i < NKB; ++i) {
        const int c = tid + i * NT;
        if (2 * BN % NT != 0 && c >= 2 * BN) break;  // wave-uniform
        const int kg = c % KGS, ng = c / KGS;
        const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 0]);
        const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 1]);
        const uint32_t* r2 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 2]);
        const uint32_t* r3 = reinterpret_cast<const uint32_t*>(&R.bv[4 * i + 3]);
        if constexpr (ES == 4) {
          // 4 k-rows x 4 columns: column e is one whole chunk (k = kg*4 .. +3)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *reinterpret_cast<uint4*>(sb + swz(ng * 4 + e, kg)) = make_uint4(r0[e], r1[e], r2[e], r3[e]);
        } else {
          // 4 k-rows x 8 columns: column e gets 4 k = half of chunk kg/2
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
            *reinterpret_cast<uint2*>(sb + swz(ng * 8 + e, kg >> 1) + (kg & 1) * 8) = col;
          }
        }
      }
    } else if constexpr (!BDMA) {
#pragma unroll
      for (int q = 0; q < KR / EPC; ++q) {
        uint4 v;
        if constexpr (ES == 4)
          v = make_uint4(R.bs[4 * q], R.bs[4 * q + 1], R.bs[4 * q + 2], R.bs[4 * q + 3]);
        else
          v = make_uint4(pack2(R.bs[8 * q], R.bs[8 * q + 1]), pack2(R.bs[8 * q + 2], R.bs[8 * q + 3]),
                         pack2(R.bs[8 * q + 4], R.bs[8 * q + 5]), pack2(R.bs[8 * q + 6], R.bs[8 * q + 7]));
        *reinterpret_cast<uint4*>(sb + swz(nl, krun * (KR / EPC) + q)) = v;
      }
    }
  };

  // ---------------------------------------------------------- compute
  f32x16 acc[TM][TN];
  const int frow = lane & 31;
  const int fc = lane >> 5;  // logical chunk within a k step
  auto compute = [&](const char* sa, const char* sb) {
    uint4 af[2][TM], bfr[2][TN];
    auto frags = [&](int kk, uint4* a, uint4* b) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const uint4*>(sa + swz(wm * WM + i * 32 + frow, kk * 2 + fc));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const uint4*>(sb + swz(wn * WN + j * 32 + frow, kk * 2 + fc));
    };
    // Fragments of step kk+1 are issued before the MFMAs of step kk and the
    // order is pinned (sched_barrier): left alone, the scheduler sinks each
    // LDS read to just before its MFMA and exposes the LDS latency every step.
    frags(0, af[0], bfr[0]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {  // 4 steps of 2 chunks = one 128-byte row
      if (kk + 1 < 4) frags(kk + 1, af[(kk + 1) & 1], bfr[(kk + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_frag<DT>(bfr[kk & 1][j], af[kk & 1][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  int unit = rb;
  if (unit >= nunits) return;
  TileState cur = tile_state(unit);
  BRegs RB;

  // the first NS-1 slices of a tile: DMA into stages 0..NS-2; register-staged
  // B slice 0 goes to LDS at the top of the tile loop, slice 1 in step 0
  // Slices past the unit's K range are not loaded at all (so no load can
  // reach past the operand); the waits below count only issued slices.
  auto prologue = [&](const TileState& st) {
    const int k0 = st.kbase;
    if constexpr (!BDMA) load_b(st, k0, RB);
    dma_slice(st, k0, stA(std::integral_constant<int, 0>{}), stB(std::integral_constant<int, 0>{}));
    if (st.kts > 1)
      dma_slice(st, k0 + BK, stA(std::integral_constant<int, 1>{}), stB(std::integral_constant<int, 1>{}));
    if constexpr (NS > 3) {
      if (st.kts > 2)
        dma_slice(st, k0 + 2 * BK, stA(std::integral_constant<int, 2>{}), stB(std::integral_constant<int, 2>{}));
    }
  };
  // s_waitcnt until slice `need` has landed, given that the unit's slices up
  // to min(newest, kts - 1) were issued after it (n of them, 0 <= n <= NS-2)
  auto wait_slice = [&](int need, int newest, int kts) {
    const int last = min(newest, kts - 1);
    const int n = last > need ? last - need : 0;
    if (n >= 2 && NS > 3) wait_vm<(NS > 3 ? 2 : 0) * DMAS>();
    else if (n >= 1) wait_vm<DMAS>();
    else wait_vm<0>();
  };

  // Step t (stage s = t % NS): request slice t+NS-1 into the stage read last
  // in step t-1 (which ended with a barrier), multiply stage s, then wait
  // until slice t+1 has landed and publish it with a barrier.
  auto step = [&](int t, auto s_tag) {
    constexpr int S = decltype(s_tag)::value;
    constexpr int S1 = (S + 1) % NS, SL = (S + NS - 1) % NS;
    using I1 = std::integral_constant<int, S1>;
    using IL = std::integral_constant<int, SL>;
    // register-staged B of slice t+1 (past K it reads zeros, never multiplied)
    if constexpr (!BDMA) load_b(cur, cur.kbase + (t + 1) * BK, RB);
    if (t + NS - 1 < cur.kts)
      dma_slice(cur, cur.kbase + (t + NS - 1) * BK, stA(IL{}), stB(IL{}));
    compute(stA(s_tag), stB(s_tag));
    if constexpr (!BDMA) store_b(stB(I1{}), RB);
    wait_slice(t + 1, t + NS - 1, cur.kts);  // slice t+1 landed, later ones may still run
    __syncthreads();
  };

  prologue(cur);
  while (true) {
    const int par = (unit / G) & 1;  // bias buffer of this unit
    if constexpr (!BDMA) store_b(stB(std::integral_constant<int, 0>{}), RB);
    if (p.bias_mode != BIAS_NONE && tid < BMAX) sbias[par][tid] = p.beta * to_f32<DT>(cur.bias_h);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    wait_slice(0, NS - 2, cur.kts);  // slice 0 landed (slices 1.. may still run)
    __syncthreads();

    const int kts = cur.kts;
    for (int t = 0; t < kts; t += NS) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < kts) step(t + 1, std::integral_constant<int, 1>{});
      if (t + 2 < kts) step(t + 2, std::integral_constant<int, 2>{});
      if constexpr (NS > 3)
        if (t + 3 < kts) step(t + 3, std::integral_constant<int, 3 % NS>{});
    }
    // the DMAs of the slices past K (zeros) land before the stages are
    // refilled for the next tile
    wait_vm<0>();
    __syncthreads();

    const int m0 = cur.m0, n0 = cur.n0, z = cur.z, tile = cur.tile, sp = cur.sp;
    const int next = unit + G;
    if (next < nunits) {  // the next unit's first slices run under this epilogue
      cur = tile_state(next);
      prologue(cur);
    }

    // split-K: this unit's partial sum (fp32) goes to slab sp of the
    // workspace, laid out like C ([batch][M][N], dense); the reduction kernel
    // sums the slabs in order and runs the epilogue.
    if (S > 1) {
      const int mrows = min(BM, M - m0);
      const rsrc_t rw = make_rsrc(p.ws + (((long long)sp * p.batch + z) * M + m0) * (long long)N + n0,
                                  (uint32_t)((mrows - 1) * N + (N - n0)) * 4u);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int row = wm * WM + i * 32 + frow;
            const int col = wn * WN + j * 32 + 8 * g + 4 * (lane >> 5);
            const uint32_t off = (uint32_t)(row * N + col) * 4u;
            if ((N & 3) == 0) {
              st_b128(make_uint4(__float_as_uint(acc[i][j][4 * g]), __float_as_uint(acc[i][j][4 * g + 1]),
                                 __float_as_uint(acc[i][j][4 * g + 2]), __float_as_uint(acc[i][j][4 * g + 3])),
                      rw, n0 + col < N ? off : OOB);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                st_b32(__float_as_uint(acc[i][j][4 * g + e]), rw, n0 + col + e < N ? off + 4u * e : OOB);
            }
          }
      if (next >= nunits) break;
      unit = next;
      continue;
    }

    // ------------------------------------------------------ epilogue
    // acc[i][j] holds C^T: lane owns row m = i*32 + lane%32 and, per register
    // group g, the 4 columns n = j*32 + 8g + 4*(lane/32) + (0..3).
    const int mrows = min(BM, M - m0);
    const rsrc_t rc = make_rsrc(Cb + ((long long)z * p.sC + (long long)m0 * p.ldc + n0) * ES,
                                (uint32_t)((mrows - 1) * p.ldc + (N - n0)) * ES);
    const bool cvec = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & (4 * ES - 1)) == 0) &&
                      ((p.sC & 3) == 0) && ((N & 3) == 0);
    // Uniform epilogue choices hoisted out of the element loop: the plain
    // forms (vector stores, no activation, no clamp; bias none / per column /
    // per row) are straight-line code, everything else takes the general form.
    // 16-bit plain forms store 16 bytes per lane: lanes l and l ^ 32 hold the
    // two 4-column halves of each 8-column run of a row and trade one half
    // (ds_bpermute), so every store writes 32 bytes of each of 32 rows (8-byte
    // stores in the MFMA layout: measured 2.6 TB/s on MI355X, 16-byte lane
    // pairs 3.9 TB/s, full 128-byte lines 4.3 TB/s).
    const bool cv16 = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0) &&
                      ((p.sC & 7) == 0) && ((N & 7) == 0);
    const bool plain = p.act == WGX_ACT_NONE && !p.has_clamp && (DT == DT_F32 ? cvec : cv16);
    const int emode = !plain ? 3 : (p.bias_mode == BIAS_COL ? 1 : (p.bias_mode == BIAS_ROW ? 2 : 0));
    auto put = [&](auto mode) {
      constexpr int MODE = decltype(mode)::value;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WM + i * 32 + frow;
        float rowb = 0.0f;
        if constexpr (MODE == 2) rowb = sbias[par][row];
        if constexpr (MODE == 3) rowb = p.bias_mode == BIAS_ROW ? sbias[par][row] : 0.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (MODE != 3 && DT != DT_F32) {
            const int fcl = lane >> 5;
            uint32_t pk[4][2];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int col = wn * WN + j * 32 + 8 * g + 4 * fcl;
              float4 bc = make_float4(0.f, 0.f, 0.f, 0.f);
              if constexpr (MODE == 1) bc = *reinterpret_cast<const float4*>(&sbias[par][col]);
              const float bb[4] = {bc.x, bc.y, bc.z, bc.w};
              uint32_t h[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) h[e] = st_bits<DT == DT_BF16>(p.alpha * acc[i][j][4 * g + e] + rowb + bb[e]);
              pk[g][0] = pack2(h[0], h[1]);
              pk[g][1] = pack2(h[2], h[3]);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const uint32_t s0 = fcl ? pk[2 * q][0] : pk[2 * q + 1][0];
              const uint32_t s1 = fcl ? pk[2 * q][1] : pk[2 * q + 1][1];
              const uint32_t r0 = (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, (int)s0);
              const uint32_t r1 = (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, (int)s1);
              const uint4 v = fcl ? make_uint4(r0, r1, pk[2 * q + 1][0], pk[2 * q + 1][1])
                                  : make_uint4(pk[2 * q][0], pk[2 * q][1], r0, r1);
              const int col = wn * WN + j * 32 + 16 * q + 8 * fcl;
              st_b128(v, rc, n0 + col < N ? (uint32_t)(row * p.ldc + col) * ES : OOB);
            }
            continue;
          }
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = wn * WN + j * 32 + 8 * g + 4 * (lane >> 5);
            float4 bc = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (MODE == 1) bc = *reinterpret_cast<const float4*>(&sbias[par][col]);
            if constexpr (MODE == 3)
              if (p.bias_mode == BIAS_COL) bc = *reinterpret_cast<const float4*>(&sbias[par][col]);
            const float bb[4] = {bc.x, bc.y, bc.z, bc.w};
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float x = p.alpha * acc[i][j][4 * g + e] + rowb + bb[e];
              if constexpr (MODE == 3) {
                x = apply_act(p.act, x);
                if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
              }
              if constexpr (DT == DT_F32) h[e] = __float_as_uint(x);
              else h[e] = st_bits<DT == DT_BF16>(x);
            }
            const uint32_t off = (uint32_t)(row * p.ldc + col) * ES;
            if (MODE != 3 || cvec) {
              if constexpr (DT == DT_F32)
                st_b128(make_uint4(h[0], h[1], h[2], h[3]), rc, n0 + col < N ? off : OOB);
              else
                st_b64(make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3])), rc, n0 + col < N ? off : OOB);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint32_t oe = n0 + col + e < N ? off + ES * e : OOB;
                if constexpr (DT == DT_F32) st_b32(h[e], rc, oe);
                else st_b16(h[e], rc, oe);
              }
            }
          }
        }
      }
    };
    if (emode == 1) put(std::integral_constant<int, 1>{});
    else if (emode == 2) put(std::integral_constant<int, 2>{});
    else if (emode == 0) put(std::integral_constant<int, 0>{});
    else put(std::integral_constant<int, 3>{});
    if (next >= nunits) break;
    unit = next;
  }
}

// ============================================================ large-tile kernel
// C = epilogue(A * B^T) with A [M, K] and B [N, K], both k-contiguous (the
// nn.Linear / W^T form of addmm, and bmm with a transposed right operand),
// float16 or bfloat16, for shapes with enough tiles of 256 rows.
//
// Why a second kernel: measured on MI355X, the L2 -> LDS path moves 35-50
// bytes per clock per CU (with 64-128 KB in flight), 128-bit LDS reads about
// 64 B/clk per CU.  A 128 x 128 block tile at the full MFMA rate needs
// 64 B/clk of operand traffic; a 256 x 192 tile needs 37 B/clk, and its
// 128 x 96 wave tiles need the fewest LDS fragment bytes per MFMA that fit in
// registers.  So: 256-row tiles, 4 waves (one per SIMD, 12 accumulators),
// RB-byte LDS rows (RB = 64: a K slice of 32, chunk c of row r stored at
// c ^ ((r / 4) % 4); RB = 128: a slice of 64, chunk c at c ^ ((r / 2) % 8);
// either way the 16 rows one 128-bit read touches per cycle cover all 64
// banks), NS stages, all loads LDS-DMA with the slice's k offset in the
// scalar offset, one barrier per slice.  The epilogue goes through the (then
// idle) stage memory so that every store instruction writes whole rows of the
// tile: full 128-byte lines, which the memory system absorbs at close to copy
// speed.  The fragment reads (about 74 B/clk at the full MFMA rate) plus the
// DMA writes bound this loop by LDS bandwidth at roughly 55-60% of the MFMA
// peak.
__device__ __forceinline__ int swz64(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }
int device_cus();

template <int BM, int BN, int WGM, int WGN, bool BF, int NS, int RB>
__global__ __launch_bounds__(WGM * WGN * 64) __attribute__((amdgpu_waves_per_eu(WGM * WGN / 4, WGM * WGN / 4))) void k_gemm_nk(KParams p) {
  constexpr int NW = WGM * WGN, NT = NW * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  constexpr int ES = 2, EPC = 8, BK = RB / ES;  // RB: LDS row bytes (64 or 128)
  constexpr int CPR = RB / 16, RPI = 1024 / RB;  // chunks per row, rows per DMA instruction
  constexpr int KS = RB / 32;                    // k-steps of 16 per slice
  constexpr int STAGE = (BM + BN) * RB;                 // bytes per stage
  constexpr int CHA = BM * RB / 1024 / NW;              // DMA instructions per wave per slice: A
  constexpr int CHB = BN * RB / 1024 / NW;              // ... B
  constexpr int DMAS = CHA + CHB;
  constexpr int CP = BN * ES + 16;                      // epilogue LDS row pitch
  // The whole C tile is staged at once (one epilogue pass): every instantiation
  // has the stage memory for it.  A split into row passes for smaller stage
  // memories gave different bits from the one-pass form in a probe at
  // 4096 x 3072 x 768 and is not offered.
  constexpr int EROWS = BM;  // rows per epilogue pass
  constexpr int BMAX = BM > BN ? BM : BN;
  static_assert(TM >= 1 && TN >= 1 && CHA >= 1 && CHB >= 1, "tile shape");
  static_assert(BM * RB % (1024 * NW) == 0 && BN * RB % (1024 * NW) == 0, "DMA split");
  static_assert(EROWS * CP <= NS * STAGE, "epilogue staging: the C tile must fit the stage memory");
  static_assert((NS - 1) * DMAS < 64 && NS >= 2 && NS <= 5 && (RB == 64 || RB == 128), "stages");

  // 16-byte chunk c of LDS row r is stored at chunk swzc(r, c): with 64-byte
  // rows c ^ ((r/4)%4), with 128-byte rows c ^ ((r/2)%8); the 16 rows one
  // 128-bit fragment read touches per cycle then cover all 64 banks
  auto swzc = [](int r, int c) { return RB == 64 ? c ^ ((r >> 2) & 3) : c ^ ((r >> 1) & 7); };
  auto swzr = [&](int r, int c) { return r * RB + (swzc(r, c) << 4); };
  __shared__ __attribute__((aligned(1024))) char stg[NS * STAGE];
  __shared__ __attribute__((aligned(16))) float sbias[BMAX];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int M = p.M, N = p.N, K = p.K;
  const int KT = (K + BK - 1) / BK;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_mn = tiles_m * p.tiles_n;
  const int ntiles = tiles_mn * p.batch;
  const int G = gridDim.x;
  const int rbk = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const char* Ab = reinterpret_cast<const char*>(p.A);
  const char* Bb = reinterpret_cast<const char*>(p.B);
  char* Cb = reinterpret_cast<char*>(p.C);
  const bool cvec = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0) && ((p.sC & 7) == 0);

  for (int tile = rbk; tile < ntiles; tile += G) {
    // grouped tile order: p.gm m-tiles are walked first, then n (a run of
    // consecutive tiles -- one XCD's share -- covers a compact rectangle)
    const int z = tile / tiles_mn, r = tile % tiles_mn;
    const int gsz = p.gm * p.tiles_n;
    const int grp = r / gsz, rr = r - grp * gsz;
    const int gmh = min(p.gm, tiles_m - grp * p.gm);
    const int m0 = (grp * p.gm + rr % gmh) * BM;
    const int n0 = (rr / gmh) * BN;
    const int mrows = min(BM, M - m0), nrows = min(BN, N - n0);
    const rsrc_t ra = make_rsrc(Ab + ((long long)z * p.sA + (long long)m0 * p.lda) * ES,
                                (uint32_t)((mrows - 1) * p.lda + K) * ES);
    const rsrc_t rbf = make_rsrc(Bb + ((long long)z * p.sB + (long long)n0 * p.ldb) * ES,
                                 (uint32_t)((nrows - 1) * p.ldb + K) * ES);
    // this lane's DMA chunk of each instruction: LDS row (i*NW + wave)*RPI +
    // lane/CPR, stored chunk lane%CPR, which holds logical chunk swzc(row, lane%CPR)
    uint32_t va[CHA], vb[CHB];
#pragma unroll
    for (int i = 0; i < CHA; ++i) {
      const int row = (i * NW + wave) * RPI + lane / CPR, chunk = swzc(row, lane % CPR);
      va[i] = row < mrows ? (uint32_t)(((long long)row * p.lda + chunk * EPC) * ES) : OOB;
    }
#pragma unroll
    for (int i = 0; i < CHB; ++i) {
      const int row = (i * NW + wave) * RPI + lane / CPR, chunk = swzc(row, lane % CPR);
      vb[i] = row < nrows ? (uint32_t)(((long long)row * p.ldb + chunk * EPC) * ES) : OOB;
    }
    // slice s into stage s % NS; a slice reaching past K masks its chunks
    auto issue = [&](int sl) {
      char* base = stg + (sl % NS) * STAGE;
      const int k0 = sl * BK;
      if (k0 + BK <= K) {
        const uint32_t so = (uint32_t)k0 * ES;
#pragma unroll
        for (int i = 0; i < CHA; ++i) dma16s(ra, base + (i * NW + wave) * 1024, va[i], so);
#pragma unroll
        for (int i = 0; i < CHB; ++i) dma16s(rbf, base + BM * RB + (i * NW + wave) * 1024, vb[i], so);
      } else {
#pragma unroll
        for (int i = 0; i < CHA; ++i) {
          const int row = (i * NW + wave) * RPI + lane / CPR, chunk = swzc(row, lane % CPR);
          const bool ok = row < mrows && k0 + chunk * EPC < K;
          dma16(ra, reinterpret_cast<const uint16_t*>(base + (i * NW + wave) * 1024),
                ok ? (uint32_t)((row * p.lda + k0 + chunk * EPC) * ES) : OOB);
        }
#pragma unroll
        for (int i = 0; i < CHB; ++i) {
          const int row = (i * NW + wave) * RPI + lane / CPR, chunk = swzc(row, lane % CPR);
          const bool ok = row < nrows && k0 + chunk * EPC < K;
          dma16(rbf, reinterpret_cast<const uint16_t*>(base + BM * RB + (i * NW + wave) * 1024),
                ok ? (uint32_t)((row * p.ldb + k0 + chunk * EPC) * ES) : OOB);
        }
      }
    };

    // bias of the tile, scaled by beta, parked in LDS (the previous tile's
    // epilogue ended with a barrier, so nobody reads the old values)
    if (p.bias_mode != BIAS_NONE) {
      const bool col = p.bias_mode == BIAS_COL;
      const int lim = col ? N : M, b0 = col ? n0 : m0, cnt = col ? BN : BM;
      const rsrc_t rbias = make_rsrc(p.bias, (uint32_t)lim * ES);
      for (int i = tid; i < cnt; i += NT) {
        const uint32_t off = b0 + i < lim ? (uint32_t)(b0 + i) * ES : OOB;
        sbias[i] = p.beta * to_f32<BF ? DT_BF16 : DT_F16>(ld_b16(rbias, off));
      }
    }

#pragma unroll 1
    for (int sl = 0; sl < NS - 1; ++sl)
      if (sl < KT) issue(sl);

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int frow = lane & 31, fc = lane >> 5;
    auto frags = [&](int sl, int kk, uint4* a, uint4* b) {
      const char* sa = stg + (sl % NS) * STAGE;
      const char* sb = sa + BM * RB;
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const uint4*>(sa + swzr(wm * WM + i * 32 + frow, kk * 2 + fc));
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *reinterpret_cast<const uint4*>(sb + swzr(wn * WN + j * 32 + frow, kk * 2 + fc));
    };
    // slice `need` has landed once at most the slices issued after it, up
    // to slice `newest` (clipped to the last one), are still outstanding
    auto wait_for = [&](int need, int newest) {
      const int after = min(newest, KT - 1) - need;
      if (after >= 3) wait_vm<3 * DMAS>();
      else if (after == 2) wait_vm<2 * DMAS>();
      else if (after == 1) wait_vm<DMAS>();
      else wait_vm<0>();
    };
    // Software pipeline over (slice, k-step): the fragments of the next
    // k-step are read while the current one's MFMAs run, also across slices.
    // The barrier of slice t+1 sits before the last k-step of slice t, so the
    // MFMAs issued before it keep the matrix cores busy while the waves meet;
    // past it slice t+1 is visible to every wave, and every wave holds all of
    // slice t in registers, so slice t's stage is refilled with slice t+NS.
    uint4 fa[2][TM], fb[2][TN];
    wait_for(0, NS - 2);
    __syncthreads();
    if (NS - 1 < KT) issue(NS - 1);
    frags(0, 0, fa[0], fb[0]);
    for (int t = 0; t < KT; ++t) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int cur = kk & 1, nxt = cur ^ 1;  // KS is even: a slice starts in buffer 0
        if (kk + 1 < KS) {
          frags(t, kk + 1, fa[nxt], fb[nxt]);
        } else if (t + 1 < KT) {
          wait_for(t + 1, t + NS - 1);
          __syncthreads();
          if (t + NS < KT) issue(t + NS);
          frags(t + 1, 0, fa[nxt], fb[nxt]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma<BF>(fb[cur][j], fa[cur][i], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();  // every wave is done with the stages: they hold the C tile now

    // ------------------------------------------------------------ epilogue
    // acc[i][j] holds C^T: this lane owns row wm*WM + i*32 + lane%32 and, per
    // register group g, columns wn*WN + j*32 + 8g + 4*(lane/32) + 0..3.
    // The bias form, activation and clamp are uniform over the launch: the
    // plain forms (no activation, no clamp; bias none / per column / per row)
    // get straight-line code, everything else the general one.  Per-element
    // uniform branches here cost more than the stores they guard.
    const bool plain = p.act == WGX_ACT_NONE && !p.has_clamp;
    const int emode = !plain ? 3 : (p.bias_mode == BIAS_COL ? 1 : (p.bias_mode == BIAS_ROW ? 2 : 0));
#pragma unroll
    for (int q = 0; q < BM / EROWS; ++q) {
      if ((wm * WM) / EROWS == q) {
        auto put = [&](auto mode) {
          constexpr int MODE = decltype(mode)::value;  // 0/1/2: plain, bias none/col/row; 3: general
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            const int row = wm * WM + i * 32 + frow;
            float rowb = 0.0f;
            if constexpr (MODE == 2) rowb = sbias[row];
            if constexpr (MODE == 3) rowb = p.bias_mode == BIAS_ROW ? sbias[row] : 0.0f;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int col = wn * WN + j * 32 + 8 * g + 4 * fc;
                float4 bc = make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (MODE == 1) bc = *reinterpret_cast<const float4*>(&sbias[col]);
                if constexpr (MODE == 3)
                  if (p.bias_mode == BIAS_COL) bc = *reinterpret_cast<const float4*>(&sbias[col]);
                const float bb[4] = {bc.x, bc.y, bc.z, bc.w};
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  float x = p.alpha * acc[i][j][4 * g + e];
                  if constexpr (MODE == 1 || MODE == 3) x += bb[e];
                  if constexpr (MODE == 2 || MODE == 3) x += rowb;
                  if constexpr (MODE == 3) {
                    x = apply_act(p.act, x);
                    if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
                  }
                  h[e] = st_bits<BF>(x);
                }
                *reinterpret_cast<uint2*>(stg + (row - q * EROWS) * CP + col * ES) =
                    make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
              }
            // keep the accumulator reads of one row block together (the
            // scheduler would otherwise hoist them all and run out of VGPRs)
            __builtin_amdgcn_sched_barrier(0);
          }
        };
        if (emode == 1) put(std::integral_constant<int, 1>{});
        else if (emode == 2) put(std::integral_constant<int, 2>{});
        else if (emode == 0) put(std::integral_constant<int, 0>{});
        else put(std::integral_constant<int, 3>{});
      }
      __syncthreads();
      // EROWS rows of BN columns: 16 bytes per lane, lanes along the rows
      constexpr int PPR = BN * ES / 16;  // 16-byte pieces per row
      for (int idx = tid; idx < EROWS * PPR; idx += NT) {
        const int rr2 = idx / PPR, pc = idx - rr2 * PPR;
        const int grow = m0 + q * EROWS + rr2, gcol = n0 + pc * EPC;
        if (grow >= M || gcol >= N) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(stg + rr2 * CP + pc * 16);
        uint16_t* dst = reinterpret_cast<uint16_t*>(Cb) + (long long)z * p.sC + (long long)grow * p.ldc + gcol;
        if (cvec && gcol + EPC <= N) {
          using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
          const u32x4 w4 = {v.x, v.y, v.z, v.w};
          if (p.nt_store) __builtin_nontemporal_store(w4, reinterpret_cast<u32x4*>(dst));
          else *reinterpret_cast<u32x4*>(dst) = w4;
        } else {
          const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int e = 0; e < EPC; ++e)
            if (gcol + e < N) dst[e] = (uint16_t)(u[e >> 1] >> (16 * (e & 1)));
        }
      }
      __syncthreads();
    }
  }
}

template <int BM, int BN, int WGM, int WGN, bool BF, int NS, int RB>
hipError_t launch_nk(const KParams& kp, int batch, hipStream_t s) {
  auto fn = k_gemm_nk<BM, BN, WGM, WGN, BF, NS, RB>;
  if (is_dry(s)) return hipSuccess;
  const long long ntiles = (long long)((kp.M + BM - 1) / BM) * kp.tiles_n * batch;
  long long grid = device_cus();  // one block per CU (the stages take most of the LDS)
  if (grid > ntiles) grid = ntiles;
  KParams k2 = kp;
  k2.batch = batch;
  {
    const int tiles_m = (kp.M + BM - 1) / BM;
    const double per_xcd = (double)(grid < 8 ? 1 : grid / 8);
    int gm = (int)lround(sqrt(per_xcd * BN / BM));
    k2.gm = gm < 1 ? 1 : (gm > tiles_m ? tiles_m : gm);
  }
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WGM * WGN * 64), 0, s, k2);
  return hipGetLastError();
}

// ============================================================ short-K kernel
// 16-bit GEMMs whose whole K (at most 64) is one LDS slice and whose output is
// large: aten.bmm [16,1024,64] x [16,64,1024] writes 33.5 MB from 4 MB of
// operands, so the output path sets the time, not the multiply.  One block of
// 4 waves owns a 128 x 128 tile: A and B are loaded once into LDS, at most 4
// k-steps of MFMAs, then the C tile goes through the same LDS and out as
// whole 256-byte rows (two full 128-byte lines each; partial lines would be
// merged in L2 or written as masked bursts).  At 35 KB of LDS several blocks
// share a CU, so one block's stores drain while another loads.
//   A, and a [N,K] B: LDS rows of 128 bytes (K padded to a multiple of 16
//     with zeros), 16-byte chunk c of row r at c ^ ((r / 2) % 8), read as
//     16-byte fragments.
//   A [K,N] B is read in place: LDS rows k of 288 bytes (128 n and a 32-byte
//     pad, so the 4 rows one 16-lane group reads start on different banks),
//     read with the gfx950 transposing read ds_read_b64_tr_b16.  Within each
//     16-lane group lane L supplies the 4 halves at its address and lane i
//     receives, as its element e, half i % 4 of lane 4e + i / 4; lane L
//     pointing at B[k0 + L/4][n0 + 4(L%4)] therefore hands lane i the halves
//     B[k0 + 0..3][n0 + i]: 4 consecutive k of its column, two reads making
//     the 8 of an MFMA fragment.
typedef short v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_tr16(const char* p) {
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(const_cast<char*>(p)));
  return make_uint2(pack2((uint16_t)v.x, (uint16_t)v.y), pack2((uint16_t)v.z, (uint16_t)v.w));
}

template <bool BF, bool BKN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_sk(KParams p) {
  constexpr int BM = 128, BN = 128, RB = 128, BP = 288, CP = BN * 2 + 16;
  constexpr int A_BYTES = BM * RB;
  constexpr int B_BYTES = BKN ? 64 * BP : BN * RB;
  __shared__ __attribute__((aligned(16))) char sab[A_BYTES + B_BYTES];
  __shared__ __attribute__((aligned(16))) char sc[BM * CP];
  // the bias of the tile's rows and of its columns (the one not in use holds
  // zeros), so the epilogue adds both without a branch
  __shared__ __attribute__((aligned(16))) float srow[128], scol[128];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // 2 x 2 waves of 64 x 64
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_mn = tiles_m * p.tiles_n;
  const int ntiles = tiles_mn * p.batch;
  const int K = p.K, KC = K >> 3;  // K <= 64, a multiple of 8: 16-byte chunks per row
  const int KS = (K + 15) >> 4;
  char* sa = sab;
  char* sb = sab + A_BYTES;
  const int frow = lane & 31, fc = lane >> 5;

  struct TileAt {
    int z, m0, n0, mrows, nrows;
  };
  auto tile_at = [&](int t) {
    TileAt ti;
    ti.z = t / tiles_mn;
    const int r = t - ti.z * tiles_mn;
    ti.m0 = (r % tiles_m) * BM;
    ti.n0 = (r / tiles_m) * BN;
    ti.mrows = min(BM, p.M - ti.m0);
    ti.nrows = min(BN, p.N - ti.n0);
    return ti;
  };

  // a tile's operands in registers: 4 16-byte chunks of A and 4 of B per
  // thread and one bias element; a tile index past the end reads zeros
  uint4 ra[4], rb[4];
  uint32_t rbias;
  auto load_regs = [&](int t) {
    const bool ok = t < ntiles;
    const TileAt ti = tile_at(ok ? t : 0);
    const rsrc_t rsa = make_rsrc(p.A + (long long)ti.z * p.sA + (long long)ti.m0 * p.lda,
                                 (uint32_t)(((long long)(ti.mrows - 1) * p.lda + K) * 2));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
      ra[i] = ld_b128(rsa, ok && row < ti.mrows && ch < KC ? (uint32_t)((row * p.lda + ch * 8) * 2) : OOB);
    }
    if constexpr (BKN) {
      const rsrc_t rsb = make_rsrc(p.B + (long long)ti.z * p.sB + ti.n0,
                                   (uint32_t)(((long long)(K - 1) * p.ldb + ti.nrows) * 2));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i, row = c >> 4, ch = c & 15;  // row: k
        rb[i] = ld_b128(rsb, ok && row < K && ch * 8 < ti.nrows ? (uint32_t)((row * p.ldb + ch * 8) * 2) : OOB);
      }
    } else {
      const rsrc_t rsb = make_rsrc(p.B + (long long)ti.z * p.sB + (long long)ti.n0 * p.ldb,
                                   (uint32_t)(((long long)(ti.nrows - 1) * p.ldb + K) * 2));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
        rb[i] = ld_b128(rsb, ok && row < ti.nrows && ch < KC ? (uint32_t)((row * p.ldb + ch * 8) * 2) : OOB);
      }
    }
    const bool col = p.bias_mode == BIAS_COL;
    const int lim = col ? p.N : p.M, idx = (col ? ti.n0 : ti.m0) + (tid & 127);
    const rsrc_t rsbias = make_rsrc(p.bias, p.bias_mode != BIAS_NONE ? (uint32_t)lim * 2u : 0u);
    rbias = ld_b16(rsbias, ok && idx < lim ? (uint32_t)idx * 2u : OOB);
  };
  // registers -> LDS (zeros stand for rows and chunks past the edges)
  auto store_lds = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
      *reinterpret_cast<uint4*>(sa + row * RB + ((ch ^ ((row >> 1) & 7)) << 4)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (BKN) {
        const int c = tid + 256 * i, row = c >> 4, ch = c & 15;
        *reinterpret_cast<uint4*>(sb + row * BP + ch * 16) = rb[i];
      } else {
        const int c = tid + 256 * i, row = c >> 3, ch = c & 7;
        *reinterpret_cast<uint4*>(sb + row * RB + ((ch ^ ((row >> 1) & 7)) << 4)) = rb[i];
      }
    }
    if (tid < 128) {
      const float v = p.beta * ld_f32<BF>((uint16_t)rbias);
      srow[tid] = p.bias_mode == BIAS_ROW ? v : 0.0f;
      scol[tid] = p.bias_mode == BIAS_COL ? v : 0.0f;
    }
  };
  // acc[i][j]: row wm*64 + i*32 + lane%32, per register group g the columns
  // wn*64 + j*32 + 8g + 4*(lane/32) + 0..3 -> the C stage
  auto epilogue = [&]<bool PLAIN>(const f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = wm * 64 + i * 32 + frow;
      const float rowb = srow[row];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = wn * 64 + j * 32 + 8 * g + 4 * fc;
          const float4 cb = *reinterpret_cast<const float4*>(scol + col);
          const float colb[4] = {cb.x, cb.y, cb.z, cb.w};
          uint32_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = p.alpha * acc[i][j][4 * g + e] + rowb + colb[e];
            if constexpr (!PLAIN) {
              x = apply_act(p.act, x);
              if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
            }
            h[e] = st_bits<BF>(x);
          }
          *reinterpret_cast<uint2*>(sc + row * CP + col * 2) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
        }
    }
  };
  // the C stage -> global memory, 16 lanes per 256-byte row, 16 rows per
  // pass; every store is issued (a piece past the tile's edge at an
  // out-of-range offset, which the buffer range check drops), so the count of
  // stores in flight is the same on every path.  aux 2: non-temporal.
  auto store_c = [&]<int AUX>(const TileAt& ti) {
    const rsrc_t rc = make_rsrc(p.C + (long long)ti.z * p.sC + (long long)ti.m0 * p.ldc + ti.n0,
                                (uint32_t)(((long long)(ti.mrows - 1) * p.ldc + ti.nrows) * 2));
    using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int pass = 0; pass < BM / 16; ++pass) {
      const int row = pass * 16 + (tid >> 4), pc = tid & 15;
      const uint4 v = *reinterpret_cast<const uint4*>(sc + row * CP + pc * 16);
      const bool in = row < ti.mrows && pc * 8 < ti.nrows;
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, rc,
                                             in ? (int)((row * p.ldc + pc * 8) * 2) : (int)OOB, 0, AUX);
    }
  };
  const bool plain = p.act == WGX_ACT_NONE && !p.has_clamp;

  int t = blockIdx.x;
  load_regs(t);
  store_lds();
  for (; t < ntiles; t += gridDim.x) {
    const TileAt ti = tile_at(t);
    // this tile's operands are in LDS; every wave has read the previous C stage
    __syncthreads();
    // the next tile's operands are in flight during this tile's multiplies
    load_regs(t + gridDim.x);

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    for (int kk = 0; kk < KS; ++kk) {
      uint4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + i * 32 + frow;
        a[i] = *reinterpret_cast<const uint4*>(sa + row * RB + (((kk * 2 + fc) ^ ((row >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (BKN) {
          const int G = lane >> 4, L = lane & 15;
          const int nb = wn * 64 + j * 32 + (G & 1) * 16, kb = kk * 16 + (G >> 1) * 8;
          const char* base = sb + (kb + (L >> 2)) * BP + (nb + 4 * (L & 3)) * 2;
          const uint2 lo = lds_tr16(base), hi = lds_tr16(base + 4 * BP);
          b[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else {
          const int row = wn * 64 + j * 32 + frow;
          b[j] = *reinterpret_cast<const uint4*>(sb + row * RB + (((kk * 2 + fc) ^ ((row >> 1) & 7)) << 4));
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma<BF>(b[j], a[i], acc[i][j]);
    }
    if (plain)
      epilogue.template operator()<true>(acc);
    else
      epilogue.template operator()<false>(acc);
    // the C stage is whole; every wave is done with the operands and the bias
    __syncthreads();
    // the next tile's operands -> LDS (waits for their loads, issued before
    // this tile's multiplies), then this tile's stores, which drain during
    // the next tile's multiplies
    store_lds();
    if (p.nt_store)
      store_c.template operator()<2>(ti);
    else
      store_c.template operator()<0>(ti);
  }
}

template <bool BF, bool BKN>
hipError_t launch_sk(const KParams& kp, int batch, hipStream_t s) {
  if (is_dry(s)) return hipSuccess;
  const long long ntiles = (long long)((kp.M + 127) / 128) * kp.tiles_n * batch;
  if (ntiles >= (1LL << 31)) return hipErrorInvalidValue;
  // persistent: two blocks per CU (about 70 KB of LDS each), block b walking
  // tiles b, b + grid, ...
  long long grid = 2LL * device_cus();
  if (const char* e = getenv("WGX_SK_BLOCKS")) grid = atoll(e) > 0 ? atoll(e) : grid;
  if (grid > ntiles) grid = ntiles;
  hipLaunchKernelGGL((k_gemm_sk<BF, BKN>), dim3((unsigned)grid), dim3(256), 0, s, kp);
  return hipGetLastError();
}

// ============================================================ [K,N] -> [N,K] staging
// The large-tile kernel reads both operands k-contiguous.  A 16-bit [K, N]
// operand (aten.mm's own layout) large enough for that kernel is first
// rewritten as [N, K] into a workspace: one pass over B (2 x 2 bytes per
// element through HBM, a few microseconds for a 768 x 3072 weight) buys the
// large-tile loop, and the GEMM then computes on exactly the values the
// [N, K] form would see, so both layouts give the same bits.
//
// One block moves a 64(k) x 64(n) tile: reads 128-byte row pieces of B
// (8 lanes per row), parks them in LDS with a 66-element row pitch, and
// writes 128-byte row pieces of B^T (8 lanes per row of 64 k).  With that
// pitch the eight rows one gather step touches (8 apart) fall on eight
// different bank groups, so the column reads are conflict free.
__global__ __launch_bounds__(256) void k_kn_to_nk(const uint16_t* __restrict__ B, uint16_t* __restrict__ BT,
                                                   int K, int N, long long ldb, long long sB, int tiles_k,
                                                   int tiles_n) {
  constexpr int P = 66;  // LDS row pitch in elements (132 bytes)
  __shared__ __attribute__((aligned(16))) uint16_t t[64 * P];
  const int tid = threadIdx.x;
  const long long tk_tn = (long long)tiles_k * tiles_n;
  const int z = (int)(blockIdx.x / tk_tn);
  const int r = (int)(blockIdx.x % tk_tn);
  const int k0 = (r / tiles_n) * 64, n0 = (r % tiles_n) * 64;
  const uint16_t* src = B + (long long)z * sB;
  uint16_t* dst = BT + (long long)z * N * K;
  const bool vec = ((ldb & 7) == 0) && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i, row = c >> 3, q = c & 7;
    const int k = k0 + row, n = n0 + q * 8;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (k < K) {
      const uint16_t* p = src + (long long)k * ldb + n;
      if (vec && n + 8 <= N) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < N) w[e >> 1] |= (uint32_t)p[e] << (16 * (e & 1));
      }
    }
    uint32_t* lp = reinterpret_cast<uint32_t*>(t + row * P + q * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) lp[e] = w[e];
  }
  __syncthreads();
  const bool ovec = ((K & 7) == 0) && ((reinterpret_cast<uintptr_t>(dst) & 15) == 0);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i, row = c >> 3, q = c & 7;  // row: n within the tile, q: 8 k
    const int n = n0 + row, k = k0 + q * 8;
    if (n >= N || k >= K) continue;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (uint32_t)t[(q * 8 + 2 * e) * P + row] | ((uint32_t)t[(q * 8 + 2 * e + 1) * P + row] << 16);
    uint16_t* p = dst + (long long)n * K + k;
    if (ovec && k + 8 <= K) {
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (k + e < K) p[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

hipError_t launch_kn_to_nk(const void* B, void* BT, int K, int N, long long ldb, long long sB, int batch,
                           hipStream_t s) {
  if (is_dry(s)) return hipSuccess;
  const int tk = (K + 63) / 64, tn = (N + 63) / 64;
  const long long grid = (long long)tk * tn * batch;
  if (grid >= (1LL << 31)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_kn_to_nk, dim3((unsigned)grid), dim3(256), 0, s, static_cast<const uint16_t*>(B),
                     static_cast<uint16_t*>(BT), K, N, ldb, sB, tk, tn);
  return hipGetLastError();
}

// ============================================================ wave-split kernel
// GEMMs with few output tiles -- convolutions as implicit im2col (B_CONV)
// or 1x1 (B_KN, the input plane as a [K, N] operand), small mm / addmm in
// either weight layout (B_KN, B_NK): a 20x20 to 80x80 map at
// batch 1 gives 25 to 400 tiles of 32 x 32 for 256 CUs, and a block of the
// tiled kernels above then waits out about one memory latency per K slice,
// its K slices one after another.  Here the W waves of a block share ONE
// output tile of (TM*32) x (TN*32) and split its K slices among themselves
// (wave w takes slices w, w+W, w+2W, ...).  Each wave loads its MFMA
// fragments from global memory straight into registers -- A rows as 16-byte
// chunks, B as 16-byte chunks of [N, K] rows or as element gathers (im2col
// taps through the per-launch tap table, kept in LDS, or n-strided rows);
// both layouts give every lane the same k run, so an mm gives the same bits
// with either weight layout -- with the next slice's loads in
// flight during the current slice's MFMAs; the K loop has no barrier.  After it every wave parks its partial
// sums in LDS and each wave finishes a share of the tile's register groups:
// the W partials are added in wave order (fixed, so the result does not
// depend on timing), then bias, activation, clamp and one rounding.
template <int DT, int BMODE, int TM, int TN, int W, bool SA>
__global__ __launch_bounds__(W * 64) void k_gemm_ws(KParams p) {
  constexpr int ES = DT == DT_F32 ? 4 : 2;
  constexpr int EPC = 16 / ES;     // elements per 16-byte chunk
  constexpr int BK = 128 / ES;     // k per slice
  constexpr int NG = TM * TN * 4;  // accumulator groups of 4 per lane
  constexpr int BM = TM * 32, BN = TN * 32;
  constexpr bool CONV = BMODE == B_CONV;
  constexpr bool NK = BMODE == B_NK;
  static_assert(SA || !NK, "[N, K] rows are always staged");
  constexpr int AROWS = SA ? TM * 32 + (NK ? TN * 32 : 0) : 0;  // rows staged per wave: A, and B for [N, K]
  // LDS: tap table (B_CONV) | per wave, its A (and [N, K] B) rows of one
  // slice (AROWS x 128 B, swizzled) | partial sums [W][NG][64] float4
  extern __shared__ uint4 ws_lds[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = p.M, N = p.N, K = p.K;
  const int KT = (K + BK - 1) / BK;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_mn = tiles_m * p.tiles_n;
  // XCD-aware numbering; m-tiles vary fastest, so the blocks of one XCD
  // share the B columns (the gathered operand) in its L2
  const int G = gridDim.x;
  const int rb = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int z = rb / tiles_mn, rt = rb - z * tiles_mn;
  const int m0 = (rt % tiles_m) * BM, n0 = (rt / tiles_m) * BN;

  const uint32_t* ktab = reinterpret_cast<const uint32_t*>(ws_lds);
  char* stage = reinterpret_cast<char*>(ws_lds + (CONV ? KT * BK / 4 : 0)) + wave * AROWS * 128;
  float4* part = reinterpret_cast<float4*>(ws_lds + (CONV ? KT * BK / 4 : 0) + W * AROWS * 8);

  const int fr = lane & 31, fc = lane >> 5;
  const int mrows = min(BM, M - m0);
  const rsrc_t ra = make_rsrc(reinterpret_cast<const char*>(p.A) + ((long long)z * p.sA + (long long)m0 * p.lda) * ES,
                              (uint32_t)((mrows - 1) * p.lda + K) * ES);
  // B_CONV: one input image; B_KN / B_NK: the [K, ldb] / [N, ldb] matrix
  // (ranges checked by the host)
  const rsrc_t rbs = make_rsrc(reinterpret_cast<const char*>(p.B) + (long long)z * p.sB * ES,
                               CONV ? p.b_bytes
                               : NK ? (uint32_t)((long long)(N - 1) * p.ldb + K) * ES
                                    : (uint32_t)((long long)(K - 1) * p.ldb + N) * ES);
  // SA: rows of A (and of a [N, K] B) are loaded coalesced, 8 lanes per
  // row's 128-byte slice, 8 rows per load instruction, and reach the MFMA
  // layout through the wave's LDS patch.  Without it each lane loads its MFMA
  // fragment directly (lane = row), 16 bytes from its own cache line: 64
  // lines per instruction, which measured as the address-FIFO bound of this
  // kernel on long K ranges and in fp32; on short fp16 ranges the LDS round
  // trip costs more than it saves.
  const int lr = lane >> 3, lc = lane & 7;  // row within 8, 16-byte chunk
  uint32_t aoff[TM * 4];
  bool aok[TM * 4];
#pragma unroll
  for (int q = 0; q < TM * 4; ++q) {
    const int row = SA ? q * 8 + lr : (q >> 2) * 32 + fr;
    aok[q] = row < mrows;
    aoff[q] = (uint32_t)(row * p.lda + (SA ? lc * EPC : 0)) * ES;
  }
  // per column: base offset of the output pixel's window and the mask of the
  // kernel taps that land inside the image (zero past N: every load reads 0)
  auto bias_at = [&](int idx) -> float {
    if constexpr (DT == DT_F32) return reinterpret_cast<const float*>(p.bias)[idx];
    else return to_f32<DT>(p.bias[idx]);
  };
  // the lane's per-row bias, fetched now: off the epilogue's critical path
  float brow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
    brow[i] = (p.bias_mode == BIAS_ROW && i * 32 + fr < mrows) ? p.beta * bias_at(m0 + i * 32 + fr) : 0.0f;
  int colbase[TN];
  unsigned long long cmask[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + j * 32 + fr;
    colbase[j] = 0;
    cmask[j] = 0ull;
    if (!CONV) {
      colbase[j] = col;
      cmask[j] = col < N ? ~0ull : 0ull;
    } else if (col < N) {
      const ConvGeom& g = p.g;
      const int oh = col / g.OW, ow = col - oh * g.OW;
      const int ih0 = oh * g.sH - g.pH, iw0 = ow * g.sW - g.pW;
      colbase[j] = ih0 * g.IW + iw0;
      for (int kh = 0; kh < g.KH; ++kh) {
        const int ih = ih0 + kh * g.dH;
        if (ih < 0 || ih >= g.IH) continue;
        for (int kw = 0; kw < g.KW; ++kw) {
          const int iw = iw0 + kw * g.dW;
          if (iw >= 0 && iw < g.IW) cmask[j] |= 1ull << (kh * g.KW + kw);
        }
      }
    }
  }
  struct Frag {
    uint4 a[TM * 4];                  // SA: row q*8 + lr, chunk lc; else MFMA fragment [i][kk] at i*4 + kk
    uint32_t b[TN][4][NK ? 1 : EPC];  // gathered elements
    uint4 bv[NK ? TN * 4 : 1];        // [N, K] rows, as A
  };
  // slice s: per k-step kk (16 bytes of k per lane), the lane's chunk kk*2+fc
  auto loadA = [&](Frag& F, int s) {
    if constexpr (SA) {
      const int kc = s * BK + lc * EPC;
#pragma unroll
      for (int q = 0; q < TM * 4; ++q) F.a[q] = ld_b128(ra, (aok[q] && kc < K) ? aoff[q] + (uint32_t)(s * BK) * ES : OOB);
    } else {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kc = s * BK + (kk * 2 + fc) * EPC;
#pragma unroll
        for (int i = 0; i < TM; ++i)
          F.a[i * 4 + kk] = ld_b128(ra, (aok[i * 4] && kc < K) ? aoff[i * 4] + (uint32_t)kc * ES : OOB);
      }
    }
  };
  auto loadB = [&](Frag& F, int s) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int kc = s * BK + (kk * 2 + fc) * EPC;
      if constexpr (CONV) {
        uint32_t ent[EPC];
#pragma unroll
        for (int q = 0; q < EPC; q += 4) {
          const uint4 e4 = *reinterpret_cast<const uint4*>(ktab + kc + q);
          ent[q] = e4.x;
          ent[q + 1] = e4.y;
          ent[q + 2] = e4.z;
          ent[q + 3] = e4.w;
        }
        // at most 31 taps (checked by the host; the table's padding entries,
        // tap 63, then read bit 31, never set): v_bfe_u32 reads the tap's
        // bit straight from the entry's low 5 bits, and a tap outside the
        // image sets bit 31 of the offset (out of range: reads 0) -- no
        // compare and select per element
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const uint32_t ok = __builtin_amdgcn_ubfe((uint32_t)cmask[j], ent[e], 1u);
            const uint32_t off = ((uint32_t)(colbase[j] + (int)(ent[e] >> 6)) * ES) | ((ok ^ 1u) << 31);
            F.b[j][kk][e] = ES == 4 ? ld_b32(rbs, off) : ld_b16(rbs, off);
          }
      } else if constexpr (NK) {
        if (kk == 0) {  // the [N, K] rows of the slice, coalesced like A
          const int kr = s * BK + lc * EPC;
#pragma unroll
          for (int q = 0; q < TN * 4; ++q) {
            const int n = n0 + q * 8 + lr;
            F.bv[q] = ld_b128(rbs, (n < N && kr < K) ? (uint32_t)(n * p.ldb + kr) * ES : OOB);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const uint32_t off = (cmask[j] && kc + e < K) ? (uint32_t)((kc + e) * p.ldb + colbase[j]) * ES : OOB;
            F.b[j][kk][e] = ES == 4 ? ld_b32(rbs, off) : ld_b16(rbs, off);
          }
      }
    }
  };
  auto load = [&](Frag& F, int s) {
    loadA(F, s);
    loadB(F, s);
  };
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  auto mma = [&](const Frag& F) {
    // SA: this wave's rows -> LDS (coalesced layout), back in the MFMA
    // layout: lane = row, chunk kk*2 + fc
    uint4 af[TM][4];
    if constexpr (SA) {
#pragma unroll
      for (int q = 0; q < TM * 4; ++q) *reinterpret_cast<uint4*>(stage + swz(q * 8 + lr, lc)) = F.a[q];
      if constexpr (NK) {
#pragma unroll
        for (int q = 0; q < TN * 4; ++q) *reinterpret_cast<uint4*>(stage + swz(TM * 32 + q * 8 + lr, lc)) = F.bv[q];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) af[i][kk] = *reinterpret_cast<const uint4*>(stage + swz(i * 32 + fr, kk * 2 + fc));
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) af[i][kk] = F.a[i * 4 + kk];
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        uint4 bq;
        if constexpr (NK)
          bq = *reinterpret_cast<const uint4*>(stage + swz(TM * 32 + j * 32 + fr, kk * 2 + fc));
        else if constexpr (ES == 4)
          bq = make_uint4(F.b[j][kk][0], F.b[j][kk][1], F.b[j][kk][2], F.b[j][kk][3]);
        else
          bq = make_uint4(pack2(F.b[j][kk][0], F.b[j][kk][1]), pack2(F.b[j][kk][2], F.b[j][kk][3]),
                          pack2(F.b[j][kk][4], F.b[j][kk][5]), pack2(F.b[j][kk][6], F.b[j][kk][7]));
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = mfma_frag<DT>(bq, af[i][kk], acc[i][j]);
      }
  };

  // two register sets: the loads of slice s+W fly while slice s is multiplied
  // The first slice's A loads go out before the tap table is staged in LDS.
  // (Measured on MI355X: this plain form beats an unconditional prefetch
  // and a schedule pinned with sched_barrier.  A slice is bound by the VALU
  // work of the gather addresses -- tap mask, offset, select: about 6
  // instructions per element, some 250 per slice against 128 MFMA cycles --
  // and 36 loads per slice in flight twice would pass the 63 that vmcnt
  // tracks.)
  Frag F0, F1;
  int s = wave;
  if (s < KT) loadA(F0, s);
  if constexpr (CONV) {
    for (int i = tid; i < KT * BK / 4; i += W * 64) ws_lds[i] = reinterpret_cast<const uint4*>(p.ktab)[i];
    __syncthreads();
  }
  if (s < KT) loadB(F0, s);
  while (s < KT) {
    if (s + W < KT) load(F1, s + W);
    mma(F0);
    s += W;
    if (s >= KT) break;
    if (s + W < KT) load(F0, s + W);
    mma(F1);
    s += W;
  }

  // partial sums -> LDS, then each wave reduces groups wave, wave+W, ...
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        part[(wave * NG + (i * TN + j) * 4 + g) * 64 + lane] =
            make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
  __syncthreads();

  const rsrc_t rc = make_rsrc(reinterpret_cast<char*>(p.C) + ((long long)z * p.sC + (long long)m0 * p.ldc + n0) * ES,
                              (uint32_t)((mrows - 1) * p.ldc + (N - n0)) * ES);
  const bool cvec = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & (4 * ES - 1)) == 0) &&
                    ((p.sC & 3) == 0) && ((N & 3) == 0);
  for (int q = wave; q < NG; q += W) {
    float4 v = part[q * 64 + lane];
    for (int w = 1; w < W; ++w) {
      const float4 t = part[(w * NG + q) * 64 + lane];
      v.x += t.x;
      v.y += t.y;
      v.z += t.z;
      v.w += t.w;
    }
    const int i = q / (TN * 4), j = (q >> 2) % TN, g = q & 3;
    const int row = i * 32 + fr;
    const int col = j * 32 + 8 * g + 4 * fc;
    if (row >= mrows) continue;
    float rowb = 0.0f;
#pragma unroll
    for (int ii = 0; ii < TM; ++ii)
      if (ii == i) rowb = brow[ii];
    const float vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = p.alpha * vv[e] + rowb;
      if (p.bias_mode == BIAS_COL && n0 + col + e < N) x += p.beta * bias_at(n0 + col + e);
      x = apply_act(p.act, x);
      if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
      if constexpr (DT == DT_F32) h[e] = __float_as_uint(x);
      else h[e] = st_bits<DT == DT_BF16>(x);
    }
    const uint32_t off = (uint32_t)(row * p.ldc + col) * ES;
    if (cvec) {
      if constexpr (DT == DT_F32)
        st_b128(make_uint4(h[0], h[1], h[2], h[3]), rc, n0 + col < N ? off : OOB);
      else
        st_b64(make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3])), rc, n0 + col < N ? off : OOB);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t oe = n0 + col + e < N ? off + ES * e : OOB;
        if constexpr (DT == DT_F32) st_b32(h[e], rc, oe);
        else st_b16(h[e], rc, oe);
      }
    }
  }
}

// Split-K reduction: C = epilogue(sum over ranges of ws[r]), the ranges
// summed in order 0..splits-1 so the result does not depend on scheduling.
// One thread per 4 consecutive outputs of a row.
template <int DT>
__global__ __launch_bounds__(256) void k_splitk_reduce(KParams p) {
  const int M = p.M, N = p.N, S = p.splits;
  const int nq = (N + 3) / 4;
  const long long total = (long long)p.batch * M * nq;
  const long long slab = (long long)p.batch * M * N;
  const bool n4 = (N & 3) == 0;  // rows of whole float4s: one 16-byte load per range
  char* Cb = reinterpret_cast<char*>(p.C);
  for (long long q = (long long)blockIdx.x * 256 + threadIdx.x; q < total; q += (long long)gridDim.x * 256) {
    const int n = (int)(q % nq) * 4;
    const long long zm = q / nq;
    const int m = (int)(zm % M), z = (int)(zm / M);
    const long long base = zm * N + n;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (n4) {
      float4 t[8];  // every range's load in flight before the sum (S <= 8)
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (r < S) t[r] = *reinterpret_cast<const float4*>(p.ws + (long long)r * slab + base);
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (r < S) {
          v[0] += t[r].x;
          v[1] += t[r].y;
          v[2] += t[r].z;
          v[3] += t[r].w;
        }
    } else {
      for (int r = 0; r < S; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) v[e] += p.ws[(long long)r * slab + base + e];
    }
    const long long cbase = (long long)z * p.sC + (long long)m * p.ldc + n;
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = p.alpha * v[e];
      if (n + e < N) {
        if (p.bias_mode == BIAS_ROW) {
          x += p.beta * (DT == DT_F32 ? reinterpret_cast<const float*>(p.bias)[m] : ld_f32<DT == DT_BF16>(p.bias[m]));
        } else if (p.bias_mode == BIAS_COL) {
          x += p.beta *
               (DT == DT_F32 ? reinterpret_cast<const float*>(p.bias)[n + e] : ld_f32<DT == DT_BF16>(p.bias[n + e]));
        }
      }
      x = apply_act(p.act, x);
      if (p.has_clamp) x = fminf(fmaxf(x, p.cmin), p.cmax);
      h[e] = DT == DT_F32 ? __float_as_uint(x) : (uint32_t)st_bits<DT == DT_BF16>(x);
    }
    const bool cv = n4 && ((p.ldc & 3) == 0) && ((p.sC & 3) == 0) &&
                    ((reinterpret_cast<uintptr_t>(p.C) & (4 * (DT == DT_F32 ? 4 : 2) - 1)) == 0);
    if constexpr (DT == DT_F32) {
      if (cv) *reinterpret_cast<uint4*>(reinterpret_cast<float*>(Cb) + cbase) = make_uint4(h[0], h[1], h[2], h[3]);
      else
        for (int e = 0; e < 4; ++e)
          if (n + e < N) reinterpret_cast<uint32_t*>(Cb)[cbase + e] = h[e];
    } else {
      if (cv) *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(Cb) + cbase) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
      else
        for (int e = 0; e < 4; ++e)
          if (n + e < N) reinterpret_cast<uint16_t*>(Cb)[cbase + e] = (uint16_t)h[e];
    }
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
  const size_t lds = stages + (size_t)(BM > BN ? BM : BN) * sizeof(float) +
                     (BMODE == B_CONV ? (size_t)conv_ktab_rows(kp.K) * sizeof(uint32_t) : 0);
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
  // group height: one XCD's share of a round (grid/8 tiles) as a rectangle
  // that is about square in elements
  {
    const int tiles_m = (kp.M + BM - 1) / BM;
    const double per_xcd = (double)(grid < 8 ? 1 : grid / 8);
    int gm = (int)lround(sqrt(per_xcd * BN / BM));
    k2.gm = gm < 1 ? 1 : (gm > tiles_m ? tiles_m : gm);
  }
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WGM * WGN * 64), lds, s, k2);
  return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int BMODE, bool BVEC, int DT, int NS = 3>
hipError_t launch_one3(const KParams& kp, int batch, hipStream_t s) {
  auto fn = k_gemm3<BM, BN, WGM, WGN, BMODE, BVEC, DT, NS>;
  const size_t dyn = BMODE == B_CONV ? (size_t)conv_ktab_rows(kp.K) * sizeof(uint32_t) : 0;
  // static LDS: the stages and two bias buffers
  constexpr size_t stat = (size_t)NS * (BM + BN) * 64 * 2 + 2 * (BM > BN ? BM : BN) * 4;
  if (stat + dyn > 160 * 1024) return hipErrorInvalidValue;
  static size_t attr_dyn = 0;  // largest dynamic size allowed so far
  if (dyn > attr_dyn && s != name_only()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn);
    if (e != hipSuccess) return e;
    attr_dyn = dyn;
  }
  if (is_dry(s)) return hipSuccess;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                   WGM * WGN * 64, dyn) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const long long ntiles = (long long)((kp.M + BM - 1) / BM) * kp.tiles_n * batch;
  long long grid = (long long)device_cus() * per_cu;
  if (grid > ntiles * kp.splits) grid = ntiles * kp.splits;
  KParams k2 = kp;
  k2.batch = batch;
  {
    const int tiles_m = (kp.M + BM - 1) / BM;
    const double per_xcd = (double)(grid < 8 ? 1 : grid / 8) / kp.splits;
    int gm = (int)lround(sqrt((per_xcd < 1 ? 1 : per_xcd) * BN / BM));
    k2.gm = gm < 1 ? 1 : (gm > tiles_m ? tiles_m : gm);
  }
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WGM * WGN * 64), dyn, s, k2);
  return hipGetLastError();
}

// Wave-split kernel configurations: wave tile (TM*32) x (TN*32), W waves.
struct WsCfg {
  int tm, tn, w;
};
constexpr WsCfg kWsCfgs[] = {{1, 1, 4}, {1, 1, 8}, {2, 1, 4}, {2, 1, 8}, {1, 2, 4}};

template <int DT, int BMODE, int TM, int TN, int W, bool SA>
hipError_t launch_ws(const KParams& kp, int batch, hipStream_t s) {
  auto fn = k_gemm_ws<DT, BMODE, TM, TN, W, SA>;
  constexpr int BK = DT == DT_F32 ? 32 : 64;
  const int kt = (kp.K + BK - 1) / BK;
  constexpr int AROWS = SA ? TM * 32 + (BMODE == B_NK ? TN * 32 : 0) : 0;
  const size_t dyn = (BMODE == B_CONV ? (size_t)kt * BK * 4 : 0) + (size_t)W * AROWS * 128 +
                     (size_t)W * TM * TN * 4 * 64 * 16;
  if (dyn > 160 * 1024) return hipErrorInvalidValue;
  static size_t attr_dyn = 0;  // largest dynamic size allowed so far
  if (dyn > attr_dyn && s != name_only()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn);
    if (e != hipSuccess) return e;
    attr_dyn = dyn;
  }
  if (is_dry(s)) return hipSuccess;
  KParams k2 = kp;
  k2.batch = batch;
  k2.tiles_n = (kp.N + TN * 32 - 1) / (TN * 32);
  const long long grid = (long long)((kp.M + TM * 32 - 1) / (TM * 32)) * k2.tiles_n * batch;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(W * 64), dyn, s, k2);
  return hipGetLastError();
}

template <int DT, int BMODE, bool SA>
hipError_t dispatch_ws(const WsCfg& c, const KParams& kp, int batch, hipStream_t s) {
  if (c.tm == 1 && c.tn == 1 && c.w == 4) return launch_ws<DT, BMODE, 1, 1, 4, SA>(kp, batch, s);
  if (c.tm == 1 && c.tn == 1 && c.w == 8) return launch_ws<DT, BMODE, 1, 1, 8, SA>(kp, batch, s);
  if (c.tm == 2 && c.tn == 1 && c.w == 4) return launch_ws<DT, BMODE, 2, 1, 4, SA>(kp, batch, s);
  if (c.tm == 2 && c.tn == 1 && c.w == 8) return launch_ws<DT, BMODE, 2, 1, 8, SA>(kp, batch, s);
  if (c.tm == 1 && c.tn == 2 && c.w == 4) return launch_ws<DT, BMODE, 1, 2, 4, SA>(kp, batch, s);
  return hipErrorNotSupported;
}

struct Tile {
  int bm, bn, wgm, wgn;
  bool autosel = true;  // considered by the automatic choice
};

constexpr Tile kTiles[] = {{256, 128, 4, 2},        {128, 256, 2, 4},        {256, 256, 2, 2, false},
                           {256, 128, 2, 2, false}, {128, 256, 2, 2, false}, {128, 128, 2, 2},
                           {128, 64, 2, 2},         {64, 64, 2, 2}};

bool use_v2();
bool getenv_is0(const char* name);

// LDS bytes of a block: three unpadded stages (pipelined kernel) or two padded
// ones (register-staged kernel), the bias buffers and the im2col table.
size_t tile_lds(const Tile& t, int bmode, int K) {
  const size_t stages = use_v2() ? (size_t)2 * (t.bm + t.bn) * RS * 2 : (size_t)3 * (t.bm + t.bn) * 64 * 2;
  return stages + (size_t)(t.bm > t.bn ? t.bm : t.bn) * 8 + (bmode == B_CONV ? (size_t)conv_ktab_rows(K) * 4 : 0);
}

// Picks the block tile: fewest rounds over the 256 CUs (a block of 8 waves
// fills a CU, two 4-wave blocks share one), weighted by tile area and a
// per-tile efficiency penalty for small tiles (less operand reuse).
Tile choose_tile(int M, int N, int K, int batch, bool avec, int bmode) {
  if (!avec) return {64, 64, 2, 2};
  const char* force = getenv("WGX_MFMA_TILE");
  if (force) {  // "BMxBNwW": block tile and wave count
    int bm = 0, bn = 0, w = 0;
    if (sscanf(force, "%dx%dw%d", &bm, &bn, &w) == 3)
      for (const Tile& t : kTiles)
        if (t.bm == bm && t.bn == bn && t.wgm * t.wgn == w && tile_lds(t, bmode, K) <= 160 * 1024) return t;
  }
  double best = 1e300;
  Tile bt = {64, 64, 2, 2};
  for (const Tile& t : kTiles) {
    if (!t.autosel || tile_lds(t, bmode, K) > 160 * 1024) continue;
    const long long tiles = (long long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    const int per_cu = t.wgm * t.wgn == 8 || tile_lds(t, bmode, K) > 80 * 1024 ? 1 : 2;
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

// True when the environment variable is set to "0".
bool getenv_is0(const char* name) {
  const char* v = getenv(name);
  return v && strcmp(v, "0") == 0;
}

bool use_v2() {
  static int v = -1;
  if (v < 0) v = getenv("WGX_GEMM_V2") ? 1 : 0;
  return v == 1;
}

// Pipelined kernel (16-byte-aligned A); nullopt-style hipErrorNotSupported
// when the tile has no pipelined instantiation.
template <int BMODE, bool BVEC, int DT>
hipError_t dispatch3(const Tile& t, const KParams& kp, int batch, hipStream_t s) {
  const int w = t.wgm * t.wgn;
  if (t.bm == 256 && t.bn == 128 && w == 8) return launch_one3<256, 128, 4, 2, BMODE, BVEC, DT>(kp, batch, s);
  if (t.bm == 128 && t.bn == 256 && w == 8) return launch_one3<128, 256, 2, 4, BMODE, BVEC, DT>(kp, batch, s);
  if (t.bm == 256 && t.bn == 128) return launch_one3<256, 128, 2, 2, BMODE, BVEC, DT>(kp, batch, s);
  if (t.bm == 128 && t.bn == 256) return launch_one3<128, 256, 2, 2, BMODE, BVEC, DT>(kp, batch, s);
  if (t.bm == 128 && t.bn == 128) return launch_one3<128, 128, 2, 2, BMODE, BVEC, DT>(kp, batch, s);
  if (t.bm == 128 && t.bn == 64) return launch_one3<128, 64, 2, 2, BMODE, BVEC, DT>(kp, batch, s);
  if (t.bm == 64 && t.bn == 64) return launch_one3<64, 64, 2, 2, BMODE, BVEC, DT>(kp, batch, s);
  return hipErrorNotSupported;
}

// Register-staged kernel (16-bit types), also the path for unaligned A.
template <int BMODE, bool AVEC, bool BVEC, bool BF>
hipError_t dispatch_tile(const Tile& t, const KParams& kp, int batch, hipStream_t s) {
  const int w = t.wgm * t.wgn;
  if constexpr (AVEC) {
    if (!use_v2()) {
      hipError_t e = dispatch3<BMODE, BVEC, BF ? DT_BF16 : DT_F16>(t, kp, batch, s);
      if (e != hipErrorNotSupported) return e;
    }
  }
  if (t.bm == 256 && t.bn == 128 && w == 8) return launch_one<256, 128, 4, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 256 && w == 8) return launch_one<128, 256, 2, 4, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if constexpr (BMODE != B_CONV) {
    if (t.bm == 256 && t.bn == 256) return launch_one<256, 256, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  }
  if (t.bm == 256 && t.bn == 128) return launch_one<256, 128, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 256) return launch_one<128, 256, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 128) return launch_one<128, 128, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  if (t.bm == 128 && t.bn == 64) return launch_one<128, 64, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
  return launch_one<64, 64, 2, 2, BMODE, AVEC, BVEC, BF>(kp, batch, s);
}

}  // namespace

namespace {

// What launch_gemm_mfma decides from the shapes alone.
struct Plan {
  bool f32, bf, avec, bvec;
  int es;
  Tile t;
  bool pipelined;  // runs k_gemm3 (split-K capable)
  bool big;        // runs k_gemm_nk with tile bt
  bool stage_b;    // big, on a [K, N] B rewritten as [N, K] first (k_kn_to_nk)
  Tile bt;
  bool sk;         // runs k_gemm_sk (K <= 64, a large output)
};

// Large-tile kernel shapes (one block of 4 waves per CU).
constexpr Tile kBigTiles[] = {{256, 192, 2, 2}, {192, 256, 2, 2}, {256, 128, 2, 2}};

// The cost model of choose_tile for one tile: rounds over the CUs times the
// tile area per round, weighted by the tile's operand-reuse penalty.
double tile_cost(const Tile& t, int M, int N, int batch, int per_cu) {
  const long long tiles = (long long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
  const double rounds = ceil((double)tiles / (256.0 * per_cu));
  return rounds * t.bm * t.bn * per_cu * (1.0 + 64.0 / t.bm + 64.0 / t.bn);
}

Plan make_plan(const GemmDesc& d) {
  Plan pl;
  pl.f32 = d.dtype == WGX_FLOAT32;
  pl.bf = d.dtype == WGX_BFLOAT16;
  pl.es = pl.f32 ? 4 : 2;
  const int epc = 16 / pl.es;
  const auto aligned16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  pl.avec = (d.K % epc == 0) && (d.lda % epc == 0) && (d.sA % epc == 0) && aligned16(d.A);
  if (d.bmode == B_NK)
    pl.bvec = (d.K % epc == 0) && (d.ldb % epc == 0) && (d.sB % epc == 0) && aligned16(d.B);
  else if (d.bmode == B_KN)
    pl.bvec = (d.N % epc == 0) && (d.ldb % epc == 0) && (d.sB % epc == 0) && aligned16(d.B);
  else
    pl.bvec = false;
  pl.t = choose_tile(d.M, d.N, d.K, d.batch, pl.avec, d.bmode);
  if (d.bmode != B_CONV && !pl.bvec) pl.t = {64, 64, 2, 2};
  if (pl.f32)
    pl.pipelined = pl.avec && (d.bmode != B_NK || pl.bvec);
  else
    pl.pipelined = pl.avec && pl.bvec == (d.bmode != B_CONV) && !use_v2() &&
                   !(pl.t.bm == 256 && pl.t.bn == 256);
  if (pl.bf && d.bmode == B_CONV) pl.pipelined = false;
  // the large-tile kernel for the [N, K] form when its tiles cost less; a
  // 16-byte-aligned [K, N] B takes it too, through the [N, K] staging pass
  // (WGX_KN_STAGE=0 keeps such GEMMs on k_gemm3)
  pl.big = false;
  pl.stage_b = false;
  const bool kn_stage = d.bmode == B_KN && pl.bvec && (d.K % epc == 0) && !getenv_is0("WGX_KN_STAGE");
  if (!pl.f32 && (d.bmode == B_NK || kn_stage) && pl.avec && pl.bvec && !use_v2()) {
    const int per_cu = pl.t.wgm * pl.t.wgn == 8 || tile_lds(pl.t, d.bmode, d.K) > 80 * 1024 ? 1 : 2;
    double best = tile_cost(pl.t, d.M, d.N, d.batch, per_cu);
    const char* force = getenv("WGX_MFMA_TILE");
    for (const Tile& t : kBigTiles) {
      const double c = tile_cost(t, d.M, d.N, d.batch, 1);
      bool take = c < best;
      if (force) {  // "BMxBNb" picks a large tile by name, any other value keeps k_gemm3's
        int bm = 0, bn = 0;
        char tag = 0;
        take = sscanf(force, "%dx%d%c", &bm, &bn, &tag) == 3 && tag == 'b' && bm == t.bm && bn == t.bn;
      }
      if (take) {
        best = c;
        pl.big = true;
        pl.bt = t;
      }
    }
    pl.stage_b = pl.big && d.bmode == B_KN;
  }
  // a short K (one LDS slice) and an output of at least 4 Mi elements: the
  // time is the output's, which the short-K kernel writes in whole rows.
  // WGX_SK=0 keeps such GEMMs on the kernels above, WGX_SK=1 takes the
  // short-K kernel for any output size.
  {
    const char* e = getenv("WGX_SK");
    const bool force = e && e[0] == '1';
    const bool cvec = (d.N % 8 == 0) && (d.ldc % 8 == 0) && (d.sC % 8 == 0) && aligned16(d.C);
    pl.sk = !pl.f32 && (d.bmode == B_NK || d.bmode == B_KN) && pl.avec && pl.bvec && cvec && d.K <= 64 &&
            (force || (long long)d.batch * d.M * d.N >= (4LL << 20)) && !getenv_is0("WGX_SK");
  }
  if (pl.sk) {
    pl.big = false;
    pl.stage_b = false;
  }
  return pl;
}

// Whether a launch runs the wave-split kernel, and with which configuration:
// convolutions (implicit im2col, fp32 / fp16) and fp32 GEMMs of either B
// layout whose 64 x 64 tiles number fewer than the CUs.  (An fp16 [K, N]
// operand loses here: its 2-byte gathers at stride N are slower than the
// tiled kernel's 16-byte row loads with an in-register transpose; [N, K]
// stays with it too, so an mm gives the same bits in either layout.)  The
// configuration aims at 1000-2000 waves: measured on MI355X over the 3x3
// and 1x1 convolutions of 20x20 to 80x80 maps, 32 x 32 tiles with 8 waves
// win up to one tile per CU, 64 x 32 tiles above that.  WGX_WS="off"
// disables the kernel, "TMxTNwW" forces a configuration wherever it applies.
bool ws_choice(const GemmDesc& d, const Plan& pl, WsCfg* cfg) {
  if (!pl.avec || pl.bf) return false;
  if (d.bmode == B_CONV) {
    if (!d.ktab || d.g.KH * d.g.KW > 31) return false;  // bit 31: the table's padding tap
  } else if (!pl.f32) {
    return false;
  } else if (d.bmode == B_KN) {
    // the [K, ldb] plane is one buffer range with 32-bit offsets
    if (((long long)(d.K - 1) * d.ldb + d.N) * pl.es >= (1LL << 31)) return false;
  } else {
    if (!pl.bvec || ((long long)(d.N - 1) * d.ldb + d.K) * pl.es >= (1LL << 31)) return false;
  }
  // the configuration's LDS: tap table, per-wave row patches, partial sums
  const auto fits = [&](const WsCfg& c) {
    const int bk = pl.f32 ? 32 : 64, kt = (d.K + bk - 1) / bk;
    const bool sa = pl.f32 || d.K >= 1024;  // as launch_gemm_mfma stages A
    const size_t rows = sa ? 32 * c.tm + (d.bmode == B_NK ? 32 * c.tn : 0) : 0;
    return (d.bmode == B_CONV ? (size_t)kt * bk * 4 : 0) + (size_t)c.w * rows * 128 +
               (size_t)c.w * c.tm * c.tn * 4 * 1024 <= 160 * 1024;
  };
  const char* force = getenv("WGX_WS");
  if (force) {
    if (strcmp(force, "off") == 0) return false;
    int tm = 0, tn = 0, w = 0;
    if (sscanf(force, "%dx%dw%d", &tm, &tn, &w) == 3)
      for (const WsCfg& c : kWsCfgs)
        if (c.tm == tm && c.tn == tn && c.w == w && fits(c)) {
          *cfg = c;
          return true;
        }
  }
  const long long cus = device_cus();
  const long long tiles64 = (long long)((d.M + 63) / 64) * ((d.N + 63) / 64) * d.batch;
  const long long tiles32 = (long long)((d.M + 31) / 32) * ((d.N + 31) / 32) * d.batch;
  const long long tiles2 = (long long)((d.M + 63) / 64) * ((d.N + 31) / 32) * d.batch;
  // a 16-bit convolution with at most 32 output channels wastes half of every
  // 64-row tile of the tiled kernel: 32 x 32 tiles of 4 waves here instead, however
  // many (measured on MI355X, fp16 [1,16,160,160]*[16,16,3,3] 9.6 -> 7.9 us,
  // [1,16,320,320]*[32,16,3,3] s2 9.9 -> 8.8 us)
  if (d.bmode == B_CONV && !pl.f32 && d.M <= 32 && tiles64 >= cus) {
    *cfg = WsCfg{1, 1, 4};
    return fits(*cfg);
  }
  if (tiles64 >= cus) return false;
  if (tiles32 <= cus) *cfg = WsCfg{1, 1, 8};
  else if (pl.f32) *cfg = WsCfg{2, 1, 4};
  else *cfg = tiles2 <= cus ? WsCfg{2, 1, 8} : WsCfg{2, 1, 4};
  // fewer K slices than waves (1x1 convolutions over few channels): the
  // 4-wave form of the same tile, the others would have no slice at all.
  // WGX_WS_FEW_K=n moves the threshold (0: always 8 waves).
  const int kt = (d.K + 128 / pl.es - 1) / (128 / pl.es);
  static const int few_k = [] {
    const char* v = getenv("WGX_WS_FEW_K");
    return v ? atoi(v) : 8;
  }();
  if (cfg->w == 8 && kt < few_k) cfg->w = 4;
  return fits(*cfg);
}

}  // namespace

// Split K when the tiles alone leave CUs idle: the number of ranges that
// brings the units nearest to one per CU (so 200 tiles on 256 CUs stay
// whole, 100 tiles become 300 units), each range at least 8 K slices long,
// at most 8 ranges.
size_t gemm_stage_b_bytes(const GemmDesc& d) {
  if (d.dtype == WGX_FLOAT32) return 0;
  const Plan pl = make_plan(d);
  return pl.stage_b ? (size_t)d.batch * d.N * d.K * 2 : 0;
}

int gemm_split_plan(const GemmDesc& d, size_t* ws_bytes) {
  *ws_bytes = 0;
  const Plan pl = make_plan(d);
  WsCfg wc;
  if (!pl.pipelined || pl.big || pl.sk || ws_choice(d, pl, &wc)) return 1;
  const long long ntiles =
      (long long)((d.M + pl.t.bm - 1) / pl.t.bm) * ((d.N + pl.t.bn - 1) / pl.t.bn) * d.batch;
  const int kt = (d.K + 128 / pl.es - 1) / (128 / pl.es);
  int splits = (int)((device_cus() + ntiles / 2) / ntiles);
  if (splits > kt / 8) splits = kt / 8;
  if (splits > 8) splits = 8;
  if (splits < 2) return 1;
  const int kchunk = (kt + splits - 1) / splits;
  splits = (kt + kchunk - 1) / kchunk;  // no empty range
  if (splits < 2) return 1;
  *ws_bytes = (size_t)splits * d.batch * d.M * d.N * sizeof(float);
  return splits;
}

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
  kp.act = d.act;
  kp.cmin = d.cmin;
  kp.cmax = d.cmax;
  kp.g = d.g;
  kp.gm = 1;
  kp.b_bytes = 0;
  // buffer offsets are 31-bit: a tile's rows of A / B, a slice's rows of a
  // [K,N] operand and one im2col input image must stay below 2 GiB
  if (d.lda >= (1LL << 22) || d.ldb >= (1LL << 22)) return hipErrorInvalidValue;
  const Plan pl = make_plan(d);
  const bool f32 = pl.f32, bf = pl.bf, avec = pl.avec, bvec = pl.bvec;
  const int es = pl.es;
  const Tile t = pl.t;
  if (d.bmode == B_CONV) {
    const long long img = (long long)d.K / (d.g.KH * d.g.KW) * d.g.IH * d.g.IW * es;
    if (img >= (1LL << 31)) return hipErrorInvalidValue;
    kp.b_bytes = (uint32_t)img;
  }
  // fp32 runs only on the pipelined kernel: A (and a [N,K] B) must be
  // 16-byte vectors; the caller takes the vector-FMA kernel otherwise
  if (f32 && !pl.pipelined) return hipErrorNotSupported;
  kp.tiles_n = (d.N + t.bn - 1) / t.bn;
  kp.splits = 1;
  kp.kchunk = 1 << 30;
  kp.ws = nullptr;
  if (d.splits > 1) {
    if (!pl.pipelined || !d.ws) return hipErrorInvalidValue;
    const int kt = (d.K + 128 / es - 1) / (128 / es);
    kp.splits = d.splits;
    kp.kchunk = (kt + d.splits - 1) / d.splits;
    kp.ws = d.ws;
  }
  kp.nt_store = 0;
  if (pl.sk && d.splits <= 1) {
    kp.tiles_n = (d.N + 127) / 128;
    kp.batch = d.batch;
    // outputs of at least 8 MB are written past the caches (bmm config 4:
    // 18.0 -> 15.7 us measured on MI355X)
    kp.nt_store = (long long)d.batch * d.M * d.N * es >= (8LL << 20) ? 1 : 0;
    if (name) {
      char buf[96];
      snprintf(buf, sizeof buf, "gemm_mfma_%s_128x128w4_%s_sk", bf ? "bf16" : "f16", d.bmode == B_KN ? "kn" : "nk");
      *name = buf;
    }
    if (d.bmode == B_KN) return bf ? launch_sk<true, true>(kp, d.batch, s) : launch_sk<false, true>(kp, d.batch, s);
    return bf ? launch_sk<true, false>(kp, d.batch, s) : launch_sk<false, false>(kp, d.batch, s);
  }
  if (pl.big && d.splits <= 1) {
    // output of at least 8 MB: written past the caches (it does not fit the
    // L2s and the next kernel streams it from HBM either way)
    kp.nt_store = (long long)d.batch * d.M * d.N * es >= (8LL << 20) ? 1 : 0;
    const Tile& b = pl.bt;
    kp.tiles_n = (d.N + b.bn - 1) / b.bn;
    if (name) {
      char buf[96];
      snprintf(buf, sizeof buf, "gemm_mfma_%s_%dx%dw%d_%snk_big", bf ? "bf16" : "f16", b.bm, b.bn,
               b.bm == 256 && b.bn == 192 ? 8 : 4, pl.stage_b ? "kn2" : "");
      *name = buf;
    }
    if (pl.stage_b) {
      // B [K, N] -> workspace [N, K] on the same stream, then the [N, K] kernel
      if (!d.bt) return is_dry(s) ? hipSuccess : hipErrorInvalidValue;
      const hipError_t e = launch_kn_to_nk(d.B, d.bt, d.K, d.N, d.ldb, d.sB, d.batch, s);
      if (e != hipSuccess) return e;
      kp.B = static_cast<const uint16_t*>(d.bt);
      kp.ldb = d.K;
      kp.sB = (long long)d.N * d.K;
    }
    // 128-byte LDS rows (8 full lines per DMA instruction) and two stages:
    // measured slightly ahead of 64-byte rows with five stages on MI355X
    if (b.bm == 256 && b.bn == 192)
      return bf ? launch_nk<256, 192, 4, 2, true, 2, 128>(kp, d.batch, s) : launch_nk<256, 192, 4, 2, false, 2, 128>(kp, d.batch, s);
    if (b.bm == 256 && b.bn == 128)
      return bf ? launch_nk<256, 128, 2, 2, true, 3, 128>(kp, d.batch, s) : launch_nk<256, 128, 2, 2, false, 3, 128>(kp, d.batch, s);
    return bf ? launch_nk<192, 256, 2, 2, true, 5, 64>(kp, d.batch, s) : launch_nk<192, 256, 2, 2, false, 5, 64>(kp, d.batch, s);
  }
  WsCfg wc;
  if (d.splits <= 1 && ws_choice(d, pl, &wc)) {
    if (name) {
      char buf[96];
      snprintf(buf, sizeof buf, "gemm_mfma_%s_%dx%dw%d_%s_ws", f32 ? "f32" : "f16", 32 * wc.tm, 32 * wc.tn, wc.w,
               d.bmode == B_CONV ? "conv" : (d.bmode == B_NK ? "nk" : "kn"));
      *name = buf;
    }
    kp.tiles_n = (d.N + 32 * wc.tn - 1) / (32 * wc.tn);
    // A rows staged through LDS: fp32 always, fp16 on long K ranges
    // (measured on MI355X: ahead from K = 1152, behind at K = 576)
    if (d.bmode == B_CONV) {
      if (f32) return dispatch_ws<DT_F32, B_CONV, true>(wc, kp, d.batch, s);
      return d.K >= 1024 ? dispatch_ws<DT_F16, B_CONV, true>(wc, kp, d.batch, s)
                         : dispatch_ws<DT_F16, B_CONV, false>(wc, kp, d.batch, s);
    }
    if (!f32) return hipErrorNotSupported;
    if (d.bmode == B_NK) return dispatch_ws<DT_F32, B_NK, true>(wc, kp, d.batch, s);
    return dispatch_ws<DT_F32, B_KN, true>(wc, kp, d.batch, s);
  }
  const bool knv = d.bmode == B_KN && bvec;
  if (name) {
    char buf[96];
    static const char* modes[] = {"nk", "kn", "conv"};
    char split[16] = "";
    if (kp.splits > 1) snprintf(split, sizeof split, "_k%d", kp.splits);
    snprintf(buf, sizeof buf, "gemm_mfma_%s_%dx%dw%d_%s%s%s%s", f32 ? "f32" : (bf ? "bf16" : "f16"), t.bm,
             t.bn, t.wgm * t.wgn, modes[d.bmode], d.bmode == B_KN ? (knv ? "4x8" : "col") : "",
             avec ? "" : "_scalarA", split);
    *name = buf;
  }
  if (bf && d.bmode == B_CONV) return hipErrorInvalidValue;  // bf16 convolution is not offered
  if (kp.splits > 1) {
    // split-K: the GEMM writes per-range partial sums, a second kernel reduces
    hipError_t e;
    const int dt = f32 ? DT_F32 : (bf ? DT_BF16 : DT_F16);
    if (dt == DT_F32) {
      e = d.bmode == B_NK ? dispatch3<B_NK, true, DT_F32>(t, kp, d.batch, s)
          : d.bmode == B_KN ? (bvec ? dispatch3<B_KN, true, DT_F32>(t, kp, d.batch, s)
                                    : dispatch3<B_KN, false, DT_F32>(t, kp, d.batch, s))
                            : dispatch3<B_CONV, false, DT_F32>(t, kp, d.batch, s);
    } else if (dt == DT_BF16) {
      e = d.bmode == B_NK ? dispatch3<B_NK, true, DT_BF16>(t, kp, d.batch, s)
                          : dispatch3<B_KN, true, DT_BF16>(t, kp, d.batch, s);
    } else {
      e = d.bmode == B_NK ? dispatch3<B_NK, true, DT_F16>(t, kp, d.batch, s)
          : d.bmode == B_KN ? dispatch3<B_KN, true, DT_F16>(t, kp, d.batch, s)
                            : dispatch3<B_CONV, false, DT_F16>(t, kp, d.batch, s);
    }
    if (e != hipSuccess || is_dry(s)) return e;
    KParams kr = kp;
    kr.batch = d.batch;
    const long long total = (long long)d.batch * d.M * ((d.N + 3) / 4);
    long long grid = (total + 255) / 256;
    if (grid > 64LL * device_cus()) grid = 64LL * device_cus();
    if (dt == DT_F32) hipLaunchKernelGGL(k_splitk_reduce<DT_F32>, dim3((unsigned)grid), dim3(256), 0, s, kr);
    else if (dt == DT_BF16) hipLaunchKernelGGL(k_splitk_reduce<DT_BF16>, dim3((unsigned)grid), dim3(256), 0, s, kr);
    else hipLaunchKernelGGL(k_splitk_reduce<DT_F16>, dim3((unsigned)grid), dim3(256), 0, s, kr);
    return hipGetLastError();
  }
  if (f32) {
    if (d.bmode == B_NK) return dispatch3<B_NK, true, DT_F32>(t, kp, d.batch, s);
    if (d.bmode == B_KN)
      return bvec ? dispatch3<B_KN, true, DT_F32>(t, kp, d.batch, s)
                  : dispatch3<B_KN, false, DT_F32>(t, kp, d.batch, s);
    return dispatch3<B_CONV, false, DT_F32>(t, kp, d.batch, s);
  }
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
    if (!bvec)
      return bf ? launch_one<64, 64, 2, 2, B_KN, true, false, true>(kp, d.batch, s)
                : launch_one<64, 64, 2, 2, B_KN, true, false, false>(kp, d.batch, s);
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
