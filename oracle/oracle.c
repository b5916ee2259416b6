/*
 * oracle.c -- CPU oracle for the GEMM-shaped hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This file is the checker, never the product.  Only tests/, the smoke check
 * in __graft_entry__.py and the cpu_baseline leg of bench.py may load it.  The
 * product path (wgpu-executorch_amd/) never links or calls it and fails loudly
 * when its HIP library is missing.
 *
 * It holds three things:
 *
 *  1. Number formats: IEEE binary16 / bfloat16 round-to-nearest-even
 *     conversions, written from the IEEE 754 definition.
 *
 *  2. fp64 brute force with PyTorch semantics (the primary parity target):
 *       orc_gemm_f64          mm / addmm / bmm, NN and NT weight layouts
 *       orc_conv2d_f64        dense / grouped / depthwise conv2d, NCHW, OIHW
 *       orc_conv_transpose2d_f64   transposed conv, written in SCATTER form
 *     Each also returns the componentwise magnitude sum (|A|.|B|)_ij that the
 *     tolerance bounds are scaled by.
 *
 *  3. A restatement of the reference WGSL kernels' arithmetic ("wgsl-emu"):
 *     the same accumulation order and the same rounding to the storage dtype
 *     after every operation (f16 kernels accumulate in f16).  Every WGSL
 *     kernel family on the path accumulates sequentially in k, so the emulator
 *     is an order-faithful sequential loop; it is also the CPU baseline that
 *     bench.py times.  f16 arithmetic is emulated by doing each operation in
 *     binary32 and rounding to binary16; since 24 >= 2*11+2 that double
 *     rounding is innocuous for +, -, * (Figueroa 1995), so each emulated f16
 *     op equals a native f16 op.  Built with -ffp-contract=off so no product
 *     is fused into an add.
 *
 * Pinning (tests/test_oracle.py): the reference's own known-answer tests
 * (tests/golden/reference_kats.json), torch float64 conv2d / conv_transpose2d
 * / matmul on the CPU as an independent library, closed forms (A.I = A, 1x1
 * identity conv, one-hot depthwise shifts) and numpy float64 brute force.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* 1. number formats                                                         */
/* ------------------------------------------------------------------------ */

/* binary32 -> binary16, round to nearest, ties to even (IEEE 754-2008 4.3.1). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan */
    return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) /* >= 65520 rounds to inf (65504 has an odd significand) */
    return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) { /* below 2^-14: binary16 subnormal, unit 2^-24 */
    float v;
    memcpy(&v, &ax, 4);
    float s = v * 16777216.0f; /* exact: scaling by a power of two */
    uint32_t m = (uint32_t)rintf(s); /* default rounding mode is RNE */
    return (uint16_t)(sign | m);
  }
  uint32_t e = (ax >> 23) - 127u + 15u;
  uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may bump the exponent */
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float r;
  if (e == 0)
    r = ldexpf((float)m, -24);
  else if (e == 31)
    r = m ? NAN : INFINITY;
  else
    r = ldexpf((float)(m | 0x400u), (int)e - 25);
  return (h & 0x8000u) ? -r : r;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t x = (uint32_t)h << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

/* storage-dtype rounding: 0 = float32, 1 = float16, 2 = bfloat16 */
static inline float rnd(int dt, float v) {
  if (dt == 1) return orc_f16_to_f32(orc_f32_to_f16(v));
  if (dt == 2) return orc_bf16_to_f32(orc_f32_to_bf16(v));
  return v;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* 2. fp64 brute force                                                       */
/* ------------------------------------------------------------------------ */

/*
 * C[b][i][n] = sum_k A[b][i][k] * B[b](k,n)  (+ bias)
 *   A row-major [M,K], batch stride sA elements (0 = shared across batch)
 *   B: b_trans == 0 -> row-major [K,N]  (aten.mm / aten.bmm operand,
 *                                        src/shaders/mm/index.ts:44-53)
 *      b_trans == 1 -> row-major [N,K]  (nn.Linear weight; the reference
 *                                        reaches it via permute_copy then mm,
 *                                        src/shaders/permute/index.ts:77-99)
 *   bias_mode 0 none, 1 per column bias[N] (addmm), 2 per row bias[M]
 *   rows: optional subset of row indices (nrows of them); output row r of C
 *         then holds A-row rows[r].  NULL -> all M rows.
 *   C, Cabs: [batch][nrows][N] doubles; Cabs = sum_k |A||B| + |bias|.
 */
void orc_gemm_f64(int batch, int M, int N, int K, const float* A, int64_t sA, const float* B,
                  int64_t sB, int b_trans, const float* bias, int bias_mode, double* C,
                  double* Cabs, const int* rows, int nrows) {
  if (!rows) nrows = M;
  int64_t total = (int64_t)batch * nrows;
#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)N * 2);
    double* aab = acc + N;
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < total; ++t) {
      int b = (int)(t / nrows), r = (int)(t % nrows);
      int i = rows ? rows[r] : r;
      const float* Ar = A + b * sA + (int64_t)i * K;
      const float* Bb = B + b * sB;
      for (int n = 0; n < N; ++n) acc[n] = aab[n] = 0.0;
      if (!b_trans) {
        for (int k = 0; k < K; ++k) {
          double a = Ar[k], aa = fabs(a);
          const float* Bk = Bb + (int64_t)k * N;
          for (int n = 0; n < N; ++n) {
            acc[n] += a * (double)Bk[n];
            aab[n] += aa * fabs((double)Bk[n]);
          }
        }
      } else {
        for (int n = 0; n < N; ++n) {
          const float* Bn = Bb + (int64_t)n * K;
          double s = 0.0, sa = 0.0;
          for (int k = 0; k < K; ++k) {
            s += (double)Ar[k] * (double)Bn[k];
            sa += fabs((double)Ar[k]) * fabs((double)Bn[k]);
          }
          acc[n] = s;
          aab[n] = sa;
        }
      }
      double* Cr = C + t * N;
      double* Ca = Cabs ? Cabs + t * N : NULL;
      for (int n = 0; n < N; ++n) {
        double bv = 0.0;
        if (bias_mode == 1) bv = bias[n];
        if (bias_mode == 2) bv = bias[i];
        Cr[n] = acc[n] + bv;
        if (Ca) Ca[n] = aab[n] + fabs(bv);
      }
    }
    free(acc);
  }
}

/*
 * Conv parameter block, in the reference's ConvParams word order
 * (src/shaders/convolution/index.ts:151-162):
 *   p[0..16] = B, IC, IH, IW, OC, OH, OW, KH, KW, sH, sW, pH, pW, dH, dW, groups, has_bias
 */
enum { P_B, P_IC, P_IH, P_IW, P_OC, P_OH, P_OW, P_KH, P_KW, P_SH, P_SW, P_PH, P_PW, P_DH, P_DW, P_G, P_HB };

/*
 * Direct conv2d (cross-correlation, PyTorch F.conv2d semantics), any groups,
 * stride, padding, dilation; zero padding.  x NCHW [B,IC,IH,IW], w OIHW
 * [OC, IC/groups, KH, KW], y NCHW [B,OC,OH,OW].  Output size follows
 * floor((I + 2p - d(K-1) - 1)/s) + 1 (src/shaders/convolution/index.ts:130-139),
 * taken from p[] as given.
 */
void orc_conv2d_f64(const int* p, const float* x, const float* w, const float* bias, double* y,
                    double* yabs) {
  int B = p[P_B], IC = p[P_IC], IH = p[P_IH], IW = p[P_IW], OC = p[P_OC], OH = p[P_OH],
      OW = p[P_OW], KH = p[P_KH], KW = p[P_KW], sH = p[P_SH], sW = p[P_SW], pH = p[P_PH],
      pW = p[P_PW], dH = p[P_DH], dW = p[P_DW], G = p[P_G], hb = p[P_HB];
  int icpg = IC / G, ocpg = OC / G;
  int64_t planes = (int64_t)B * OC;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t pl = 0; pl < planes; ++pl) {
    int b = (int)(pl / OC), oc = (int)(pl % OC), g = oc / ocpg;
    for (int oh = 0; oh < OH; ++oh)
      for (int ow = 0; ow < OW; ++ow) {
        double s = hb ? (double)bias[oc] : 0.0, sa = fabs(s);
        for (int icg = 0; icg < icpg; ++icg) {
          int ic = g * icpg + icg;
          for (int kh = 0; kh < KH; ++kh) {
            int ih = oh * sH - pH + kh * dH;
            if (ih < 0 || ih >= IH) continue;
            for (int kw = 0; kw < KW; ++kw) {
              int iw = ow * sW - pW + kw * dW;
              if (iw < 0 || iw >= IW) continue;
              double xv = x[(((int64_t)b * IC + ic) * IH + ih) * IW + iw];
              double wv = w[(((int64_t)oc * icpg + icg) * KH + kh) * KW + kw];
              s += xv * wv;
              sa += fabs(xv) * fabs(wv);
            }
          }
        }
        int64_t o = (pl * OH + oh) * OW + ow;
        y[o] = s;
        if (yabs) yabs[o] = sa;
      }
  }
}

/*
 * Transposed conv2d (PyTorch F.conv_transpose2d semantics), written in
 * SCATTER form: every input pixel adds x*w into the outputs it reaches.  The
 * reference kernel is the gather form (src/shaders/convolution/
 * conv-transpose2d.wgsl.ts:48-99); using the other form here means the two
 * formulations check each other.  w [IC, OC/groups, KH, KW]; OH/OW from p[].
 */
void orc_conv_transpose2d_f64(const int* p, const float* x, const float* w, const float* bias,
                              double* y, double* yabs) {
  int B = p[P_B], IC = p[P_IC], IH = p[P_IH], IW = p[P_IW], OC = p[P_OC], OH = p[P_OH],
      OW = p[P_OW], KH = p[P_KH], KW = p[P_KW], sH = p[P_SH], sW = p[P_SW], pH = p[P_PH],
      pW = p[P_PW], dH = p[P_DH], dW = p[P_DW], G = p[P_G], hb = p[P_HB];
  int icpg = IC / G, ocpg = OC / G;
  int64_t n = (int64_t)B * OC * OH * OW;
  for (int64_t i = 0; i < n; ++i) {
    int oc = (int)((i / ((int64_t)OH * OW)) % OC);
    y[i] = hb ? (double)bias[oc] : 0.0;
    if (yabs) yabs[i] = fabs(y[i]);
  }
  for (int b = 0; b < B; ++b)
    for (int ic = 0; ic < IC; ++ic) {
      int g = ic / icpg;
      for (int ih = 0; ih < IH; ++ih)
        for (int iw = 0; iw < IW; ++iw) {
          double xv = x[(((int64_t)b * IC + ic) * IH + ih) * IW + iw];
          for (int ocg = 0; ocg < ocpg; ++ocg) {
            int oc = g * ocpg + ocg;
            for (int kh = 0; kh < KH; ++kh) {
              int oh = ih * sH - pH + kh * dH;
              if (oh < 0 || oh >= OH) continue;
              for (int kw = 0; kw < KW; ++kw) {
                int ow = iw * sW - pW + kw * dW;
                if (ow < 0 || ow >= OW) continue;
                double wv = w[(((int64_t)ic * ocpg + ocg) * KH + kh) * KW + kw];
                int64_t o = (((int64_t)b * OC + oc) * OH + oh) * OW + ow;
                y[o] += xv * wv;
                if (yabs) yabs[o] += fabs(xv) * fabs(wv);
              }
            }
          }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* 3. wgsl-emu: the reference kernels' arithmetic, order-faithful            */
/* ------------------------------------------------------------------------ */

/*
 * mm / bmm, every variant (tiled, vec4, 64x64; f32 and f16).
 * All variants accumulate each output sequentially in k from a zero
 * accumulator of the storage type, one product then one add per step:
 *   mm-64x64.wgsl.ts:88-91 and mm-64x64-f16.wgsl.ts:90-93
 *     acc = acc + b0*a.x + b1*a.y + b2*a.z + b3*a.w   (left to right)
 *   mm-vec4.wgsl.ts:76 (the same four-term form), mm-tiled.wgsl.ts:72-79 (acc + aval*b)
 *   bmm-64x64 / bmm-vec4 / bmm-tiled: the same bodies per batch.
 * Zero-padded tails add 0*0, which leaves the accumulator unchanged, so the
 * variant choice (mm/index.ts:65-78) does not change the result.
 * dt: 0 f32, 1 f16.  Inputs are float arrays holding dt-representable values;
 * output likewise.  b_trans = 1 reads B as [N,K] (the permute_copy'd weight).
 */
void orc_emu_gemm(int dt, int batch, int M, int N, int K, const float* A, int64_t sA,
                  const float* B, int64_t sB, int b_trans, float* C, const int* rows,
                  int nrows) {
  if (!rows) nrows = M;
  int64_t total = (int64_t)batch * nrows;
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)N);
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < total; ++t) {
      int b = (int)(t / nrows), r = (int)(t % nrows);
      int i = rows ? rows[r] : r;
      const float* Ar = A + b * sA + (int64_t)i * K;
      const float* Bb = B + b * sB;
      for (int n = 0; n < N; ++n) acc[n] = 0.0f;
      if (dt == 0) {
        if (!b_trans) {
          for (int k = 0; k < K; ++k) {
            float a = Ar[k];
            const float* Bk = Bb + (int64_t)k * N;
            for (int n = 0; n < N; ++n) acc[n] = acc[n] + Bk[n] * a;
          }
        } else {
          for (int n = 0; n < N; ++n) {
            float s = 0.0f;
            for (int k = 0; k < K; ++k) s = s + Bb[(int64_t)n * K + k] * Ar[k];
            acc[n] = s;
          }
        }
      } else {
        for (int k = 0; k < K; ++k) {
          float a = Ar[k];
          for (int n = 0; n < N; ++n) {
            float bv = b_trans ? Bb[(int64_t)n * K + k] : Bb[(int64_t)k * N + n];
            acc[n] = rnd(dt, acc[n] + rnd(dt, bv * a));
          }
        }
      }
      memcpy(C + t * N, acc, sizeof(float) * (size_t)N);
    }
    free(acc);
  }
}

/*
 * addmm as the reference would have to compose it (it has no addmm operator,
 * src/shaders/index.ts:39-51):  t = mm(X, W)  rounded to the storage dtype,
 * then aten.add.Tensor with broadcast bias: out = t + dt(alpha) * bias
 * (add-broadcast-f16.wgsl.ts:33-58 with alpha = 1).  The W^T form first goes
 * through permute_copy (an exact copy), so it has the same numerics.
 */
void orc_emu_addmm(int dt, int M, int N, int K, const float* X, const float* W, int w_trans,
                   const float* bias, float* out, const int* rows, int nrows) {
  if (!rows) nrows = M;
  orc_emu_gemm(dt, 1, M, N, K, X, 0, W, 0, w_trans, out, rows, nrows);
  int64_t total = (int64_t)nrows * N;
#pragma omp parallel for
  for (int64_t t = 0; t < total; ++t) {
    int n = (int)(t % N);
    out[t] = rnd(dt, out[t] + rnd(dt, 1.0f * bias[n]));
  }
}

/*
 * convolution, following the variant the reference driver selects
 * (src/shaders/convolution/index.ts:171-238):
 *  - transposed: gather form, bias first; the f16 twin accumulates in f32
 *    and rounds once (conv-transpose2d-f16.wgsl.ts:62-95).
 *  - depthwise (groups == OC == IC, weight dim1 == 1, KH*KW <= 49): bias
 *    first, then taps kh-outer / kw-inner, out-of-bounds taps skipped
 *    (conv2d-depthwise.wgsl.ts:77-129; the 3x3 halo kernel sums row 0..2 in
 *    the same order, conv2d-depthwise-3x3-f16.wgsl.ts:78-128).
 *  - groups == 1 (1x1 tile32/tile64/vec4/scalar, dense tile32/tile64, GEMM):
 *    zero accumulator, k = (ic, kh, kw) in order, padding taps read as 0,
 *    bias added once at the end (conv2d-tile64.wgsl.ts:130-164,
 *    conv2d-gemm.wgsl.ts:147-164, conv2d-1x1.wgsl.ts final loop).
 *  - other groups: direct kernel, bias first then (icg, kh, kw) skipping
 *    out-of-bounds taps (conv2d.wgsl.ts:61-88).
 * dt: 0 f32, 1 f16.
 */
void orc_emu_conv2d(int dt, const int* p, int transposed, const float* x, const float* w,
                    const float* bias, float* y) {
  int B = p[P_B], IC = p[P_IC], IH = p[P_IH], IW = p[P_IW], OC = p[P_OC], OH = p[P_OH],
      OW = p[P_OW], KH = p[P_KH], KW = p[P_KW], sH = p[P_SH], sW = p[P_SW], pH = p[P_PH],
      pW = p[P_PW], dH = p[P_DH], dW = p[P_DW], G = p[P_G], hb = p[P_HB];
  int icpg = IC / G, ocpg = OC / G;
  int depthwise = !transposed && G == OC && IC == OC && icpg == 1 && KH * KW <= 49 &&
                  (int64_t)B * OC <= 65535;
  int64_t planes = (int64_t)B * OC;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t pl = 0; pl < planes; ++pl) {
    int b = (int)(pl / OC), oc = (int)(pl % OC), g = oc / ocpg;
    float bv = hb ? bias[oc] : 0.0f;
    for (int oh = 0; oh < OH; ++oh)
      for (int ow = 0; ow < OW; ++ow) {
        float acc;
        if (transposed) {
          float a32 = bv;
          int oc_in_g = oc % ocpg;
          for (int kh = 0; kh < KH; ++kh) {
            int nh = oh + pH - kh * dH;
            if (nh % sH != 0) continue;
            int ih = nh / sH;
            if (ih < 0 || ih >= IH) continue;
            for (int kw = 0; kw < KW; ++kw) {
              int nw = ow + pW - kw * dW;
              if (nw % sW != 0) continue;
              int iw = nw / sW;
              if (iw < 0 || iw >= IW) continue;
              for (int icg = 0; icg < icpg; ++icg) {
                int ic = g * icpg + icg;
                float xv = x[(((int64_t)b * IC + ic) * IH + ih) * IW + iw];
                float wv = w[(((int64_t)ic * ocpg + oc_in_g) * KH + kh) * KW + kw];
                if (dt == 0)
                  a32 = a32 + xv * wv;
                else
                  a32 = a32 + xv * wv; /* f32 accumulate in the f16 twin too */
              }
            }
          }
          acc = rnd(dt, a32);
        } else if (depthwise || G != 1) {
          acc = bv;
          for (int icg = 0; icg < icpg; ++icg) {
            int ic = g * icpg + icg;
            for (int kh = 0; kh < KH; ++kh) {
              int ih = oh * sH - pH + kh * dH;
              if (ih < 0 || ih >= IH) continue;
              for (int kw = 0; kw < KW; ++kw) {
                int iw = ow * sW - pW + kw * dW;
                if (iw < 0 || iw >= IW) continue;
                float xv = x[(((int64_t)b * IC + ic) * IH + ih) * IW + iw];
                float wv = w[(((int64_t)oc * icpg + icg) * KH + kh) * KW + kw];
                acc = rnd(dt, acc + rnd(dt, xv * wv));
              }
            }
          }
        } else {
          acc = 0.0f;
          for (int ic = 0; ic < IC; ++ic)
            for (int kh = 0; kh < KH; ++kh) {
              int ih = oh * sH - pH + kh * dH;
              for (int kw = 0; kw < KW; ++kw) {
                int iw = ow * sW - pW + kw * dW;
                if (ih < 0 || ih >= IH || iw < 0 || iw >= IW) continue;
                float xv = x[(((int64_t)b * IC + ic) * IH + ih) * IW + iw];
                float wv = w[(((int64_t)oc * IC + ic) * KH + kh) * KW + kw];
                acc = rnd(dt, acc + rnd(dt, xv * wv));
              }
            }
          acc = rnd(dt, acc + bv);
        }
        y[(pl * OH + oh) * OW + ow] = acc;
      }
  }
}
