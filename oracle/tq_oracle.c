/*
 * tq_oracle.c -- CPU restatement of TileQuant's mixed INT8/BF16 tile path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (tilequant_amd/) links,
 * loads or calls this file.  It is used by tests/ as the checker, by
 * __graft_entry__.smoke() as the checker, and by bench.py as the timed CPU
 * baseline ("port").
 *
 * Every function states the reference lines it follows (paths relative to the
 * TileQuant repository root).  Numerics (IEEE fp32, round-half-even):
 *
 *   activation scale  sx[c] = a == 0 ? 1 : f32(round_dtype(f32(a) / 127))
 *                     a = max |x[n, 64c:64c+64]| over ALL rows n
 *                     (src/kernels/triton/quantize_activation.py:29-43, 100-106;
 *                      src/kernels/quant_utils.py:68-74)
 *   activation code   q = clamp(rint(f32(x) / sx[c]), -127, 127)
 *                     (quantize_activation.py:69-71, 108-109; quant_utils.py:109-115)
 *   weight scale      sw = a == 0 ? 1 : f32(a) / 127    (not rounded to bf16)
 *   weight code       q = clamp(rint(f32(w) / sw), -127, 127)
 *                     (src/kernels/pack.py:119-130, 163-167)
 *   tile GEMM         per output row tile, INT8 tiles in ascending column order
 *                     acc += f32(int32 dot) * (sx[c] * sw[t]), then BF16 tiles
 *                     acc += fp32 dot; y = round(acc); y = round(f32(y) + bias)
 *                     (src/kernels/triton/gemm_rows_splitk_64x64.py:119-153, 184-190)
 *
 * The code is plain C99 with optional OpenMP over output row tiles.  It needs
 * the default floating-point environment (round-to-nearest-even) and must be
 * built without -ffast-math or FMA contraction surprises: every fused
 * multiply-add below is an explicit fmaf().
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define TQO_TILE 64

/* ---- dtype grids ----------------------------------------------------- */

/* float -> nearest bf16 value (round-half-even on the bit pattern). */
static float round_bf16(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return v; /* inf / nan unchanged */
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* float -> nearest fp16 value, returned as float (RNE, subnormals kept,
 * overflow to inf).  Scaling by a power of two is exact, so the division by
 * the quantum below is exact and nearbyintf does the half-even rounding. */
static float round_fp16(float v) {
  if (!isfinite(v) || v == 0.0f) return v;
  float a = fabsf(v);
  if (a >= 65520.0f) return copysignf(INFINITY, v);
  int e;
  frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) -> unbiased exponent e-1 */
  int exp_unb = e - 1;
  if (exp_unb < -14) exp_unb = -14;
  float quantum = ldexpf(1.0f, exp_unb - 10);
  float r = nearbyintf(a / quantum) * quantum;
  return copysignf(r, v);
}

float tqo_round_to_dtype(float v, int is_bf16) {
  return is_bf16 ? round_bf16(v) : round_fp16(v);
}

/* ---- activation quantization ------------------------------------------ */

/* x: float values of a bf16/fp16 matrix [N, K] with row stride ldx.
 * sx: [n_tc] out.  Follows quantize_activation.py:29-43 / quant_utils.py:68-74. */
void tqo_act_scales(const float* x, long ldx, int N, int K, int is_bf16, float* sx) {
  int n_tc = (K + TQO_TILE - 1) / TQO_TILE;
  for (int c = 0; c < n_tc; ++c) {
    float a = 0.0f;
    int k0 = c * TQO_TILE, k1 = k0 + TQO_TILE < K ? k0 + TQO_TILE : K;
    for (int n = 0; n < N; ++n)
      for (int k = k0; k < k1; ++k) {
        float v = fabsf(x[(long)n * ldx + k]);
        if (v > a) a = v;
      }
    sx[c] = (a > 0.0f) ? tqo_round_to_dtype(a / 127.0f, is_bf16) : 1.0f;
  }
}

/* max(min(q, 127), -127) with NaN-ignoring min/max, in the reference
 * kernel's order (quantize_activation.py:71): 0/0 from a zero scale -> 127. */
static int8_t quant_code(float v, float s) {
  float q = rintf(v / s);
  q = fmaxf(fminf(q, 127.0f), -127.0f);
  return (int8_t)q;
}

/* Codes from given scales.  Follows quantize_activation.py:66-74. */
void tqo_act_quant(const float* x, long ldx, int N, int K, const float* sx,
                   int8_t* q, long ldq) {
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k)
      q[(long)n * ldq + k] = quant_code(x[(long)n * ldx + k], sx[k / TQO_TILE]);
}

/* ---- weight tile quantization (load-time packer numerics) ------------- */

/* src: T tiles of 64x64 float values (row-major within a tile).
 * sw: [T] out, q: [T, 64, 64] out (row-major).  Follows pack.py:119-130,
 * 160-167 (the "gi" branch; the IAA candidate search is not restated). */
void tqo_weight_tiles_quant(const float* src, long T, float* sw, int8_t* q) {
  for (long t = 0; t < T; ++t) {
    const float* w = src + t * 4096;
    float a = 0.0f;
    for (int i = 0; i < 4096; ++i) {
      float v = fabsf(w[i]);
      if (v > a) a = v;
    }
    float s = (a == 0.0f) ? 1.0f : a / 127.0f;
    sw[t] = s;
    for (int i = 0; i < 4096; ++i) q[t * 4096 + i] = quant_code(w[i], s);
  }
}

/* ---- tile GEMM ---------------------------------------------------------- */

static inline int32_t dot_i8_64(const int8_t* a, const int8_t* b, int kmax) {
  int32_t s = 0;
  for (int k = 0; k < kmax; ++k) s += (int32_t)a[k] * (int32_t)b[k];
  return s;
}

/* Exact INT32 products of every INT8 tile with every token row:
 * out[t, n, j] = sum_k xq[n, 64c+k] * wq[t, j, k], c = ids[t] % n_tc,
 * columns >= K read as 0 (gemm_rows_splitk_64x64.py:126-134). */
void tqo_tile_products_i32(const int8_t* xq, long ldq, int N, int K, const int8_t* wq,
                           const int32_t* ids, long T, int n_tc, int32_t* out) {
#pragma omp parallel for schedule(static)
  for (long t = 0; t < T; ++t) {
    int c = ids[t] % n_tc;
    int kmax = K - c * TQO_TILE;
    if (kmax > TQO_TILE) kmax = TQO_TILE;
    for (int n = 0; n < N; ++n)
      for (int j = 0; j < TQO_TILE; ++j)
        out[(t * N + n) * TQO_TILE + j] =
            dot_i8_64(xq + (long)n * ldq + c * TQO_TILE, wq + t * 4096 + j * TQO_TILE, kmax);
  }
}

/* Mixed tile GEMM in the reference's order with SPLIT_K = 1
 * (gemm_rows_splitk_64x64.py:119-153, 184-190).
 *
 * xq [N, ldq] int8 codes; x [N, ldx] float values of the bf16 activation;
 * w8 [T8, 64, 64] row-major int8 tiles, sw8 [T8], ids8 [T8], rp8 [n_tr+1];
 * w16 [T16, 64, 64] row-major float values of the bf16 tiles, ids16, rp16;
 * bias [M] float values already on the output grid, or NULL.
 *
 * y32 [N, M]  out: the fp32 accumulator rounded to the output dtype (then
 *             bias added and rounded again), as float values.
 * acc64 [N, M] out (nullable): the same sum in float64 without any rounding.
 * sumabs [N, M] out (nullable): sum of |term| in float64 (error bound input).
 */
void tqo_gemm_mixed(const int8_t* xq, long ldq, const float* sx, const float* x, long ldx,
                    const int8_t* w8, const float* sw8, const int32_t* ids8, const int32_t* rp8,
                    const float* w16, const int32_t* ids16, const int32_t* rp16,
                    const float* bias, int N, int M, int K, int n_tr, int n_tc, int out_is_bf16,
                    float* y32, double* acc64, double* sumabs) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int r = 0; r < n_tr; ++r) {
    for (int n = 0; n < N; ++n) {
      for (int j = 0; j < TQO_TILE; ++j) {
        int col = r * TQO_TILE + j;
        if (col >= M) continue;
        float acc = 0.0f;
        double a64 = 0.0, s64 = 0.0;
        for (int p = rp8[r]; p < rp8[r + 1]; ++p) {
          int c = ids8[p] % n_tc;
          int kmax = K - c * TQO_TILE;
          if (kmax > TQO_TILE) kmax = TQO_TILE;
          int32_t P = dot_i8_64(xq + (long)n * ldq + c * TQO_TILE,
                                w8 + (long)p * 4096 + j * TQO_TILE, kmax);
          float s = sx[c] * sw8[p];
          acc = fmaf((float)P, s, acc);
          double term = (double)P * (double)sx[c] * (double)sw8[p];
          a64 += term;
          s64 += fabs(term);
        }
        if (w16 != NULL) {
          for (int p = rp16[r]; p < rp16[r + 1]; ++p) {
            int c = ids16[p] % n_tc;
            int kmax = K - c * TQO_TILE;
            if (kmax > TQO_TILE) kmax = TQO_TILE;
            const float* xr = x + (long)n * ldx + c * TQO_TILE;
            const float* wr = w16 + (long)p * 4096 + j * TQO_TILE;
            double d = 0.0, da = 0.0;
            for (int k = 0; k < kmax; ++k) {
              double term = (double)xr[k] * (double)wr[k];
              d += term;
              da += fabs(term);
            }
            /* products of two bf16 values are exact in fp32 and a 64-term
             * sum is within a few ulp; the fp32 image of the exact dot is
             * the tolerance anchor, not a bit-exact claim. */
            acc += (float)d;
            a64 += d;
            s64 += da;
          }
        }
        float y = tqo_round_to_dtype(acc, out_is_bf16);
        if (bias != NULL) y = tqo_round_to_dtype(y + bias[col], out_is_bf16);
        y32[(long)n * M + col] = y;
        if (acc64) acc64[(long)n * M + col] = a64;
        if (sumabs) sumabs[(long)n * M + col] = s64;
      }
    }
  }
}

/* Number of threads OpenMP will use (1 when built without OpenMP). */
int tqo_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
