// tq_fused.hip -- decode-step glue kernels that feed the mixed tile GEMMs
// their INT8 activations directly, for gfx950.
//
// A Llama / Qwen2 decoder layer at decode runs, between its GEMMs, a residual
// add, an RMSNorm, RoPE, a KV-cache write, SiLU * up, and the activation
// quantization of every GEMM input -- each a separate small launch in the
// Hugging Face modules.  These kernels do each producer and the quantization
// of its output in one launch:
//   add_rmsnorm_quant  h = x + delta (rounded to the 16-bit type), y = w * rmsnorm(h),
//                      and y's per-64-column-tile INT8 codes and scales;
//   silu_mul_quant     y = silu(gate) * up of a stacked gate/up output, and its codes;
//   rope_cache         RoPE on the q/k heads of a stacked q/k/v output, k and v
//                      written into the static cache at the device-held position.
// Rounding follows the module code op by op (every intermediate the modules
// materialise in the 16-bit type is rounded to it here too); only the order
// of the fp32 sum of squares differs.  The quantization is the closed form of
// tq_act_quant (scale over ALL rows of the call), bit for bit.
//
// Quantizing kernels run one workgroup per 64-column tile, so the tile's
// absmax over all rows is local to the workgroup.
#include <algorithm>

#include "tq_common.h"

namespace tq {

constexpr int kFuseThreads = 256;

// Max over the workgroup of a non-negative value (all threads receive it).
// The barriers wait for LDS traffic only: the caller's global stores issued
// just before stay in flight (__syncthreads() would wait for them too).
__device__ inline float wg_max_nonneg(float v, float* red) {
  v = wave_max_nonneg(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  lds_barrier();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
  lds_barrier();
  return r;
}

// Sum over a wave (every lane receives it), fixed order: DPP sums within
// rows of 16 lanes, then gfx950's v_permlane16_swap / v_permlane32_swap
// across rows ((r0 + r1) + (r2 + r3) in every lane).
__device__ inline float wave_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  u2 r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

struct NormArgs {
  const uint16_t* x;      // [n, k], row stride ldx
  const uint16_t* delta;  // nullable, row stride ldd
  const uint16_t* w;      // [k]
  uint16_t* h;            // nullable: h = x + delta, row stride ldh
  uint16_t* y;            // [n, k], row stride ldy
  int8_t* q;              // nullable: codes [n, k], row stride ldq
  float* sx;              // [n_tc] when q
  int64_t ldx, ldd, ldh, ldy, ldq;
  int n, k;
  float eps;
};

// Buffer range over rows [0, n) of a [*, k] 16-bit matrix with row stride ld
// (elements): offsets of rows >= n fall past it, so loads there read 0 and
// stores are dropped -- every access in the kernels below is unconditional,
// which keeps all loads of a phase in flight together (per-row branches made
// the compiler wait for each load before the next).  A null pointer gives an
// empty range.
__device__ inline __amdgpu_buffer_rsrc_t rows_rsrc(const void* p, int64_t ld, int n, int k, int esize) {
  return row_rsrc(p, p ? (int)(((int64_t)(n - 1) * ld + k) * esize) : 0);
}

// workgroup c: every row's sum of squares over all k columns (each wave takes
// rows wave, wave + 4, ...), then the 64 columns of tile c for every row.
// acc + lo^2 + hi^2 of a packed pair of 16-bit values (v_dot2_f32_bf16 /
// v_dot2_f32_f16: exact products, fp32 sums)
template <class XT>
__device__ inline float dot2sq(uint32_t w, float acc) {
  if constexpr (std::is_same<XT, Bf16>::value) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 v = __builtin_bit_cast(bf2, w);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = __builtin_bit_cast(h2, w);
    return __builtin_amdgcn_fdot2(v, v, acc, false);
  }
}

// Byte offset of element (row, col) of a [*, k] matrix with row stride ld
// (elements), or an offset past any buffer range for rows >= n: the load
// reads 0 and the store is dropped, with no branch.  Rows < n fit 31 bits
// (the host checks ((n - 1) * ld + k) * esize < 2^31).
__device__ inline int row_off(int row, int n, int64_t ld, int col, int esize) {
  return row < n ? (int)(((int64_t)row * ld + col) * esize) : 0x7fffffff;
}

// workgroup c: every row's sum of squares over all k columns (each wave takes
// rows wave, wave + 4, ...), then the 64 columns of tile c for every row:
// thread t takes rows wave + 4 i, i < TR (TR >= n / 4, a template constant so
// that no slot costs a branch), column c * 64 + t % 64.
template <class XT, bool HAS_DELTA, int TR>
__global__ void __launch_bounds__(kFuseThreads)
add_rmsnorm_quant_kernel(NormArgs a, L2Warm warm) {
  __shared__ float rinv[64];          // 1 / sqrt(mean(h^2) + eps) per row (n <= 64)
  __shared__ float red[kFuseThreads / kWave];
  TQ_ARGS_IN_SGPRS("s"(a.x), "s"(a.delta), "s"(a.w), "s"(a.h), "s"(a.y), "s"(a.q), "s"(a.sx), "s"(a.ldx),
                   "s"(a.ldd), "s"(a.ldh), "s"(a.ldy), "s"(a.ldq), "s"(a.n), "s"(a.k), "s"(a.eps), "s"(warm.first));
  if ((int)blockIdx.x >= warm.first) {   // the warm-up workgroups (none without a warm-up)
    __shared__ uint32_t warm_sink[64];
    l2_warm_rows<kFuseThreads>(warm, warm_sink);
    return;
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int c = blockIdx.x;
  const int cpr = a.k >> 3;           // 8-element chunks per row
  const __amdgpu_buffer_rsrc_t xr = rows_rsrc(a.x, a.ldx, a.n, a.k, 2);
  const __amdgpu_buffer_rsrc_t dr = rows_rsrc(a.delta, a.ldd, a.n, a.k, 2);
  // This workgroup's tile, loaded first: it does not depend on the row norms,
  // so its round trip overlaps the row loads below.  Without a delta h = x
  // (not x + 0: -0 stays -0).
  const int col = c * 64 + lane;
  uint32_t xt[TR], dt[TR];   // one register per value: no packing right after each load
#pragma unroll
  for (int i = 0; i < TR; ++i) {
    const int row = wave + 4 * i;
    xt[i] = __builtin_amdgcn_raw_buffer_load_b16(xr, row_off(row, a.n, a.ldx, col, 2), 0, 0);
    dt[i] = HAS_DELTA ? __builtin_amdgcn_raw_buffer_load_b16(dr, row_off(row, a.n, a.ldd, col, 2), 0, 0) : 0u;
  }
  const uint16_t wraw = a.w[col];
  // Passes of kNormBatch chunks per lane: all loads of a pass are issued
  // before the first use (one memory round trip per pass, not per chunk).
  // Chunks past the row end read 0 (an offset past the range) and add 0.
  constexpr int kNormBatch = 8;
  for (int row = wave; row < a.n; row += kFuseThreads / kWave) {
    // one partial sum per load slot j (eight independent fma chains instead
    // of one 64 long), combined pairwise in a fixed order
    float ssj[kNormBatch];
#pragma unroll
    for (int j = 0; j < kNormBatch; ++j) ssj[j] = 0.0f;
    for (int c0 = 0; c0 < cpr; c0 += kNormBatch * kWave) {
      u32x4 xv[kNormBatch], dv[kNormBatch];
#pragma unroll
      for (int j = 0; j < kNormBatch; ++j) {
        const int ch = c0 + j * kWave + lane;
        const int ox = ch < cpr ? (int)(((int64_t)row * a.ldx + ch * 8) * 2) : 0x7fffffff;
        xv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, ox, 0, 0));
        if constexpr (HAS_DELTA) {
          const int od = ch < cpr ? (int)(((int64_t)row * a.ldd + ch * 8) * 2) : 0x7fffffff;
          dv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(dr, od, 0, 0));
        }
      }
#pragma unroll
      for (int j = 0; j < kNormBatch; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // h of two elements, rounded as a pair (one v_cvt_pk_*), then both
          // squares in one v_dot2 (exact products, fp32 sums)
          const uint32_t xw = xv[j][i];
          uint32_t hp = xw;
          if constexpr (HAS_DELTA) {
            const uint32_t dw = dv[j][i];
            hp = XT::pack2(XT::to_f32((uint16_t)xw) + XT::to_f32((uint16_t)dw),
                           XT::to_f32((uint16_t)(xw >> 16)) + XT::to_f32((uint16_t)(dw >> 16)));
          }
          ssj[j] = dot2sq<XT>(hp, ssj[j]);
        }
      }
    }
    float ss = ((ssj[0] + ssj[1]) + (ssj[2] + ssj[3])) + ((ssj[4] + ssj[5]) + (ssj[6] + ssj[7]));
    ss = wave_sum(ss);
    if (lane == 0) rinv[row] = rsqrtf(ss / (float)a.k + a.eps);
  }
  lds_barrier();
  // tile c (rows >= n: zero values, stores dropped by the ranges)
  const __amdgpu_buffer_rsrc_t hr = rows_rsrc(HAS_DELTA ? a.h : nullptr, a.ldh, a.n, a.k, 2);
  const __amdgpu_buffer_rsrc_t yr = rows_rsrc(a.y, a.ldy, a.n, a.k, 2);
  float am = 0.0f;
  float yv[TR];
  const float wv = XT::to_f32(wraw);
#pragma unroll
  for (int i = 0; i < TR; ++i) {
    const int row = wave + 4 * i;
    const bool live = row < a.n;
    const float xf = XT::to_f32((uint16_t)xt[i]);
    const float hv = HAS_DELTA ? XT::round(xf + XT::to_f32((uint16_t)dt[i])) : xf;
    __builtin_amdgcn_raw_buffer_store_b16(XT::from_f32(hv), hr, row_off(row, a.n, a.ldh, col, 2), 0, 0);
    const float nrm = XT::round(hv * (live ? rinv[row] : 0.0f));   // hidden_states.to(input_dtype)
    const float y = XT::round(wv * nrm);                          // weight * hidden_states
    __builtin_amdgcn_raw_buffer_store_b16(XT::from_f32(y), yr, row_off(row, a.n, a.ldy, col, 2), 0, 0);
    yv[i] = live ? y : 0.0f;
    am = fmaxf(am, fabsf(yv[i]));
  }
  if (a.q == nullptr) return;
  const float s = act_scale_from_absmax<XT>(wg_max_nonneg(am, red));
  const CodeScale cs(s);
  const __amdgpu_buffer_rsrc_t qr = rows_rsrc(a.q, a.ldq, a.n, a.k, 1);
#pragma unroll
  for (int i = 0; i < TR; ++i)
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)cs.code(yv[i]), qr, row_off(wave + 4 * i, a.n, a.ldq, col, 1), 0, 0);
  if (t == 0) a.sx[c] = s;
}

struct SiluArgs {
  const uint16_t* gu;   // [n, 2 * inter]: gate columns [0, inter), up [inter, 2 inter)
  uint16_t* y;          // [n, inter]
  int8_t* q;            // nullable codes [n, inter]
  float* sx;
  int64_t ldg, ldy, ldq;
  int n, inter;
};

// y = silu(gate) * up with the module's roundings: silu in fp32 rounded to the
// 16-bit type, the product rounded again.  Workgroup c = 64-column tile c;
// thread t takes rows wave + 4 i, i < TR (TR >= n / 4).
template <class XT, int TR>
__global__ void __launch_bounds__(kFuseThreads)
silu_mul_quant_kernel(SiluArgs a, L2Warm warm) {
  __shared__ float red[kFuseThreads / kWave];
  TQ_ARGS_IN_SGPRS("s"(a.gu), "s"(a.y), "s"(a.q), "s"(a.sx), "s"(a.ldg), "s"(a.ldy), "s"(a.ldq), "s"(a.n),
                   "s"(a.inter), "s"(warm.first));
  if ((int)blockIdx.x >= warm.first) {   // the warm-up workgroups (none without a warm-up)
    __shared__ uint32_t warm_sink[64];
    l2_warm_rows<kFuseThreads>(warm, warm_sink);
    return;
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int col = blockIdx.x * 64 + lane;
  // rows >= n read 0 and their stores are dropped (buffer ranges); every
  // load is issued before the first use
  const __amdgpu_buffer_rsrc_t gr = rows_rsrc(a.gu, a.ldg, a.n, 2 * a.inter, 2);
  const __amdgpu_buffer_rsrc_t yr = rows_rsrc(a.y, a.ldy, a.n, a.inter, 2);
  uint32_t gw[TR], uw[TR];
#pragma unroll
  for (int i = 0; i < TR; ++i) {
    const int row = wave + 4 * i;
    gw[i] = __builtin_amdgcn_raw_buffer_load_b16(gr, row_off(row, a.n, a.ldg, col, 2), 0, 0);
    uw[i] = __builtin_amdgcn_raw_buffer_load_b16(gr, row_off(row, a.n, a.ldg, col + a.inter, 2), 0, 0);
  }
  float am = 0.0f;
  float yv[TR];
#pragma unroll
  for (int i = 0; i < TR; ++i) {
    const int row = wave + 4 * i;
    const float g = XT::to_f32((uint16_t)gw[i]);
    const float u = XT::to_f32((uint16_t)uw[i]);
    const float sg = XT::round(g / (1.0f + expf(-g)));
    const float y = XT::round(sg * u);
    __builtin_amdgcn_raw_buffer_store_b16(XT::from_f32(y), yr, row_off(row, a.n, a.ldy, col, 2), 0, 0);
    yv[i] = row < a.n ? y : 0.0f;
    am = fmaxf(am, fabsf(yv[i]));
  }
  if (a.q == nullptr) return;
  const float s = act_scale_from_absmax<XT>(wg_max_nonneg(am, red));
  const CodeScale cs(s);
  const __amdgpu_buffer_rsrc_t qr = rows_rsrc(a.q, a.ldq, a.n, a.inter, 1);
#pragma unroll
  for (int i = 0; i < TR; ++i)
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)cs.code(yv[i]), qr, row_off(wave + 4 * i, a.n, a.ldq, col, 1), 0, 0);
  if (t == 0) a.sx[blockIdx.x] = s;
}

struct RopeArgs {
  const uint16_t* qkv;   // [n, (hq + 2 hkv) * 128], row stride ldqkv
  const uint16_t* cos;   // [128] at the decode position
  const uint16_t* sin;
  const int64_t* pos;    // device position (cache index)
  uint16_t* q_out;       // [n, hq, 128] rotated queries, strides q_sb, q_sh
  uint16_t* k_cache;     // [n, hkv, L, 128] with strides c_sb, c_sh, c_sl (shared by v)
  uint16_t* v_cache;
  int64_t ldqkv, q_sb, q_sh, c_sb, c_sh, c_sl;
  int n, hq, hkv, max_len;
};

// Workgroup (row b, head slot j < hq + 2 hkv), 64 threads, lane d rotates the
// pair (d, d + 64): out[d] = q[d] cos[d] - q[d+64] sin[d],
// out[d+64] = q[d+64] cos[d+64] + q[d] sin[d+64], each product and the sum
// rounded to the 16-bit type as the modules do (q * cos + rotate_half(q) * sin).
template <class XT>
__global__ void __launch_bounds__(64)
rope_cache_kernel(RopeArgs a) {
  const int b = blockIdx.x, j = blockIdx.y, d = threadIdx.x;
  // every load first (none depends on the position), then the position check
  const uint16_t* src = a.qkv + (int64_t)b * a.ldqkv + (int64_t)j * 128;
  const uint16_t rlo = src[d], rhi = src[d + 64];
  const uint16_t rc0 = a.cos[d], rc1 = a.cos[d + 64], rs0 = a.sin[d], rs1 = a.sin[d + 64];
  const int64_t p = a.pos[0];
  if (p < 0 || p >= a.max_len) return;   // never indexes outside the cache
  const float lo = XT::to_f32(rlo), hi = XT::to_f32(rhi);
  if (j >= a.hq + a.hkv) {   // v head: copy into the cache
    uint16_t* dst = a.v_cache + (int64_t)b * a.c_sb + (int64_t)(j - a.hq - a.hkv) * a.c_sh + p * a.c_sl;
    dst[d] = rlo;
    dst[d + 64] = rhi;
    return;
  }
  const float c0 = XT::to_f32(rc0), c1 = XT::to_f32(rc1);
  const float s0 = XT::to_f32(rs0), s1 = XT::to_f32(rs1);
  const float o0 = XT::round(XT::round(lo * c0) + XT::round(-hi * s0));
  const float o1 = XT::round(XT::round(hi * c1) + XT::round(lo * s1));
  uint16_t* dst = (j < a.hq) ? a.q_out + (int64_t)b * a.q_sb + (int64_t)j * a.q_sh
                             : a.k_cache + (int64_t)b * a.c_sb + (int64_t)(j - a.hq) * a.c_sh + p * a.c_sl;
  dst[d] = XT::from_f32(o0);
  dst[d + 64] = XT::from_f32(o1);
}

// ---- greedy decode step: argmax over the vocabulary + token bookkeeping ----
//
// torch.argmax semantics (ATen's GreaterOrNan): a NaN beats every number,
// equal values (or two NaNs) go to the lower index.
struct ArgBest {
  float v;
  int i;
};
__device__ inline bool arg_better(float a, int ia, float b, int ib) {
  if (a != a) return b != b ? ia < ib : true;
  if (b != b) return false;
  return a == b ? ia < ib : a > b;
}
__device__ inline ArgBest arg_pick(ArgBest x, float v, int i) { return arg_better(v, i, x.v, x.i) ? ArgBest{v, i} : x; }
// wave-wide best (every lane receives it); the pairing order does not matter:
// the rule is a total order with a unique winner
__device__ inline ArgBest wave_arg_best(ArgBest x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float v = __shfl_xor(x.v, off);
    const int i = __shfl_xor(x.i, off);
    x = arg_pick(x, v, i);
  }
  return x;
}

constexpr int kArgSplits = 32;      // partial results per row
constexpr int kArgThreads = 256;

// workgroup (split s, row b): best of logits[b, s * per .. (s + 1) * per)
template <class XT>
__global__ void __launch_bounds__(kArgThreads)
argmax_partial_kernel(const uint16_t* __restrict__ x, int64_t ldx, int m, int per, float* __restrict__ pv,
                      int* __restrict__ pi) {
  __shared__ ArgBest red[kArgThreads / kWave];
  const int s = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const uint16_t* row = x + (int64_t)b * ldx;
  const int lo = s * per, hi = min(lo + per, m);
  ArgBest best{-INFINITY, 0x7fffffff};
  constexpr int kBatch = 8;   // independent loads in flight per thread
  for (int j0 = lo + t; j0 < hi; j0 += kArgThreads * kBatch) {
    uint16_t r[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + u * kArgThreads;
      r[u] = row[min(j, hi - 1)];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + u * kArgThreads;
      if (j < hi) best = arg_pick(best, XT::to_f32(r[u]), j);
    }
  }
  best = wave_arg_best(best);
  if ((t & 63) == 0) red[t >> 6] = best;
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kArgThreads / kWave; ++w) best = arg_pick(best, red[w].v, red[w].i);
    pv[b * kArgSplits + s] = best.v;
    pi[b * kArgSplits + s] = best.i;
  }
}

// One workgroup: wave w finishes rows w, w + 4, ...; then the bookkeeping of
// the reference's greedy loop (src/runtime/graph_decode.py:347-385): the
// token is fed back, recorded at column position - prompt_len + 1 of
// `generated`, the position advances and seq_used becomes new position + 1.
__global__ void __launch_bounds__(kArgThreads)
greedy_finish_kernel(const float* __restrict__ pv, const int* __restrict__ pi, int n, int64_t* __restrict__ next,
                     int64_t* __restrict__ token, int64_t* __restrict__ gen, int64_t ldg, int gen_len,
                     int64_t* __restrict__ position, int prompt_len, int32_t* __restrict__ seq_used) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t pos = position[0];
  for (int b = wave; b < n; b += kArgThreads / kWave) {
    ArgBest best{-INFINITY, 0x7fffffff};
    if (lane < kArgSplits) best = ArgBest{pv[b * kArgSplits + lane], pi[b * kArgSplits + lane]};
    best = wave_arg_best(best);
    if (lane == 0) {
      next[b] = best.i;
      token[b] = best.i;
      const int64_t col = pos - prompt_len + 1;
      if (gen != nullptr && col >= 0 && col < gen_len) gen[(int64_t)b * ldg + col] = best.i;
    }
  }
  __syncthreads();   // every wave has read the position
  if (t < n && seq_used != nullptr) seq_used[t] = (int32_t)(pos + 2);
  if (t == 0) position[0] = pos + 1;
}

// ---- prefill glue: the same arithmetic on thousands of rows ---------------
//
// At prefill (B x P rows) these are bandwidth-bound: one wave per row for the
// norm (the row's sum of squares stays in the wave), elementwise grids for
// SiLU * up and RoPE.

// One wave per row: h = x + delta (rounded; h = x without delta), y = w *
// round(h * rsqrt(mean(h^2) + eps)) -- add_rmsnorm_quant's element arithmetic
// (only the fp32 order of the sum of squares differs).  CPL 16-byte chunks per
// lane hold the row between the two passes (k <= 512 * CPL).
template <class XT, int CPL>
__global__ void __launch_bounds__(256)
add_rmsnorm_rows_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6), nw = gridDim.x * 4;
  const int cpr = a.k >> 3;   // 8-element chunks per row
  const bool has_delta = a.delta != nullptr;
  u32x4 wv[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = min(lane + 64 * i, cpr - 1);
    wv[i] = *reinterpret_cast<const u32x4*>(a.w + ch * 8);
  }
  for (int row = gw; row < a.n; row += nw) {
    const uint16_t* xr = a.x + (int64_t)row * a.ldx;
    const uint16_t* dr = has_delta ? a.delta + (int64_t)row * a.ldd : xr;
    u32x4 hv[CPL], dv[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = min(lane + 64 * i, cpr - 1);
      hv[i] = *reinterpret_cast<const u32x4*>(xr + ch * 8);
      dv[i] = *reinterpret_cast<const u32x4*>(dr + ch * 8);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const bool live = lane + 64 * i < cpr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t xw = hv[i][e], dw = dv[i][e];
        if (has_delta)
          hv[i][e] = XT::pack2(XT::to_f32((uint16_t)xw) + XT::to_f32((uint16_t)dw),
                               XT::to_f32((uint16_t)(xw >> 16)) + XT::to_f32((uint16_t)(dw >> 16)));
        if (live) ss = dot2sq<XT>(hv[i][e], ss);
      }
    }
    ss = wave_sum(ss);
    const float rinv = rsqrtf(ss / (float)a.k + a.eps);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = lane + 64 * i;
      if (ch >= cpr) continue;
      u32x4 yv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t h2 = hv[i][e], w2 = wv[i][e];
        const float n0 = XT::round(XT::to_f32((uint16_t)h2) * rinv);           // hidden_states.to(input_dtype)
        const float n1 = XT::round(XT::to_f32((uint16_t)(h2 >> 16)) * rinv);
        yv[e] = XT::pack2(XT::to_f32((uint16_t)w2) * n0, XT::to_f32((uint16_t)(w2 >> 16)) * n1);   // weight * hidden
      }
      *reinterpret_cast<u32x4*>(a.y + (int64_t)row * a.ldy + ch * 8) = yv;
      if (has_delta) *reinterpret_cast<u32x4*>(a.h + (int64_t)row * a.ldh + ch * 8) = hv[i];
    }
  }
}

// y = round(round(silu(gate)) * up) over [n, inter] from [n, 2 inter]: one
// thread per 8 columns of one row.
template <class XT>
__global__ void __launch_bounds__(256)
silu_mul_rows_kernel(SiluArgs a) {
  const int cpr = a.inter >> 3;
  const int64_t total = (int64_t)a.n * cpr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int row = (int)(i / cpr), ch = (int)(i - (int64_t)row * cpr);
    const uint16_t* g = a.gu + (int64_t)row * a.ldg + ch * 8;
    const u32x4 gv = *reinterpret_cast<const u32x4*>(g);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(g + a.inter);
    u32x4 yv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float y2[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float gf = XT::to_f32((uint16_t)(gv[e] >> (16 * hh)));
        const float uf = XT::to_f32((uint16_t)(uv[e] >> (16 * hh)));
        const float sg = XT::round(gf / (1.0f + expf(-gf)));
        y2[hh] = sg * uf;
      }
      yv[e] = XT::pack2(y2[0], y2[1]);
    }
    *reinterpret_cast<u32x4*>(a.y + (int64_t)row * a.ldy + ch * 8) = yv;
  }
}

// RoPE of a prompt: rows n = b * P + p of the stacked q/k/v output, position
// p; rotated q to q_out[b, j, p, :] (strides q_sb, q_sh, q_sp), rotated k and
// v into the caches at index p.  cos / sin: [>= P, 128] tables.  One thread
// per (row, head, 8-element chunk t of the low half): it rotates elements
// 8t .. 8t + 7 with their partners 64 + 8t .. (16-byte loads and stores) with
// rope_cache_kernel's roundings.
struct RopePrefillArgs {
  const uint16_t* qkv;
  const uint16_t* cos;
  const uint16_t* sin;
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t ldqkv, ldcs, q_sb, q_sh, q_sp, c_sb, c_sh, c_sl;
  int P, hq, hkv, n;
};

template <class XT>
__global__ void __launch_bounds__(256)
rope_prefill_kernel(RopePrefillArgs a) {
  const int nh = a.hq + 2 * a.hkv;
  const int64_t total = (int64_t)a.n * nh * 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int t = (int)(i & 7);
    const int64_t rh = i >> 3;
    const int row = (int)(rh / nh), j = (int)(rh - (int64_t)row * nh);
    const int b = row / a.P, p = row - b * a.P;
    const uint16_t* src = a.qkv + (int64_t)row * a.ldqkv + (int64_t)j * 128 + 8 * t;
    const u32x4 lo = *reinterpret_cast<const u32x4*>(src);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(src + 64);
    uint16_t* dst;
    if (j >= a.hq + a.hkv) {   // v head: copy into the cache
      dst = a.v_cache + (int64_t)b * a.c_sb + (int64_t)(j - a.hq - a.hkv) * a.c_sh + (int64_t)p * a.c_sl + 8 * t;
      *reinterpret_cast<u32x4*>(dst) = lo;
      *reinterpret_cast<u32x4*>(dst + 64) = hi;
      continue;
    }
    const uint16_t* cr = a.cos + (int64_t)p * a.ldcs + 8 * t;
    const uint16_t* sr = a.sin + (int64_t)p * a.ldcs + 8 * t;
    const u32x4 c0 = *reinterpret_cast<const u32x4*>(cr), c1 = *reinterpret_cast<const u32x4*>(cr + 64);
    const u32x4 s0 = *reinterpret_cast<const u32x4*>(sr), s1 = *reinterpret_cast<const u32x4*>(sr + 64);
    u32x4 o0, o1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r0[2], r1[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int sh = 16 * hh;
        const float l = XT::to_f32((uint16_t)(lo[e] >> sh)), h = XT::to_f32((uint16_t)(hi[e] >> sh));
        const float cl = XT::to_f32((uint16_t)(c0[e] >> sh)), ch = XT::to_f32((uint16_t)(c1[e] >> sh));
        const float sl = XT::to_f32((uint16_t)(s0[e] >> sh)), shi = XT::to_f32((uint16_t)(s1[e] >> sh));
        r0[hh] = XT::round(l * cl) - XT::round(h * sl);   // round(-x) == -round(x) (half-even)
        r1[hh] = XT::round(h * ch) + XT::round(l * shi);
      }
      o0[e] = (uint32_t)XT::from_f32(r0[0]) | ((uint32_t)XT::from_f32(r0[1]) << 16);
      o1[e] = (uint32_t)XT::from_f32(r1[0]) | ((uint32_t)XT::from_f32(r1[1]) << 16);
    }
    dst = (j < a.hq) ? a.q_out + (int64_t)b * a.q_sb + (int64_t)j * a.q_sh + (int64_t)p * a.q_sp + 8 * t
                     : a.k_cache + (int64_t)b * a.c_sb + (int64_t)(j - a.hq) * a.c_sh + (int64_t)p * a.c_sl + 8 * t;
    *reinterpret_cast<u32x4*>(dst) = o0;
    *reinterpret_cast<u32x4*>(dst + 64) = o1;
  }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Launches a glue kernel instantiated for TR = tile rows per wave, the
// smallest of 1, 2, 4, 16 with 4 * TR >= n (n <= 64).
template <class XT, bool HAS_DELTA>
struct NormLaunch {
  template <int TR>
  static void go(dim3 grid, hipStream_t s, const NormArgs& a, const L2Warm& w) {
    hipLaunchKernelGGL((add_rmsnorm_quant_kernel<XT, HAS_DELTA, TR>), grid, dim3(kFuseThreads), 0, s, a, w);
  }
};
template <class XT>
struct SiluLaunch {
  template <int TR>
  static void go(dim3 grid, hipStream_t s, const SiluArgs& a, const L2Warm& w) {
    hipLaunchKernelGGL((silu_mul_quant_kernel<XT, TR>), grid, dim3(kFuseThreads), 0, s, a, w);
  }
};
template <class L, class Args>
static void launch_by_rows(int n, dim3 grid, hipStream_t s, const Args& a, const L2Warm& w) {
  if (n <= 4) L::template go<1>(grid, s, a, w);
  else if (n <= 8) L::template go<2>(grid, s, a, w);
  else if (n <= 16) L::template go<4>(grid, s, a, w);
  else L::template go<16>(grid, s, a, w);
}

}  // namespace tq

using namespace tq;

extern "C" int tq_add_rmsnorm_quant(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                                    const void* weight, float eps, void* h_out, int64_t h_stride, void* y_out,
                                    int64_t y_stride, int8_t* q_out, int64_t q_stride, float* sx_out, int dtype,
                                    int n, int k, const tq_l2_warm* warm_in, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (n < 0 || k < 0 || n > 64 || (k % 64) != 0) return TQ_ERR_ARG;
  if (n == 0 || k == 0) return TQ_OK;
  if (!x || !weight || !y_out || (q_out && !sx_out) || (delta && !h_out)) return TQ_ERR_ARG;
  if (!al16(x) || (x_stride % 8) || (delta && (!al16(delta) || (delta_stride % 8)))) return TQ_ERR_ALIGN;
  // every row range is addressed through a 32-bit buffer offset
  const int64_t ld_max = std::max({x_stride, delta ? delta_stride : 0, h_out ? h_stride : 0, y_stride,
                                   q_out ? q_stride : 0});
  if (ld_max < k || ((int64_t)(n - 1) * ld_max + k) * 2 >= (1LL << 31)) return TQ_ERR_ARG;
  NormArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.delta = static_cast<const uint16_t*>(delta);
  a.w = static_cast<const uint16_t*>(weight);
  a.h = static_cast<uint16_t*>(h_out); a.y = static_cast<uint16_t*>(y_out); a.q = q_out; a.sx = sx_out;
  a.ldx = x_stride; a.ldd = delta_stride; a.ldh = h_stride; a.ldy = y_stride; a.ldq = q_stride;
  a.n = n; a.k = k; a.eps = eps;
  L2Warm warm;
  const int rc = l2_warm_args(warm_in, k / 64, warm);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(k / 64 + warm.blocks);
  if (dtype == TQ_DTYPE_BF16) {
    if (delta) launch_by_rows<NormLaunch<Bf16, true>>(n, grid, s, a, warm);
    else launch_by_rows<NormLaunch<Bf16, false>>(n, grid, s, a, warm);
  } else {
    if (delta) launch_by_rows<NormLaunch<Fp16, true>>(n, grid, s, a, warm);
    else launch_by_rows<NormLaunch<Fp16, false>>(n, grid, s, a, warm);
  }
  return (int)hipGetLastError();
}

extern "C" int tq_silu_mul_quant(const void* gate_up, int64_t gu_stride, void* y_out, int64_t y_stride,
                                 int8_t* q_out, int64_t q_stride, float* sx_out, int dtype, int n, int inter,
                                 const tq_l2_warm* warm_in, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (n < 0 || inter < 0 || n > 64 || (inter % 64) != 0) return TQ_ERR_ARG;
  if (n == 0 || inter == 0) return TQ_OK;
  if (!gate_up || !y_out || (q_out && !sx_out)) return TQ_ERR_ARG;
  const int64_t ld_max = std::max({gu_stride, y_stride, q_out ? q_stride : 0});
  if (gu_stride < 2 * (int64_t)inter || y_stride < inter || (q_out && q_stride < inter) ||
      ((int64_t)(n - 1) * ld_max + 2 * (int64_t)inter) * 2 >= (1LL << 31))
    return TQ_ERR_ARG;
  SiluArgs a{};
  a.gu = static_cast<const uint16_t*>(gate_up); a.y = static_cast<uint16_t*>(y_out); a.q = q_out; a.sx = sx_out;
  a.ldg = gu_stride; a.ldy = y_stride; a.ldq = q_stride; a.n = n; a.inter = inter;
  L2Warm warm;
  const int rc = l2_warm_args(warm_in, inter / 64, warm);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(inter / 64 + warm.blocks);
  if (dtype == TQ_DTYPE_BF16) launch_by_rows<SiluLaunch<Bf16>>(n, grid, s, a, warm);
  else launch_by_rows<SiluLaunch<Fp16>>(n, grid, s, a, warm);
  return (int)hipGetLastError();
}

extern "C" int tq_rope_cache(const void* qkv, int64_t qkv_stride, const void* cos, const void* sin,
                             const int64_t* position, void* q_out, int64_t q_stride_b, int64_t q_stride_h,
                             void* k_cache, void* v_cache, int64_t cache_stride_b, int64_t cache_stride_h,
                             int64_t cache_stride_l, int dtype, int n, int q_heads, int kv_heads, int head_dim,
                             int max_len, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (head_dim != 128 || n < 0 || q_heads <= 0 || kv_heads <= 0 || max_len <= 0) return TQ_ERR_ARG;
  if (n == 0) return TQ_OK;
  if (!qkv || !cos || !sin || !position || !q_out || !k_cache || !v_cache) return TQ_ERR_ARG;
  RopeArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv); a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin); a.pos = position;
  a.q_out = static_cast<uint16_t*>(q_out); a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.ldqkv = qkv_stride; a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.c_sb = cache_stride_b; a.c_sh = cache_stride_h; a.c_sl = cache_stride_l;
  a.n = n; a.hq = q_heads; a.hkv = kv_heads; a.max_len = max_len;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(n, q_heads + 2 * kv_heads);
  if (dtype == TQ_DTYPE_BF16) hipLaunchKernelGGL(rope_cache_kernel<Bf16>, grid, dim3(64), 0, s, a);
  else hipLaunchKernelGGL(rope_cache_kernel<Fp16>, grid, dim3(64), 0, s, a);
  return (int)hipGetLastError();
}

extern "C" int tq_add_rmsnorm_rows(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                                   const void* weight, float eps, void* h_out, int64_t h_stride, void* y_out,
                                   int64_t y_stride, int dtype, int n, int k, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (n < 0 || k < 0 || (k % 8) != 0 || k > 8192) return TQ_ERR_ARG;
  if (n == 0 || k == 0) return TQ_OK;
  if (!x || !weight || !y_out || (delta && !h_out)) return TQ_ERR_ARG;
  if (x_stride < k || y_stride < k || (delta && (delta_stride < k || h_stride < k))) return TQ_ERR_ARG;
  if (!al16(x) || !al16(weight) || !al16(y_out) || (x_stride % 8) || (y_stride % 8) ||
      (delta && (!al16(delta) || !al16(h_out) || (delta_stride % 8) || (h_stride % 8))))
    return TQ_ERR_ALIGN;
  NormArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.delta = static_cast<const uint16_t*>(delta);
  a.w = static_cast<const uint16_t*>(weight);
  a.h = static_cast<uint16_t*>(h_out); a.y = static_cast<uint16_t*>(y_out);
  a.ldx = x_stride; a.ldd = delta_stride; a.ldh = h_stride; a.ldy = y_stride;
  a.n = n; a.k = k; a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(std::min((n + 3) / 4, 2048)), block(256);
  const bool wide = k > 4096;
  if (dtype == TQ_DTYPE_BF16) {
    if (wide) hipLaunchKernelGGL((add_rmsnorm_rows_kernel<Bf16, 16>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((add_rmsnorm_rows_kernel<Bf16, 8>), grid, block, 0, s, a);
  } else {
    if (wide) hipLaunchKernelGGL((add_rmsnorm_rows_kernel<Fp16, 16>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((add_rmsnorm_rows_kernel<Fp16, 8>), grid, block, 0, s, a);
  }
  return (int)hipGetLastError();
}

extern "C" int tq_silu_mul_rows(const void* gate_up, int64_t gu_stride, void* y_out, int64_t y_stride, int dtype,
                                int n, int inter, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (n < 0 || inter < 0 || (inter % 8) != 0) return TQ_ERR_ARG;
  if (n == 0 || inter == 0) return TQ_OK;
  if (!gate_up || !y_out || gu_stride < 2 * (int64_t)inter || y_stride < inter) return TQ_ERR_ARG;
  if (!al16(gate_up) || !al16(y_out) || (gu_stride % 8) || (y_stride % 8)) return TQ_ERR_ALIGN;
  SiluArgs a{};
  a.gu = static_cast<const uint16_t*>(gate_up); a.y = static_cast<uint16_t*>(y_out);
  a.ldg = gu_stride; a.ldy = y_stride; a.n = n; a.inter = inter;
  const int64_t total = (int64_t)n * (inter / 8);
  const dim3 grid((unsigned)std::min<int64_t>((total + 255) / 256, 8192)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TQ_DTYPE_BF16) hipLaunchKernelGGL(silu_mul_rows_kernel<Bf16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(silu_mul_rows_kernel<Fp16>, grid, block, 0, s, a);
  return (int)hipGetLastError();
}

extern "C" int tq_rope_prefill(const void* qkv, int64_t qkv_stride, const void* cos, const void* sin,
                               int64_t table_stride, void* q_out, int64_t q_stride_b, int64_t q_stride_h,
                               int64_t q_stride_p, void* k_cache, void* v_cache, int64_t cache_stride_b,
                               int64_t cache_stride_h, int64_t cache_stride_l, int dtype, int batch, int prompt_len,
                               int q_heads, int kv_heads, int head_dim, int max_len, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (head_dim != 128 || batch < 0 || prompt_len < 0 || q_heads <= 0 || kv_heads <= 0 || prompt_len > max_len ||
      table_stride < 128)
    return TQ_ERR_ARG;
  if (batch == 0 || prompt_len == 0) return TQ_OK;
  if ((int64_t)batch * prompt_len >= (1LL << 31) || qkv_stride < (int64_t)(q_heads + 2 * kv_heads) * 128) return TQ_ERR_ARG;
  if (!qkv || !cos || !sin || !q_out || !k_cache || !v_cache) return TQ_ERR_ARG;
  // 16-byte accesses: every row, head, table row and cache slot starts 16-byte aligned
  if (!al16(qkv) || !al16(cos) || !al16(sin) || !al16(q_out) || !al16(k_cache) || !al16(v_cache) || (qkv_stride % 8) ||
      (table_stride % 8) || (q_stride_b % 8) || (q_stride_h % 8) || (q_stride_p % 8) || (cache_stride_b % 8) ||
      (cache_stride_h % 8) || (cache_stride_l % 8))
    return TQ_ERR_ALIGN;
  RopePrefillArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv); a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin); a.q_out = static_cast<uint16_t*>(q_out);
  a.k_cache = static_cast<uint16_t*>(k_cache); a.v_cache = static_cast<uint16_t*>(v_cache);
  a.ldqkv = qkv_stride; a.ldcs = table_stride; a.q_sb = q_stride_b; a.q_sh = q_stride_h; a.q_sp = q_stride_p;
  a.c_sb = cache_stride_b; a.c_sh = cache_stride_h; a.c_sl = cache_stride_l;
  a.P = prompt_len; a.hq = q_heads; a.hkv = kv_heads; a.n = batch * prompt_len;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t total = (int64_t)a.n * (q_heads + 2 * kv_heads) * 8;
  const dim3 grid((unsigned)std::min<int64_t>((total + 255) / 256, 16384));
  if (dtype == TQ_DTYPE_BF16) hipLaunchKernelGGL(rope_prefill_kernel<Bf16>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(rope_prefill_kernel<Fp16>, grid, dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

extern "C" int64_t tq_greedy_step_workspace_elems(int batch) {
  return batch > 0 ? (int64_t)batch * kArgSplits * 2 : 0;
}

extern "C" int tq_greedy_step(const void* logits, int64_t logits_stride, int dtype, int batch, int vocab,
                              int32_t* workspace, int64_t workspace_elems, int64_t* next_token, int64_t* token,
                              int64_t* generated, int64_t generated_stride, int generated_len, int64_t* position,
                              int prompt_len, int32_t* seq_used, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (batch < 0 || vocab <= 0 || batch > kArgThreads || logits_stride < vocab) return TQ_ERR_ARG;
  if (batch == 0) return TQ_OK;
  if (!logits || !next_token || !token || !position) return TQ_ERR_ARG;
  if (!workspace || workspace_elems < tq_greedy_step_workspace_elems(batch)) return TQ_ERR_WORKSPACE;
  float* pv = reinterpret_cast<float*>(workspace);
  int* pi = workspace + (int64_t)batch * kArgSplits;
  const int per = (vocab + kArgSplits - 1) / kArgSplits;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* x = static_cast<const uint16_t*>(logits);
  if (dtype == TQ_DTYPE_BF16)
    hipLaunchKernelGGL(argmax_partial_kernel<Bf16>, dim3(kArgSplits, batch), dim3(kArgThreads), 0, s, x,
                       logits_stride, vocab, per, pv, pi);
  else
    hipLaunchKernelGGL(argmax_partial_kernel<Fp16>, dim3(kArgSplits, batch), dim3(kArgThreads), 0, s, x,
                       logits_stride, vocab, per, pv, pi);
  hipLaunchKernelGGL(greedy_finish_kernel, dim3(1), dim3(kArgThreads), 0, s, pv, pi, batch, next_token, token,
                     generated, generated_stride, generated_len, position, prompt_len, seq_used);
  return (int)hipGetLastError();
}
