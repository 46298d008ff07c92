// tq_act_quant.hip -- per-64-column-tile INT8 activation quantization (gfx950).
//
// Numerics (one scale per 64-column tile, shared by ALL rows of the call):
//   a     = max |x[:, 64c:64c+64]|                       (exact in the 16-bit type)
//   sx[c] = a == 0 ? 1 : f32(round_to_x_dtype(f32(a) / 127))     IEEE divide
//   q     = max(min(rint(f32(x) / sx[c]), 127), -127)            IEEE divide, half-even
// following src/kernels/triton/quantize_activation.py:29-43, 66-71, 96-112.
// The clamp is min-then-max with NaN-ignoring min/max, as the reference
// kernel's tl.minimum / tl.maximum, so a zero-scale tile (a < 127 * 2^-134)
// maps x == 0 to 127; the codes of such a tile never reach the output
// because every product with it is scaled by sx == 0.
//
// Kernels
//   act_quant_fused      grid n_tc, 256 threads: absmax -> scale -> codes in one
//                        launch (reference :77-112 for n <= 128; any n works).
//   act_quant_small      the same for n <= 8 rows: one wave per tile, values
//                        loaded once, wave-level absmax.
//   act_absmax_partial   grid (n_tc, n_rb): max over a 256-row block; writes the
//                        scale directly when n_rb == 1, else a partial.
//   act_scales_finalize  max over the n_rb partials (fixed order; max is exact
//                        so the result is order-free) -> scale.
//   act_quant_scaled     codes from given scales, 8 elements (16 B in, 8 B out)
//                        per thread on the aligned path.
// Every kernel has a vector path (unit column stride, 16-byte aligned rows,
// full tiles) and a scalar path for everything else.
#include <algorithm>

#include "tq_common.h"

namespace tq {

constexpr int kQuantThreads = 256;
constexpr int kRowsPerPass = kQuantThreads / 8;  // 8 threads x 8 elements per 64-col row
constexpr int kPartialRows = 256;                 // rows per absmax partial block
constexpr int kSinglePassMaxRows = 512;           // above this the scales are two-level

struct XView {
  const uint16_t* x;
  int64_t sn, sk;
  int n, k;
};

// Loads 8 consecutive elements of row `row`, columns col..col+7 (vector path).
__device__ inline u32x4 load8(const XView& v, int row, int col) {
  return *reinterpret_cast<const u32x4*>(v.x + (int64_t)row * v.sn + col);
}

// Vector path is legal for tile c when rows are 16-byte aligned, the column
// stride is 1 and the tile lies fully inside k.
__device__ inline bool tile_vec_ok(const XView& v, int c) {
  return v.sk == 1 && (v.sn % 8) == 0 && aligned16(v.x) && (c + 1) * kTile <= v.k;
}

template <class T>
__device__ float tile_absmax(const XView& v, int c, int row0, int row1) {
  const int t = threadIdx.x;
  float m = 0.0f;
  if (tile_vec_ok(v, c)) {
    const int col = c * kTile + (t % 8) * 8;
    for (int row = row0 + t / 8; row < row1; row += kRowsPerPass) m = max8<T>(load8(v, row, col), m);
  } else {
    const int cols = min(kTile, v.k - c * kTile);
    for (int64_t e = t; e < (int64_t)(row1 - row0) * kTile; e += kQuantThreads) {
      int row = row0 + (int)(e / kTile), kk = (int)(e % kTile);
      if (kk < cols) m = fmaxf(m, fabsf(T::to_f32(v.x[(int64_t)row * v.sn + (int64_t)(c * kTile + kk) * v.sk])));
    }
  }
  return m;
}

// Byte offset of the 8 codes of row `row`, columns col .. col + 7 (col % 8 == 0)
// in token-blocked codes with nb 16-row blocks per column tile (TQ_XQ_TOKEN_BLOCKED):
// block (c, row / 16) is the MFMA A operand of that 16 x 64 slice, 16-byte run
// l = 16 kq + row % 16 holding columns 64 c + 16 kq .. + 15.
__device__ inline int64_t blocked_offset(int row, int col, int nb) {
  const int c = col >> 6, kq = (col & 63) >> 4;
  return ((int64_t)(c * nb + (row >> 4)) * 64 + kq * 16 + (row & 15)) * 16 + (col & 15);
}

// nb > 0: codes token-blocked with nb 16-row blocks per column tile (vector
// path only; rows n .. 16 nb - 1 are written as zeros), else row-major with
// row stride ldq.
template <class T>
__global__ void __launch_bounds__(kQuantThreads)
act_quant_fused_kernel(XView v, int8_t* __restrict__ q, int64_t ldq, float* __restrict__ sx, int nb) {
  __shared__ float red[kQuantThreads / kWave];
  TQ_ARGS_IN_SGPRS("s"(v.x), "s"(v.sn), "s"(v.sk), "s"(v.n), "s"(v.k), "s"(q), "s"(ldq), "s"(sx), "s"(nb));
  const int c = blockIdx.x, t = threadIdx.x;
  const bool qvec = ((ldq % 8) == 0) && (((uintptr_t)q & 7u) == 0);
  if (v.n <= 2 * kRowsPerPass && tile_vec_ok(v, c) && (nb > 0 || qvec)) {
    // Up to 64 rows a thread's share is two 8-element groups: loaded once and
    // kept in registers from the absmax to the codes (one global round trip
    // instead of two; same closed form, same codes).
    const int col = c * kTile + (t % 8) * 8;
    u32x4 w[2];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = t / 8 + i * kRowsPerPass;
      w[i] = row < v.n ? load8(v, row, col) : u32x4{0u, 0u, 0u, 0u};
      m = max8<T>(w[i], m);
    }
    const float s = act_scale_from_absmax<T>(block_max(m, red, kQuantThreads / kWave));
    const CodeScale cs(s);
    if (t == 0) sx[c] = s;
    const int rows = nb > 0 ? 16 * nb : v.n;   // token-blocked: padding rows are written as zeros
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = t / 8 + i * kRowsPerPass;
      if (row >= rows) continue;
      const u32x2 code = row < v.n ? codes8<T>(w[i], cs) : u32x2{0u, 0u};
      if (nb > 0) *reinterpret_cast<u32x2*>(q + blocked_offset(row, col, nb)) = code;
      else *reinterpret_cast<u32x2*>(q + (int64_t)row * ldq + col) = code;
    }
    return;
  }
  const float a = block_max(tile_absmax<T>(v, c, 0, v.n), red, kQuantThreads / kWave);
  const float s = act_scale_from_absmax<T>(a);
  const CodeScale cs(s);
  if (t == 0) sx[c] = s;
  if (tile_vec_ok(v, c) && qvec) {
    const int col = c * kTile + (t % 8) * 8;
    for (int row = t / 8; row < v.n; row += kRowsPerPass)
      *reinterpret_cast<u32x2*>(q + (int64_t)row * ldq + col) = codes8<T>(load8(v, row, col), cs);
  } else {
    const int cols = min(kTile, v.k - c * kTile);
    for (int64_t e = t; e < (int64_t)v.n * kTile; e += kQuantThreads) {
      int row = (int)(e / kTile), kk = (int)(e % kTile);
      if (kk < cols) {
        float xv = T::to_f32(v.x[(int64_t)row * v.sn + (int64_t)(c * kTile + kk) * v.sk]);
        q[(int64_t)row * ldq + c * kTile + kk] = (int8_t)cs.code(xv);
      }
    }
  }
}

// Few rows (n <= 8, the decode case): one wave per column tile, lane l holds
// row l / 8, columns 8 (l % 8) .. +7, loaded once; the tile's absmax is a
// wave reduction (no LDS, no barrier) and the codes come from the same
// registers.  Same closed form as act_quant_fused_kernel, bit for bit (the
// absmax is exact and order-free).  Vector layout only: unit column stride,
// 16-byte aligned rows, k a multiple of 64, 8-byte aligned code rows.
constexpr int kSmallMaxRows = 8;

template <class T>
__global__ void __launch_bounds__(kQuantThreads)
act_quant_small_kernel(XView v, int8_t* __restrict__ q, int64_t ldq, float* __restrict__ sx, int n_tc) {
  TQ_ARGS_IN_SGPRS("s"(v.x), "s"(v.sn), "s"(v.n), "s"(q), "s"(ldq), "s"(sx), "s"(n_tc));
  const int lane = threadIdx.x & (kWave - 1);
  const int c = blockIdx.x * (kQuantThreads / kWave) + (threadIdx.x >> 6);
  if (c >= n_tc) return;   // whole waves
  const int row = lane >> 3, col = c * kTile + (lane & 7) * 8;
  u32x4 w = u32x4{0, 0, 0, 0};
  if (row < v.n) w = load8(v, row, col);
  const float a = wave_max_nonneg(max8<T>(w, 0.0f));
  const float s = act_scale_from_absmax<T>(a);
  const CodeScale cs(s);
  if (lane == 0) sx[c] = s;
  if (row < v.n) *reinterpret_cast<u32x2*>(q + (int64_t)row * ldq + col) = codes8<T>(w, cs);
}

template <class T>
__global__ void __launch_bounds__(kQuantThreads)
act_absmax_partial_kernel(XView v, float* __restrict__ out, int rows_per_block, int write_scale) {
  __shared__ float red[kQuantThreads / kWave];
  const int c = blockIdx.x, rb = blockIdx.y;
  const int row0 = rb * rows_per_block, row1 = min(v.n, row0 + rows_per_block);
  const float a = block_max(tile_absmax<T>(v, c, row0, row1), red, kQuantThreads / kWave);
  if (threadIdx.x == 0) {
    const int n_tc = gridDim.x;
    if (write_scale) out[c] = act_scale_from_absmax<T>(a);
    else out[(int64_t)rb * n_tc + c] = a;
  }
}

template <class T>
__global__ void act_scales_finalize_kernel(const float* __restrict__ partial, int n_rb, int n_tc,
                                           float* __restrict__ sx) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n_tc) return;
  float a = 0.0f;
  for (int rb = 0; rb < n_rb; ++rb) a = fmaxf(a, partial[(int64_t)rb * n_tc + c]);
  sx[c] = act_scale_from_absmax<T>(a);
}

// Codes of rows [rb * kPartialRows, ...) of column tile c, the tile's scale
// taken from the absmax partials of every row block (the finalize step folded
// in: every workgroup reduces its column's partials; block 0 stores sx[c]).
// The row loads go out before the partials are read, so both arrive in one
// round trip.  Vector layout only (unit column stride, 16-byte aligned rows,
// k a multiple of 64, 8-byte aligned code rows).  Same closed forms as
// act_scales_finalize_kernel + act_quant_scaled_kernel, bit for bit.
template <class T>
__global__ void __launch_bounds__(kQuantThreads)
act_quant_block_kernel(XView v, const float* __restrict__ partial, int n_rb, int8_t* __restrict__ q, int64_t ldq,
                       float* __restrict__ sx) {
  __shared__ float scale;
  const int c = blockIdx.x, rb = blockIdx.y, t = threadIdx.x, n_tc = gridDim.x;
  const int row0 = rb * kPartialRows, row1 = min(v.n, row0 + kPartialRows);
  const int col = c * kTile + (t % 8) * 8;
  constexpr int kPer = kPartialRows / kRowsPerPass;
  u32x4 w[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) w[i] = load8(v, min(row0 + t / 8 + i * kRowsPerPass, row1 - 1), col);
  if (t < kWave) {
    float a = 0.0f;
    for (int i = t; i < n_rb; i += kWave) a = fmaxf(a, partial[(int64_t)i * n_tc + c]);
    a = wave_max_nonneg(a);
    if (t == 0) {
      const float s = act_scale_from_absmax<T>(a);
      scale = s;
      if (rb == 0) sx[c] = s;
    }
  }
  __syncthreads();
  const CodeScale cs(scale);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int row = row0 + t / 8 + i * kRowsPerPass;
    if (row < row1) *reinterpret_cast<u32x2*>(q + (int64_t)row * ldq + col) = codes8<T>(w[i], cs);
  }
}

template <class T>
__global__ void __launch_bounds__(kQuantThreads)
act_quant_scaled_kernel(XView v, const float* __restrict__ sx, int8_t* __restrict__ q, int64_t ldq,
                        int vec) {
  const int64_t stride = (int64_t)gridDim.x * kQuantThreads;
  const int64_t first = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x;
  if (vec) {
    const int kv = v.k / 8;
    const int64_t items = (int64_t)v.n * kv;
    for (int64_t it = first; it < items; it += stride) {
      const int row = (int)(it / kv), col = (int)(it % kv) * 8;
      const CodeScale cs(sx[col / kTile]);
      *reinterpret_cast<u32x2*>(q + (int64_t)row * ldq + col) = codes8<T>(load8(v, row, col), cs);
    }
  } else {
    const int64_t items = (int64_t)v.n * v.k;
    for (int64_t it = first; it < items; it += stride) {
      const int row = (int)(it / v.k), col = (int)(it % v.k);
      const float xv = T::to_f32(v.x[(int64_t)row * v.sn + (int64_t)col * v.sk]);
      q[(int64_t)row * ldq + col] = (int8_t)quant_code(xv, sx[col / kTile]);
    }
  }
}

// ---- one scale for a whole tensor ------------------------------------------
//
// quantize_activation_absmax / quantize_weight_tile_absmax
// (src/kernels/quant_utils.py:17-37, 138-148), which are torch expressions:
//   a = max |x|                      (exact in x's dtype)
//   s = a == 0 ? 1 : f32(x_dtype(f32(a) / 127))      (max_abs / 127.0 stays in x's dtype)
//   q = clamp(rint(x_dtype(f32(x) / s)), -127, 127)  (a 16-bit tensor divided by a 0-dim
//       fp32 tensor stays 16-bit in torch, so the quotient is rounded to x's dtype
//       before torch.round -- unlike the tile kernels above, which round fl32(x / s))
// IEEE divides, half-even rint.  fp32 inputs skip both dtype roundings.
// Small tensors take one workgroup (absmax then codes); larger ones a
// partial-max pass and a codes pass that reduces the partials itself.
struct F32 {
  __device__ static inline float to_f32(uint32_t b) { return __uint_as_float(b); }
  __device__ static inline float round(float f) { return f; }
};

template <class T>
__device__ inline int8_t tensor_code(float v, float s) {
  const float t = __builtin_rintf(T::round(v / s));
  return (int8_t)(int)fmaxf(fminf(t, 127.0f), -127.0f);
}

constexpr int64_t kTensorOneGroupMax = 1 << 16;   // elements quantized by a single workgroup
constexpr int kTensorPartials = 1024;              // partial maxima of the two-pass form

template <class T, class S>
__global__ void __launch_bounds__(kQuantThreads)
tensor_absmax_partial_kernel(const S* __restrict__ x, int64_t n, float* __restrict__ partial) {
  __shared__ float red[kQuantThreads / kWave];
  float m = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kQuantThreads)
    m = fmaxf(m, fabsf(T::to_f32(x[i])));
  m = block_max(m, red, kQuantThreads / kWave);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// partial == nullptr: this (single) workgroup takes the absmax itself.
template <class T, class S>
__global__ void __launch_bounds__(kQuantThreads)
tensor_quant_kernel(const S* __restrict__ x, int64_t n, const float* __restrict__ partial, int n_partial,
                    int8_t* __restrict__ q, float* __restrict__ s_out) {
  __shared__ float red[kQuantThreads / kWave];
  float m = 0.0f;
  if (partial == nullptr) {
    for (int64_t i = threadIdx.x; i < n; i += kQuantThreads) m = fmaxf(m, fabsf(T::to_f32(x[i])));
  } else {
    for (int i = threadIdx.x; i < n_partial; i += kQuantThreads) m = fmaxf(m, partial[i]);
  }
  const float s = act_scale_from_absmax<T>(block_max(m, red, kQuantThreads / kWave));
  if (blockIdx.x == 0 && threadIdx.x == 0) *s_out = s;
  for (int64_t i = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kQuantThreads)
    q[i] = tensor_code<T>(T::to_f32(x[i]), s);
}

static int n_tiles_of(int k) { return (k + kTile - 1) / kTile; }

static int check_x(const void* x, int64_t sn, int64_t sk, int dtype, int n, int k) {
  if (n < 0 || k < 0 || sn < 0 || sk < 0) return TQ_ERR_ARG;
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (n > 0 && k > 0 && x == nullptr) return TQ_ERR_ARG;
  return TQ_OK;
}

}  // namespace tq

using namespace tq;

extern "C" int tq_act_quant_fused(const void* x, int64_t x_stride_n, int64_t x_stride_k, int x_dtype,
                                  int n, int k, int8_t* q, int64_t q_stride_n, float* sx,
                                  void* stream) {
  int rc = check_x(x, x_stride_n, x_stride_k, x_dtype, n, k);
  if (rc) return rc;
  if (k == 0) return TQ_OK;
  if (sx == nullptr || (n > 0 && (q == nullptr || q_stride_n < k))) return TQ_ERR_ARG;
  XView v{static_cast<const uint16_t*>(x), x_stride_n, x_stride_k, n, k};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int n_tc = n_tiles_of(k);
  if (n > 0 && n <= kSmallMaxRows && x_stride_k == 1 && (x_stride_n % 8) == 0 && aligned16(x) && (k % kTile) == 0 &&
      (q_stride_n % 8) == 0 && ((uintptr_t)q & 7u) == 0) {
    const dim3 g((n_tc + kQuantThreads / kWave - 1) / (kQuantThreads / kWave));
    if (x_dtype == TQ_DTYPE_BF16)
      hipLaunchKernelGGL(act_quant_small_kernel<Bf16>, g, dim3(kQuantThreads), 0, s, v, q, q_stride_n, sx, n_tc);
    else
      hipLaunchKernelGGL(act_quant_small_kernel<Fp16>, g, dim3(kQuantThreads), 0, s, v, q, q_stride_n, sx, n_tc);
    return (int)hipGetLastError();
  }
  dim3 grid(n_tc);
  if (x_dtype == TQ_DTYPE_BF16)
    hipLaunchKernelGGL(act_quant_fused_kernel<Bf16>, grid, dim3(kQuantThreads), 0, s, v, q, q_stride_n, sx, 0);
  else
    hipLaunchKernelGGL(act_quant_fused_kernel<Fp16>, grid, dim3(kQuantThreads), 0, s, v, q, q_stride_n, sx, 0);
  return (int)hipGetLastError();
}

extern "C" int tq_act_quant_token_blocked(const void* x, int64_t x_stride_n, int x_dtype, int n, int k, int8_t* q,
                                          float* sx, void* stream) {
  int rc = check_x(x, x_stride_n, 1, x_dtype, n, k);
  if (rc) return rc;
  if (n < 1 || n > 64 || k < kTile || (k % kTile) != 0 || q == nullptr || sx == nullptr) return TQ_ERR_ARG;
  if ((x_stride_n % 8) != 0 || !aligned16(x) || ((uintptr_t)q & 7u) != 0) return TQ_ERR_ALIGN;
  XView v{static_cast<const uint16_t*>(x), x_stride_n, 1, n, k};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nb = (n + 15) / 16;
  dim3 grid(n_tiles_of(k));
  if (x_dtype == TQ_DTYPE_BF16)
    hipLaunchKernelGGL(act_quant_fused_kernel<Bf16>, grid, dim3(kQuantThreads), 0, s, v, q, (int64_t)0, sx, nb);
  else
    hipLaunchKernelGGL(act_quant_fused_kernel<Fp16>, grid, dim3(kQuantThreads), 0, s, v, q, (int64_t)0, sx, nb);
  return (int)hipGetLastError();
}

extern "C" int64_t tq_act_absmax_workspace_elems(int n, int k) {
  if (n <= kSinglePassMaxRows || k <= 0) return 0;
  const int64_t n_rb = (n + kPartialRows - 1) / kPartialRows;
  return n_rb * n_tiles_of(k);
}

extern "C" int tq_act_absmax_scales(const void* x, int64_t x_stride_n, int64_t x_stride_k, int x_dtype,
                                    int n, int k, float* sx, float* workspace, int64_t workspace_elems,
                                    void* stream) {
  int rc = check_x(x, x_stride_n, x_stride_k, x_dtype, n, k);
  if (rc) return rc;
  if (k == 0) return TQ_OK;
  if (sx == nullptr) return TQ_ERR_ARG;
  const int n_tc = n_tiles_of(k);
  XView v{static_cast<const uint16_t*>(x), x_stride_n, x_stride_k, n, k};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t need = tq_act_absmax_workspace_elems(n, k);
  const bool bf = x_dtype == TQ_DTYPE_BF16;
  if (need == 0) {
    // one block per tile covers every row; n == 0 gives a == 0 -> scale 1
    dim3 grid(n_tc, 1);
    if (bf) hipLaunchKernelGGL(act_absmax_partial_kernel<Bf16>, grid, dim3(kQuantThreads), 0, s, v, sx, n, 1);
    else hipLaunchKernelGGL(act_absmax_partial_kernel<Fp16>, grid, dim3(kQuantThreads), 0, s, v, sx, n, 1);
    return (int)hipGetLastError();
  }
  if (workspace == nullptr || workspace_elems < need) return TQ_ERR_WORKSPACE;
  const int n_rb = (n + kPartialRows - 1) / kPartialRows;
  dim3 grid(n_tc, n_rb);
  dim3 fgrid((n_tc + 255) / 256);
  if (bf) {
    hipLaunchKernelGGL(act_absmax_partial_kernel<Bf16>, grid, dim3(kQuantThreads), 0, s, v, workspace, kPartialRows, 0);
    hipLaunchKernelGGL(act_scales_finalize_kernel<Bf16>, fgrid, dim3(256), 0, s, workspace, n_rb, n_tc, sx);
  } else {
    hipLaunchKernelGGL(act_absmax_partial_kernel<Fp16>, grid, dim3(kQuantThreads), 0, s, v, workspace, kPartialRows, 0);
    hipLaunchKernelGGL(act_scales_finalize_kernel<Fp16>, fgrid, dim3(256), 0, s, workspace, n_rb, n_tc, sx);
  }
  return (int)hipGetLastError();
}

extern "C" int tq_act_quant_with_scales(const void* x, int64_t x_stride_n, int64_t x_stride_k,
                                        int x_dtype, int n, int k, const float* sx, int8_t* q,
                                        int64_t q_stride_n, void* stream) {
  int rc = check_x(x, x_stride_n, x_stride_k, x_dtype, n, k);
  if (rc) return rc;
  if (k == 0 || n == 0) return TQ_OK;
  if (sx == nullptr || q == nullptr || q_stride_n < k) return TQ_ERR_ARG;
  XView v{static_cast<const uint16_t*>(x), x_stride_n, x_stride_k, n, k};
  const int vec = (x_stride_k == 1 && (x_stride_n % 8) == 0 && (k % 8) == 0 && aligned16(x) &&
                   (q_stride_n % 8) == 0 && (((uintptr_t)q & 7u) == 0)) ? 1 : 0;
  const int64_t items = vec ? (int64_t)n * (k / 8) : (int64_t)n * k;
  int64_t blocks = (items + kQuantThreads - 1) / kQuantThreads;
  if (blocks > 8192) blocks = 8192;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == TQ_DTYPE_BF16)
    hipLaunchKernelGGL(act_quant_scaled_kernel<Bf16>, dim3((unsigned)blocks), dim3(kQuantThreads), 0, s, v, sx, q, q_stride_n, vec);
  else
    hipLaunchKernelGGL(act_quant_scaled_kernel<Fp16>, dim3((unsigned)blocks), dim3(kQuantThreads), 0, s, v, sx, q, q_stride_n, vec);
  return (int)hipGetLastError();
}

extern "C" int tq_act_quant_two_level(const void* x, int64_t x_stride_n, int x_dtype, int n, int k, int8_t* q,
                                      int64_t q_stride_n, float* sx, float* workspace, int64_t workspace_elems,
                                      void* stream) {
  int rc = check_x(x, x_stride_n, 1, x_dtype, n, k);
  if (rc) return rc;
  if (k == 0 || n == 0) return TQ_OK;
  if (sx == nullptr || q == nullptr || q_stride_n < k) return TQ_ERR_ARG;
  if ((k % kTile) != 0 || (x_stride_n % 8) != 0 || !aligned16(x) || (q_stride_n % 8) != 0 ||
      ((uintptr_t)q & 7u) != 0)
    return TQ_ERR_ALIGN;
  const int64_t need = tq_act_absmax_workspace_elems(n, k);
  if (need == 0) return TQ_ERR_ARG;   // few rows: tq_act_quant_fused / single-pass scales
  if (workspace == nullptr || workspace_elems < need) return TQ_ERR_WORKSPACE;
  const int n_tc = n_tiles_of(k), n_rb = (n + kPartialRows - 1) / kPartialRows;
  XView v{static_cast<const uint16_t*>(x), x_stride_n, 1, n, k};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(n_tc, n_rb);
  if (x_dtype == TQ_DTYPE_BF16) {
    hipLaunchKernelGGL(act_absmax_partial_kernel<Bf16>, grid, dim3(kQuantThreads), 0, s, v, workspace, kPartialRows, 0);
    hipLaunchKernelGGL(act_quant_block_kernel<Bf16>, grid, dim3(kQuantThreads), 0, s, v, workspace, n_rb, q, q_stride_n, sx);
  } else {
    hipLaunchKernelGGL(act_absmax_partial_kernel<Fp16>, grid, dim3(kQuantThreads), 0, s, v, workspace, kPartialRows, 0);
    hipLaunchKernelGGL(act_quant_block_kernel<Fp16>, grid, dim3(kQuantThreads), 0, s, v, workspace, n_rb, q, q_stride_n, sx);
  }
  return (int)hipGetLastError();
}

extern "C" int64_t tq_quant_tensor_workspace_elems(int64_t numel) {
  return numel > kTensorOneGroupMax ? kTensorPartials : 0;
}

template <class T, class S>
static void launch_tensor_quant(const void* x, int64_t numel, int8_t* q, float* s_out, float* ws, hipStream_t s) {
  const S* xs = static_cast<const S*>(x);
  if (numel <= kTensorOneGroupMax) {
    hipLaunchKernelGGL((tensor_quant_kernel<T, S>), dim3(1), dim3(kQuantThreads), 0, s, xs, numel, nullptr, 0, q, s_out);
    return;
  }
  hipLaunchKernelGGL((tensor_absmax_partial_kernel<T, S>), dim3(kTensorPartials), dim3(kQuantThreads), 0, s, xs, numel,
                     ws);
  const int64_t blocks = std::min<int64_t>((numel + 8 * kQuantThreads - 1) / (8 * kQuantThreads), 4096);
  hipLaunchKernelGGL((tensor_quant_kernel<T, S>), dim3((unsigned)blocks), dim3(kQuantThreads), 0, s, xs, numel, ws,
                     kTensorPartials, q, s_out);
}

extern "C" int tq_quant_tensor_absmax(const void* x, int64_t numel, int x_dtype, int8_t* q, float* scale,
                                      float* workspace, int64_t workspace_elems, void* stream) {
  if (numel < 0 || scale == nullptr || (numel > 0 && (x == nullptr || q == nullptr))) return TQ_ERR_ARG;
  if (x_dtype != TQ_DTYPE_BF16 && x_dtype != TQ_DTYPE_FP16 && x_dtype != TQ_DTYPE_FP32) return TQ_ERR_DTYPE;
  if (numel == 0) return TQ_OK;   // the caller's scale is 1 (no launch)
  const int64_t need = tq_quant_tensor_workspace_elems(numel);
  if (need > 0 && (workspace == nullptr || workspace_elems < need)) return TQ_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == TQ_DTYPE_BF16) launch_tensor_quant<Bf16, uint16_t>(x, numel, q, scale, workspace, s);
  else if (x_dtype == TQ_DTYPE_FP16) launch_tensor_quant<Fp16, uint16_t>(x, numel, q, scale, workspace, s);
  else launch_tensor_quant<F32, uint32_t>(x, numel, q, scale, workspace, s);
  return (int)hipGetLastError();
}
