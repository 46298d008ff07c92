// tq_gemm.hip -- mixed INT8/BF16 64x64-tile GEMM for gfx950 (row-owned schedule).
//
// out[n, m] = sum_{INT8 tiles t of row tile r}  f32(P_t[n, m%64]) * (sx[c_t] * sw[t])
//           + sum_{16-bit tiles t of row tile r} fp32 dot(x[n, tile c_t], W_t[m%64, :])
// with P_t the exact INT32 product over the tile's 64 input columns
// (src/kernels/triton/gemm_rows_splitk_64x64.py:119-153), rounded to the
// output dtype, then bias added and rounded again (:178-190).
//
// Schedule ("row-owned", the reference's decomposition re-cut for CDNA4):
//   workgroup (blockIdx.x = 4 * r + jb, blockIdx.y = token block) owns the 16
//   output features jb*16 .. jb*16+15 of row tile r for 16*TB tokens.  Its W
//   waves take the tile list of row r round-robin (INT8 positions first, the
//   16-bit positions continue the rotation), so each wave streams every W-th
//   tile's 1 KiB j-block.  Per INT8 tile a wave issues one
//   v_mfma_i32_16x16x64_i8 per 16-token block (the whole 64-deep tile in one
//   instruction, INT32 accumulate from zero), converts to fp32 and FMAs by
//   sx[c] * sw[t].  Per 16-bit tile it issues two v_mfma_f32_16x16x32_{bf16,f16}
//   per token block accumulating straight into the fp32 accumulator.
//   The W partial accumulators are then summed through LDS in wave order
//   0..W-1 -- a fixed order, so results are bitwise reproducible -- and the
//   epilogue rounds, adds bias and stores.  No atomics, no global workspace.
//
// MFMA operand layouts (gfx950, checked on hardware):
//   A (16 x 64 int8):  lane l holds row l%16, k = 16*(l/16) .. +16
//   B (64 x 16 int8):  lane l holds col l%16, k = 16*(l/16) .. +16
//   A/B 16-bit x32:    lane l holds row/col l%16, k = 8*(l/16) .. +8
//   D (16 x 16):       lane l holds col l%16, rows 4*(l/16) + v, v = 0..3
// With A = activations (rows = tokens) and B = a weight tile's j-block
// (B[k][j] = W[j][k]), D[token][j] lands in lane j%16.  The packer's MFMA
// tile layout stores each j-block's B operand as one contiguous 1 KiB run
// (lane l's 16 bytes at l*16), so the weight load is a single coalesced
// global_load_dwordx4 per tile; the reference's row-major tile order is also
// accepted (same 1 KiB run, permuted 16-byte chunks).
#include "tq_common.h"

namespace tq {

struct GemmArgs {
  const int8_t* xq;
  int64_t ldq;
  const float* sx;
  const int8_t* w8;
  const float* sw8;
  const int32_t* ids8;
  const int32_t* rp8;
  const uint16_t* xf;
  int64_t ldx;
  const uint16_t* w16;
  const int32_t* ids16;
  const int32_t* rp16;
  uint16_t* out;
  int64_t ldo;
  const uint16_t* bias;
  int32_t* dump;
  int n, m, k, n_tr, n_tc;
  int out_bf16;   // output dtype: 1 bf16, 0 fp16
  int layout;     // TQ_LAYOUT_*
  int xvec;       // activations allow 16-byte loads (aligned rows, k == 64 * n_tc)
};

constexpr int kMaxWaves = 16;
constexpr int kUnroll8 = 4;   // INT8 tiles in flight per wave
constexpr int kUnroll16 = 2;  // 16-bit tiles in flight per wave

// ---- operand loads --------------------------------------------------------

// B operand of INT8 tile p, j-block jb, for this lane.
__device__ inline v4i load_w8(const GemmArgs& a, int p, int jb, int lane) {
  const int8_t* base = a.w8 + (int64_t)p * 4096;
  int off = (a.layout == TQ_LAYOUT_MFMA) ? jb * 1024 + lane * 16
                                          : (jb * 16 + (lane & 15)) * 64 + (lane >> 4) * 16;
  return *reinterpret_cast<const v4i*>(base + off);
}

// B operand of 16-bit tile p, j-block jb, k-half h.
__device__ inline v4i load_w16(const GemmArgs& a, int p, int jb, int h, int lane) {
  const uint16_t* base = a.w16 + (int64_t)p * 4096;
  int off = (a.layout == TQ_LAYOUT_MFMA) ? (jb * 2 + h) * 512 + lane * 8
                                          : (jb * 16 + (lane & 15)) * 64 + h * 32 + (lane >> 4) * 8;
  return *reinterpret_cast<const v4i*>(base + off);
}

// A operand: 16 int8 codes of token row `row`, columns col .. col+15.
__device__ inline v4i load_xq(const GemmArgs& a, int row, int col) {
  if (row >= a.n) return v4i{0, 0, 0, 0};
  const int8_t* p = a.xq + (int64_t)row * a.ldq + col;
  if (a.xvec) return *reinterpret_cast<const v4i*>(p);
  uint32_t w[4] = {0, 0, 0, 0};
  for (int e = 0; e < 16; ++e)
    if (col + e < a.k) w[e >> 2] |= (uint32_t)(uint8_t)p[e] << (8 * (e & 3));
  return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// A operand: 8 16-bit activations of row `row`, columns col .. col+7.
__device__ inline v4i load_xf(const GemmArgs& a, int row, int col) {
  if (row >= a.n) return v4i{0, 0, 0, 0};
  const uint16_t* p = a.xf + (int64_t)row * a.ldx + col;
  if (a.xvec) return *reinterpret_cast<const v4i*>(p);
  uint32_t w[4] = {0, 0, 0, 0};
  for (int e = 0; e < 8; ++e)
    if (col + e < a.k) w[e >> 1] |= (uint32_t)p[e] << (16 * (e & 1));
  return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

template <class XT>
__device__ inline v4f mfma16(v4i av, v4i bv, v4f c);

template <>
__device__ inline v4f mfma16<Bf16>(v4i av, v4i bv, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, av),
                                                 __builtin_bit_cast(v8bf, bv), c, 0, 0, 0);
}
template <>
__device__ inline v4f mfma16<Fp16>(v4i av, v4i bv, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, av),
                                                __builtin_bit_cast(v8h, bv), c, 0, 0, 0);
}

// Column tile of a tile id owned by row tile r (id = r * n_tc + c).  Clamped so
// that a malformed pack can never index sx / x out of range.
__device__ inline int col_of(int id, int rbase, int n_tc) {
  return (int)min((unsigned)(id - rbase), (unsigned)(n_tc - 1));
}

// ---- the kernel -----------------------------------------------------------

// 64-token blocks hold 4x the accumulators: cap them at 8 waves (256 VGPRs).
constexpr int max_waves_for(int tb) { return tb == 4 ? 8 : kMaxWaves; }

template <class XT, int TB, bool DUMP>
__global__ void __launch_bounds__(max_waves_for(TB) * kWave)
gemm_rows_kernel(GemmArgs a) {
  extern __shared__ float red[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int r = blockIdx.x >> 2, jb = blockIdx.x & 3;
  const int n0 = blockIdx.y * 16 * TB;
  const int arow = lane & 15;       // A operand token row within a 16-block
  const int akq = lane >> 4;        // A operand k chunk
  const int rbase = r * a.n_tc;     // tile id = r * n_tc + c for tiles of row r

  v4f acc[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) acc[tb] = v4f{0.f, 0.f, 0.f, 0.f};

  // ---------------- INT8 tiles ----------------
  const int lo8 = a.rp8[r], hi8 = a.rp8[r + 1];
  int p = lo8 + wave;
  for (; p + (kUnroll8 - 1) * W < hi8; p += kUnroll8 * W) {
    int c[kUnroll8];
    float s[kUnroll8];
    v4i bw[kUnroll8];
    v4i ax[kUnroll8][TB];
#pragma unroll
    for (int u = 0; u < kUnroll8; ++u) {
      const int pu = p + u * W;
      c[u] = col_of(a.ids8[pu], rbase, a.n_tc);
      bw[u] = load_w8(a, pu, jb, lane);
    }
#pragma unroll
    for (int u = 0; u < kUnroll8; ++u) {
      if constexpr (!DUMP) s[u] = a.sx[c[u]] * a.sw8[p + u * W];
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) ax[u][tb] = load_xq(a, n0 + tb * 16 + arow, c[u] * 64 + akq * 16);
    }
#pragma unroll
    for (int u = 0; u < kUnroll8; ++u) {
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[u][tb], bw[u], v4i{0, 0, 0, 0}, 0, 0, 0);
        if constexpr (DUMP) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = n0 + tb * 16 + 4 * akq + v;
            if (row < a.n) a.dump[((int64_t)(p + u * W) * a.n + row) * 64 + jb * 16 + arow] = d[v];
          }
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[tb][v] = fmaf((float)d[v], s[u], acc[tb][v]);
        }
      }
    }
  }
  for (; p < hi8; p += W) {
    const int c = col_of(a.ids8[p], rbase, a.n_tc);
    const v4i bw = load_w8(a, p, jb, lane);
    float s = 0.0f;
    if constexpr (!DUMP) s = a.sx[c] * a.sw8[p];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const v4i ax = load_xq(a, n0 + tb * 16 + arow, c * 64 + akq * 16);
      v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, bw, v4i{0, 0, 0, 0}, 0, 0, 0);
      if constexpr (DUMP) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = n0 + tb * 16 + 4 * akq + v;
          if (row < a.n) a.dump[((int64_t)p * a.n + row) * 64 + jb * 16 + arow] = d[v];
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[tb][v] = fmaf((float)d[v], s, acc[tb][v]);
      }
    }
  }
  if constexpr (DUMP) return;

  // ---------------- 16-bit tiles ----------------
  if (a.w16 != nullptr) {
    const int lo16 = a.rp16[r], hi16 = a.rp16[r + 1];
    // continue the round-robin where the INT8 tiles stopped
    const int n8 = hi8 - lo8;
    const int first = (wave - (n8 % W) + W) % W;
    int q = lo16 + first;
    for (; q + (kUnroll16 - 1) * W < hi16; q += kUnroll16 * W) {
      int c[kUnroll16];
      v4i bw[kUnroll16][2];
      v4i ax[kUnroll16][TB][2];
#pragma unroll
      for (int u = 0; u < kUnroll16; ++u) {
        c[u] = col_of(a.ids16[q + u * W], rbase, a.n_tc);
        bw[u][0] = load_w16(a, q + u * W, jb, 0, lane);
        bw[u][1] = load_w16(a, q + u * W, jb, 1, lane);
      }
#pragma unroll
      for (int u = 0; u < kUnroll16; ++u)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            ax[u][tb][h] = load_xf(a, n0 + tb * 16 + arow, c[u] * 64 + h * 32 + akq * 8);
#pragma unroll
      for (int u = 0; u < kUnroll16; ++u)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          acc[tb] = mfma16<XT>(ax[u][tb][0], bw[u][0], acc[tb]);
          acc[tb] = mfma16<XT>(ax[u][tb][1], bw[u][1], acc[tb]);
        }
    }
    for (; q < hi16; q += W) {
      const int c = col_of(a.ids16[q], rbase, a.n_tc);
      const v4i b0 = load_w16(a, q, jb, 0, lane), b1 = load_w16(a, q, jb, 1, lane);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        const v4i a0 = load_xf(a, n0 + tb * 16 + arow, c * 64 + akq * 8);
        const v4i a1 = load_xf(a, n0 + tb * 16 + arow, c * 64 + 32 + akq * 8);
        acc[tb] = mfma16<XT>(a0, b0, acc[tb]);
        acc[tb] = mfma16<XT>(a1, b1, acc[tb]);
      }
    }
  }

  // ---------------- fixed-order reduction over waves + epilogue ----------------
  constexpr int E = TB * 4 * 64;
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[(wave * TB * 4 + tb * 4 + v) * 64 + lane] = acc[tb][v];
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float sum = red[e];
    for (int w = 1; w < W; ++w) sum += red[w * E + e];
    const int ln = e & 63, tv = e >> 6, tb = tv >> 2, v = tv & 3;
    const int row = n0 + tb * 16 + 4 * (ln >> 4) + v;
    const int col = r * 64 + jb * 16 + (ln & 15);
    if (row < a.n && col < a.m) {
      uint16_t y;
      if (a.out_bf16) {
        y = Bf16::from_f32(sum);
        if (a.bias) y = Bf16::from_f32(Bf16::to_f32(y) + Bf16::to_f32(a.bias[col]));
      } else {
        y = Fp16::from_f32(sum);
        if (a.bias) y = Fp16::from_f32(Fp16::to_f32(y) + Fp16::to_f32(a.bias[col]));
      }
      a.out[(int64_t)row * a.ldo + col] = y;
    }
  }
}

// ---- host side -----------------------------------------------------------

static int pick_tb(int n) { return n <= 16 ? 1 : (n <= 32 ? 2 : 4); }

// Waves per workgroup: aim for ~8 resident waves per CU over 256 CUs, keep at
// least 4 tiles per wave.
static int pick_waves(int n_tr, int n_tc, int tok_blocks, int split_k) {
  if (split_k > 0) return split_k < kMaxWaves ? split_k : kMaxWaves;
  const long groups = (long)n_tr * 4 * tok_blocks;
  long w = (2048 + groups - 1) / groups;
  long cap = (n_tc + 3) / 4;
  if (w > cap) w = cap;
  if (w > kMaxWaves) w = kMaxWaves;
  if (w < 1) w = 1;
  return (int)w;
}

template <class XT, bool DUMP>
static hipError_t launch(const GemmArgs& a, int W, hipStream_t s) {
  const int tb = DUMP ? 1 : pick_tb(a.n);
  if (W > max_waves_for(tb)) W = max_waves_for(tb);
  const int tok = (a.n + 16 * tb - 1) / (16 * tb);
  dim3 grid(a.n_tr * 4, tok);
  dim3 block(W * kWave);
  size_t lds = DUMP ? 0 : (size_t)W * tb * 4 * 64 * sizeof(float);
  if constexpr (DUMP) {
    hipLaunchKernelGGL((gemm_rows_kernel<XT, 1, true>), grid, block, lds, s, a);
  } else {
    switch (tb) {
      case 1: hipLaunchKernelGGL((gemm_rows_kernel<XT, 1, false>), grid, block, lds, s, a); break;
      case 2: hipLaunchKernelGGL((gemm_rows_kernel<XT, 2, false>), grid, block, lds, s, a); break;
      default: hipLaunchKernelGGL((gemm_rows_kernel<XT, 4, false>), grid, block, lds, s, a); break;
    }
  }
  return hipGetLastError();
}

static bool xvec_ok(const GemmArgs& a) {
  return a.k == a.n_tc * 64 && (a.ldq % 16) == 0 && aligned16(a.xq) &&
         (a.xf == nullptr || ((a.ldx % 8) == 0 && aligned16(a.xf)));
}

}  // namespace tq

using namespace tq;

extern "C" int64_t tq_gemm_workspace_elems(int n, int m, int n_tr, int n_tc, int split_k) {
  (void)n; (void)m; (void)n_tr; (void)n_tc; (void)split_k;
  return 0;  // the row-owned schedule reduces inside the workgroup
}

extern "C" int tq_gemm_mixed_rows(const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx,
                                  const int8_t* int8_tiles, const float* int8_scales,
                                  const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                                  const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                                  const void* fp16_tiles, const int32_t* fp16_tile_ids,
                                  const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                                  int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                                  int n_tc, int split_k, int tile_layout, float* workspace,
                                  int64_t workspace_elems, void* stream) {
  (void)workspace; (void)workspace_elems;
  if (n < 0 || m < 0 || k < 0 || n_tr < 0 || n_tc < 0) return TQ_ERR_ARG;
  if ((int64_t)n_tr * 64 < m || (int64_t)n_tc * 64 < k) return TQ_ERR_ARG;
  if (x_dtype != TQ_DTYPE_BF16 && x_dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (out_dtype != TQ_DTYPE_BF16 && out_dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (tile_layout != TQ_LAYOUT_ROW_MAJOR && tile_layout != TQ_LAYOUT_MFMA) return TQ_ERR_DTYPE;
  if (n == 0 || m == 0) return TQ_OK;
  if (out == nullptr || out_stride_n < m || int8_row_ptr == nullptr || x_int8 == nullptr || sx == nullptr)
    return TQ_ERR_ARG;
  if (x_int8_stride_n < k) return TQ_ERR_ARG;
  const bool has16 = fp16_tiles != nullptr && fp16_tile_ids != nullptr && fp16_row_ptr != nullptr;
  if (has16 && (x_fp == nullptr || x_fp_stride_n < k)) return TQ_ERR_ARG;
  if (!aligned16(int8_tiles) || (has16 && !aligned16(fp16_tiles))) return TQ_ERR_ALIGN;
  GemmArgs a{};
  a.xq = x_int8; a.ldq = x_int8_stride_n; a.sx = sx;
  a.w8 = int8_tiles; a.sw8 = int8_scales; a.ids8 = int8_tile_ids; a.rp8 = int8_row_ptr;
  a.xf = has16 ? static_cast<const uint16_t*>(x_fp) : nullptr; a.ldx = x_fp_stride_n;
  a.w16 = has16 ? static_cast<const uint16_t*>(fp16_tiles) : nullptr;
  a.ids16 = fp16_tile_ids; a.rp16 = fp16_row_ptr;
  a.out = static_cast<uint16_t*>(out); a.ldo = out_stride_n;
  a.bias = static_cast<const uint16_t*>(bias);
  a.dump = nullptr;
  a.n = n; a.m = m; a.k = k; a.n_tr = n_tr; a.n_tc = n_tc;
  a.out_bf16 = out_dtype == TQ_DTYPE_BF16;
  a.layout = tile_layout;
  a.xvec = xvec_ok(a);
  const int tb = pick_tb(n);
  const int W = pick_waves(n_tr, n_tc, (n + 16 * tb - 1) / (16 * tb), split_k);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = (x_dtype == TQ_DTYPE_BF16) ? launch<Bf16, false>(a, W, s) : launch<Fp16, false>(a, W, s);
  return (int)e;
}

extern "C" int tq_gemm_tile_products_i32(const int8_t* x_int8, int64_t x_int8_stride_n,
                                         const int8_t* int8_tiles, const int32_t* int8_tile_ids,
                                         const int32_t* int8_row_ptr, int n, int k, int n_tr, int n_tc,
                                         int tile_layout, int32_t* products, void* stream) {
  if (n < 0 || k < 0 || n_tr < 0 || n_tc < 0) return TQ_ERR_ARG;
  if ((int64_t)n_tc * 64 < k) return TQ_ERR_ARG;
  if (tile_layout != TQ_LAYOUT_ROW_MAJOR && tile_layout != TQ_LAYOUT_MFMA) return TQ_ERR_DTYPE;
  if (n == 0 || n_tr == 0) return TQ_OK;
  if (x_int8 == nullptr || int8_row_ptr == nullptr || products == nullptr || x_int8_stride_n < k)
    return TQ_ERR_ARG;
  if (!aligned16(int8_tiles)) return TQ_ERR_ALIGN;
  GemmArgs a{};
  a.xq = x_int8; a.ldq = x_int8_stride_n;
  a.w8 = int8_tiles; a.ids8 = int8_tile_ids; a.rp8 = int8_row_ptr;
  a.dump = products;
  a.n = n; a.m = n_tr * 64; a.k = k; a.n_tr = n_tr; a.n_tc = n_tc;
  a.layout = tile_layout;
  a.xvec = xvec_ok(a);
  a.sx = nullptr; a.sw8 = nullptr;  // the dump path reads no scales
  return (int)launch<Bf16, true>(a, 4, static_cast<hipStream_t>(stream));
}
