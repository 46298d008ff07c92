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

#include <algorithm>
#include <atomic>
#include <vector>

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
  // DUMP instantiations only: int32 [T8, dump_n, 64] products of token rows
  // dump_r0 .. dump_r0 + dump_n - 1 (see dump_i32)
  int32_t* dump;
  int dump_r0, dump_n;
  int n, m, k, n_tr, n_tc;
  int out_bf16;   // output dtype: 1 bf16, 0 fp16
  int layout;     // TQ_LAYOUT_*
  int xvec;       // activations allow 16-byte loads (aligned rows, k == 64 * n_tc)
  int ovec;       // output rows allow 16-byte stores (16-byte aligned base, ldo % 8 == 0)
  int xblk;       // > 0: xq is token-blocked (TQ_XQ_TOKEN_BLOCKED) with xblk 16-row blocks per column tile
  int splits;       // split-K decode kernel: splits per row tile
  int32_t* counters;  // [n_tr] arrival counters (zero between launches)
  float* partials;    // [n_tr, splits, n, 64] fp32 split partials
  // Prefill work plan (nullptr: row pairs in order).  units[u] = first row
  // tile | kUnitSingle when the unit is that row tile alone; the first
  // n_first units take all their token blocks before the others start.
  const int32_t* units;
  int n_units, n_first;
  // Cooperative quantize + GEMM (gemm_decode_kernel<..., COOP>): the first
  // coop_p workgroups write the activation codes to xq / sx; coop is the
  // workspace head of ready flags and counts (kCoop* below); a GEMM workgroup
  // waits at most coop_spin polls, then quantizes locally.
  int32_t* coop;
  int coop_p, coop_spin;
};

// COOP workspace head (int32 entries, zero between launches): GEMM workgroup
// c polls the ready flag of group g = c % kCoopGroups at kCoopStride * g, and
// counts itself passed right after it; the producers count themselves done at
// kCoopCount.  One flag per group and one 128-byte line per flag: a single
// flag polled by every workgroup of a large grid serialises the polls (and
// the counts) at one memory channel.
constexpr int kCoopGroups = 64;
constexpr int kCoopStride = 32;
constexpr int kCoopCount = kCoopGroups * kCoopStride;

constexpr int32_t kUnitSingle = 1 << 30;

constexpr int kDecodeMaxTokens = 64;  // token counts served by gemm_splitk_kernel
constexpr int kFusedMaxTokens = 16;   // token counts the fused quantize+GEMM path takes
constexpr size_t kFusedMaxLds = 64 * 1024;   // the fused path keeps n x k int8 codes in LDS

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
// XVEC (aligned rows, k == 64 * n_tc) is a template switch in the split-K
// kernel and a runtime one in the general kernel.
template <int XVEC = -1>
__device__ inline v4i load_xq(const GemmArgs& a, int row, int col) {
  if constexpr (XVEC == 1) {
    // branch-free: read a valid row, zero the padding rows with a select
    const v4i v = *reinterpret_cast<const v4i*>(a.xq + (int64_t)min(row, a.n - 1) * a.ldq + col);
    return row < a.n ? v : v4i{0, 0, 0, 0};
  }
  if (row >= a.n) return v4i{0, 0, 0, 0};
  const int8_t* p = a.xq + (int64_t)row * a.ldq + col;
  if (XVEC == 1 || (XVEC == -1 && a.xvec)) return *reinterpret_cast<const v4i*>(p);
  uint32_t w[4] = {0, 0, 0, 0};
  for (int e = 0; e < 16; ++e)
    if (col + e < a.k) w[e >> 2] |= (uint32_t)(uint8_t)p[e] << (8 * (e & 3));
  return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// A operand: 8 16-bit activations of row `row`, columns col .. col+7.
template <int XVEC = -1>
__device__ inline v4i load_xf(const GemmArgs& a, int row, int col) {
  if constexpr (XVEC == 1) {
    const v4i v = *reinterpret_cast<const v4i*>(a.xf + (int64_t)min(row, a.n - 1) * a.ldx + col);
    return row < a.n ? v : v4i{0, 0, 0, 0};
  }
  if (row >= a.n) return v4i{0, 0, 0, 0};
  const uint16_t* p = a.xf + (int64_t)row * a.ldx + col;
  if (XVEC == 1 || (XVEC == -1 && a.xvec)) return *reinterpret_cast<const v4i*>(p);
  uint32_t w[4] = {0, 0, 0, 0};
  for (int e = 0; e < 8; ++e)
    if (col + e < a.k) w[e >> 1] |= (uint32_t)p[e] << (16 * (e & 1));
  return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// Column tile of a tile id owned by row tile r (id = r * n_tc + c).  Clamped so
// that a malformed pack can never index sx / x out of range.
__device__ inline int col_of(int id, int rbase, int n_tc) {
  return (int)min((unsigned)(id - rbase), (unsigned)(n_tc - 1));
}

// Test instantiations (DUMP = true) of the production kernels: the exact
// INT32 result d of an INT8 tile's v_mfma_i32_16x16x64_i8, before its scale
// FMA, is also written to a.dump[p][row - dump_r0][col] for the token rows
// row0 + v (v = 0..3, the D layout) inside [dump_r0, dump_r0 + dump_n).  p is
// the tile's INT8 position, col the output feature inside the row tile.
// Everything else in the kernel is unchanged, so the products come from the
// very instruction stream that computes the outputs.
template <bool DUMP>
__device__ inline void dump_i32(const GemmArgs& a, int p, int row0, int col, const v4i& d) {
  if constexpr (DUMP) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int rr = row0 + v - a.dump_r0;
      if ((unsigned)rr < (unsigned)a.dump_n) a.dump[((int64_t)p * a.dump_n + rr) * 64 + col] = d[v];
    }
  }
}

// The W wave partials of element e (red[w * E + e]) summed in wave order --
// bitwise the loop sum = red[e]; sum += red[w * E + e] for w = 1 .. W - 1 --
// with every LDS read issued before the first add (reads for w >= W re-read
// wave W - 1 and are not added).  Used where a thread sums several elements:
// the rolled loop waits one LDS round trip per wave and element.
template <int WMAX>
__device__ inline float wave_order_sum(const float* red, int E, int e, int W) {
  float v[WMAX];
#pragma unroll
  for (int w = 0; w < WMAX; ++w) v[w] = red[min(w, W - 1) * E + e];
  float sum = v[0];
#pragma unroll
  for (int w = 1; w < WMAX; ++w) sum = w < W ? sum + v[w] : sum;
  return sum;
}

// ---- split-K decode kernel (N <= 64 tokens) ---------------------------------
//
// Workgroup (r, s), s < S, owns split s of row tile r: INT8 positions
// [lo8 + n8*s/S, lo8 + n8*(s+1)/S) and 16-bit positions likewise (the
// reference's row-owned split-K, gemm_rows_splitk_64x64.py:121-124, 140-143).
// Each of its W waves takes WHOLE 4 KiB tiles round-robin and issues the
// four 1 KiB j-block loads of up to U tiles before any dependent work, so a
// wave streams contiguous memory and has U*4 KiB in flight.  Per INT8 tile:
// 4 j-blocks x TB token blocks of v_mfma_i32_16x16x64_i8, fp32 FMA by
// sx[c]*sw[t]; per 16-bit tile: 4 x TB x 2 v_mfma_f32_16x16x32_{bf16,f16}.
//
// FUSED: the wave quantizes column tile c of the activation itself (absmax
// over all n <= 16 rows, bf16/fp16-rounded scale, IEEE-divide codes -- the
// same closed form as tq_act_quant) into a 1 KiB LDS slot and reads its A
// operand back from there.  A split only needs its own column tiles, so the
// activation quantization costs one extra pass per row tile instead of a
// launch, and its results are bitwise those of the separate quantizer.
//
// Reduction: waves sum through LDS in wave order; with S > 1 every split
// stores its fp32 partial (rows < n only), releases it at device scope and
// bumps the row tile's arrival counter; the last arriver acquires, sums the
// S partials in split order 0..S-1 (bitwise reproducible) and resets the
// counter to zero for the next launch, as the reference's semaphore epilogue
// (gemm_rows_splitk_64x64.py:159-183).  No waiting: no workgroup ever spins.

template <int NPOW>
struct QuantLanes {
  static constexpr int kVpl = NPOW;          // values per lane
  static constexpr int kLpr = 64 / NPOW;     // lanes per row
};

// This lane's VPL raw 16-bit activations of column tile c: row lane / lpr,
// columns c*64 + (lane % lpr)*VPL .. +VPL, zero past k or at rows >= n.
template <int NPOW, bool XVEC>
struct XSlice {
  static constexpr int kVpl = NPOW, kLpr = 64 / NPOW;
  uint16_t raw[kVpl];
  __device__ inline void load(const GemmArgs& a, int c, int lane) {
    const int row = lane / kLpr;
    const int col0 = c * 64 + (lane % kLpr) * kVpl;
    if constexpr (XVEC) {
      // branch-free: read a valid row, zero rows >= n afterwards
      const uint16_t* p = a.xf + (int64_t)min(row, a.n - 1) * a.ldx + col0;
      if constexpr (kVpl >= 8) {
#pragma unroll
        for (int i = 0; i < kVpl / 8; ++i) {
          const u32x4 w = reinterpret_cast<const u32x4*>(p)[i];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            raw[8 * i + 2 * j] = (uint16_t)(w[j] & 0xffffu);
            raw[8 * i + 2 * j + 1] = (uint16_t)(w[j] >> 16);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < kVpl; ++i) raw[i] = p[i];
      }
      if (row >= a.n) {
#pragma unroll
        for (int i = 0; i < kVpl; ++i) raw[i] = 0;
      }
      return;
    }
    const uint16_t* p = a.xf + (int64_t)row * a.ldx + col0;
    if (row >= a.n) {
#pragma unroll
      for (int i = 0; i < kVpl; ++i) raw[i] = 0;
    } else {
#pragma unroll
      for (int i = 0; i < kVpl; ++i) raw[i] = (XVEC || col0 + i < a.k) ? p[i] : (uint16_t)0;
    }
  }
};

// Quantizes a loaded column tile c into slot[row*ld + col] (int8 codes,
// rows < n, columns of the tile) and returns sx[c]: the closed form of
// tq_act_quant over all n rows.  Columns >= k get code 0, as the masked loads
// of the unfused GEMM read them.
template <class XT, int NPOW, bool XVEC>
__device__ inline float quant_col_tile(const GemmArgs& a, const XSlice<NPOW, XVEC>& xs, int c, int lane,
                                       int8_t* slot, int ld) {
  constexpr int kVpl = NPOW, kLpr = 64 / NPOW;
  const int row = lane / kLpr;
  const int col0 = c * 64 + (lane % kLpr) * kVpl;
  float v[kVpl];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    v[i] = XT::to_f32(xs.raw[i]);
    m = fmaxf(m, fabsf(v[i]));
  }
  const float s = act_scale_from_absmax<XT>(wave_max_nonneg(m));
  const CodeScale cs(s);
  if (row < a.n) {
    uint32_t words[(kVpl + 3) / 4] = {};
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
      const int q = (XVEC || col0 + i < a.k) ? cs.code(v[i]) : 0;
      words[i / 4] |= (uint32_t)(q & 0xff) << (8 * (i % 4));
    }
    int8_t* dst = slot + row * ld + (lane % kLpr) * kVpl;
    if constexpr (kVpl >= 4) {
#pragma unroll
      for (int w = 0; w < kVpl / 4; ++w) reinterpret_cast<uint32_t*>(dst)[w] = words[w];
    } else {
#pragma unroll
      for (int i = 0; i < kVpl; ++i) dst[i] = (int8_t)((words[0] >> (8 * i)) & 0xff);
    }
  }
  return s;
}

// JBW = j-blocks (16 output features each) per workgroup: 4 = whole 4 KiB
// tiles per wave; 2 = half tiles (two workgroups per row tile); 1 = one 1 KiB
// j-block of each tile (four workgroups share a row tile, so narrow outputs
// still fill the GPU without any cross-workgroup reduction).  Launch bound:
// 16 waves at JBW 1, 8 at JBW 2 and 4.
// XBLK: the codes are token-blocked (a.xblk blocks of 16 rows per column
// tile): each activation operand is one contiguous 1 KiB load.
template <class XT, int TB, int U, bool FUSED, int NPOW, bool XVEC, int JBW, bool XBLK = false, bool DUMP = false>
__global__ void __launch_bounds__(JBW == 1 ? 1024 : 512)
gemm_splitk_kernel(GemmArgs a) {
  static_assert(!(XBLK && FUSED), "the fused prologue stages its own codes");
  // a batch of U tiles must never straddle two 64-tile metadata windows
  static_assert(64 % U == 0, "U must divide the 64-tile window");
  // dynamic LDS: FUSED codes [n][64*n_tc] + sx[n_tc] during the main loop,
  // the wave partials for the reduction afterwards (the two never overlap in time)
  extern __shared__ float red[];
  __shared__ int last_arriver;
  constexpr int NJG = 4 / JBW;                  // j-block groups per row tile
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int S = a.splits;
  const int unit = blockIdx.x / S, s = blockIdx.x - (blockIdx.x / S) * S;
  const int r = unit / NJG, jb0 = (unit - (unit / NJG) * NJG) * JBW;
  const int arow = lane & 15, akq = lane >> 4;
  const int rbase = r * a.n_tc;

  v4f acc[JBW][TB];
#pragma unroll
  for (int j = 0; j < JBW; ++j)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[j][tb] = v4f{0.f, 0.f, 0.f, 0.f};

  const int lo8r = a.rp8[r], hi8r = a.rp8[r + 1];
  const int n8r = hi8r - lo8r;
  const int lo8 = lo8r + (n8r * s) / S, hi8 = lo8r + (n8r * (s + 1)) / S;
  const int n8 = hi8 - lo8;

  // ---------------- INT8 tiles: wave takes positions lo8 + wave + i*W ----------------
  // Batches of U tiles: weights and activation operands of a batch are all in
  // flight before the first wait; the load phases are branch-free (positions
  // past the batch re-read the last valid tile, an L2 hit, and are never used).
  v4i bw[U][JBW];
  const int first_p = lo8 + wave;
  auto load_weights = [&](int p0, v4i (&dst)[U][JBW]) {   // need no id
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pu = min(p0 + u * W, hi8 - 1);
#pragma unroll
      for (int j = 0; j < JBW; ++j) dst[u][j] = load_w8(a, pu, jb0 + j, lane);
    }
  };
  if (first_p < hi8) load_weights(first_p, bw);   // the first batch streams during the prologue

  const int ldc = a.n_tc * 64;                    // FUSED: LDS code row stride
  int8_t* codes = reinterpret_cast<int8_t*>(red);
  float* sxl = reinterpret_cast<float*>(codes + ((a.n * ldc + 15) & ~15));
  if constexpr (FUSED) {
    // Prologue: the waves quantize column tiles c = wave, wave + W, ... of the
    // activation into LDS (closed form of tq_act_quant), QB tiles per pass
    // with all their loads issued first, while the weights are in flight.
    constexpr int QB = 4;
    for (int c0 = wave; c0 < a.n_tc; c0 += QB * W) {
      XSlice<NPOW, XVEC> xs[QB];
#pragma unroll
      for (int q = 0; q < QB; ++q) xs[q].load(a, min(c0 + q * W, a.n_tc - 1), lane);
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int c = c0 + q * W;
        if (c < a.n_tc) {
          const float sxc = quant_col_tile<XT, NPOW, XVEC>(a, xs[q], c, lane, codes + c * 64, ldc);
          if (lane == 0) sxl[c] = sxc;
        }
      }
    }
    __syncthreads();
  }

  // Whole-tile (JBW 4) waves issue the next batch's weights after this
  // batch's activation loads and before its MFMAs, so one batch's compute and
  // the next one's HBM round trip overlap (vmcnt returns in order: the MFMAs
  // wait for the activation only).  One-j-block waves have no registers to
  // spare for it at 16 waves per workgroup.
  constexpr bool PREFETCH = JBW == 4;
  v4i bwn[U][JBW];
  // The ids, weight scales and activation scales of up to 64 of the wave's
  // tiles come with one vector load each (lane i: the wave's tile w0 + i W;
  // past the end the last tile again), once per window of 64 tiles and
  // outside the batch loop.  The batch loop then issues no conditional loads,
  // so its waits count exactly: a window reload inside it made every batch
  // wait for all of its loads (the next batch's prefetched weights included),
  // and a scalar load of sx[c] per tile put a scalar round trip before each
  // tile's MFMAs.  Same tiles, same order: outputs are unchanged.
  for (int w0 = first_p; w0 < hi8; w0 += 64 * W) {
    const int pc = min(w0 + lane * W, hi8 - 1);
    const int cl = col_of(a.ids8[pc], rbase, a.n_tc);
    const float swl = a.sw8[pc];
    float sxv;
    if constexpr (FUSED) sxv = sxl[cl];
    else sxv = a.sx[cl];
    const int wend = min(hi8, w0 + 64 * W);   // 64 is a multiple of U: batches never straddle windows
    for (int p0 = w0; p0 < wend; p0 += U * W) {
      const int k0 = (p0 - w0) / W;
      const int nu = min(U, (hi8 - p0 + W - 1) / W);   // valid tiles in this batch (uniform)
      // Activation operands first, then (one-j-block waves) this batch's
      // weights: both round trips in flight together.  Issued the other way
      // round, the compiler's wait before the activation addresses (the
      // previous batch's loads) also waited for the weights just issued.
      v4i ax[U][TB];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = __builtin_amdgcn_readlane(cl, k0 + u);
        if constexpr (FUSED) {
          ax[u][0] = (arow < a.n) ? *reinterpret_cast<const v4i*>(codes + arow * ldc + c * 64 + akq * 16)
                                  : v4i{0, 0, 0, 0};
        } else {
#pragma unroll
          for (int tb = 0; tb < TB; ++tb) {
            if constexpr (XBLK) {   // blocks past the last one: zero operand (clamped read stays in the buffer)
              const v4i v = *reinterpret_cast<const v4i*>(
                  a.xq + ((int64_t)(c * a.xblk + min(tb, a.xblk - 1)) * 64 + lane) * 16);
              ax[u][tb] = tb < a.xblk ? v : v4i{0, 0, 0, 0};
            } else {
              ax[u][tb] = load_xq<XVEC ? 1 : 0>(a, tb * 16 + arow, c * 64 + akq * 16);
            }
          }
        }
      }
      if (p0 != first_p) {
        if constexpr (PREFETCH) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int j = 0; j < JBW; ++j) bw[u][j] = bwn[u][j];
        } else {
          load_weights(p0, bw);
        }
      }
      if (PREFETCH && p0 + U * W < hi8) load_weights(p0 + U * W, bwn);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < nu) {
          const float sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sxv), k0 + u)) *
                           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(swl), k0 + u));
#pragma unroll
          for (int j = 0; j < JBW; ++j)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
              const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[u][tb], bw[u][j], v4i{0, 0, 0, 0}, 0, 0, 0);
              dump_i32<DUMP>(a, p0 + u * W, tb * 16 + 4 * akq, (jb0 + j) * 16 + arow, d);
#pragma unroll
              for (int v = 0; v < 4; ++v) acc[j][tb][v] = fmaf((float)d[v], sc, acc[j][tb][v]);
            }
        }
    }
  }

  // ---------------- 16-bit tiles: rotation continues after the INT8 ones ----------------
  if (a.w16 != nullptr) {
    const int lo16r = a.rp16[r], hi16r = a.rp16[r + 1];
    const int n16r = hi16r - lo16r;
    const int lo16 = lo16r + (n16r * s) / S, hi16 = lo16r + (n16r * (s + 1)) / S;
    const int first = (wave - (n8 % W) + W) % W;
    for (int q = lo16 + first; q < hi16; q += W) {
      const int c = col_of(a.ids16[q], rbase, a.n_tc);
      v4i bw[JBW][2];
#pragma unroll
      for (int j = 0; j < JBW; ++j) {
        bw[j][0] = load_w16(a, q, jb0 + j, 0, lane);
        bw[j][1] = load_w16(a, q, jb0 + j, 1, lane);
      }
      v4i ax[TB][2];
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int h = 0; h < 2; ++h) ax[tb][h] = load_xf<XVEC ? 1 : 0>(a, tb * 16 + arow, c * 64 + h * 32 + akq * 8);
#pragma unroll
      for (int j = 0; j < JBW; ++j)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          acc[j][tb] = mfma16<XT>(ax[tb][0], bw[j][0], acc[j][tb]);
          acc[j][tb] = mfma16<XT>(ax[tb][1], bw[j][1], acc[j][tb]);
        }
    }
  }

  // ---------------- waves -> LDS -> one partial per workgroup ----------------
  constexpr int E = JBW * TB * 4 * 64;   // (j, tb, v, lane)
  if constexpr (FUSED) __syncthreads();   // every wave is done reading the codes
#pragma unroll
  for (int j = 0; j < JBW; ++j)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave * E + ((j * TB + tb) * 4 + v) * 64 + lane] = acc[j][tb][v];
  __syncthreads();

  // element e -> (row, column within the row tile); rows >= n are padding
  auto coords = [&](int e, int& row, int& jcol) {
    const int ln = e & 63, t = e >> 6, v = t & 3, tb = (t >> 2) % TB, j = (t >> 2) / TB;
    row = tb * 16 + 4 * (ln >> 4) + v;
    jcol = (jb0 + j) * 16 + (ln & 15);
  };
  auto store = [&](int row, int jcol, float sum) {
    const int col = r * 64 + jcol;
    if (col >= a.m) return;
    uint16_t y;
    if (a.out_bf16) {
      y = Bf16::from_f32(sum);
      if (a.bias) y = Bf16::from_f32(Bf16::to_f32(y) + Bf16::to_f32(a.bias[col]));
    } else {
      y = Fp16::from_f32(sum);
      if (a.bias) y = Fp16::from_f32(Fp16::to_f32(y) + Fp16::to_f32(a.bias[col]));
    }
    a.out[(int64_t)row * a.ldo + col] = y;
  };

  if (S == 1) {
    if (JBW == 4 && E >= 4 * (int)blockDim.x) {
      // whole-tile workgroups at 33-64 rows: 8+ elements per thread, four at a
      // time with all of their reads in flight together (the rolled loop below
      // took ~3.7 us on the stacked Gate/Up at 64 rows)
      for (int e0 = threadIdx.x; e0 < E; e0 += 4 * blockDim.x) {
        float sums[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sums[i] = wave_order_sum<8>(red, E, min(e0 + i * (int)blockDim.x, E - 1), W);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = e0 + i * (int)blockDim.x;
          int row, jcol;
          coords(min(e, E - 1), row, jcol);
          if (e < E && row < a.n) store(row, jcol, sums[i]);
        }
      }
      return;
    }
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      int row, jcol;
      coords(e, row, jcol);
      if (row >= a.n) continue;
      float sum = red[e];
      for (int w = 1; w < W; ++w) sum += red[w * E + e];
      store(row, jcol, sum);
    }
    return;
  }

  // Cross-workgroup hand-off without cache-wide maintenance: partials are
  // written with agent-scope (sc1, write-through) stores, every thread waits
  // for its stores to complete, then one thread bumps the counter; the last
  // arriver reads the partials with agent-scope loads that bypass the
  // non-coherent L1/L2 copies.  (A device-scope __threadfence() would instead
  // write back and invalidate the whole L2 of the XCD.)
  float* part = a.partials + ((int64_t)unit * S + s) * a.n * 64;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int row, jcol;
    coords(e, row, jcol);
    if (row >= a.n) continue;
    float sum = red[e];
    for (int w = 1; w < W; ++w) sum += red[w * E + e];
    __hip_atomic_store(part + row * 64 + jcol, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // every thread's stores must be complete (acknowledged at the coherence
  // point) before the counter moves: on gfx9 stores count in vmcnt
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(a.counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_arriver = (prev == S - 1);
  }
  __syncthreads();
  if (!last_arriver) return;
  const float* unitp = a.partials + (int64_t)unit * S * a.n * 64;
  for (int e = threadIdx.x; e < a.n * JBW * 16; e += blockDim.x) {
    const int row = e / (JBW * 16), jcol = jb0 * 16 + e % (JBW * 16);
    const int off = row * 64 + jcol;
    float sum = __hip_atomic_load(unitp + off, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int t = 1; t < S; ++t)
      sum += __hip_atomic_load(unitp + (int64_t)t * a.n * 64 + off, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    store(row, jcol, sum);
  }
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- decode kernel with the activation staged in LDS ------------------------
//
// Same unit decomposition as gemm_splitk_kernel with one split: workgroup =
// (row tile r, group of JBW j-blocks), W waves taking the row's tiles
// round-robin.  A decode GEMM lasts a few microseconds, so its duration is set
// by the number of DEPENDENT memory round trips, not by arithmetic.  This
// kernel has two: the row's tile range (row_ptr), then everything else.
//   1. At entry every thread issues its share of the activation -- int8 codes
//      and sx, or (QUANT) the raw 16-bit values -- which depends on nothing.
//   2. Each wave issues all of its tiles (up to UMAX per batch; one 16-byte
//      load per lane per j-block) with their ids and scales.
//   3. While the weights stream, the activation goes to LDS.  QUANT computes
//      the codes there first, by the closed form of tq_act_quant: an LDS
//      atomic max per column tile over all n rows, the scale rounded to the
//      input dtype, IEEE-exact codes -- bit for bit the separate kernel's.
//      The hand-offs use lds_barrier(), which leaves the weight loads in
//      flight.
//   4. MFMAs read their A operand from LDS at the tile's column: no global
//      load waits for a tile id.
// Codes live in LDS as [n][k + 16] (16-byte row padding spreads the rows of one
// A-operand read over different banks); the reduction buffer reuses the area
// afterwards.  Needs k == 64 * n_tc, 16-byte aligned activation rows, S == 1.

// LDS bytes for staged codes.  144 KiB takes k = 8192 up to 16 rows (Down of
// Llama-3.2-3B: a 16-wave workgroup is alone on its CU anyway); measured on
// MI355X, Down at 9 / 12 / 16 rows 10.14 / 10.17 / 10.20 us on the split-K
// kernel (token-blocked codes) -> 8.98 / 9.03 / 9.15 us staged, bitwise equal.
constexpr int kDecCodesMax = 144 * 1024;

// ---- cooperative activation quantization (COOP decode launches) -------------
// The decode GEMM's input codes are a function of all n rows of each 64-column
// tile (the scale is the tile's absmax over every row), so a GEMM workgroup
// cannot start its MFMAs before the whole tile is quantized.  Two launches
// (quantizer, then GEMM) pay a launch; quantizing in every GEMM workgroup
// repeats the work hundreds of times.  COOP launches do it once: producer
// workgroup p < P quantizes column tiles [n_tc p / P, n_tc (p + 1) / P) with
// the closed form of tq_act_quant, stores codes and scales with write-through
// (agent-scope, sc1) stores, waits until they are acknowledged and counts
// itself done; the GEMM workgroups issue their weight loads first and fetch
// the codes, with agent-scope loads, once all P producers are done.

// Group g of a COOP launch is passed by each of its GEMM workgroups (after its
// last poll) and by the last producer (after raising the flag); whoever
// brings the count to the group's size + 1 zeroes the flag and the count, so
// no poll and no count of this launch lands after the reset.
__device__ inline void coop_pass(const GemmArgs& a, int g) {
  const int consumers = (int)gridDim.x - a.coop_p;
  const int size = consumers / kCoopGroups + (g < consumers % kCoopGroups ? 1 : 0);
  int32_t* f = a.coop + g * kCoopStride;
  const int prev = __hip_atomic_fetch_add(f + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (prev == size) {
    __hip_atomic_store(f, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(f + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Producer p: codes of its column tiles, over all n <= 16 rows, into a.xq
// (row stride a.ldq) and a.sx.  dsm holds [tiles] absmax bit patterns.
template <class XT>
__device__ void coop_produce(const GemmArgs& a, int p, int8_t* dsm) {
  const int P = a.coop_p;
  const int c0 = (int)((int64_t)a.n_tc * p / P), c1 = (int)((int64_t)a.n_tc * (p + 1) / P);
  const int nt = c1 - c0;
  const int T = blockDim.x;
  uint32_t* amax = reinterpret_cast<uint32_t*>(dsm);
  for (int i = threadIdx.x; i < nt; i += T) amax[i] = 0u;
  __syncthreads();
  // item i = ((row * nt) + tile) * 8 + chunk: the 8 chunks of a (row, tile)
  // are 8 aligned consecutive lanes (items and T are multiples of 8)
  const int items = a.n * nt * 8;
  auto x_at = [&](int i, int& row, int& c, int& col) {
    row = i / (nt * 8);
    const int rem = i - row * nt * 8;
    c = c0 + (rem >> 3);
    col = c * 64 + (rem & 7) * 8;
    return *reinterpret_cast<const u32x4*>(a.xf + (int64_t)row * a.ldx + col);
  };
  for (int i = threadIdx.x; i < items; i += T) {
    int row, c, col;
    const u32x4 x = x_at(i, row, c, col);
    uint32_t m = __float_as_uint(max8<XT>(x, 0.0f));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));    // quad_perm 1,0,3,2
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));    // quad_perm 2,3,0,1
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));   // row_half_mirror
    if ((threadIdx.x & 7) == 0) __hip_atomic_fetch_max(amax + (c - c0), m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t qr = row_rsrc(a.xq, (int)((int64_t)(a.n - 1) * a.ldq + a.k));
  for (int i = threadIdx.x; i < items; i += T) {
    int row, c, col;
    const u32x4 x = x_at(i, row, c, col);
    const float s = act_scale_from_absmax<XT>(__uint_as_float(amax[c - c0]));
    const CodeScale cq(s, 1.0f / s);
    const u32x2 q = codes8<XT>(x, cq);
    // write-through to the coherence point (sc1), like the agent-scope stores
    __builtin_amdgcn_raw_buffer_store_b64(q, qr, (int)((int64_t)row * a.ldq + col), 0, 16);
  }
  for (int t = threadIdx.x; t < nt; t += T) {
    const float s = act_scale_from_absmax<XT>(__uint_as_float(amax[t]));
    __hip_atomic_store(const_cast<float*>(a.sx) + c0 + t, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // every store acknowledged before the count moves (gfx9 stores count in vmcnt)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < 64) {
    int prev = 0;
    if (threadIdx.x == 0) prev = __hip_atomic_fetch_add(a.coop + kCoopCount, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev == P - 1) {
      // the last producer: every code and scale is acknowledged.  Zero the
      // count (all P have landed), raise the 64 groups' flags (lane g: group
      // g), and once they are acknowledged count itself into every group.
      if (threadIdx.x == 0) __hip_atomic_store(a.coop + kCoopCount, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.coop + threadIdx.x * kCoopStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      coop_pass(a, threadIdx.x);
    }
  }
}


// Byte offset of this lane's 16-byte B-operand chunk of j-block jb, k-half h
// inside a 16-bit tile (the element offsets of load_w16, times two).
__device__ inline int w16_lane_offset(int layout, int jb, int h, int lane) {
  return layout == TQ_LAYOUT_MFMA ? (jb * 2 + h) * 1024 + lane * 16
                                  : jb * 2048 + (lane & 15) * 128 + h * 64 + (lane >> 4) * 16;
}

// Byte offset of this lane's 16-byte B-operand chunk of j-block 0 inside an
// INT8 tile (add jb * 1024 in the MFMA layout; the row-major layout places
// j-block jb at rows 16 jb .. 16 jb + 15, i.e. also + jb * 1024).
__device__ inline int w8_lane_offset(int layout, int lane) {
  return layout == TQ_LAYOUT_MFMA ? lane * 16 : (lane & 15) * 64 + (lane >> 4) * 16;
}

// COOP (one token block, one-j-block workgroups, codes not quantized in the
// workgroup): a cooperative quantize + GEMM launch.  Workgroups below a.coop_p
// are producers (coop_produce); the others are GEMM units with one extra
// wave, the loader, beyond the W waves that take tiles.  The loader polls the
// producers' count (bounded by a.coop_spin), then every thread loads the codes
// with agent-scope loads into LDS -- or, if the count never arrived, the
// workgroup quantizes the activation itself (same closed form, same codes).
// The W tile waves issue their weights first, so the wait overlaps them.
//
// HELP (QUANT, one token block, one-j-block workgroups): k / 512 helper waves
// beyond the W tile waves load the raw activation and quantize it by lanes
// (one thread per 8-column chunk of a row) into LDS while the tile waves wait
// on their weight issue, which the memory system throttles for microseconds;
// in the plain QUANT kernel the same quantization runs in the tile waves after
// their issue, on the critical path.  Same W, same per-wave tile order, same
// codes: bitwise the plain kernel's outputs.
template <class XT, int TB, int JBW, int UMAX, bool QUANT, int CMAX, bool DUMP = false, bool COOP = false,
          bool HELP = false>
__global__ void __launch_bounds__(JBW == 4 ? 512 : 1024)
gemm_decode_kernel(GemmArgs a) {
  static_assert(!COOP || (!QUANT && TB == 1 && JBW == 1), "cooperative launches: codes from producers, n <= 16");
  static_assert(!HELP || (QUANT && !COOP && TB == 1 && JBW == 1 && UMAX <= 8), "helper waves: lane quantizer");
  extern __shared__ __align__(16) int8_t dsm[];
  constexpr int NJG = 4 / JBW;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int T = blockDim.x, W = (T >> 6) - (COOP ? 1 : (HELP ? (a.k >> 9) : 0));
  int bid = blockIdx.x;
  if constexpr (COOP) {
    if (bid < a.coop_p) {
      coop_produce<XT>(a, bid, dsm);
      return;
    }
    bid -= a.coop_p;   // coop_p % 8 == 0: the unit keeps its XCD
  }
  const bool loader = COOP && wave == W;
  const bool idle = (COOP || HELP) && wave >= W;   // no tiles: the COOP loader, the HELP helpers
  // HELP: helper thread tq of Tq = k / 8 takes chunk tq of every row
  const int tq = HELP ? (int)threadIdx.x - W * 64 : (int)threadIdx.x;
  const int Tq = HELP ? T - W * 64 : T;
  // Workgroups are dealt to the 8 XCDs round-robin, so ids b, b+8, b+16, b+24
  // share an XCD: with one j-block per workgroup they take the four quarters
  // of the same row tile, back to back (each 4 KiB tile is then read by one
  // XCD in close succession instead of by four; a bijection on the units
  // when n_tr % 8 == 0, the identity otherwise).
  int unit = bid;
  if (NJG == 4 && (a.n_tr & 7) == 0) {
    const int b = bid, xcd = b & 7, slot = b >> 3;
    unit = (((slot >> 2) << 3) + xcd) * 4 + (slot & 3);
  }
  const int r = unit / NJG, jb0 = (unit - (unit / NJG) * NJG) * JBW;
  const int arow = lane & 15, akq = lane >> 4;
  const int rbase = r * a.n_tc;
  const int n_tc = a.n_tc;
  const int ldc = a.k + 16;
  int8_t* codes = dsm;                                                  // [n][ldc]
  float* sxl = reinterpret_cast<float*>(dsm + a.n * ldc);               // [n_tc] scales
  float* rcpl = sxl + n_tc;                                             // QUANT: [n_tc] 1 / scale
  uint32_t* amax = reinterpret_cast<uint32_t*>(rcpl + n_tc);            // QUANT: [n_tc] absmax bits

  // ---- 1. activation share (16-byte chunks; duplicates past the end rewrite
  //         the last chunk with identical data, so the phase is branch-free)
  const int cpr = QUANT ? (a.k >> 3) : (a.k >> 4);   // chunks per row
  const int total = a.n * cpr;
  u32x4 xr[CMAX];
  float sxr[2] = {0.0f, 0.0f};
  if (!COOP && (!HELP || idle)) {   // COOP: the codes are read once the producers are done
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
      const int i = min(tq + j * Tq, total - 1);
      const int row = i / cpr, ch = i - row * cpr;
      if constexpr (QUANT) xr[j] = *reinterpret_cast<const u32x4*>(a.xf + (int64_t)row * a.ldx + ch * 8);
      else xr[j] = *reinterpret_cast<const u32x4*>(a.xq + (int64_t)row * a.ldq + ch * 16);
    }
    if constexpr (!QUANT) {
#pragma unroll
      for (int h = 0; h < 2; ++h) sxr[h] = a.sx[min((int)threadIdx.x + h * T, n_tc - 1)];
    }
  }

  // Quantization by lanes (one thread per 8-element chunk of a row, Tq == cpr):
  // thread tq holds chunk tq of rows 0 .. n-1 (slot j = row j), so the 8
  // chunks of column tile tq / 8 sit in 8 aligned consecutive lanes.  Absmax
  // over the thread's rows, then over the 8 lanes by DPP; every lane of the
  // group derives the scale, 1 / scale and its codes from the same bits -- no
  // LDS atomics.  Same maximum (bit patterns of non-negative floats), same
  // scale, same codes as the general path of step 3.
  auto quantize_by_lanes = [&]() {
    uint32_t m = 0u;
#pragma unroll
    for (int j = 0; j < CMAX; ++j)
      if (j < a.n) m = max(m, __float_as_uint(max8<XT>(xr[j], 0.0f)));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));    // quad_perm 1,0,3,2
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));    // quad_perm 2,3,0,1
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));   // row_half_mirror
    const float s = act_scale_from_absmax<XT>(__uint_as_float(m));
    const CodeScale cq(s, 1.0f / s);
#pragma unroll
    for (int j = 0; j < CMAX; ++j)
      if (j < a.n) *reinterpret_cast<u32x2*>(codes + j * ldc + tq * 8) = codes8<XT>(xr[j], cq);
    if ((tq & 7) == 0) sxl[tq >> 3] = s;
  };
  // HELP: the helper waves' activation loads are their only loads, so they
  // quantize as soon as those arrive, before any row-pointer round trip.
  if constexpr (HELP) {
    if (idle) quantize_by_lanes();
  }

  // ---- 2. this wave's first batch of INT8 tiles, issued unconditionally:
  //         buffer loads bounded to the row's own tiles return 0 past its end
  //         instead of faulting, so no branch guards them and the waits below
  //         count exactly the loads issued before the weights.  Lane u < UMAX
  //         fetches the id and scale of batch tile u with a VECTOR load (read
  //         back with v_readlane): scalar loads would share lgkmcnt with the
  //         LDS traffic, so every lds_barrier() below would wait for them.
  const int lo8 = a.rp8[r], hi8 = a.rp8[r + 1];
  // The row's 16-bit range: HELP kernels load it with the INT8 range (their
  // tile waves go from the weight issue straight to the staging barrier);
  // the others after issuing their INT8 weights, which then do not wait for
  // it (measured 0.3-0.5 us faster per launch).
  const bool has16 = a.w16 != nullptr;
  const int32_t* rp16p = has16 ? a.rp16 : a.rp8;
  int lo16 = 0, n16 = 0;
  if constexpr (HELP) {
    lo16 = rp16p[r];
    n16 = has16 ? rp16p[r + 1] - lo16 : 0;
  }
  const int n8 = hi8 - lo8;
  const __amdgpu_buffer_rsrc_t wrs = row_rsrc(a.w8 + (int64_t)lo8 * 4096, n8 * 4096);
  const __amdgpu_buffer_rsrc_t irs = row_rsrc(a.ids8 + lo8, n8 * 4);
  const __amdgpu_buffer_rsrc_t srs = row_rsrc(a.sw8 + lo8, n8 * 4);
  const int woff = w8_lane_offset(a.layout, lane);
  int idl;
  float swl;
  v4i bw[UMAX][JBW];
  auto load_meta = [&](int q0) {   // q0: position relative to lo8
    const int ql = (q0 + min(lane, UMAX - 1) * W) * 4;
    idl = __builtin_amdgcn_raw_buffer_load_b32(irs, ql, 0, 0);
    swl = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, ql, 0, 0));
  };
  auto load_tile = [&](int q0, int u) {
#pragma unroll
    for (int j = 0; j < JBW; ++j)
      bw[u][j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                             wrs, (q0 + u * W) * 4096 + woff + (jb0 + j) * 1024, 0, 0));
  };
  auto load_batch = [&](int q0) {
    load_meta(q0);
#pragma unroll
    for (int u = 0; u < UMAX; ++u) load_tile(q0, u);
  };
  // The first batch: its first IA tiles now; each later one is issued right
  // after the MFMAs of the tile IA places before it.  The memory system
  // throttles the weight issue for microseconds (a wave could spend most of
  // the kernel issuing), so a wave now processes arrived tiles in between
  // instead of issuing its whole batch first.  Measured on MI355X (cold
  // weights, codes given, 4 tokens, per launch): Llama-3.2-3B Q/K/V 7.36 ->
  // 6.59 us, O 5.61 -> 5.10, Down 8.81 -> 8.16, Gate/Up (12-tile batches,
  // IA 6) 12.07 -> 11.43; Qwen2.5-7B keep10 Q/K/V 8.68 -> 8.37, O 7.98 ->
  // 7.84, Down 25.77 -> 25.45.  Whole-tile waves (6-tile batches of 4 KiB
  // tiles, 9-16 rows) lead by 2: stacked Gate/Up at 16 rows 13.90 -> 12.65 us,
  // at 9 rows 13.56 -> 12.44.  16-tile batches keep issuing at once (their
  // Gate/Up is slower with any shorter lead).
  constexpr int IA = UMAX == 8 ? 4 : (UMAX == 12 ? 6 : (UMAX == 6 ? 2 : UMAX));
  const int first_q = wave;
  if (!idle) {   // the COOP loader and HELP helper waves take no tiles
    load_meta(first_q);
#pragma unroll
    for (int u = 0; u < IA; ++u) load_tile(first_q, u);
  }

  // The first U16 16-bit tiles of this wave (their rotation continues after
  // the INT8 tiles), prefetched the same way.  Without 16-bit tiles the
  // ranges are empty and these loads touch no memory.
  constexpr int U16 = JBW == 1 ? 2 : 1;
  if constexpr (!HELP) {
    lo16 = rp16p[r];
    n16 = has16 ? rp16p[r + 1] - lo16 : 0;
  }
  const __amdgpu_buffer_rsrc_t w16rs =
      row_rsrc(has16 ? (const void*)(a.w16 + (int64_t)lo16 * 4096) : (const void*)a.rp8, n16 * 8192);
  const __amdgpu_buffer_rsrc_t i16rs = row_rsrc(has16 ? (const void*)(a.ids16 + lo16) : (const void*)a.rp8, n16 * 4);
  const int first16 = (wave - (n8 % W) + W) % W;
  // Lane i: the id of the wave's 16-bit tile i (position first16 + i W), for
  // its first 64 tiles -- the prefetched ones and the first window of the
  // loop below, which then needs no ids round trip of its own.
  int id16l = 0;
  if (!idle) id16l = __builtin_amdgcn_raw_buffer_load_b32(i16rs, (first16 + lane * W) * 4, 0, 0);
  v4i b16p[U16][JBW][2];
  auto load_w16_at = [&](v4i (&dst)[JBW][2], int q) {
#pragma unroll
    for (int j = 0; j < JBW; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        dst[j][h] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                                w16rs, q * 8192 + w16_lane_offset(a.layout, jb0 + j, h, lane), 0, 0));
  };
  if (!idle) {
#pragma unroll
    for (int u = 0; u < U16; ++u) load_w16_at(b16p[u], first16 + u * W);
  }

  // ---- 3. activation -> LDS
  bool staged = false;   // COOP fallback: the workgroup quantized into LDS itself
  if constexpr (COOP) {
    // the loader polls the producers' count; its verdict goes to every wave
    // through LDS (the barrier waits for LDS operations only: the weights
    // stay in flight)
    __shared__ int coop_ready;
    if (loader) {
      int ready = 0;
      for (int it = 0; it < a.coop_spin; ++it) {
        if (__hip_atomic_load(a.coop + (bid % kCoopGroups) * kCoopStride, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT) != 0) {
          ready = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (lane == 0) coop_ready = ready;
    }
    lds_barrier();
    if (coop_ready) {
      // the codes (and scales) the producers wrote through to the coherence
      // point, read past this XCD's L2 (sc1), CMAX 16-byte chunks per thread
      // the codes are the workspace's [n][k] (row stride k: 32-bit offsets)
      const __amdgpu_buffer_rsrc_t xqr = row_rsrc(a.xq, a.n * a.k);
      const __amdgpu_buffer_rsrc_t sxr_rs = row_rsrc(a.sx, n_tc * 4);
#pragma unroll
      for (int j = 0; j < CMAX; ++j) {
        const int i = min((int)threadIdx.x + j * T, total - 1);
        xr[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xqr, i * 16, 0, 16));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
        sxr[h] = __int_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(sxr_rs, min((int)threadIdx.x + h * T, n_tc - 1) * 4, 0, 16));
    } else {
      // the producers' count never arrived within the poll budget: quantize
      // here (the closed form of tq_act_quant: the codes are the same)
      uint32_t* amx = reinterpret_cast<uint32_t*>(sxl + n_tc);   // [n_tc]
      const int cq8 = a.k >> 3;                                  // 8-value chunks per row
      for (int c = threadIdx.x; c < n_tc; c += T) amx[c] = 0u;
      lds_barrier();
      for (int i = threadIdx.x; i < a.n * cq8; i += T) {   // 8 chunks of a (row, tile): 8 aligned lanes
        const int row = i / cq8, ch = i - row * cq8;
        const u32x4 x = *reinterpret_cast<const u32x4*>(a.xf + (int64_t)row * a.ldx + ch * 8);
        uint32_t m = __float_as_uint(max8<XT>(x, 0.0f));
        m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));    // quad_perm 1,0,3,2
        m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));    // quad_perm 2,3,0,1
        m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));   // row_half_mirror
        if ((threadIdx.x & 7) == 0) __hip_atomic_fetch_max(amx + (ch >> 3), m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      lds_barrier();
      for (int c = threadIdx.x; c < n_tc; c += T) sxl[c] = act_scale_from_absmax<XT>(__uint_as_float(amx[c]));
      lds_barrier();
      for (int i = threadIdx.x; i < a.n * cq8; i += T) {
        const int row = i / cq8, ch = i - row * cq8;
        const u32x4 x = *reinterpret_cast<const u32x4*>(a.xf + (int64_t)row * a.ldx + ch * 8);
        const float sc = sxl[ch >> 3];
        *reinterpret_cast<u32x2*>(codes + row * ldc + ch * 8) = codes8<XT>(x, CodeScale(sc, 1.0f / sc));
      }
      staged = true;
    }
  }
  // Quantization by lanes (quantize_by_lanes) where the workgroup has one
  // thread per 8-element chunk of a row (T == cpr): one barrier instead of
  // four.  The many-unit batches (UMAX 12 / 16) run 4 waves on more than 32 column
  // tiles, so T < cpr there: not compiled in (it would cost them registers).
  // Measured on MI355X (Llama-3.2-3B projections, cold weights): 0.4-1.8 us
  // faster per launch at 2-4 rows; at one row 0.2 us faster with 16 waves
  // (four barriers cost more there) but 0.1-0.3 us slower with 6, so one-row
  // launches of fewer than 16 waves keep the general path.
  constexpr bool kQuantByLanes = QUANT && UMAX <= 8;
  if (kQuantByLanes && (HELP || (T == cpr && (a.n >= 2 || T >= 1024)))) {
    if constexpr (!HELP) quantize_by_lanes();   // HELP: the helpers did it before step 2
  } else if constexpr (QUANT && !HELP) {
    for (int c = threadIdx.x; c < n_tc; c += T) amax[c] = 0u;
    lds_barrier();
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
      const int i = min((int)threadIdx.x + j * T, total - 1);
      const int c = (i - (i / cpr) * cpr) >> 3;   // 8 chunks of 8 values per column tile
      // The 8 chunks of one (row, column tile) sit in 8 aligned consecutive
      // lanes (cpr and T are multiples of 8; clamped tail chunks form whole
      // groups): reduce them with DPP, then one LDS atomic per group.
      // Absolute values are non-negative, so their bit patterns order like the floats.
      uint32_t m = __float_as_uint(max8<XT>(xr[j], 0.0f));
      m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
      m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
      m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));  // row_half_mirror
      if ((lane & 7) == 0) __hip_atomic_fetch_max(amax + c, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    lds_barrier();
    for (int c = threadIdx.x; c < n_tc; c += T) {
      const float s = act_scale_from_absmax<XT>(__uint_as_float(amax[c]));
      sxl[c] = s;
      rcpl[c] = 1.0f / s;
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
      const int i = min((int)threadIdx.x + j * T, total - 1);
      const int row = i / cpr, ch = i - row * cpr;
      const int c = ch >> 3;
      const CodeScale cq(sxl[c], rcpl[c]);
      *reinterpret_cast<u32x2*>(codes + row * ldc + ch * 8) = codes8<XT>(xr[j], cq);
    }
  } else if (!staged) {
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
      const int i = min((int)threadIdx.x + j * T, total - 1);
      const int row = i / cpr, ch = i - row * cpr;
      *reinterpret_cast<u32x4*>(codes + row * ldc + ch * 16) = xr[j];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if ((int)threadIdx.x + h * T < n_tc) sxl[threadIdx.x + h * T] = sxr[h];
  }
  lds_barrier();

  v4f acc[JBW][TB];
#pragma unroll
  for (int j = 0; j < JBW; ++j)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[j][tb] = v4f{0.f, 0.f, 0.f, 0.f};

  if (!idle) {   // the COOP loader and HELP helpers have no tiles: no partial of theirs is summed
  // ---- 4. INT8 tiles: A operand from LDS
  auto int8_tile = [&](int u, int q0) {
    const int c = col_of(__builtin_amdgcn_readlane(idl, u), rbase, n_tc);
    const float sc = sxl[c] * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(swl), u));
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int row = tb * 16 + arow;   // rows >= n: zero operand (clamped read stays in the buffer)
      const v4i xv = *reinterpret_cast<const v4i*>(codes + min(row, a.n - 1) * ldc + c * 64 + akq * 16);
      const v4i ax = row < a.n ? xv : v4i{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < JBW; ++j) {
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, bw[u][j], v4i{0, 0, 0, 0}, 0, 0, 0);
        dump_i32<DUMP>(a, lo8 + q0 + u * W, tb * 16 + 4 * akq, (jb0 + j) * 16 + arow, d);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[j][tb][v] = fmaf((float)d[v], sc, acc[j][tb][v]);
      }
    }
  };
  if (first_q < n8) {   // the first batch, its later tiles issued as the earlier ones are used
    const int nu = min(UMAX, (n8 - first_q + W - 1) / W);   // valid tiles (wave-uniform)
#pragma unroll
    for (int u = 0; u < UMAX; ++u) {
      if (u < nu) int8_tile(u, first_q);
      if (u + IA < UMAX) load_tile(first_q, u + IA);   // past the row's range: reads nothing
    }
  }
  for (int q0 = first_q + UMAX * W; q0 < n8; q0 += UMAX * W) {
    load_batch(q0);
    const int nu = min(UMAX, (n8 - q0 + W - 1) / W);
#pragma unroll
    for (int u = 0; u < UMAX; ++u)
      if (u < nu) int8_tile(u, q0);
  }

  // ---- 16-bit tiles (positions first16 + i*W, ascending); A from global
  auto tile16 = [&](const v4i (&b16)[JBW][2], int id) {
    const int c = col_of(id, rbase, n_tc);
    v4i ax[TB][2];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int h = 0; h < 2; ++h) ax[tb][h] = load_xf<1>(a, tb * 16 + arow, c * 64 + h * 32 + akq * 8);
#pragma unroll
    for (int j = 0; j < JBW; ++j)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        acc[j][tb] = mfma16<XT>(ax[tb][0], b16[j][0], acc[j][tb]);
        acc[j][tb] = mfma16<XT>(ax[tb][1], b16[j][1], acc[j][tb]);
      }
  };
#pragma unroll
  for (int u = 0; u < U16; ++u)
    if (first16 + u * W < n16) tile16(b16p[u], __builtin_amdgcn_readlane(id16l, u));
  // The wave's remaining 16-bit tiles (tile indices t >= U16, positions
  // first16 + t W, ascending: the same order as one at a time), in windows of
  // tile indices [t0, next multiple of 64): the first window's ids are lanes
  // U16.. of id16l, each later window's come with one vector load.  Each
  // batch of U16B tiles then issues its weights and activation operands
  // together -- one round trip per batch instead of two per tile (rows that
  // are mostly 16-bit, as clustered masks give, have dozens).  Rows past n
  // read row n - 1: their products land in output rows that are never stored.
  constexpr int U16B = JBW == 1 ? 4 : 2;
  for (int t0 = U16; first16 + t0 * W < n16; t0 = (t0 & ~63) + 64) {
    const int q0 = first16 + t0 * W;
    const int lane0 = t0 & 63;   // lane of the window's first id
    const int idv = t0 < 64 ? id16l : __builtin_amdgcn_raw_buffer_load_b32(i16rs, (q0 + lane * W) * 4, 0, 0);
    const int cnt = min(64 - lane0, (n16 - q0 + W - 1) / W);
    for (int i0 = 0; i0 < cnt; i0 += U16B) {
      v4i bb[U16B][JBW][2], ab[U16B][TB][2];
#pragma unroll
      for (int u = 0; u < U16B; ++u) {
        const int i = min(i0 + u, cnt - 1);   // past the end: the last tile again, not used
        load_w16_at(bb[u], q0 + i * W);
        const int c = col_of(__builtin_amdgcn_readlane(idv, lane0 + i), rbase, n_tc);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            ab[u][tb][h] = *reinterpret_cast<const v4i*>(a.xf + (int64_t)min(tb * 16 + arow, a.n - 1) * a.ldx +
                                                          c * 64 + h * 32 + akq * 8);
      }
#pragma unroll
      for (int u = 0; u < U16B; ++u)
        if (i0 + u < cnt) {
#pragma unroll
          for (int j = 0; j < JBW; ++j)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
              acc[j][tb] = mfma16<XT>(ab[u][tb][0], bb[u][j][0], acc[j][tb]);
              acc[j][tb] = mfma16<XT>(ab[u][tb][1], bb[u][j][1], acc[j][tb]);
            }
        }
    }
  }

  }   // !idle

  // ---- waves -> LDS (reusing the code area) -> sum in wave order -> store
  constexpr int E = JBW * TB * 4 * 64;   // (j, tb, v, lane)
  float* red = reinterpret_cast<float*>(dsm);
  lds_barrier();   // every wave is done reading codes and scales
  if (!idle) {
#pragma unroll
    for (int j = 0; j < JBW; ++j)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[wave * E + ((j * TB + tb) * 4 + v) * 64 + lane] = acc[j][tb][v];
  }
  lds_barrier();
  for (int e = threadIdx.x; e < E; e += T) {
    const int ln = e & 63, t = e >> 6, v = t & 3, tb = (t >> 2) % TB, j = (t >> 2) / TB;
    const int row = tb * 16 + 4 * (ln >> 4) + v;
    const int col = r * 64 + (jb0 + j) * 16 + (ln & 15);
    if (row >= a.n || col >= a.m) continue;
    float sum = red[e];
    for (int w = 1; w < W; ++w) sum += red[w * E + e];
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
  if constexpr (COOP) {
    if (threadIdx.x == 0) coop_pass(a, bid % kCoopGroups);
  }
}

// ---- prefill kernel (N > 64 tokens) ----------------------------------------
//
// Compute-bound schedule.  Workgroup (row tile r, token block of BN = 256)
// has 4 waves; wave w owns tokens w*64 .. w*64+63 (4 token blocks) x the 64
// features of r (4 j-blocks): 16 v_mfma_i32_16x16x64_i8 per INT8 tile, then
// 64 fp32 FMAs per lane by sx[c]*sw[t] (the epilogue the reference applies
// per K tile, gemm_rows_splitk_64x64.py:134-137).  Each K step's 4 KiB weight
// tile and 16 KiB activation slice (256 tokens x 64 codes) are staged in LDS,
// double-buffered: the 256 threads load step k+1 into registers while the
// MFMAs read step k, then write it into the other buffer already permuted to
// MFMA operand order ([token block][lane][16 bytes]), so every ds_read_b128
// is conflict-free.  The (rare) 16-bit tiles follow, read straight from
// global memory, accumulating into the same fp32 accumulators.
// Tile order per row: INT8 tiles ascending, then 16-bit tiles ascending --
// the reference's order (split_k = 1).

constexpr int kPfTokens = 256;                  // tokens per workgroup
constexpr int kPfThreads = 256;                 // 4 waves
constexpr int kPfXBytes = kPfTokens * 64;       // activation slice per K step

template <class XT, bool DUMP = false>
__global__ void __launch_bounds__(kPfThreads)
gemm_prefill_kernel(GemmArgs a) {
  __shared__ __align__(16) int8_t wbuf[2][4096];
  __shared__ __align__(16) int8_t xbuf[2][kPfXBytes];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = blockIdx.x;
  const int n0 = blockIdx.y * kPfTokens;
  const int rbase = r * a.n_tc;
  const int arow = lane & 15, akq = lane >> 4;

  v4f acc[4][4];   // [token block][j-block]
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) acc[tb][jb] = v4f{0.f, 0.f, 0.f, 0.f};

  const int lo8 = a.rp8[r], hi8 = a.rp8[r + 1];

  // ---- staging: thread t moves one 16-byte weight chunk and four activation chunks
  // weight chunk t of the tile, LDS chunk in MFMA order
  const int wj = t >> 2, wkq = t & 3;
  const int w_src = (a.layout == TQ_LAYOUT_MFMA) ? t * 16 : wj * 64 + wkq * 16;
  const int w_dst = (a.layout == TQ_LAYOUT_MFMA) ? t * 16 : ((wj >> 4) * 64 + wkq * 16 + (wj & 15)) * 16;
  // activation chunk ids t + i*256 -> (token, k chunk); LDS [token/16][kq*16 + token%16][16 B]
  int x_tok[4], x_kq[4], x_dst[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = t + i * kPfThreads;
    x_tok[i] = id >> 2;
    x_kq[i] = id & 3;
    x_dst[i] = ((x_tok[i] >> 4) * 64 + x_kq[i] * 16 + (x_tok[i] & 15)) * 16;
  }
  v4i wreg, xreg[4];
  auto fetch = [&](int p) {
    const int c = col_of(a.ids8[p], rbase, a.n_tc);
    wreg = *reinterpret_cast<const v4i*>(a.w8 + (int64_t)p * 4096 + w_src);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xreg[i] = load_xq<-1>(a, n0 + x_tok[i], c * 64 + x_kq[i] * 16);
  };
  auto stash = [&](int buf) {
    *reinterpret_cast<v4i*>(&wbuf[buf][w_dst]) = wreg;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(&xbuf[buf][x_dst[i]]) = xreg[i];
  };

  if (lo8 < hi8) {
    fetch(lo8);
    stash(0);
  }
  __syncthreads();
  for (int p = lo8; p < hi8; ++p) {
    const int buf = (p - lo8) & 1;
    const bool more = p + 1 < hi8;
    if (more) fetch(p + 1);
    const int c = col_of(a.ids8[p], rbase, a.n_tc);
    const float sc = a.sx[c] * a.sw8[p];
    v4i bw[4], ax[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) bw[jb] = *reinterpret_cast<const v4i*>(&wbuf[buf][jb * 1024 + lane * 16]);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
      ax[tb] = *reinterpret_cast<const v4i*>(&xbuf[buf][(wave * 4 + tb) * 1024 + lane * 16]);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[tb], bw[jb], v4i{0, 0, 0, 0}, 0, 0, 0);
        dump_i32<DUMP>(a, p, n0 + wave * 64 + tb * 16 + 4 * akq, jb * 16 + arow, d);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[tb][jb][v] = fmaf((float)d[v], sc, acc[tb][jb][v]);
      }
    if (more) stash(buf ^ 1);
    __syncthreads();
  }

  // ---- 16-bit tiles (straight from global; rare by construction)
  if (a.w16 != nullptr) {
    const int lo16 = a.rp16[r], hi16 = a.rp16[r + 1];
    for (int q = lo16; q < hi16; ++q) {
      const int c = col_of(a.ids16[q], rbase, a.n_tc);
      v4i bw[4][2];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        bw[jb][0] = load_w16(a, q, jb, 0, lane);
        bw[jb][1] = load_w16(a, q, jb, 1, lane);
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int row = n0 + wave * 64 + tb * 16 + arow;
        const v4i a0 = load_xf<-1>(a, row, c * 64 + akq * 8);
        const v4i a1 = load_xf<-1>(a, row, c * 64 + 32 + akq * 8);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          acc[tb][jb] = mfma16<XT>(a0, bw[jb][0], acc[tb][jb]);
          acc[tb][jb] = mfma16<XT>(a1, bw[jb][1], acc[tb][jb]);
        }
      }
    }
  }

  // ---- epilogue: every wave owns distinct outputs, no reduction
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = n0 + wave * 64 + tb * 16 + 4 * akq + v;
        const int col = r * 64 + jb * 16 + arow;
        if (row < a.n && col < a.m) {
          const float sum = acc[tb][jb][v];
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

// ---- prefill kernel, asynchronous LDS pipeline ------------------------------
//
// Same workgroup decomposition and arithmetic as gemm_prefill_kernel, with
// the K-step operands moved by global_load_lds_dwordx4 (gfx950: each lane's
// 16 bytes land at LDS base + lane*16, no VGPRs) through a P-stage ring of
// 20 KiB stages.  Per stage each wave issues five DMA loads: its 1 KiB j-block
// of the weight tile and 4 KiB (four 16-token blocks) of the activation
// slice, with per-lane source addresses chosen so the data lands in MFMA
// operand order.  Loop step p: wait for stage p (the P-2 younger stages stay
// in flight: vmcnt = 5*(P-2)), one barrier, issue tile p+P-1 into the stage
// consumed at step p-1, then 16 MFMA + the fp32 epilogue on stage p.  Tail
// steps re-issue the last tile so the vmcnt arithmetic stays constant.  Rows
// past n read a clamped valid row: they only feed output rows >= n, which are
// never stored.  Needs 16-byte aligned activation rows and k == 64 * n_tc.

constexpr int kPfStage = 4096 + kPfXBytes;
constexpr int kPfStages = 3;
constexpr int kPfMeta = 512;

// LDS byte address of a __shared__ object
__device__ inline uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

__device__ inline int lds_read_i32(uint32_t addr) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(addr) : "memory");
  return v;
}

template <int V>
__device__ inline void wait_vmcnt() {
  // s_waitcnt with vmcnt = V (gfx9 split field) and expcnt / lgkmcnt at their maxima
  __builtin_amdgcn_s_waitcnt((V & 0xF) | ((V >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <class XT, int P, bool DUMP = false>
__global__ void __launch_bounds__(kPfThreads)
gemm_prefill_async_kernel(GemmArgs a) {
  __shared__ __align__(16) int8_t smem[P * kPfStage];
  __shared__ int meta_x[kPfMeta];
  __shared__ float meta_s[kPfMeta];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = blockIdx.x;
  const int n0 = blockIdx.y * kPfTokens;
  const int rbase = r * a.n_tc;
  const int arow = lane & 15, akq = lane >> 4;

  v4f acc[4][4];   // [token block][j-block]
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) acc[tb][jb] = v4f{0.f, 0.f, 0.f, 0.f};

  const int lo8 = a.rp8[r], hi8 = a.rp8[r + 1];
  // this lane's weight chunk offset inside a tile: j-block `wave`, lane slot `lane`
  const int w_off = (a.layout == TQ_LAYOUT_MFMA) ? wave * 1024 + lane * 16
                                                 : (wave * 16 + (lane & 15)) * 64 + (lane >> 4) * 16;
  // this lane's activation rows for token blocks wave*4 + i
  int64_t x_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x_row[i] = (int64_t)min(n0 + (wave * 4 + i) * 16 + arow, a.n - 1) * a.ldq + akq * 16;

  auto issue = [&](int p, int xoff, int stage) {
    int8_t* st = smem + stage * kPfStage;
    __builtin_amdgcn_global_load_lds(a.w8 + (int64_t)p * 4096 + w_off, st + wave * 1024, 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(a.xq + x_row[i] + xoff, st + 4096 + (wave * 4 + i) * 1024, 16, 0, 0);
  };

  // LDS reads inside the pipeline are inline asm: the compiler cannot tell
  // which LDS bytes an in-flight DMA load writes, so it would put a full
  // vmcnt(0) before every ordinary LDS read and drain the pipeline.  The
  // explicit vmcnt wait + barrier at the top of each step orders them instead.
  const uint32_t smem_lds = lds_addr(smem);
  const uint32_t mx_lds = lds_addr(meta_x), ms_lds = lds_addr(meta_s);
  const uint32_t w_rd = smem_lds + lane * 16;
  const uint32_t x_rd = smem_lds + 4096 + wave * 4096 + lane * 16;

  // Tile metadata (activation byte offset, combined scale) is staged through
  // LDS per chunk of kPfMeta tiles: loading it from global inside the loop
  // would share the in-order vmcnt with the DMA loads and drain the pipeline.
  for (int base = lo8; base < hi8; base += kPfMeta) {
    const int end = min(base + kPfMeta, hi8);
    __syncthreads();   // the previous chunk's readers are done with meta and stages
    for (int t = base + (int)threadIdx.x; t < end; t += kPfThreads) {
      const int c = col_of(a.ids8[t], rbase, a.n_tc);
      meta_x[t - base] = c * 64;
      meta_s[t - base] = a.sx[c] * a.sw8[t];
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < P - 1; ++s) {
      const int p = min(base + s, end - 1);
      issue(p, __builtin_amdgcn_readfirstlane(lds_read_i32(mx_lds + 4 * (p - base))), s);
    }
    // Software pipeline across K steps: the 16 MFMAs of step p are issued
    // before the fp32 epilogue (cvt + FMA by its scale) of step p - 1, so the
    // VALU epilogue of one step runs while the matrix cores work on the next.
    // Two result sets alternate (the loop is unrolled by two so they stay in
    // registers).
    auto step = [&](int p, v4i (&dnew)[4][4], float& snew) {
      const int stage = (p - base) % P;
      if constexpr (DUMP) wait_vmcnt<0>();   // stores count in vmcnt too
      else wait_vmcnt<5 * (P - 2)>();
      // s_barrier without __syncthreads' release fence: that fence waits for
      // every outstanding load (vmcnt(0)), in-flight DMA included.  The DMA
      // writes are ordered by the vmcnt wait above; the asm LDS reads below
      // complete (lgkmcnt(0)) before their step ends.
      asm volatile("s_barrier" ::: "memory");
      const int pn = min(p + P - 1, end - 1);
      int xo;
      float sc;
      asm volatile(
          "ds_read_b32 %0, %2\n\t"
          "ds_read_b32 %1, %3\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(xo), "=&v"(sc)
          : "v"(mx_lds + 4 * (pn - base)), "v"(ms_lds + 4 * (p - base))
          : "memory");
      issue(pn, __builtin_amdgcn_readfirstlane(xo), (stage + P - 1) % P);
      v4i bw[4], ax[4];
      const uint32_t so = stage * kPfStage;
      asm volatile(
          "ds_read_b128 %0, %8\n\t"
          "ds_read_b128 %1, %8 offset:1024\n\t"
          "ds_read_b128 %2, %8 offset:2048\n\t"
          "ds_read_b128 %3, %8 offset:3072\n\t"
          "ds_read_b128 %4, %9\n\t"
          "ds_read_b128 %5, %9 offset:1024\n\t"
          "ds_read_b128 %6, %9 offset:2048\n\t"
          "ds_read_b128 %7, %9 offset:3072\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(bw[0]), "=&v"(bw[1]), "=&v"(bw[2]), "=&v"(bw[3]),
            "=&v"(ax[0]), "=&v"(ax[1]), "=&v"(ax[2]), "=&v"(ax[3])
          : "v"(w_rd + so), "v"(x_rd + so)
          : "memory");
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
          dnew[tb][jb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[tb], bw[jb], v4i{0, 0, 0, 0}, 0, 0, 0);
      if constexpr (DUMP) {
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) dump_i32<DUMP>(a, p, n0 + wave * 64 + tb * 16 + 4 * akq, jb * 16 + arow, dnew[tb][jb]);
      }
      snew = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sc)));
      // gfx9 counts stores in vmcnt too: drain the dump's stores so the next
      // step's vmcnt wait counts ring loads only
      if constexpr (DUMP) wait_vmcnt<0>();
    };
    auto epilogue = [&](const v4i (&d)[4][4], float sc) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[tb][jb][v] = fmaf((float)d[tb][jb][v], sc, acc[tb][jb][v]);
    };
    v4i d0[4][4], d1[4][4];
    float s0 = 0.0f, s1 = 0.0f;
    int p = base;
    if (p < end) step(p++, d0, s0);
    while (p + 1 < end) {
      step(p++, d1, s1);
      epilogue(d0, s0);
      step(p++, d0, s0);
      epilogue(d1, s1);
    }
    if (p < end) {
      step(p++, d1, s1);
      epilogue(d0, s0);
      epilogue(d1, s1);
    } else if (end > base) {
      epilogue(d0, s0);
    }
    wait_vmcnt<0>();   // drain the re-issued tail loads before the stages are reused
  }

  // ---- 16-bit tiles (straight from global; rare by construction)
  if (a.w16 != nullptr) {
    const int lo16 = a.rp16[r], hi16 = a.rp16[r + 1];
    for (int q = lo16; q < hi16; ++q) {
      const int c = col_of(a.ids16[q], rbase, a.n_tc);
      v4i bw[4][2];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        bw[jb][0] = load_w16(a, q, jb, 0, lane);
        bw[jb][1] = load_w16(a, q, jb, 1, lane);
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int row = n0 + wave * 64 + tb * 16 + arow;
        const v4i a0 = load_xf<1>(a, row, c * 64 + akq * 8);
        const v4i a1 = load_xf<1>(a, row, c * 64 + 32 + akq * 8);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          acc[tb][jb] = mfma16<XT>(a0, bw[jb][0], acc[tb][jb]);
          acc[tb][jb] = mfma16<XT>(a1, bw[jb][1], acc[tb][jb]);
        }
      }
    }
  }

#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = n0 + wave * 64 + tb * 16 + 4 * akq + v;
        const int col = r * 64 + jb * 16 + arow;
        if (row < a.n && col < a.m) {
          const float sum = acc[tb][jb][v];
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

// ---- prefill kernel v3: two row tiles per workgroup, 4-stage DMA ring ------
//
// Workgroup (row-tile pair r0 = 2 bx, r0 + 1; token block of 256), 8 waves:
// wave w computes tokens (w & 3) * 64 .. + 64 of row tile r0 + (w >> 2), i.e.
// 16 v_mfma_i32_16x16x64_i8 per K step, as gemm_prefill_async_kernel.  The
// 16 KiB activation slice of a K step is shared by both row tiles (half the
// activation traffic per MFMA), and four stages of 24 KiB (slice + two weight
// tiles) keep three K steps of global -> LDS DMA in flight.  The K loop runs
// over every column tile c; an LDS map gives each row's INT8 position at c
// (or -1 where the tile is 16-bit: that row's MFMAs skip the step), so the
// INT8 tiles of each row are still accumulated in ascending column order,
// then its 16-bit tiles -- the reference's order.  Eight waves per workgroup
// (two per SIMD) let one wave's fp32 epilogue overlap another's MFMAs.  LDS
// reads inside the pipeline are inline asm for the reason given at
// gemm_prefill_async_kernel.
constexpr int kP3Threads = 512;
constexpr int kP3Stage = kPfXBytes + 2 * 4096;
constexpr int kP3Stages = 4;
constexpr int kP3MaxCols = 512;   // k <= 32768

template <class XT, bool DUMP = false>
__global__ void __launch_bounds__(kP3Threads)
gemm_prefill_v3_kernel(GemmArgs a) {
  __shared__ __align__(16) int8_t smem[kP3Stages * kP3Stage];
  __shared__ int pos8[2][kP3MaxCols];
  __shared__ float scl[2][kP3MaxCols];
  constexpr int P = kP3Stages;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int tq = wave & 3, rt = wave >> 2;
  const int r0 = blockIdx.x * 2, r = r0 + rt;
  const int n0 = blockIdx.y * kPfTokens;
  const int arow = lane & 15, akq = lane >> 4;
  const int n_tc = a.n_tc;
  const int t8 = a.rp8[a.n_tr];

  // ---- position / scale map of the two row tiles
  for (int i = t; i < 2 * kP3MaxCols; i += kP3Threads) (&pos8[0][0])[i] = -1;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int rr = r0 + j;
    if (rr >= a.n_tr) continue;
    const int lo = a.rp8[rr], hi = a.rp8[rr + 1];
    for (int p = lo + t; p < hi; p += kP3Threads) {
      const int c = col_of(a.ids8[p], rr * n_tc, n_tc);
      pos8[j][c] = p;
      scl[j][c] = a.sx[c] * a.sw8[p];
    }
  }
  __syncthreads();

  v4f acc[4][4];   // [token block][j-block]
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) acc[tb][jb] = v4f{0.f, 0.f, 0.f, 0.f};

  if (t8 > 0) {
    // DMA lanes: wave w moves token blocks 2w, 2w + 1 of the slice and 1 KiB
    // (j-block w & 3) of the weight tile of row r0 + (w >> 2)
    int64_t xrow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      xrow[i] = (int64_t)min(n0 + (2 * wave + i) * 16 + arow, a.n - 1) * a.ldq + akq * 16;
    const int wj = wave >> 2, wjb = wave & 3;
    const int w_off = (a.layout == TQ_LAYOUT_MFMA) ? wjb * 1024 + lane * 16
                                                   : (wjb * 16 + (lane & 15)) * 64 + (lane >> 4) * 16;
    const uint32_t smem_lds = lds_addr(smem);
    const uint32_t pos_lds = lds_addr(&pos8[0][0]), scl_lds = lds_addr(&scl[0][0]);
    auto meta_pos = [&](int j, int c) {   // INT8 position of tile (r0 + j, c), -1 if 16-bit
      int v;
      asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v)
                   : "v"(pos_lds + 4 * (j * kP3MaxCols + c)) : "memory");
      return __builtin_amdgcn_readfirstlane(v);
    };
    auto issue = [&](int c, int st, int pw) {   // pw: this wave's weight position (>= 0)
      int8_t* sp = smem + st * kP3Stage;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        __builtin_amdgcn_global_load_lds(a.xq + xrow[i] + c * 64, sp + (2 * wave + i) * 1024, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(a.w8 + (int64_t)pw * 4096 + w_off, sp + kPfXBytes + wj * 4096 + wjb * 1024,
                                       16, 0, 0);
    };
    // a 16-bit position has no INT8 tile: the weight DMA reads a valid tile instead (never used)
    auto pos_or_any = [&](int p) { return p >= 0 ? p : 0; };
#pragma unroll
    for (int st = 0; st < P - 1; ++st) {
      const int c = min(st, n_tc - 1);
      issue(c, st, pos_or_any(meta_pos(wj, c)));
    }
    const uint32_t w_rd = smem_lds + kPfXBytes + rt * 4096 + lane * 16;
    const uint32_t x_rd = smem_lds + tq * 4096 + lane * 16;

    for (int c = 0; c < n_tc; ++c) {
      const int stage = c % P;
      if constexpr (DUMP) wait_vmcnt<0>();   // stores count in vmcnt too
      else wait_vmcnt<3 * (P - 2)>();
      asm volatile("s_barrier" ::: "memory");
      const int cn = min(c + P - 1, n_tc - 1);
      int pn, pc;
      float sc;
      asm volatile(
          "ds_read_b32 %0, %3\n\t"
          "ds_read_b32 %1, %4\n\t"
          "ds_read_b32 %2, %5\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(pn), "=&v"(pc), "=&v"(sc)
          : "v"(pos_lds + 4 * (wj * kP3MaxCols + cn)), "v"(pos_lds + 4 * (rt * kP3MaxCols + c)),
            "v"(scl_lds + 4 * (rt * kP3MaxCols + c))
          : "memory");
      issue(cn, (stage + P - 1) % P, pos_or_any(__builtin_amdgcn_readfirstlane(pn)));
      const bool has = __builtin_amdgcn_readfirstlane(pc) >= 0 && r < a.n_tr;
      if (!has) continue;   // 16-bit tile (or no row): this wave skips the step
      const float scu = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sc)));
      v4i bw[4], ax[4];
      const uint32_t so = stage * kP3Stage;
      asm volatile(
          "ds_read_b128 %0, %8\n\t"
          "ds_read_b128 %1, %8 offset:1024\n\t"
          "ds_read_b128 %2, %8 offset:2048\n\t"
          "ds_read_b128 %3, %8 offset:3072\n\t"
          "ds_read_b128 %4, %9\n\t"
          "ds_read_b128 %5, %9 offset:1024\n\t"
          "ds_read_b128 %6, %9 offset:2048\n\t"
          "ds_read_b128 %7, %9 offset:3072\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(bw[0]), "=&v"(bw[1]), "=&v"(bw[2]), "=&v"(bw[3]),
            "=&v"(ax[0]), "=&v"(ax[1]), "=&v"(ax[2]), "=&v"(ax[3])
          : "v"(w_rd + so), "v"(x_rd + so)
          : "memory");
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[tb], bw[jb], v4i{0, 0, 0, 0}, 0, 0, 0);
          dump_i32<DUMP>(a, __builtin_amdgcn_readfirstlane(pc), n0 + tq * 64 + tb * 16 + 4 * akq, jb * 16 + arow, d);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[tb][jb][v] = fmaf((float)d[v], scu, acc[tb][jb][v]);
        }
      if constexpr (DUMP) wait_vmcnt<0>();   // the dump's stores count in vmcnt: keep the ring's count exact
    }
    wait_vmcnt<0>();   // drain the re-issued tail loads
  }

  if (r >= a.n_tr) return;   // odd row-tile count: the second half of the last pair is empty
  // ---- 16-bit tiles of row r (straight from global; rare by construction)
  if (a.w16 != nullptr) {
    const int lo16 = a.rp16[r], hi16 = a.rp16[r + 1];
    for (int q = lo16; q < hi16; ++q) {
      const int c = col_of(a.ids16[q], r * n_tc, n_tc);
      v4i bw[4][2];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        bw[jb][0] = load_w16(a, q, jb, 0, lane);
        bw[jb][1] = load_w16(a, q, jb, 1, lane);
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int row = n0 + tq * 64 + tb * 16 + arow;
        const v4i a0 = load_xf<1>(a, row, c * 64 + akq * 8);
        const v4i a1 = load_xf<1>(a, row, c * 64 + 32 + akq * 8);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          acc[tb][jb] = mfma16<XT>(a0, bw[jb][0], acc[tb][jb]);
          acc[tb][jb] = mfma16<XT>(a1, bw[jb][1], acc[tb][jb]);
        }
      }
    }
  }

#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = n0 + tq * 64 + tb * 16 + 4 * akq + v;
        const int col = r * 64 + jb * 16 + arow;
        if (row < a.n && col < a.m) {
          const float sum = acc[tb][jb][v];
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

// ---- prefill kernel v5: 64 x 128 wave tiles, 16-bit tiles in the ring -------
//
// Two row tiles x 256 tokens per workgroup, 4 waves that each own 64 tokens x
// both row tiles (32 MFMAs per K step for 12 KiB of LDS operand reads).  The
// K loop is one list of steps fed through a 3-stage DMA ring
// (global_load_lds, 24 KiB per stage, two workgroups per CU):
//   steps 0 .. n_tc-1      INT8 column c: 256 x 64 codes + both rows' 4 KiB
//                          weight tiles (a row whose tile at c is 16-bit
//                          skips its MFMAs)
//   then 2 per 16-bit tile half h of the tile: 256 x 32 activations (16 KiB)
//                          + the tile's 64 x 32 half (4 KiB), 16 bf16/fp16
//                          MFMAs into the row's accumulators
// so the accumulation order per output is the reference's: INT8 tiles by
// column, then 16-bit tiles by position, K halves in order.  Columns where no
// row of the unit has an INT8 tile take no step.  The epilogue stages the
// rounded outputs through LDS and writes 16-byte row chunks.
// Work units: a 1-D grid over (unit, token block), the unit index fastest (on
// MI355X 11% faster than the same pairs as a 2-D grid).  Units are row pairs,
// or, with a plan (a.units), the plan's pairs and single row tiles, the units
// carrying many 16-bit tiles first so that they do not finish last.  A unit's
// per-output arithmetic is the same either way.
constexpr int kP5Threads = 256;
template <class T> struct TypeTag { using type = T; };
constexpr int kP5Stages = 3;
constexpr int kP5MaxCols = 304;   // k <= 19456 (Qwen2.5-7B down: 296 column tiles); LDS 81 KB
constexpr int kP5OutRow = 272;    // LDS bytes per staged output row (256 + 16: no bank conflicts)
static_assert(4 * 64 * kP5OutRow <= kP5Stages * kP3Stage, "output staging fits the ring");

// DUMP instantiations run one wave per SIMD: the dump's addresses then fit in
// registers (at two waves per SIMD they spilled to scratch).
template <class XT, bool DUMP = false>
__global__ void __launch_bounds__(kP5Threads) __attribute__((amdgpu_waves_per_eu(DUMP ? 1 : 2, DUMP ? 1 : 2)))
gemm_prefill_v5_kernel(GemmArgs a) {
  __shared__ __align__(16) int8_t smem[kP5Stages * kP3Stage];
  __shared__ int pos8[2][kP5MaxCols];
  __shared__ float scl[2][kP5MaxCols];
  __shared__ int list16[2 * kP5MaxCols];   // (q << 10) | (row << 9) | column
  __shared__ int wcount[8];
  constexpr int P = kP5Stages;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  int r0, n0;
  bool has1;
  const int ntb = (a.n + kPfTokens - 1) / kPfTokens;
  if (a.units == nullptr) {   // row pairs, the pair index fastest
    const int n_pairs = (a.n_tr + 1) / 2;
    r0 = (blockIdx.x % n_pairs) * 2;
    n0 = (blockIdx.x / n_pairs) * kPfTokens;
    has1 = r0 + 1 < a.n_tr;   // odd row-tile count: the last pair has one row
  } else {
    int b = blockIdx.x, u, tbk;
    if (b < a.n_first * ntb) {
      u = b % a.n_first;
      tbk = b / a.n_first;
    } else {
      b -= a.n_first * ntb;
      const int rest = a.n_units - a.n_first;
      u = a.n_first + b % rest;
      tbk = b / rest;
    }
    const int w = a.units[u];
    r0 = w & (kUnitSingle - 1);
    n0 = tbk * kPfTokens;
    has1 = !(w & kUnitSingle) && r0 + 1 < a.n_tr;
    if (r0 >= a.n_tr) return;   // not a plan for this matrix
  }
  const int arow = lane & 15, akq = lane >> 4;
  const int n_tc = a.n_tc;
  int n8s = 0;   // INT8 steps: the columns where a row of the unit has an INT8 tile
  int n16 = 0, n16_0 = 0;
  if (a.w16 != nullptr) {
    const int lo0 = a.rp16[r0], c0 = a.rp16[r0 + 1] - lo0;
    n16_0 = c0;
    const int lo1 = has1 ? a.rp16[r0 + 1] : 0, c1 = has1 ? a.rp16[r0 + 2] - lo1 : 0;
    n16 = c0 + c1;
    for (int i = t; i < n16; i += kP5Threads) {
      const int j = i >= c0;
      const int q = j ? lo1 + (i - c0) : lo0 + i;
      list16[i] = (q << 10) | (j << 9) | col_of(a.ids16[q], (r0 + j) * n_tc, n_tc);
    }
  }
  for (int i = t; i < 2 * kP5MaxCols; i += kP5Threads) (&pos8[0][0])[i] = -1;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int rr = r0 + j;
    if (j == 1 && !has1) continue;
    const int lo = a.rp8[rr], hi = a.rp8[rr + 1];
    for (int p = lo + t; p < hi; p += kP5Threads) {
      const int c = col_of(a.ids8[p], rr * n_tc, n_tc);
      pos8[j][c] = p;
      scl[j][c] = a.sx[c] * a.sw8[p];
    }
  }
  __syncthreads();
  // Compact the columns with an INT8 tile, in column order, in place: entry i
  // becomes (position << 9) | column, or (-512 | column) for a row whose tile
  // there is 16-bit (position < 2^22, column < 512).  All reads precede the
  // count barrier; the writes follow it.
  {
    static_assert(kP5MaxCols <= 2 * kP5Threads && kP5MaxCols < 512, "two columns per thread");
    int pv[2][2];
    float sv[2][2];
    bool keep[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = t + h * kP5Threads;
      keep[h] = false;
      if (c < n_tc) {
        pv[h][0] = pos8[0][c]; pv[h][1] = pos8[1][c];
        sv[h][0] = scl[0][c]; sv[h][1] = scl[1][c];
        keep[h] = pv[h][0] >= 0 || pv[h][1] >= 0;
      }
    }
    const uint64_t b0 = __ballot(keep[0]), b1 = __ballot(keep[1]);
    if (lane == 0) {
      wcount[wave] = __popcll(b0);
      wcount[4 + wave] = __popcll(b1);
    }
    __syncthreads();
    int base0 = 0, base1 = 0, tot0 = 0, tot1 = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      base0 += w < wave ? wcount[w] : 0;
      base1 += w < wave ? wcount[4 + w] : 0;
      tot0 += wcount[w];
      tot1 += wcount[4 + w];
    }
    n8s = tot0 + tot1;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (!keep[h]) continue;
      const int c = t + h * kP5Threads;
      const int i = h == 0 ? base0 + __popcll(b0 & below) : tot0 + base1 + __popcll(b1 & below);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        pos8[j][i] = pv[h][j] >= 0 ? ((pv[h][j] << 9) | c) : (-512 | c);
        scl[j][i] = sv[h][j];
      }
    }
  }
  __syncthreads();

  v4f acc[4][8];   // [token block][row tile * 4 + j-block]
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 8; ++jb) acc[tb][jb] = v4f{0.f, 0.f, 0.f, 0.f};

  const int S = n8s + 2 * n16;
  if (S > 0) {
    // DMA lanes: INT8 steps move token blocks 4w .. 4w + 3 and j-blocks
    // 2(w & 1), 2(w & 1) + 1 of row r0 + (w >> 1); 16-bit steps move the same
    // token blocks and j-block w of the tile half.  6 loads per wave per step.
    int64_t xrow8[4], xrow16[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = min(n0 + (4 * wave + i) * 16 + arow, a.n - 1);
      xrow8[i] = row * a.ldq + akq * 16;
      xrow16[i] = row * a.ldx + akq * 8;
    }
    const int wj = wave >> 1;
    int w_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int jb = 2 * (wave & 1) + i;
      w_off[i] = (a.layout == TQ_LAYOUT_MFMA) ? jb * 1024 + lane * 16
                                              : (jb * 16 + (lane & 15)) * 64 + (lane >> 4) * 16;
    }
    const int w16_off = (a.layout == TQ_LAYOUT_MFMA) ? wave * 1024 + lane * 8
                                                     : (wave * 16 + (lane & 15)) * 64 + (lane >> 4) * 8;
    const uint32_t smem_lds = lds_addr(smem);
    const uint32_t pos_lds = lds_addr(&pos8[0][0]), scl_lds = lds_addr(&scl[0][0]);
    const uint32_t l16_lds = lds_addr(list16);
    // LDS byte address of the DMA metadata of step sn (INT8: this wave's row position; 16-bit: list entry)
    auto dma_meta_addr = [&](int sn) -> uint32_t {
      return sn < n8s ? pos_lds + 4 * (wj * kP5MaxCols + sn) : l16_lds + 4 * ((sn - n8s) >> 1);
    };
    // The step's 6 loads in 3 parts of 2, issued at points spread over the
    // MFMA phase: a burst of all waves' loads right after the barrier backs
    // up the texture path and stalls the issuing waves.
    auto issue_part = [&](int sn, int st, int meta, int part) {
      int8_t* sp = smem + st * kP3Stage;
      if (sn < n8s) {
        if (part < 2) {
          const int col = meta & 511;
#pragma unroll
          for (int i = 2 * part; i < 2 * part + 2; ++i)
            __builtin_amdgcn_global_load_lds(a.xq + xrow8[i] + col * 64, sp + (4 * wave + i) * 1024, 16, 0, 0);
        } else {
          const int pw = meta >= 0 ? meta >> 9 : 0;   // a 16-bit tile here: any valid INT8 tile, unused
#pragma unroll
          for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(a.w8 + (int64_t)pw * 4096 + w_off[i],
                                             sp + kPfXBytes + wj * 4096 + (2 * (wave & 1) + i) * 1024, 16, 0, 0);
        }
      } else {
        const int h = (sn - n8s) & 1;
        if (part < 2) {
          const int col = (meta & 511) * 64 + h * 32;
#pragma unroll
          for (int i = 2 * part; i < 2 * part + 2; ++i)
            __builtin_amdgcn_global_load_lds(a.xf + xrow16[i] + col, sp + (4 * wave + i) * 1024, 16, 0, 0);
        } else {
          const int64_t q = (unsigned)meta >> 10;
          const uint16_t* wsrc = a.w16 + q * 4096 + w16_off + ((a.layout == TQ_LAYOUT_MFMA) ? h * 512 : h * 32);
          // the same 1 KiB twice keeps the per-step load count at 6
          __builtin_amdgcn_global_load_lds(wsrc, sp + kPfXBytes + wave * 1024, 16, 0, 0);
          __builtin_amdgcn_global_load_lds(wsrc, sp + kPfXBytes + wave * 1024, 16, 0, 0);
        }
      }
    };
    auto issue = [&](int sn, int st, int meta) {
      issue_part(sn, st, meta, 0);
      issue_part(sn, st, meta, 1);
      issue_part(sn, st, meta, 2);
    };
    auto read_meta = [&](uint32_t addr) {
      int v;
      asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(addr) : "memory");
      return __builtin_amdgcn_readfirstlane(v);
    };
#pragma unroll
    for (int st = 0; st < P - 1; ++st) {
      const int sn = min(st, S - 1);
      issue(sn, st, read_meta(dma_meta_addr(sn)));
    }
    const uint32_t w_rd = smem_lds + kPfXBytes + lane * 16;
    const uint32_t x_rd = smem_lds + wave * 4096 + lane * 16;

    // Step metadata (DMA position, tile positions, scales) in VGPRs, lane i
    // holding step base + i of a 64-step window loaded once per window: each
    // step takes its values with v_readlane instead of five LDS reads and a
    // wait (2.5% per Llama layer at 8192 tokens, up to 5% on O).
    int w_mn = 0, w_m0 = 0, w_m1 = 0, w_sc0 = 0, w_sc1 = 0;
    auto step = [&](auto mode_tag, int s) {
      constexpr int MODE = decltype(mode_tag)::value;
      const int stage = s % P;
      // DUMP: every vector memory operation drained (stores and any spill
      // traffic count in vmcnt too), so stage s has certainly landed
      if constexpr (DUMP) wait_vmcnt<0>();
      else wait_vmcnt<6 * (P - 2)>();
      asm volatile("s_barrier" ::: "memory");
      const int sn = min(s + P - 1, S - 1);
      constexpr bool is8 = MODE == 0;
      const int wi = s & 63;
      if (wi == 0) {
        const int ls = min(s + lane, S - 1);
        const int lsn = min(ls + P - 1, S - 1);
        const int lc8 = max(min(ls, n8s - 1), 0);
        asm volatile(
            "ds_read_b32 %0, %5\n\t"
            "ds_read_b32 %1, %6\n\t"
            "ds_read_b32 %2, %7\n\t"
            "ds_read_b32 %3, %8\n\t"
            "ds_read_b32 %4, %9\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w_mn), "=&v"(w_m0), "=&v"(w_m1), "=&v"(w_sc0), "=&v"(w_sc1)
            : "v"(dma_meta_addr(lsn)), "v"(ls < n8s ? pos_lds + 4 * ls : l16_lds + 4 * ((ls - n8s) >> 1)),
              "v"(pos_lds + 4 * (kP5MaxCols + lc8)), "v"(scl_lds + 4 * lc8), "v"(scl_lds + 4 * (kP5MaxCols + lc8))
            : "memory");
      }
      const int mn = __builtin_amdgcn_readlane(w_mn, wi);
      const int m0 = __builtin_amdgcn_readlane(w_m0, wi);
      const int m1 = __builtin_amdgcn_readlane(w_m1, wi);
      const float sc0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(w_sc0, wi));
      const float sc1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(w_sc1, wi));
      const int dst = (stage + P - 1) % P, dmeta = __builtin_amdgcn_readfirstlane(mn);
      issue_part(sn, dst, dmeta, 0);
      const int meta0 = __builtin_amdgcn_readfirstlane(m0);
      const uint32_t so = stage * kP3Stage;
      if constexpr (is8) {
        const bool h0 = meta0 >= 0;
        const bool h1 = __builtin_amdgcn_readfirstlane(m1) >= 0 && has1;
        if (!h0 && !h1) {
          issue_part(sn, dst, dmeta, 1);
          issue_part(sn, dst, dmeta, 2);
          return;
        }
        const float s0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sc0)));
        const float s1 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sc1)));
        v4i ax[4], bw[8];
        // operand reads in the order the MFMAs use them -- row 0's weights, the
        // four token blocks, row 1's weights -- each MFMA group waiting only
        // for its own reads (LDS reads complete in order)
        asm volatile(
            "ds_read_b128 %0, %12\n\t"
            "ds_read_b128 %1, %12 offset:1024\n\t"
            "ds_read_b128 %2, %12 offset:2048\n\t"
            "ds_read_b128 %3, %12 offset:3072\n\t"
            "ds_read_b128 %4, %13\n\t"
            "ds_read_b128 %5, %13 offset:1024\n\t"
            "ds_read_b128 %6, %13 offset:2048\n\t"
            "ds_read_b128 %7, %13 offset:3072\n\t"
            "ds_read_b128 %8, %12 offset:4096\n\t"
            "ds_read_b128 %9, %12 offset:5120\n\t"
            "ds_read_b128 %10, %12 offset:6144\n\t"
            "ds_read_b128 %11, %12 offset:7168\n\t"
            : "=&v"(bw[0]), "=&v"(bw[1]), "=&v"(bw[2]), "=&v"(bw[3]),
              "=&v"(ax[0]), "=&v"(ax[1]), "=&v"(ax[2]), "=&v"(ax[3]),
              "=&v"(bw[4]), "=&v"(bw[5]), "=&v"(bw[6]), "=&v"(bw[7])
            : "v"(w_rd + so), "v"(x_rd + so)
            : "memory");
        if constexpr (DUMP)   // all 12 reads landed: the partial lgkmcnt waits below are then no-ops
          asm volatile("s_waitcnt lgkmcnt(0)"
                       : "+v"(bw[0]), "+v"(bw[1]), "+v"(bw[2]), "+v"(bw[3]), "+v"(ax[0]), "+v"(ax[1]),
                         "+v"(ax[2]), "+v"(ax[3]), "+v"(bw[4]), "+v"(bw[5]), "+v"(bw[6]), "+v"(bw[7])::"memory");
        // wait for the reads up to token block tb (row 0) -- outstanding <= 7 - tb
        auto wait_tb = [&](int tb) {
          if (tb == 0) asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(bw[0]), "+v"(bw[1]), "+v"(bw[2]), "+v"(bw[3]), "+v"(ax[0]) :: "memory");
          else if (tb == 1) asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(ax[1]) :: "memory");
          else if (tb == 2) asm volatile("s_waitcnt lgkmcnt(5)" : "+v"(ax[2]) :: "memory");
          else asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(ax[3]) :: "memory");
        };
        // one row tile's 16 MFMAs (+ epilogue), with a load part issued after the first 8
        auto row_mfma = [&](auto j_tag, float sc, int part, bool first, int pos) {
          constexpr int J = decltype(j_tag)::value;
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            if (first) wait_tb(tb);
            if (tb == 2) {
              __builtin_amdgcn_sched_barrier(0);
              issue_part(sn, dst, dmeta, part);
              __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
              const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[tb], bw[J + jb], v4i{0, 0, 0, 0}, 0, 0, 0);
              dump_i32<DUMP>(a, pos, n0 + wave * 64 + tb * 16 + 4 * akq, jb * 16 + arow, d);
#pragma unroll
              for (int v = 0; v < 4; ++v) acc[tb][J + jb][v] = fmaf((float)d[v], sc, acc[tb][J + jb][v]);
            }
          }
        };
        if (h0) row_mfma(std::integral_constant<int, 0>{}, s0, 1, true, meta0 >> 9);
        else issue_part(sn, dst, dmeta, 1);
        // everything else (row 1's weights; row 0's operands when row 0 took no MFMAs)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(bw[4]), "+v"(bw[5]), "+v"(bw[6]), "+v"(bw[7]), "+v"(ax[0]), "+v"(ax[1]), "+v"(ax[2]),
                       "+v"(ax[3]) :: "memory");
        if (h1) row_mfma(std::integral_constant<int, 4>{}, s1, 2, false, __builtin_amdgcn_readfirstlane(m1) >> 9);
        else issue_part(sn, dst, dmeta, 2);
        // gfx9 counts stores in vmcnt too: drain the dump's stores so the next
        // step's vmcnt wait counts ring loads only
        if constexpr (DUMP) wait_vmcnt<0>();
      } else {
        v4i ax[4], bw[4];
        asm volatile(
            "ds_read_b128 %0, %8\n\t"
            "ds_read_b128 %1, %8 offset:1024\n\t"
            "ds_read_b128 %2, %8 offset:2048\n\t"
            "ds_read_b128 %3, %8 offset:3072\n\t"
            "ds_read_b128 %4, %9\n\t"
            "ds_read_b128 %5, %9 offset:1024\n\t"
            "ds_read_b128 %6, %9 offset:2048\n\t"
            "ds_read_b128 %7, %9 offset:3072\n\t"
            : "=&v"(bw[0]), "=&v"(bw[1]), "=&v"(bw[2]), "=&v"(bw[3]),
              "=&v"(ax[0]), "=&v"(ax[1]), "=&v"(ax[2]), "=&v"(ax[3])
            : "v"(w_rd + so), "v"(x_rd + so)
            : "memory");
        constexpr int J = MODE == 2 ? 4 : 0;   // the row's accumulators
        issue_part(sn, dst, dmeta, 1);
        issue_part(sn, dst, dmeta, 2);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          if (tb == 0) asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(bw[0]), "+v"(bw[1]), "+v"(bw[2]), "+v"(bw[3]), "+v"(ax[0]) :: "memory");
          else if (tb == 1) asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(ax[1]) :: "memory");
          else if (tb == 2) asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(ax[2]) :: "memory");
          else asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ax[3]) :: "memory");
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) acc[tb][J + jb] = mfma16<XT>(ax[tb], bw[jb], acc[tb][J + jb]);
        }
      }
    };
    // list16 holds row r0's 16-bit tiles before row r0 + 1's: three loops, one accumulator set each
    for (int s = 0; s < n8s; ++s) step(std::integral_constant<int, 0>{}, s);
    for (int s = n8s; s < n8s + 2 * n16_0; ++s) step(std::integral_constant<int, 1>{}, s);
    for (int s = n8s + 2 * n16_0; s < S; ++s) step(std::integral_constant<int, 2>{}, s);
    wait_vmcnt<0>();
  }
  __syncthreads();   // every wave is done with the ring: reuse it for the outputs

  // ---- epilogue: round, bias (double rounding), stage rows in LDS, 16-byte stores
  uint16_t* so16 = reinterpret_cast<uint16_t*>(smem + wave * 64 * kP5OutRow);
  auto stage_out = [&](auto out_tag, auto bias_tag) {
    using OT = typename decltype(out_tag)::type;
    constexpr bool HB = decltype(bias_tag)::value;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int col = (r0 + (jj >> 2)) * 64 + (jj & 3) * 16 + arow;
        float bv = 0.f;
        if constexpr (HB) bv = OT::to_f32(a.bias[min(col, a.m - 1)]);
        uint16_t* dst = so16 + (tb * 16 + 4 * akq) * (kP5OutRow / 2) + jj * 16 + arow;
#pragma unroll
        for (int v = 0; v < 4; v += 2) {
          uint32_t y2 = OT::pack2(acc[tb][jj][v], acc[tb][jj][v + 1]);
          if constexpr (HB)   // the reference's double rounding: round(round(acc) + bias)
            y2 = OT::pack2(OT::to_f32((uint16_t)y2) + bv, OT::to_f32((uint16_t)(y2 >> 16)) + bv);
          dst[v * (kP5OutRow / 2)] = (uint16_t)y2;
          dst[(v + 1) * (kP5OutRow / 2)] = (uint16_t)(y2 >> 16);
        }
      }
  };
  if (a.out_bf16) {
    if (a.bias) stage_out(TypeTag<Bf16>{}, std::true_type{});
    else stage_out(TypeTag<Bf16>{}, std::false_type{});
  } else {
    if (a.bias) stage_out(TypeTag<Fp16>{}, std::true_type{});
    else stage_out(TypeTag<Fp16>{}, std::false_type{});
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave reads back only its own rows
  const int cw = has1 ? 128 : 64;       // valid staged columns
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int rr = i * 4 + (lane >> 4);   // staged row 0..63
    const int ch = lane & 15;             // 16-byte chunk: columns ch*8 .. ch*8+7
    const int row = n0 + wave * 64 + rr;
    const int col = r0 * 64 + ch * 8;
    if (row >= a.n || ch * 8 >= cw || col >= a.m) continue;
    const v4i val = *reinterpret_cast<const v4i*>(smem + wave * 64 * kP5OutRow + rr * kP5OutRow + ch * 16);
    uint16_t* dst = a.out + (int64_t)row * a.ldo + col;
    if (a.ovec && col + 8 <= a.m) {
      *reinterpret_cast<v4i*>(dst) = val;
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (col + u < a.m) dst[u] = (uint16_t)((uint32_t)val[u >> 1] >> (16 * (u & 1)));
    }
  }
}

// ---- host side -----------------------------------------------------------

static int pick_tb(int n) { return n <= 16 ? 1 : (n <= 32 ? 2 : 4); }

static bool xvec_ok(const GemmArgs& a) {
  return a.k == a.n_tc * 64 && (a.ldq % 16) == 0 && aligned16(a.xq) &&
         (a.xf == nullptr || ((a.ldx % 8) == 0 && aligned16(a.xf)));
}

// Decode schedule.  Cross-workgroup reduction costs several microseconds of
// serial latency on MI355X (write-through stores, a counter RMW, coherent
// reads), more than the data time of a small GEMM, so the automatic plan
// never splits: whole-tile workgroups (JBW 4) when the row tiles alone give
// enough workgroups, else one 16-feature j-block per workgroup (JBW 1), and
// W waves so each wave keeps a batch of U tiles in flight.  An explicit
// split_k > 1 runs S = split_k splits with the reduction.
// Whole-tile workgroups (JBW 4) only where one-j-block workgroups would each
// stage a large activation: with many row tiles and more than 8 tokens.  Below
// that, four workgroups per row tile (one 16-feature j-block each) give 4x the
// workgroups, which streams the weights faster (measured on MI355X: the stacked
// gate/up projection at 1-4 tokens runs ~13% faster).
constexpr int kWideRowTiles = 192;
constexpr int kWideMinTokens = 9;
static int pick_jbw(int n, int n_tr) { return (n_tr >= kWideRowTiles && n >= kWideMinTokens) ? 4 : 1; }

// The arrival counters occupy a FIXED region at the head of the workspace so
// that calls with different shapes never see another call's partials as
// counters; shapes with more units than the cap run with one split.
constexpr int kCounterCap = 4096;
static int64_t counter_elems(int units) { (void)units; return kCounterCap; }

struct SplitPlan {
  int S, W, tb, jbw;
};

static int plan_u(int jbw, int tb) { return jbw == 1 ? (tb == 1 ? 8 : 4) : (tb == 1 ? 4 : 2); }

static int plan_max_waves(int jbw, int tb) {
  // LDS for the reduction: W * jbw * tb * 1 KiB <= 64 KiB (128 KiB for four
  // token blocks, whose waves otherwise take a dozen tiles each one batch at a
  // time); launch bound 16 / 8 waves
  int w = (tb == 4 ? 128 : 64) / (jbw * tb);
  const int bound = jbw == 1 ? 16 : 8;
  return w < bound ? w : bound;
}

// Waves per workgroup of the unsplit decode schedules.  gemm_decode_kernel and
// gemm_splitk_kernel both take a row tile's tiles round-robin over W waves and
// sum the wave partials in wave order, so with the same W they add the same
// terms in the same order: their outputs are bitwise equal (the fused path
// falls back to gemm_splitk_kernel where gemm_decode_kernel cannot stage the
// activation).  About UMAX tiles per wave; at most 8 waves for whole-tile
// (JBW 4) workgroups.
constexpr int kDecUmaxJb1 = 8;   // one-j-block workgroups: tiles per wave and batch
constexpr int kDecUmaxJb4 = 6;   // whole-tile workgroups
// Grids of more than kDecManyUnits one-j-block workgroups run several per CU;
// there a wave count that is not a multiple of 4 (e.g. 6 waves for 48 column
// tiles) leaves wave slots of the four SIMDs unusable, and only ~3 of the 4
// workgroups per CU that the registers allow start together (measured on
// MI355X for the stacked gate/up projection: 1024 workgroups, ~770 in the first
// round).  Those grids use 4 waves with batches of up to 16 tiles (32 < n_tc
// <= 64): 6% faster there, slower on grids of <= 2 workgroups per CU.
constexpr int kDecManyUnits = 512;
static bool decode_wide_batches(int jbw, int tb, int units, int n_tc) {
  return jbw == 1 && tb == 1 && units > kDecManyUnits && n_tc > 32 && n_tc <= 64;
}
static int decode_umax(int jbw, int tb, int units, int n_tc) {
  if (decode_wide_batches(jbw, tb, units, n_tc)) return n_tc <= 48 ? 12 : 16;
  return jbw == 1 ? kDecUmaxJb1 : kDecUmaxJb4;
}
static int decode_waves(int jbw, int tb, int units, int n_tc) {
  const int umax = decode_umax(jbw, tb, units, n_tc);
  const int wmax = jbw == 1 ? 16 : 8;
  int W = (n_tc + umax - 1) / umax;
  return W < 4 ? 4 : (W > wmax ? wmax : W);
}

static SplitPlan plan_split(int n, int n_tr, int n_tc, int split_k) {
  SplitPlan p;
  p.tb = pick_tb(n);
  p.jbw = pick_jbw(n, n_tr);
  // 17-32 rows: wide projections take half tiles per workgroup (twice the
  // workgroups); measured on MI355X, stacked Gate/Up at 17 / 24 / 32 rows
  // 15.49 / 15.59 / 15.82 -> 14.46 / 14.57 / 14.69 us, bitwise unchanged (the
  // same tiles per wave in the same order).  At 33-64 rows whole tiles stay
  // (half tiles 18.7 -> 21.6 us at 64 rows).
  if (p.jbw == 4 && p.tb == 2) p.jbw = 2;
  p.S = split_k > 1 ? split_k : 1;
  const int units = n_tr * (4 / p.jbw);
  if (p.S > 1 && units > kCounterCap) p.S = 1;
  const int per_split = (n_tc + p.S - 1) / p.S;
  const int U = plan_u(p.jbw, p.tb);
  int W = p.S == 1 ? decode_waves(p.jbw, p.tb, units, n_tc) : (per_split + U - 1) / U;
  const int wmax = plan_max_waves(p.jbw, p.tb);
  if (W > wmax) W = wmax;
  p.W = W < 1 ? 1 : W;
  return p;
}

static int64_t split_workspace_elems(const SplitPlan& p, int n, int n_tr) {
  const int64_t units = (int64_t)n_tr * (4 / p.jbw);
  return p.S > 1 ? counter_elems((int)units) + units * p.S * n * 64 : 0;
}

// Dynamic LDS beyond the default per-kernel limit needs that limit raised
// (gfx950: 160 KiB per workgroup, static + dynamic).  Raised per kernel (the
// kernel is the template argument) to the largest dynamic size requested so
// far; a failure is returned so that the launch is not attempted.
template <auto Kern>
static hipError_t allow_lds(size_t dyn_bytes) {
  static std::atomic<size_t> raised{0};
  if (dyn_bytes <= 32 * 1024 || dyn_bytes <= raised.load(std::memory_order_relaxed)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(Kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn_bytes);
  if (e == hipSuccess) raised.store(dyn_bytes, std::memory_order_relaxed);
  return e;
}

template <auto Kern>
static hipError_t launch_split_kernel(dim3 grid, dim3 block, size_t lds, hipStream_t s, const GemmArgs& a) {
  const hipError_t e = allow_lds<Kern>(lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(Kern, grid, block, lds, s, a);
  return hipGetLastError();
}

template <class XT, bool FUSED, bool XVEC, int JBW, bool DUMP>
static hipError_t launch_split_v(const GemmArgs& a, const SplitPlan& p, dim3 grid, dim3 block, size_t lds,
                                 hipStream_t s) {
  constexpr int U1 = JBW == 1 ? 8 : 4, U2 = JBW == 1 ? 4 : 2, U4 = JBW == 1 ? 4 : 2;
  if constexpr (FUSED) {
    const int n = a.n;
    if (n <= 1)
      return launch_split_kernel<gemm_splitk_kernel<XT, 1, U1, true, 1, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
    if (n <= 2)
      return launch_split_kernel<gemm_splitk_kernel<XT, 1, U1, true, 2, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
    if (n <= 4)
      return launch_split_kernel<gemm_splitk_kernel<XT, 1, U1, true, 4, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
    if (n <= 8)
      return launch_split_kernel<gemm_splitk_kernel<XT, 1, U1, true, 8, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
    return launch_split_kernel<gemm_splitk_kernel<XT, 1, (U1 > 4 ? 4 : U1), true, 16, XVEC, JBW, false, DUMP>>(
        grid, block, lds, s, a);
  } else if (a.xblk > 0) {
    switch (p.tb) {
      case 1:
        return launch_split_kernel<gemm_splitk_kernel<XT, 1, U1, false, 1, true, JBW, true, DUMP>>(grid, block, lds, s, a);
      case 2:
        return launch_split_kernel<gemm_splitk_kernel<XT, 2, U2, false, 1, true, JBW, true, DUMP>>(grid, block, lds, s, a);
      default:
        return launch_split_kernel<gemm_splitk_kernel<XT, 4, U4, false, 1, true, JBW, true, DUMP>>(grid, block, lds, s, a);
    }
  } else {
    switch (p.tb) {
      case 1:
        return launch_split_kernel<gemm_splitk_kernel<XT, 1, U1, false, 1, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
      case 2:
        return launch_split_kernel<gemm_splitk_kernel<XT, 2, U2, false, 1, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
      default:
        return launch_split_kernel<gemm_splitk_kernel<XT, 4, U4, false, 1, XVEC, JBW, false, DUMP>>(grid, block, lds, s, a);
    }
  }
}

// LDS of the fused prologue: codes [n][64 * n_tc] (16-byte aligned) + sx[n_tc].
static size_t fused_lds_bytes(int n, int n_tc) {
  return (((size_t)n * n_tc * 64 + 15) & ~(size_t)15) + (size_t)n_tc * sizeof(float);
}

template <class XT, bool FUSED, bool DUMP = false>
static hipError_t launch_split(GemmArgs a, const SplitPlan& p, float* ws, hipStream_t s) {
  a.splits = p.S;
  const int units = a.n_tr * (4 / p.jbw);
  a.counters = reinterpret_cast<int32_t*>(ws);
  a.partials = ws ? ws + counter_elems(units) : nullptr;
  dim3 grid(units * p.S), block(p.W * kWave);
  size_t lds = (size_t)p.W * p.jbw * p.tb * 4 * 64 * sizeof(float);
  if (FUSED && fused_lds_bytes(a.n, a.n_tc) > lds) lds = fused_lds_bytes(a.n, a.n_tc);
  if (p.jbw == 4)
    return a.xvec ? launch_split_v<XT, FUSED, true, 4, DUMP>(a, p, grid, block, lds, s)
                  : launch_split_v<XT, FUSED, false, 4, DUMP>(a, p, grid, block, lds, s);
  if (p.jbw == 2)
    return a.xvec ? launch_split_v<XT, FUSED, true, 2, DUMP>(a, p, grid, block, lds, s)
                  : launch_split_v<XT, FUSED, false, 2, DUMP>(a, p, grid, block, lds, s);
  return a.xvec ? launch_split_v<XT, FUSED, true, 1, DUMP>(a, p, grid, block, lds, s)
                : launch_split_v<XT, FUSED, false, 1, DUMP>(a, p, grid, block, lds, s);
}

// Chooses the split plan and checks the workspace; without a (large enough)
// workspace an automatic plan falls back to S = 1, an explicit split_k > 1 is
// an error.
static int resolve_plan(SplitPlan& p, int n, int n_tr, int split_k, float* ws, int64_t ws_elems) {
  const int64_t need = split_workspace_elems(p, n, n_tr);
  if (need == 0) return TQ_OK;
  if (ws != nullptr && ws_elems >= need && ((uintptr_t)ws & 3u) == 0) return TQ_OK;
  if (split_k > 1) return TQ_ERR_WORKSPACE;
  p.S = 1;
  return TQ_OK;
}

// Plan of gemm_decode_kernel: wave count, batch size, activation chunks per
// thread, LDS bytes.  ok == false when the activation does not fit LDS or a
// size limit is exceeded; the caller then uses gemm_splitk_kernel.
struct DecodePlan {
  int W, tb, jbw, umax, cmax;
  size_t lds;
  bool ok;
};

static DecodePlan plan_decode(int n, int k, int n_tr, int n_tc, bool quant) {
  DecodePlan p{};
  p.ok = false;
  p.tb = pick_tb(n);
  p.jbw = pick_jbw(n, n_tr);
  const int units = n_tr * (4 / p.jbw);
  p.umax = decode_umax(p.jbw, p.tb, units, n_tc);
  if (n < 1 || n > kDecodeMaxTokens || k != n_tc * 64 || (quant && n > kFusedMaxTokens)) return p;
  const int W = decode_waves(p.jbw, p.tb, units, n_tc);
  p.W = W;
  const int64_t T = (int64_t)W * kWave;
  const int64_t codes = (int64_t)n * (k + 16);
  const int64_t meta = (int64_t)n_tc * 4 * (quant ? 3 : 1);
  const int64_t red = (int64_t)W * p.jbw * p.tb * 1024;
  const int64_t chunks = quant ? (int64_t)n * k / 8 : (int64_t)n * k / 16;
  const int64_t per = (chunks + T - 1) / T;
  p.cmax = per <= 1 ? 1 : (per <= 2 ? 2 : (per <= 4 ? 4 : 8));
  p.lds = (size_t)(codes + meta > red ? codes + meta : red);
  // 16-token blocks: one or two (more than 32 rows use gemm_splitk_kernel)
  p.ok = p.tb <= 2 && per <= (quant ? 4 : 8) && codes <= kDecCodesMax && n_tc <= 2 * T && p.lds <= 160 * 1024;
  return p;
}

template <class XT, int TB, int JBW, int UMAX, bool QUANT, int CMAX, bool DUMP>
static hipError_t launch_decode_one(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  constexpr auto kern = gemm_decode_kernel<XT, TB, JBW, UMAX, QUANT, CMAX, DUMP>;
  const hipError_t e = allow_lds<kern>(p.lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(a.n_tr * (4 / JBW)), dim3(p.W * kWave), p.lds, s, a);
  return hipGetLastError();
}

template <class XT, int TB, int JBW, int UMAX, bool QUANT, bool DUMP>
static hipError_t launch_decode_c(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  switch (p.cmax) {
    case 1: return launch_decode_one<XT, TB, JBW, UMAX, QUANT, 1, DUMP>(a, p, s);
    case 2: return launch_decode_one<XT, TB, JBW, UMAX, QUANT, 2, DUMP>(a, p, s);
    case 4: return launch_decode_one<XT, TB, JBW, UMAX, QUANT, 4, DUMP>(a, p, s);
    default:
      if constexpr (!QUANT) return launch_decode_one<XT, TB, JBW, UMAX, QUANT, 8, DUMP>(a, p, s);
      return hipErrorInvalidValue;   // QUANT plans stop at 4 chunks
  }
}

// ---- quantizing decode kernel with helper waves ------------------------------
// gemm_decode_kernel<..., QUANT, ..., HELP>: the plain (non-quantizing) decode
// plan's W tile waves -- so the sums are the two-launch path's, bit for bit --
// plus k / 512 helper waves that quantize by lanes, one thread per 8-column
// chunk of a row, all n <= 8 rows (CMAX = n rounded up), as soon as their
// activation loads arrive.  For one-j-block workgroups with 8-tile batches and
// at most 16 waves in all (Llama-3.2-3B Q/K/V and O: 6 + 6; Qwen2.5-7B: 7 + 7),
// at 1-2 rows and where the plain quantizing kernel does not fit.  Measured on
// MI355X (cold weights, per launch, plain -> helpers): Llama Q/K/V at one row
// 8.42 -> 7.46 us, O 6.12 -> 5.29; at 2 rows 8.51 -> 8.53 and 6.09 -> 5.93;
// at 4 rows Q/K/V 10.14 -> 10.00 but O 7.04 -> 7.30 (the helpers' quantization
// then runs while the tile waves issue their weights and slows that issue),
// so 4 rows keep the plain kernel.
static DecodePlan plan_help(int n, int k, int n_tr, int n_tc) {
  DecodePlan p = plan_decode(n, k, n_tr, n_tc, false);
  const bool shape = p.ok && p.jbw == 1 && p.tb == 1 && p.umax == kDecUmaxJb1 && n <= 8 && (k & 511) == 0 &&
                     p.W + k / 512 <= 16 && (n <= 2 || !plan_decode(n, k, n_tr, n_tc, true).ok);
  p.ok = false;
  if (!shape) return p;
  p.cmax = n <= 1 ? 1 : (n <= 2 ? 2 : (n <= 4 ? 4 : 8));
  const int64_t codes = (int64_t)n * (k + 16), meta = (int64_t)n_tc * 4 * 3, red = (int64_t)p.W * 1024;
  p.lds = (size_t)std::max(codes + meta, red);
  p.ok = codes <= kDecCodesMax;
  return p;
}

static int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < 64) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Launches the helper-wave kernel, or returns hipErrorNotSupported (nothing
// launched) when its grid would not be resident at once: the helper waves
// cost registers, and a second round of workgroups costs far more than the
// helpers save (Qwen2.5-7B Q/K/V: 14-wave workgroups, two per CU needed).
template <class XT, int CMAX, bool DUMP>
static hipError_t launch_help_one(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  constexpr auto kern = gemm_decode_kernel<XT, 1, 1, kDecUmaxJb1, true, CMAX, DUMP, false, true>;
  const int threads = (p.W + a.k / 512) * kWave;
  const hipError_t e = allow_lds<kern>(p.lds);
  if (e != hipSuccess) return e;
  // resident workgroups per CU, cached per (waves, KiB of LDS): the query is
  // host work every eager launch would repeat
  static std::atomic<int> cache[17][161];
  const size_t kib = (p.lds + 1023) / 1024;
  std::atomic<int>* slot = (threads / kWave <= 16 && kib <= 160) ? &cache[threads / kWave][kib] : nullptr;
  int per_cu = slot ? slot->load(std::memory_order_relaxed) : 0;
  if (per_cu <= 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, kib * 1024) != hipSuccess) per_cu = 0;
    if (slot && per_cu > 0) slot->store(per_cu, std::memory_order_relaxed);
  }
  if ((int64_t)per_cu * device_cus() < (int64_t)a.n_tr * 4) return hipErrorNotSupported;
  hipLaunchKernelGGL(kern, dim3(a.n_tr * 4), dim3(threads), p.lds, s, a);
  return hipGetLastError();
}

template <class XT, bool DUMP = false>
static hipError_t launch_help(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  switch (p.cmax) {
    case 1: return launch_help_one<XT, 1, DUMP>(a, p, s);
    case 2: return launch_help_one<XT, 2, DUMP>(a, p, s);
    case 4: return launch_help_one<XT, 4, DUMP>(a, p, s);
    default: return launch_help_one<XT, 8, DUMP>(a, p, s);
  }
}

// ---- cooperative quantize + GEMM plan ----------------------------------------
// COOP launches (gemm_decode_kernel<..., COOP>, one token block, one-j-block
// units) take the one-launch shapes the LDS-staged quantizing decode kernel
// cannot (too many rows x columns for its chunks per thread), which otherwise
// go to the quantizing split-K kernel.  Measured on MI355X (cold weights, per
// launch): Llama-3.2-3B Q/K/V at 8 rows 10.4 us vs 18.0, at 16 rows 12.5 vs
// 22.7; Gate/Up at 4 rows 20.9 vs 22.3; Qwen2.5-7B Gate/Up at 4 rows 44.0 vs
// 54.2.  Where the LDS-staged kernel applies it stays: its workgroups start
// their MFMAs without the hand-off's round trips (write-through codes, a
// count, a flag, a poll and coherent reloads, ~3-5 us), e.g. Q/K/V at one row
// 8.4 us vs 9.7 cooperative.  Producers: 8 (one per XCD, so the units keep
// their XCD).  Workspace (fp32 elements): the
// flags and counts (kCoopCount + 1 entries, inside the split-K counter region:
// both leave it zero), then the codes [n][k] and the scales [n_tc].
constexpr int kCoopProducers = 8;
constexpr int kCoopSpin = 4096;   // polls (plus s_sleep) before a workgroup quantizes itself
// The codes go where split-K launches put their scratch partials: after the
// counter region, which must stay zero between launches.
constexpr int64_t kCoopHead = kCounterCap;
static_assert(kCoopCount + 1 <= kCoopHead && kCoopGroups == 64, "COOP flags: one per lane, inside the head");
// Poll budget of COOP launches (-1: kCoopSpin); tests set 0 to make every
// GEMM workgroup take its quantize-locally path.
static std::atomic<int> g_coop_spin{-1};

struct CoopPlan {
  DecodePlan d;   // W = tile waves; the launch adds the loader wave
  bool ok;
};

static CoopPlan plan_coop(int n, int k, int n_tr, int n_tc) {
  CoopPlan c{};
  c.ok = false;
  if (n < 1 || n > kFusedMaxTokens || k != 64 * n_tc) return c;
  c.d = plan_decode(n, k, n_tr, n_tc, false);
  if (!c.d.ok || c.d.jbw != 1 || c.d.tb != 1 || c.d.W > 15) return c;
  if (plan_decode(n, k, n_tr, n_tc, true).ok) return c;   // the LDS-staged quantizing kernel takes it
  // codes chunks per thread with the loader wave; the fallback's absmax array after the scales
  const int64_t T = (int64_t)(c.d.W + 1) * kWave;
  const int64_t per = ((int64_t)n * k / 16 + T - 1) / T;
  c.d.cmax = per <= 1 ? 1 : (per <= 2 ? 2 : (per <= 4 ? 4 : 8));
  if (per > 8 || n_tc > 2 * T || (c.d.umax == 16 && per > 4)) return c;   // (16-tile batches + 8 chunks spill)
  const int64_t codes = (int64_t)n * (k + 16), meta = (int64_t)n_tc * 8, red = (int64_t)c.d.W * 1024;
  const int64_t prod = (int64_t)(n_tc / kCoopProducers + 1) * 4;
  c.d.lds = (size_t)std::max({codes + meta, red, prod});
  c.ok = c.d.lds <= kDecCodesMax + 16 * 1024;
  return c;
}

static int64_t coop_workspace_elems(int n, int k, int n_tc) {
  return kCoopHead + (((int64_t)n * k + 15) / 16) * 4 + n_tc;
}

template <class XT, int UMAX, int CMAX, bool DUMP>
static hipError_t launch_coop_one(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  constexpr auto kern = gemm_decode_kernel<XT, 1, 1, UMAX, false, CMAX, DUMP, true>;
  const hipError_t e = allow_lds<kern>(p.lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(a.coop_p + a.n_tr * 4), dim3((p.W + 1) * kWave), p.lds, s, a);
  return hipGetLastError();
}

template <class XT, int UMAX, bool DUMP>
static hipError_t launch_coop_c(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  switch (p.cmax) {
    case 1: return launch_coop_one<XT, UMAX, 1, DUMP>(a, p, s);
    case 2: return launch_coop_one<XT, UMAX, 2, DUMP>(a, p, s);
    case 4: return launch_coop_one<XT, UMAX, 4, DUMP>(a, p, s);
    default: return launch_coop_one<XT, UMAX, 8, DUMP>(a, p, s);
  }
}

// a.xq / a.sx / a.coop point into the workspace (coop_workspace_elems).
template <class XT, bool DUMP = false>
static hipError_t launch_coop(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  if (p.umax == 12) return launch_coop_c<XT, 12, DUMP>(a, p, s);
  if (p.umax == 16) return launch_coop_c<XT, 16, DUMP>(a, p, s);
  return launch_coop_c<XT, kDecUmaxJb1, DUMP>(a, p, s);
}

template <class XT, bool QUANT, bool DUMP = false>
static hipError_t launch_decode(const GemmArgs& a, const DecodePlan& p, hipStream_t s) {
  if (p.jbw == 4) {
    if constexpr (QUANT) return launch_decode_c<XT, 1, 4, kDecUmaxJb4, true, DUMP>(a, p, s);
    else if (p.tb == 1) return launch_decode_c<XT, 1, 4, kDecUmaxJb4, false, DUMP>(a, p, s);
    else return launch_decode_c<XT, 2, 4, kDecUmaxJb4, false, DUMP>(a, p, s);
  }
  // p.umax is kDecUmaxJb1 except for many-unit grids with one token block
  if (p.tb == 1 && p.umax == 12) return launch_decode_c<XT, 1, 1, 12, QUANT, DUMP>(a, p, s);
  if (p.tb == 1 && p.umax == 16) return launch_decode_c<XT, 1, 1, 16, QUANT, DUMP>(a, p, s);
  if constexpr (QUANT) return launch_decode_c<XT, 1, 1, kDecUmaxJb1, true, DUMP>(a, p, s);
  else if (p.tb == 1) return launch_decode_c<XT, 1, 1, kDecUmaxJb1, false, DUMP>(a, p, s);
  else return launch_decode_c<XT, 2, 1, kDecUmaxJb1, false, DUMP>(a, p, s);
}

}  // namespace tq

using namespace tq;

extern "C" int64_t tq_gemm_workspace_elems(int n, int m, int n_tr, int n_tc, int split_k) {
  (void)m;
  if (n <= 0 || n_tr <= 0 || n > kDecodeMaxTokens) return 0;   // larger n: no workspace
  return split_workspace_elems(plan_split(n, n_tr, n_tc, split_k), n, n_tr);
}

static int check_gemm_common(int n, int m, int k, int n_tr, int n_tc, int x_dtype, int out_dtype,
                             int tile_layout) {
  if (n < 0 || m < 0 || k < 0 || n_tr < 0 || n_tc < 0) return TQ_ERR_ARG;
  if ((int64_t)n_tr * 64 < m || (int64_t)n_tc * 64 < k) return TQ_ERR_ARG;
  if (x_dtype != TQ_DTYPE_BF16 && x_dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (out_dtype != TQ_DTYPE_BF16 && out_dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (tile_layout != TQ_LAYOUT_ROW_MAJOR && tile_layout != TQ_LAYOUT_MFMA) return TQ_ERR_DTYPE;
  return TQ_OK;
}

// Launches the GEMM the automatic schedule picks for this shape (or, with
// DUMP, that kernel's DUMP instantiation, bf16 activations only) and, when
// `kernel` is non-null, stores its TQ_KERNEL_* family there.
template <bool DUMP>
static int gemm_mixed_rows(const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx,
                           const int8_t* int8_tiles, const float* int8_scales,
                           const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                           const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                           const void* fp16_tiles, const int32_t* fp16_tile_ids,
                           const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                           int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                           int n_tc, int split_k, int tile_layout, float* workspace,
                           int64_t workspace_elems, const int32_t* units, int n_units, int n_first,
                           int32_t* dump, int dump_r0, int dump_n, int* kernel, void* stream) {
  const bool xblk = (tile_layout & TQ_XQ_TOKEN_BLOCKED) != 0;   // token-blocked codes
  tile_layout &= ~TQ_XQ_TOKEN_BLOCKED;
  int rc = check_gemm_common(n, m, k, n_tr, n_tc, x_dtype, out_dtype, tile_layout);
  if (rc) return rc;
  if (DUMP && x_dtype != TQ_DTYPE_BF16) return TQ_ERR_DTYPE;
  if (units != nullptr && (n_units < 1 || n_units > n_tr || n_first < 0 || n_first > n_units))
    return TQ_ERR_ARG;
  if (xblk && (n > kDecodeMaxTokens || k != n_tc * 64)) return TQ_ERR_ARG;
  if (n == 0 || m == 0) return TQ_OK;
  if (out == nullptr || out_stride_n < m || int8_row_ptr == nullptr || x_int8 == nullptr || sx == nullptr)
    return TQ_ERR_ARG;
  if (!xblk && x_int8_stride_n < k) return TQ_ERR_ARG;
  const bool has16 = fp16_tiles != nullptr && fp16_tile_ids != nullptr && fp16_row_ptr != nullptr;
  if (has16 && (x_fp == nullptr || x_fp_stride_n < k)) return TQ_ERR_ARG;
  if (!aligned16(int8_tiles) || (has16 && !aligned16(fp16_tiles))) return TQ_ERR_ALIGN;
  if (DUMP && (dump == nullptr || dump_r0 < 0 || dump_n < 1 || dump_n > n - dump_r0)) return TQ_ERR_ARG;
  GemmArgs a{};
  a.xq = x_int8; a.ldq = x_int8_stride_n; a.sx = sx;
  a.w8 = int8_tiles; a.sw8 = int8_scales; a.ids8 = int8_tile_ids; a.rp8 = int8_row_ptr;
  a.xf = has16 ? static_cast<const uint16_t*>(x_fp) : nullptr; a.ldx = x_fp_stride_n;
  a.w16 = has16 ? static_cast<const uint16_t*>(fp16_tiles) : nullptr;
  a.ids16 = fp16_tile_ids; a.rp16 = fp16_row_ptr;
  a.out = static_cast<uint16_t*>(out); a.ldo = out_stride_n;
  a.bias = static_cast<const uint16_t*>(bias);
  a.dump = dump; a.dump_r0 = dump_r0; a.dump_n = dump_n;
  a.n = n; a.m = m; a.k = k; a.n_tr = n_tr; a.n_tc = n_tc;
  a.out_bf16 = out_dtype == TQ_DTYPE_BF16;
  a.layout = tile_layout;
  if (xblk) a.ldq = k;   // the stride argument is ignored for token-blocked codes
  a.xvec = xvec_ok(a);
  a.ovec = (a.ldo % 8) == 0 && aligned16(a.out);
  if (xblk) {   // read by gemm_splitk_kernel only, on its vector path
    if (!a.xvec || !aligned16(x_int8)) return TQ_ERR_ALIGN;
    a.xblk = (n + 15) / 16;
  }
  int fam = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (n <= kDecodeMaxTokens && split_k <= 1 && a.xvec && !xblk && plan_decode(n, k, n_tr, n_tc, false).ok) {
    const DecodePlan d = plan_decode(n, k, n_tr, n_tc, false);
    fam = TQ_KERNEL_DECODE;
    if constexpr (DUMP) e = launch_decode<Bf16, false, true>(a, d, s);
    else e = (x_dtype == TQ_DTYPE_BF16) ? launch_decode<Bf16, false>(a, d, s) : launch_decode<Fp16, false>(a, d, s);
  } else if (n <= kDecodeMaxTokens) {
    SplitPlan p = plan_split(n, n_tr, n_tc, split_k);
    rc = resolve_plan(p, n, n_tr, split_k, workspace, workspace_elems);
    if (rc) return rc;
    fam = xblk ? TQ_KERNEL_SPLITK_TOKEN_BLOCKED : TQ_KERNEL_SPLITK;
    if constexpr (DUMP) e = launch_split<Bf16, false, true>(a, p, workspace, s);
    else e = (x_dtype == TQ_DTYPE_BF16) ? launch_split<Bf16, false>(a, p, workspace, s)
                                        : launch_split<Fp16, false>(a, p, workspace, s);
  } else {
    dim3 grid(n_tr, (n + kPfTokens - 1) / kPfTokens), block(kPfThreads);
    const int64_t v5_blocks = (int64_t)(units != nullptr ? n_units : (n_tr + 1) / 2) * ((n + kPfTokens - 1) / kPfTokens);
    const bool bf = DUMP || x_dtype == TQ_DTYPE_BF16;
    if (a.xvec && n_tc <= kP5MaxCols && (a.w16 == nullptr || a.xf != nullptr) && (int64_t)n_tr * n_tc < (1 << 22) &&
        v5_blocks < (1ll << 31)) {
      // DMA ring, 64 x 128 wave tiles, 16-bit tiles in the ring
      const int ntb = (n + kPfTokens - 1) / kPfTokens;
      dim3 g5(((n_tr + 1) / 2) * ntb, 1);
      if (units != nullptr) {
        a.units = units; a.n_units = n_units; a.n_first = n_first;
        g5 = dim3(n_units * ntb, 1);
      }
      fam = TQ_KERNEL_PREFILL_V5;
      if (bf) hipLaunchKernelGGL((gemm_prefill_v5_kernel<Bf16, DUMP>), g5, dim3(kP5Threads), 0, s, a);
      else hipLaunchKernelGGL(gemm_prefill_v5_kernel<Fp16>, g5, dim3(kP5Threads), 0, s, a);
    } else if (a.xvec && n_tc <= kP3MaxCols) {   // DMA path, two row tiles per workgroup
      const dim3 g3((n_tr + 1) / 2, (n + kPfTokens - 1) / kPfTokens);
      fam = TQ_KERNEL_PREFILL_V3;
      if (bf) hipLaunchKernelGGL((gemm_prefill_v3_kernel<Bf16, DUMP>), g3, dim3(kP3Threads), 0, s, a);
      else hipLaunchKernelGGL(gemm_prefill_v3_kernel<Fp16>, g3, dim3(kP3Threads), 0, s, a);
    } else if (a.xvec) {   // DMA path: whole 16-byte activation chunks, aligned rows
      fam = TQ_KERNEL_PREFILL_ASYNC;
      if (bf) hipLaunchKernelGGL((gemm_prefill_async_kernel<Bf16, kPfStages, DUMP>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((gemm_prefill_async_kernel<Fp16, kPfStages>), grid, block, 0, s, a);
    } else {
      fam = TQ_KERNEL_PREFILL_REGISTER;
      if (bf) hipLaunchKernelGGL((gemm_prefill_kernel<Bf16, DUMP>), grid, block, 0, s, a);
      else hipLaunchKernelGGL(gemm_prefill_kernel<Fp16>, grid, block, 0, s, a);
    }
    e = hipGetLastError();
  }
  if (kernel != nullptr) *kernel = fam;
  return (int)e;
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
  return gemm_mixed_rows<false>(x_int8, x_int8_stride_n, sx, int8_tiles, int8_scales, int8_tile_ids, int8_row_ptr,
                         x_fp, x_fp_stride_n, x_dtype, fp16_tiles, fp16_tile_ids, fp16_row_ptr, out,
                         out_stride_n, out_dtype, bias, n, m, k, n_tr, n_tc, split_k, tile_layout, workspace,
                         workspace_elems, nullptr, 0, 0, nullptr, 0, 0, nullptr, stream);
}

extern "C" int tq_gemm_mixed_rows_planned(const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx,
                                          const int8_t* int8_tiles, const float* int8_scales,
                                          const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                                          const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                                          const void* fp16_tiles, const int32_t* fp16_tile_ids,
                                          const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                                          int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                                          int n_tc, int split_k, int tile_layout, float* workspace,
                                          int64_t workspace_elems, const int32_t* prefill_units,
                                          int n_units, int n_first, void* stream) {
  return gemm_mixed_rows<false>(x_int8, x_int8_stride_n, sx, int8_tiles, int8_scales, int8_tile_ids, int8_row_ptr,
                         x_fp, x_fp_stride_n, x_dtype, fp16_tiles, fp16_tile_ids, fp16_row_ptr, out,
                         out_stride_n, out_dtype, bias, n, m, k, n_tr, n_tc, split_k, tile_layout, workspace,
                         workspace_elems, prefill_units, n_units, n_first, nullptr, 0, 0, nullptr, stream);
}

// Prefill work plan (host code).  Cost of a unit in ring steps of a pair's
// INT8 step: a fixed part for set-up and epilogue, one step per column where
// a row of the unit has an INT8 tile (a step that multiplies only one row
// costs 0.68: half the MFMAs and epilogue), and two half steps of 0.63 per
// 16-bit tile (weights measured on MI355X at 8192 tokens, K = 8192).  A pair
// far above the median pair (a row tile mostly in 16 bits) is split into its
// two row tiles when that shortens it: its workgroups would otherwise finish
// long after the rest.  Units stay in row order: dispatching the heavy units
// first measured no faster than splitting alone.
namespace {
constexpr double kCostFixed = 8.0, kCostInt8Pair = 1.0, kCostInt8Single = 0.68, kCost16Half = 0.63;
constexpr double kSplitAbove = 1.5;   // split pairs costing more than this x the median pair ...
constexpr double kSplitGain = 0.9;    // ... when each single row costs less than this x the pair
}

extern "C" int tq_gemm_prefill_plan(const int32_t* int8_row_ptr, const int32_t* int8_tile_ids,
                                    const int32_t* fp16_row_ptr, int n_tr, int n_tc, int32_t* units,
                                    int max_units, int* n_first) {
  if (int8_row_ptr == nullptr || units == nullptr || n_first == nullptr || n_tr < 1 || n_tc < 1 ||
      max_units < n_tr || n_tr >= kUnitSingle)
    return TQ_ERR_ARG;
  if (int8_row_ptr[n_tr] > 0 && int8_tile_ids == nullptr) return TQ_ERR_ARG;
  std::vector<uint8_t> rows8((size_t)n_tc);   // bit j: row r + j has an INT8 tile in this column
  std::vector<double> pair_cost, single_cost;
  for (int r = 0; r < n_tr; r += 2) {
    const int rows = r + 1 < n_tr ? 2 : 1;
    int n8[2] = {0, 0}, n16[2] = {0, 0};
    std::fill(rows8.begin(), rows8.end(), 0);
    for (int j = 0; j < rows; ++j) {
      const int rr = r + j;
      const int lo = int8_row_ptr[rr], hi = int8_row_ptr[rr + 1];
      if (hi < lo) return TQ_ERR_ARG;
      for (int q = lo; q < hi; ++q) {
        const int64_t c = (int64_t)int8_tile_ids[q] - (int64_t)rr * n_tc;
        if (c < 0 || c >= n_tc) return TQ_ERR_ARG;
        rows8[c] |= (uint8_t)(1 << j);
      }
      n8[j] = hi - lo;
      if (fp16_row_ptr != nullptr) {
        n16[j] = fp16_row_ptr[rr + 1] - fp16_row_ptr[rr];
        if (n16[j] < 0) return TQ_ERR_ARG;
      }
    }
    int both = 0, one = 0;
    for (int c = 0; c < n_tc; ++c) {
      both += rows8[c] == 3;
      one += rows8[c] == 1 || rows8[c] == 2;
    }
    pair_cost.push_back(kCostFixed + kCostInt8Pair * both + kCostInt8Single * one +
                        2 * kCost16Half * (n16[0] + n16[1]));
    for (int j = 0; j < 2; ++j)
      single_cost.push_back(kCostFixed + kCostInt8Single * n8[j] + 2 * kCost16Half * n16[j]);
  }
  std::vector<double> sorted(pair_cost);
  std::sort(sorted.begin(), sorted.end());
  const double median = sorted[sorted.size() / 2];
  int n = 0;
  bool split_any = false;
  for (size_t i = 0; i < pair_cost.size(); ++i) {
    const int r = (int)(2 * i);
    const bool two = r + 1 < n_tr;
    if (two && pair_cost[i] > kSplitAbove * median &&
        std::max(single_cost[2 * i], single_cost[2 * i + 1]) < kSplitGain * pair_cost[i]) {
      units[n++] = r | kUnitSingle;
      units[n++] = (r + 1) | kUnitSingle;
      split_any = true;
    } else {
      units[n++] = r;
    }
  }
  *n_first = 0;
  return split_any ? n : 0;   // 0: the plain pair order is the plan
}

// gemm_decode_kernel takes row tile r on workgroups b with b % 8 == r % 8:
// whole-tile workgroups (JBW 4) are unit = b = r, and one-j-block workgroups
// are dealt so that the four j-blocks of r run on XCD r % 8 when n_tr % 8 == 0
// (the identity order otherwise spreads them over four XCDs).
extern "C" int tq_gemm_l2_warm_ok(int n, int k, int n_tr, int n_tc) {
  if (n < 1 || n > kDecodeMaxTokens || n_tr < 1 || n_tc < 1 || k != 64 * n_tc) return 0;
  const DecodePlan d = plan_decode(n, k, n_tr, n_tc, false);
  return d.ok && (d.jbw == 4 || (n_tr & 7) == 0) ? 1 : 0;
}

constexpr int kDecLongRowTiles = 256;

extern "C" int tq_gemm_prefers_token_blocked(int n, int k, int n_tr, int n_tc) {
  if (n < 1 || n > kDecodeMaxTokens || n_tr < 1 || k != n_tc * 64) return 0;
  // 17..64 rows: the split-K kernel on token-blocked codes beats the
  // LDS-staged kernel wherever that one fits (Llama-3.2-3B projections at 32
  // tokens on MI355X: QKV 13.2 -> 9.7 us, O 8.9 -> 7.7, Gate/Up 17.1 -> 16.7);
  // up to 16 rows only where the codes do not fit the staged kernel's LDS
  // (kDecCodesMax), and for the long rows below.
  if (n > 16) return 1;
  // Rows of 256+ column tiles (k >= 16384): the split-K kernel at every row
  // count.  Measured on MI355X, Qwen2.5-7B Down (3584 x 18944, clustered keep10,
  // cold weights), staged -> split-K: 1 row 23.69 -> 21.85 us, 4 rows 25.68 ->
  // 22.30, 6 rows 26.21 -> 22.61, 12-16 rows within 0.1 us; k = 13824 (216
  // tiles) and below stay faster staged (Qwen2.5-14B Down at 4 rows 22.81 vs
  // 24.95).  Bitwise the same outputs either way.
  if (n_tc >= kDecLongRowTiles) return 1;
  return plan_decode(n, k, n_tr, n_tc, false).ok ? 0 : 1;
}

extern "C" int tq_linear_mixed_fused_max_tokens(int k) {
  const int n_tc = (k + 63) / 64;
  int n = kFusedMaxTokens;
  while (n > 0 && fused_lds_bytes(n, n_tc) > kFusedMaxLds) --n;
  return n;
}

template <bool DUMP>
static int linear_mixed_fused(const void* x_fp, int64_t x_fp_stride_n, int x_dtype, const int8_t* int8_tiles,
                              const float* int8_scales, const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                              const void* fp16_tiles, const int32_t* fp16_tile_ids, const int32_t* fp16_row_ptr,
                              void* out, int64_t out_stride_n, int out_dtype, const void* bias, int n, int m, int k,
                              int n_tr, int n_tc, int split_k, int tile_layout, float* workspace,
                              int64_t workspace_elems, int32_t* dump, int dump_r0, int dump_n, int* kernel,
                              void* stream) {
  int rc = check_gemm_common(n, m, k, n_tr, n_tc, x_dtype, out_dtype, tile_layout);
  if (rc) return rc;
  if (DUMP && x_dtype != TQ_DTYPE_BF16) return TQ_ERR_DTYPE;
  if (n > kFusedMaxTokens || fused_lds_bytes(n, n_tc) > kFusedMaxLds) return TQ_ERR_ARG;
  if (n == 0 || m == 0) return TQ_OK;
  if (out == nullptr || out_stride_n < m || int8_row_ptr == nullptr || x_fp == nullptr || x_fp_stride_n < k)
    return TQ_ERR_ARG;
  const bool has16 = fp16_tiles != nullptr && fp16_tile_ids != nullptr && fp16_row_ptr != nullptr;
  if (!aligned16(int8_tiles) || (has16 && !aligned16(fp16_tiles))) return TQ_ERR_ALIGN;
  if (DUMP && (dump == nullptr || dump_r0 < 0 || dump_n < 1 || dump_n > n - dump_r0)) return TQ_ERR_ARG;
  GemmArgs a{};
  a.w8 = int8_tiles; a.sw8 = int8_scales; a.ids8 = int8_tile_ids; a.rp8 = int8_row_ptr;
  a.xf = static_cast<const uint16_t*>(x_fp); a.ldx = x_fp_stride_n;
  a.w16 = has16 ? static_cast<const uint16_t*>(fp16_tiles) : nullptr;
  a.ids16 = fp16_tile_ids; a.rp16 = fp16_row_ptr;
  a.out = static_cast<uint16_t*>(out); a.ldo = out_stride_n;
  a.bias = static_cast<const uint16_t*>(bias);
  a.dump = dump; a.dump_r0 = dump_r0; a.dump_n = dump_n;
  a.n = n; a.m = m; a.k = k; a.n_tr = n_tr; a.n_tc = n_tc;
  a.out_bf16 = out_dtype == TQ_DTYPE_BF16;
  a.layout = tile_layout;
  a.xvec = (k == n_tc * 64 && (x_fp_stride_n % 8) == 0 && aligned16(x_fp)) ? 1 : 0;
  a.ovec = (a.ldo % 8) == 0 && aligned16(a.out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (split_k <= 1 && a.xvec && workspace != nullptr && ((uintptr_t)workspace & 15u) == 0) {
    const CoopPlan c = plan_coop(n, k, n_tr, n_tc);
    if (c.ok && workspace_elems >= coop_workspace_elems(n, k, n_tc)) {
      a.coop = reinterpret_cast<int32_t*>(workspace);
      a.coop_p = kCoopProducers;
      const int spin = g_coop_spin.load(std::memory_order_relaxed);
      a.coop_spin = spin >= 0 ? spin : kCoopSpin;
      a.xq = reinterpret_cast<int8_t*>(workspace + kCoopHead);
      a.ldq = k;
      a.sx = workspace + kCoopHead + (((int64_t)n * k + 15) / 16) * 4;
      if (kernel != nullptr) *kernel = TQ_KERNEL_DECODE_COOP;
      if constexpr (DUMP) e = launch_coop<Bf16, true>(a, c.d, s);
      else e = (x_dtype == TQ_DTYPE_BF16) ? launch_coop<Bf16>(a, c.d, s) : launch_coop<Fp16>(a, c.d, s);
      return (int)e;
    }
  }
  if (split_k <= 1 && a.xvec) {
    const DecodePlan h = plan_help(n, k, n_tr, n_tc);
    if (h.ok) {
      if constexpr (DUMP) e = launch_help<Bf16, true>(a, h, s);
      else e = (x_dtype == TQ_DTYPE_BF16) ? launch_help<Bf16>(a, h, s) : launch_help<Fp16>(a, h, s);
      if (e != hipErrorNotSupported) {   // not resident at once: the plain quantizing kernel below
        if (kernel != nullptr) *kernel = TQ_KERNEL_DECODE_QUANT_HELP;
        return (int)e;
      }
    }
  }
  if (split_k <= 1 && a.xvec && plan_decode(n, k, n_tr, n_tc, true).ok) {
    const DecodePlan d = plan_decode(n, k, n_tr, n_tc, true);
    if (kernel != nullptr) *kernel = TQ_KERNEL_DECODE_QUANT;
    if constexpr (DUMP) e = launch_decode<Bf16, true, true>(a, d, s);
    else e = (x_dtype == TQ_DTYPE_BF16) ? launch_decode<Bf16, true>(a, d, s) : launch_decode<Fp16, true>(a, d, s);
    return (int)e;
  }
  SplitPlan p = plan_split(n, n_tr, n_tc, split_k);
  rc = resolve_plan(p, n, n_tr, split_k, workspace, workspace_elems);
  if (rc) return rc;
  if (kernel != nullptr) *kernel = TQ_KERNEL_SPLITK_QUANT;
  if constexpr (DUMP) e = launch_split<Bf16, true, true>(a, p, workspace, s);
  else e = (x_dtype == TQ_DTYPE_BF16) ? launch_split<Bf16, true>(a, p, workspace, s)
                                      : launch_split<Fp16, true>(a, p, workspace, s);
  return (int)e;
}

extern "C" int64_t tq_linear_mixed_fused_workspace_elems(int n, int m, int k, int n_tr, int n_tc, int split_k) {
  if (n <= 0 || n_tr <= 0 || n_tc <= 0 || n > kDecodeMaxTokens) return 0;
  int64_t need = split_workspace_elems(plan_split(n, n_tr, n_tc, split_k), n, n_tr);
  (void)m;
  if (split_k <= 1 && n <= kFusedMaxTokens && fused_lds_bytes(n, n_tc) <= kFusedMaxLds && plan_coop(n, k, n_tr, n_tc).ok)
    need = std::max(need, coop_workspace_elems(n, k, n_tc));
  return need;
}

extern "C" void tq_test_set_coop_spin(int polls) { g_coop_spin.store(polls < 0 ? -1 : polls); }

extern "C" int tq_linear_mixed_fused(const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                                     const int8_t* int8_tiles, const float* int8_scales,
                                     const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                                     const void* fp16_tiles, const int32_t* fp16_tile_ids,
                                     const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                                     int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                                     int n_tc, int split_k, int tile_layout, float* workspace,
                                     int64_t workspace_elems, void* stream) {
  return linear_mixed_fused<false>(x_fp, x_fp_stride_n, x_dtype, int8_tiles, int8_scales, int8_tile_ids,
                                   int8_row_ptr, fp16_tiles, fp16_tile_ids, fp16_row_ptr, out, out_stride_n,
                                   out_dtype, bias, n, m, k, n_tr, n_tc, split_k, tile_layout, workspace,
                                   workspace_elems, nullptr, 0, 0, nullptr, stream);
}

extern "C" int tq_linear_forward(const tq_linear_desc* d) {
  if (d == nullptr) return TQ_ERR_ARG;
  if (d->fused)
    return tq_linear_mixed_fused(d->x, d->x_stride, d->x_dtype, d->int8_tiles, d->int8_scales, d->int8_tile_ids,
                                 d->int8_row_ptr, d->fp16_tiles, d->fp16_tile_ids, d->fp16_row_ptr, d->out,
                                 d->out_stride, d->out_dtype, d->bias, d->n, d->m, d->k, d->n_tr, d->n_tc, 0,
                                 d->tile_layout, d->workspace, d->workspace_elems, d->stream);
  const int rc = (d->tile_layout & TQ_XQ_TOKEN_BLOCKED)
                     ? tq_act_quant_token_blocked(d->x, d->x_stride, d->x_dtype, d->n, d->k, d->x_int8, d->sx, d->stream)
                     : tq_act_quant_fused(d->x, d->x_stride, 1, d->x_dtype, d->n, d->k, d->x_int8, d->k, d->sx,
                                          d->stream);
  if (rc != 0) return rc;
  return tq_gemm_mixed_rows(d->x_int8, d->k, d->sx, d->int8_tiles, d->int8_scales, d->int8_tile_ids, d->int8_row_ptr,
                            d->x, d->x_stride, d->x_dtype, d->fp16_tiles, d->fp16_tile_ids, d->fp16_row_ptr, d->out,
                            d->out_stride, d->out_dtype, d->bias, d->n, d->m, d->k, d->n_tr, d->n_tc, 0,
                            d->tile_layout, d->workspace, d->workspace_elems, d->stream);
}

extern "C" int tq_gemm_mixed_rows_products_i32(
    const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx, const int8_t* int8_tiles,
    const float* int8_scales, const int32_t* int8_tile_ids, const int32_t* int8_row_ptr, const void* x_fp,
    int64_t x_fp_stride_n, int x_dtype, const void* fp16_tiles, const int32_t* fp16_tile_ids,
    const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n, int out_dtype, const void* bias, int n, int m,
    int k, int n_tr, int n_tc, int split_k, int tile_layout, float* workspace, int64_t workspace_elems,
    const int32_t* prefill_units, int n_units, int n_first, int32_t* products, int row0, int rows, int* kernel,
    void* stream) {
  return gemm_mixed_rows<true>(x_int8, x_int8_stride_n, sx, int8_tiles, int8_scales, int8_tile_ids, int8_row_ptr,
                               x_fp, x_fp_stride_n, x_dtype, fp16_tiles, fp16_tile_ids, fp16_row_ptr, out,
                               out_stride_n, out_dtype, bias, n, m, k, n_tr, n_tc, split_k, tile_layout, workspace,
                               workspace_elems, prefill_units, n_units, n_first, products, row0, rows, kernel,
                               stream);
}

extern "C" int tq_linear_mixed_fused_products_i32(
    const void* x_fp, int64_t x_fp_stride_n, int x_dtype, const int8_t* int8_tiles, const float* int8_scales,
    const int32_t* int8_tile_ids, const int32_t* int8_row_ptr, const void* fp16_tiles, const int32_t* fp16_tile_ids,
    const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n, int out_dtype, const void* bias, int n, int m,
    int k, int n_tr, int n_tc, int split_k, int tile_layout, float* workspace, int64_t workspace_elems,
    int32_t* products, int row0, int rows, int* kernel, void* stream) {
  return linear_mixed_fused<true>(x_fp, x_fp_stride_n, x_dtype, int8_tiles, int8_scales, int8_tile_ids,
                                  int8_row_ptr, fp16_tiles, fp16_tile_ids, fp16_row_ptr, out, out_stride_n,
                                  out_dtype, bias, n, m, k, n_tr, n_tc, split_k, tile_layout, workspace,
                                  workspace_elems, products, row0, rows, kernel, stream);
}

// ---- measurement helper: a plain read of HBM --------------------------------
//
// Context for the decode GEMM's roofline: the time a kernel that does nothing
// but read the same number of bytes takes per launch, timed the same way
// (bench.py).  Each thread loads four 16-byte words, all in flight together
// (indexes past the end re-read the last word), and folds them into one word
// that is stored only if it equals a constant: the loads cannot be dropped and
// nothing is written in practice.  sink holds 256 words.
constexpr int kReadProbeThreads = 256;
constexpr int kReadProbeWords = 4;

__global__ void __launch_bounds__(kReadProbeThreads)
read_probe_kernel(const u32x4* __restrict__ p, int64_t n16, uint32_t* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * (kReadProbeThreads * kReadProbeWords) + threadIdx.x;
  u32x4 v[kReadProbeWords];
#pragma unroll
  for (int u = 0; u < kReadProbeWords; ++u) v[u] = p[min(base + (int64_t)u * kReadProbeThreads, n16 - 1)];
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < kReadProbeWords; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  if (x == 0x9e3779b9u) sink[blockIdx.x & 255] = x;
}

extern "C" int tq_read_probe(const void* data, int64_t bytes, uint32_t* sink, void* stream) {
  if (bytes < 0 || (bytes & 15) != 0) return TQ_ERR_ARG;
  if (bytes == 0) return TQ_OK;
  if (data == nullptr || sink == nullptr) return TQ_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(data) & 15) != 0) return TQ_ERR_ALIGN;
  const int64_t n16 = bytes / 16;
  const int64_t per_block = (int64_t)kReadProbeThreads * kReadProbeWords;
  const int64_t blocks = (n16 + per_block - 1) / per_block;
  if (blocks > 0x7fffffff) return TQ_ERR_ARG;
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)blocks), dim3(kReadProbeThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(data), n16, sink);
  return (int)hipGetLastError();
}
