// tq_common.h -- shared device helpers for the TileQuant gfx950 kernels.
//
// Everything here is written for CDNA4 (gfx950, wave64).  16-bit floating
// point data is carried as raw uint16_t bit patterns in memory and widened
// to fp32 in registers; the MFMA builtins take 8-element vectors of __bf16 /
// _Float16 that are bit-cast from 16-byte loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tilequant.h"

namespace tq {

constexpr int kTile = 64;          // tile edge (rows and columns)
constexpr int kWave = 64;          // gfx950 wavefront size

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- 16-bit float <-> fp32 ---------------------------------------------

struct Bf16 {
  static constexpr int kDtype = TQ_DTYPE_BF16;
  __device__ static inline float to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
  // round-half-even to bf16, NaN quieted ((bits >> 16) | 0x40): gfx950's
  // v_cvt_pk_bf16_f32, which matches that rule bit for bit (checked on
  // hardware over ties, subnormals, infinities, NaN payloads and 2^20
  // random patterns)
  __device__ static inline uint16_t from_f32(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{lo, hi}), bf2));
  }
  __device__ static inline float round(float f) { return to_f32(from_f32(f)); }
};

struct Fp16 {
  static constexpr int kDtype = TQ_DTYPE_FP16;
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
  // v_cvt_f16_f32 rounds to nearest-even in the default mode (IEEE
  // overflow to inf, subnormals kept: fp16 denormals are on for gfx9).
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return (uint32_t)from_f32(lo) | ((uint32_t)from_f32(hi) << 16);
  }
  __device__ static inline float round(float f) { return to_f32(from_f32(f)); }
};

// 16x16x32 MFMA on 16-bit operands (8 per lane: row / column lane % 16, k
// 8 (lane / 16) .. + 7), fp32 accumulators; D[4 (lane / 16) + v][lane % 16].
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

// ---- quantization closed forms -----------------------------------------

// Activation scale of one 64-column tile from its absmax a (already |x| max,
// exact in the 16-bit input type): 1 when a == 0, else the input dtype's
// nearest value to f32(a) / 127 (IEEE divide), widened back to fp32.
template <class T>
__device__ inline float act_scale_from_absmax(float a) {
  return (a > 0.0f) ? T::round(a / 127.0f) : 1.0f;
}

// max(min(rint(v / s), 127), -127) with an IEEE divide and half-even rint.
// min/max ignore a NaN operand, so 0/0 (a zero scale) yields 127.
__device__ inline int quant_code(float v, float s) {
  float q = __builtin_rintf(v / s);
  q = fmaxf(fminf(q, 127.0f), -127.0f);
  return (int)q;
}

// Codes of a whole tile share one scale s: q = rint(v * (1/s)) equals
// rint(fl(v / s)) for 16-bit v and s except when v / s is exactly a
// half-integer k + 0.5 (then the product may land on either side).  Proof
// sketch: v = a*2^e, s = b*2^f with integer a, b < 2^11, so a quotient that is
// not a half-integer is at least 1/(2*2047) from every half-integer within
// the clamp range (|v/s| <= 128), while two roundings move the product by at
// most 128 * 2^-23 = 2^-16.  An exact half is detected exactly with one fma:
// h = floor(t) + 0.5 and h*s are exact (<= 19 significant bits), so
// fma(-h, s, v) == 0 iff v == h*s; rint(h) then rounds half to even like the
// reference.  Subnormal scales (1/s overflows) take the IEEE divide.
struct CodeScale {
  float s, rcp;
  bool exact_div;
  __device__ explicit CodeScale(float scale)
      : s(scale), rcp(1.0f / scale), exact_div(!(scale >= 1.1754943508222875e-38f)) {}
  // with rcp == 1.0f / scale computed elsewhere (IEEE divide)
  __device__ CodeScale(float scale, float recip)
      : s(scale), rcp(recip), exact_div(!(scale >= 1.1754943508222875e-38f)) {}
  // Normal scales only (!exact_div).  q is never NaN here, so the clamp is
  // a single v_med3_f32.
  __device__ inline int code_fast(float v) const {
    const float t = v * rcp;
    const float h = __builtin_floorf(t) + 0.5f;
    const float q = (__builtin_fmaf(-h, s, v) == 0.0f) ? __builtin_rintf(h) : __builtin_rintf(t);
    return (int)__builtin_amdgcn_fmed3f(q, -127.0f, 127.0f);
  }
  __device__ inline int code(float v) const { return exact_div ? quant_code(v, s) : code_fast(v); }
};

// 8 consecutive 16-bit values packed in a 16-byte word: absmax and codes.
template <class T>
__device__ inline float max8(u32x4 w, float m) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m = fmaxf(m, fabsf(T::to_f32((uint16_t)(w[i] & 0xffffu))));
    m = fmaxf(m, fabsf(T::to_f32((uint16_t)(w[i] >> 16))));
  }
  return m;
}

template <class T, bool EXACT>
__device__ inline u32x2 codes8_impl(u32x4 w, const CodeScale& s) {
  u32x2 out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t word = w[h * 2 + i];
      const float a = T::to_f32((uint16_t)(word & 0xffffu)), b = T::to_f32((uint16_t)(word >> 16));
      const uint32_t lo = (uint32_t)((EXACT ? quant_code(a, s.s) : s.code_fast(a)) & 0xff);
      const uint32_t hi = (uint32_t)((EXACT ? quant_code(b, s.s) : s.code_fast(b)) & 0xff);
      packed |= (lo | (hi << 8)) << (16 * i);
    }
    out[h] = packed;
  }
  return out;
}

// One branch per 8 values (the scale is shared): the IEEE-divide path only for
// subnormal scales.
template <class T>
__device__ inline u32x2 codes8(u32x4 w, const CodeScale& s) {
  return s.exact_div ? codes8_impl<T, true>(w, s) : codes8_impl<T, false>(w, s);
}

// ---- wave reductions ----------------------------------------------------

// Max over the 64 lanes of a NON-NEGATIVE float (absolute values): integer
// order of the bit patterns is float order, so DPP row operations (quad
// swaps, half-row and row mirrors) reduce each 16-lane row in registers and
// four v_readlane finish in scalar registers -- no LDS round trips.
__device__ inline float wave_max_nonneg(float x) {
  uint32_t v = __float_as_uint(x);
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
  return __uint_as_float(max(max(a, b), max(c, d)));
}

__device__ inline float wave_max(float v) { return wave_max_nonneg(v); }

// Block-wide max over `nwaves` waves through a small LDS array; every thread
// receives the result.  `red` must hold at least nwaves floats.
__device__ inline float block_max(float v, float* red, int nwaves) {
  v = wave_max(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < nwaves; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

// Raw buffer resource over `bytes` bytes at p (stride 0): loads at offsets >=
// bytes return 0 and touch no memory.  Word 3 = 0x00020000 is the gfx9-family
// descriptor format (32-bit data format, no swizzle).
__device__ inline __amdgpu_buffer_rsrc_t row_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

__host__ __device__ inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---- L2 warm-up of the next decode GEMM's weights -------------------------
// A producer kernel launched with `blocks` extra workgroups after its own
// `first` ones hands those to l2_warm_rows.  Workgroups are dealt to the 8
// XCDs round-robin by id, so workgroup b runs on XCD b % 8; the decode GEMM
// reads row tile r only from XCD r % 8.  The blocks / 8 warm-up workgroups of
// an XCD split each of that XCD's row tiles (r = XCD + 8 j) into equal
// 64-byte-aligned shares, and every lane reads one dword of each 64-byte
// sector of its share with an LDS DMA load (global_load_lds_dword) into a
// 256-byte sink: nothing is kept in registers, so the loads of all rows go
// out back to back and the workgroup waits once, at its end.  Each lane's
// offset is checked against its share (global loads have no range check).
struct L2Warm {
  const int8_t* w8;
  const int8_t* w16;
  const int32_t* rp8;
  const int32_t* rp16;
  int n_tr, blocks, first;
};

template <int NT>
__device__ __attribute__((always_inline)) inline void l2_warm_span(const int8_t* base, int64_t lo, int64_t hi,
                                                                   uint32_t* sink) {
  for (int64_t o = lo + (int64_t)threadIdx.x * 64; o < hi; o += (int64_t)NT * 64)
    __builtin_amdgcn_global_load_lds(base + o, sink, 4, 0, 0);
}

// NT: the producer's threads per workgroup.  sink: 256 bytes of LDS (64
// dwords), shared by all waves (the data is never read).  The row ranges of
// up to 64 row tiles come with one vector load per pointer array (lane j: row
// XCD + 8 j) before any DMA load is issued, so waiting for them never waits
// for the DMA loads of earlier rows.
template <int NT>
__device__ __attribute__((always_inline)) inline void l2_warm_rows(const L2Warm& w, uint32_t* sink) {
  const int p = (int)blockIdx.x - w.first;
  const int xcd = blockIdx.x & 7, slot = p >> 3, per = w.blocks >> 3;
  const int lane = threadIdx.x & 63;
  const int32_t* rp16 = w.w16 != nullptr ? w.rp16 : w.rp8;
  for (int r0 = xcd; r0 < w.n_tr; r0 += 8 * 64) {
    const int rl = min(r0 + 8 * lane, w.n_tr - 1);
    const int lo8v = w.rp8[rl], hi8v = w.rp8[rl + 1], lo16v = rp16[rl], hi16v = rp16[rl + 1];
    const int nrows = min(64, (w.n_tr - r0 + 7) / 8);
    for (int j = 0; j < nrows; ++j) {
      const int lo8 = __builtin_amdgcn_readlane(lo8v, j), hi8 = __builtin_amdgcn_readlane(hi8v, j);
      // shares counted in 64-byte sectors (64 per INT8 tile, 128 per 16-bit
      // tile: below 2^27 for any row of fewer than 2^20 column tiles)
      const uint32_t u8 = (uint32_t)(hi8 - lo8) * 64u, q8 = (u8 + per - 1) / (uint32_t)per;
      l2_warm_span<NT>(w.w8 + (int64_t)lo8 * 4096, (int64_t)slot * q8 * 64,
                       (int64_t)min(u8, (uint32_t)(slot + 1) * q8) * 64, sink);
      if (w.w16 != nullptr) {
        const int lo16 = __builtin_amdgcn_readlane(lo16v, j), hi16 = __builtin_amdgcn_readlane(hi16v, j);
        const uint32_t u16 = (uint32_t)(hi16 - lo16) * 128u, q16 = (u16 + per - 1) / (uint32_t)per;
        l2_warm_span<NT>(w.w16 + (int64_t)lo16 * 8192, (int64_t)slot * q16 * 64,
                         (int64_t)min(u16, (uint32_t)(slot + 1) * q16) * 64, sink);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Host: the kernel-side form of a tq_l2_warm (blocks 0 when absent), after
// checking it; `first` is the producer's own workgroup count.
inline int l2_warm_args(const tq_l2_warm* in, int first, L2Warm& out) {
  out = L2Warm{nullptr, nullptr, nullptr, nullptr, 0, 0, first};
  if (in == nullptr || in->blocks == 0) return TQ_OK;
  if (in->blocks < 0 || in->blocks > 1024 || (in->blocks & 7) != 0 || in->n_tr <= 0 || in->int8_row_ptr == nullptr ||
      (in->fp16_tiles != nullptr && in->fp16_row_ptr == nullptr))
    return TQ_ERR_ARG;
  out.w8 = static_cast<const int8_t*>(in->int8_tiles);
  out.w16 = static_cast<const int8_t*>(in->fp16_tiles);
  out.rp8 = in->int8_row_ptr;
  out.rp16 = in->fp16_row_ptr;
  out.n_tr = in->n_tr;
  out.blocks = in->blocks;
  return TQ_OK;
}

// Kernel arguments into SGPRs at kernel entry, all in one scalar round trip:
// TQ_ARGS_IN_SGPRS("s"(a.x), "s"(a.n), ...).  Left alone, the compiler loads
// each argument just before its first use, so a uniform branch or an early
// return between two uses puts a whole scalar memory round trip in front of
// the kernel's first vector load (the decode glue kernels paid two or three
// of them).
#define TQ_ARGS_IN_SGPRS(...) asm volatile("" ::__VA_ARGS__)

// Workgroup barrier for LDS hand-offs that leaves outstanding global loads in
// flight: waits only for this wave's LDS operations (lgkmcnt(0); vmcnt and
// expcnt at their maxima in the gfx9 s_waitcnt encoding), then s_barrier.
// __syncthreads() would also wait for every outstanding global load
// (vmcnt(0)), serialising prefetched weight streams behind the barrier.  The
// "memory" clobber keeps the compiler from moving memory operations across.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("s_barrier" ::: "memory");
}

}  // namespace tq

// Host-side error plumbing shared by the C-ABI entry points.
#define TQ_RETURN_IF_HIP_ERROR(expr)                 \
  do {                                               \
    hipError_t tq_err_ = (expr);                     \
    if (tq_err_ != hipSuccess) return (int)tq_err_;  \
  } while (0)
