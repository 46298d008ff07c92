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
  // round-half-even to bf16; NaN stays a quiet NaN
  __device__ static inline uint16_t from_f32(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
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
  __device__ static inline float round(float f) { return to_f32(from_f32(f)); }
};

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

// ---- wave reductions ----------------------------------------------------

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

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

__host__ __device__ inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace tq

// Host-side error plumbing shared by the C-ABI entry points.
#define TQ_RETURN_IF_HIP_ERROR(expr)                 \
  do {                                               \
    hipError_t tq_err_ = (expr);                     \
    if (tq_err_ != hipSuccess) return (int)tq_err_;  \
  } while (0)
