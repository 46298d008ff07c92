// tq_attention.hip -- one-token (decode) attention over a static KV cache, gfx950.
//
// For batch b and query head h (kv head h / G, G = q_heads / kv_heads):
//   out[b, h, :] = softmax_t(scale * q[b, h, :] . k[b, t, h/G, :]) v[b, t, h/G, :],  t < seq_used[b]
// The cache is read only over its valid prefix, whose length lives on the
// device, so one captured launch serves every decode position -- the job of
// aten._flash_attention_forward(..., seqused_k=...) in the reference's graph
// decoder (src/runtime/graph_decode.py:56-71).
//
// Split-sequence schedule (flash decoding): workgroup (split s, b * kv_heads +
// kvh) takes keys [s * kChunk, (s + 1) * kChunk) for the G query heads sharing
// kv head kvh and writes a partial (running max m, sum l, unnormalised o[D])
// per query head; a second kernel merges the splits of each (b, h) in split
// order.  Splits past seq_used write m = -inf, l = 0.
//   QK: a wave covers 4 keys per step, 16 lanes per key row (16 bytes = 8
//       elements each, so each row is one coalesced 256-byte read); the 8-wide
//       partial dots are summed across the 16 lanes with DPP.
//   softmax: scores (pre-multiplied by scale * log2 e) in LDS, workgroup
//       max / exp2 / sum.
//   PV: same lane mapping over V; per-lane accumulators for G heads x 8
//       dimensions, reduced across the wave with ds_swizzle-free xor shuffles,
//       then across the 4 waves through LDS in wave order.
// Everything accumulates in fp32; results are bitwise reproducible.
#include "tq_common.h"

namespace tq {

constexpr int kAttnD = 128;        // head dimension served
constexpr int kAttnChunk = 256;    // keys per split
constexpr int kAttnThreads = 256;  // 4 waves
constexpr int kAttnMaxG = 8;       // query heads per kv head
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_sl, kv_sh;
  const int32_t* seq_used;
  uint16_t* out;
  int64_t o_sb, o_sh;
  float* part;       // [batch * q_heads][n_splits][D + 2]
  int batch, q_heads, kv_heads, G, max_len, n_splits;
  float scale_log2;  // scale * log2(e)
};

// sum over the 16 lanes of a DPP row (every lane receives the sum)
__device__ inline float row16_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
  return x;
}

template <class XT>
__device__ inline void unpack8(u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = XT::to_f32((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = XT::to_f32((uint16_t)(w[i] >> 16));
  }
}

template <class XT>
__global__ void __launch_bounds__(kAttnThreads)
attn_split_kernel(AttnArgs a) {
  __shared__ float sc[kAttnMaxG][kAttnChunk];        // scores, then probabilities
  __shared__ float wred[kAttnThreads / kWave][kAttnMaxG];
  __shared__ float opart[kAttnThreads / kWave][kAttnMaxG][kAttnD];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int s = blockIdx.x;
  const int b = blockIdx.y / a.kv_heads, kvh = blockIdx.y - (blockIdx.y / a.kv_heads) * a.kv_heads;
  const int G = a.G;
  const int len = min(max(a.seq_used[b], 0), a.max_len);
  const int key0 = s * kAttnChunk;
  const int kl = lane >> 4, ch = lane & 15;   // key within a step of 4, 8-element chunk

  // this lane's 8 query values of each head of the group
  float qv[kAttnMaxG][8];
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g) {
    if (g < G) {
      const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(kvh * G + g) * a.q_sh + ch * 8;
      unpack8<XT>(*reinterpret_cast<const u32x4*>(qp), qv[g]);
    }
  }

  const int64_t kv_base = (int64_t)b * a.kv_sb + (int64_t)kvh * a.kv_sh + ch * 8;
  // ---- QK: wave covers keys key0 + wave*64 + 4*i + kl
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int kloc = wave * 64 + 4 * i + kl;
    const int key = key0 + kloc;
    const bool valid = key < len;
    u32x4 kw = u32x4{0, 0, 0, 0};
    if (valid) kw = *reinterpret_cast<const u32x4*>(a.k + kv_base + (int64_t)key * a.kv_sl);
    float kf[8];
    unpack8<XT>(kw, kf);
#pragma unroll
    for (int g = 0; g < kAttnMaxG; ++g) {
      if (g < G) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qv[g][e], kf[e], d);
        d = row16_sum(d);
        if (ch == 0) sc[g][kloc] = valid ? d * a.scale_log2 : -INFINITY;
      }
    }
  }
  __syncthreads();

  // ---- softmax over the chunk: thread t owns key t
  float mloc[kAttnMaxG], lsum[kAttnMaxG];
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g) {
    if (g < G) {
      float m = sc[g][t];
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      if (lane == 0) wred[wave][g] = m;
    }
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g) {
    if (g < G) {
      float m = wred[0][g];
      for (int w = 1; w < kAttnThreads / kWave; ++w) m = fmaxf(m, wred[w][g]);
      mloc[g] = m;
    }
  }
  __syncthreads();   // wred is reused for the sums
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g) {
    if (g < G) {
      const float p = (mloc[g] == -INFINITY) ? 0.0f : exp2f(sc[g][t] - mloc[g]);
      sc[g][t] = p;
      float l = p;
      for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
      if (lane == 0) wred[wave][g] = l;
    }
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g) {
    if (g < G) {
      float l = wred[0][g];
      for (int w = 1; w < kAttnThreads / kWave; ++w) l += wred[w][g];
      lsum[g] = l;
    }
  }

  // ---- PV: same lane mapping, accumulate G heads x 8 dims per lane
  float o[kAttnMaxG][8];
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int kloc = wave * 64 + 4 * i + kl;
    const int key = key0 + kloc;
    u32x4 vw = u32x4{0, 0, 0, 0};
    if (key < len) vw = *reinterpret_cast<const u32x4*>(a.v + kv_base + (int64_t)key * a.kv_sl);
    float vf[8];
    unpack8<XT>(vw, vf);
#pragma unroll
    for (int g = 0; g < kAttnMaxG; ++g) {
      if (g < G) {
        const float p = sc[g][kloc];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(p, vf[e], o[g][e]);
      }
    }
  }
  // reduce the 4 keys-per-step lanes (lane, lane^16, lane^32, lane^48) in a fixed order
#pragma unroll
  for (int g = 0; g < kAttnMaxG; ++g) {
    if (g < G) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = o[g][e];
        x += __shfl_xor(x, 16);
        x += __shfl_xor(x, 32);
        if (kl == 0) opart[wave][g][ch * 8 + e] = x;
      }
    }
  }
  __syncthreads();
  // partial record per query head: o[D], m, l (m in log2 units of the scaled score)
  for (int e = t; e < G * kAttnD; e += kAttnThreads) {
    const int g = e / kAttnD, d = e - g * kAttnD;
    float x = opart[0][g][d];
    for (int w = 1; w < kAttnThreads / kWave; ++w) x += opart[w][g][d];
    const int h = kvh * G + g;
    float* rec = a.part + ((int64_t)(b * a.q_heads + h) * a.n_splits + s) * (kAttnD + 2);
    rec[d] = x;
    if (d == 0) {
      rec[kAttnD] = mloc[g];
      rec[kAttnD + 1] = lsum[g];
    }
  }
}

template <class XT>
__global__ void __launch_bounds__(kAttnD)
attn_merge_kernel(AttnArgs a) {
  const int bh = blockIdx.x, d = threadIdx.x;
  const int b = bh / a.q_heads, h = bh - (bh / a.q_heads) * a.q_heads;
  const float* rec = a.part + (int64_t)bh * a.n_splits * (kAttnD + 2);
  float M = -INFINITY;
  for (int s = 0; s < a.n_splits; ++s) M = fmaxf(M, rec[(int64_t)s * (kAttnD + 2) + kAttnD]);
  float L = 0.0f, acc = 0.0f;
  for (int s = 0; s < a.n_splits; ++s) {
    const float* r = rec + (int64_t)s * (kAttnD + 2);
    const float m = r[kAttnD];
    if (m == -INFINITY) continue;
    const float w = exp2f(m - M);
    L = fmaf(w, r[kAttnD + 1], L);
    acc = fmaf(w, r[d], acc);
  }
  const float y = L > 0.0f ? acc / L : 0.0f;
  a.out[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d] = XT::from_f32(y);
}

static int attn_splits(int max_len) { return (max_len + kAttnChunk - 1) / kAttnChunk; }

}  // namespace tq

using namespace tq;

extern "C" int64_t tq_decode_attention_workspace_elems(int batch, int q_heads, int max_len) {
  if (batch <= 0 || q_heads <= 0 || max_len <= 0) return 0;
  return (int64_t)batch * q_heads * attn_splits(max_len) * (kAttnD + 2);
}

extern "C" int tq_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                   const void* v, int64_t kv_stride_b, int64_t kv_stride_l,
                                   int64_t kv_stride_h, const int32_t* seq_used, void* out,
                                   int64_t out_stride_b, int64_t out_stride_h, int dtype, int batch,
                                   int q_heads, int kv_heads, int head_dim, int max_len, float scale,
                                   float* workspace, int64_t workspace_elems, void* stream) {
  if (dtype != TQ_DTYPE_BF16 && dtype != TQ_DTYPE_FP16) return TQ_ERR_DTYPE;
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || max_len < 0) return TQ_ERR_ARG;
  if (head_dim != kAttnD || q_heads % kv_heads != 0 || q_heads / kv_heads > kAttnMaxG) return TQ_ERR_ARG;
  if (batch == 0 || max_len == 0) return TQ_OK;
  if (!q || !k || !v || !seq_used || !out) return TQ_ERR_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (q_stride_b % 8) || (q_stride_h % 8) ||
      (kv_stride_b % 8) || (kv_stride_l % 8) || (kv_stride_h % 8))
    return TQ_ERR_ALIGN;
  if (workspace == nullptr || workspace_elems < tq_decode_attention_workspace_elems(batch, q_heads, max_len))
    return TQ_ERR_WORKSPACE;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.k = static_cast<const uint16_t*>(k); a.v = static_cast<const uint16_t*>(v);
  a.kv_sb = kv_stride_b; a.kv_sl = kv_stride_l; a.kv_sh = kv_stride_h;
  a.seq_used = seq_used;
  a.out = static_cast<uint16_t*>(out); a.o_sb = out_stride_b; a.o_sh = out_stride_h;
  a.part = workspace;
  a.batch = batch; a.q_heads = q_heads; a.kv_heads = kv_heads; a.G = q_heads / kv_heads;
  a.max_len = max_len; a.n_splits = attn_splits(max_len);
  a.scale_log2 = scale * kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g1(a.n_splits, batch * kv_heads), g2(batch * q_heads);
  if (dtype == TQ_DTYPE_BF16) {
    hipLaunchKernelGGL(attn_split_kernel<Bf16>, g1, dim3(kAttnThreads), 0, s, a);
    hipLaunchKernelGGL(attn_merge_kernel<Bf16>, g2, dim3(kAttnD), 0, s, a);
  } else {
    hipLaunchKernelGGL(attn_split_kernel<Fp16>, g1, dim3(kAttnThreads), 0, s, a);
    hipLaunchKernelGGL(attn_merge_kernel<Fp16>, g2, dim3(kAttnD), 0, s, a);
  }
  return (int)hipGetLastError();
}
