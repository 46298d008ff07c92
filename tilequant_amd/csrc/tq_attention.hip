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
// kvh) takes keys [s C, (s + 1) C) of the sequence's seq_used[b] keys, C =
// ceil(seq_used[b] / n_splits) <= 32 W (W waves of 32 keys; n_splits and W
// from a host plan that gives every CU the same share), for the G query heads
// sharing kv head kvh, and writes a partial (running max m, sum l,
// unnormalised o[D]) per query head; a second kernel merges the splits of
// each (b, h) in split order.  Empty splits write m = -inf, l = 0.
//   loads: all K rows of a wave's 32 keys are issued at entry (8 16-byte
//       loads per lane), its V rows (8 more) right after the QK MFMAs.
//   QK on the matrix cores: per 16-key block, 4 v_mfma_f32_16x16x32 with the
//       keys as A rows and the G query heads as B columns; each A operand is a
//       plain 16-byte load of a key row.  The kernel is VALU-bound once its
//       data has arrived, and this replaces 8 dot2 + 8 DPP adds per (key,
//       head) group of lanes.
//   softmax per wave: a lane holds 8 scores of one head; max and sum over
//       them, then over the head's 4 lanes (gfx950 v_permlane16_swap /
//       v_permlane32_swap).  The probabilities go through LDS ([head][key],
//       within the wave) to the PV layout: a lane takes 8 keys x 8 dimensions
//       of the value rows, fp32 FMAs; the 4 key groups of a wave are summed
//       with the same butterflies.
//   the W waves' partials (max, sum, o) are combined through LDS in wave
//       order, rescaled to the chunk max, with one barrier.
// Everything accumulates in fp32; results are bitwise reproducible.
//
// RoPE form (tq_decode_attention_rope): the split kernel reads q from the
// stacked q/k/v projection output and applies RoPE itself, each (head, 8-element
// chunk) once, shared through LDS; the workgroup whose chunk holds the new
// position (the last split when the position is past seq_used) writes that
// token's rotated k and its v into the caches and substitutes them for the
// rows it loaded before writing.  This replaces a separate RoPE + cache-write
// launch per layer, bit for bit.
#include "tq_common.h"

#include <atomic>

namespace tq {

constexpr int kAttnD = 128;            // head dimension served
constexpr int kAttnKeysPerWave = 32;   // keys per wave of the split kernel
constexpr int kAttnMaxWaves = 4;       // waves per split workgroup (2..4)
constexpr int kAttnMaxG = 8;           // query heads per kv head
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
  int waves;         // waves per split workgroup
  float scale_log2;  // scale * log2(e)
  // RoPE-fused form: q (= qkv rows) is the raw stacked projection output
  // [batch, (q_heads + 2 kv_heads) * D] with row stride q_sb; the new token's
  // rotated k and raw v go to the caches at *pos.
  const uint16_t* cos;   // [max_len, D] tables; row *pos (clamped into the table) is used
  const uint16_t* sin;
  const int64_t* pos;
  uint16_t* k_out;       // the k / v caches, writable
  uint16_t* v_out;
};

// RoPE of one 8-element chunk (HF apply_rotary_pos_emb: q * cos +
// rotate_half(q) * sin, each product and the sum rounded to the 16-bit type):
// own = elements 8ch .. 8ch+7 of the head, partner = those of chunk ch ^ 8
// (d +- 64); the first half subtracts partner * sin, the second adds it.
template <class XT>
__device__ inline u32x4 rope8(u32x4 own, u32x4 partner, u32x4 c, u32x4 sn, bool first_half) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float x = XT::to_f32((uint16_t)(own[i] >> (16 * j)));
      const float y = XT::to_f32((uint16_t)(partner[i] >> (16 * j)));
      const float cc = XT::to_f32((uint16_t)(c[i] >> (16 * j)));
      const float ss = XT::to_f32((uint16_t)(sn[i] >> (16 * j)));
      const float o = XT::round(XT::round(x * cc) + XT::round((first_half ? -y : y) * ss));
      w |= (uint32_t)XT::from_f32(o) << (16 * j);
    }
    r[i] = w;
  }
  return r;
}

// sum over the 16 lanes of a DPP row (every lane receives the sum)
__device__ inline float row16_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
  return x;
}

// Sum / max over the 4 rows of 16 lanes (lanes l, l^16, l^32, l^48), the
// same value and the same association ((r0 o r1) o (r2 o r3)) in every lane.
__device__ inline float rows4_sum(float x) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const unsigned b = __float_as_uint(x);
  u2 r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const unsigned c = __float_as_uint(x);
  r = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float rows4_max(float x) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const unsigned b = __float_as_uint(x);
  u2 r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const unsigned c = __float_as_uint(x);
  r = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Dot product of 8 packed 16-bit values with an fp32 accumulator, two
// products per v_dot2 instruction (exact products, fp32 sums) -- half the
// instructions of unpacking both operands and chaining fmas.
template <class XT>
__device__ inline float dot8(u32x4 x, u32x4 y, float acc) {
  if constexpr (std::is_same<XT, Bf16>::value) {
    const v8bf xv = __builtin_bit_cast(v8bf, x), yv = __builtin_bit_cast(v8bf, y);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(xv, xv, 0, 1), __builtin_shufflevector(yv, yv, 0, 1), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(xv, xv, 2, 3), __builtin_shufflevector(yv, yv, 2, 3), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(xv, xv, 4, 5), __builtin_shufflevector(yv, yv, 4, 5), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(xv, xv, 6, 7), __builtin_shufflevector(yv, yv, 6, 7), acc, false);
  } else {
    const v8h xv = __builtin_bit_cast(v8h, x), yv = __builtin_bit_cast(v8h, y);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(xv, xv, 0, 1), __builtin_shufflevector(yv, yv, 0, 1), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(xv, xv, 2, 3), __builtin_shufflevector(yv, yv, 2, 3), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(xv, xv, 4, 5), __builtin_shufflevector(yv, yv, 4, 5), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(xv, xv, 6, 7), __builtin_shufflevector(yv, yv, 6, 7), acc, false);
  }
  return acc;
}

template <class XT>
__device__ inline void unpack8(u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = XT::to_f32((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = XT::to_f32((uint16_t)(w[i] >> 16));
  }
}

template <class XT, int G, bool ROPE, int W>
__global__ void __launch_bounds__(W * kWave)
attn_split_kernel(AttnArgs a) {
  constexpr int kWaves = W;
  constexpr int kThreads = W * kWave;
  constexpr int kKeysW = kAttnKeysPerWave;      // keys per wave: two 16-key MFMA blocks
  constexpr int kSteps = kKeysW / 4;            // PV: 8 keys per lane
  static_assert(kKeysW == 32 && G <= 16, "two 16-key blocks per wave, at most 16 query heads");
  static_assert(!ROPE || 16 * (G + 2) <= kThreads, "the RoPE prologue needs 16 (G + 2) threads");
  // per-wave unnormalised o; for G <= 4 per key group kl as well (summed in
  // the combine instead of by cross-lane butterflies in every wave)
  constexpr bool kLdsSum = G <= 4;
  constexpr int KG = kLdsSum ? 4 : 1;
  __shared__ __align__(16) float wo[kWaves][KG][G][kAttnD];
  __shared__ float wml[kWaves][G][2];       // per-wave max, sum
  __shared__ __align__(16) float pl[kWaves][G][kKeysW];   // per-wave probabilities [head][key]
  TQ_ARGS_IN_SGPRS("s"(a.q), "s"(a.q_sb), "s"(a.q_sh), "s"(a.k), "s"(a.v), "s"(a.kv_sb), "s"(a.kv_sl),
                   "s"(a.kv_sh), "s"(a.seq_used), "s"(a.part), "s"(a.q_heads), "s"(a.kv_heads), "s"(a.max_len),
                   "s"(a.n_splits), "s"(a.scale_log2));
  if constexpr (ROPE) TQ_ARGS_IN_SGPRS("s"(a.cos), "s"(a.sin), "s"(a.pos), "s"(a.k_out), "s"(a.v_out));
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int s = blockIdx.x;
  const int b = blockIdx.y / a.kv_heads, kvh = blockIdx.y - (blockIdx.y / a.kv_heads) * a.kv_heads;
  const int len = min(max(a.seq_used[b], 0), a.max_len);
  // this split's keys: [key0, hi), the sequence cut into n_splits chunks of
  // C <= 32 W keys (so every split has work and the CUs get equal shares)
  const int C = max(1, (len + a.n_splits - 1) / a.n_splits);
  const int key0 = s * C, hi = min(key0 + C, len);
  const int wkey0 = key0 + wave * kKeysW;
  const int kl = lane >> 4, ch = lane & 15;   // PV layout: keys 8 kl .. 8 kl + 7, 8-element chunk ch
  const int mr = lane & 15, mg = lane >> 4;   // MFMA layout: row / column index, k group

  // ---- the loads go out up front: q, then all K rows of this wave's keys
  //      (keys past the valid length are not read); the V rows after the QK.
  //      MFMA step ks covers dimensions 32 ks .. 32 ks + 31: lane (mr, mg)
  //      holds chunk 4 ks + mg of key mr of a 16-key block (A operand) and of
  //      query head mr (B operand; columns >= G repeat head G - 1, unused).
  u32x4 qa[4];
  if constexpr (!ROPE) {
    const int hq = kvh * G + min(mr, G - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qa[ks] = *reinterpret_cast<const u32x4*>(a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh + (4 * ks + mg) * 8);
  }
  // RoPE form: thread t < 16 (G + 2) owns chunk ich of item it -- query head
  // g < G, the new token's k (it = G) or v (it = G + 1) -- and loads that
  // chunk, its RoPE partner chunk ich ^ 8 and the cos / sin table rows at the
  // position (read in the same scalar round trip as seq_used, so the K/V and
  // table loads go out together).  Each (item, chunk) is rotated once and
  // shared through LDS (every lane needs several of them).
  __shared__ u32x4 rq[ROPE ? G + 2 : 1][16];
  const int it = t >> 4, ich = t & 15;
  u32x4 own{}, partner{}, cw{}, sw{};
  int64_t pos = -1;
  if constexpr (ROPE) {
    pos = a.pos[0];
    const int64_t trow = min(max(pos, (int64_t)0), (int64_t)a.max_len - 1) * kAttnD;
    if (it < G + 2) {
      const uint16_t* row = a.q + (int64_t)b * a.q_sb;
      const int64_t head = it < G ? (int64_t)(kvh * G + it) * a.q_sh
                                  : (int64_t)(a.q_heads + (it - G) * a.kv_heads + kvh) * kAttnD;
      own = *reinterpret_cast<const u32x4*>(row + head + ich * 8);
      if (it <= G) {
        partner = *reinterpret_cast<const u32x4*>(row + head + (ich ^ 8) * 8);
        cw = *reinterpret_cast<const u32x4*>(a.cos + trow + ich * 8);
        sw = *reinterpret_cast<const u32x4*>(a.sin + trow + ich * 8);
      }
    }
  }
  // K/V rows through buffer resources spanning the valid prefix of this
  // (b, kv head): keys past seq_used read as 0 without touching memory, so
  // every load is unconditional and all of them stay in flight together.
  const int64_t kv_base = (int64_t)b * a.kv_sb + (int64_t)kvh * a.kv_sh;
  const int span = len > 0 ? (int)(((int64_t)(len - 1) * a.kv_sl + kAttnD) * 2) : 0;
  const __amdgpu_buffer_rsrc_t krs = row_rsrc(a.k + kv_base, span);
  const __amdgpu_buffer_rsrc_t vrs = row_rsrc(a.v + kv_base, span);
  // a key past the prefix gets an offset past the span (rows are not always packed: kv_sl >= D)
  auto kv_off = [&](int key, int chunk) { return key < hi ? (int)(((int64_t)key * a.kv_sl + chunk * 8) * 2) : span; };
  u32x4 kb[2][4], vw[kSteps];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kb[blk][ks] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  krs, kv_off(wkey0 + 16 * blk + mr, 4 * ks + mg), 0, 0));
  __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the first use

  // RoPE form: the workgroup whose chunk holds the new position writes the
  // token's rotated k and its v into the caches (the bytes tq_rope_cache
  // writes) and uses them in registers for that key (pk; -1 elsewhere): its
  // own cache rows were loaded before they were written.  The new key's
  // scores come from MFMAs of their own and replace that key's scores by a
  // per-lane select, so no wait for the other rows.
  u32x4 kn[4], vnw{};
  int pk = -1;
  if constexpr (ROPE) {
    // the split whose chunk holds the position (the last one past the length)
    const bool mine = pos >= 0 && pos < a.max_len && min(pos / C, (int64_t)a.n_splits - 1) == s;
    if (it < G + 2) {
      const u32x4 r = it <= G ? rope8<XT>(own, partner, cw, sw, ich < 8) : own;
      rq[it][ich] = r;
      if (it >= G && mine)
        *reinterpret_cast<u32x4*>((it == G ? a.k_out : a.v_out) + kv_base + pos * a.kv_sl + ich * 8) = r;
    }
    lds_barrier();   // the K/V loads stay in flight
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qa[ks] = rq[min(mr, G - 1)][4 * ks + mg];
      kn[ks] = rq[G][4 * ks + mg];
    }
    vnw = rq[G + 1][ch];
    if (mine) pk = (int)pos;
  }

  // ---- QK on the matrix cores: sacc[blk][v] = k[key wkey0 + 16 blk + 4 mg + v] . q[head mr]
  v4f sacc[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    sacc[blk] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      sacc[blk] = mfma16<XT>(__builtin_bit_cast(v4i, kb[blk][ks]), __builtin_bit_cast(v4i, qa[ks]), sacc[blk]);
  }
  v4f snew = v4f{0.f, 0.f, 0.f, 0.f};   // RoPE form: the new key's scores (every row holds them)
  if constexpr (ROPE) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      snew = mfma16<XT>(__builtin_bit_cast(v4i, kn[ks]), __builtin_bit_cast(v4i, qa[ks]), snew);
  }
  // The value rows go out only now.  Every workgroup requests its K and V at
  // once and the memory system accepts the loads only as earlier ones return,
  // so a wave with V loads still waiting to issue could not start its QK on
  // keys that had long arrived (measured on MI355X, configs[4] decode shape:
  // split + merge 15.2 -> 14.1 us per layer; after the softmax 14.1, half
  // before and half after the QK 14.5).  In the RoPE form the split that
  // writes the new token's v may read that row back here: the value it reads
  // is replaced by vnw in the PV either way.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kSteps; ++i)
    vw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, kv_off(wkey0 + 8 * kl + i, ch), 0, 0));
  __builtin_amdgcn_sched_barrier(0);

  // ---- this wave's softmax over its 32 keys: lane (mr, mg) holds 8 scores of
  //      head mr; max and sum over them, then over the 4 lanes of the head
  //      (lanes mr + 16 j, permlane butterflies).  Probabilities go to LDS as
  //      [head][key] for the PV layout.
  float pr[2][4];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int key = wkey0 + 16 * blk + 4 * mg + v;
      const float raw = (ROPE && key == pk) ? snew[v] : sacc[blk][v];
      pr[blk][v] = key < hi ? raw * a.scale_log2 : -INFINITY;
    }
  float mx = fmaxf(fmaxf(fmaxf(pr[0][0], pr[0][1]), fmaxf(pr[0][2], pr[0][3])),
                   fmaxf(fmaxf(pr[1][0], pr[1][1]), fmaxf(pr[1][2], pr[1][3])));
  mx = rows4_max(mx);
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int v = 0; v < 4; ++v)   // exp2 of a non-positive argument (-inf for keys past the prefix)
      pr[blk][v] = mx == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pr[blk][v] - mx);
  const float ls = rows4_sum(((pr[0][0] + pr[0][1]) + (pr[0][2] + pr[0][3])) +
                             ((pr[1][0] + pr[1][1]) + (pr[1][2] + pr[1][3])));
  if (mr < G) {
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
      *reinterpret_cast<v4f*>(&pl[wave][mr][16 * blk + 4 * mg]) = v4f{pr[blk][0], pr[blk][1], pr[blk][2], pr[blk][3]};
    if (mg == 0) {
      wml[wave][mr][0] = mx;
      wml[wave][mr][1] = ls;
    }
  }
  // the probabilities are read back by other lanes of the same wave: LDS
  // executes a wave's accesses in order, so waiting for the writes suffices
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");

  // ---- PV: lane (kl, ch) takes keys 8 kl .. 8 kl + 7 of the wave, 8
  //      dimensions of each value row (16 lanes per 256-byte row)
  float o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  float pg[G][kSteps];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const v4f p0 = *reinterpret_cast<const v4f*>(&pl[wave][g][8 * kl]);
    const v4f p1 = *reinterpret_cast<const v4f*>(&pl[wave][g][8 * kl + 4]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      pg[g][v] = p0[v];
      pg[g][4 + v] = p1[v];
    }
  }
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    float vf[8];
    unpack8<XT>((ROPE && wkey0 + 8 * kl + i == pk) ? vnw : vw[i], vf);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pg[g][i], vf[e], o[g][e]);
  }
  if constexpr (kLdsSum) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      *reinterpret_cast<v4f*>(&wo[wave][kl][g][ch * 8]) = v4f{o[g][0], o[g][1], o[g][2], o[g][3]};
      *reinterpret_cast<v4f*>(&wo[wave][kl][g][ch * 8 + 4]) = v4f{o[g][4], o[g][5], o[g][6], o[g][7]};
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = rows4_sum(o[g][e]);
        if (kl == 0) wo[wave][0][g][ch * 8 + e] = x;
      }
  }
  __syncthreads();
  // ---- combine the waves in wave order, rescaled to the chunk max; one
  //      partial record per query head: o[D], m, l (m in log2 units)
  for (int e = t; e < G * kAttnD; e += kThreads) {
    const int g = e / kAttnD, d = e - g * kAttnD;
    float M = wml[0][g][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, wml[w][g][0]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mwv = wml[w][g][0];
      const float c = mwv == -INFINITY ? 0.0f : exp2f(mwv - M);
      // the wave's key groups in the association of the butterflies: (0 + 1) + (2 + 3)
      const float ow = kLdsSum ? (wo[w][0][g][d] + wo[w][KG > 1 ? 1 : 0][g][d]) +
                                     (wo[w][KG > 2 ? 2 : 0][g][d] + wo[w][KG > 3 ? 3 : 0][g][d])
                               : wo[w][0][g][d];
      O = fmaf(c, ow, O);
      L = fmaf(c, wml[w][g][1], L);
    }
    float* rec = a.part + ((int64_t)(b * a.q_heads + kvh * G + g) * a.n_splits + s) * (kAttnD + 2);
    rec[d] = O;
    if (d == 0) {
      rec[kAttnD] = M;
      rec[kAttnD + 1] = L;
    }
  }
}

// Merge of the split partials of one (b, h) for dimension d: online over
// batches of NB splits (NB = the split count rounded up to 8, at most
// kMergeBatch), every load of a batch issued before its first use.  Within
// one batch this is the plain two-pass formula (batch max, then the weighted
// sums in split order).  Each split's (m, l) pair is the same for every lane;
// it is read with a vector load all the same (an offset the compiler cannot
// see is zero): as scalar loads, which may return out of order, the 24 or
// more pairs of a batch took more than one round trip (measured 1.6 us slower).
constexpr int kMergeBatch = 64;

template <int NB>
__device__ inline float merge_splits(const AttnArgs& a, const float* rec, int d) {
  int vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  float M = -INFINITY, L = 0.0f, acc = 0.0f;
  for (int s0 = 0; s0 < a.n_splits; s0 += NB) {
    float m[NB], l[NB], o[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int sj = min(s0 + j, a.n_splits - 1);
      const float* r = rec + (int64_t)sj * (kAttnD + 2);
      const float2 ml = *reinterpret_cast<const float2*>(r + kAttnD + vzero);
      m[j] = s0 + j < a.n_splits ? ml.x : -INFINITY;
      l[j] = ml.y;
      o[j] = r[d];
    }
    // Branch-free (an early exit here made the compiler load l and o only
    // after m had arrived: two round trips): empty splits and padding get
    // weight 0, which adds an exact 0 to the finite partial sums.
    float Mb = M;
#pragma unroll
    for (int j = 0; j < NB; ++j) Mb = fmaxf(Mb, m[j]);
    const bool any = Mb != -INFINITY;
    const float r = any ? exp2f(M - Mb) : 1.0f;   // 0 while nothing has been accumulated (M = -inf)
    L *= r;
    acc *= r;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float w = m[j] == -INFINITY ? 0.0f : exp2f(m[j] - Mb);
      L = fmaf(w, l[j], L);
      acc = fmaf(w, o[j], acc);
    }
    M = any ? Mb : M;
  }
  return L > 0.0f ? acc / L : 0.0f;
}

template <class XT, int NB>
__global__ void __launch_bounds__(kAttnD)
attn_merge_kernel(AttnArgs a, L2Warm warm) {
  TQ_ARGS_IN_SGPRS("s"(a.part), "s"(a.out), "s"(a.o_sb), "s"(a.o_sh), "s"(a.q_heads), "s"(a.n_splits),
                   "s"(warm.first));
  if ((int)blockIdx.x >= warm.first) {   // the warm-up workgroups (none without a warm-up)
    __shared__ uint32_t warm_sink[64];
    l2_warm_rows<kAttnD>(warm, warm_sink);
    return;
  }
  const int bh = blockIdx.x, d = threadIdx.x;
  const int b = bh / a.q_heads, h = bh - (bh / a.q_heads) * a.q_heads;
  const float* rec = a.part + (int64_t)bh * a.n_splits * (kAttnD + 2);
  a.out[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d] = XT::from_f32(merge_splits<NB>(a, rec, d));
}

// Merge + INT8 quantization of the attention output for the next projection:
// workgroup (h, half) = column tile 2h + half of the [batch, q_heads * 128]
// projection input (dimensions 64 half .. 64 half + 63 of query head h) for
// ALL batch rows (b < batch <= 16): wave rg takes rows rg, rg + 4, ... (RPW
// per wave), lane = dimension.  The tile is whole inside the workgroup:
// absmax over the batch rows, scale, codes -- the closed form of
// tq_act_quant, bit for bit.  Per batch of NB splits every load goes out at
// once: the lanes' o values first, then each (row, split)'s (m, l) pair once
// per workgroup (into LDS), so one round trip serves the batch and no lane
// re-reads the pairs.
constexpr int kMergeQuantMaxRows = 16;
constexpr int kMergeQuantThreads = 256;   // 4 waves (row groups) x 64 dimensions

template <class XT, int NB, int RPW>
__global__ void __launch_bounds__(kMergeQuantThreads)
attn_merge_quant_kernel(AttnArgs a, int8_t* __restrict__ q, int64_t ldq, float* __restrict__ sx, L2Warm warm) {
  constexpr int kGroups = kMergeQuantThreads / kWave;
  __shared__ float2 mls[kGroups * RPW][NB];
  TQ_ARGS_IN_SGPRS("s"(a.part), "s"(a.out), "s"(a.o_sb), "s"(a.o_sh), "s"(a.batch), "s"(a.q_heads),
                   "s"(a.n_splits), "s"(q), "s"(ldq), "s"(sx), "s"(warm.first));
  if ((int)blockIdx.x >= warm.first) {   // the warm-up workgroups (none without a warm-up)
    __shared__ uint32_t warm_sink[64];
    l2_warm_rows<kMergeQuantThreads>(warm, warm_sink);
    return;
  }
  __shared__ float red[kGroups];
  const int h = blockIdx.x >> 1, half = blockIdx.x & 1;
  // the row group is wave-uniform: as a scalar, the buffer resources below
  // are too (else every load of them is wrapped in a readfirstlane loop)
  const int t = threadIdx.x, lane = t & 63, rg = __builtin_amdgcn_readfirstlane(t >> 6);
  const int d = half * 64 + lane;
  const int S = a.n_splits;
  const int64_t rec_elems = (int64_t)S * (kAttnD + 2);   // one (b, h)'s records
  __amdgpu_buffer_rsrc_t rs[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int b = rg + kGroups * i;   // rows past the batch: empty range, loads read 0
    rs[i] = row_rsrc(a.part + (int64_t)(min(b, a.batch - 1) * a.q_heads + h) * rec_elems,
                     b < a.batch ? (int)(rec_elems * 4) : 0);
  }
  const int n_ml = a.batch * NB;
  float M[RPW], L[RPW], acc[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    M[i] = -INFINITY;
    L[i] = 0.0f;
    acc[i] = 0.0f;
  }
  for (int s0 = 0; s0 < S; s0 += NB) {
    float o[RPW][NB];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        o[i][j] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            rs[i], (int)(((int64_t)min(s0 + j, S - 1) * (kAttnD + 2) + d) * 4), 0, 0));
    // (m, l) of entries e = (row b, split s0 + j), issued after the o loads
    // (the wait for them then covers those too); padding splits get m = -inf
    constexpr int kML = (kGroups * RPW * NB + kMergeQuantThreads - 1) / kMergeQuantThreads;
    float2 ml[kML];
#pragma unroll
    for (int u = 0; u < kML; ++u) {
      const int e = min(t + u * kMergeQuantThreads, n_ml - 1), eb = e / NB, ej = e - eb * NB;
      ml[u] = *reinterpret_cast<const float2*>(a.part + (int64_t)(eb * a.q_heads + h) * rec_elems +
                                               (int64_t)min(s0 + ej, S - 1) * (kAttnD + 2) + kAttnD);
    }
#pragma unroll
    for (int u = 0; u < kML; ++u) {
      const int e = t + u * kMergeQuantThreads, eb = e / NB, ej = e - eb * NB;
      if (e < n_ml) mls[eb][ej] = float2{s0 + ej < S ? ml[u].x : -INFINITY, ml[u].y};
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int b = min(rg + kGroups * i, a.batch - 1);
      // the same arithmetic as merge_splits: batch max, rescale, weighted sums in split order
      float Mb = M[i];
#pragma unroll
      for (int j = 0; j < NB; ++j) Mb = fmaxf(Mb, mls[b][j].x);
      const bool any = Mb != -INFINITY;
      const float r = any ? exp2f(M[i] - Mb) : 1.0f;
      L[i] *= r;
      acc[i] *= r;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const float2 mj = mls[b][j];
        const float w = mj.x == -INFINITY ? 0.0f : exp2f(mj.x - Mb);
        L[i] = fmaf(w, mj.y, L[i]);
        acc[i] = fmaf(w, o[i][j], acc[i]);
      }
      M[i] = any ? Mb : M[i];
    }
    __syncthreads();   // the next batch rewrites mls
  }
  float y[RPW];
  float am = 0.0f;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const bool live = rg + kGroups * i < a.batch;
    y[i] = live ? XT::round(L[i] > 0.0f ? acc[i] / L[i] : 0.0f) : 0.0f;
    am = fmaxf(am, fabsf(y[i]));
  }
  const float wm = wave_max_nonneg(am);
  if (lane == 0) red[rg] = wm;
  __syncthreads();
  const float tm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = act_scale_from_absmax<XT>(tm);
  const CodeScale cs(s);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int b = rg + kGroups * i;
    if (b < a.batch) {
      a.out[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d] = XT::from_f32(y[i]);
      q[(int64_t)b * ldq + h * kAttnD + d] = (int8_t)cs.code(y[i]);
    }
  }
  if (t == 0) sx[2 * h + half] = s;
}

// The merge's own grid (workgroups before any warm-up ones).
static int merge_blocks(const AttnArgs& a, bool quant) { return quant ? a.q_heads * 2 : a.batch * a.q_heads; }

// Merge launches: NB = splits rounded up to 8 (at most kMergeBatch), so no
// load of a batch is wasted on padding below kMergeBatch splits.
template <class XT, int NB>
static void launch_merge_nb(const AttnArgs& a, int8_t* q_out, int64_t ldq, float* sx, const L2Warm& warm,
                            hipStream_t s) {
  const dim3 g(merge_blocks(a, q_out != nullptr) + warm.blocks), bq(kMergeQuantThreads);
  if (!q_out)
    hipLaunchKernelGGL((attn_merge_kernel<XT, NB>), g, dim3(kAttnD), 0, s, a, warm);
  else if (a.batch <= 4)
    hipLaunchKernelGGL((attn_merge_quant_kernel<XT, NB, 1>), g, bq, 0, s, a, q_out, ldq, sx, warm);
  else if (a.batch <= 8)
    hipLaunchKernelGGL((attn_merge_quant_kernel<XT, NB, 2>), g, bq, 0, s, a, q_out, ldq, sx, warm);
  else
    hipLaunchKernelGGL((attn_merge_quant_kernel<XT, NB, 4>), g, bq, 0, s, a, q_out, ldq, sx, warm);
}

// warm: its `first` must be merge_blocks(a, q_out != nullptr).
template <class XT>
static void launch_merge(const AttnArgs& a, int8_t* q_out, int64_t ldq, float* sx, const L2Warm& warm,
                         hipStream_t s) {
  switch ((min(a.n_splits, kMergeBatch) + 7) / 8) {
    case 1: launch_merge_nb<XT, 8>(a, q_out, ldq, sx, warm, s); break;
    case 2: launch_merge_nb<XT, 16>(a, q_out, ldq, sx, warm, s); break;
    case 3: launch_merge_nb<XT, 24>(a, q_out, ldq, sx, warm, s); break;
    case 4: launch_merge_nb<XT, 32>(a, q_out, ldq, sx, warm, s); break;
    case 5: launch_merge_nb<XT, 40>(a, q_out, ldq, sx, warm, s); break;
    case 6: launch_merge_nb<XT, 48>(a, q_out, ldq, sx, warm, s); break;
    case 7: launch_merge_nb<XT, 56>(a, q_out, ldq, sx, warm, s); break;
    default: launch_merge_nb<XT, 64>(a, q_out, ldq, sx, warm, s); break;
  }
}

// No warm-up: the merge's own grid only.
static L2Warm no_warm(const AttnArgs& a, bool quant) {
  return L2Warm{nullptr, nullptr, nullptr, nullptr, 0, 0, merge_blocks(a, quant)};
}

// Split plan.  Workgroups are dealt evenly to the compute units, so the
// split kernel ends when the most loaded CU is done: pick the waves per
// workgroup W and the split count S (each split <= 32 W keys) that minimise
// that CU's keys, ceil(pairs S / CUs) * ceil(max_len / S); ties go to fewer
// splits (a cheaper merge), then fewer waves.  B = 4 x 8 kv heads at 2304
// keys: 3 waves x 24 splits (768 workgroups, 3 per CU) instead of 18 splits of
// 128 keys (576 workgroups: a quarter of the CUs carried a third one and
// finished last).  The split count is capped (at most 64 below 2048 keys),
// which bounds the workspace.
static int attn_split_cap(int max_len) {
  const int s_big = (max_len + kAttnMaxWaves * kAttnKeysPerWave - 1) / (kAttnMaxWaves * kAttnKeysPerWave);
  return max(s_big, min(64, (max_len + kAttnKeysPerWave - 1) / kAttnKeysPerWave));
}

// CU count of the current device, cached per device (threads may launch
// concurrently; they store the same value)
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

struct AttnPlan {
  int S, W;
};

static AttnPlan attn_plan(int max_len, int pairs, int G, bool rope, int cus) {
  AttnPlan best{attn_split_cap(max_len), kAttnMaxWaves};
  int64_t best_load = -1;
  const int cap = attn_split_cap(max_len);
  for (int W = 2; W <= kAttnMaxWaves; ++W) {
    if (rope && 16 * (G + 2) > W * kWave) continue;
    const int per = W * kAttnKeysPerWave;
    for (int S = (max_len + per - 1) / per; S <= cap; ++S) {
      const int64_t rounds = ((int64_t)pairs * S + cus - 1) / cus;
      const int64_t load = rounds * ((max_len + S - 1) / S);
      if (best_load < 0 || load < best_load || (load == best_load && (S < best.S || (S == best.S && W < best.W)))) {
        best = AttnPlan{S, W};
        best_load = load;
      }
    }
  }
  return best;
}

template <class XT, int G, bool ROPE, int W>
static void launch_split_gw(const AttnArgs& a, dim3 grid, hipStream_t s) {
  if constexpr (!ROPE || 16 * (G + 2) <= W * kWave)
    hipLaunchKernelGGL((attn_split_kernel<XT, G, ROPE, W>), grid, dim3(W * kWave), 0, s, a);
}

template <class XT, int G, bool ROPE>
static void launch_split_g(const AttnArgs& a, dim3 grid, hipStream_t s) {
  switch (a.waves) {
    case 2: launch_split_gw<XT, G, ROPE, 2>(a, grid, s); break;
    case 3: launch_split_gw<XT, G, ROPE, 3>(a, grid, s); break;
    default: launch_split_gw<XT, G, ROPE, 4>(a, grid, s); break;
  }
}

template <class XT, bool ROPE = false>
static void launch_split(const AttnArgs& a, dim3 grid, hipStream_t s) {
  switch (a.G) {
    case 1: launch_split_g<XT, 1, ROPE>(a, grid, s); break;
    case 2: launch_split_g<XT, 2, ROPE>(a, grid, s); break;
    case 3: launch_split_g<XT, 3, ROPE>(a, grid, s); break;
    case 4: launch_split_g<XT, 4, ROPE>(a, grid, s); break;
    case 5: launch_split_g<XT, 5, ROPE>(a, grid, s); break;
    case 6: launch_split_g<XT, 6, ROPE>(a, grid, s); break;
    case 7: launch_split_g<XT, 7, ROPE>(a, grid, s); break;
    default: launch_split_g<XT, 8, ROPE>(a, grid, s); break;
  }
}

}  // namespace tq

using namespace tq;

extern "C" int tq_decode_attention_plan(int batch, int q_heads, int kv_heads, int max_len, int rope, int cus,
                                        int* n_splits, int* waves) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || max_len <= 0 || cus <= 0 || q_heads % kv_heads != 0 ||
      q_heads / kv_heads > kAttnMaxG || n_splits == nullptr || waves == nullptr)
    return TQ_ERR_ARG;
  const AttnPlan p = attn_plan(max_len, batch * kv_heads, q_heads / kv_heads, rope != 0, cus);
  *n_splits = p.S;
  *waves = p.W;
  return TQ_OK;
}

extern "C" int64_t tq_decode_attention_workspace_elems(int batch, int q_heads, int max_len) {
  if (batch <= 0 || q_heads <= 0 || max_len <= 0) return 0;
  return (int64_t)batch * q_heads * attn_split_cap(max_len) * (kAttnD + 2);
}

static int attn_setup(AttnArgs& a, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                      const void* v, int64_t kv_stride_b, int64_t kv_stride_l, int64_t kv_stride_h,
                      const int32_t* seq_used, void* out, int64_t out_stride_b, int64_t out_stride_h, int dtype,
                      int batch, int q_heads, int kv_heads, int head_dim, int max_len, float scale,
                      float* workspace, int64_t workspace_elems, bool rope) {
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
  // one (b, kv head)'s valid rows are addressed through a 32-bit buffer range
  if (kv_stride_l < head_dim || ((int64_t)max_len * kv_stride_l + head_dim) * 2 >= (1LL << 31)) return TQ_ERR_ARG;
  a.q = static_cast<const uint16_t*>(q); a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.k = static_cast<const uint16_t*>(k); a.v = static_cast<const uint16_t*>(v);
  a.kv_sb = kv_stride_b; a.kv_sl = kv_stride_l; a.kv_sh = kv_stride_h;
  a.seq_used = seq_used;
  a.out = static_cast<uint16_t*>(out); a.o_sb = out_stride_b; a.o_sh = out_stride_h;
  a.part = workspace;
  a.batch = batch; a.q_heads = q_heads; a.kv_heads = kv_heads; a.G = q_heads / kv_heads;
  a.max_len = max_len;
  const AttnPlan plan = attn_plan(max_len, batch * kv_heads, a.G, rope, device_cus());
  a.n_splits = plan.S;
  a.waves = plan.W;
  a.scale_log2 = scale * kLog2e;
  return 1;   // ready to launch
}

extern "C" int tq_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                   const void* v, int64_t kv_stride_b, int64_t kv_stride_l,
                                   int64_t kv_stride_h, const int32_t* seq_used, void* out,
                                   int64_t out_stride_b, int64_t out_stride_h, int dtype, int batch,
                                   int q_heads, int kv_heads, int head_dim, int max_len, float scale,
                                   float* workspace, int64_t workspace_elems, void* stream) {
  AttnArgs a{};
  const int rc = attn_setup(a, q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_l, kv_stride_h, seq_used,
                            out, out_stride_b, out_stride_h, dtype, batch, q_heads, kv_heads, head_dim, max_len,
                            scale, workspace, workspace_elems, false);
  if (rc != 1) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g1(a.n_splits, batch * kv_heads);
  if (dtype == TQ_DTYPE_BF16) {
    launch_split<Bf16>(a, g1, s);
    launch_merge<Bf16>(a, nullptr, 0, nullptr, no_warm(a, false), s);
  } else {
    launch_split<Fp16>(a, g1, s);
    launch_merge<Fp16>(a, nullptr, 0, nullptr, no_warm(a, false), s);
  }
  return (int)hipGetLastError();
}

extern "C" int tq_decode_attention_quant(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                         const void* v, int64_t kv_stride_b, int64_t kv_stride_l,
                                         int64_t kv_stride_h, const int32_t* seq_used, void* out,
                                         int64_t out_stride_b, int64_t out_stride_h, int8_t* q_out,
                                         int64_t q_out_stride_b, float* sx_out, int dtype, int batch, int q_heads,
                                         int kv_heads, int head_dim, int max_len, float scale, float* workspace,
                                         int64_t workspace_elems, void* stream) {
  if (batch > kMergeQuantMaxRows || (batch > 0 && (!q_out || !sx_out))) return TQ_ERR_ARG;
  AttnArgs a{};
  const int rc = attn_setup(a, q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_l, kv_stride_h, seq_used,
                            out, out_stride_b, out_stride_h, dtype, batch, q_heads, kv_heads, head_dim, max_len,
                            scale, workspace, workspace_elems, false);
  if (rc != 1) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g1(a.n_splits, batch * kv_heads);
  if (dtype == TQ_DTYPE_BF16) {
    launch_split<Bf16>(a, g1, s);
    launch_merge<Bf16>(a, q_out, q_out_stride_b, sx_out, no_warm(a, true), s);
  } else {
    launch_split<Fp16>(a, g1, s);
    launch_merge<Fp16>(a, q_out, q_out_stride_b, sx_out, no_warm(a, true), s);
  }
  return (int)hipGetLastError();
}

extern "C" int tq_decode_attention_rope(const void* qkv, int64_t qkv_stride, const void* cos_table, const void* sin_table,
                                        const int64_t* position, void* k_cache, void* v_cache,
                                        int64_t cache_stride_b, int64_t cache_stride_l, int64_t cache_stride_h,
                                        const int32_t* seq_used, void* out, int64_t out_stride_b,
                                        int64_t out_stride_h, int8_t* q_out, int64_t q_out_stride_b,
                                        float* sx_out, int dtype, int batch, int q_heads, int kv_heads,
                                        int head_dim, int max_len, float scale, float* workspace,
                                        int64_t workspace_elems, const tq_l2_warm* warm_in, void* stream) {
  if (q_out != nullptr && (batch > kMergeQuantMaxRows || sx_out == nullptr)) return TQ_ERR_ARG;
  if (batch > 0 && max_len > 0 && (!cos_table || !sin_table || !position)) return TQ_ERR_ARG;
  if ((cos_table && !aligned16(cos_table)) || (sin_table && !aligned16(sin_table))) return TQ_ERR_ALIGN;
  if (qkv_stride < (int64_t)(q_heads + 2 * kv_heads) * head_dim) return TQ_ERR_ARG;
  AttnArgs a{};
  const int rc = attn_setup(a, qkv, qkv_stride, head_dim, k_cache, v_cache, cache_stride_b, cache_stride_l,
                            cache_stride_h, seq_used, out, out_stride_b, out_stride_h, dtype, batch, q_heads,
                            kv_heads, head_dim, max_len, scale, workspace, workspace_elems, true);
  if (rc != 1) return rc;
  a.cos = static_cast<const uint16_t*>(cos_table);
  a.sin = static_cast<const uint16_t*>(sin_table);
  a.pos = position;
  a.k_out = static_cast<uint16_t*>(k_cache);
  a.v_out = static_cast<uint16_t*>(v_cache);
  L2Warm warm;
  const int wrc = l2_warm_args(warm_in, merge_blocks(a, q_out != nullptr), warm);
  if (wrc) return wrc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g1(a.n_splits, batch * kv_heads);
  if (dtype == TQ_DTYPE_BF16) {
    launch_split<Bf16, true>(a, g1, s);
    launch_merge<Bf16>(a, q_out, q_out_stride_b, sx_out, warm, s);
  } else {
    launch_split<Fp16, true>(a, g1, s);
    launch_merge<Fp16>(a, q_out, q_out_stride_b, sx_out, warm, s);
  }
  return (int)hipGetLastError();
}

// ---- allocation-free variant -------------------------------------------------
// tq_decode_attention with the split records in a file-scope device array
// instead of a caller workspace, for callers that cannot allocate.  Every GPU
// the library runs on holds its own copy of the array from module load until
// the process ends.  On the host the array's name is only a stand-in: its
// device address comes from hipGetSymbolAddress, looked up once per device
// (with that device current) and cached.
constexpr int64_t kAttnScratchFloats = (int64_t)4 << 20;   // 16 MiB
static __device__ __align__(256) float scratch[kAttnScratchFloats];

// Address of this device's scratch array; nullptr (and *err set) on failure.
static float* attn_scratch_for(int dev, hipError_t* err) {
  static std::atomic<float*> cached[64];
  if (dev < 0 || dev >= 64) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  float* p = cached[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  void* addr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || addr == nullptr) {
    *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
    return nullptr;
  }
  p = static_cast<float*>(addr);
  cached[dev].store(p, std::memory_order_release);
  return p;
}

extern "C" int tq_decode_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                           const void* v, int64_t kv_stride_b, int64_t kv_stride_l,
                                           int64_t kv_stride_h, const int32_t* seq_used, void* out,
                                           int64_t out_stride_b, int64_t out_stride_h, int dtype, int batch,
                                           int q_heads, int kv_heads, int head_dim, int max_len, float scale,
                                           void* stream) {
  if (batch > 0 && q_heads > 0 && max_len > 0 &&
      tq_decode_attention_workspace_elems(batch, q_heads, max_len) > kAttnScratchFloats)
    return TQ_ERR_WORKSPACE;   // beyond the fixed scratch: use tq_decode_attention with a workspace
  int dev = 0;
  TQ_RETURN_IF_HIP_ERROR(hipGetDevice(&dev));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (s != nullptr) {   // the scratch looked up is the current device's: the stream must be on it
    hipDevice_t sdev = 0;
    TQ_RETURN_IF_HIP_ERROR(hipStreamGetDevice(s, &sdev));
    if (sdev != dev) return TQ_ERR_ARG;
  }
  hipError_t err = hipSuccess;
  float* ws = attn_scratch_for(dev, &err);
  if (ws == nullptr) return (int)err;
  return tq_decode_attention(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_l, kv_stride_h, seq_used, out,
                             out_stride_b, out_stride_h, dtype, batch, q_heads, kv_heads, head_dim, max_len, scale,
                             ws, kAttnScratchFloats, stream);
}
