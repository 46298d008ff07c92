/*
 * tilequant.h -- C ABI of the MI355X (gfx950) TileQuant mixed INT8/BF16 tile
 * path, exported by tilequant_amd/_lib/libtilequant_hip.so.
 *
 * Conventions
 *  - Every pointer is a device pointer owned by the caller (plain hipMalloc /
 *    torch allocations).  The library allocates and frees nothing.
 *  - Matrices are row-major with an explicit row stride in ELEMENTS; unless a
 *    parameter says otherwise the column stride is 1.
 *  - `stream` is a hipStream_t (0 = null stream).  Work is only enqueued; no
 *    entry point synchronizes the host, so every call is hipGraph-capturable.
 *  - Return value: 0 on success, a positive hipError_t from the launch, or a
 *    negative TQ_ERR_* for an argument error (nothing is enqueued then).
 *    tq_error_string() names either kind.
 *  - Activation / 16-bit tile dtypes are TQ_DTYPE_BF16 or TQ_DTYPE_FP16.
 *
 * Reference interface each entry point replaces (paths relative to the
 * TileQuant repository root) is cited above each declaration.
 */
#ifndef TILEQUANT_H
#define TILEQUANT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TQ_DTYPE_BF16 = 0, TQ_DTYPE_FP16 = 1, TQ_DTYPE_FP32 = 2 /* tq_quant_tensor_absmax only */ };

/* Storage order of the 64x64 elements inside one packed tile.
 * ROW_MAJOR: tile[j][k] at j*64+k (the reference packer's order, pack.py:115-175).
 * MFMA: operand-major order of the gfx950 MFMA B operand: 16-row block jb of the
 *   tile is one contiguous 1 KiB run in which lane l (kq = l / 16, j = l % 16)
 *   holds W[16 jb + j][16 kq .. 16 kq + 15] (INT8) -- one 16-byte load per lane.
 *   16-bit tiles: 512-element runs per (jb, K half h), lane l holding
 *   W[16 jb + j][32 h + 8 kq .. + 7]. */
enum { TQ_LAYOUT_ROW_MAJOR = 0, TQ_LAYOUT_MFMA = 1 };

/* Flag OR'ed into the tile_layout argument of the GEMM entries (and the
 * descriptor's tile_layout): the INT8 activation codes x_int8 are TOKEN-BLOCKED
 * instead of row-major.  Token-blocked codes of n rows, k = 64 * n_tc columns
 * are n_tc * ceil(n / 16) blocks of 1 KiB, block (c, b) at offset
 * (c * ceil(n / 16) + b) * 1024, in the MFMA A-operand order: 16-byte run l
 * (kq = l / 16, j = l % 16) holds the codes of row 16 b + j, columns
 * 64 c + 16 kq .. + 15; rows n .. 16 ceil(n / 16) - 1 hold zeros.  Each
 * operand load of the GEMM is then one contiguous 1 KiB (8 whole cache
 * lines) instead of 16 row pieces of 64 bytes.  Accepted for 1 <= n <= 64
 * with k = 64 * n_tc (x_int8_stride_n is ignored); the result is bitwise that
 * of the same codes row-major.  tq_act_quant_token_blocked writes them.  No
 * reference counterpart (the reference keeps codes row-major). */
enum { TQ_XQ_TOKEN_BLOCKED = 0x100 };

enum {
  TQ_OK = 0,
  TQ_ERR_ARG = -1,       /* bad size / null pointer / inconsistent shape */
  TQ_ERR_DTYPE = -2,     /* unsupported dtype or layout code */
  TQ_ERR_ALIGN = -3,     /* a tile pointer is not 16-byte aligned */
  TQ_ERR_WORKSPACE = -4  /* workspace missing or too small */
};

const char* tq_error_string(int code);
/* ABI version of this header (bumped on any signature change). */
int tq_abi_version(void);

/* ---- activation quantization ------------------------------------------
 * Per 64-column tile c of x [n, k]:  a = max |x[:, 64c:64c+64]| over ALL n
 * rows;  sx[c] = 1 if a == 0 else f32(round_to_x_dtype(f32(a) / 127));
 * q = clamp(rint(f32(x) / sx[c]), -127, 127).  q is written [n, k] with row
 * stride q_stride_n; sx has ceil(k / 64) entries.                        */

/* Replaces quantize_activation_tile_absmax_fused
 * (src/kernels/triton/quantize_activation.py:118-155, kernel :77-112).
 * One launch; any n (the reference routes n <= 128 here, quant_utils.py:119-134). */
int tq_act_quant_fused(const void* x, int64_t x_stride_n, int64_t x_stride_k, int x_dtype,
                       int n, int k, int8_t* q, int64_t q_stride_n, float* sx, void* stream);

/* tq_act_quant_fused writing the codes TOKEN-BLOCKED (see TQ_XQ_TOKEN_BLOCKED):
 * q has 16 * ceil(n / 16) * k bytes, padding rows zero; same scales and code
 * values.  1 <= n <= 64, k a multiple of 64, unit column stride, 16-byte
 * aligned rows (x_stride_n % 8 == 0).  Counterpart of the reference's
 * quantize_activation_tile_absmax_fused (quantize_activation.py:118-155) for
 * the token-blocked operand format the 17..64-token GEMM reads. */
int tq_act_quant_token_blocked(const void* x, int64_t x_stride_n, int x_dtype, int n, int k, int8_t* q,
                               float* sx, void* stream);

/* Elements of fp32 workspace tq_act_absmax_scales needs for (n, k); 0 when
 * the scales are produced in a single pass. */
int64_t tq_act_absmax_workspace_elems(int n, int k);

/* Replaces activation_tile_absmax_scales_64_fused
 * (quantize_activation.py:158-176, kernel :13-44) / activation_tile_absmax_scales
 * (src/kernels/quant_utils.py:41-74).  Scales only. */
int tq_act_absmax_scales(const void* x, int64_t x_stride_n, int64_t x_stride_k, int x_dtype,
                         int n, int k, float* sx, float* workspace, int64_t workspace_elems,
                         void* stream);

/* Replaces quantize_activation_tile_with_scales_64_fused
 * (quantize_activation.py:179-203, kernel :47-74) / quantize_activation_tile_with_scales
 * (quant_utils.py:78-115).  Codes from given scales. */
int tq_act_quant_with_scales(const void* x, int64_t x_stride_n, int64_t x_stride_k,
                             int x_dtype, int n, int k, const float* sx, int8_t* q,
                             int64_t q_stride_n, void* stream);

/* tq_act_absmax_scales followed by tq_act_quant_with_scales for inputs that
 * need the two-level scales (more than 512 rows), in two launches instead of
 * three: the codes kernel reduces its column's absmax partials itself (the
 * finalize step folded in).  Unit column stride, 16-byte aligned rows, k a
 * multiple of 64, 8-byte aligned code rows (TQ_ERR_ALIGN otherwise);
 * workspace = tq_act_absmax_workspace_elems(n, k) floats.  Codes and scales
 * are bitwise those of the two calls.  No reference counterpart: the
 * reference's dispatcher (quant_utils.py:119-134) runs the scales kernel and
 * the codes kernel one after the other. */
int tq_act_quant_two_level(const void* x, int64_t x_stride_n, int x_dtype, int n, int k, int8_t* q,
                           int64_t q_stride_n, float* sx, float* workspace, int64_t workspace_elems,
                           void* stream);

/* One scale for a whole tensor: replaces quantize_activation_absmax /
 * quantize_activation_per_tensor_absmax (src/kernels/quant_utils.py:17-37) and
 * quantize_weight_tile_absmax (:138-148), torch expressions there:
 *   a = max |x|;  scale = a == 0 ? 1 : f32(x_dtype(f32(a) / 127));
 *   q = clamp(rint(x_dtype(f32(x) / scale)), -127, 127)
 * -- the quotient is rounded to x's dtype before rint (a 16-bit tensor divided
 * by a 0-dim fp32 tensor stays 16-bit in torch); fp32 inputs skip both
 * roundings.  x: numel contiguous elements of x_dtype (BF16, FP16 or FP32);
 * q: numel int8; scale: one float written on the device.  numel == 0 writes
 * nothing (the reference returns scale 1).  workspace:
 * tq_quant_tensor_workspace_elems(numel) floats (0: none needed).  A tensor
 * whose scale underflows to 0 (max |x| < 127 * 2^-134 in bf16) gets codes
 * 127 for x == 0, where the reference's int8 cast of NaN is undefined. */
int64_t tq_quant_tensor_workspace_elems(int64_t numel);
int tq_quant_tensor_absmax(const void* x, int64_t numel, int x_dtype, int8_t* q, float* scale,
                           float* workspace, int64_t workspace_elems, void* stream);

/* ---- mixed INT8/BF16 tile GEMM -----------------------------------------
 * out[n, m] = sum over the INT8 tiles t of output row tile r = m / 64:
 *               f32(int32 dot(x_int8[n, 64c:64c+64], tile_t[m % 64, :])) * (sx[c] * sw[t])
 *           + sum over the 16-bit tiles of r: fp32 dot(x_fp[n, tile c], tile[m % 64, :])
 * rounded to out_dtype; with bias: round(f32(y) + f32(bias[m])).
 * Tiles of row tile r occupy positions row_ptr[r] .. row_ptr[r+1]-1 of their
 * arena, in ascending tile id (id = r * n_tc + c).  Columns >= k read as 0,
 * output columns >= m are not written.  x_fp and the 16-bit tiles share
 * x_dtype; bias (nullable) has out_dtype.  split_k <= 0 selects the schedule
 * automatically; a positive value fixes how many partitions of each row
 * tile's tile list are reduced (deterministically, in fixed order) per
 * output tile.  Results are bitwise reproducible for fixed arguments.
 *
 * Replaces gemm_mixed_rows_splitk (src/kernels/triton/gemm_rows_splitk_64x64.py:225-323,
 * kernel :78-190).  `workspace` is the reference's per-stream split-K buffer
 * (:193-215): tq_gemm_workspace_elems() fp32 elements, ZERO-FILLED before its
 * first use.  Its first 4096 elements are int32 arrival counters (one per row
 * tile; more row tiles than that run unsplit), the fp32 split partials follow.
 * Each launch leaves its arrival counters at zero again, so one
 * buffer serves every launch on one stream (launches on different streams
 * need different buffers).  Without a large enough workspace an automatic
 * schedule uses one split; an explicit split_k > 1 then fails with
 * TQ_ERR_WORKSPACE. */
int64_t tq_gemm_workspace_elems(int n, int m, int n_tr, int n_tc, int split_k);
int tq_gemm_mixed_rows(const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx,
                       const int8_t* int8_tiles, const float* int8_scales,
                       const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                       const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                       const void* fp16_tiles, const int32_t* fp16_tile_ids,
                       const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                       int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                       int n_tc, int split_k, int tile_layout, float* workspace,
                       int64_t workspace_elems, void* stream);

/* tq_gemm_mixed_rows with a work plan for its prefill kernel (n > 64):
 * prefill_units[0 .. n_units) from tq_gemm_prefill_plan for the same row
 * pointers, the first n_first of them dispatched before the others.  The
 * outputs are bitwise those of tq_gemm_mixed_rows; only the order and grouping
 * of the workgroups change.  Ignored for n <= 64.  No reference counterpart:
 * the reference's grid is one program per (row tile, split)
 * (gemm_rows_splitk_64x64.py:275-322). */
int tq_gemm_mixed_rows_planned(const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx,
                               const int8_t* int8_tiles, const float* int8_scales,
                               const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                               const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                               const void* fp16_tiles, const int32_t* fp16_tile_ids,
                               const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                               int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                               int n_tc, int split_k, int tile_layout, float* workspace,
                               int64_t workspace_elems, const int32_t* prefill_units, int n_units,
                               int n_first, void* stream);

/* Host function: the prefill work plan of one packed weight, from HOST copies
 * of its row pointers and INT8 tile ids (fp16_row_ptr may be NULL).  Writes
 * units (row tile | 1 << 30 for a single row tile, else a row-tile pair), in
 * row order, into units[0 .. max_units), max_units >= n_tr, and 0 into
 * *n_first.  Returns the unit count, 0 when no pair needs splitting (the plain
 * pair order is the plan), or TQ_ERR_ARG.  A pair whose 16-bit tiles make it
 * cost well above the median pair is split into its two row tiles when that
 * shortens it (its workgroups would otherwise finish long after the rest). */
int tq_gemm_prefill_plan(const int32_t* int8_row_ptr, const int32_t* int8_tile_ids,
                         const int32_t* fp16_row_ptr, int n_tr, int n_tc, int32_t* units, int max_units,
                         int* n_first);

/* Workspace (fp32 elements, zero-filled before first use, one per stream) that
 * tq_linear_mixed_fused needs for these arguments: the split-K counters and
 * partials (split_k > 1), or the cooperative launch's counters, codes and
 * scales (see tq_linear_mixed_fused); 0 when it needs none.  Without it the
 * call still runs, with a launch that needs none. */
int64_t tq_linear_mixed_fused_workspace_elems(int n, int m, int k, int n_tr, int n_tc, int split_k);

/* TEST-ONLY.  Poll budget of the cooperative launches of tq_linear_mixed_fused
 * in this process: polls >= 0 (0 makes every GEMM workgroup quantize the
 * activation itself instead of waiting for the producers; the outputs are the
 * same), < 0 restores the default.  No reference counterpart. */
void tq_test_set_coop_spin(int polls);

/* Largest n tq_linear_mixed_fused accepts for input width k: at most 16, and
 * the n x ceil(k/64)*64 int8 codes (+ scales) must fit 64 KiB of LDS. */
int tq_linear_mixed_fused_max_tokens(int k);

/* Activation quantization + the mixed tile GEMM in one launch, for decode
 * sizes (n <= tq_linear_mixed_fused_max_tokens(k)).  Equivalent, bit for bit, to tq_act_quant_fused followed by
 * tq_gemm_mixed_rows with the same split_k: each workgroup quantizes the
 * column tiles of its own split (same closed form) instead of reading codes
 * from memory.  No reference counterpart: the reference always runs the two
 * kernels (src/models/mixed_linear.py:233-239 -> quant_utils.py:119-134 and
 * gemm_rows_splitk_64x64.py:225-323).  Where the rows x columns are too
 * many for the LDS-staged quantizing kernel (e.g. 8+ rows of a 3072-wide
 * input, 4 rows of Gate/Up), and a workspace of
 * tq_linear_mixed_fused_workspace_elems is given, the launch is cooperative
 * instead of split-K: 8 extra workgroups quantize the activation once into the
 * workspace, and the GEMM workgroups, whose weight loads are already in
 * flight, read the codes when the producers are done (a bounded wait; past it
 * a workgroup quantizes by itself).  Same codes either way, so the outputs
 * equal the two-launch sequence's bitwise.  Launches on one stream share its
 * workspace in turn (each leaves the flags and counts zero); launches that
 * overlap on one workspace race.  At 1-2 rows (and where neither the plain
 * kernel nor a cooperative launch applies) the quantizing kernel may carry
 * k / 512 extra helper waves that quantize while its tile waves issue their
 * weights; same tile order, same outputs. */
int tq_linear_mixed_fused(const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                          const int8_t* int8_tiles, const float* int8_scales,
                          const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                          const void* fp16_tiles, const int32_t* fp16_tile_ids,
                          const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                          int out_dtype, const void* bias, int n, int m, int k, int n_tr, int n_tc,
                          int split_k, int tile_layout, float* workspace, int64_t workspace_elems,
                          void* stream);

/* One MixedLinear forward at decode sizes from a prebuilt descriptor: the
 * activation quantization (tq_act_quant_fused into x_int8 / sx) followed by
 * tq_gemm_mixed_rows, or, with fused = 1, tq_linear_mixed_fused -- the same
 * launches, arguments and results as calling those entry points.  Everything
 * but x, out and stream stays fixed between calls, so a caller builds the
 * descriptor once (validating shapes, dtypes, alignment and scratch sizes
 * then) and each call patches three fields and makes one foreign call.
 * Replaces the launch-overhead removal of the reference's CachedLauncher
 * (src/kernels/triton/launch.py:9-79, used at gemm_rows_splitk_64x64.py:275-322
 * and quantize_activation.py:115-155). */
typedef struct tq_linear_desc {
  /* per call */
  const void* x;          /* [n, k] activations, x_dtype, row stride x_stride */
  void* out;              /* [n, m] out_dtype, row stride out_stride */
  void* stream;
  /* fixed */
  int64_t x_stride, out_stride;
  int n, m, k, n_tr, n_tc, x_dtype, out_dtype, tile_layout;
  int fused;              /* 1: one-launch quantize + GEMM (n <= tq_linear_mixed_fused_max_tokens(k)) */
  int8_t* x_int8;         /* [n, k] scratch codes (unused when fused); with TQ_XQ_TOKEN_BLOCKED in
                             tile_layout: [16 ceil(n / 16), k], token-blocked */
  float* sx;              /* [ceil(k/64)] scratch scales (unused when fused) */
  const int8_t* int8_tiles;
  const float* int8_scales;
  const int32_t* int8_tile_ids;
  const int32_t* int8_row_ptr;
  const void* fp16_tiles; /* NULL when the pack has no 16-bit tiles */
  const int32_t* fp16_tile_ids;
  const int32_t* fp16_row_ptr;
  const void* bias;       /* out_dtype [m] or NULL */
  float* workspace;       /* split-K workspace (NULL: automatic plan) */
  int64_t workspace_elems;
} tq_linear_desc;

int tq_linear_forward(const tq_linear_desc* d);

/* Host function: 1 when the automatic GEMM schedule for n rows of a weight
 * with n_tr x n_tc tiles (k = 64 * n_tc) runs faster on token-blocked codes
 * (TQ_XQ_TOKEN_BLOCKED) -- 17..64 rows, and up to 16 rows where the codes do
 * not fit the LDS-staged kernel (more than 144 KiB of them) or a row holds
 * 256+ column tiles (k >= 16384) -- else 0.  No reference counterpart (the
 * reference keeps codes row-major); MixedLinear asks it per row count. */
int tq_gemm_prefers_token_blocked(int n, int k, int n_tr, int n_tc);

/* MEASUREMENT HELPER.  One kernel that reads bytes (a multiple of 16) from a
 * 16-byte aligned device buffer once and writes nothing in practice (sink: 256
 * device words, stored to only if the folded data equals a fixed constant).
 * bench.py times it per launch beside the decode GEMM, over as many bytes as
 * a GEMM launch reads, as the context of the GEMM's HBM roofline fraction.
 * No reference counterpart. */
int tq_read_probe(const void* data, int64_t bytes, uint32_t* sink, void* stream);

/* TEST-ONLY.  Kernel families of the automatic GEMM schedule, as reported by
 * the *_products_i32 entries below. */
enum {
  TQ_KERNEL_DECODE = 1,                 /* LDS-staged decode kernel on given codes (n <= 32) */
  TQ_KERNEL_DECODE_QUANT = 2,           /* the same kernel quantizing the activation itself (n <= 16) */
  TQ_KERNEL_SPLITK = 3,                 /* split-K decode kernel, row-major codes (n <= 64) */
  TQ_KERNEL_SPLITK_TOKEN_BLOCKED = 4,   /* split-K decode kernel, token-blocked codes */
  TQ_KERNEL_SPLITK_QUANT = 5,           /* split-K decode kernel quantizing the activation itself */
  TQ_KERNEL_PREFILL_V5 = 6,             /* prefill DMA ring, two row tiles, 16-bit tiles in the ring */
  TQ_KERNEL_PREFILL_V3 = 7,             /* prefill DMA ring for k > 19456 */
  TQ_KERNEL_PREFILL_ASYNC = 8,          /* prefill DMA ring for k > 32768 */
  TQ_KERNEL_PREFILL_REGISTER = 9,       /* prefill through registers (unaligned rows or k % 64 != 0) */
  TQ_KERNEL_DECODE_COOP = 10,           /* LDS-staged decode kernel, codes from its producer workgroups */
  TQ_KERNEL_DECODE_QUANT_HELP = 11      /* quantizing decode kernel, helper waves quantize */
};

/* TEST-ONLY.  tq_gemm_mixed_rows_planned (prefill_units may be NULL, then it
 * is tq_gemm_mixed_rows) launching the DUMP instantiation of the very kernel
 * the automatic schedule picks for these arguments: besides writing out as
 * usual, every INT8 tile's exact INT32 product -- the v_mfma_i32_16x16x64_i8
 * result before its scale FMA -- is written for the token rows row0 ..
 * row0 + rows - 1 into products, int32 [T8][rows][64]: products[p][i][j] =
 * sum_k x_int8[row0 + i][64 c + k] * W8_p[j][k] for the INT8 tile at position
 * p (column tile c).  *kernel (host pointer, nullable) receives the
 * TQ_KERNEL_* family that ran.  bf16 activations only (TQ_ERR_DTYPE
 * otherwise); 0 <= row0, 1 <= rows <= n - row0.  No reference counterpart: it
 * exposes the quantity the reference's tl.dot produces at
 * src/kernels/triton/gemm_rows_splitk_64x64.py:125-137, for every kernel. */
int tq_gemm_mixed_rows_products_i32(const int8_t* x_int8, int64_t x_int8_stride_n, const float* sx,
                                    const int8_t* int8_tiles, const float* int8_scales,
                                    const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                                    const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                                    const void* fp16_tiles, const int32_t* fp16_tile_ids,
                                    const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                                    int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                                    int n_tc, int split_k, int tile_layout, float* workspace,
                                    int64_t workspace_elems, const int32_t* prefill_units, int n_units,
                                    int n_first, int32_t* products, int row0, int rows, int* kernel,
                                    void* stream);

/* TEST-ONLY.  The same for tq_linear_mixed_fused: the products are those of
 * the codes the kernel computes from x_fp itself. */
int tq_linear_mixed_fused_products_i32(const void* x_fp, int64_t x_fp_stride_n, int x_dtype,
                                       const int8_t* int8_tiles, const float* int8_scales,
                                       const int32_t* int8_tile_ids, const int32_t* int8_row_ptr,
                                       const void* fp16_tiles, const int32_t* fp16_tile_ids,
                                       const int32_t* fp16_row_ptr, void* out, int64_t out_stride_n,
                                       int out_dtype, const void* bias, int n, int m, int k, int n_tr,
                                       int n_tc, int split_k, int tile_layout, float* workspace,
                                       int64_t workspace_elems, int32_t* products, int row0, int rows,
                                       int* kernel, void* stream);

/* ---- decode attention ----------------------------------------------------
 * One query token per sequence over a static KV cache read up to a length
 * held on the device (so a captured graph serves every position):
 *   out[b, h, :] = softmax_t(scale * q[b, h, :] . k[b, t, h / G, :]) v[b, t, h / G, :]
 *   for t < min(seq_used[b], max_len), G = q_heads / kv_heads (<= 8), head_dim 128.
 * q, out: [batch, q_heads, head_dim] with strides (elements) per batch / head;
 * k, v: caches sharing strides per batch / position / kv head, unit stride
 * inside a head.  16-byte aligned pointers, strides multiples of 8.  fp32
 * accumulation; workspace = tq_decode_attention_workspace_elems() fp32 elements
 * (split partials; no initialisation needed).
 * Replaces the torch.ops.aten._flash_attention_forward(..., seqused_k=...)
 * call of _cuda_graph_attention (src/runtime/graph_decode.py:56-71). */
int64_t tq_decode_attention_workspace_elems(int batch, int q_heads, int max_len);
/* The split plan the attention entry points use for a device with `cus`
 * compute units (no GPU needed): *n_splits chunks of each sequence, *waves
 * waves of 32 keys per split workgroup, chosen so every CU gets the same
 * keys.  No reference counterpart (flash-decoding's split heuristic lives
 * inside aten._flash_attention_forward, src/runtime/graph_decode.py:56-71);
 * exposed for tests and capacity planning. */
int tq_decode_attention_plan(int batch, int q_heads, int kv_heads, int max_len, int rope, int cus,
                             int* n_splits, int* waves);
int tq_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                        const void* v, int64_t kv_stride_b, int64_t kv_stride_l, int64_t kv_stride_h,
                        const int32_t* seq_used, void* out, int64_t out_stride_b, int64_t out_stride_h,
                        int dtype, int batch, int q_heads, int kv_heads, int head_dim, int max_len,
                        float scale, float* workspace, int64_t workspace_elems, void* stream);

/* No reference counterpart: tq_decode_attention without a workspace, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  The split records live
 * in a fixed 16 MiB device array of the library, one per GPU, held until the
 * process ends; shapes needing more
 * (tq_decode_attention_workspace_elems(batch, q_heads, max_len) > 4 Mi floats,
 * e.g. batch * q_heads > 504 at long lengths) return TQ_ERR_WORKSPACE.  The
 * stream must belong to the current device.  All calls of one process on one
 * GPU share the array (each process that loads the library has its own copy):
 * overlapping calls from the same process on one GPU (different streams or
 * threads) race and must be serialized by the caller.  Nothing in it needs
 * clearing between calls (each call writes every record it reads).  Results
 * are bitwise those of tq_decode_attention. */
int tq_decode_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                const void* v, int64_t kv_stride_b, int64_t kv_stride_l, int64_t kv_stride_h,
                                const int32_t* seq_used, void* out, int64_t out_stride_b, int64_t out_stride_h,
                                int dtype, int batch, int q_heads, int kv_heads, int head_dim, int max_len,
                                float scale, void* stream);

/* ---- warming the next decode GEMM's weights into the right L2 ---------------
 * On MI355X each of the 8 XCDs has its own L2, and workgroups are dealt to
 * the XCDs round-robin by workgroup id.  The decode GEMM's schedule reads row
 * tile r only from XCD r mod 8 (tq_gemm_l2_warm_ok says for which shapes).  A
 * producer kernel that runs just before such a GEMM (the ones below that
 * take a tq_l2_warm) can then spend its idle memory time reading the GEMM's
 * packed tiles from the XCD that will need them: `blocks` extra workgroups
 * (a multiple of 8, at most 1024) each touch every 64-byte sector of the row
 * tiles r = (its XCD) + 8 j.  The outputs are unchanged; only where the bytes
 * sit when the GEMM starts changes.  warm NULL or blocks == 0: no warm-up.
 * No reference counterpart (a scheduling aid of this build). */
typedef struct tq_l2_warm {
  const void* int8_tiles;         /* the GEMM's packed INT8 tiles [T8, 64, 64] */
  const void* fp16_tiles;         /* its 16-bit tiles [T16, 64, 64], or NULL */
  const int32_t* int8_row_ptr;    /* [n_tr + 1] */
  const int32_t* fp16_row_ptr;    /* [n_tr + 1]; NULL when fp16_tiles is NULL */
  int n_tr;
  int blocks;
} tq_l2_warm;

/* 1 when the automatic schedule of tq_gemm_mixed_rows for these arguments
 * (split_k <= 1, row-major codes, 16-byte aligned rows with k == 64 n_tc)
 * reads row tile r only from XCD r mod 8, else 0. */
int tq_gemm_l2_warm_ok(int n, int k, int n_tr, int n_tc);

/* As tq_decode_attention, and the attention output (the [batch, q_heads *
 * head_dim] input of the next projection) is also quantized like
 * tq_act_quant_fused: q_out int8 with row stride q_out_stride_b, sx_out
 * [q_heads * head_dim / 64].  batch <= 16.  No reference counterpart (the
 * reference quantizes the projection input in a separate launch,
 * src/models/mixed_linear.py:233-239). */
int tq_decode_attention_quant(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                              const void* v, int64_t kv_stride_b, int64_t kv_stride_l, int64_t kv_stride_h,
                              const int32_t* seq_used, void* out, int64_t out_stride_b,
                              int64_t out_stride_h, int8_t* q_out, int64_t q_out_stride_b, float* sx_out,
                              int dtype, int batch, int q_heads, int kv_heads, int head_dim, int max_len,
                              float scale, float* workspace, int64_t workspace_elems, void* stream);

/* tq_rope_cache followed by tq_decode_attention (q_out NULL) or
 * tq_decode_attention_quant, in one split pass: qkv is the stacked [batch,
 * (q_heads + 2 kv_heads) * 128] q/k/v projection output (row stride
 * qkv_stride); cos_table / sin_table are [max_len, 128] (row stride 128) and
 * their rows at *position are the RoPE factors (the row index is clamped into
 * the table).  The split kernel applies RoPE to the q heads it reads, and the
 * workgroup whose key chunk holds *position (the last one when *position is
 * past seq_used) writes that token's rotated k and its v into the caches
 * (nothing is written when *position is outside [0, max_len)) and uses them
 * in registers.  Outputs, codes, scales and cache
 * contents are bitwise those of the two-launch sequence with the table rows.  No reference
 * counterpart: it fuses the Hugging Face rotary embedding and StaticCache
 * update that precede _cuda_graph_attention (src/runtime/graph_decode.py:56-71). */
int tq_decode_attention_rope(const void* qkv, int64_t qkv_stride, const void* cos_table, const void* sin_table,
                             const int64_t* position, void* k_cache, void* v_cache, int64_t cache_stride_b,
                             int64_t cache_stride_l, int64_t cache_stride_h, const int32_t* seq_used, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, int8_t* q_out, int64_t q_out_stride_b,
                             float* sx_out, int dtype, int batch, int q_heads, int kv_heads, int head_dim,
                             int max_len, float scale, float* workspace, int64_t workspace_elems,
                             const tq_l2_warm* warm, void* stream);

/* ---- decode-step producers fused with the activation quantization ---------
 * Each computes a decoder-layer step that feeds a mixed tile GEMM and, when
 * q_out is non-null, quantizes its output like tq_act_quant_fused (scales over
 * ALL n rows, sx_out[k / 64]).  Rounding follows the Hugging Face module code
 * op by op.  n <= 64 rows; widths multiples of 64; 16-bit rows 16-byte
 * aligned.  No reference counterparts: the reference runs the model's own
 * modules and quantizes inside every MixedLinear call
 * (src/models/mixed_linear.py:233-239); these replace those chains inside a
 * captured decode step (src/runtime/graph_decode.py:350-385). */

/* h = x + delta (rounded; skipped when delta is NULL, then h = x and h_out is
 * unused), y = weight * round(h * rsqrt(mean(h^2) + eps)) (LlamaRMSNorm). */
int tq_add_rmsnorm_quant(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                         const void* weight, float eps, void* h_out, int64_t h_stride, void* y_out,
                         int64_t y_stride, int8_t* q_out, int64_t q_stride, float* sx_out, int dtype, int n,
                         int k, const tq_l2_warm* warm, void* stream);

/* y = round(round(silu(gate)) * up) for gate_up = [gate | up] of width 2 * inter. */
int tq_silu_mul_quant(const void* gate_up, int64_t gu_stride, void* y_out, int64_t y_stride, int8_t* q_out,
                      int64_t q_stride, float* sx_out, int dtype, int n, int inter, const tq_l2_warm* warm,
                      void* stream);

/* RoPE (q * cos + rotate_half(q) * sin, head_dim 128) on the q and k heads of
 * a stacked [n, (q_heads + 2 kv_heads) * 128] q/k/v projection output; rotated
 * q to q_out [n, q_heads, 128]; rotated k and v written to the caches at
 * index *position (device int64; no write when outside [0, max_len)).
 * cos / sin: the 128 values at the position. */
int tq_rope_cache(const void* qkv, int64_t qkv_stride, const void* cos, const void* sin, const int64_t* position,
                  void* q_out, int64_t q_stride_b, int64_t q_stride_h, void* k_cache, void* v_cache,
                  int64_t cache_stride_b, int64_t cache_stride_h, int64_t cache_stride_l, int dtype, int n,
                  int q_heads, int kv_heads, int head_dim, int max_len, void* stream);

/* Prefill forms of the glue above, for the B x P rows of a prompt (one wave
 * per row for the norm, elementwise grids otherwise; same element arithmetic
 * as the decode forms).  They replace the modules' RMSNorm (input and
 * post-attention), act_fn(gate) * up, apply_rotary_pos_emb and the static
 * cache update inside the decoder's captured prefill
 * (src/runtime/graph_decode.py:238-268 runs the model's forward there).
 * tq_add_rmsnorm_rows: as tq_add_rmsnorm_quant without the codes, any n,
 * k <= 8192 a multiple of 8, 16-byte aligned rows.
 * tq_silu_mul_rows: as tq_silu_mul_quant without the codes, any n, inter a
 * multiple of 8, 16-byte aligned rows.
 * tq_rope_prefill: row b * prompt_len + p of qkv is token p of sequence b,
 * rotated with row p of the cos / sin tables (row stride table_stride); q to
 * q_out[b, h, p, :] (strides q_stride_b, q_stride_h, q_stride_p), k and v into
 * the caches at index p (prompt_len <= max_len); 16-byte aligned base pointers,
 * every stride a multiple of 8 elements. */
int tq_add_rmsnorm_rows(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                        const void* weight, float eps, void* h_out, int64_t h_stride, void* y_out, int64_t y_stride,
                        int dtype, int n, int k, void* stream);
int tq_silu_mul_rows(const void* gate_up, int64_t gu_stride, void* y_out, int64_t y_stride, int dtype, int n,
                     int inter, void* stream);
int tq_rope_prefill(const void* qkv, int64_t qkv_stride, const void* cos, const void* sin, int64_t table_stride,
                    void* q_out, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_p, void* k_cache,
                    void* v_cache, int64_t cache_stride_b, int64_t cache_stride_h, int64_t cache_stride_l, int dtype,
                    int batch, int prompt_len, int q_heads, int kv_heads, int head_dim, int max_len, void* stream);

/* Greedy decoding step on the device: next_token[b] = token[b] = argmax_v
 * logits[b, v] (torch.argmax order: NaN first, lowest index among equals),
 * generated[b, *position - prompt_len + 1] = that token (no write outside
 * [0, generated_len) or when generated is NULL), then *position += 1 and
 * seq_used[b] = *position + 1 (seq_used nullable).  batch <= 256; logits
 * 16-bit [batch, vocab] with row stride logits_stride; workspace =
 * tq_greedy_step_workspace_elems(batch) int32 elements.  Replaces the
 * argmax / scatter / token copy / position update of the reference's captured
 * decode loop (src/runtime/graph_decode.py:347-385). */
int64_t tq_greedy_step_workspace_elems(int batch);
int tq_greedy_step(const void* logits, int64_t logits_stride, int dtype, int batch, int vocab, int32_t* workspace,
                   int64_t workspace_elems, int64_t* next_token, int64_t* token, int64_t* generated,
                   int64_t generated_stride, int generated_len, int64_t* position, int prompt_len,
                   int32_t* seq_used, void* stream);

/* ---- load-time packing -------------------------------------------------
 * w [m, k] (x_dtype, row stride w_stride_m) is read as if zero-padded to
 * multiples of 64.  tile_ids are flat ids r * n_tc + c.                  */

/* Replaces the INT8 branch of _pack_weight_with_tile_ids (src/kernels/pack.py:119-167):
 * per tile sw = 1 if a == 0 else f32(a) / 127, codes clamp(rint(f32(w) / sw)).
 * col_importance (nullable, fp32 [n_tc * 64]) selects the IAA search over
 * sw * {0.75, 1, 1.25} (pack.py:132-159): lowest mean((dq - w)^2 * max(imp, 1e-8)),
 * first candidate kept on ties.  Tiles are written in `layout`. */
int tq_pack_int8_tiles(const void* w, int64_t w_stride_m, int w_dtype, int m, int k,
                       const int32_t* tile_ids, int64_t n_tiles, int n_tc, int layout,
                       const float* col_importance, int8_t* tiles, float* scales,
                       void* stream);

/* Replaces the 16-bit branch of _pack_weight_with_tile_ids (pack.py:172-175):
 * copies the selected tiles unchanged, in `layout`. */
int tq_pack_16bit_tiles(const void* w, int64_t w_stride_m, int w_dtype, int m, int k,
                        const int32_t* tile_ids, int64_t n_tiles, int n_tc, int layout,
                        void* tiles, void* stream);

/* No reference counterpart (the reference has one tile order): converts
 * n_tiles packed tiles of elem_bytes (1 or 2) between layouts.  src and dst
 * must not overlap. */
int tq_tiles_relayout(const void* src, void* dst, int64_t n_tiles, int elem_bytes,
                      int from_layout, int to_layout, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TILEQUANT_H */
