// Internal interface between the HIP kernel files and the runtime
// (runtime.hip).  Nothing here crosses the public C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "akasha_hip.h"

namespace akh {

// Rows of the batched decode path: every fused decode kernel holds all
// sequences of a step in one or two 32-row MFMA tiles (activations
// [tiles][K/4][32][4]), so each weight byte is read once per step for up to
// 64 sequences.
constexpr int kMaxBatch = 64;

// ---------------------------------------------------------------------------
// Per-shader launchers (shader_kernels.hip): the reference Shader semantics,
// metas read from device memory when the kernel runs.
// ---------------------------------------------------------------------------

hipError_t shader_embedding(const uint32_t* tokens, const float* table,
                            float* out, akh_embedding_meta shape,
                            const akh_embedding_meta* meta, hipStream_t s);
hipError_t shader_rmsnorm(const float* x, const float* w, float* out,
                          akh_norm_meta shape, const akh_norm_meta* meta,
                          hipStream_t s);
// MATMUL / GEMV (accumulate = 0) and MATMUL_ADD / GEMV_ADD (accumulate = 1).
// `ws` (kGemvWsFloats floats) and `cnt` (kGemvSlabs counters, zero between
// launches) serve the K-split small-m path; null: one split.
constexpr size_t kGemvWsFloats = (size_t)4 << 20;
constexpr int kGemvSlabs = 1 << 16;
hipError_t shader_matmul(const float* a, const float* b, float* c,
                         akh_matmul_meta shape, const akh_matmul_meta* meta,
                         int accumulate, float* ws, int* cnt, hipStream_t s);
hipError_t shader_head_gather(const float* src, float* dst,
                              akh_head_move_meta shape,
                              const akh_head_move_meta* meta, hipStream_t s);
hipError_t shader_rope(float* buf, uint32_t seq_len, uint32_t dim,
                       const uint32_t* meta_u32, int with_offset,
                       hipStream_t s);
hipError_t shader_cache_write(const float* src, float* cache,
                              akh_cache_write_meta shape,
                              const akh_cache_write_meta* meta, hipStream_t s);
hipError_t shader_flash_attention(const float* q, const float* k,
                                  const float* v, float* out, float* lse,
                                  akh_flash_attn_meta shape,
                                  const akh_flash_attn_meta* meta,
                                  uint32_t batch, hipStream_t s);
hipError_t shader_attn_qk_cached(const float* q, const float* kc,
                                 float* scores, uint32_t num_heads,
                                 uint32_t max_attn_len,
                                 const akh_attn_cached_meta* meta,
                                 hipStream_t s);
hipError_t shader_softmax_rect(float* x, akh_softmax_rect_meta shape,
                               const akh_softmax_rect_meta* meta,
                               hipStream_t s);
hipError_t shader_attn_av_cached(const float* scores, const float* vc,
                                 float* out, uint32_t dim,
                                 const akh_attn_cached_meta* meta,
                                 hipStream_t s);
hipError_t shader_silu(float* buf, uint32_t len, hipStream_t s);
hipError_t shader_qkv_split(const float* src, float* q, float* k, float* v,
                            akh_head_move_meta shape, const akh_head_move_meta* meta,
                            hipStream_t s);
hipError_t shader_rope_qk(float* q, float* k, akh_rope_meta shape, const akh_rope_meta* meta,
                          hipStream_t s);
hipError_t shader_add(const float* a, const float* b, float* out, uint32_t len, hipStream_t s);
hipError_t shader_silu_out(const float* x, float* out, uint32_t len, hipStream_t s);
// CROSS_ENTROPY over `rows` rows (grid); the live meta bounds the work.
hipError_t launch_cross_entropy(float* logits, const uint32_t* targets, float* losses,
                                uint32_t rows, const akh_cross_entropy_meta* meta,
                                hipStream_t s);
hipError_t shader_argmax_rows(const float* logits, uint32_t rows, uint32_t n,
                              uint32_t* out, hipStream_t s);

// ---------------------------------------------------------------------------
// Prefill (prefill_kernels.hip)
// ---------------------------------------------------------------------------

enum GemmEpi : int {
  GEMM_STORE = 0,  // C = A B
  GEMM_ADD = 1,    // C += A B          (fused residual)
  GEMM_SILU = 2,   // C = silu(A B)     (ffn_up + SILU)
  GEMM_QKV = 3,    // RoPE(Q), RoPE(K) -> cache, V -> cache
};

struct GemmParams {
  const float* a;  // [M, K] row-major
  const float* b;  // [K, N] row-major
  float* c;        // [M, N]
  int M, N, K;
  const akh_matmul_meta* meta;  // if set, M, N, K are read from it
  // GEMM_QKV: rows are sequence-major (row = seq * S + t, position t).
  float* q_out;
  float* kcache;
  float* vcache;
  long seq_stride;
  int S;
  const float2* rope;  // [max_ctx, head_dim / 2] (cos, sin)
  int dim, head_dim;
  // bfloat16 path (launch_gemm_bf16): the transposed weights in bfloat16
  // and A either in bfloat16 (a16) or fp32 (a, split into hi + lo parts).
  const uint16_t* a16;   // [M, K]
  const uint16_t* bt16;  // [N, K]
  // launch_gemm_x6 / launch_gemm_h3: the transposed fp32 weights.
  const float* bt;  // [N, K]
  // launch_gemm_h3: the weights' fp16 planes (launch_split_weights_f16),
  // and a flag set to 1 when a result is not finite.
  const uint16_t* bp16;
  int* range_flag;
  // GEMM_QKV on ragged prompts packed back to back: row m is position
  // rowmap[m].y of sequence rowmap[m].x (instead of m / S, m % S).
  const int2* rowmap;
  // GEMM_QKV: K and V rows go to kcache / vcache at row m (rows packed like
  // the prompt's) instead of sequence * seq_stride + position.
  int kv_packed;
  // launch_gemm_bf16 with an fp32 A: round A to bfloat16 (one product)
  // instead of splitting it into hi + lo (two).
  int a_hi_only;
  // launch_gemm with a workspace (kGemvWsFloats floats, kGemvSlabs counters
  // at zero): grids too small for the part split K over several blocks per
  // tile.  Null: no split.
  float* split_ws;
  int* split_cnt;
  int split_kc;  // set by launch_gemm: rows of K per split
};

enum { FLASH_X6 = 1, FLASH_H3 = 2, FLASH_FP32 = 3 };  // FlashParams::x6

struct FlashParams {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  float* lse;              // optional [S, H] per sequence: max + ln(sum)
  long q_bs, kv_bs, o_bs;  // per-sequence strides (elements)
  long lse_bs;             // per-sequence stride of lse
  int S, d, hd;
  float scale;
  const akh_flash_attn_meta* meta;  // per-shader path: S, dim, scale and
                                    // row_offset come from it (1 sequence)
  uint16_t* o16;  // launch_flash_bf16: bfloat16 output (o unused)
  int x6;         // launch_flash, head_dim 64 / 128: split-bfloat16 MFMAs
                  // (fp32 accuracy) instead of fp32 MFMAs; FLASH_H3: split
                  // fp16 MFMAs (fp32 accuracy), setting *range_flag when an
                  // operand is beyond fp16's range (grids of fewer blocks
                  // than CUs recompute such tiles themselves); FLASH_FP32:
                  // fp32 accuracy without a flag (split-fp16 tiles that
                  // recompute themselves on split-bfloat16; split-bfloat16
                  // throughout for head size 128 on large grids)
  int* range_flag;
  // Ragged prompts packed back to back: sequence b's rows of q, o (and lse)
  // are [rows_at[b], rows_at[b + 1]) and its length is their count (S is
  // then the longest); K and V rows likewise if kv_packed, else at
  // b * kv_bs.  Null: the uniform layout above.
  const int* rows_at;
  int kv_packed;
};

hipError_t launch_gemm(const GemmParams& p, int epi, hipStream_t s);
hipError_t launch_flash(const FlashParams& p, int batch, int max_rows,
                        hipStream_t s);
hipError_t launch_rows_rmsnorm(const float* x, const float* w, float* out,
                               int rows, int size, float eps, hipStream_t s);

// The optional bfloat16-MFMA prefill: bfloat16 MFMA operands (round to
// nearest even), fp32 accumulation, fp32 residual stream and KV cache.
// Weights are read from a transposed bfloat16 copy [N, K]; A is p.a16
// (bfloat16) or p.a (fp32, entering as hi + lo bfloat16 parts).  K % 8 == 0.
hipError_t launch_gemm_bf16(const GemmParams& p, int epi, hipStream_t s);
// wt[n, k] = bf16(w[k, n]) for a [K, N] row-major matrix.
hipError_t launch_transpose_bf16(const float* w, int K, int N, uint16_t* wt, hipStream_t s);
// fp32-accurate GEMM on bfloat16 MFMAs: A (p.a, fp32 [M, K]) and the
// transposed fp32 weights (p.bt, [N, K]) enter as three bfloat16 terms
// each, six products accumulated in fp32.  K % 8 == 0.
hipError_t launch_gemm_x6(const GemmParams& p, int epi, hipStream_t s);
// fp32-accurate GEMM on fp16 MFMAs: A (p.a, fp32 [M, K]) split into two fp16
// terms as it is staged, the weights' fp16 planes (p.bp16), three products
// per multiply-add.  Sets *p.range_flag when a result is not finite (an
// operand beyond fp16's range); the caller then recomputes in fp32.  K % 8 == 0.
hipError_t launch_gemm_h3(const GemmParams& p, int epi, hipStream_t s);
// The fp16 planes of a [K, N] row-major matrix for launch_gemm_h3 (K * N * 4 bytes).
hipError_t launch_split_weights_f16(const float* w, int K, int N, uint16_t* wp, hipStream_t s);
// wt[n, k] = w[k, n] for a [K, N] row-major matrix.
hipError_t launch_transpose_f32(const float* w, int K, int N, float* wt, hipStream_t s);
// Causal flash attention (head_dim 64 or 128) with bfloat16 QK^T and PV
// MFMAs; writes p.o16.
hipError_t launch_flash_bf16(const FlashParams& p, int batch, int max_rows, hipStream_t s);
hipError_t launch_embedding_rows(const uint32_t* tokens, const float* table,
                                 float* out, int rows, int d, uint32_t vocab,
                                 hipStream_t s);

// ---------------------------------------------------------------------------
// Batched decode (decode_kernels.hip).  Activations that feed a GEMM live in
// the k-quad layout [K/4][32][4] (see kq_index in common.h).
// ---------------------------------------------------------------------------

enum DecEpi : int {
  DEC_PART = 0,    // y[split, m, n] = partial tile of K chunk `split`
  DEC_PART_T = 1,  // the same, each partial tile in the k-quad layout
  DEC_LOGITS = 2,  // y[m, n] = whole-K result + per-tile argmax partials
  DEC_SILU_T = 3,  // y = silu(whole-K result) in the k-quad layout (one split)
  // k-quad partial tiles as DEC_PART_T; the last block of each column tile
  // then adds their sum to the residual rows `res` and writes the tile's
  // per-row sums of squares (the residual add of the next RMSNorm).
  DEC_RESID = 4,
};

enum DecPro : int {
  PRO_NONE = 0,        // A = xt
  PRO_SILU_SUM = 1,    // A = silu(sum of nparts k-quad partial tiles at xt)
  PRO_ATTN_MERGE = 2,  // A = merge of nparts attention splits (xt, ml)
  PRO_NORM = 3,        // A = RMSNorm(xt) * gain, from the sums of squares ssq
};

// Most splits of one (sequence, head) attention.
constexpr int kMaxAttnSplits = 4;

// Roles of the decode GEMMs; each has its own launch shape.
enum DecCfg : int {
  DEC_CFG_QKV = 0,   // qkv_proj  -> partials (summed by attention)
  DEC_CFG_OUT = 1,   // out_proj  -> residual add (DEC_RESID)
  DEC_CFG_UP = 2,    // ffn_up    -> k-quad partials (summed by down)
  DEC_CFG_DOWN = 3,  // ffn_down on silu(sum) -> residual add (DEC_RESID)
  DEC_CFG_LM = 4,    // lm_head   -> logits + argmax partials
};

struct DecGemmParams {
  const float* xt;  // A operand (k-quad), or nparts k-quad partial tiles
  int nparts;
  const float* w;   // weights packed by launch_pack_tiles (Kp rows per tile)
  int wbf16;        // w holds bfloat16 k-octet tiles
  int wh3;          // lm_head only: w holds fp16 hi/lo k-octet tiles (launch_pack_lm_h3)
  int M, N, K, Kp;
  float* y;         // partial tiles or logits
  uint2* amax;      // DEC_LOGITS: [32, parts] (value bits, index)
  const float2* ml;  // PRO_ATTN_MERGE: per split (max, sum) [nparts][K/hd][32]
  int hd;            // PRO_ATTN_MERGE: head_dim
  int kpass;         // set by the launcher: K passes per block (grid.y chunks)
  int mt;            // 32-row tiles of the rows (1 or 2); partial tiles and
                     // attention splits hold 32 * mt rows
  // PRO_NORM: xt holds the residual rows; A = xt * rs(m) * gain with
  // rs(m) = 1 / sqrt(sum_t ssq[m, t] / K + eps) over the K / 32 column tiles.
  const float* ssq;
  const float* gain;
  float eps;
  // DEC_RESID: res (k-quad, [32 * mt][N] residual rows) += the sum of the
  // partial tiles at y; ssq_out[m, tile] = sum over the tile's 32 columns of
  // the new res[m, n]^2.  count[tile] (zero between launches) counts the
  // finished blocks of a column tile.
  float* res;
  float* ssq_out;
  int* count;
};

// Decode weights are read from a copy packed once at upload: 32-column
// tiles, each [Kp/4][32][4] (element (k, n) of tile t = n / 32 at
// ((k / 4) * 32 + n % 32) * 4 + k % 4), zero-filled beyond K and N.  A block
// streams one contiguous region, and a lane's float4 holds four consecutive
// k of its column: four MFMA B operands in one load.  With bf16 the tiles
// hold bfloat16 k-octets instead (element (k, n) at ((k / 8) * 32 + n % 32)
// * 8 + k % 8), for matrices whose values are all bfloat16: half the bytes,
// the same products.
hipError_t launch_pack_tiles(const float* w, int K, int N, int Kp, float* out, bool bf16,
                             hipStream_t s);
// *flag |= 1 if any of w[0..n) is not a bfloat16 value (low 16 bits set).
hipError_t launch_check_bf16(const float* w, size_t n, int* flag, hipStream_t s);
// The persistent lm_head's split-fp16 tiles: element (k, n) of tile
// t = n / 32 as two fp16 terms (w = hi + 2^-11 lo to within 2^-22 |w|) at
// (((k / 8) * 32 + n % 32) * 2 + plane) * 8 + k % 8, the same 4 bytes per
// element as the float tiles (Kp a multiple of 8).  *flag = 1 if a weight is
// beyond fp16's range (|w| >= 65520: the tiles are then unusable).
hipError_t launch_pack_lm_h3(const float* w, int K, int N, int Kp, uint16_t* out, int* flag,
                             hipStream_t s);
// Whether the lm_head of a (K, N) matrix runs the persistent kernel for
// sessions of one and two row tiles (its tiles may then be split-fp16).
bool dec_lm_h3_capable(int K, int N);
// Rows Kp of a role's packed tiles (K rounded up to 8, or more for
// lm_head's padding).
int dec_packed_rows(int role, int K);
// Whether a role's GEMM for [K, N] weights runs on bfloat16 tiles.
bool dec_bf16_capable(int role, int K, int N);

// Number of K chunks (partial tiles) a role's GEMM produces for contraction
// length K.
int dec_gemm_splits(int role, int K, int N);
// Whether the RMSNorm folds into the decode GEMMs (PRO_NORM / DEC_RESID)
// for a residual width of K: a multiple of 128, at most 4096.
bool dec_norm_fusable(int K);
// Whether a model of dim d, head size hd and ffn_hidden F decodes on the
// batched kernels (else on decode_generic.hip's).
bool dec_fast_shape(int d, int hd, int F);
hipError_t launch_dec_gemm(const DecGemmParams& p, int role, hipStream_t s);

// lm_head: logits y[M, N] = xt . w and argmax partials amax[M, parts], where
// parts = dec_lm_parts(N, K, num_cus, mt, h3) (each the first maximum of the
// row over a subset of the columns; h3: the tiles are split-fp16).  The
// float tiles' count is the larger: size buffers with h3 = false.
int dec_lm_parts(int N, int K, int num_cus, int mt, bool h3);
hipError_t launch_dec_lm(const DecGemmParams& p, int num_cus, hipStream_t s);

struct DecAttnParams {
  const float* qkv;  // nparts partial tiles [nparts][rows][3*d]
  int nparts;
  const float2* rope;  // [max_ctx, head_dim / 2] (cos, sin)
  void* kc;          // sequence b at kc + b * seq_stride, rows of d elements
  void* vc;          // (float, or bfloat16 when kv16)
  int kv16;
  float* out_t;      // per split, unnormalised o in k-quad tiles
                     // [splits][rows / 32][d/4][32][4]
  float2* ml;        // per split (max, sum) [splits][H][rows]
  const int* pos;    // position of the new token of each sequence
  const int* active;  // sequences with active[b] == 0 are skipped (none if null)
  long seq_stride;
  int H, d;
  float scale;
  int rows;          // 32 * the row tiles of the session
};

// act = silu(sum of nparts k-quad partial tiles), n elements per tile,
// summed in split order (what PRO_SILU_SUM computes while loading A).
hipError_t launch_silu_sum(const float* parts, int nparts, float* act, size_t n,
                           hipStream_t s);

// Splits per (sequence, head): the partial states the out_proj GEMM merges,
// for a session of `batch` sequences, `heads` heads and context max_ctx
// (launch_dec_attn picks the same launch shape from the same facts), and
// the most any session uses (the size of its split buffers).
int dec_attn_splits(int batch, int heads, long max_ctx, bool kv16);
int dec_attn_max_splits();
// Prefill rows k, v [rows, d] (fp32) into a bfloat16 KV cache (sequence b
// at b * seq_stride, position t at t * d): row = b * S + t, or, for ragged
// prompts packed back to back, (b, t) = rowmap[row].
hipError_t launch_kv_store_bf16(const float* k, const float* v, uint16_t* kc, uint16_t* vc,
                                size_t rows, int S, int d, long seq_stride,
                                const int2* rowmap, hipStream_t s);
// Decode for shapes the batched decode kernels do not take
// (decode_generic.hip): activations in row-major rows [B, *].
struct GenAttnParams {
  const float* qkv;     // [B, 3d]: q, k, v of the step's token
  const float2* rope;   // [max_ctx, hd / 2] (cos, sin)
  void* kc;             // layer's K cache: sequence b at b * seq_stride (f32 or bf16)
  void* vc;
  long seq_stride;      // elements
  const int* pos;       // per-sequence position of the token
  const int* active;    // optional: rows with 0 are skipped
  float* out;           // [B, d]
  int d, hd;
  float scale;
  int kv16;
};
hipError_t launch_gen_attn(const GenAttnParams& p, int batch, hipStream_t s);
// The first-max partial (value bits, index) of each of `rows` rows of n logits.
hipError_t launch_gen_argmax_part(const float* logits, int rows, int n, uint2* part,
                                  hipStream_t s);
// dst row m = src row (src_rows ? src_rows[m] : row0 + m * row_stride), d floats.
hipError_t launch_gen_gather_rows(const float* src, float* dst, int rows, int d, long row0,
                                  long row_stride, const int* src_rows, hipStream_t s);

// N(0, 1) values (hash of seed and element offset) in rows [0, len) of
// `planes` KV planes of [max_ctx][d] (f32, or bfloat16 when kv16).
hipError_t launch_fill_kv_synthetic(void* kv, bool kv16, size_t planes, int len, int d,
                                    long max_ctx, uint64_t seed, hipStream_t s);
// With t0 and t1 set, the dispatch records them at its own start and end.
hipError_t launch_dec_attn(const DecAttnParams& p, int batch, int hd,
                           hipStream_t s, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);

// Per-row residual update + RMSNorm: x = table[ids[m]] (zero row if the id
// is out of vocab), or src row (row0 + m * row_stride), or xt + the sum of
// nparts row-major partial tiles [nparts][32][d]; xt <- x (k-quad) and
// xnt <- x * rsqrt(mean(x^2) + eps) * gain (k-quad).
struct RowsNormParams {
  const float* table;
  const uint32_t* ids;
  uint32_t vocab;
  const float* src;
  long row0, row_stride;
  const int* src_rows;  // if set, row m of src is src_rows[m] (ragged last rows)
  const float* parts;
  int nparts;
  float* xt;
  const float* gain;
  float eps;
  float* xnt;
  int d;
  int rows;  // 32 * the row tiles: xt / xnt are [rows / 32][d/4][32][4] and
             // the partial tiles [nparts][rows][d]
  // If set: xt already holds the residual rows and ssq[m, d / 32] their
  // per-column-tile sums of squares (DEC_RESID); only xnt is written.
  const float* ssq;
};

hipError_t launch_rows_norm(const RowsNormParams& p, int M, hipStream_t s);

// Greedy token per row from the lm_head partials; with `logits` (row m at
// m * lstride), a row whose first logit is NaN takes token 0, as the
// reference's scan from index 0 does.  With `pos`, also the
// decode step's bookkeeping on the device: hist[m, pos] = consumed token,
// hist[m, pos + 1] = chosen token, pos[m] += 1.  Without it (prefill) the
// chosen token is recorded at hist[m, next_pos], or at hist[m, at[m]] when
// `at` is given (ragged prompts).
hipError_t launch_argmax_final(const uint2* part, int ntiles, int M,
                               uint32_t* tok, int* pos, uint32_t* hist,
                               int hist_stride, int next_pos, hipStream_t s,
                               const int* at = nullptr, const float* logits = nullptr,
                               long lstride = 0);

// ---------------------------------------------------------------------------
// Token sampling (sample_kernels.hip): sample_token of sampling.rs:3-81 per
// row of logits, with the draw of rand::random() given per row.
// ---------------------------------------------------------------------------

constexpr int kMaxSampleVocab = 1 << 20;  // seen-id bitmap held in LDS

struct SampleArgs {
  const float* logits;  // row m at logits + m * row_stride
  int n;
  long row_stride;
  float temperature;
  int top_k;
  float top_p;
  float penalty;             // repetition penalty (1 = off)
  const uint32_t* seen;      // row m's seen ids at seen + m * seen_stride
  long seen_stride;
  const uint32_t* seen_len;  // [rows]
  const double* uniform;     // [rows] draws in [0, 1)
  double* wbuf;              // scratch, sample_scratch_bytes(rows, n)
  uint32_t* out;             // [rows]
  // Per-row arrival counters, zero between launches (kSampleCounters of
  // them), or nullptr: with them a row sampled with 0 < top_k <= 256 may be
  // split over several blocks whose last one merges the parts.
  int* cnt;

  // Session mode (tok != nullptr), one round of InferenceSession::generate
  // (inference.rs:303-323) per launch.  A row with done[m] set is skipped
  // (active[m] = 0).  Otherwise its seen ids are hist[m, start[m] .. pos[m])
  // (this call's prompt and generated tokens), its draw is
  // uniform[count[m] * rows + m], and its pick p is recorded:
  // gen[m, count[m]++] = p, hist[m, pos[m]] = p, tok[m] = p; active[m] =
  // (p != eos && pos[m] < max_ctx) -- the token is decoded next -- and
  // done[m] once it stopped or produced max_new tokens.
  uint32_t* tok;
  const int* pos;
  uint32_t* hist;
  long hist_stride;
  const int* start;
  int* active;
  int* done;
  uint32_t* count;
  uint32_t* gen;  // [rows, max_new]
  int max_new;
  int max_ctx;
  uint32_t eos;
};

size_t sample_scratch_bytes(int rows, int n);
constexpr int kSampleCounters = 4096;

// The allocation-free sampler's workspace: a device array of
// kNoAllocSampleElems doubles (rows * n at most), one copy per GPU.
// sample_noalloc_scratch resolves its address on `device`, which must be the
// current device, once per device (later calls return the kept address).
constexpr size_t kNoAllocSampleElems = (size_t)1 << 21;
constexpr int kMaxDevices = 64;
hipError_t sample_noalloc_scratch(int device, double** ptr);
hipError_t launch_sample_rows(const SampleArgs& a, int rows, hipStream_t s);
// pos[m] += active[m] for m < rows: the positions of the rows decoded.  With
// tok, each active row first records its decoded token tok[m] at
// hist[m, pos[m]].
hipError_t launch_advance(int* pos, const int* active, int rows, hipStream_t s,
                          const uint32_t* tok = nullptr, uint32_t* hist = nullptr,
                          long hist_stride = 0);

}  // namespace akh
