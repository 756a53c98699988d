// Internal interface between the HIP kernels (kernels.hip) and the runtime
// (runtime.hip).  Nothing here crosses the public C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "akasha_hip.h"

namespace akh {

// Rows of the batched decode path: every fused decode kernel holds all
// sequences of a step in one 32-row MFMA tile.
constexpr int kMaxBatch = 32;
// Column-slot width of the sum-of-squares partials that carry RMSNorm
// statistics from a residual GEMM epilogue to the next GEMM's prologue.
constexpr int kSlotW = 32;

enum Epi : int {
  EPI_STORE = 0,   // Y = acc                    (MATMUL / GEMV)
  EPI_ADD = 1,     // Y += acc                   (MATMUL_ADD / GEMV_ADD)
  EPI_SILU = 2,    // Y = silu(acc)              (ffn_up + SILU)
  EPI_QKV = 3,     // RoPE(Q), RoPE(K) + KV-cache append, V append
  EPI_LOGITS = 4,  // Y = acc + per-tile argmax partials
};

// Skinny GEMM, M <= 32 rows: Y[M,N] (epi) X[M,K] . W[K,N].
struct SkinnyParams {
  const float* x;
  const float* w;
  float* y;
  int M, N, K;
  const akh_matmul_meta* meta;  // if set, M, N, K are read from it
  int ksplit;                   // work-groups along K
  float* ws;                    // split-K partials
  unsigned* cnt;                // per-N-tile arrival counters (zeroed)
  // RMSNorm prologue: a = x * rsqrt(sum(ss_in[m,:]) / K + eps) * gain[k]
  const float* ss_in;
  int ss_slots;
  const float* gain;
  float eps;
  // EPI_ADD: ss_out[m, tile] = sum of squares of the new Y over the tile
  float* ss_out;
  // EPI_QKV
  float* q_out;       // [M, dim]
  float* kcache;      // sequence m at kcache + m * seq_stride
  float* vcache;
  long seq_stride;    // elements between sequences' caches
  const int* pos;     // per-row cache position
  const float2* rope; // [max_ctx, head_dim/2] (cos, sin)
  int dim, head_dim;
  // EPI_LOGITS
  uint2* amax;        // [M, ntiles] (value bits, index)
};

// Tiled MFMA GEMM for M > 32 (prefill).
struct GemmParams {
  const float* a;
  const float* b;
  float* c;
  int M, N, K;
  const akh_matmul_meta* meta;
  // EPI_QKV (rows are sequence-major: row = seq * S + t, position t)
  float* q_out;
  float* kcache;
  float* vcache;
  long seq_stride;
  int S;
  const float2* rope;
  int dim, head_dim;
};

// Causal attention for prefill.
struct FlashParams {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  float* lse;          // optional [S, H]: max + ln(sum)
  long q_bs, kv_bs, o_bs;  // per-sequence strides (elements)
  int S, d, hd, H;
  float scale;
  const akh_flash_attn_meta* meta;  // per-shader path: read S, dim, scale,
                                    // row_offset from it (one sequence)
};

// Single-query attention over the KV cache (decode), split along T.
struct DecodeAttnParams {
  const float* q;      // [B, d]
  const float* kc;     // sequence b at kc + b * seq_stride, rows of d
  const float* vc;
  float* out;          // [B, d]
  const int* pos;      // attends to rows 0..pos[b]
  float* ws;
  unsigned* cnt;
  long seq_stride;
  int B, H, d, nsplit;
  float scale;
};

hipError_t launch_skinny(const SkinnyParams& p, int epi, bool norm,
                         int grid_x, hipStream_t s);
hipError_t launch_gemm(const GemmParams& p, int epi, int grid_x, int grid_y,
                       hipStream_t s);
hipError_t launch_flash(const FlashParams& p, int batch, int max_rows,
                        hipStream_t s);
hipError_t launch_decode_attn(const DecodeAttnParams& p, int hd,
                              hipStream_t s);
// dst[m, :] = row m's source (table[ids[m]] or src[m * S + S - 1]) and
// ss[m, slot] = sum of its squares per kSlotW columns.
hipError_t launch_gather_rows(const float* table, const uint32_t* ids,
                              uint32_t vocab, const float* src, long src_row0,
                              long src_row_stride, float* dst, int M, int d,
                              float* ss, hipStream_t s);
// Greedy token per row from the lm_head partials; with `pos` it also does
// the decode step's bookkeeping (token history, position advance), without
// it records the token at `next_pos` of the history (prefill).
hipError_t launch_argmax_final(const uint2* part, int ntiles, int M,
                               uint32_t* tok, int* pos, uint32_t* hist,
                               int hist_stride, int next_pos, hipStream_t s);
hipError_t launch_rows_rmsnorm(const float* x, const float* w, float* out,
                               int rows, int size, float eps, hipStream_t s);
hipError_t launch_embedding_rows(const uint32_t* tokens, const float* table,
                                 float* out, int rows, int d, uint32_t vocab,
                                 hipStream_t s);

// Per-shader launchers (live device metas).
hipError_t shader_embedding(const uint32_t* tokens, const float* table,
                            float* out, akh_embedding_meta shape,
                            const akh_embedding_meta* meta, hipStream_t s);
hipError_t shader_rmsnorm(const float* x, const float* w, float* out,
                          akh_norm_meta shape, const akh_norm_meta* meta,
                          hipStream_t s);
hipError_t shader_head_gather(const float* src, float* dst,
                              akh_head_move_meta shape,
                              const akh_head_move_meta* meta, hipStream_t s);
hipError_t shader_rope(float* buf, uint32_t seq_len, uint32_t dim,
                       const uint32_t* meta_u32, int with_offset,
                       hipStream_t s);
hipError_t shader_cache_write(const float* src, float* cache,
                              akh_cache_write_meta shape,
                              const akh_cache_write_meta* meta, hipStream_t s);
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
hipError_t shader_argmax_rows(const float* logits, uint32_t rows, uint32_t n,
                              uint32_t* out, hipStream_t s);

}  // namespace akh
