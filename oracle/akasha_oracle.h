/*
 * akasha_oracle.h -- CPU restatement of the akasha-core inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend and the "port" CPU baseline timed by bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (libakasha_hip.so) never links or calls it.
 *
 * Every function restates one reference function (file:line under the
 * akasha-core source tree, paths relative to its root) with the same loop
 * order and the same f32 left-fold summations, so results are bit-faithful to
 * the reference CPU backend wherever the reference defines the order.  Build
 * with -ffp-contract=off (no fused multiply-add: Rust never contracts).
 *
 * Parity pinning (what checks each function beyond retyping it) is listed per
 * function in tests/test_oracle.py.  One row is tolerance-pinned only: the
 * GEMM/GEMV summation order of the absent wilupgu builtins (assumed textbook,
 * k ascending).
 */
#ifndef AKASHA_ORACLE_H
#define AKASHA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic generators ------------------------------------------ */

/* src/nn/ops/emit.rs:910-921 (rand_vec): LCG, 24 high bits -> [-1, 1]. */
void ora_rand_vec(float* out, size_t n, uint64_t seed);
/* src/nn/train.rs:818-828 (rand_tokens): same LCG, (state >> 33) % vocab. */
void ora_rand_tokens(uint32_t* out, size_t n, uint32_t vocab, uint64_t seed);

/* ---- kernels (src/shaders/cpu.rs and the wilupgu builtins) ------------- */

/* cpu.rs:25-41 */
void ora_embedding(const uint32_t* tokens, const float* table, float* out,
                   uint32_t vocab_size, uint32_t dim, uint32_t seq_len);
/* cpu.rs:205-222 */
void ora_rmsnorm(const float* x, const float* w, float* out, uint32_t rows,
                 uint32_t size, float eps);
/* wilupgu MATMUL / GEMV (emit.rs:19-57; layout pinned by emit.rs:1449-1455):
 * C[m,n] = sum_k A[m,k] * B[k,n], k ascending left fold from 0. */
void ora_matmul(const float* a, const float* b, float* c, uint32_t m,
                uint32_t n, uint32_t k);
/* wilupgu MATMUL_ADD / GEMV_ADD (emit.rs:91-126): C[m,n] += (sum_k ...). */
void ora_matmul_add(const float* a, const float* b, float* c, uint32_t m,
                    uint32_t n, uint32_t k);
/* cpu.rs:238-255 */
void ora_head_gather(const float* src, float* dst, uint32_t seq_len,
                     uint32_t full_dim, uint32_t head_dim,
                     uint32_t head_offset);
/* cpu.rs:84-109 (position = row index) */
void ora_rope(float* x, uint32_t seq_len, uint32_t dim, uint32_t head_dim);
/* cpu.rs:111-142 (position = pos_offset + row index) */
void ora_rope_offset(float* x, uint32_t seq_len, uint32_t dim,
                     uint32_t head_dim, uint32_t pos_offset);
/* cpu.rs:224-236 */
void ora_cache_write(const float* src, float* dst, uint32_t row_count,
                     uint32_t width, uint32_t dst_row_offset);
/* cpu.rs:144-162: scores[h*attn_len + j] = q_h . K[j, h] (unscaled) */
void ora_attn_qk_cached(const float* q, const float* k_cache, float* scores,
                        uint32_t attn_len, uint32_t dim, uint32_t head_dim);
/* cpu.rs:180-203 */
void ora_softmax_rect(float* x, uint32_t num_rows, uint32_t width,
                      float scale);
/* cpu.rs:164-178 */
void ora_attn_av_cached(const float* scores, const float* v_cache, float* out,
                        uint32_t attn_len, uint32_t dim, uint32_t head_dim);
/* cpu.rs:63-69 */
void ora_silu(float* x, size_t n);
/* src/nn/ops/emit.rs:931-999 (cpu_attention, forward half): causal
 * softmax(scale * Q K^T) V per head, scale = 1/sqrt(head_dim); rows are
 * [seq_len, dim] with head h at columns h*head_dim. */
void ora_causal_attention(const float* q, const float* k, const float* v,
                          float* out, uint32_t seq_len, uint32_t dim,
                          uint32_t head_dim);
/* ---- the trainer's forward shaders (src/nn/train.rs:256-275) ----------- */

/* QKV_SPLIT (src/shaders/mod.rs:376-395).  The reference has no CPU twin;
 * this follows its CUDA twin (src/shaders/cuda.rs:296-318): for row <
 * seq_len and col < head_dim, q/k/v[row * head_dim + col] = src[row *
 * full_dim + role * head_dim + col], role 0/1/2. */
void ora_qkv_split(const float* src, float* q, float* k, float* v, uint32_t seq_len,
                   uint32_t full_dim, uint32_t head_dim);
/* ROPE_QK (src/shaders/mod.rs:139-158; no CPU twin, CUDA twin
 * cuda.rs:152-185): RoPE on rows row_offset .. row_offset + seq_len of both
 * q and k ([*, dim]), at local positions 0 .. seq_len - 1, with cpu.rs's
 * angle (cpu.rs:98-100). */
void ora_rope_qk(float* q, float* k, uint32_t seq_len, uint32_t dim, uint32_t head_dim,
                 uint32_t row_offset);
/* ADD (src/shaders/cpu.rs:77-82): out = a + b. */
void ora_add(const float* a, const float* b, float* out, size_t n);
/* RESIDUAL_ADD builtin, ops::residual_add (src/nn/ops/emit.rs:733-748):
 * target += source.  The builtin lives in the absent wilupgu; the emitter's
 * doc comment and binding modes (Accumulate, Input) fix the semantics. */
void ora_residual_add(float* target, const float* source, size_t n);
/* SILU_OUT (src/shaders/cpu.rs:71-75): out = x / (1 + e^-x). */
void ora_silu_out(const float* x, float* out, size_t n);
/* CROSS_ENTROPY (src/shaders/cpu.rs:277-306), in place: per row of
 * [rows, vocab] logits, m = max (fold from -inf), s = sum of e^(x - m) (a
 * sequential fold), losses[row] = -(x[target] - m - ln s), and x becomes
 * the softmax probabilities e^(x - m) / s. */
void ora_cross_entropy(float* x, const uint32_t* targets, float* losses, uint32_t vocab_size,
                       uint32_t num_rows);
/* src/nn/sampling.rs:83-91: first index of the maximum (strict >). */
uint32_t ora_argmax(const float* logits, uint32_t n);
/* sampling.rs:3-81: repetition penalty, temperature, top-k, top-p, and the
 * walk of the distribution with the draw r in [0, 1).  Ties in the sort are
 * broken by the lower index (the reference's unstable sort leaves them
 * unspecified). */
uint32_t ora_sample_token(const float* logits, uint32_t n, float temperature,
                          uint32_t top_k, float top_p, const uint32_t* seen,
                          uint32_t n_seen, float repetition_penalty, double r);

/* ---- model + session (src/nn/inference.rs, inference_graphs.rs) -------- */

/* src/config.rs:1-30 (ModelConfig; ffn_hidden = 4*dim, eps = 1e-5). */
typedef struct {
  uint32_t vocab_size;
  uint32_t dim;
  uint32_t num_heads;
  uint32_t num_layers;
  uint32_t ffn_hidden;
  float norm_eps;
  uint32_t eos_token;
} ora_config;

/* src/nn/weights.rs:32-47; one pointer per tensor, laid out exactly as the
 * reference's ModelWeights ([in, out] row-major matrices, qkv rows
 * interleaved [Q_row | K_row | V_row] per weights.rs:49-58).  Per-layer
 * arrays have num_layers entries. */
typedef struct {
  const float* embedding;      /* [vocab, dim] */
  const float* const* norm_1;  /* [dim] each */
  const float* const* qkv_proj; /* [dim, 3*dim] */
  const float* const* out_proj; /* [dim, dim] */
  const float* const* norm_2;   /* [dim] */
  const float* const* ffn_up;   /* [dim, ffn] */
  const float* const* ffn_down; /* [ffn, dim] */
  const float* final_norm;      /* [dim] */
  const float* lm_head;         /* [dim, vocab] */
} ora_weights;

typedef struct ora_session ora_session;

/* Error codes follow src/lib.rs:10-17 (AkashaError). */
enum {
  ORA_OK = 0,
  ORA_E_EMPTY_PROMPT = 1,
  ORA_E_PROMPT_TOO_LONG = 2,
  ORA_E_CONTEXT_FULL = 3,
  ORA_E_NO_CACHE = 4,
  ORA_E_CACHE_NOT_EMPTY = 5
};

/* InferenceSession::new + replace_cache(Cache::new) (inference.rs:25-54,
 * inference_graphs.rs:511-538).  The weights are borrowed, not copied. */
ora_session* ora_session_new(const ora_config* cfg, const ora_weights* w,
                             uint32_t max_context_len);
void ora_session_free(ora_session* s);
/* Cache::reset (inference_graphs.rs:540-542). */
void ora_session_reset(ora_session* s);
uint32_t ora_session_cur_len(const ora_session* s);
/* InferenceSession::prefill (inference.rs:61-176): logits of the last row. */
int ora_session_prefill(ora_session* s, const uint32_t* tokens, uint32_t n,
                        float* logits);
/* InferenceSession::decode_step (inference.rs:178-262). */
int ora_session_decode_step(ora_session* s, uint32_t token, float* logits);
/* Pointers into the session's cache (per layer [max_ctx, dim]). */
const float* ora_session_k_cache(const ora_session* s, uint32_t layer);
const float* ora_session_v_cache(const ora_session* s, uint32_t layer);

/* Benchmark hook: pretend `len` tokens are cached (their rows keep whatever
 * the cache holds, zeros for a fresh session), so a decode step at
 * position `len` can be timed without a long CPU prefill first. */
void ora_session_set_len(ora_session* s, uint32_t len);

/* Trainer::forward then CrossEntropy (src/nn/train.rs:256-275, 394-401;
 * TransformerBlock, layers.rs:551-760; CrossEntropy, layers.rs:465-522) over
 * batch sequences of seq_len tokens with row_offset batching.  Writes
 * losses[batch * seq_len]; probs (optional) receives the CE's in-place
 * probabilities [rows, vocab]; hidden (optional) the last block's add_2
 * output [rows, dim].  Returns CrossEntropy::loss(), the mean loss. */
float ora_forward_train(const ora_config* cfg, const ora_weights* w, const uint32_t* tokens,
                        const uint32_t* targets, uint32_t batch, uint32_t seq_len,
                        float* losses, float* probs, float* hidden);


/* Host-thread count used by ora_matmul / ora_matmul_add (OpenMP over
 * output columns; every output element keeps its own k-ascending fold, so
 * results are identical for any count).  Default 1. */
void ora_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
