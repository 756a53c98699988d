/*
 * akasha_hip.h -- C ABI of libakasha_hip.so, the MI355X (gfx950) backend for
 * akasha-core's inference path.
 *
 * This is the surface a Rust `hip` feature of akasha-core / wilupgu binds
 * through a thin FFI crate.  It has
 * three layers, each replacing a reference interface:
 *
 *   1. Backend, tensors and graphs: wilupgu's Backend / Tensor / ComputeGraph
 *      (reference call sites: src/nn/inference.rs:83,170,189,257,261;
 *      src/nn/ops/meta.rs:4-16; src/main.rs:366).
 *   2. One launcher per reference Shader or matmul builtin on the inference
 *      path, with buffers in binding-slot order and the meta structs of
 *      src/nn/ops/meta.rs byte for byte.  Each launcher mirrors an `*_with`
 *      emitter of src/nn/ops/emit.rs: `shape` is the build-time meta (it
 *      sizes the launch, as the emitter's grid does) and `meta` is the device
 *      meta tensor the kernel reads when it executes, so a captured graph
 *      follows metas rewritten between executions.
 *   3. A batched InferenceSession (src/nn/inference.rs:13-326): B independent
 *      sequences, each with its own KV cache, sharing one read of the
 *      weights per step.
 *
 * Conventions: all pointers named dev/device are device pointers from
 * akh_tensor_alloc; everything else is host memory.  Calls on one backend
 * are not re-entrant (the reference's devices are single-threaded too:
 * README.md:55-57).  No exception crosses this ABI: every entry returns an
 * akh_status, and akh_last_error() describes the last failure.
 */
#ifndef AKASHA_HIP_H
#define AKASHA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AKH_ABI_VERSION 1

/* Status codes.  1..5 are AkashaError's variants (src/lib.rs:10-17). */
typedef enum {
  AKH_OK = 0,
  AKH_E_EMPTY_PROMPT = 1,      /* AkashaError::EmptyPrompt */
  AKH_E_PROMPT_TOO_LONG = 2,   /* AkashaError::PromptTooLong { len, max } */
  AKH_E_CONTEXT_FULL = 3,      /* AkashaError::ContextFull { max } */
  AKH_E_NO_CACHE = 4,          /* AkashaError::NoCache */
  AKH_E_CACHE_NOT_EMPTY = 5,   /* AkashaError::CacheNotEmpty { cur_len } */
  AKH_E_INVALID = 6,           /* a precondition the reference assert!s */
  AKH_E_HIP = 7,               /* HIP runtime error */
  AKH_E_IO = 8                 /* a file cannot be opened or read */
} akh_status;

/* ---- metas: src/nn/ops/meta.rs, #[repr(C)] u32/f32 --------------------- */
typedef struct { uint32_t m, n, k; } akh_matmul_meta;                 /* :19-25 */
typedef struct { uint32_t seq_len, size; float eps; } akh_norm_meta;  /* :29-35 */
typedef struct {
  uint32_t seq_len, full_dim, head_dim, head_offset;
} akh_head_move_meta;                                                  /* :40-47 */
typedef struct { uint32_t attn_len, dim, head_dim; } akh_attn_cached_meta; /* :62-68 */
typedef struct { uint32_t num_rows, width; float scale; } akh_softmax_rect_meta; /* :72-78 */
typedef struct { uint32_t seq_len, dim, head_dim, row_offset; } akh_rope_meta; /* :82-89 */
typedef struct { uint32_t seq_len, dim, head_dim, pos; } akh_rope_offset_meta; /* :93-100 */
typedef struct { uint32_t row_count, width, dst_row_offset; } akh_cache_write_meta; /* :104-110 */
typedef struct { uint32_t vocab_size, dim, seq_len; } akh_embedding_meta; /* :114-120 */
typedef struct {
  uint32_t seq_len, dim, head_dim;
  float scale;
  uint32_t row_offset;
} akh_flash_attn_meta;                                                 /* :156-164 */
typedef struct { uint32_t vocab_size, num_rows; } akh_cross_entropy_meta; /* :124-130 */

/* ---- 1. backend, tensors, graphs ----------------------------------------- */

typedef struct akh_backend akh_backend;
typedef struct akh_graph akh_graph;

/* HipBackend::new(device), the counterpart of CudaBackend::new(0)
 * (src/main.rs:366).  Creates one stream at default priority. */
akh_status akh_backend_new(int device, akh_backend** out);
void akh_backend_free(akh_backend* be);
/* Backend::synchronize (src/nn/ops/emit.rs:1052). */
akh_status akh_synchronize(akh_backend* be);
/* Text of the last failure on this thread ("" if none). */
const char* akh_last_error(void);
int akh_abi_version(void);

/* Tensor::init_from_cpu / copy_from_cpu / to_cpu (inference.rs:83,189,261).
 * akh_tensor_alloc returns zeroed device memory.  Alloc, free and upload are
 * ordered on the backend's stream and do not wait for it: the zeroing and
 * the copy are queued behind the work already issued, a freed block (kept by
 * the backend, up to 8 GB) is reused only by a later alloc, and an upload of
 * up to 64 KB copies the host bytes out before it returns (larger ones wait
 * for their copy).  Download waits for the stream.  So a tensor is used on
 * the backend that made it, or after akh_synchronize.  Freeing a tensor
 * twice returns AKH_E_INVALID. */
akh_status akh_tensor_alloc(akh_backend* be, size_t bytes, void** dev);
akh_status akh_tensor_free(akh_backend* be, void* dev);
akh_status akh_tensor_upload(akh_backend* be, void* dev, const void* host,
                             size_t bytes);
/* Tensor::init_from_cpu (inference.rs:83) in one call: a device tensor of
 * `bytes` holding a copy of host[0 .. bytes), ordered on the stream as
 * akh_tensor_alloc followed by akh_tensor_upload, without the zeroing that
 * the upload would overwrite. */
akh_status akh_tensor_from_host(akh_backend* be, const void* host, size_t bytes, void** dev);
akh_status akh_tensor_download(akh_backend* be, void* host, const void* dev,
                               size_t bytes);

/* ComputeGraph::new / add_node / execute (src/nn/ops/emit.rs:36-45,
 * inference.rs:170,257).  Launchers called between begin and end are
 * recorded into a hipGraph instead of running; akh_graph_execute replays it
 * on the backend's stream.  Metas are read from device memory at replay. */
akh_status akh_graph_begin(akh_backend* be);
akh_status akh_graph_end(akh_backend* be, akh_graph** out);
akh_status akh_graph_execute(akh_graph* g);
void akh_graph_free(akh_graph* g);

/* ---- 2. launchers (one per Shader / builtin; src/shaders/mod.rs) --------- */

/* EMBEDDING, ops::embedding_with (emit.rs:228-244; cpu.rs:25-41). */
akh_status akh_embedding(akh_backend* be, const uint32_t* tokens,
                         const float* table, float* out,
                         akh_embedding_meta shape,
                         const akh_embedding_meta* meta);
/* RMSNORM, ops::rmsnorm_with (emit.rs:151-168; cpu.rs:205-222). */
akh_status akh_rmsnorm(akh_backend* be, const float* input,
                       const float* weight, float* output,
                       akh_norm_meta shape, const akh_norm_meta* meta);
/* MATMUL / GEMV builtins, ops::matmul_with (emit.rs:19-45):
 * C[m,n] = A[m,k] B[k,n], row-major, B stored [in, out].  Output binding:
 * every element of C[0..m, 0..n] is written. */
akh_status akh_matmul(akh_backend* be, const float* a, const float* b,
                      float* c, akh_matmul_meta shape,
                      const akh_matmul_meta* meta);
/* MATMUL_ADD / GEMV_ADD builtins, ops::matmul_add_with (emit.rs:91-114):
 * C += A B (Accumulate binding). */
akh_status akh_matmul_add(akh_backend* be, const float* a, const float* b,
                          float* c, akh_matmul_meta shape,
                          const akh_matmul_meta* meta);
/* HEAD_GATHER, ops::head_gather_with (emit.rs:405-413; cpu.rs:238-255). */
akh_status akh_head_gather(akh_backend* be, const float* src, float* dst,
                           akh_head_move_meta shape,
                           const akh_head_move_meta* meta);
/* ROPE, ops::rope (emit.rs:306-313; cpu.rs:84-109): in place, position =
 * row index. */
akh_status akh_rope(akh_backend* be, float* buf, akh_rope_meta shape,
                    const akh_rope_meta* meta);
/* ROPE_OFFSET, ops::rope_offset_with (emit.rs:325-342; cpu.rs:111-142). */
akh_status akh_rope_offset(akh_backend* be, float* buf,
                           akh_rope_offset_meta shape,
                           const akh_rope_offset_meta* meta);
/* CACHE_WRITE, ops::cache_write_with (emit.rs:649-666; cpu.rs:224-236). */
akh_status akh_cache_write(akh_backend* be, const float* src, float* cache,
                           akh_cache_write_meta shape,
                           const akh_cache_write_meta* meta);
/* FLASH_ATTENTION, ops::flash_attention (emit.rs:556-597): causal
 * softmax(scale Q K^T) V for one sequence of rows [row_offset,
 * row_offset+seq_len) of [*, dim] buffers; l_cache[row*H + h] receives
 * max + ln(sum).  head_dim <= 128 (emit.rs:564-567).  Every head size
 * keeps fp32-level error.  head_dim 64 (and 128 on grids of fewer 128-row
 * blocks than CUs) runs split-fp16 MFMA tiles: two fp16 terms per operand,
 * three products, and a tile whose operands leave fp16's range recomputes
 * itself on split-bfloat16.  head_dim 128 on larger grids and 33..127
 * otherwise run split-bfloat16 MFMAs throughout: three bfloat16 terms per
 * operand, six products.  head_dim <= 32 runs a scalar fp32 kernel. */
akh_status akh_flash_attention(akh_backend* be, const float* q,
                               const float* k, const float* v, float* out,
                               float* l_cache, akh_flash_attn_meta shape,
                               const akh_flash_attn_meta* meta);
/* SelfAttention's forward (layers.rs:408-421): its batch_size
 * FLASH_ATTENTION nodes, node b at row_offset meta->row_offset + b *
 * seq_len, as one launch.  l_cache holds the nodes' [seq_len, H] blocks one
 * after another (batch * seq_len * H floats). */
akh_status akh_flash_attention_batched(akh_backend* be, const float* q, const float* k,
                                       const float* v, float* out, float* l_cache,
                                       akh_flash_attn_meta shape,
                                       const akh_flash_attn_meta* meta, uint32_t batch);
/* ATTN_QK_CACHED, ops::attn_qk_cached_with (emit.rs:485-504). */
akh_status akh_attn_qk_cached(akh_backend* be, const float* q,
                              const float* k_cache, float* scores,
                              uint32_t num_heads, uint32_t max_attn_len,
                              const akh_attn_cached_meta* meta);
/* SOFTMAX_RECT, ops::softmax_rect_with (emit.rs:528-542). */
akh_status akh_softmax_rect(akh_backend* be, float* scores,
                            akh_softmax_rect_meta shape,
                            const akh_softmax_rect_meta* meta);
/* ATTN_AV_CACHED, ops::attn_av_cached_with (emit.rs:507-525). */
akh_status akh_attn_av_cached(akh_backend* be, const float* scores,
                              const float* v_cache, float* out, uint32_t dim,
                              const akh_attn_cached_meta* meta);
/* SILU, ops::silu (emit.rs:686-696): in place x / (1 + e^-x). */
akh_status akh_silu(akh_backend* be, float* buf, uint32_t len);
/* Greedy token choice, sample_token with temperature <= 0 and no
 * repetition penalty (src/nn/sampling.rs:30-32, 83-91): out[r] = first
 * index of the maximum of logits[r, 0..n]. */
akh_status akh_argmax_rows(akh_backend* be, const float* logits,
                           uint32_t rows, uint32_t n, uint32_t* out);

/* The trainer's forward shaders (Trainer::forward, src/nn/train.rs:256-275). */
/* QKV_SPLIT, ops::qkv_split (emit.rs:438-458; CUDA twin cuda.rs:296-318):
 * q/k/v[row, col] = src[row, role * head_dim + col] for row < seq_len,
 * col < head_dim, src rows full_dim wide.  Slots: src, q, k, v, meta. */
akh_status akh_qkv_split(akh_backend* be, const float* src, float* q, float* k, float* v,
                         akh_head_move_meta shape, const akh_head_move_meta* meta);
/* ROPE_QK, ops::rope_qk (emit.rs:344-360; CUDA twin cuda.rs:152-185): RoPE
 * in place on rows row_offset .. row_offset + seq_len of q and k, at local
 * positions 0 .. seq_len - 1.  Slots: q, k, meta. */
akh_status akh_rope_qk(akh_backend* be, float* q, float* k, akh_rope_meta shape,
                       const akh_rope_meta* meta);
/* ADD, ops::add_out (emit.rs:750-767; cpu.rs:77-82): out = a + b. */
akh_status akh_add(akh_backend* be, const float* a, const float* b, float* out, uint32_t len);
/* RESIDUAL_ADD builtin, ops::residual_add (emit.rs:733-748): target += source. */
akh_status akh_residual_add(akh_backend* be, float* target, const float* source,
                            uint32_t len);
/* SILU_OUT, ops::silu_out (emit.rs:698-713; cpu.rs:71-75): out = x / (1 + e^-x). */
akh_status akh_silu_out(akh_backend* be, const float* input, float* out, uint32_t len);
/* CROSS_ENTROPY, ops::cross_entropy (emit.rs:864-882; cpu.rs:277-306), in
 * place: each row of logits [num_rows, vocab] becomes its softmax and
 * losses[row] = -(x[target] - max - ln sum).  A target id >= vocab_size
 * gives a NaN loss (the reference indexes out of bounds).  Slots: logits,
 * targets, losses, meta. */
akh_status akh_cross_entropy(akh_backend* be, float* logits, const uint32_t* targets,
                             float* losses, akh_cross_entropy_meta shape,
                             const akh_cross_entropy_meta* meta);

/* Parameters of sample_token (src/nn/sampling.rs:18-25). */
typedef struct {
  float temperature;
  uint32_t top_k;
  float top_p;
  float repetition_penalty;
} akh_sampling;

/* sample_token (sampling.rs:3-81) for `rows` rows of device logits [rows, n]:
 * the repetition penalty over each row's seen ids, then the argmax
 * (temperature <= 0) or temperature / top_k / top_p sampling, with the
 * device draw uniforms[r] in [0, 1) standing in for rand::random().  seen is
 * [rows, seen_stride] with seen_len[rows] valid entries (NULL: no seen ids);
 * uniforms may be NULL when temperature <= 0.  Ids with equal logits are
 * ordered lower index first (the reference's unstable sort leaves that
 * order unspecified).  n <= 2^20. */
akh_status akh_sample_rows(akh_backend* be, const float* logits, uint32_t rows,
                           uint32_t n, akh_sampling params, const uint32_t* seen,
                           uint32_t seen_stride, const uint32_t* seen_len,
                           const double* uniforms, uint32_t* out);
/* akh_sample_rows without any allocation: no counterpart in the reference.
 * It is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, checks and results as akh_sample_rows; its workspace is a fixed
 * per-GPU device array of 2^21 doubles (16 MiB, held until the process
 * ends), so rows * n must be at most 2^21 (AKH_E_INVALID beyond).  All calls
 * on one GPU share that array: calls that overlap on one GPU (other streams
 * or backends) race. */
akh_status akh_sample_rows_noalloc(akh_backend* be, const float* logits, uint32_t rows,
                                   uint32_t n, akh_sampling params, const uint32_t* seen,
                                   uint32_t seen_stride, const uint32_t* seen_len,
                                   const double* uniforms, uint32_t* out);

/* ---- 3. model weights and the batched session ---------------------------- */

/* ModelConfig (src/config.rs:1-30). */
typedef struct {
  uint32_t vocab_size, dim, num_heads, num_layers, ffn_hidden;
  float norm_eps;
  uint32_t eos_token;
} akh_model_config;

typedef struct akh_model akh_model;
typedef struct akh_session akh_session;

/* ModelWeights::zeros (src/nn/weights.rs:125-156) on the device. */
akh_status akh_model_new(akh_backend* be, const akh_model_config* cfg,
                         akh_model** out);
void akh_model_free(akh_model* m);
/* Number of tensors in ModelWeights::params() order (weights.rs:158-171):
 * embedding, then per layer norm_1, qkv_proj, out_proj, norm_2, ffn_up,
 * ffn_down, then final_norm, lm_head. */
uint32_t akh_model_num_params(const akh_model* m);
/* Device pointer and element count of parameter `index`, in the reference
 * layout.  A read-only view: the decode kernels read the matrices through
 * a tiled copy that akh_model_upload_param refreshes, so parameters change
 * only through akh_model_upload_param. */
akh_status akh_model_param(akh_model* m, uint32_t index, float** dev,
                           size_t* count);
/* Copy `count` floats from host into parameter `index` (count must match),
 * and refresh the decode path's tiled copy of a weight matrix.  A matrix
 * whose every value is a bfloat16 (low 16 mantissa bits zero, e.g. weights
 * trained or stored in bf16) is tiled in bfloat16: half the bytes per
 * decode step, and bf16 MFMAs on the activations split exactly into three
 * bfloat16 terms, so every product is exact (fp32-accurate results, summed
 * in another order than f32 tiles). */
akh_status akh_model_upload_param(akh_model* m, uint32_t index,
                                  const float* host, size_t count);
/* No reference counterpart (the reference keeps f32 device weights): allow
 * (1, the default) or forbid (0) bfloat16 tiles, re-tiling every decode
 * matrix now; `n_bf16` (optional) receives how many matrices are tiled in
 * bfloat16 afterwards. */
akh_status akh_model_set_bf16_tiles(akh_model* m, int allow, uint32_t* n_bf16);
/* No reference counterpart (the reference computes prefill in f32): with
 * enable = 1, prefill runs its layer GEMMs and flash attention on the
 * bfloat16 MFMAs with fp32 accumulation.  Weights are rounded to bfloat16
 * (exact for bf16-valued weights); the QKV, ffn_up and ffn_down GEMMs take
 * their fp32 inputs as bfloat16 hi + lo pairs, out_proj and attention take
 * bfloat16 operands.  The residual stream, KV cache, final norm, lm_head and
 * decode stay f32.  This is the optional bf16-MFMA path: logits track the
 * f32 path within 2e-2 instead of 1e-3.  While enabled the model keeps a
 * transposed bfloat16 copy of every layer matrix (refreshed by
 * akh_model_upload_param).  Needs head_dim 64 or 128 and dim, ffn_hidden
 * multiples of 8. */
akh_status akh_model_set_prefill_bf16(akh_model* m, int enable);
/* No reference counterpart (a choice of kernel, not of numerics): the
 * kernels of the f32 prefill's layer GEMMs and of the trainer forward's
 * lm_head, all fp32-accurate (the f32 path's 1e-3 bar):
 *   AKH_SPLIT_H3 (the default when dim and ffn_hidden are multiples of 8):
 *     fp16 MFMAs with each fp32 operand split into two fp16 terms, x = hi +
 *     2^-11 lo (the scaled-residual split of Ootomo and Yokota), and the
 *     three products down to 2^-22 of the full product accumulated in fp32
 *     (hi.hi apart from the two cross terms).  An operand beyond fp16's range
 *     (|x| >= 65520) is detected from the non-finite results it causes, and
 *     that prefill or forward is recomputed on the fp32-MFMA kernels.
 *   AKH_SPLIT_X6: bfloat16 MFMAs with each operand split exactly into three
 *     bfloat16 terms and six products (each product within 2^-23).
 *   AKH_SPLIT_NONE: the fp32 MFMAs (v_mfma_f32_32x32x2_f32).
 * Either split keeps a copy of every layer matrix and of lm_head (4 bytes an
 * element: fp16 planes, or transposed fp32), refreshed by
 * akh_model_upload_param.  Flash attention (head_dim 64 / 128) follows the
 * split: AKH_SPLIT_H3 runs it on split-fp16 MFMAs (two terms, three
 * products), flagged and rerun in fp32 like the GEMMs when an operand is
 * out of fp16's range; AKH_SPLIT_X6 runs it on split-bfloat16 MFMAs.  The
 * per-shader FLASH_ATTENTION launchers, whatever the split, run split-fp16
 * tiles that recompute themselves on split-bfloat16 MFMAs when an operand is
 * out of fp16's range (split-bfloat16 throughout at head_dim 128 on grids
 * that fill the part).  The bf16-MFMA prefill (akh_model_set_prefill_bf16),
 * when on, takes precedence. */
#define AKH_SPLIT_NONE 0
#define AKH_SPLIT_X6 1
#define AKH_SPLIT_H3 2
akh_status akh_model_set_prefill_split(akh_model* m, int kind);
int akh_model_prefill_split(const akh_model* m);
/* akh_model_set_prefill_split(m, enable ? AKH_SPLIT_X6 : AKH_SPLIT_NONE). */
akh_status akh_model_set_prefill_x6(akh_model* m, int enable);

/* ---- the trainer's fused forward: src/nn/train.rs:256-275, 394-401 ------- */

/* Trainer::forward over batch sequences of seq_len tokens with row_offset
 * batching (TransformerBlock, layers.rs:551-760), the lm_head on every row
 * and CrossEntropy (layers.rs:465-522), on the prefill kernels: one
 * `fused_forward_graph.execute_captured()` plus `CrossEntropy::loss()`
 * (train.rs:380-385).  Any batch; head_dim even, at most 128 (a multiple
 * of 4 above 32).  Runs
 * the bf16-MFMA layers when the model has akh_model_set_prefill_bf16 on. */
typedef struct akh_forward akh_forward;
akh_status akh_forward_new(akh_model* m, uint32_t batch, uint32_t seq_len, akh_forward** out);
void akh_forward_free(akh_forward* f);
/* tokens, targets: host [batch * seq_len] (the trainer's input_tokens and
 * cross_entropy.target_tokens).  losses (optional): host [batch * seq_len].
 * mean_loss: CrossEntropy::loss(), the f32 mean of the row losses.  A
 * target id >= vocab_size is AKH_E_INVALID (the reference panics). */
akh_status akh_forward_loss(akh_forward* f, const uint32_t* tokens, const uint32_t* targets,
                            float* losses, float* mean_loss);
/* After akh_forward_loss: softmax probabilities of rows [row0, row0 + n)
 * (what CROSS_ENTROPY leaves in the logits buffer), host [n, vocab]. */
akh_status akh_forward_probs(akh_forward* f, uint32_t row0, uint32_t n, float* host);
/* After akh_forward_loss: the last block's add_2 output, host [rows, dim]. */
akh_status akh_forward_hidden(akh_forward* f, float* host);

/* ---- checkpoints: src/nn/checkpoint.rs (format V3) ---------------------- */

/* V3Body's header and the shape of its tensor lists (checkpoint.rs:20-35). */
typedef struct {
  uint32_t vocab_size, dim, num_heads;
  uint64_t num_layers;
  uint32_t seq_len, ffn_hidden;
  uint64_t train_step;
  uint32_t schedule_step;
  uint64_t num_params, total_param_floats, num_moment_pairs;
} akh_checkpoint_info_t;

/* Read and check the structure of a V3 file ("AKV3" + bincode fixint body)
 * without a device.  AKH_E_INVALID: not a V3 file; AKH_E_IO: unreadable or
 * truncated. */
akh_status akh_checkpoint_info(const char* path, akh_checkpoint_info_t* info);
/* checkpoint::load (checkpoint.rs:98-187): the file's parameters into the
 * model, in params() order, with the reference's checks and messages: the
 * whole body must parse (else AKH_E_IO); architecture (vocab_size, dim,
 * num_heads, num_layers, ffn_hidden), tensor count and each tensor's size
 * must match the model (else AKH_E_INVALID; tensors before a mismatching one
 * are already loaded, as copy_params leaves them); a non-empty moment list
 * must have one pair per parameter (checked after the weights are loaded).
 * train_step and has_optimizer (moments present) may be NULL. */
akh_status akh_model_load_checkpoint(akh_model* m, const char* path,
                                     uint64_t* train_step, int* has_optimizer);

/* InferenceSession::new + replace_cache(Cache::new(...)) for `batch`
 * independent sequences (inference.rs:25-54; inference_graphs.rs:520-538).
 * batch <= 64: up to two 32-row MFMA tiles share every weight read. */
akh_status akh_session_new(akh_model* m, uint32_t max_context_len,
                           uint32_t batch, akh_session** out);
void akh_session_free(akh_session* s);
/* Cache::reset for every sequence (inference_graphs.rs:540-542). */
akh_status akh_session_reset(akh_session* s);
/* cur_len of every sequence (host copy). */
akh_status akh_session_cur_len(const akh_session* s, uint32_t* out);
/* InferenceSession::prefill (inference.rs:61-176) on all sequences at once:
 * tokens is [batch, prompt_len].  logits ([batch, vocab], last row of each
 * sequence) and next ([batch], greedy argmax) may be NULL. */
akh_status akh_session_prefill(akh_session* s, const uint32_t* tokens,
                               uint32_t prompt_len, float* logits,
                               uint32_t* next);
/* InferenceSession::prefill (inference.rs:61-176, one &[u32] per session)
 * with a prompt length per sequence: tokens holds the prompts back to back
 * (sequence b's prompt_lens[b] tokens after those of sequences 0..b-1).
 * Each prompt is checked as the reference checks it (EmptyPrompt,
 * PromptTooLong, NoCache, CacheNotEmpty); cur_len[b] = prompt_lens[b]. */
akh_status akh_session_prefill_ragged(akh_session* s, const uint32_t* tokens,
                                      const uint32_t* prompt_lens, float* logits,
                                      uint32_t* next);
/* InferenceSession::decode_step (inference.rs:178-262) for every sequence:
 * tokens is [batch] (NULL = feed each sequence its previous greedy token,
 * kept on the device).  logits / next may be NULL. */
akh_status akh_session_decode_step(akh_session* s, const uint32_t* tokens,
                                   float* logits, uint32_t* next);
/* `steps` greedy decode steps back to back, each feeding the previous
 * step's argmax, with no host synchronisation in between (the hot loop of
 * InferenceSession::generate at temperature 0, inference.rs:303-323).
 * out_tokens ([steps, batch]) may be NULL. */
akh_status akh_session_decode_greedy(akh_session* s, uint32_t steps,
                                     uint32_t* out_tokens);
/* InferenceSession::generate (inference.rs:264-326) for every sequence,
 * returning token ids (the reference decodes them to text).  The prompt
 * (tokens: [batch, prompt_len]) is prefilled if every cache is empty, or fed
 * one decode step per token if every sequence holds a cache (a mix is
 * AKH_E_INVALID); its errors are returned as the reference returns them.
 * Then up to max_new_tokens rounds run on the device with no host round
 * trip: sample_token over the sequence's history (this call's prompt and
 * generated tokens) with params and the draw uniforms[round * batch + seq]
 * (host array [max_new_tokens, batch]; may be NULL when temperature <= 0),
 * then a decode step of the sampled token.  A sequence stops after sampling
 * eos (returned, not decoded) or a token its full context cannot take
 * (returned, not decoded: ContextFull ends generate quietly).  out_tokens is
 * [batch, max_new_tokens] with out_counts[batch] valid tokens per row;
 * cur_len follows each sequence's decoded tokens. */
akh_status akh_session_generate(akh_session* s, const uint32_t* tokens,
                                uint32_t prompt_len, uint32_t max_new_tokens,
                                akh_sampling params, const double* uniforms,
                                uint32_t* out_tokens, uint32_t* out_counts);
/* akh_session_generate with a prompt length per sequence (the prompts back
 * to back, as akh_session_prefill_ragged takes them): prefilled on empty
 * caches; on resumed caches fed as decode steps right-aligned, so every
 * sequence decodes its last prompt token in the same final step. */
akh_status akh_session_generate_ragged(akh_session* s, const uint32_t* tokens,
                                       const uint32_t* prompt_lens, uint32_t max_new_tokens,
                                       akh_sampling params, const double* uniforms,
                                       uint32_t* out_tokens, uint32_t* out_counts);
/* Set every sequence's cached length to `len` (<= max_ctx) without touching
 * the cache rows, as assigning the reference's public Cache::cur_len does
 * (inference_graphs.rs:515); rows below `len` keep whatever they hold.  Used
 * to time decode at a given context length. */
akh_status akh_session_set_len(akh_session* s, uint32_t len);
/* No reference counterpart (measurement only): fill rows [0, len) of every
 * sequence's K and V caches, all layers, with N(0, 1) values from a hash of
 * `seed` and the element's offset (bfloat16-rounded in a bf16 cache), then
 * set every cur_len to `len` as akh_session_set_len does.  Decode over a
 * long context can then be timed without prefilling it. */
akh_status akh_session_fill_cache_synthetic(akh_session* s, uint32_t len, uint64_t seed);
/* No reference counterpart (the reference's Cache is f32): with enable = 1
 * the session's KV cache holds bfloat16 rows (rounded to nearest even),
 * half the bytes decode attention streams; decode still computes in f32.
 * Part of the optional bf16 path: logits track the f32 path within 2e-2.
 * Needs every cache empty (AKH_E_CACHE_NOT_EMPTY otherwise); take_cache,
 * replace_cache and download_cache convert to and from f32. */
akh_status akh_session_set_kv_bf16(akh_session* s, int enable);
/* Shorten every sequence to `len` cached tokens (len <= min cur_len); the
 * rows below `len` are kept.  Used to replay a timed decode window. */
akh_status akh_session_truncate(akh_session* s, uint32_t len);
/* InferenceSession::take_cache (inference.rs:56-59) for sequence `seq`: its
 * K and V ([layers, max_ctx, dim] host arrays, either may be NULL) and
 * cur_len are copied out and the sequence is left without a cache, so that
 * prefill and decode steps fail with AKH_E_NO_CACHE until a cache is
 * installed (generate makes a fresh one, inference.rs:278-287).  had_cache
 * reports whether there was one (the reference's Option). */
akh_status akh_session_take_cache(akh_session* s, uint32_t seq, float* k, float* v,
                                  uint32_t* cur_len, int* had_cache);
/* replace_cache (inference.rs:42-54): install K, V ([layers, max_ctx, dim],
 * the session's own shape) with cur_len cached tokens for sequence `seq`.
 * The installed cache carries no token history. */
akh_status akh_session_replace_cache(akh_session* s, uint32_t seq, const float* k,
                                     const float* v, uint32_t cur_len);
/* Copy sequence `seq`'s K or V cache of layer `layer` ([max_ctx, dim]) to
 * host (which: 0 = K, 1 = V). */
akh_status akh_session_download_cache(akh_session* s, uint32_t layer,
                                      uint32_t seq, int which, float* host);

/* ---- timing (HIP events on the backend's stream) ------------------------- */

/* Start / stop an event pair around whatever is enqueued in between; stop
 * waits for completion and returns the elapsed milliseconds. */
akh_status akh_timer_start(akh_backend* be);
akh_status akh_timer_stop(akh_backend* be, float* ms);
/* Replay one kernel of the decode step `reps` times between events and
 * report its mean duration.  kernel: 0 = attention, 1 = qkv projection,
 * 2 = out projection, 3 = ffn up, 4 = ffn down, 5 = lm_head, 6 = residual
 * add + RMSNorm.  Launches cycle over the layers, so each one reads weights
 * and KV rows that the other layers' launches have pushed out of the
 * caches, as in a decode step (lm_head has one weight matrix).  The step's
 * buffers are reused: the residual stream is clobbered until the next decode
 * step rewrites it from the embedding, and attention writes the cache row at
 * each sequence's next position, which the next decode step rewrites before
 * reading it. */
akh_status akh_session_time_decode_kernel(akh_session* s, int kernel,
                                          uint32_t reps, float* avg_ms);
/* The decode attention kernel alone: `reps` (at most 4096) dispatches
 * cycling over the layers, as akh_session_time_decode_kernel(s, 0, ...),
 * each carrying its own start and end events (hipExtLaunchKernelGGL), so
 * the mean excludes the gaps between dispatches.  No counterpart in the
 * reference (measurement only). */
akh_status akh_session_time_decode_attn(akh_session* s, uint32_t reps, float* avg_ms);
/* Kernel launches in one decode step: the kernel nodes of the captured
 * one-step decode graph (captured here if it is not yet).  No counterpart
 * in the reference (measurement only; the reference dispatches ~195 nodes
 * per sequence per token, inference_graphs.rs:339-509). */
akh_status akh_session_decode_launches(akh_session* s, uint32_t* launches);
/* Fold each layer's two residual adds + RMSNorms into the decode GEMMs
 * (enable != 0): out_proj and ffn_down add their sums to the residual
 * themselves (the last block of each column tile to finish sums the K
 * splits' partial tiles, handed over at device scope) and write per-tile
 * sums of squares; qkv_proj, ffn_up and the final norm scale their A
 * operand by each row's RMSNorm.  Five launches per layer instead of seven,
 * the same results to rounding.  Off by default, because on MI355X the
 * handoff costs more than the two kernel boundaries it saves (config 4:
 * 0.677 against 0.632 ms per step).  Needs a decode session whose dim is a
 * multiple of 128 (at most 4096); drops the captured graphs.  No
 * counterpart in the reference (a launch-structure choice). */
akh_status akh_session_set_fused_norm(akh_session* s, int enable);

#ifdef __cplusplus
}
#endif
#endif
