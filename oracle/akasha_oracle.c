/*
 * akasha_oracle.c -- CPU restatement of the akasha-core inference path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the "port" CPU baseline.
 * The product library never links or calls this file.  Each function cites
 * the reference function it restates (paths relative to the akasha-core
 * source root).  Summations are sequential f32 left folds in the reference's
 * order; compile with -ffp-contract=off so no multiply-add is fused.
 */
#include "akasha_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void ora_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

/* ---- generators ---------------------------------------------------------- */

/* emit.rs:910-921: state = seed + 0x9E3779B97F4A7C15, then per draw
 * state = state*6364136223846793005 + 1442695040888963407 (wrapping),
 * bits = (state >> 40) & 0xFFFFFF, value = bits / 0xFFFFFF * 2 - 1 in f32. */
void ora_rand_vec(float* out, size_t n, uint64_t seed) {
  uint64_t state = seed + 0x9E3779B97F4A7C15ULL;
  for (size_t i = 0; i < n; ++i) {
    state = state * 6364136223846793005ULL + 1442695040888963407ULL;
    uint32_t bits = (uint32_t)(state >> 40) & 0x00FFFFFFu;
    out[i] = ((float)bits / (float)0x00FFFFFF) * 2.0f - 1.0f;
  }
}

/* train.rs:818-828: same LCG, token = (u32)(state >> 33) % vocab. */
void ora_rand_tokens(uint32_t* out, size_t n, uint32_t vocab, uint64_t seed) {
  uint64_t state = seed + 0x9E3779B97F4A7C15ULL;
  for (size_t i = 0; i < n; ++i) {
    state = state * 6364136223846793005ULL + 1442695040888963407ULL;
    out[i] = ((uint32_t)(state >> 33)) % vocab;
  }
}

/* ---- kernels ------------------------------------------------------------- */

/* cpu.rs:25-41: out[t,:] = table[tok[t],:]; ids >= vocab leave a zero row. */
void ora_embedding(const uint32_t* tokens, const float* table, float* out,
                   uint32_t vocab_size, uint32_t dim, uint32_t seq_len) {
  memset(out, 0, sizeof(float) * (size_t)seq_len * dim);
  for (uint32_t t = 0; t < seq_len; ++t) {
    uint32_t id = tokens[t];
    if (id < vocab_size)
      memcpy(out + (size_t)t * dim, table + (size_t)id * dim,
             sizeof(float) * dim);
  }
}

/* cpu.rs:205-222: ss = sum x^2 (left fold), r = 1/sqrt(ss/size + eps),
 * out = x * r * w (left to right). */
void ora_rmsnorm(const float* x, const float* w, float* out, uint32_t rows,
                 uint32_t size, float eps) {
  for (uint32_t r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * size;
    float* o = out + (size_t)r * size;
    float ss = 0.0f;
    for (uint32_t i = 0; i < size; ++i) ss += xr[i] * xr[i];
    float rs = 1.0f / sqrtf((ss / (float)size) + eps);
    for (uint32_t i = 0; i < size; ++i) o[i] = xr[i] * rs * w[i];
  }
}

/* One output row: acc[n] = sum_k a[k] * b[k, n], k ascending.  The k-outer
 * loop keeps every element's own left fold, so the result equals the
 * textbook per-element dot product bit for bit. */
static void row_times_matrix(const float* a, const float* b, float* acc,
                             uint32_t n0, uint32_t n1, uint32_t n,
                             uint32_t k) {
  for (uint32_t j = n0; j < n1; ++j) acc[j] = 0.0f;
  for (uint32_t kk = 0; kk < k; ++kk) {
    const float av = a[kk];
    const float* br = b + (size_t)kk * n;
    for (uint32_t j = n0; j < n1; ++j) acc[j] += av * br[j];
  }
}

static void matmul_impl(const float* a, const float* b, float* c, uint32_t m,
                        uint32_t n, uint32_t k, int accumulate) {
  float* tmp = (float*)malloc(sizeof(float) * n);
  for (uint32_t i = 0; i < m; ++i) {
    const float* ar = a + (size_t)i * k;
#ifdef _OPENMP
#pragma omp parallel num_threads(g_threads)
    {
      int nt = omp_get_num_threads(), tid = omp_get_thread_num();
      uint32_t chunk = (n + nt - 1) / nt;
      uint32_t n0 = tid * chunk, n1 = n0 + chunk > n ? n : n0 + chunk;
      if (n0 < n1) row_times_matrix(ar, b, tmp, n0, n1, n, k);
    }
#else
    row_times_matrix(ar, b, tmp, 0, n, n, k);
#endif
    float* cr = c + (size_t)i * n;
    if (accumulate)
      for (uint32_t j = 0; j < n; ++j) cr[j] = cr[j] + tmp[j];
    else
      memcpy(cr, tmp, sizeof(float) * n);
  }
  free(tmp);
}

void ora_matmul(const float* a, const float* b, float* c, uint32_t m,
                uint32_t n, uint32_t k) {
  matmul_impl(a, b, c, m, n, k, 0);
}

void ora_matmul_add(const float* a, const float* b, float* c, uint32_t m,
                    uint32_t n, uint32_t k) {
  matmul_impl(a, b, c, m, n, k, 1);
}

/* cpu.rs:238-255 */
void ora_head_gather(const float* src, float* dst, uint32_t seq_len,
                     uint32_t full_dim, uint32_t head_dim,
                     uint32_t head_offset) {
  for (uint32_t r = 0; r < seq_len; ++r)
    memcpy(dst + (size_t)r * head_dim,
           src + (size_t)r * full_dim + head_offset,
           sizeof(float) * head_dim);
}

/* cpu.rs:84-142: pairs (2i, 2i+1) of every head rotated by
 * angle = pos * (1 / 10000^(2i/head_dim)), all in f32. */
static void rope_rows(float* x, uint32_t seq_len, uint32_t dim,
                      uint32_t head_dim, uint32_t pos_offset) {
  uint32_t num_heads = dim / head_dim;
  for (uint32_t t = 0; t < seq_len; ++t) {
    uint32_t pos = t + pos_offset;
    for (uint32_t di = 0; di < head_dim; di += 2) {
      for (uint32_t h = 0; h < num_heads; ++h) {
        size_t off = (size_t)t * dim + (size_t)h * head_dim + di;
        float x0 = x[off], x1 = x[off + 1];
        float freq = 1.0f / powf(10000.0f, (float)di / (float)head_dim);
        float angle = (float)pos * freq;
        float s = sinf(angle), c = cosf(angle);
        x[off] = x0 * c - x1 * s;
        x[off + 1] = x0 * s + x1 * c;
      }
    }
  }
}

void ora_rope(float* x, uint32_t seq_len, uint32_t dim, uint32_t head_dim) {
  rope_rows(x, seq_len, dim, head_dim, 0);
}

void ora_rope_offset(float* x, uint32_t seq_len, uint32_t dim,
                     uint32_t head_dim, uint32_t pos_offset) {
  rope_rows(x, seq_len, dim, head_dim, pos_offset);
}

/* cpu.rs:224-236 */
void ora_cache_write(const float* src, float* dst, uint32_t row_count,
                     uint32_t width, uint32_t dst_row_offset) {
  for (uint32_t r = 0; r < row_count; ++r)
    memcpy(dst + (size_t)(dst_row_offset + r) * width,
           src + (size_t)r * width, sizeof(float) * width);
}

/* cpu.rs:144-162 */
void ora_attn_qk_cached(const float* q, const float* k_cache, float* scores,
                        uint32_t attn_len, uint32_t dim, uint32_t head_dim) {
  uint32_t num_heads = dim / head_dim;
  for (uint32_t h = 0; h < num_heads; ++h) {
    uint32_t q_off = h * head_dim;
    for (uint32_t j = 0; j < attn_len; ++j) {
      const float* kr = k_cache + (size_t)j * dim + q_off;
      float s = 0.0f;
      for (uint32_t c = 0; c < head_dim; ++c) s += q[q_off + c] * kr[c];
      scores[(size_t)h * attn_len + j] = s;
    }
  }
}

/* cpu.rs:180-203: max of scale*x (fold from -inf), e = exp(scale*x - max),
 * divide by the left-fold sum of e. */
void ora_softmax_rect(float* x, uint32_t num_rows, uint32_t width,
                      float scale) {
  for (uint32_t r = 0; r < num_rows; ++r) {
    float* row = x + (size_t)r * width;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < width; ++i) mx = fmaxf(mx, row[i] * scale);
    float sum = 0.0f;
    for (uint32_t i = 0; i < width; ++i) {
      float e = expf(row[i] * scale - mx);
      row[i] = e;
      sum += e;
    }
    for (uint32_t i = 0; i < width; ++i) row[i] /= sum;
  }
}

/* cpu.rs:164-178 */
void ora_attn_av_cached(const float* scores, const float* v_cache, float* out,
                        uint32_t attn_len, uint32_t dim, uint32_t head_dim) {
  for (uint32_t d = 0; d < dim; ++d) {
    const float* p = scores + (size_t)(d / head_dim) * attn_len;
    float s = 0.0f;
    for (uint32_t j = 0; j < attn_len; ++j) s += p[j] * v_cache[(size_t)j * dim + d];
    out[d] = s;
  }
}

/* cpu.rs:63-69 */
void ora_silu(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* QKV_SPLIT: cuda.rs:296-318 (no CPU twin). */
void ora_qkv_split(const float* src, float* q, float* k, float* v, uint32_t seq_len,
                   uint32_t full_dim, uint32_t head_dim) {
  for (uint32_t row = 0; row < seq_len; ++row)
    for (uint32_t col = 0; col < head_dim; ++col) {
      const float* r = src + (size_t)row * full_dim;
      q[(size_t)row * head_dim + col] = r[col];
      k[(size_t)row * head_dim + col] = r[head_dim + col];
      v[(size_t)row * head_dim + col] = r[2 * head_dim + col];
    }
}

/* ROPE_QK: cuda.rs:152-185 (no CPU twin); local positions, rows shifted by
 * row_offset. */
void ora_rope_qk(float* q, float* k, uint32_t seq_len, uint32_t dim, uint32_t head_dim,
                 uint32_t row_offset) {
  rope_rows(q + (size_t)row_offset * dim, seq_len, dim, head_dim, 0);
  rope_rows(k + (size_t)row_offset * dim, seq_len, dim, head_dim, 0);
}

/* cpu.rs:77-82 */
void ora_add(const float* a, const float* b, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* emit.rs:733-748 (RESIDUAL_ADD, target += source) */
void ora_residual_add(float* target, const float* source, size_t n) {
  for (size_t i = 0; i < n; ++i) target[i] += source[i];
}

/* cpu.rs:71-75 */
void ora_silu_out(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* cpu.rs:277-306 */
void ora_cross_entropy(float* x, const uint32_t* targets, float* losses, uint32_t vocab_size,
                       uint32_t num_rows) {
  for (uint32_t row = 0; row < num_rows; ++row) {
    float* r = x + (size_t)row * vocab_size;
    float m = -INFINITY;
    for (uint32_t i = 0; i < vocab_size; ++i) m = fmaxf(m, r[i]);
    float s = 0.0f;
    for (uint32_t i = 0; i < vocab_size; ++i) s += expf(r[i] - m);
    losses[row] = -(r[targets[row]] - m - logf(s));
    for (uint32_t i = 0; i < vocab_size; ++i) r[i] = expf(r[i] - m) / s;
  }
}

/* emit.rs:931-999, forward half of cpu_attention. */
void ora_causal_attention(const float* q, const float* k, const float* v,
                          float* out, uint32_t seq_len, uint32_t dim,
                          uint32_t head_dim) {
  const float scale = 1.0f / sqrtf((float)head_dim);
  float* p = (float*)malloc(sizeof(float) * (size_t)seq_len);
  memset(out, 0, sizeof(float) * (size_t)seq_len * dim);
  for (uint32_t h0 = 0; h0 < dim; h0 += head_dim) {
    for (uint32_t i = 0; i < seq_len; ++i) {
      const float* qi = q + (size_t)i * dim + h0;
      for (uint32_t j = 0; j <= i; ++j) {
        const float* kj = k + (size_t)j * dim + h0;
        float s = 0.0f;
        for (uint32_t c = 0; c < head_dim; ++c) s += qi[c] * kj[c];
        p[j] = scale * s;
      }
      float mx = -INFINITY;
      for (uint32_t j = 0; j <= i; ++j) mx = fmaxf(mx, p[j]);
      float sum = 0.0f;
      for (uint32_t j = 0; j <= i; ++j) {
        p[j] = expf(p[j] - mx);
        sum += p[j];
      }
      for (uint32_t j = 0; j <= i; ++j) p[j] /= sum;
      float* oi = out + (size_t)i * dim + h0;
      for (uint32_t j = 0; j <= i; ++j) {
        const float* vj = v + (size_t)j * dim + h0;
        for (uint32_t c = 0; c < head_dim; ++c) oi[c] += p[j] * vj[c];
      }
    }
  }
  free(p);
}

/* sampling.rs:83-91 */
uint32_t ora_argmax(const float* logits, uint32_t n) {
  uint32_t best = 0;
  for (uint32_t i = 0; i < n; ++i)
    if (logits[i] > logits[best]) best = i;
  return best;
}

/* sampling.rs:3-16 (apply_repetition_penalty) and 18-81 (sample_token), with
 * the draw r = rand::random() passed in.  The reference sorts with
 * sort_unstable_by, whose order among equal logits is unspecified; this
 * restatement breaks ties by the lower index first. */
static _Thread_local const float* ora_sort_logits;

static int ora_desc_cmp(const void* pa, const void* pb) {
  const uint32_t a = *(const uint32_t*)pa, b = *(const uint32_t*)pb;
  const float la = ora_sort_logits[a], lb = ora_sort_logits[b];
  if (la > lb) return -1;
  if (la < lb) return 1;
  return a < b ? -1 : a > b ? 1 : 0;
}

uint32_t ora_sample_token(const float* logits_in, uint32_t n, float temperature,
                          uint32_t top_k, float top_p, const uint32_t* seen,
                          uint32_t n_seen, float repetition_penalty, double r) {
  float* logits = (float*)malloc((size_t)n * sizeof(float));
  memcpy(logits, logits_in, (size_t)n * sizeof(float));
  if (repetition_penalty != 1.0f) {
    /* Every distinct seen id once, from its original value. */
    for (uint32_t s = 0; s < n_seen; ++s) {
      const uint32_t id = seen[s];
      if (id >= n) continue;
      int dup = 0;
      for (uint32_t t = 0; t < s; ++t)
        if (seen[t] == id) dup = 1;
      if (dup) continue;
      const float l = logits[id];
      logits[id] = l > 0.0f ? l / repetition_penalty : l * repetition_penalty;
    }
  }
  if (temperature <= 0.0f) {
    const uint32_t best = ora_argmax(logits, n);
    free(logits);
    return best;
  }
  uint32_t* idx = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
  for (uint32_t i = 0; i < n; ++i) idx[i] = i;
  ora_sort_logits = logits;
  qsort(idx, n, sizeof(uint32_t), ora_desc_cmp);
  uint32_t len = n;
  if (top_k > 0 && top_k < len) len = top_k;
  const double mx = (double)logits[idx[0]];
  double* probs = (double*)malloc((size_t)len * sizeof(double));
  double sum = 0.0;
  for (uint32_t i = 0; i < len; ++i) {
    probs[i] = exp(((double)logits[idx[i]] - mx) / (double)temperature);
  }
  for (uint32_t i = 0; i < len; ++i) sum += probs[i];
  for (uint32_t i = 0; i < len; ++i) probs[i] /= sum;
  if (top_p < 1.0f) {
    double cum = 0.0;
    uint32_t keep = len;
    for (uint32_t i = 0; i < len; ++i) {
      cum += probs[i];
      if (cum >= (double)top_p) {
        keep = i + 1;
        break;
      }
    }
    len = keep;
    double s = 0.0;
    for (uint32_t i = 0; i < len; ++i) s += probs[i];
    for (uint32_t i = 0; i < len; ++i) probs[i] /= s;
  }
  uint32_t pick = idx[len - 1];
  for (uint32_t i = 0; i < len; ++i) {
    if (r < probs[i]) {
      pick = idx[i];
      break;
    }
    r -= probs[i];
  }
  free(probs);
  free(idx);
  free(logits);
  return pick;
}

/* ---- session ------------------------------------------------------------- */

struct ora_session {
  ora_config cfg;
  ora_weights w;
  uint32_t max_ctx;
  uint32_t cur_len;
  float** k_cache; /* per layer [max_ctx, dim] (inference_graphs.rs:511-538) */
  float** v_cache;
};

ora_session* ora_session_new(const ora_config* cfg, const ora_weights* w,
                             uint32_t max_context_len) {
  ora_session* s = (ora_session*)calloc(1, sizeof(ora_session));
  s->cfg = *cfg;
  s->w = *w;
  s->max_ctx = max_context_len;
  s->k_cache = (float**)calloc(cfg->num_layers, sizeof(float*));
  s->v_cache = (float**)calloc(cfg->num_layers, sizeof(float*));
  for (uint32_t l = 0; l < cfg->num_layers; ++l) {
    s->k_cache[l] = (float*)calloc((size_t)max_context_len * cfg->dim, 4);
    s->v_cache[l] = (float*)calloc((size_t)max_context_len * cfg->dim, 4);
  }
  return s;
}

void ora_session_free(ora_session* s) {
  if (!s) return;
  for (uint32_t l = 0; l < s->cfg.num_layers; ++l) {
    free(s->k_cache[l]);
    free(s->v_cache[l]);
  }
  free(s->k_cache);
  free(s->v_cache);
  free(s);
}

void ora_session_reset(ora_session* s) { s->cur_len = 0; }
void ora_session_set_len(ora_session* s, uint32_t len) {
  s->cur_len = len < s->max_ctx ? len : s->max_ctx;
}
uint32_t ora_session_cur_len(const ora_session* s) { return s->cur_len; }
const float* ora_session_k_cache(const ora_session* s, uint32_t l) {
  return s->k_cache[l];
}
const float* ora_session_v_cache(const ora_session* s, uint32_t l) {
  return s->v_cache[l];
}

/* Final norm + lm_head on one hidden row (inference.rs:120-168, 228-252). */
static void logits_tail(const ora_session* s, const float* row,
                        float* logits) {
  const ora_config* c = &s->cfg;
  float* normed = (float*)malloc(sizeof(float) * c->dim);
  ora_rmsnorm(row, s->w.final_norm, normed, 1, c->dim, c->norm_eps);
  ora_matmul(normed, s->w.lm_head, logits, 1, c->vocab_size, c->dim);
  free(normed);
}

/* inference.rs:61-176 with build_prefill_layer (inference_graphs.rs:198-337).
 * The reference CPU backend has no flash-attention kernel (shaders/mod.rs:422,
 * cpu: None); attention is restated from cpu_attention (emit.rs:931-999),
 * which the reference's flash test holds the GPU kernels to. */
int ora_session_prefill(ora_session* s, const uint32_t* tokens, uint32_t n,
                        float* logits) {
  if (n == 0) return ORA_E_EMPTY_PROMPT;
  if (n > s->max_ctx) return ORA_E_PROMPT_TOO_LONG;
  if (s->cur_len != 0) return ORA_E_CACHE_NOT_EMPTY;
  const ora_config* c = &s->cfg;
  const uint32_t d = c->dim, hd = d / c->num_heads, f = c->ffn_hidden;
  size_t rd = (size_t)n * d;
  float* hidden = (float*)malloc(4 * rd);
  float* norm = (float*)malloc(4 * rd);
  float* qkv = (float*)malloc(4 * rd * 3);
  float* q = (float*)malloc(4 * rd);
  float* k = (float*)malloc(4 * rd);
  float* v = (float*)malloc(4 * rd);
  float* attn = (float*)malloc(4 * rd);
  float* ffn = (float*)malloc(4 * (size_t)n * f);

  ora_embedding(tokens, s->w.embedding, hidden, c->vocab_size, d, n);
  for (uint32_t l = 0; l < c->num_layers; ++l) {
    ora_rmsnorm(hidden, s->w.norm_1[l], norm, n, d, c->norm_eps);
    ora_matmul(norm, s->w.qkv_proj[l], qkv, n, 3 * d, d);
    ora_head_gather(qkv, q, n, 3 * d, d, 0);
    ora_head_gather(qkv, k, n, 3 * d, d, d);
    ora_head_gather(qkv, v, n, 3 * d, d, 2 * d);
    ora_rope(q, n, d, hd);
    ora_rope(k, n, d, hd);
    ora_cache_write(k, s->k_cache[l], n, d, 0);
    ora_cache_write(v, s->v_cache[l], n, d, 0);
    ora_causal_attention(q, k, v, attn, n, d, hd);
    ora_matmul_add(attn, s->w.out_proj[l], hidden, n, d, d);
    ora_rmsnorm(hidden, s->w.norm_2[l], norm, n, d, c->norm_eps);
    ora_matmul(norm, s->w.ffn_up[l], ffn, n, f, d);
    ora_silu(ffn, (size_t)n * f);
    ora_matmul_add(ffn, s->w.ffn_down[l], hidden, n, d, f);
  }
  logits_tail(s, hidden + (size_t)(n - 1) * d, logits);
  s->cur_len = n;
  free(hidden); free(norm); free(qkv); free(q); free(k); free(v);
  free(attn); free(ffn);
  return ORA_OK;
}

/* Trainer::forward (train.rs:256-275) with TransformerBlock's node order
 * (layers.rs:551-760): norm_1, qkv_proj, qkv_split, rope_qk and flash
 * attention per sequence at row_offset b * seq_len, out_proj, add_1, norm_2,
 * ffn_up, silu_out, ffn_down, add_2; then final_norm and lm_head on every
 * row and CrossEntropy (layers.rs:465-522).  Flash attention has no CPU twin
 * (shaders/mod.rs:422); it is restated from cpu_attention (emit.rs:931-999)
 * as for prefill. */
float ora_forward_train(const ora_config* c, const ora_weights* w, const uint32_t* tokens,
                        const uint32_t* targets, uint32_t batch, uint32_t seq_len,
                        float* losses, float* probs, float* hidden) {
  const uint32_t d = c->dim, hd = d / c->num_heads, f = c->ffn_hidden, V = c->vocab_size;
  const uint32_t rows = batch * seq_len;
  const size_t rd = (size_t)rows * d;
  float* x = (float*)malloc(4 * rd);
  float* x1 = (float*)malloc(4 * rd);
  float* norm = (float*)malloc(4 * rd);
  float* qkv = (float*)malloc(4 * rd * 3);
  float* q = (float*)malloc(4 * rd);
  float* k = (float*)malloc(4 * rd);
  float* v = (float*)malloc(4 * rd);
  float* attn = (float*)malloc(4 * rd);
  float* proj = (float*)malloc(4 * rd);
  float* up = (float*)malloc(4 * (size_t)rows * f);
  float* act = (float*)malloc(4 * (size_t)rows * f);
  float* logits = (float*)malloc(4 * (size_t)rows * V);

  ora_embedding(tokens, w->embedding, x, V, d, rows);
  for (uint32_t l = 0; l < c->num_layers; ++l) {
    ora_rmsnorm(x, w->norm_1[l], norm, rows, d, c->norm_eps);
    ora_matmul(norm, w->qkv_proj[l], qkv, rows, 3 * d, d);
    ora_qkv_split(qkv, q, k, v, rows, 3 * d, d);
    for (uint32_t b = 0; b < batch; ++b) ora_rope_qk(q, k, seq_len, d, hd, b * seq_len);
    for (uint32_t b = 0; b < batch; ++b) {
      const size_t o = (size_t)b * seq_len * d;
      ora_causal_attention(q + o, k + o, v + o, attn + o, seq_len, d, hd);
    }
    ora_matmul(attn, w->out_proj[l], proj, rows, d, d);
    ora_add(x, proj, x1, rd);
    ora_rmsnorm(x1, w->norm_2[l], norm, rows, d, c->norm_eps);
    ora_matmul(norm, w->ffn_up[l], up, rows, f, d);
    ora_silu_out(up, act, (size_t)rows * f);
    ora_matmul(act, w->ffn_down[l], proj, rows, d, f);
    ora_add(x1, proj, x, rd);
  }
  if (hidden) memcpy(hidden, x, 4 * rd);
  ora_rmsnorm(x, w->final_norm, norm, rows, d, c->norm_eps);
  ora_matmul(norm, w->lm_head, logits, rows, V, d);
  ora_cross_entropy(logits, targets, losses, V, rows);
  if (probs) memcpy(probs, logits, 4 * (size_t)rows * V);
  /* CrossEntropy::loss (layers.rs:512-515): sequential f32 sum / len. */
  float sum = 0.0f;
  for (uint32_t r = 0; r < rows; ++r) sum += losses[r];
  free(x); free(x1); free(norm); free(qkv); free(q); free(k); free(v); free(attn);
  free(proj); free(up); free(act); free(logits);
  return sum / (float)rows;
}

/* inference.rs:178-262 with build_decode_layer (inference_graphs.rs:339-509)
 * and the per-step metas of DecodeScratch::update_for_step (:164-195). */
int ora_session_decode_step(ora_session* s, uint32_t token, float* logits) {
  if (s->cur_len >= s->max_ctx) return ORA_E_CONTEXT_FULL;
  const ora_config* c = &s->cfg;
  const uint32_t d = c->dim, hd = d / c->num_heads, f = c->ffn_hidden;
  const uint32_t pos = s->cur_len, attn_len = pos + 1;
  const float scale = 1.0f / sqrtf((float)hd);
  float* hidden = (float*)malloc(4 * (size_t)d);
  float* norm = (float*)malloc(4 * (size_t)d);
  float* qkv = (float*)malloc(4 * (size_t)d * 3);
  float* q = (float*)malloc(4 * (size_t)d);
  float* k = (float*)malloc(4 * (size_t)d);
  float* v = (float*)malloc(4 * (size_t)d);
  float* scores = (float*)malloc(4 * (size_t)c->num_heads * attn_len);
  float* attn = (float*)malloc(4 * (size_t)d);
  float* ffn = (float*)malloc(4 * (size_t)f);

  ora_embedding(&token, s->w.embedding, hidden, c->vocab_size, d, 1);
  for (uint32_t l = 0; l < c->num_layers; ++l) {
    ora_rmsnorm(hidden, s->w.norm_1[l], norm, 1, d, c->norm_eps);
    ora_matmul(norm, s->w.qkv_proj[l], qkv, 1, 3 * d, d);
    ora_head_gather(qkv, q, 1, 3 * d, d, 0);
    ora_head_gather(qkv, k, 1, 3 * d, d, d);
    ora_head_gather(qkv, v, 1, 3 * d, d, 2 * d);
    ora_rope_offset(q, 1, d, hd, pos);
    ora_rope_offset(k, 1, d, hd, pos);
    ora_cache_write(k, s->k_cache[l], 1, d, pos);
    ora_cache_write(v, s->v_cache[l], 1, d, pos);
    ora_attn_qk_cached(q, s->k_cache[l], scores, attn_len, d, hd);
    ora_softmax_rect(scores, c->num_heads, attn_len, scale);
    ora_attn_av_cached(scores, s->v_cache[l], attn, attn_len, d, hd);
    ora_matmul_add(attn, s->w.out_proj[l], hidden, 1, d, d);
    ora_rmsnorm(hidden, s->w.norm_2[l], norm, 1, d, c->norm_eps);
    ora_matmul(norm, s->w.ffn_up[l], ffn, 1, f, d);
    ora_silu(ffn, f);
    ora_matmul_add(ffn, s->w.ffn_down[l], hidden, 1, d, f);
  }
  logits_tail(s, hidden, logits);
  s->cur_len = pos + 1;
  free(hidden); free(norm); free(qkv); free(q); free(k); free(v);
  free(scores); free(attn); free(ffn);
  return ORA_OK;
}
