// HIP kernels of the akasha-core inference path, written for CDNA4 (gfx950).
//
// Two families live here:
//  * per-shader kernels with the semantics of the reference's Shader
//    registry (src/shaders/mod.rs), reading their meta from device memory at
//    execution time like the reference's generic CUDA launch ABI;
//  * fused kernels of the batched session: a skinny fp32-MFMA GEMM for the
//    <= 32-row decode step with the RMSNorm folded into its A-operand
//    prologue and bias-free epilogues (residual add, SiLU, RoPE + KV append,
//    logits + argmax partials), split-T single-query attention over the KV
//    cache, a 128x128 LDS-tiled fp32-MFMA GEMM for prefill and an MFMA
//    causal flash attention.
//
// MFMA used: v_mfma_f32_32x32x2f32.  Operand layout (wave64): lane l
// supplies A[l % 32][l / 32] and B[l / 32][l % 32]; accumulator register r
// of lane l holds D[(r / 4) * 8 + (l / 32) * 4 + r % 4][l % 32].
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kernels.h"

namespace akh {

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row (within a 32x32 tile) held by accumulator register r of a lane in
// half h (= lane / 32).
__device__ __forceinline__ int acc_row(int r, int h) {
  return (r >> 2) * 8 + h * 4 + (r & 3);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over a 256-thread block; every thread gets the total.  The order is
// fixed (butterfly within waves, then waves 0..3), so results are
// reproducible run to run.
__device__ float block_sum256(float v, float* red4) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  return ((red4[0] + red4[1]) + red4[2]) + red4[3];
}

__device__ float block_max256(float v, float* red4) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
}

// x0*c - x1*s and x0*s + x1*c, each product rounded separately as the
// reference's CPU RoPE does (src/shaders/cpu.rs:102-103).
__device__ __forceinline__ void rope_pair(float& x0, float& x1, float c,
                                          float s) {
  float a = __fmul_rn(x0, c), b = __fmul_rn(x1, s);
  float e = __fmul_rn(x0, s), f = __fmul_rn(x1, c);
  x0 = __fsub_rn(a, b);
  x1 = __fadd_rn(e, f);
}

// ===========================================================================
// Per-shader kernels (live metas)
// ===========================================================================

// EMBEDDING (src/shaders/cpu.rs:25-41): ids >= vocab give a zero row.
__global__ void k_embedding(const uint32_t* tokens, const float* table,
                            float* out, const akh_embedding_meta* meta) {
  const uint32_t vocab = meta->vocab_size, dim = meta->dim;
  const uint32_t t = blockIdx.y;
  if (t >= meta->seq_len) return;
  const uint32_t id = tokens[t];
  for (uint32_t c = blockIdx.x * blockDim.x + threadIdx.x; c < dim;
       c += gridDim.x * blockDim.x)
    out[(size_t)t * dim + c] = id < vocab ? table[(size_t)id * dim + c] : 0.f;
}

// Host-sized variant for the batched prefill.
__global__ void k_embedding_rows(const uint32_t* tokens, const float* table,
                                 float* out, int d, uint32_t vocab) {
  const int t = blockIdx.x;
  const uint32_t id = tokens[t];
  const float4* src = reinterpret_cast<const float4*>(table + (size_t)id * d);
  float4* dst = reinterpret_cast<float4*>(out + (size_t)t * d);
  for (int c = threadIdx.x; c < d / 4; c += blockDim.x)
    dst[c] = id < vocab ? src[c] : make_float4(0.f, 0.f, 0.f, 0.f);
}

// RMSNORM (src/shaders/cpu.rs:205-222), one 256-thread block per row.
__device__ void rmsnorm_row(const float* xr, const float* w, float* o,
                            uint32_t size, float eps) {
  __shared__ float red4[4];
  float ss = 0.f;
  for (uint32_t c = threadIdx.x; c < size; c += 256) ss += xr[c] * xr[c];
  ss = block_sum256(ss, red4);
  const float rs = 1.0f / sqrtf(ss / (float)size + eps);
  for (uint32_t c = threadIdx.x; c < size; c += 256)
    o[c] = __fmul_rn(__fmul_rn(xr[c], rs), w[c]);
}

__global__ __launch_bounds__(256) void k_rmsnorm(const float* x,
                                                 const float* w, float* out,
                                                 const akh_norm_meta* meta) {
  const uint32_t r = blockIdx.x;
  if (r >= meta->seq_len) return;
  const uint32_t size = meta->size;
  rmsnorm_row(x + (size_t)r * size, w, out + (size_t)r * size, size,
              meta->eps);
}

__global__ __launch_bounds__(256) void k_rows_rmsnorm(const float* x,
                                                      const float* w,
                                                      float* out, int size,
                                                      float eps) {
  const size_t r = blockIdx.x;
  rmsnorm_row(x + r * size, w, out + r * size, size, eps);
}

// HEAD_GATHER (src/shaders/cpu.rs:238-255).
__global__ void k_head_gather(const float* src, float* dst,
                              const akh_head_move_meta* meta) {
  const uint32_t rows = meta->seq_len, full = meta->full_dim,
                 hd = meta->head_dim, off = meta->head_offset;
  const size_t total = (size_t)rows * hd;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / hd, c = i % hd;
    dst[i] = src[r * full + off + c];
  }
}

// ROPE / ROPE_OFFSET (src/shaders/cpu.rs:84-142): in place, pairs
// (2i, 2i+1) of each head rotated by pos * 10000^(-2i/head_dim).
__global__ void k_rope(float* x, const uint32_t* meta, int with_offset) {
  const uint32_t rows = meta[0], dim = meta[1], hd = meta[2];
  const uint32_t pos0 = with_offset ? meta[3] : 0u;
  const size_t pairs = (size_t)rows * (dim / 2);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t t = (uint32_t)(i / (dim / 2));
    const uint32_t c = (uint32_t)(i % (dim / 2)) * 2u;
    const uint32_t di = c % hd;
    const float freq = 1.0f / powf(10000.0f, (float)di / (float)hd);
    const float angle = (float)(t + pos0) * freq;
    float sn, cs;
    sincosf(angle, &sn, &cs);
    float* p = x + (size_t)t * dim + c;
    float x0 = p[0], x1 = p[1];
    rope_pair(x0, x1, cs, sn);
    p[0] = x0;
    p[1] = x1;
  }
}

// CACHE_WRITE (src/shaders/cpu.rs:224-236).
__global__ void k_cache_write(const float* src, float* dst,
                              const akh_cache_write_meta* meta) {
  const uint32_t rows = meta->row_count, width = meta->width,
                 off = meta->dst_row_offset;
  const size_t total = (size_t)rows * width;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x)
    dst[(size_t)off * width + i] = src[i];
}

// ATTN_QK_CACHED (src/shaders/cpu.rs:144-162): one thread per (row j, head).
__global__ void k_attn_qk_cached(const float* q, const float* kc,
                                 float* scores,
                                 const akh_attn_cached_meta* meta) {
  const uint32_t len = meta->attn_len, dim = meta->dim, hd = meta->head_dim;
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x, h = blockIdx.y;
  if (j >= len || h >= dim / hd) return;
  const float* qh = q + h * hd;
  const float* kr = kc + (size_t)j * dim + h * hd;
  float s = 0.f;
  for (uint32_t c = 0; c < hd; ++c) s += qh[c] * kr[c];
  scores[(size_t)h * len + j] = s;
}

// SOFTMAX_RECT (src/shaders/cpu.rs:180-203), one block per row.
__global__ __launch_bounds__(256) void k_softmax_rect(
    float* x, const akh_softmax_rect_meta* meta) {
  __shared__ float red4[4];
  const uint32_t r = blockIdx.x;
  if (r >= meta->num_rows) return;
  const uint32_t width = meta->width;
  const float scale = meta->scale;
  float* row = x + (size_t)r * width;
  float mx = -INFINITY;
  for (uint32_t i = threadIdx.x; i < width; i += 256)
    mx = fmaxf(mx, row[i] * scale);
  mx = block_max256(mx, red4);
  float sum = 0.f;
  for (uint32_t i = threadIdx.x; i < width; i += 256) {
    const float e = expf(row[i] * scale - mx);
    row[i] = e;
    sum += e;
  }
  sum = block_sum256(sum, red4);
  for (uint32_t i = threadIdx.x; i < width; i += 256) row[i] = row[i] / sum;
}

// ATTN_AV_CACHED (src/shaders/cpu.rs:164-178): one thread per channel.
__global__ void k_attn_av_cached(const float* p, const float* vc, float* out,
                                 const akh_attn_cached_meta* meta) {
  const uint32_t len = meta->attn_len, dim = meta->dim, hd = meta->head_dim;
  const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= dim) return;
  const float* ph = p + (size_t)(d / hd) * len;
  float s = 0.f;
  for (uint32_t j = 0; j < len; ++j) s += ph[j] * vc[(size_t)j * dim + d];
  out[d] = s;
}

// SILU (src/shaders/cpu.rs:63-69).
__global__ void k_silu(float* x, uint32_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float v = x[i];
    x[i] = v / (1.0f + expf(-v));
  }
}

// Greedy argmax per row (src/nn/sampling.rs:83-91): the first index of the
// maximum.  Candidates are merged with "larger wins, equal -> lower index",
// which equals the sequential strict-> scan for any split of the row.
__device__ __forceinline__ void amax_merge(float& bv, uint32_t& bi, float v,
                                           uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__device__ void block_amax256(float& bv, uint32_t& bi) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    amax_merge(bv, bi, ov, oi);
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  bv = sv[0];
  bi = si[0];
  for (int k = 1; k < 4; ++k) amax_merge(bv, bi, sv[k], si[k]);
}

__global__ __launch_bounds__(256) void k_argmax_rows(const float* logits,
                                                     uint32_t n,
                                                     uint32_t* out) {
  const float* row = logits + (size_t)blockIdx.x * n;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = threadIdx.x; i < n; i += 256) amax_merge(bv, bi, row[i], i);
  block_amax256(bv, bi);
  if (threadIdx.x == 0) out[blockIdx.x] = bi == 0xFFFFFFFFu ? 0u : bi;
}

// ===========================================================================
// Batched decode path
// ===========================================================================

// Gather M rows into dst [M, d] (embedding lookup or last-row pick) and
// emit their sum-of-squares partials per kSlotW columns.  One block per row.
__global__ __launch_bounds__(256) void k_gather_rows(
    const float* table, const uint32_t* ids, uint32_t vocab, const float* src,
    long src_row0, long src_row_stride, float* dst, int d, float* ss) {
  const int m = blockIdx.x;
  const float* row = nullptr;
  if (ids) {
    const uint32_t id = ids[m];
    row = id < vocab ? table + (size_t)id * d : nullptr;
  } else {
    row = src + (size_t)(src_row0 + (long)m * src_row_stride) * d;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nslots = d / kSlotW;
  for (int sl = w; sl < nslots; sl += 4) {
    const int c = sl * kSlotW + lane;
    float v = 0.f;
    if (lane < kSlotW) {
      v = row ? row[c] : 0.f;
      dst[(size_t)m * d + c] = v;
    }
    // Left-to-right over the slot's columns via a fixed butterfly.
    const float s = wave_sum(v * v);
    if (lane == 0) ss[(size_t)m * nslots + sl] = s;
  }
}

// Per-row rsqrt from the slot partials, summed in slot order.
__device__ __forceinline__ float norm_rscale(const float* ss, int m,
                                             int nslots, int size,
                                             float eps) {
  float t = 0.f;
  for (int i = 0; i < nslots; ++i) t += ss[(size_t)m * nslots + i];
  return 1.0f / sqrtf(t / (float)size + eps);
}

// Epilogue on an adjacent column pair (n, n + 1), n even, of row m.
template <int EPI>
__device__ __forceinline__ void epi_pair_skinny(const SkinnyParams& p, int M,
                                                int N, int m, int n, float v0,
                                                float v1) {
  if (m >= M || n >= N) return;
  const bool has1 = n + 1 < N;
  if (EPI == EPI_STORE || EPI == EPI_LOGITS) {
    float* y = p.y + (size_t)m * N + n;
    y[0] = v0;
    if (has1) y[1] = v1;
  } else if (EPI == EPI_ADD) {
    float* y = p.y + (size_t)m * N + n;
    y[0] = y[0] + v0;
    if (has1) y[1] = y[1] + v1;
  } else if (EPI == EPI_SILU) {
    float* y = p.y + (size_t)m * N + n;
    y[0] = v0 / (1.0f + expf(-v0));
    if (has1) y[1] = v1 / (1.0f + expf(-v1));
  } else if (EPI == EPI_QKV) {
    const int dim = p.dim;
    const int region = n / dim, c = n - region * dim;
    const int pos = p.pos[m];
    if (region < 2) {
      const int i = (c % p.head_dim) >> 1;
      const float2 cs = p.rope[(size_t)pos * (p.head_dim >> 1) + i];
      rope_pair(v0, v1, cs.x, cs.y);
    }
    float* dst;
    if (region == 0)
      dst = p.q_out + (size_t)m * dim + c;
    else
      dst = (region == 1 ? p.kcache : p.vcache) + (size_t)m * p.seq_stride +
            (size_t)pos * dim + c;
    dst[0] = v0;
    dst[1] = v1;
  }
}

// Skinny GEMM for M <= 32 (every decode matmul and the prefill lm_head).
//
// Grid (N tiles of NT = 32*C columns, ksplit).  Each 256-thread block owns
// one N tile and one K chunk; its four waves split the chunk again and each
// runs v_mfma_f32_32x32x2f32 with all 32 rows as the A operand, so every
// weight byte is read once per step for the whole batch.  Within a wave,
// half h of the lanes walks rows kbase_h + s; a lane loads C consecutive
// weights of one row (column n0 + C*j + c feeds MFMA tile c), so a wave
// load instruction covers two full 128*C-byte row segments.  Partials are
// reduced across waves in LDS and, for ksplit > 1, across blocks by the last
// block to arrive at the tile's counter (fixed summation order, so results
// are deterministic).
template <int C, int EPI, bool NORM>
__global__ __launch_bounds__(256) void k_skinny(SkinnyParams p) {
  constexpr int NT = 32 * C;
  __shared__ float red[4][32][NT + 1];
  __shared__ float sq[32][NT + 1];
  __shared__ int s_last;

  int M = p.M, N = p.N, K = p.K;
  if (p.meta) {
    M = (int)p.meta->m;
    N = (int)p.meta->n;
    K = (int)p.meta->k;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int tile = blockIdx.x, ks = blockIdx.y;
  const int n0 = tile * NT;
  if (n0 >= N) return;  // a grid sized for a larger shape

  // K chunk of this block (multiple of 64 so each half-wave gets a
  // multiple of 8 rows), then this wave's quarter and this half's rows.
  // Derived from the launched grid, so the number of chunks never exceeds
  // what the host sized the workspace for, whatever the live meta says.
  const int kc = max(64, (((K + (int)gridDim.y - 1) / (int)gridDim.y) + 63) & ~63);
  const int nks = max(1, (K + kc - 1) / kc);
  if (ks >= nks) return;
  const int kb = ks * kc;
  const int ke = min(K, kb + kc);
  const int hl = kc / 8;  // rows per half-wave
  const int kbase = kb + wave * (kc / 4) + h * hl;

  float rs = 0.f;
  if (NORM && j < M) rs = norm_rscale(p.ss_in, j, p.ss_slots, K, p.eps);

  f32x16 acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) acc[c] = zero16();

  const bool row_ok = j < M;
  const float* xrow = p.x + (size_t)(row_ok ? j : 0) * K;
  const int ncol = n0 + C * j;
  bool col_ok[C];
#pragma unroll
  for (int c = 0; c < C; ++c) col_ok[c] = ncol + c < N;
  const bool full_cols = ncol + C <= N;

  constexpr int U = 8;
  for (int s0 = 0; s0 < hl; s0 += U) {
    float a[U];
    float b[U][C];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kbase + s0 + u;
      const bool kok = k < ke;
      const int kk = kok ? k : 0;
      const float* wr = p.w + (size_t)kk * N + ncol;
      if (C == 4 && full_cols && (N & 3) == 0) {
        const float4 t = *reinterpret_cast<const float4*>(wr);
        b[u][0] = t.x;
        b[u][C > 1 ? 1 : 0] = t.y;
        b[u][C > 2 ? 2 : 0] = t.z;
        b[u][C > 3 ? 3 : 0] = t.w;
      } else if (C == 2 && full_cols && (N & 1) == 0) {
        const float2 t = *reinterpret_cast<const float2*>(wr);
        b[u][0] = t.x;
        b[u][C > 1 ? 1 : 0] = t.y;
      } else {
#pragma unroll
        for (int c = 0; c < C; ++c) b[u][c] = col_ok[c] ? wr[c] : 0.f;
      }
#pragma unroll
      for (int c = 0; c < C; ++c) b[u][c] = kok ? b[u][c] : 0.f;
      float av = (row_ok && kok) ? xrow[kk] : 0.f;
      if (NORM) av = (row_ok && kok) ? __fmul_rn(__fmul_rn(av, rs), p.gain[kk]) : 0.f;
      a[u] = av;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] = mfma32(a[u], b[u][c], acc[c]);
  }

  // Cross-wave reduction in LDS.
#pragma unroll
  for (int c = 0; c < C; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][acc_row(r, h)][C * j + c] = acc[c][r];
  __syncthreads();

  constexpr int PAIRS = 32 * NT / 2;  // column pairs in the tile
  constexpr int PER = PAIRS / 256;    // per thread (C >= 1 -> >= 2)
  float v0s[PER], v1s[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = threadIdx.x + 256 * i;
    const int m = idx / (NT / 2), col = (idx % (NT / 2)) * 2;
    v0s[i] = ((red[0][m][col] + red[1][m][col]) + red[2][m][col]) + red[3][m][col];
    v1s[i] = ((red[0][m][col + 1] + red[1][m][col + 1]) + red[2][m][col + 1]) +
             red[3][m][col + 1];
  }

  if (nks > 1) {
    // Publish this block's partial tile; the last block sums all of them.
    float* mine = p.ws + ((size_t)tile * nks + ks) * 32 * NT;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int m = idx / (NT / 2), col = (idx % (NT / 2)) * 2;
      *reinterpret_cast<float2*>(mine + m * NT + col) = make_float2(v0s[i], v1s[i]);
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned prev = atomicAdd(&p.cnt[tile], 1u);
      s_last = prev == (unsigned)(nks - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float* all = p.ws + (size_t)tile * nks * 32 * NT;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int m = idx / (NT / 2), col = (idx % (NT / 2)) * 2;
      float t0 = 0.f, t1 = 0.f;
      for (int q = 0; q < nks; ++q) {
        const float* src = all + (size_t)q * 32 * NT + m * NT + col;
        t0 += __builtin_nontemporal_load(src);
        t1 += __builtin_nontemporal_load(src + 1);
      }
      v0s[i] = t0;
      v1s[i] = t1;
    }
    if (threadIdx.x == 0) atomicExch(&p.cnt[tile], 0u);
  }

#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = threadIdx.x + 256 * i;
    const int m = idx / (NT / 2), col = (idx % (NT / 2)) * 2;
    const int n = n0 + col;
    epi_pair_skinny<EPI>(p, M, N, m, n, v0s[i], v1s[i]);
    if (EPI == EPI_ADD && p.ss_out) {
      float y0 = 0.f, y1 = 0.f;
      if (m < M && n < N) y0 = p.y[(size_t)m * N + n];
      if (m < M && n + 1 < N) y1 = p.y[(size_t)m * N + n + 1];
      sq[m][col] = y0 * y0;
      sq[m][col + 1] = y1 * y1;
    }
    if (EPI == EPI_LOGITS) {
      sq[m][col] = (m < M && n < N) ? v0s[i] : -INFINITY;
      sq[m][col + 1] = (m < M && n + 1 < N) ? v1s[i] : -INFINITY;
    }
  }
  if (EPI == EPI_ADD && p.ss_out) {
    __syncthreads();
    if (threadIdx.x < 32 && (int)threadIdx.x < M) {
      const int m = threadIdx.x;
      // One slot per kSlotW columns; NT is a multiple of kSlotW.
      for (int sl = 0; sl < NT / kSlotW; ++sl) {
        float t = 0.f;
        for (int c = 0; c < kSlotW; ++c) t += sq[m][sl * kSlotW + c];
        p.ss_out[(size_t)m * (N / kSlotW) + (n0 / kSlotW) + sl] = t;
      }
    }
  }
  if (EPI == EPI_LOGITS) {
    __syncthreads();
    if (threadIdx.x < 32 && (int)threadIdx.x < M) {
      const int m = threadIdx.x;
      float bv = sq[m][0];
      int bi = 0;
      for (int c = 1; c < NT; ++c)
        if (sq[m][c] > bv) {
          bv = sq[m][c];
          bi = c;
        }
      const int ntiles = (N + NT - 1) / NT;
      p.amax[(size_t)m * ntiles + tile] =
          make_uint2(__float_as_uint(bv), (uint32_t)(n0 + bi));
    }
  }
}

// Final argmax over the lm_head tiles' partials, plus the step's
// bookkeeping on the device.  hist[m, p] is the token at position p of
// sequence m.  Decode (pos set): record the consumed token at pos[m], the
// chosen one at pos[m] + 1, advance pos[m].  Prefill (pos null): record the
// chosen token at position `next_pos`.
__global__ __launch_bounds__(256) void k_argmax_final(
    const uint2* part, int ntiles, uint32_t* tok, int* pos, uint32_t* hist,
    int hist_stride, int next_pos) {
  const int m = blockIdx.x;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (int t = threadIdx.x; t < ntiles; t += 256) {
    const uint2 v = part[(size_t)m * ntiles + t];
    amax_merge(bv, bi, __uint_as_float(v.x), v.y);
  }
  block_amax256(bv, bi);
  if (threadIdx.x == 0) {
    const uint32_t id = bi == 0xFFFFFFFFu ? 0u : bi;
    uint32_t* hrow = hist ? hist + (size_t)m * hist_stride : nullptr;
    if (pos) {
      const int p = pos[m];
      if (hrow) {
        hrow[p] = tok[m];
        hrow[p + 1] = id;
      }
      pos[m] = p + 1;
    } else if (hrow) {
      hrow[next_pos] = id;
    }
    tok[m] = id;
  }
}

// Single-query attention over the KV cache, split along T (decode).
//
// Grid (B*H, nsplit), 256 threads.  HD/4 lanes cover one cached row with a
// float4 each, so a wave reads 64*16 contiguous-per-row bytes per load; the
// block walks its T chunk, keeps the scaled scores in LDS, exponentiates
// against the chunk maximum and accumulates p*V.  Chunk partials
// (max, sum, o[HD]) are merged by the last block of each (b, h).
template <int HD>
__global__ __launch_bounds__(256) void k_decode_attn(DecodeAttnParams p) {
  constexpr int LPR = HD / 4;       // lanes per row
  constexpr int RPW = 64 / LPR;     // rows per wave per step
  constexpr int RPB = 4 * RPW;      // rows per block per step
  constexpr int MAXC = 1024;        // chunk capacity (host keeps chunk <= this)
  __shared__ float sc[MAXC];
  __shared__ float red4[4];
  __shared__ float4 ored[4][LPR];
  __shared__ int s_last;

  const int bh = blockIdx.x, sidx = blockIdx.y;
  const int b = bh / p.H, hh = bh - b * p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane % LPR, rl = lane / LPR;
  const int T = p.pos[b] + 1;
  const int chunk = (T + p.nsplit - 1) / p.nsplit;
  const int r0 = sidx * chunk;
  const int r1 = min(T, r0 + chunk);
  const int len = max(0, r1 - r0);

  const float4 q4 = *reinterpret_cast<const float4*>(p.q + (size_t)b * p.d + hh * HD + 4 * g);
  const float* kbase = p.kc + (size_t)b * p.seq_stride + hh * HD + 4 * g;
  const float* vbase = p.vc + (size_t)b * p.seq_stride + hh * HD + 4 * g;

  // Scores.
  for (int base = 0; base < len; base += RPB) {
    const int r = base + wave * RPW + rl;
    float s = 0.f;
    if (r < len) {
      const float4 k4 = *reinterpret_cast<const float4*>(kbase + (size_t)(r0 + r) * p.d);
      s = q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (g == 0 && r < len) sc[r] = s * p.scale;
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < len; i += 256) mx = fmaxf(mx, sc[i]);
  mx = block_max256(mx, red4);
  float l = 0.f;
  for (int i = threadIdx.x; i < len; i += 256) {
    const float e = expf(sc[i] - mx);
    sc[i] = e;
    l += e;
  }
  l = block_sum256(l, red4);  // contains the barrier that publishes sc[]

  // p . V
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int base = 0; base < len; base += RPB) {
    const int r = base + wave * RPW + rl;
    if (r < len) {
      const float pr = sc[r];
      const float4 v4 = *reinterpret_cast<const float4*>(vbase + (size_t)(r0 + r) * p.d);
      acc.x += pr * v4.x;
      acc.y += pr * v4.y;
      acc.z += pr * v4.z;
      acc.w += pr * v4.w;
    }
  }
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) {
    acc.x += __shfl_xor(acc.x, o, 64);
    acc.y += __shfl_xor(acc.y, o, 64);
    acc.z += __shfl_xor(acc.z, o, 64);
    acc.w += __shfl_xor(acc.w, o, 64);
  }
  if (rl == 0) ored[wave][g] = acc;
  __syncthreads();

  float* out = p.out + (size_t)b * p.d + hh * HD;
  if (p.nsplit == 1) {
    if (threadIdx.x < LPR) {
      const int t = threadIdx.x;
      float4 o = ored[0][t];
      for (int w = 1; w < 4; ++w) {
        o.x += ored[w][t].x; o.y += ored[w][t].y;
        o.z += ored[w][t].z; o.w += ored[w][t].w;
      }
      *reinterpret_cast<float4*>(out + 4 * t) =
          make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
    }
    return;
  }

  // Publish (max, sum, o) of this chunk; the last chunk block merges.
  constexpr int REC = HD + 4;
  float* rec = p.ws + ((size_t)bh * p.nsplit + sidx) * REC;
  if (threadIdx.x < LPR) {
    const int t = threadIdx.x;
    float4 o = ored[0][t];
    for (int w = 1; w < 4; ++w) {
      o.x += ored[w][t].x; o.y += ored[w][t].y;
      o.z += ored[w][t].z; o.w += ored[w][t].w;
    }
    *reinterpret_cast<float4*>(rec + 4 + 4 * t) = o;
    if (t == 0) {
      rec[0] = len > 0 ? mx : -INFINITY;
      rec[1] = l;
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&p.cnt[bh], 1u);
    s_last = prev == (unsigned)(p.nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* recs = p.ws + (size_t)bh * p.nsplit * REC;
  if (threadIdx.x < LPR) {
    const int t = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < p.nsplit; ++s)
      M = fmaxf(M, __builtin_nontemporal_load(recs + (size_t)s * REC));
    float L = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < p.nsplit; ++s) {
      const float ms = __builtin_nontemporal_load(recs + (size_t)s * REC);
      const float ls = __builtin_nontemporal_load(recs + (size_t)s * REC + 1);
      const float wgt = ms == -INFINITY ? 0.f : expf(ms - M);
      const float* os = recs + (size_t)s * REC + 4 + 4 * t;
      L += wgt * ls;
      o.x += wgt * __builtin_nontemporal_load(os);
      o.y += wgt * __builtin_nontemporal_load(os + 1);
      o.z += wgt * __builtin_nontemporal_load(os + 2);
      o.w += wgt * __builtin_nontemporal_load(os + 3);
    }
    *reinterpret_cast<float4*>(out + 4 * t) =
        make_float4(o.x / L, o.y / L, o.z / L, o.w / L);
  }
  if (threadIdx.x == 0) atomicExch(&p.cnt[bh], 0u);
}

// ===========================================================================
// Prefill: LDS-tiled fp32 MFMA GEMM
// ===========================================================================

template <int EPI>
__device__ __forceinline__ void epi_pair_gemm(const GemmParams& p, int M,
                                              int N, int m, int n, float v0,
                                              float v1) {
  if (m >= M || n >= N) return;
  const bool has1 = n + 1 < N;
  if (EPI == EPI_STORE) {
    float* y = p.c + (size_t)m * N + n;
    y[0] = v0;
    if (has1) y[1] = v1;
  } else if (EPI == EPI_ADD) {
    float* y = p.c + (size_t)m * N + n;
    y[0] = y[0] + v0;
    if (has1) y[1] = y[1] + v1;
  } else if (EPI == EPI_SILU) {
    float* y = p.c + (size_t)m * N + n;
    y[0] = v0 / (1.0f + expf(-v0));
    if (has1) y[1] = v1 / (1.0f + expf(-v1));
  } else if (EPI == EPI_QKV) {
    const int dim = p.dim;
    const int region = n / dim, c = n - region * dim;
    const int seq = m / p.S, t = m - seq * p.S;
    if (region < 2) {
      const int i = (c % p.head_dim) >> 1;
      const float2 cs = p.rope[(size_t)t * (p.head_dim >> 1) + i];
      rope_pair(v0, v1, cs.x, cs.y);
    }
    float* dst;
    if (region == 0)
      dst = p.q_out + (size_t)m * dim + c;
    else
      dst = (region == 1 ? p.kcache : p.vcache) + (size_t)seq * p.seq_stride +
            (size_t)t * dim + c;
    dst[0] = v0;
    dst[1] = v1;
  }
}

// C[M,N] = A[M,K] B[K,N], 128x128 block tile, BK = 16, 4 waves in 2x2,
// each wave a 64x64 sub-tile as 2x2 MFMA 32x32 tiles.  A is staged
// transposed in LDS so MFMA A-operand reads are contiguous; within a wave's
// 64 columns, lane j of N tile t owns column 2j + t so each lane holds
// adjacent column pairs (float2 B reads, paired epilogue for RoPE).
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  constexpr int BM = 128, BN = 128, BK = 16;
  constexpr int APAD = 4;
  __shared__ float As[BK][BM + APAD];
  __shared__ float Bs[BK][BN];

  int M = p.M, N = p.N, K = p.K;
  if (p.meta) {
    M = (int)p.meta->m;
    N = (int)p.meta->n;
    K = (int)p.meta->k;
  }
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  if (m0 >= M || n0 >= N) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  // Global load mapping.  A: 128 rows x 16 k -> thread loads row tid/2,
  // k 8*(tid&1) .. +7 (two float4).  B: 16 rows x 128 cols -> thread loads
  // rows tid/32 and tid/32 + 8, cols 4*(tid&31) .. +3.
  const int a_row = tid >> 1, a_k = (tid & 1) * 8;
  const int b_row = tid >> 5, b_col = (tid & 31) * 4;
  const bool a_vec = (K & 3) == 0;
  const bool b_vec = (N & 3) == 0;

  float ra[8], rb[8];
  auto load_tile = [&](int k0) {
    const int gm = m0 + a_row;
    const float* ap = p.a + (size_t)(gm < M ? gm : 0) * K;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int gk = k0 + a_k + 4 * q;
      if (gm < M && a_vec && gk + 3 < K) {
        const float4 t = *reinterpret_cast<const float4*>(ap + gk);
        ra[4 * q] = t.x; ra[4 * q + 1] = t.y; ra[4 * q + 2] = t.z; ra[4 * q + 3] = t.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ra[4 * q + e] = (gm < M && gk + e < K) ? ap[gk + e] : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int gk = k0 + b_row + 8 * q;
      const int gn = n0 + b_col;
      const float* bp = p.b + (size_t)(gk < K ? gk : 0) * N + gn;
      if (gk < K && b_vec && gn + 3 < N) {
        const float4 t = *reinterpret_cast<const float4*>(bp);
        rb[4 * q] = t.x; rb[4 * q + 1] = t.y; rb[4 * q + 2] = t.z; rb[4 * q + 3] = t.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rb[4 * q + e] = (gk < K && gn + e < N) ? bp[e] : 0.f;
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int e = 0; e < 8; ++e) As[a_k + e][a_row] = ra[e];
#pragma unroll
    for (int q = 0; q < 2; ++q)
      *reinterpret_cast<float4*>(&Bs[b_row + 8 * q][b_col]) =
          make_float4(rb[4 * q], rb[4 * q + 1], rb[4 * q + 2], rb[4 * q + 3]);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[a][t] = zero16();

  const int nk = (K + BK - 1) / BK;
  load_tile(0);
  store_tile();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_tile((kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
      const int kk = 2 * s + h;
      const float a0 = As[kk][wm * 64 + j];
      const float a1 = As[kk][wm * 64 + 32 + j];
      const float2 bb = *reinterpret_cast<const float2*>(&Bs[kk][wn * 64 + 2 * j]);
      acc[0][0] = mfma32(a0, bb.x, acc[0][0]);
      acc[0][1] = mfma32(a0, bb.y, acc[0][1]);
      acc[1][0] = mfma32(a1, bb.x, acc[1][0]);
      acc[1][1] = mfma32(a1, bb.y, acc[1][1]);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      store_tile();
      __syncthreads();
    }
  }

#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wm * 64 + a * 32 + acc_row(r, h);
      const int n = n0 + wn * 64 + 2 * j;
      epi_pair_gemm<EPI>(p, M, N, m, n, acc[a][0][r], acc[a][1][r]);
    }
}

// ===========================================================================
// Prefill: causal flash attention
// ===========================================================================

// MFMA version for head_dim 64.  Block = 4 waves x 32 queries of one
// (sequence, head); keys stream through LDS in blocks of 32.  Each wave
// computes S^T = K Q^T so every lane owns one query (column) and 16 keys,
// making the online-softmax row statistics lane-local (plus one exchange
// between the two half-waves); P^T then feeds O^T += V^T P^T directly from
// the accumulator registers.
__global__ __launch_bounds__(256) void k_flash64(FlashParams p) {
  constexpr int HD = 64, QB = 128, KB = 32;
  __shared__ float Ks[KB][HD + 1];
  __shared__ float Vs[KB][HD];
  __shared__ float Os[4][32][HD + 1];

  int S = p.S, d = p.d;
  float scale = p.scale;
  long roff = 0;
  if (p.meta) {
    S = (int)p.meta->seq_len;
    d = (int)p.meta->dim;
    scale = p.meta->scale;
    roff = (long)p.meta->row_offset * d;
  }
  const int H = d / HD;
  const int qblk = blockIdx.x, hh = blockIdx.y, b = blockIdx.z;
  const int q0 = qblk * QB;
  if (q0 >= S) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  const float* qp = p.q + roff + (size_t)b * p.q_bs + hh * HD;
  const float* kp = p.k + roff + (size_t)b * p.kv_bs + hh * HD;
  const float* vp = p.v + roff + (size_t)b * p.kv_bs + hh * HD;

  // This lane's query row and its 32 dims (half h).
  const int qi = q0 + wave * 32 + j;
  float qreg[32];
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + 32 * h;
#pragma unroll
    for (int s = 0; s < 32; s += 4) {
      const float4 t = *reinterpret_cast<const float4*>(qr + s);
      qreg[s] = t.x; qreg[s + 1] = t.y; qreg[s + 2] = t.z; qreg[s + 3] = t.w;
    }
  }
  f32x16 o0 = zero16(), o1 = zero16();
  float mrow = -INFINITY, lrow = 0.f;

  const int wave_qmax = q0 + wave * 32 + 31;
  const int kend = min(S, q0 + QB);  // keys needed by the block
  const int nkb = (kend + KB - 1) / KB;

  // Cooperative K/V block load: 32 rows x 64 floats each = 512 float4 per
  // tensor; thread t loads rows t/16 and t/16 + 16, float4 column t%16.
  const int lr = tid >> 4, lc = (tid & 15) * 4;
  float4 kr[2], vr[2];
  auto load_kv = [&](int kb) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int key = kb * KB + lr + 16 * q;
      const size_t off = (size_t)(key < S ? key : 0) * d + lc;
      kr[q] = *reinterpret_cast<const float4*>(kp + off);
      vr[q] = *reinterpret_cast<const float4*>(vp + off);
    }
  };
  load_kv(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int r = lr + 16 * q;
      Ks[r][lc] = kr[q].x; Ks[r][lc + 1] = kr[q].y;
      Ks[r][lc + 2] = kr[q].z; Ks[r][lc + 3] = kr[q].w;
      *reinterpret_cast<float4*>(&Vs[r][lc]) = vr[q];
    }
    __syncthreads();
    if (kb + 1 < nkb) load_kv(kb + 1);
    const int j0 = kb * KB;
    if (j0 > wave_qmax) continue;  // block entirely above this wave's rows

    // S^T tile: rows = keys, cols = this wave's queries.
    f32x16 st = zero16();
#pragma unroll
    for (int s = 0; s < 32; ++s) st = mfma32(Ks[j][32 * h + s], qreg[s], st);

    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = j0 + acc_row(r, h);
      float v = st[r] * scale;
      if (key > qi || key >= S) v = -INFINITY;
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float mnew = fmaxf(mrow, pm);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = st[r] == -INFINITY ? 0.f : expf(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = mrow == -INFINITY ? 0.f : expf(mrow - mnew);
    lrow = lrow * corr + ps;
    mrow = mnew;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o0[r] *= corr;
      o1[r] *= corr;
    }
    // O^T += V^T P^T: step s uses key acc_row(s, h) on both operands.
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int key = acc_row(s, h);
      o0 = mfma32(Vs[key][j], st[s], o0);
      o1 = mfma32(Vs[key][32 + j], st[s], o1);
    }
  }

  // O^T (rows = dims) -> LDS -> coalesced row writes.
  const float inv = 1.0f / lrow;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    Os[wave][j][acc_row(r, h)] = o0[r] * inv;
    Os[wave][j][32 + acc_row(r, h)] = o1[r] * inv;
  }
  __syncthreads();
  float* op = p.o + roff + (size_t)b * p.o_bs + hh * HD;
  for (int e = lane; e < 32 * HD; e += 64) {
    const int r = e / HD, c = e % HD;
    const int qrow = q0 + wave * 32 + r;
    if (qrow < S) op[(size_t)qrow * d + c] = Os[wave][r][c];
  }
  if (p.lse && h == 0 && qi < S) p.lse[(size_t)qi * H + hh] = mrow + logf(lrow);
}

// Generic causal flash attention for head_dim HD (any size up to 128):
// one thread per query row with an HD-float accumulator, keys staged
// through LDS in blocks of 64 shared by the block's 64 queries.
template <int HD>
__global__ __launch_bounds__(64) void k_flash_generic(FlashParams p) {
  constexpr int KB = 64;
  __shared__ float Ks[KB][HD];
  __shared__ float Vs[KB][HD];
  int S = p.S, d = p.d;
  float scale = p.scale;
  long roff = 0;
  if (p.meta) {
    S = (int)p.meta->seq_len;
    d = (int)p.meta->dim;
    scale = p.meta->scale;
    roff = (long)p.meta->row_offset * d;
  }
  const int H = d / HD;
  const int hh = blockIdx.y, b = blockIdx.z;
  const int q0 = blockIdx.x * 64;
  if (q0 >= S) return;
  const int i = q0 + threadIdx.x;
  const float* qp = p.q + roff + (size_t)b * p.q_bs + hh * HD;
  const float* kp = p.k + roff + (size_t)b * p.kv_bs + hh * HD;
  const float* vp = p.v + roff + (size_t)b * p.kv_bs + hh * HD;
  float q[HD], acc[HD];
#pragma unroll
  for (int c = 0; c < HD; ++c) {
    q[c] = i < S ? qp[(size_t)i * d + c] : 0.f;
    acc[c] = 0.f;
  }
  float mrow = -INFINITY, lrow = 0.f;
  const int kend = min(S, q0 + 64);
  for (int k0 = 0; k0 < kend; k0 += KB) {
    __syncthreads();
    for (int e = threadIdx.x; e < KB * HD; e += 64) {
      const int r = e / HD, c = e % HD;
      const int key = k0 + r;
      Ks[r][c] = key < S ? kp[(size_t)key * d + c] : 0.f;
      Vs[r][c] = key < S ? vp[(size_t)key * d + c] : 0.f;
    }
    __syncthreads();
    const int lim = min(KB, (i < S ? i : -1) - k0 + 1);
    for (int r = 0; r < lim; ++r) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < HD; ++c) s += q[c] * Ks[r][c];
      s *= scale;
      const float mnew = fmaxf(mrow, s);
      const float corr = mrow == -INFINITY ? 0.f : expf(mrow - mnew);
      const float e = expf(s - mnew);
      lrow = lrow * corr + e;
#pragma unroll
      for (int c = 0; c < HD; ++c) acc[c] = acc[c] * corr + e * Vs[r][c];
      mrow = mnew;
    }
  }
  if (i >= S) return;
  float* op = p.o + roff + (size_t)b * p.o_bs + hh * HD + (size_t)i * d;
#pragma unroll
  for (int c = 0; c < HD; ++c) op[c] = acc[c] / lrow;
  if (p.lse) p.lse[(size_t)i * H + hh] = mrow + logf(lrow);
}

// ===========================================================================
// Host launchers
// ===========================================================================

template <int C, int EPI, bool NORM>
static hipError_t skinny_go(const SkinnyParams& p, int grid_x, hipStream_t s) {
  hipLaunchKernelGGL((k_skinny<C, EPI, NORM>), dim3(grid_x, p.ksplit),
                     dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_skinny(const SkinnyParams& p, int epi, bool norm,
                         int grid_x, hipStream_t s) {
  switch (epi) {
    case EPI_STORE:
      return norm ? skinny_go<1, EPI_STORE, true>(p, grid_x, s)
                  : skinny_go<1, EPI_STORE, false>(p, grid_x, s);
    case EPI_ADD:
      return skinny_go<1, EPI_ADD, false>(p, grid_x, s);
    case EPI_SILU:
      return norm ? skinny_go<1, EPI_SILU, true>(p, grid_x, s)
                  : skinny_go<1, EPI_SILU, false>(p, grid_x, s);
    case EPI_QKV:
      return norm ? skinny_go<1, EPI_QKV, true>(p, grid_x, s)
                  : skinny_go<1, EPI_QKV, false>(p, grid_x, s);
    case EPI_LOGITS:
      return norm ? skinny_go<1, EPI_LOGITS, true>(p, grid_x, s)
                  : skinny_go<1, EPI_LOGITS, false>(p, grid_x, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(const GemmParams& p, int epi, int grid_x, int grid_y,
                       hipStream_t s) {
  dim3 g(grid_x, grid_y), b(256);
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL(k_gemm<EPI_STORE>, g, b, 0, s, p); break;
    case EPI_ADD: hipLaunchKernelGGL(k_gemm<EPI_ADD>, g, b, 0, s, p); break;
    case EPI_SILU: hipLaunchKernelGGL(k_gemm<EPI_SILU>, g, b, 0, s, p); break;
    case EPI_QKV: hipLaunchKernelGGL(k_gemm<EPI_QKV>, g, b, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_flash(const FlashParams& p, int batch, int max_rows,
                        hipStream_t s) {
  const int H = p.d / p.hd;
  if (p.hd == 64) {
    hipLaunchKernelGGL(k_flash64, dim3((max_rows + 127) / 128, H, batch),
                       dim3(256), 0, s, p);
    return hipGetLastError();
  }
  dim3 g((max_rows + 63) / 64, H, batch), b(64);
  switch (p.hd) {
    case 2: hipLaunchKernelGGL(k_flash_generic<2>, g, b, 0, s, p); break;
    case 4: hipLaunchKernelGGL(k_flash_generic<4>, g, b, 0, s, p); break;
    case 8: hipLaunchKernelGGL(k_flash_generic<8>, g, b, 0, s, p); break;
    case 16: hipLaunchKernelGGL(k_flash_generic<16>, g, b, 0, s, p); break;
    case 32: hipLaunchKernelGGL(k_flash_generic<32>, g, b, 0, s, p); break;
    case 128: hipLaunchKernelGGL(k_flash_generic<128>, g, b, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode_attn(const DecodeAttnParams& p, int hd,
                              hipStream_t s) {
  dim3 g(p.B * p.H, p.nsplit), b(256);
  switch (hd) {
    case 4: hipLaunchKernelGGL(k_decode_attn<4>, g, b, 0, s, p); break;
    case 8: hipLaunchKernelGGL(k_decode_attn<8>, g, b, 0, s, p); break;
    case 16: hipLaunchKernelGGL(k_decode_attn<16>, g, b, 0, s, p); break;
    case 32: hipLaunchKernelGGL(k_decode_attn<32>, g, b, 0, s, p); break;
    case 64: hipLaunchKernelGGL(k_decode_attn<64>, g, b, 0, s, p); break;
    case 128: hipLaunchKernelGGL(k_decode_attn<128>, g, b, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gather_rows(const float* table, const uint32_t* ids,
                              uint32_t vocab, const float* src, long src_row0,
                              long src_row_stride, float* dst, int M, int d,
                              float* ss, hipStream_t s) {
  hipLaunchKernelGGL(k_gather_rows, dim3(M), dim3(256), 0, s, table, ids,
                     vocab, src, src_row0, src_row_stride, dst, d, ss);
  return hipGetLastError();
}

hipError_t launch_argmax_final(const uint2* part, int ntiles, int M,
                               uint32_t* tok, int* pos, uint32_t* hist,
                               int hist_stride, int next_pos, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_final, dim3(M), dim3(256), 0, s, part, ntiles,
                     tok, pos, hist, hist_stride, next_pos);
  return hipGetLastError();
}

hipError_t launch_rows_rmsnorm(const float* x, const float* w, float* out,
                               int rows, int size, float eps, hipStream_t s) {
  hipLaunchKernelGGL(k_rows_rmsnorm, dim3(rows), dim3(256), 0, s, x, w, out,
                     size, eps);
  return hipGetLastError();
}

hipError_t launch_embedding_rows(const uint32_t* tokens, const float* table,
                                 float* out, int rows, int d, uint32_t vocab,
                                 hipStream_t s) {
  hipLaunchKernelGGL(k_embedding_rows, dim3(rows), dim3(256), 0, s, tokens,
                     table, out, d, vocab);
  return hipGetLastError();
}

static unsigned grid1d(size_t n, unsigned block) {
  size_t g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > 65535u * 16u) g = 65535u * 16u;
  return (unsigned)g;
}

hipError_t shader_embedding(const uint32_t* tokens, const float* table,
                            float* out, akh_embedding_meta shape,
                            const akh_embedding_meta* meta, hipStream_t s) {
  if (shape.seq_len == 0) return hipSuccess;
  hipLaunchKernelGGL(k_embedding, dim3((shape.dim + 255) / 256, shape.seq_len),
                     dim3(256), 0, s, tokens, table, out, meta);
  return hipGetLastError();
}

hipError_t shader_rmsnorm(const float* x, const float* w, float* out,
                          akh_norm_meta shape, const akh_norm_meta* meta,
                          hipStream_t s) {
  if (shape.seq_len == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rmsnorm, dim3(shape.seq_len), dim3(256), 0, s, x, w,
                     out, meta);
  return hipGetLastError();
}

hipError_t shader_head_gather(const float* src, float* dst,
                              akh_head_move_meta shape,
                              const akh_head_move_meta* meta, hipStream_t s) {
  hipLaunchKernelGGL(k_head_gather,
                     dim3(grid1d((size_t)shape.seq_len * shape.head_dim, 256)),
                     dim3(256), 0, s, src, dst, meta);
  return hipGetLastError();
}

hipError_t shader_rope(float* buf, uint32_t seq_len, uint32_t dim,
                       const uint32_t* meta_u32, int with_offset,
                       hipStream_t s) {
  hipLaunchKernelGGL(k_rope, dim3(grid1d((size_t)seq_len * (dim / 2), 256)),
                     dim3(256), 0, s, buf, meta_u32, with_offset);
  return hipGetLastError();
}

hipError_t shader_cache_write(const float* src, float* cache,
                              akh_cache_write_meta shape,
                              const akh_cache_write_meta* meta,
                              hipStream_t s) {
  hipLaunchKernelGGL(k_cache_write,
                     dim3(grid1d((size_t)shape.row_count * shape.width, 256)),
                     dim3(256), 0, s, src, cache, meta);
  return hipGetLastError();
}

hipError_t shader_attn_qk_cached(const float* q, const float* kc,
                                 float* scores, uint32_t num_heads,
                                 uint32_t max_attn_len,
                                 const akh_attn_cached_meta* meta,
                                 hipStream_t s) {
  hipLaunchKernelGGL(k_attn_qk_cached,
                     dim3((max_attn_len + 255) / 256, num_heads), dim3(256), 0,
                     s, q, kc, scores, meta);
  return hipGetLastError();
}

hipError_t shader_softmax_rect(float* x, akh_softmax_rect_meta shape,
                               const akh_softmax_rect_meta* meta,
                               hipStream_t s) {
  if (shape.num_rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_softmax_rect, dim3(shape.num_rows), dim3(256), 0, s, x,
                     meta);
  return hipGetLastError();
}

hipError_t shader_attn_av_cached(const float* scores, const float* vc,
                                 float* out, uint32_t dim,
                                 const akh_attn_cached_meta* meta,
                                 hipStream_t s) {
  hipLaunchKernelGGL(k_attn_av_cached, dim3((dim + 255) / 256), dim3(256), 0,
                     s, scores, vc, out, meta);
  return hipGetLastError();
}

hipError_t shader_silu(float* buf, uint32_t len, hipStream_t s) {
  if (len == 0) return hipSuccess;
  hipLaunchKernelGGL(k_silu, dim3(grid1d(len, 256)), dim3(256), 0, s, buf,
                     len);
  return hipGetLastError();
}

hipError_t shader_argmax_rows(const float* logits, uint32_t rows, uint32_t n,
                              uint32_t* out, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_argmax_rows, dim3(rows), dim3(256), 0, s, logits, n,
                     out);
  return hipGetLastError();
}

}  // namespace akh
