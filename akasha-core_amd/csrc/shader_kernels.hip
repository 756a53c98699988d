// Per-shader kernels: one per reference Shader / matmul builtin on the
// inference path (src/shaders/mod.rs), with the reference's semantics and
// the meta read from device memory when the kernel runs, so a captured graph
// follows metas rewritten between replays.  The launch is sized from the
// build-time shape and the live meta bounds the work, as in the reference
// (ARCHITECTURE.md "live metas").
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace akh {

namespace {

unsigned grid1d(size_t n, unsigned block) {
  size_t g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > 65535u * 16u) g = 65535u * 16u;
  return (unsigned)g;
}

}  // namespace

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

// RMSNORM (src/shaders/cpu.rs:205-222), one 256-thread block per row:
// y = x * (1 / sqrt(sum(x^2) / size + eps)) * w.  Rows of up to 1024 are held
// in registers, their x and w loaded together; each thread sums its columns
// c, c + 256, ... in that order either way.
__global__ __launch_bounds__(256) void k_rmsnorm(const float* x,
                                                 const float* w, float* out,
                                                 const akh_norm_meta* meta) {
  constexpr uint32_t U = 4;
  __shared__ float red4[4];
  const uint32_t r = blockIdx.x;
  if (r >= meta->seq_len) return;
  const uint32_t size = meta->size;
  const float* xr = x + (size_t)r * size;
  float* yr = out + (size_t)r * size;
  if (size <= 256 * U) {
    float xv[U], wv[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t c = threadIdx.x + 256 * u;
      xv[u] = c < size ? xr[c] : 0.f;
      wv[u] = c < size ? w[c] : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) ss += xv[u] * xv[u];
    ss = block_sum256(ss, red4);
    const float rs = 1.0f / sqrtf(ss / (float)size + meta->eps);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t c = threadIdx.x + 256 * u;
      if (c < size) yr[c] = __fmul_rn(__fmul_rn(xv[u], rs), wv[u]);
    }
    return;
  }
  float ss = 0.f;
  for (uint32_t c = threadIdx.x; c < size; c += 256) ss += xr[c] * xr[c];
  ss = block_sum256(ss, red4);
  const float rs = 1.0f / sqrtf(ss / (float)size + meta->eps);
  for (uint32_t c = threadIdx.x; c < size; c += 256)
    yr[c] = __fmul_rn(__fmul_rn(xr[c], rs), w[c]);
}

// MATMUL / GEMV and MATMUL_ADD / GEMV_ADD for m <= 32 (the reference routes
// m == 1 to GEMV, emit.rs:31-33): C[m, n] (+)= A[m, k] B[k, n].
//
// B streams once over the whole part.  A block takes a slab of 4 CG columns
// and one of `splits` ranges of `kchunk` rows of B.  With 16-byte rows
// (CG = 8), thread t reads row t / 8 of each 32-row round and columns
// 4 (t % 8) .. + 3 of it with one 16-byte load, so a wave's load is 1 KB of
// eight rows; other rows take lane-adjacent columns (LC: t % CG + CG c), so
// a load instruction reads whole runs of a row.  GR rounds are in flight;
// a thread keeps the sums of up to MR rows of A.  The row lanes of each
// column meet through lane exchanges and LDS.  With one split
// the block writes C.  Otherwise it writes its partial sums to the
// workspace (through to device scope), waits for them to complete and counts
// itself; the last block of the slab adds the partials in split order (the
// same sums whichever block arrives last) and writes C.  Few splits per slab
// (their counts meet at one address), many slabs.  The grid and the splits
// come from the recorded shape; M, N and K from the meta (at most the
// recorded ones).
constexpr int kGemvMaxSplits = 8;

struct GemvParams {
  const float* a;
  const float* b;
  float* c;
  const akh_matmul_meta* meta;
  int accumulate;
  int mrec, nrec;  // the recorded shape: the workspace's layout
  int krec;        // the recorded K: a live K is clamped to it
  int splits, kchunk;
  float* ws;
  int* cnt;
  int vec;  // B 16-byte aligned and the recorded N a multiple of 4
};

template <int MR, int CG, bool LC, int NTB = 256>
__global__ __launch_bounds__(NTB) void k_shader_gemv(GemvParams g) {
#ifndef AKH_GEMV_GR
#define AKH_GEMV_GR 4
#endif
  constexpr int NWB = NTB / 64;  // waves of the block
  constexpr int SW = 4 * CG;     // slab columns
  constexpr int RL = NTB / CG;   // row lanes of the block
  constexpr int GR = NTB > 256 ? 6 : MR > 4 ? 2 : AKH_GEMV_GR;  // rounds of RL rows in flight
  __shared__ float red[NWB][MR][SW];
  __shared__ int last_block;
  const int M = min((int)g.meta->m, min(g.mrec, MR)), N = min((int)g.meta->n, g.nrec);
  const int K = min((int)g.meta->k, g.krec);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * SW;
  if (n0 >= N || M <= 0) return;  // the whole slab: no block of it counts
  // Thread columns: four adjacent ones (one 16-byte load), or with LC the
  // columns n0 + t % CG + CG c, so a load instruction's lanes read adjacent
  // words of a row (rows whose 16-byte pieces straddle cache lines).
  const int rl = tid / CG, nc = LC ? n0 + tid % CG : n0 + 4 * (tid % CG);
  constexpr int CS = LC ? CG : 1;  // column step between a thread's columns
  const int k0 = min(K, blockIdx.y * g.kchunk), k1 = min(K, k0 + g.kchunk);
  const bool vec = !LC && g.vec && N % 4 == 0;
  float acc[MR][4];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.f;
  for (int kg = k0 + rl; kg < k1; kg += RL * GR) {
    float w[GR][4];
#pragma unroll
    for (int u = 0; u < GR; ++u) {
      const int k = kg + RL * u;
      const bool ok = k < k1 && nc < N;
      const float* src = g.b + (size_t)(ok ? k : 0) * N + (ok ? nc : 0);
      if (vec) {
        const float4 t = ok ? *reinterpret_cast<const float4*>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
        w[u][0] = t.x;
        w[u][1] = t.y;
        w[u][2] = t.z;
        w[u][3] = t.w;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) w[u][c] = ok && nc + CS * c < N ? src[CS * c] : 0.f;
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) continue;
      const float* ar = g.a + (size_t)m * K;
#pragma unroll
      for (int u = 0; u < GR; ++u) {
        const int k = kg + RL * u;
        const float x = k < k1 ? ar[k] : 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(x, w[u][c], acc[m][c]);
      }
    }
  }
  // Rows: the wave's row lanes of each column (lanes CG, 2 CG, ... apart),
  // then the four waves through LDS.  Thread t < SW then holds column n0 + t.
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float v = acc[m][c];
#pragma unroll
      for (int o = CG; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
      acc[m][c] = v;
    }
  if (lane < CG)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave][m][LC ? lane + CG * c : 4 * lane + c] = acc[m][c];
  __syncthreads();
  const int n = n0 + tid;
  const bool col = tid < SW && n < N;
  float tot[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int t = tid % SW;
    float v = red[0][m][t];
#pragma unroll
    for (int q = 1; q < NWB; ++q) v += red[q][m][t];
    tot[m] = v;
  }
  if (g.splits == 1) {
    if (col)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) {
          float* y = g.c + (size_t)m * N + n;
          *y = g.accumulate ? *y + tot[m] : tot[m];
        }
    return;
  }
  const size_t plane = (size_t)g.mrec * g.nrec;
  if (col)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M)
        __hip_atomic_store(g.ws + blockIdx.y * plane + (size_t)m * g.nrec + n, tot[m],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const int done =
        __hip_atomic_fetch_add(g.cnt + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_block = done == g.splits - 1;
    if (last_block)  // zero for the next launch
      __hip_atomic_store(g.cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last_block || !col) return;
  // At most kGemvMaxSplits partials per value, all loads in flight at once.
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= M) continue;
    const float* q = g.ws + (size_t)m * g.nrec + n;
    float t[kGemvMaxSplits];
#pragma unroll
    for (int sp = 0; sp < kGemvMaxSplits; ++sp)
      t[sp] = sp < g.splits ? __hip_atomic_load(q + sp * plane, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0.f;
    float sum = 0.f;
#pragma unroll
    for (int sp = 0; sp < kGemvMaxSplits; ++sp) sum += t[sp];
    float* y = g.c + (size_t)m * N + n;
    *y = g.accumulate ? *y + sum : sum;
  }
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
// (2i, 2i+1) of each head rotated by pos * 10000^(-2i/head_dim), position =
// row (+ meta pos for ROPE_OFFSET).
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

// ATTN_QK_CACHED (src/shaders/cpu.rs:144-162): scores[h][j] = q_h . K[j]_h
// for j < attn_len.  Sixteen lanes per (row, head): lane l takes columns
// l, l + 16, ... of the head, up to eight of them loaded before any is
// summed (one memory round trip per 128 columns), and the sixteen partial
// sums meet by lane exchanges.  A block of 256 threads takes 16 rows.
__global__ __launch_bounds__(256) void k_attn_qk_cached(const float* q, const float* kc,
                                                        float* scores,
                                                        const akh_attn_cached_meta* meta) {
  const uint32_t len = meta->attn_len, dim = meta->dim, hd = meta->head_dim;
  const uint32_t sub = threadIdx.x & 15;
  const uint32_t j = blockIdx.x * 16 + (threadIdx.x >> 4), h = blockIdx.y;
  if (blockIdx.x * 16 >= len || h >= dim / hd) return;  // whole block
  const bool live = j < len;
  const float* qh = q + h * hd;
  const float* kr = kc + (size_t)(live ? j : 0) * dim + h * hd;
  float s = 0.f;
  for (uint32_t c0 = 0; c0 < hd; c0 += 128) {
    float kv[8], qv[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
      const uint32_t c = c0 + sub + 16 * u;
      const bool ok = live && c < hd;
      kv[u] = ok ? kr[c] : 0.f;
      qv[u] = ok ? qh[c] : 0.f;
    }
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) s = fmaf(qv[u], kv[u], s);
  }
  s += __shfl_xor(s, 8, 64);
  s += __shfl_xor(s, 4, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 1, 64);
  if (live && sub == 0) scores[(size_t)h * len + j] = s;
}

// SOFTMAX_RECT (src/shaders/cpu.rs:180-203), one block per row; rows of up
// to 1024 stay in registers between the passes.
__global__ __launch_bounds__(256) void k_softmax_rect(
    float* x, const akh_softmax_rect_meta* meta) {
  constexpr uint32_t U = 4;
  __shared__ float red4[4];
  const uint32_t r = blockIdx.x;
  if (r >= meta->num_rows) return;
  const uint32_t width = meta->width;
  const float scale = meta->scale;
  float* row = x + (size_t)r * width;
  if (width <= 256 * U) {
    float v[U];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + 256 * u;
      v[u] = i < width ? row[i] * scale : -INFINITY;
      mx = fmaxf(mx, v[u]);
    }
    mx = block_max256(mx, red4);
    float sum = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + 256 * u;
      v[u] = i < width ? expf(v[u] - mx) : 0.f;
      sum += v[u];
    }
    sum = block_sum256(sum, red4);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = threadIdx.x + 256 * u;
      if (i < width) row[i] = v[u] / sum;
    }
    return;
  }
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

// ATTN_AV_CACHED (src/shaders/cpu.rs:164-178): out[d] = sum_j p[h(d)][j] V[j][d].
// A block of 512 threads takes 64 channels: wave w sums rows w, w + 8, ...
// with 16 rows' loads in flight per lane (one memory round trip per 128
// rows), and the eight waves' sums meet in LDS in wave order.
__global__ __launch_bounds__(512) void k_attn_av_cached(const float* p, const float* vc,
                                                        float* out,
                                                        const akh_attn_cached_meta* meta) {
  constexpr uint32_t W = 8, U = 16;
  __shared__ float part[W][64];
  const uint32_t len = meta->attn_len, dim = meta->dim, hd = meta->head_dim;
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t d = blockIdx.x * 64 + lane;
  const bool live = d < dim;
  const float* ph = p + (size_t)(live ? d / hd : 0) * len;
  const float* vd = vc + (live ? d : 0);
  float s = 0.f;
  for (uint32_t j0 = w; j0 < len; j0 += W * U) {
    float pv[U], vv[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t j = j0 + W * u;
      const bool ok = live && j < len;
      pv[u] = ok ? ph[j] : 0.f;
      vv[u] = ok ? vd[(size_t)j * dim] : 0.f;
    }
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) s = fmaf(pv[u], vv[u], s);
  }
  part[w][lane] = s;
  __syncthreads();
  if (w == 0 && live) {
    float t = part[0][lane];
#pragma unroll
    for (uint32_t i = 1; i < W; ++i) t += part[i][lane];
    out[d] = t;
  }
}

// SILU (src/shaders/cpu.rs:63-69).
__global__ void k_silu(float* x, uint32_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float v = x[i];
    x[i] = v / (1.0f + expf(-v));
  }
}

// Greedy argmax of each row (sampling.rs:83-91).
__global__ __launch_bounds__(256) void k_argmax_rows(const float* logits,
                                                     uint32_t n,
                                                     uint32_t* out) {
  const float* row = logits + (size_t)blockIdx.x * n;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = threadIdx.x; i < n; i += 256) amax_merge(bv, bi, row[i], i);
  block_amax256(bv, bi);
  // The reference's scan (sampling.rs:83-91) starts from index 0; a NaN
  // there never loses a comparison, so it stays the answer.
  if (threadIdx.x == 0) out[blockIdx.x] = bi == 0xFFFFFFFFu || __builtin_isnan(row[0]) ? 0u : bi;
}

// ---------------------------------------------------------------------------

hipError_t shader_embedding(const uint32_t* tokens, const float* table,
                            float* out, akh_embedding_meta shape,
                            const akh_embedding_meta* meta, hipStream_t s) {
  if (shape.seq_len == 0 || shape.dim == 0) return hipSuccess;
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

hipError_t shader_matmul(const float* a, const float* b, float* c,
                         akh_matmul_meta shape, const akh_matmul_meta* meta,
                         int accumulate, float* ws, int* cnt, hipStream_t s) {
  if (shape.m == 0 || shape.n == 0) return hipSuccess;
  if (shape.m <= 32u) {
    // Column slabs over at most 8 ranges of K (at least 128 rows each),
    // about 256 blocks where the slabs are fewer.
#ifndef AKH_GEMV_TARGET
#define AKH_GEMV_TARGET 256
#endif
#ifndef AKH_GEMV_SMAX
#define AKH_GEMV_SMAX kGemvMaxSplits
#endif
#ifndef AKH_GEMV_KMIN
#define AKH_GEMV_KMIN 128
#endif
    GemvParams g{a, b, c, meta, accumulate, (int)shape.m, (int)shape.n, (int)shape.k,
                 1, 1, ws, cnt, 0};
    g.vec = shape.n % 4 == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0;
    // Rows that are not whole 16-byte pieces take lane-adjacent columns, for
    // m <= 4 in the widest slabs (up to 256 columns) that still number 128:
    // measured at m = 1, K = 768, N = 50257 took 47.7 us on 32-column slabs
    // of four adjacent columns per lane and 29.1 us on 256-column ones, and
    // N = 771 9.4 us at 256 columns, 5.8 us at 64.
    int cg = 8;
    if (!g.vec && shape.m <= 4u) {
      cg = 64;
      while (cg > 16 && (shape.n + 4 * cg - 1) / (4 * cg) < 128) cg /= 2;
    }
    const int slabs = (int)((shape.n + 4 * cg - 1) / (4 * cg)), K = (int)shape.k;
    int splits = std::min(AKH_GEMV_SMAX, std::max(1, (AKH_GEMV_TARGET + slabs - 1) / slabs));
    splits = std::min(splits, std::max(1, K / AKH_GEMV_KMIN));
    if (!ws || !cnt || slabs > kGemvSlabs) splits = 1;
    const size_t plane = (size_t)shape.m * shape.n;
    if ((size_t)splits * plane > kGemvWsFloats) splits = (int)std::max<size_t>(1, kGemvWsFloats / plane);
    g.kchunk = std::max(1, (K + splits - 1) / splits);
    g.splits = std::max(1, (K + g.kchunk - 1) / g.kchunk);
    const dim3 grid(slabs, g.splits);
#define AKH_GEMV_GO(MR, CG, LC) \
  hipLaunchKernelGGL((k_shader_gemv<MR, CG, LC>), grid, dim3(256), 0, s, g)
    // m = 1 on 16-byte rows: 1024-thread blocks, each over one range of at
    // most 768 rows of K (a single round of 6 x 128 rows in flight); one range
    // needs no partial sums, more are added by the slab's last block.
    // Measured at m = 1 against 256-thread blocks over up to 8 ranges:
    // K = 768: N = 2304 7.1 -> 5.1 us, 768 5.2 -> 4.3, 3072 7.2 -> 5.2;
    // K = 3072, N = 768 (four ranges) 9.5 -> 6.9 us.
    const int wranges = ((int)shape.k + 767) / 768;
    if (g.vec && shape.m == 1 && shape.k > 0 &&
        (wranges == 1 || (ws && cnt && slabs <= kGemvSlabs && wranges <= kGemvMaxSplits &&
                          (size_t)wranges * shape.n <= kGemvWsFloats))) {
      g.splits = wranges;
      g.kchunk = wranges == 1 ? (int)shape.k : 768;
      hipLaunchKernelGGL((k_shader_gemv<1, 8, false, 1024>), dim3(slabs, wranges), dim3(1024), 0, s, g);
    } else if (g.vec) {
      if (shape.m == 1) AKH_GEMV_GO(1, 8, false);
      else if (shape.m <= 4) AKH_GEMV_GO(4, 8, false);
      else AKH_GEMV_GO(32, 8, false);
    } else if (shape.m > 4) {
      AKH_GEMV_GO(32, 8, true);
    } else if (cg == 8) {
      if (shape.m == 1) AKH_GEMV_GO(1, 8, true); else AKH_GEMV_GO(4, 8, true);
    } else if (cg == 16) {
      if (shape.m == 1) AKH_GEMV_GO(1, 16, true); else AKH_GEMV_GO(4, 16, true);
    } else if (cg == 32) {
      if (shape.m == 1) AKH_GEMV_GO(1, 32, true); else AKH_GEMV_GO(4, 32, true);
    } else {
      if (shape.m == 1) AKH_GEMV_GO(1, 64, true); else AKH_GEMV_GO(4, 64, true);
    }
#undef AKH_GEMV_GO
    return hipGetLastError();
  }
  GemmParams p{};
  p.a = a;
  p.b = b;
  p.c = c;
  p.M = shape.m;
  p.N = shape.n;
  p.K = shape.k;
  p.meta = meta;
  p.split_ws = ws;  // prompt-sized m: K split where the tiles are few
  p.split_cnt = cnt;
  return launch_gemm(p, accumulate ? GEMM_ADD : GEMM_STORE, s);
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

hipError_t shader_flash_attention(const float* q, const float* k,
                                  const float* v, float* out, float* lse,
                                  akh_flash_attn_meta shape,
                                  const akh_flash_attn_meta* meta,
                                  uint32_t batch, hipStream_t s) {
  if (shape.seq_len == 0 || batch == 0) return hipSuccess;
  FlashParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = out;
  p.lse = lse;
  p.S = shape.seq_len;
  p.d = shape.dim;
  p.hd = shape.head_dim;
  p.scale = shape.scale;
  p.meta = meta;
  // Sequence b is the node at row_offset + b * seq_len.
  p.q_bs = p.kv_bs = p.o_bs = (long)shape.seq_len * shape.dim;
  p.lse_bs = (long)shape.seq_len * (shape.dim / shape.head_dim);
  // head_dim 64 / 128: fp32 accuracy on split MFMAs, no flag to read back.
  p.x6 = FLASH_FP32;
  return launch_flash(p, (int)batch, shape.seq_len, s);
}

hipError_t shader_attn_qk_cached(const float* q, const float* kc,
                                 float* scores, uint32_t num_heads,
                                 uint32_t max_attn_len,
                                 const akh_attn_cached_meta* meta,
                                 hipStream_t s) {
  if (max_attn_len == 0 || num_heads == 0) return hipSuccess;
  hipLaunchKernelGGL(k_attn_qk_cached,
                     dim3((max_attn_len + 15) / 16, num_heads), dim3(256), 0,
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
  if (dim == 0) return hipSuccess;
  hipLaunchKernelGGL(k_attn_av_cached, dim3((dim + 63) / 64), dim3(512), 0,
                     s, scores, vc, out, meta);
  return hipGetLastError();
}

// ---- the trainer's forward shaders (src/nn/train.rs:256-275) -------------

// QKV_SPLIT (src/shaders/mod.rs:376-395, CUDA twin cuda.rs:296-318): the
// three head_dim-wide column slices of each src row.
__global__ void k_qkv_split(const float* src, float* q, float* k, float* v,
                            const akh_head_move_meta* meta) {
  const uint32_t rows = meta->seq_len, full = meta->full_dim, w = meta->head_dim;
  const size_t n = (size_t)rows * w;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t row = i / w, col = i % w;
    const float* r = src + row * full;
    q[i] = r[col];
    k[i] = r[w + col];
    v[i] = r[2 * w + col];
  }
}

// ROPE_QK (src/shaders/mod.rs:139-158, CUDA twin cuda.rs:152-185): RoPE on
// rows row_offset + t of q and k at local position t (cpu.rs:98-103 angle).
__global__ void k_rope_qk(float* q, float* k, const akh_rope_meta* meta) {
  const uint32_t rows = meta->seq_len, dim = meta->dim, hd = meta->head_dim;
  const size_t base = (size_t)meta->row_offset * dim;
  const size_t pairs = (size_t)rows * (dim / 2);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t t = (uint32_t)(i / (dim / 2));
    const uint32_t c = (uint32_t)(i % (dim / 2)) * 2u;
    const float freq = 1.0f / powf(10000.0f, (float)(c % hd) / (float)hd);
    float sn, cs;
    sincosf((float)t * freq, &sn, &cs);
    const size_t o = base + (size_t)t * dim + c;
    float a0 = q[o], a1 = q[o + 1];
    rope_pair(a0, a1, cs, sn);
    q[o] = a0;
    q[o + 1] = a1;
    float b0 = k[o], b1 = k[o + 1];
    rope_pair(b0, b1, cs, sn);
    k[o] = b0;
    k[o + 1] = b1;
  }
}

// ADD (cpu.rs:77-82) with sub == 0: out = a + b; the RESIDUAL_ADD builtin
// (emit.rs:733-748) is the same kernel with out == a.
__global__ void k_add(const float* a, const float* b, float* out, uint32_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = a[i] + b[i];
}

// SILU_OUT (cpu.rs:71-75).
__global__ void k_silu_out(const float* x, float* out, uint32_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = x[i] / (1.0f + expf(-x[i]));
}

// Reductions over a 1024-thread block in a fixed order.
__device__ __forceinline__ float block_red1024(float v, float* red, bool is_max) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < 16; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

// CROSS_ENTROPY (cpu.rs:277-306), one 1024-thread block per row, in place:
// m = row max, s = sum of e^(x - m), loss = -(x[target] - m - ln s), and the
// row becomes e^(x - m) / s.  A target id >= vocab has no logit; its loss is
// NaN (the reference indexes out of bounds there).  The first 1024 * kCeRegs
// entries of the row stay in registers between the passes (one read and one
// write of the row for vocabularies up to 65536); entries past them are
// re-read.  They move through a buffer resource over the row: one
// per-lane offset and a scalar offset per entry instead of a 64-bit address
// each, and reads past the row return zero.  Each thread folds its entries
// in index order either way, so the results do not depend on where an entry
// was held.
constexpr int kCeRegs = 64;
__global__ __launch_bounds__(1024) void k_cross_entropy(float* x, const uint32_t* targets,
                                                        float* losses,
                                                        const akh_cross_entropy_meta* meta) {
  __shared__ float red[16];
  const uint32_t V = meta->vocab_size, row = blockIdx.x;
  if (row >= meta->num_rows) return;
  float* r = x + (size_t)row * V;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(r, (short)0, (int)(V * 4u), 0x00020000);
  const uint32_t tid = threadIdx.x, held = 1024u * kCeRegs;
  const int vo = (int)(tid * 4u);
  float v[kCeRegs];
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < kCeRegs; ++e) {
    const float t = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, vo, e * 4096, 0));
    v[e] = tid + 1024u * e < V ? t : -INFINITY;
    m = fmaxf(m, v[e]);
  }
  for (uint32_t i = held + tid; i < V; i += 1024) m = fmaxf(m, r[i]);
  m = block_red1024(m, red, true);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < kCeRegs; ++e) {
    v[e] = expf(v[e] - m);  // 0 past the end of the row
    sum += v[e];
  }
  for (uint32_t i = held + tid; i < V; i += 1024) sum += expf(r[i] - m);
  sum = block_red1024(sum, red, false);
  if (tid == 0) {
    const uint32_t t = targets[row];
    losses[row] = t < V ? -(r[t] - m - logf(sum)) : __builtin_nanf("");
  }
  __syncthreads();  // the target's logit is read before the row is rewritten
  // Stores past the end of the row are dropped by the resource's range.
#pragma unroll
  for (int e = 0; e < kCeRegs; ++e)
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[e] / sum), rs, vo, e * 4096, 0);
  for (uint32_t i = held + tid; i < V; i += 1024) r[i] = expf(r[i] - m) / sum;
}

hipError_t shader_qkv_split(const float* src, float* q, float* k, float* v,
                            akh_head_move_meta shape, const akh_head_move_meta* meta,
                            hipStream_t s) {
  const size_t n = (size_t)shape.seq_len * shape.head_dim;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_qkv_split, dim3(grid1d(n, 256)), dim3(256), 0, s, src, q, k, v, meta);
  return hipGetLastError();
}

hipError_t shader_rope_qk(float* q, float* k, akh_rope_meta shape, const akh_rope_meta* meta,
                          hipStream_t s) {
  const size_t n = (size_t)shape.seq_len * (shape.dim / 2);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rope_qk, dim3(grid1d(n, 256)), dim3(256), 0, s, q, k, meta);
  return hipGetLastError();
}

hipError_t shader_add(const float* a, const float* b, float* out, uint32_t len, hipStream_t s) {
  if (len == 0) return hipSuccess;
  hipLaunchKernelGGL(k_add, dim3(grid1d(len, 256)), dim3(256), 0, s, a, b, out, len);
  return hipGetLastError();
}

hipError_t shader_silu_out(const float* x, float* out, uint32_t len, hipStream_t s) {
  if (len == 0) return hipSuccess;
  hipLaunchKernelGGL(k_silu_out, dim3(grid1d(len, 256)), dim3(256), 0, s, x, out, len);
  return hipGetLastError();
}

hipError_t launch_cross_entropy(float* logits, const uint32_t* targets, float* losses,
                                uint32_t rows, const akh_cross_entropy_meta* meta,
                                hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_cross_entropy, dim3(rows), dim3(1024), 0, s, logits, targets, losses,
                     meta);
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
