// Prefill kernels: the LDS-tiled fp32 MFMA GEMM (every prefill matmul and
// the per-shader MATMUL for m > 32), causal flash attention, row RMSNorm and
// the embedding gather.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace akh {

// Host-sized embedding gather for the batched prefill (cpu.rs:25-41).
__global__ void k_embedding_rows(const uint32_t* tokens, const float* table,
                                 float* out, int d, uint32_t vocab) {
  const int t = blockIdx.x;
  const uint32_t id = tokens[t];
  if (d % 4 != 0) {  // rows without 16-byte alignment: element by element
    for (int c = threadIdx.x; c < d; c += blockDim.x)
      out[(size_t)t * d + c] = id < vocab ? table[(size_t)id * d + c] : 0.f;
    return;
  }
  const float4* src = reinterpret_cast<const float4*>(table + (size_t)id * d);
  float4* dst = reinterpret_cast<float4*>(out + (size_t)t * d);
  for (int c = threadIdx.x; c < d / 4; c += blockDim.x)
    dst[c] = id < vocab ? src[c] : make_float4(0.f, 0.f, 0.f, 0.f);
}

// RMSNorm of every row (cpu.rs:205-222), one 256-thread block per row.
// Rows of up to 4096 floats (a multiple of 4): one wave per row, four rows
// per block, the row held in registers between the sum of squares (a wave
// butterfly, no LDS or barrier) and the scaling, read and written 16 bytes
// at a time.  Other sizes: one block per row, element by element.
template <int QL>  // float4 per lane: size <= 256 QL
__global__ __launch_bounds__(256) void k_rows_rmsnorm(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ out, int rows,
                                                      int size, float eps) {
  if (QL > 0) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * size);
    float4* o = reinterpret_cast<float4*>(out + (size_t)row * size);
    const float4* g4 = reinterpret_cast<const float4*>(w);
    const int nq = size >> 2;
    float4 v[QL > 0 ? QL : 1], g[QL > 0 ? QL : 1];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < QL; ++i) {
      const int q = lane + 64 * i;
      v[i] = q < nq ? xr[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      g[i] = q < nq ? g4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    ss = wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / (float)size + eps);
#pragma unroll
    for (int i = 0; i < QL; ++i) {
      const int q = lane + 64 * i;
      if (q < nq)
        o[q] = make_float4(
            __fmul_rn(__fmul_rn(v[i].x, rs), g[i].x), __fmul_rn(__fmul_rn(v[i].y, rs), g[i].y),
            __fmul_rn(__fmul_rn(v[i].z, rs), g[i].z), __fmul_rn(__fmul_rn(v[i].w, rs), g[i].w));
    }
    return;
  }
  __shared__ float red4[4];
  const float* xr = x + (size_t)blockIdx.x * size;
  float* o = out + (size_t)blockIdx.x * size;
  float ss = 0.f;
  for (int c = threadIdx.x; c < size; c += 256) ss += xr[c] * xr[c];
  ss = block_sum256(ss, red4);
  const float rs = 1.0f / sqrtf(ss / (float)size + eps);
  for (int c = threadIdx.x; c < size; c += 256)
    o[c] = __fmul_rn(__fmul_rn(xr[c], rs), w[c]);
}

// m / S and m % S for 0 <= m < 2^23 through a float reciprocal (a quotient
// off by at most one, then corrected): a few instructions instead of an
// integer division per row of the QKV epilogue.
__device__ __forceinline__ void div_rows(int m, int S, int& q, int& r) {
  q = (int)((float)m * __builtin_amdgcn_rcpf((float)S));
  r = m - q * S;
  if (r < 0) {
    --q;
    r += S;
  } else if (r >= S) {
    ++q;
    r -= S;
  }
}

// Epilogue on the adjacent column pair (n, n + 1), n even, of row m.  With
// N even a pair is one 8-byte-aligned store (an odd N, as a vocabulary-wide
// lm_head, stores the two floats apart); the QKV destinations have even
// strides.  After inlining into a kernel's unrolled output loop, everything
// that depends on n alone is computed once per lane.
template <int EPI>
__device__ __forceinline__ void epi_pair_gemm(const GemmParams& p, int M,
                                              int N, int m, int n, float v0,
                                              float v1) {
  if (m >= M || n >= N) return;
  const bool has1 = n + 1 < N, pair = (N & 1) == 0;
  float* y = p.c + (size_t)m * N + n;
  auto put = [&](float* dst, float a, float b) {
    if (pair) {
      *reinterpret_cast<float2*>(dst) = make_float2(a, b);
    } else {
      dst[0] = a;
      if (has1) dst[1] = b;
    }
  };
  if (EPI == GEMM_STORE) {
    put(y, v0, v1);
  } else if (EPI == GEMM_ADD) {
    if (pair) {
      const float2 o = *reinterpret_cast<const float2*>(y);
      *reinterpret_cast<float2*>(y) = make_float2(o.x + v0, o.y + v1);
    } else {
      y[0] = y[0] + v0;
      if (has1) y[1] = y[1] + v1;
    }
  } else if (EPI == GEMM_SILU) {
    // x / (1 + e^-x) as x * rcp(1 + 2^(-x log2 e)): within a few ulp of the
    // IEEE expression, at a fraction of its instructions.
    auto silu = [](float v) {
      return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.44269504088896341f));
    };
    put(y, silu(v0), silu(v1));
  } else if (EPI == GEMM_QKV) {
    // Columns [0, d) are Q, [d, 2d) K, [2d, 3d) V (weights.rs:49-58).
    const int dim = p.dim;
    const int region = n / dim, c = n - region * dim;
    int seq, t;
    if (p.rowmap) {
      const int2 st = p.rowmap[m];
      seq = st.x;
      t = st.y;
    } else {
      div_rows(m, p.S, seq, t);
    }
    if (region < 2) {
      const int i = (c % p.head_dim) >> 1;
      const float2 cs = p.rope[(size_t)t * (p.head_dim >> 1) + i];
      rope_pair(v0, v1, cs.x, cs.y);
    }
    float* dst;
    if (region == 0)
      dst = p.q_out + (size_t)m * dim + c;
    else if (p.kv_packed)
      dst = (region == 1 ? p.kcache : p.vcache) + (size_t)m * dim + c;
    else
      dst = (region == 1 ? p.kcache : p.vcache) + (size_t)seq * p.seq_stride +
            (size_t)t * dim + c;
    *reinterpret_cast<float2*>(dst) = make_float2(v0, v1);
  }
}

// The epilogue of one 32-row MFMA tile pair as a lane holds it: rows
// mbase + acc_row(r, h), r = 0..15, columns n and n + 1 (n even).  Every load
// the epilogue needs (the residual of GEMM_ADD, the RoPE table and row map of
// GEMM_QKV) is issued for all 16 rows before the first store: stores may
// alias those loads as far as the compiler knows, so pair by pair each load
// would wait out the previous store and its own latency in turn.
template <int EPI>
__device__ __forceinline__ void epi_tile(const GemmParams& p, int M, int N, int mbase, int n,
                                         const float (&v0)[16], const float (&v1)[16]) {
  const int h = (threadIdx.x & 63) >> 5;
  if (EPI == GEMM_ADD && (N & 1) == 0 && n < N) {
    float2 old[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mbase + acc_row(r, h);
      old[r] = m < M ? *reinterpret_cast<const float2*>(p.c + (size_t)m * N + n)
                     : make_float2(0.f, 0.f);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mbase + acc_row(r, h);
      if (m < M)
        *reinterpret_cast<float2*>(p.c + (size_t)m * N + n) =
            make_float2(old[r].x + v0[r], old[r].y + v1[r]);
    }
    return;
  }
  if (EPI == GEMM_QKV && n < N) {
    const int dim = p.dim, region = n / dim, c = n - region * dim;
    const int i = (c % p.head_dim) >> 1, half_hd = p.head_dim >> 1;
    int seq[16], t[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = min(mbase + acc_row(r, h), M - 1);
      if (p.rowmap) {
        const int2 st = p.rowmap[m];
        seq[r] = st.x;
        t[r] = st.y;
      } else {
        div_rows(m, p.S, seq[r], t[r]);
      }
    }
    float2 cs[16];
    if (region < 2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) cs[r] = p.rope[(size_t)t[r] * half_hd + i];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mbase + acc_row(r, h);
      if (m >= M) continue;
      float a = v0[r], b = v1[r];
      if (region < 2) rope_pair(a, b, cs[r].x, cs[r].y);
      float* dst;
      if (region == 0)
        dst = p.q_out + (size_t)m * dim + c;
      else if (p.kv_packed)
        dst = (region == 1 ? p.kcache : p.vcache) + (size_t)m * dim + c;
      else
        dst = (region == 1 ? p.kcache : p.vcache) + (size_t)seq[r] * p.seq_stride +
              (size_t)t[r] * dim + c;
      *reinterpret_cast<float2*>(dst) = make_float2(a, b);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) epi_pair_gemm<EPI>(p, M, N, mbase + acc_row(r, h), n, v0[r], v1[r]);
}

// C[M,N] = A[M,K] B[K,N], 128x128 block tile, BK = 16, 4 waves in 2x2,
// each wave a 64x64 sub-tile as 2x2 MFMA 32x32 tiles.  A is staged
// transposed in LDS so MFMA A-operand reads are contiguous; within a wave's
// 64 columns, lane j of N tile t owns column 2j + t so each lane holds
// adjacent column pairs (float2 B reads, paired epilogue for RoPE).  The
// next K tile is fetched into registers while the current one is consumed.
// SPLIT: the grid's z splits K over p.split_kc rows per block, the tile's
// last block adding the splits (a separate instantiation: the split code
// made the unsplit kernel 30 % slower on config 3's fp32-MFMA prefill).
template <int EPI, bool SPLIT = false>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  constexpr int BM = 128, BN = 128, BK = 16;
  constexpr int APAD = 4;
  __shared__ float As[BK][BM + APAD];
  __shared__ float Bs[BK][BN];

  int M = p.M, N = p.N, K = p.K;
  if (p.meta) {
    // The live shape, at most the recorded one (the grid, the split ranges
    // and the caller's buffers are sized by the recorded shape).
    M = min((int)p.meta->m, p.M);
    N = min((int)p.meta->n, p.N);
    K = min((int)p.meta->k, p.K);
  }
  // Each XCD takes a contiguous run of tiles (see k_gemm_bf16).
  int id = blockIdx.x + gridDim.x * blockIdx.y;
  const int per_xcd = (int)(gridDim.x * gridDim.y) / 8;
  if (id < per_xcd * 8) id = (id % 8) * per_xcd + id / 8;
  const int m0 = (id / gridDim.x) * BM, n0 = (id % gridDim.x) * BN;
  if (m0 >= M || n0 >= N) return;  // every split of the tile returns here
  // This block's rows of K: all of them, or split blockIdx.z's p.split_kc.
  const int kbeg = SPLIT ? min(K, (int)blockIdx.z * p.split_kc) : 0;
  const int kend = SPLIT ? min(K, kbeg + p.split_kc) : K;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  // A: 128 rows x 16 k -> thread loads row tid/2, k 8*(tid&1) .. +7.
  // B: 16 rows x 128 cols -> rows tid/32 and tid/32 + 8, cols 4*(tid&31).
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
      if (gm < M && a_vec && gk + 3 < kend) {
        const float4 t = *reinterpret_cast<const float4*>(ap + gk);
        ra[4 * q] = t.x; ra[4 * q + 1] = t.y; ra[4 * q + 2] = t.z; ra[4 * q + 3] = t.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ra[4 * q + e] = (gm < M && gk + e < kend) ? ap[gk + e] : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int gk = k0 + b_row + 8 * q;
      const int gn = n0 + b_col;
      const float* bp = p.b + (size_t)(gk < kend ? gk : 0) * N + gn;
      if (gk < kend && b_vec && gn + 3 < N) {
        const float4 t = *reinterpret_cast<const float4*>(bp);
        rb[4 * q] = t.x; rb[4 * q + 1] = t.y; rb[4 * q + 2] = t.z; rb[4 * q + 3] = t.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rb[4 * q + e] = (gk < kend && gn + e < N) ? bp[e] : 0.f;
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

  const int nk = (kend - kbeg + BK - 1) / BK;
  load_tile(kbeg);
  store_tile();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_tile(kbeg + (kt + 1) * BK);
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

  if constexpr (SPLIT) {
    __shared__ int last_split;
    // A split tile: each block stores its sums (written through to device
    // scope, lane-major), waits until they have completed and counts
    // itself; the last of the tile's blocks adds every split's sums in split
    // order (the same float sums whichever block is last) and runs the
    // epilogue.
    constexpr int TILE = BM * BN;
    const int tile = blockIdx.x + gridDim.x * blockIdx.y;
    const int tiles = gridDim.x * gridDim.y;
    auto at = [&](int a, int t, int r) { return (((wave * 2 + a) * 2 + t) * 16 + r) * 64 + lane; };
    float* mine = p.split_ws + ((size_t)blockIdx.z * tiles + tile) * TILE;
    // A wave whose 64 rows all lie past M neither stores nor reads partials.
    const bool live = m0 + wm * 64 < M;
    if (live)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            __hip_atomic_store(mine + at(a, t, r), acc[a][t][r], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int done =
          __hip_atomic_fetch_add(p.split_cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_split = done == (int)gridDim.z - 1;
      if (last_split)  // zero for the next launch
        __hip_atomic_store(p.split_cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_split) return;
    // Split by split, each split's 64 values per lane all in flight at once.
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][t][r] = 0.f;
    for (int sp = 0; live && sp < (int)gridDim.z; ++sp) {
      const float* part = p.split_ws + ((size_t)sp * tiles + tile) * TILE;
      float v[2][2][16];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            v[a][t][r] = __hip_atomic_load(part + at(a, t, r), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[a][t][r] += v[a][t][r];
    }
  }
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    float v0[16], v1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      v0[r] = acc[a][0][r];
      v1[r] = acc[a][1][r];
    }
    epi_tile<EPI>(p, M, N, m0 + wm * 64 + a * 32, n0 + wn * 64 + 2 * j, v0, v1);
    }
}

// The shape a flash block works on: the recorded one, or the live meta of a
// per-shader launch (FlashAttnMeta, read when the kernel runs; meta.rs).  A
// live meta may shrink the recorded shape the grid was sized for, never grow
// it or change the head size; for such a meta, and for a head past the live
// head count (the reference kernel returns for head >= num_heads,
// cuda.rs:647), the block returns false and touches no memory.
//
// It also places sequence b: element offsets of its first row in q, in k
// and v, and in o, and of its lse rows -- per-sequence strides, the live
// meta's row_offset, or, for ragged prompts packed back to back, the rows
// rows_at[b] .. rows_at[b + 1] (whose count is then its length S).
struct FlashSeq {
  int S, d;
  float scale;
  long q, kv, o, l;
};
//
// The kernels' HD is a register-tile size; the head size is p.hd <= HD (a
// head_dim that is not a power of two runs in the next larger kernel, its
// columns past p.hd read as zero and never stored).
template <int HD>
__device__ __forceinline__ bool flash_seq(const FlashParams& p, int hh, int b, FlashSeq& f) {
  f.S = p.S;
  f.d = p.d;
  f.scale = p.scale;
  long roff = 0;
  if (p.hd > HD) return false;
  if (p.meta) {
    const akh_flash_attn_meta m = *p.meta;
    if ((int)m.head_dim != p.hd || (int)m.seq_len > p.S || (int)m.dim > p.d) return false;
    f.S = (int)m.seq_len;
    f.d = (int)m.dim;
    f.scale = m.scale;
    roff = (long)m.row_offset * f.d;
  }
  if (hh >= f.d / p.hd) return false;
  if (p.rows_at) {
    const int r0 = p.rows_at[b];
    f.S = min(p.rows_at[b + 1] - r0, p.S);
    f.q = f.o = (long)r0 * f.d;
    f.kv = p.kv_packed ? f.q : (long)b * p.kv_bs;
    f.l = (long)r0 * (f.d / p.hd);
  } else {
    f.q = roff + (long)b * p.q_bs;
    f.kv = roff + (long)b * p.kv_bs;
    f.o = roff + (long)b * p.o_bs;
    f.l = (long)b * p.lse_bs;
  }
  return true;
}

// Causal flash attention on MFMA for head_dim 64 and 128.  Block = 4 waves x
// 32 queries of one (sequence, head); keys stream through LDS in blocks of
// 32.  Each wave computes S^T = K Q^T so every lane owns one query (column)
// and 16 keys, making the online-softmax row statistics lane-local (plus one
// exchange between the two half-waves); P^T then feeds O^T += V^T P^T
// straight from the accumulator registers, one 32-dim tile per HD/32.
// Query blocks run in reverse order so the longest (last) ones start first.
template <int HD>
__global__ __launch_bounds__(256, HD == 64 ? 3 : 2) void k_flash_mfma(FlashParams p) {
  constexpr int QB = 128, KB = 32, NT = HD / 32, HQ = HD / 2;
  constexpr int KP = HD + 1;            // padded K row
  constexpr int CPR = HD / 4;           // float4 per K/V row
  constexpr int RPP = 256 / CPR;        // rows per cooperative pass
  constexpr int NP = KB / RPP;          // passes per key block
  constexpr int KV_FLOATS = KB * KP + KB * HD;
  constexpr int O_FLOATS = 4 * 32 * 33;  // one 32x32 tile per wave
  __shared__ float lds[KV_FLOATS > O_FLOATS ? KV_FLOATS : O_FLOATS];
  float (*Ks)[KP] = reinterpret_cast<float (*)[KP]>(lds);
  float (*Vs)[HD] = reinterpret_cast<float (*)[HD]>(lds + KB * KP);

  const int qblk = gridDim.z - 1 - blockIdx.z, hh = blockIdx.x, b = blockIdx.y;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return;
  const int S = fs.S, d = fs.d;
  const float scale = fs.scale;
  const int H = d / HD;
  const float qscale = scale * 1.44269504088896341f;
  const int q0 = qblk * QB;
  if (q0 >= S) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  const float* qp = p.q + fs.q + hh * HD;
  const float* kp = p.k + fs.kv + hh * HD;
  const float* vp = p.v + fs.kv + hh * HD;

  // This lane's query row and its HD/2 dims (half h).
  const int qi = q0 + wave * 32 + j;
  float qreg[HQ];
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + HQ * h;
#pragma unroll
    for (int s = 0; s < HQ; s += 4) {
      const float4 t = *reinterpret_cast<const float4*>(qr + s);
      qreg[s] = t.x; qreg[s + 1] = t.y; qreg[s + 2] = t.z; qreg[s + 3] = t.w;
    }
  }
  f32x16 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = zero16();
  float mrow = -INFINITY, lrow = 0.f;

  const int wave_qmax = q0 + wave * 32 + 31;
  const int kend = min(S, q0 + QB);  // keys needed by the block
  const int nkb = (kend + KB - 1) / KB;

  // Cooperative K/V block load: thread t loads float4 column t % CPR of rows
  // t / CPR + RPP * q, of both tensors.
  const int lr = tid / CPR, lc = (tid % CPR) * 4;
  float4 kr[NP], vr[NP];
  auto load_kv = [&](int kb) {
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int key = kb * KB + lr + RPP * q;
      const size_t off = (size_t)(key < S ? key : 0) * d + lc;
      kr[q] = *reinterpret_cast<const float4*>(kp + off);
      vr[q] = *reinterpret_cast<const float4*>(vp + off);
    }
  };
  load_kv(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int r = lr + RPP * q;
      Ks[r][lc] = kr[q].x; Ks[r][lc + 1] = kr[q].y;
      Ks[r][lc + 2] = kr[q].z; Ks[r][lc + 3] = kr[q].w;
      *reinterpret_cast<float4*>(&Vs[r][lc]) =
          make_float4(vr[q].x, vr[q].y, vr[q].z, vr[q].w);
    }
    __syncthreads();
    load_kv(kb + 1);  // rows past S read row 0: harmless, never used
    const int j0 = kb * KB;
    if (j0 > wave_qmax) continue;  // block entirely above this wave's rows

    f32x16 st = zero16();
#pragma unroll
    for (int s = 0; s < HQ; ++s) st = mfma32(Ks[j][HQ * h + s], qreg[s], st);

    // Scores in the log2 domain (exp(scale x - m) = exp2(scale log2(e) x -
    // m')); keys above a query or past S exist only in diagonal or ragged
    // blocks, the only ones masked.
    const bool masked = j0 + KB - 1 > q0 + wave * 32 || j0 + KB > S;
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * qscale;
      if (masked) {
        const int key = j0 + acc_row(r, h);
        if (key > qi || key >= S) v = -INFINITY;
      }
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float mnew = fmaxf(mrow, pm);  // finite: key 0 is in every query's range
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(mrow - mnew);  // 0 on the first block
    lrow = lrow * corr + ps;
    if (__any(mnew != mrow)) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    }
    mrow = mnew;
    // O^T += V^T P^T: step s uses key acc_row(s, h) on both operands.
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int key = acc_row(s, h);
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] = mfma32(Vs[key][32 * t + j], st[s], o[t]);
    }
  }

  // O^T (rows = dims) -> LDS, one 32-dim tile at a time -> coalesced rows.
  const float inv = 1.0f / lrow;
  float (*Os)[33] = reinterpret_cast<float (*)[33]>(lds + wave * 32 * 33);
  float* op = p.o + fs.o + hh * HD;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) Os[j][acc_row(r, h)] = o[t][r] * inv;
    __syncthreads();
    for (int e = lane; e < 32 * 32; e += 64) {
      const int r = e >> 5, c = e & 31;
      const int qrow = q0 + wave * 32 + r;
      if (qrow < S) op[(size_t)qrow * d + 32 * t + c] = Os[r][c];
    }
  }
  if (p.lse && h == 0 && qi < S)  // max + ln(sum), back in natural units
    p.lse[fs.l + (size_t)qi * H + hh] =
        mrow * 0.69314718055994531f + logf(lrow);
}

// Causal flash attention for the small head sizes (2..32; the reference
// allows up to 128, emit.rs:564-567): one thread per query row with an HD-float
// accumulator, keys staged through LDS in blocks of 64 shared by the
// block's 64 queries.
template <int HD>
__global__ __launch_bounds__(64) void k_flash_generic(FlashParams p) {
  constexpr int KB = 64;
  __shared__ float Ks[KB][HD];
  __shared__ float Vs[KB][HD];
  const int hh = blockIdx.y, b = blockIdx.z;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return;
  const int S = fs.S, d = fs.d, hd = p.hd;  // head size hd <= HD
  const float scale = fs.scale;
  const int H = d / hd;
  const int q0 = blockIdx.x * 64;
  if (q0 >= S) return;
  const int i = q0 + threadIdx.x;
  const float* qp = p.q + fs.q + hh * hd;
  const float* kp = p.k + fs.kv + hh * hd;
  const float* vp = p.v + fs.kv + hh * hd;
  float q[HD], acc[HD];
#pragma unroll
  for (int c = 0; c < HD; ++c) {
    q[c] = i < S && c < hd ? qp[(size_t)i * d + c] : 0.f;
    acc[c] = 0.f;
  }
  float mrow = -INFINITY, lrow = 0.f;
  const int kend = min(S, q0 + 64);
  for (int k0 = 0; k0 < kend; k0 += KB) {
    __syncthreads();
    for (int e = threadIdx.x; e < KB * HD; e += 64) {
      const int r = e / HD, c = e % HD;
      const int key = k0 + r;
      Ks[r][c] = key < S && c < hd ? kp[(size_t)key * d + c] : 0.f;
      Vs[r][c] = key < S && c < hd ? vp[(size_t)key * d + c] : 0.f;
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
  float* op = p.o + fs.o + hh * hd + (size_t)i * d;
#pragma unroll
  for (int c = 0; c < HD; ++c)
    if (c < hd) op[c] = acc[c] / lrow;
  if (p.lse) p.lse[fs.l + (size_t)i * H + hh] = mrow + logf(lrow);
}

// ---------------------------------------------------------------------------
// bfloat16-MFMA prefill

// wt[n, k] = bf16(w[k, n]) through a 32x32 LDS tile.
__global__ __launch_bounds__(256) void k_transpose_bf16(const float* __restrict__ w, int K,
                                                        int N, uint16_t* __restrict__ wt) {
  __shared__ float t[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int c = threadIdx.x & 31, r = threadIdx.x >> 5;
  for (int i = r; i < 32; i += 8) {
    const int k = k0 + i, n = n0 + c;
    t[i][c] = (k < K && n < N) ? w[(size_t)k * N + n] : 0.f;
  }
  __syncthreads();
  for (int i = r; i < 32; i += 8) {
    const int n = n0 + i, k = k0 + c;
    if (n < N && k < K) wt[(size_t)n * K + k] = (uint16_t)bf16_bits(t[c][i]);
  }
}

// C[M,N] = A[M,K] B[K,N] with bfloat16 A [M, K] and B^T [N, K], fp32
// accumulation on v_mfma_f32_32x32x16_bf16.  Block tile 256x256, BK = 32,
// 8 waves as 2 (rows) x 4 (columns), each wave 128x64 as 4x2 MFMA tiles.
// Tiles are staged in LDS k-contiguous (rows padded to 80 bytes, so the
// 16-byte fragment reads of 16 consecutive rows hit distinct banks), double
// buffered with the next tile's global loads issued before the MFMAs.  B
// rows are stored permuted so lane j of column tile t reads the row of
// column 2j + t: each lane ends up with adjacent column pairs, as the
// paired epilogues (RoPE) need.
//
// AM (A's form): 0, A is bfloat16 (p.a16); 1, A is fp32 (p.a) and enters as
// two bfloat16 parts, hi = bf16(a) and lo = bf16(a - hi), each multiplied by
// B (two MFMAs): with bfloat16-exact weights the products then carry a's
// first 16 significant bits; 2, A is fp32 rounded to bfloat16 as it is
// staged (one MFMA).
template <int EPI, int AM>
__global__ __launch_bounds__(512) void k_gemm_bf16(GemmParams p) {
  constexpr int BM = 256, BN = 256, BK = 32, LD = BK + 8;
  constexpr bool A32 = AM != 0;
  constexpr int NA = AM == 1 ? 2 : 1;
  __shared__ __align__(16) uint16_t As[NA][2][BM][LD];
  __shared__ __align__(16) uint16_t Bs[2][BN][LD];

  const int M = p.M, N = p.N, K = p.K;
  // Workgroups go to the 8 XCDs round-robin in launch order; give each XCD
  // a contiguous run of tiles (N fastest) so the blocks sharing an A panel
  // share that XCD's L2.
  int id = blockIdx.x + gridDim.x * blockIdx.y;
  const int per_xcd = (int)(gridDim.x * gridDim.y) / 8;
  if (id < per_xcd * 8) id = (id % 8) * per_xcd + id / 8;
  const int m0 = (id / gridDim.x) * BM, n0 = (id % gridDim.x) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int j = lane & 31, h = lane >> 5;

  // Global -> register staging: rows tid / 4 and tid / 4 + 128, eight k at
  // (tid % 4) * 8, of B^T and of a bfloat16 A; an fp32 A (four times the
  // pieces) goes as row f / 8, k 4 (f % 8) .. + 3 for piece f = tid + 512 i,
  // so eight consecutive lanes read one row's 128-byte line.  Loads go
  // through buffer resources bounded to the block's rows; rows past M or N
  // and pieces past K (given an offset outside the resource) read zeros
  // from the hardware.
  const int sr = tid >> 2, sk = (tid & 3) * 8;
  // Two register sets: the loads of step s + 2 are issued at the start of
  // step s, and step s + 1's are stored to LDS after step s's MFMAs.
  uint4 ra[2][2], rb[2][2];
  float4 fa[2][4];  // A32 staging
  const int ea = A32 ? 4 : 2;  // bytes per A element
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      A32 ? (void*)(p.a + (size_t)m0 * K) : (void*)(p.a16 + (size_t)m0 * K), (short)0,
      min(M - m0, BM) * K * ea, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.bt16 + (size_t)n0 * K), (short)0, min(N - n0, BN) * K * 2, 0x00020000);
  auto ld = [](__amdgpu_buffer_rsrc_t rs, uint32_t vo, int so) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vo, so, 0));
  };
  auto gload = [&](int k0, int set) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = sr + 128 * i, k = k0 + sk;
      const uint32_t off = (uint32_t)(r * K + k);
      const uint32_t va = k < K ? off * ea : 0x80000000u, vb = k < K ? off * 2 : 0x80000000u;
      if (!A32) ra[set][i] = ld(rsa, va, 0);
      rb[set][i] = ld(rsb, vb, 0);
    }
    if (A32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = tid + 512 * i, r = f >> 3, k = k0 + 4 * (f & 7);
        const uint32_t va = k < K ? (uint32_t)(r * K + k) * 4u : 0x80000000u;
        fa[set][i] = __builtin_bit_cast(float4, ld(rsa, va, 0));
      }
    }
  };
  auto lstore = [&](int buf, int set) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = sr + 128 * i;
      // Column c = 64 g + 2 jj + t of the block lives at LDS row 64 g + 32 t + jj.
      const int br = (r & ~63) | ((r & 1) << 5) | ((r & 63) >> 1);
      if (!A32) *reinterpret_cast<uint4*>(&As[0][buf][r][sk]) = ra[set][i];
      *reinterpret_cast<uint4*>(&Bs[buf][br][sk]) = rb[set][i];
    }
    if (A32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = tid + 512 * i, r = f >> 3, k = 4 * (f & 7);
        const float4 x = fa[set][i];
        const uint2 hi = make_uint2(cvt_pk_bf16(x.x, x.y), cvt_pk_bf16(x.z, x.w));
        *reinterpret_cast<uint2*>(&As[0][buf][r][k]) = hi;
        if constexpr (NA == 2) {
          const uint2 lo = make_uint2(
              cvt_pk_bf16(x.x - __uint_as_float(hi.x << 16), x.y - __uint_as_float(hi.x & 0xFFFF0000u)),
              cvt_pk_bf16(x.z - __uint_as_float(hi.y << 16), x.w - __uint_as_float(hi.y & 0xFFFF0000u)));
          *reinterpret_cast<uint2*>(&As[NA - 1][buf][r][k]) = lo;
        }
      }
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[a][t] = zero16();

  const int nk = (K + BK - 1) / BK;
  gload(0, 0);
  gload(BK, 1);
  lstore(0, 0);
  __syncthreads();
  // Step kt computes on LDS buffer kt % 2.  Steps past the end load zeros.
  auto stepk = [&](int kt, int buf) {
    __builtin_amdgcn_sched_barrier(0);
    gload((kt + 2) * BK, buf);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8 bfr[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        bfr[t] = bf16x8_of(*reinterpret_cast<const uint4*>(
            &Bs[buf][wn * 64 + t * 32 + j][ks * 16 + 8 * h]));
#pragma unroll
      for (int part = 0; part < NA; ++part) {
        bf16x8 af[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
          af[a] = bf16x8_of(*reinterpret_cast<const uint4*>(
              &As[part][buf][wm * 128 + a * 32 + j][ks * 16 + 8 * h]));
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[a], bfr[t], acc[a][t]);
      }
    }
    lstore(buf ^ 1, buf ^ 1);
    __syncthreads();
  };
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    stepk(kt, 0);
    stepk(kt + 1, 1);
  }
  if (kt < nk) stepk(kt, 0);

#pragma unroll
  for (int a = 0; a < 4; ++a) {
    float v0[16], v1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      v0[r] = acc[a][0][r];
      v1[r] = acc[a][1][r];
    }
    epi_tile<EPI>(p, M, N, m0 + wm * 128 + a * 32, n0 + wn * 64 + 2 * j, v0, v1);
    }
}

// ---------------------------------------------------------------------------
// fp32 GEMM on bfloat16 MFMAs (launch_gemm_x6)

// wt[n, k] = w[k, n] for a [K, N] row-major matrix, through a 32x32 LDS tile.
__global__ __launch_bounds__(256) void k_transpose_f32(const float* __restrict__ w, int K, int N,
                                                       float* __restrict__ wt) {
  __shared__ float t[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int c = threadIdx.x & 31, r = threadIdx.x >> 5;
  for (int i = r; i < 32; i += 8) {
    const int k = k0 + i, n = n0 + c;
    t[i][c] = (k < K && n < N) ? w[(size_t)k * N + n] : 0.f;
  }
  __syncthreads();
  for (int i = r; i < 32; i += 8) {
    const int n = n0 + i, k = k0 + c;
    if (n < N && k < K) wt[(size_t)n * K + k] = t[c][i];
  }
}

// The fp16 planes of k_gemm_h3's weights: for a [K, N] row-major matrix,
// wp[((n K/8 + k/8) 2 + p) 8 + k%8] = plane p (0: hi, 1: lo) of w[k, n] as
// split by split2_f16, so one 32-byte run holds the hi and lo octets of
// eight consecutive k of column n.  K % 8 == 0.  A 32 x 32 tile through LDS;
// thread (n, octet) writes its 32 bytes.
__global__ __launch_bounds__(256) void k_split_weights_f16(const float* __restrict__ w, int K,
                                                           int N, uint16_t* __restrict__ wp) {
  __shared__ float t[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int c = threadIdx.x & 31, r = threadIdx.x >> 5;
  for (int i = r; i < 32; i += 8) {
    const int k = k0 + i, n = n0 + c;
    t[i][c] = (k < K && n < N) ? w[(size_t)k * N + n] : 0.f;
  }
  __syncthreads();
  if (threadIdx.x >= 128) return;
  const int nl = threadIdx.x >> 2, q = threadIdx.x & 3;
  const int n = n0 + nl, k = k0 + 8 * q;
  if (n >= N || k >= K) return;
  const float4 x0 = make_float4(t[8 * q][nl], t[8 * q + 1][nl], t[8 * q + 2][nl], t[8 * q + 3][nl]);
  const float4 x1 =
      make_float4(t[8 * q + 4][nl], t[8 * q + 5][nl], t[8 * q + 6][nl], t[8 * q + 7][nl]);
  uint4 hi, lo;
  split2_f16(x0, x1, hi, lo);
  uint4* dst = reinterpret_cast<uint4*>(wp + ((size_t)n * (K / 8) + k / 8) * 16);
  dst[0] = hi;
  dst[1] = lo;
}

// C[M,N] = A[M,K] B[K,N] in fp32 accuracy on v_mfma_f32_32x32x16_bf16.
// A (p.a, [M, K]) and the transposed weights B^T (p.bt, [N, K]) are fp32;
// each element enters LDS as three bfloat16 terms (split3_rne: a = a1 + a2
// + a3 exactly, |a2| <= 2^-8 |a|, |a3| <= 2^-16 |a|).  Every product of
// terms is exact in fp32; the six whose size reaches 2^-16 |a b| are
// accumulated (a1b1, a1b2, a2b1, a1b3, a2b2, a3b1), so each product a.b is
// carried to within 2^-23 relative, about fp32's own rounding, at 6 x 32
// instead of 8 x 64 MFMA cycles per 16 k.
//
// Block tile BM x BN, BK = 16, waves WM (rows) x WN (columns); a wave owns
// (BM / WM) x 64 as TA x 2 MFMA tiles.  LDS holds the three planes of both
// operands k-contiguous (rows of 16 k padded to 48 bytes, so 16-byte
// fragment reads of 8 consecutive rows hit distinct banks), double
// buffered.  Global loads run two k steps ahead through two register sets;
// each step splits and stores step k + 1 (loaded a step earlier) in the same
// straight-line block as step k's MFMAs, so the split's VALU work and the
// LDS writes overlap the matrix pipe.  K % 8 == 0.
template <int EPI, int BM, int BN, int WM, int WN, bool IL>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_x6(GemmParams p) {
  constexpr int BK = 16, LD = BK + 8, NT = 64 * WM * WN;
  constexpr int TA = BM / WM / 32;
  static_assert(BN == 64 * WN && BM % (32 * WM) == 0, "wave tiles are (32 TA) x 64");
  constexpr int OA = 2 * BM / NT, OB = 2 * BN / NT;  // k-octets staged per thread
  static_assert(OA >= 1 && OB >= 1 && OA * NT == 2 * BM && OB * NT == 2 * BN,
                "every thread stages whole octets of both operands");
  __shared__ __align__(16) uint16_t As[2][3][BM][LD];
  __shared__ __align__(16) uint16_t Bs[2][3][BN][LD];

  const int M = p.M, N = p.N, K = p.K;
  // Each XCD takes a contiguous run of tiles (see k_gemm_bf16).
  int id = blockIdx.x + gridDim.x * blockIdx.y;
  const int per_xcd = (int)(gridDim.x * gridDim.y) / 8;
  if (id < per_xcd * 8) id = (id % 8) * per_xcd + id / 8;
  const int m0 = (id / gridDim.x) * BM, n0 = (id % gridDim.x) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int j = lane & 31, h = lane >> 5;

  // Staging: octet o = tid + NT * i covers LDS row (o % 16) + 16 (o / 32),
  // k 8 ((o / 16) % 2) .. + 7: lanes l and l + 16 load the two halves of one
  // row in the same instruction, and 16 consecutive lanes write 16
  // consecutive 48-byte rows (conflict-free).  B's LDS row L = 64 g + 32 t + jj holds column 64 g +
  // 2 jj + t of the block (lane j of column tile t then reads column 2j + t:
  // adjacent column pairs for the paired epilogues).
  // Loads go through buffer resources bounded to the block's rows of A and
  // B^T: octets past M or N fall outside them, octets past K get an offset
  // outside them, and the hardware returns zeros for both.  The loads stay
  // unconditional (no exec-masked branch) and nothing touches their
  // registers before the split, so the compiler can count them and wait for
  // one register set while the other's loads are still in flight.
  float4 ra[2][OA][2], rb[2][OB][2];
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.a + (size_t)m0 * K), (short)0, min(M - m0, BM) * K * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.bt + (size_t)n0 * K), (short)0, min(N - n0, BN) * K * 4, 0x00020000);
  auto ld4 = [](__amdgpu_buffer_rsrc_t rs, uint32_t vo, int so) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vo, so, 0));
    return make_float4(v.x, v.y, v.z, v.w);
  };
  auto bcol = [](int L) { return (L & ~63) | ((L & 31) << 1) | ((L >> 5) & 1); };
  auto orow = [](int o) { return (o & 15) | ((o >> 5) << 4); };
  auto okof = [](int o) { return ((o >> 4) & 1) * 8; };
  auto gload = [&](int k0, int set) {
#pragma unroll
    for (int i = 0; i < OA; ++i) {
      const int o = tid + NT * i, k = k0 + okof(o);
      const uint32_t vo = k < K ? (uint32_t)(orow(o) * K + k) * 4u : 0x80000000u;
      ra[set][i][0] = ld4(rsa, vo, 0);
      ra[set][i][1] = ld4(rsa, vo, 16);
    }
#pragma unroll
    for (int i = 0; i < OB; ++i) {
      const int o = tid + NT * i, k = k0 + okof(o);
      const uint32_t vo = k < K ? (uint32_t)(bcol(orow(o)) * K + k) * 4u : 0x80000000u;
      rb[set][i][0] = ld4(rsb, vo, 0);
      rb[set][i][1] = ld4(rsb, vo, 16);
    }
  };
  auto lstore = [&](int buf, int set) {
#pragma unroll
    for (int i = 0; i < OA; ++i) {
      const int o = tid + NT * i, r = orow(o), k = okof(o);
      uint4 t0, t1, t2;
      split3_rne(ra[set][i][0], ra[set][i][1], t0, t1, t2);
      *reinterpret_cast<uint4*>(&As[buf][0][r][k]) = t0;
      *reinterpret_cast<uint4*>(&As[buf][1][r][k]) = t1;
      *reinterpret_cast<uint4*>(&As[buf][2][r][k]) = t2;
    }
#pragma unroll
    for (int i = 0; i < OB; ++i) {
      const int o = tid + NT * i, L = orow(o), k = okof(o);
      uint4 t0, t1, t2;
      split3_rne(rb[set][i][0], rb[set][i][1], t0, t1, t2);
      *reinterpret_cast<uint4*>(&Bs[buf][0][L][k]) = t0;
      *reinterpret_cast<uint4*>(&Bs[buf][1][L][k]) = t1;
      *reinterpret_cast<uint4*>(&Bs[buf][2][L][k]) = t2;
    }
  };

  f32x16 acc[TA][2];
#pragma unroll
  for (int a = 0; a < TA; ++a)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[a][t] = zero16();

  // One k step: in two parts (the fragment reads of LDS buffer `buf`, the
  // MFMAs on them) for the interleaved schedule, in one (`step`) otherwise.
  typedef bf16x8 Frags[2 + TA][3];  // [0..1]: B column tiles, [2 + a]: A row tiles
  auto frags = [&](int buf, Frags& f) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        f[t][pl] = bf16x8_of(
            *reinterpret_cast<const uint4*>(&Bs[buf][pl][wn * 64 + t * 32 + j][8 * h]));
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        f[2 + a][pl] = bf16x8_of(
            *reinterpret_cast<const uint4*>(&As[buf][pl][wm * (32 * TA) + a * 32 + j][8 * h]));
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int a = 0; a < TA; ++a) {
      const bf16x8* af = f[2 + a];
      // Smallest terms first.
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[2], f[t][0], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[1], f[t][1], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[0], f[t][2], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[1], f[t][0], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[0], f[t][1], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[0], f[t][0], acc[a][t]);
    }
  };
  auto step = [&](int buf) {
    bf16x8 bfr[2][3];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        bfr[t][pl] = bf16x8_of(
            *reinterpret_cast<const uint4*>(&Bs[buf][pl][wn * 64 + t * 32 + j][8 * h]));
#pragma unroll
    for (int a = 0; a < TA; ++a) {
      bf16x8 af[3];
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        af[pl] = bf16x8_of(
            *reinterpret_cast<const uint4*>(&As[buf][pl][wm * (32 * TA) + a * 32 + j][8 * h]));
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[2], bfr[t][0], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[1], bfr[t][1], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[0], bfr[t][2], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[1], bfr[t][0], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[0], bfr[t][1], acc[a][t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[a][t] = mfma_bf16(af[0], bfr[t][0], acc[a][t]);
    }
  };
  // Step `buf` while the next step (register set `set`) is split into the
  // other buffer.  Without IL the compiler issues the whole split, then the
  // MFMAs (the fragment reads follow the LDS writes, which may alias them).
  // With IL the reads come first and the MFMAs are spread one per group of
  // VALU instructions, so the matrix pipe runs while the same wave splits;
  // it measured faster for K = 768 and slower for K = 3072 and at 256 x 256.
  auto half = [&](int buf, int set) {
    Frags f;
    if constexpr (IL) {
      frags(buf, f);
      lstore(1 - buf, set);
      mma(f);
      constexpr int NMF = TA * 2 * 6;
      constexpr int NVAL = (OA + OB) * 44 / NMF + 1;
      __builtin_amdgcn_sched_group_barrier(0x100, 6 + 3 * TA, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < NMF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, NVAL, 0);  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x200, 3 * (OA + OB), 0);  // DS writes
    } else {
      lstore(1 - buf, set);
      step(buf);
    }
  };

  // Steps past the end load zeros (k >= K), so the pipeline needs no tail
  // cases beyond skipping the last stores.
  const int nk = (K + BK - 1) / BK;
  gload(0, 0);
  gload(BK, 1);
  lstore(0, 0);
  __syncthreads();
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    // Step kt (buffer 0, register set 1 holds step kt + 1), then kt + 1.
    // Scheduling barriers keep each half's instructions in its half: the
    // prefetch is issued first, and nothing that reads its registers moves
    // up next to it (which would make the half wait for it).
    __builtin_amdgcn_sched_barrier(0);
    gload((kt + 2) * BK, 0);
    __builtin_amdgcn_sched_barrier(0);
    half(0, 1);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    gload((kt + 3) * BK, 1);
    __builtin_amdgcn_sched_barrier(0);
    half(1, 0);
    __syncthreads();
  }
  __builtin_amdgcn_sched_barrier(0);
  if (kt < nk) step(0);  // odd step count: the last step sits in buffer 0

#pragma unroll
  for (int a = 0; a < TA; ++a) {
    float v0[16], v1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      v0[r] = acc[a][0][r];
      v1[r] = acc[a][1][r];
    }
    epi_tile<EPI>(p, M, N, m0 + wm * (32 * TA) + a * 32, n0 + wn * 64 + 2 * j, v0, v1);
    }
}

// C[M,N] = A[M,K] B[K,N] in fp32 accuracy on v_mfma_f32_32x32x16_f16.  Each
// fp32 element enters LDS as two fp16 terms (split2_f16: x = hi + 2^-11 lo,
// to within 2^-22 |x|): A is split while it is staged, the weights once, into
// fp16 planes (p.bp16, k_split_weights_f16), so their staging is a plain
// copy.  A product takes three MFMAs: hi.hi into one accumulator, hi.lo +
// lo.hi into a second, summed as acc + 2^-11 acc' at the end; the dropped
// lo.lo term is below 2^-22 |a b|.  So a product costs 3 x 32 MFMA cycles per
// 16 k (6 x 32 on k_gemm_x6) and four LDS fragments (six).  An operand beyond
// fp16's range (|x| >= 65520) becomes an infinite hi, which makes every sum
// it enters infinite or NaN: a block with a non-finite result sets
// *p.range_flag, and the caller recomputes on the fp32 kernels (non-finite
// inputs flag too, and come out the same there).
//
// Block tile BM x BN, BK = 32, waves WM (rows) x WN (columns), each owning
// (BM / WM) x 64 as TA x 2 MFMA tiles.  Staging reads whole 128-byte lines:
// piece f of a step is row f / 8, bytes 16 (f % 8) .. + 15 of that row's
// step, so eight consecutive lanes read one row's line (loads that scatter
// a wave over 32 rows, as in k_gemm_x6, ran at half the speed: the vector
// cache serves a wave's lines one by one).  A B row's 128 bytes are the hi
// and lo planes of its four k-octets, at the byte offset of the same k in
// an fp32 [N, K] matrix.  LDS holds both planes of both operands k-contiguous
// (rows of 32 k padded to 80 bytes: 16-byte fragment reads of 8 consecutive
// rows hit distinct banks), double buffered; the global loads of step s + 2
// are issued before step s + 1 is stored.  K % 8 == 0.
template <int EPI, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN, 2) void k_gemm_h3(GemmParams p) {
  constexpr int BK = 32, LD = BK + 8, NT = 64 * WM * WN, NU = BK / 16;
  constexpr int TA = BM / WM / 32;
  static_assert(BN == 64 * WN && BM % (32 * WM) == 0, "wave tiles are (32 TA) x 64");
  constexpr int PR = BK / 4;  // 16-byte pieces per row and step
  constexpr int FA = PR * BM / NT, FB = PR * BN / NT;
  static_assert(FA >= 1 && FB >= 1 && FA * NT == PR * BM && FB * NT == PR * BN,
                "every thread stages whole pieces of both operands");
  __shared__ __align__(16) uint16_t As[2][2][BM][LD];
  __shared__ __align__(16) uint16_t Bs[2][2][BN][LD];

  const int M = p.M, N = p.N, K = p.K;
  // Each XCD takes a contiguous run of tiles (see k_gemm_bf16).
  int id = blockIdx.x + gridDim.x * blockIdx.y;
  const int per_xcd = (int)(gridDim.x * gridDim.y) / 8;
  if (id < per_xcd * 8) id = (id % 8) * per_xcd + id / 8;
  const int m0 = (id / gridDim.x) * BM, n0 = (id % gridDim.x) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int j = lane & 31, h = lane >> 5;

  // Loads go through buffer resources bounded to the block's rows of A and
  // of the planes: pieces past M or N fall outside them, pieces past K get
  // an offset outside them, and the hardware returns zeros for both.  B's
  // LDS row L = 64 g + 32 t + jj holds column 64 g + 2 jj + t of the block
  // (lane j of column tile t then reads column 2j + t: adjacent column pairs
  // for the paired epilogues).
  float4 ra[2][FA], rb[2][FB];
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.a + (size_t)m0 * K), (short)0, min(M - m0, BM) * K * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.bp16 + (size_t)n0 * K * 2), (short)0, min(N - n0, BN) * K * 4,
      0x00020000);
  auto ld4 = [](__amdgpu_buffer_rsrc_t rs, uint32_t vo) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vo, 0, 0));
    return make_float4(v.x, v.y, v.z, v.w);
  };
  auto bcol = [](int L) { return (L & ~63) | ((L & 31) << 1) | ((L >> 5) & 1); };
  auto gload = [&](int k0, int set) {
#pragma unroll
    for (int i = 0; i < FA; ++i) {
      const int f = tid + NT * i, r = f / PR, q = f % PR;
      const uint32_t vo = k0 + 4 * q < K ? (uint32_t)(r * K + k0 + 4 * q) * 4u : 0x80000000u;
      ra[set][i] = ld4(rsa, vo);
    }
#pragma unroll
    for (int i = 0; i < FB; ++i) {
      // Piece q of a B row: plane q % 2 of k-octet q / 2.
      const int f = tid + NT * i, L = f / PR, q = f % PR;
      const uint32_t vo =
          k0 + 8 * (q >> 1) < K ? (uint32_t)(bcol(L) * K + k0) * 4u + 16u * q : 0x80000000u;
      rb[set][i] = ld4(rsb, vo);
    }
  };
  auto lstore = [&](int buf, int set) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < FA; ++i) {
      const int f = tid + NT * i, r = f / PR, q = f % PR;
      const float4 x = ra[set][i];
      const uint32_t h0 = cvt_pk_f16(x.x, x.y), h1 = cvt_pk_f16(x.z, x.w);
      const h2 a0 = __builtin_bit_cast(h2, h0), a1 = __builtin_bit_cast(h2, h1);
      const uint32_t l0 = cvt_pk_f16((x.x - (float)a0[0]) * 2048.f, (x.y - (float)a0[1]) * 2048.f);
      const uint32_t l1 = cvt_pk_f16((x.z - (float)a1[0]) * 2048.f, (x.w - (float)a1[1]) * 2048.f);
      *reinterpret_cast<uint2*>(&As[buf][0][r][4 * q]) = make_uint2(h0, h1);
      *reinterpret_cast<uint2*>(&As[buf][1][r][4 * q]) = make_uint2(l0, l1);
    }
#pragma unroll
    for (int i = 0; i < FB; ++i) {
      const int f = tid + NT * i, L = f / PR, q = f % PR;
      *reinterpret_cast<float4*>(&Bs[buf][q & 1][L][8 * (q >> 1)]) = rb[set][i];
    }
  };

  f32x16 acc[TA][2], cor[TA][2];
#pragma unroll
  for (int a = 0; a < TA; ++a)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      acc[a][t] = zero16();
      cor[a][t] = zero16();
    }
  // One step: fragments of both 16-k halves of buffer `buf`, then the MFMAs.
  auto step = [&](int buf) {
    f16x8 f[NU][2 + TA][2];  // [0..1]: B column tiles, [2 + a]: A row tiles
#pragma unroll
    for (int u = 0; u < NU; ++u) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
          f[u][t][pl] = f16x8_of(*reinterpret_cast<const uint4*>(
              &Bs[buf][pl][wn * 64 + t * 32 + j][16 * u + 8 * h]));
#pragma unroll
      for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
          f[u][2 + a][pl] = f16x8_of(*reinterpret_cast<const uint4*>(
              &As[buf][pl][wm * (32 * TA) + a * 32 + j][16 * u + 8 * h]));
    }
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int a = 0; a < TA; ++a) {
#pragma unroll
        for (int t = 0; t < 2; ++t) cor[a][t] = mfma_f16(f[u][2 + a][1], f[u][t][0], cor[a][t]);
#pragma unroll
        for (int t = 0; t < 2; ++t) cor[a][t] = mfma_f16(f[u][2 + a][0], f[u][t][1], cor[a][t]);
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[a][t] = mfma_f16(f[u][2 + a][0], f[u][t][0], acc[a][t]);
      }
  };

  // Step s computes on LDS buffer s % 2 after storing step s + 1 (register
  // set (s + 1) % 2, loaded a step earlier) into the other buffer and issuing
  // the loads of step s + 2 into set s % 2.  Steps past the end load zeros.
  const int nk = (K + BK - 1) / BK;
  gload(0, 0);
  gload(BK, 1);
  lstore(0, 0);
  __syncthreads();
  auto stepk = [&](int s, int buf) {
    __builtin_amdgcn_sched_barrier(0);
    gload((s + 2) * BK, buf);
    __builtin_amdgcn_sched_barrier(0);
    lstore(1 - buf, 1 - buf);
    step(buf);
    __syncthreads();
  };
  int s = 0;
  for (; s + 2 <= nk; s += 2) {
    stepk(s, 0);
    stepk(s + 1, 1);
  }
  if (s < nk) stepk(s, 0);

  bool finite = true;
#pragma unroll
  for (int a = 0; a < TA; ++a) {
    float v0[16], v1[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      v0[r] = acc[a][0][r] + cor[a][0][r] * 0x1p-11f;
      v1[r] = acc[a][1][r] + cor[a][1][r] * 0x1p-11f;
      finite = finite && __builtin_isfinite(v0[r]) && __builtin_isfinite(v1[r]);
    }
    epi_tile<EPI>(p, M, N, m0 + wm * (32 * TA) + a * 32, n0 + wn * 64 + 2 * j, v0, v1);
    }
  if (!finite) *p.range_flag = 1;
}

// Causal flash attention with bfloat16 MFMAs (head_dim 64 or 128), the
// structure of k_flash_mfma: block = 4 waves x 32 queries, keys in blocks of
// 32, S^T = K Q^T per wave so each lane owns one query.  Q, K and V are
// rounded to bfloat16 (Q once into registers, K row-major and V transposed
// into LDS per key block); P^T feeds O^T += V^T P^T from the accumulator
// registers: MFMA 0 of a 32-key block takes accumulator entries 0..7 of each
// lane (keys acc_row(0..7, h)), MFMA 1 entries 8..15, and the V^T fragment
// reads the same keys, one 16-byte run (V^T keys are stored with bits 2 and
// 3 of their index swapped).  Softmax statistics are fp32; the
// output is bfloat16.
template <int HD>
__global__ __launch_bounds__(256, 2) void k_flash_bf16(FlashParams p) {
  constexpr int QB = 128, KB = 32, NT = HD / 32, NQ = HD / 16;
  constexpr int KP = HD + 8;   // K row stride (bf16)
  constexpr int VP = KB + 8;   // V^T row stride (bf16)
  constexpr int CPR = HD / 4;  // float4 per K/V row
  constexpr int KPT = KB * CPR / 256;  // consecutive keys staged per thread
  static_assert(KPT == 2 || KPT == 4, "staging covers 2 or 4 keys per thread");
  constexpr int KV_BYTES = (KB * KP + HD * VP) * 2;
  constexpr int O_BYTES = 4 * 32 * 33 * 4;
  __shared__ __align__(16) unsigned char lds[KV_BYTES > O_BYTES ? KV_BYTES : O_BYTES];
  uint16_t (*Ks)[KP] = reinterpret_cast<uint16_t (*)[KP]>(lds);
  uint16_t (*Vt)[VP] = reinterpret_cast<uint16_t (*)[VP]>(lds + KB * KP * 2);

  const int qblk = gridDim.z - 1 - blockIdx.z, hh = blockIdx.x, b = blockIdx.y;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return;
  const int S = fs.S, d = fs.d;
  // Scores in the log2 domain: exp(scale x - m) = exp2(scale log2(e) x - m').
  const float qscale = fs.scale * 1.44269504088896341f;
  const int q0 = qblk * QB;
  if (q0 >= S) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  const float* qp = p.q + fs.q + hh * HD;
  const float* kp = p.k + fs.kv + hh * HD;
  const float* vp = p.v + fs.kv + hh * HD;

  const int qi = q0 + wave * 32 + j;
  bf16x8 qf[NQ];  // dims 16 s + 8 h .. + 7 of query qi
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + 8 * h;
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      qf[s] = bf16x8_of(*reinterpret_cast<const float4*>(qr + 16 * s),
                        *reinterpret_cast<const float4*>(qr + 16 * s + 4));
  }
  f32x16 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = zero16();
  float mrow = -INFINITY, lrow = 0.f;

  const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
  const int kend = min(S, q0 + QB);
  const int nkb = (kend + KB - 1) / KB;

  // Staging: thread t takes dims 4 (t % CPR) .. + 3 of KPT consecutive keys
  // from KPT (t / CPR), so K rows and V^T rows are both written 4 or 8 bytes
  // at a time.
  const int sc = (tid % CPR) * 4, sk = (tid / CPR) * KPT;
  float4 kr[KPT], vr[KPT];
  auto load_kv = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int key = kb * KB + sk + i;
      const size_t off = (size_t)(key < S ? key : 0) * d + sc;
      kr[i] = *reinterpret_cast<const float4*>(kp + off);
      vr[i] = *reinterpret_cast<const float4*>(vp + off);
    }
  };
  load_kv(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      *reinterpret_cast<uint2*>(&Ks[sk + i][sc]) =
          make_uint2(pack_bf16x2(kr[i].x, kr[i].y), pack_bf16x2(kr[i].z, kr[i].w));
    // V^T keys at their permuted positions (bits 2 and 3 of the key swapped,
    // so the eight keys an MFMA lane takes are one 16-byte run).
    const int vk = (sk & ~12) | ((sk >> 1) & 4) | ((sk << 1) & 8);
    if constexpr (KPT == 4) {
      *reinterpret_cast<uint2*>(&Vt[sc][vk]) =
          make_uint2(pack_bf16x2(vr[0].x, vr[1].x), pack_bf16x2(vr[2].x, vr[3].x));
      *reinterpret_cast<uint2*>(&Vt[sc + 1][vk]) =
          make_uint2(pack_bf16x2(vr[0].y, vr[1].y), pack_bf16x2(vr[2].y, vr[3].y));
      *reinterpret_cast<uint2*>(&Vt[sc + 2][vk]) =
          make_uint2(pack_bf16x2(vr[0].z, vr[1].z), pack_bf16x2(vr[2].z, vr[3].z));
      *reinterpret_cast<uint2*>(&Vt[sc + 3][vk]) =
          make_uint2(pack_bf16x2(vr[0].w, vr[1].w), pack_bf16x2(vr[2].w, vr[3].w));
    } else {
      *reinterpret_cast<uint32_t*>(&Vt[sc][vk]) = pack_bf16x2(vr[0].x, vr[1].x);
      *reinterpret_cast<uint32_t*>(&Vt[sc + 1][vk]) = pack_bf16x2(vr[0].y, vr[1].y);
      *reinterpret_cast<uint32_t*>(&Vt[sc + 2][vk]) = pack_bf16x2(vr[0].z, vr[1].z);
      *reinterpret_cast<uint32_t*>(&Vt[sc + 3][vk]) = pack_bf16x2(vr[0].w, vr[1].w);
    }
    __syncthreads();
    load_kv(kb + 1);  // rows past S read row 0: harmless, never used
    const int j0 = kb * KB;
    if (j0 > wave_qmax) continue;

    f32x16 st = zero16();
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      st = mfma_bf16(bf16x8_of(*reinterpret_cast<const uint4*>(&Ks[j][16 * s + 8 * h])), qf[s],
                     st);

    // Keys above a query (the diagonal block) or past S are masked.
    const bool masked = j0 + KB - 1 > wave_qmin || j0 + KB > S;
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * qscale;
      if (masked) {
        const int key = j0 + acc_row(r, h);
        if (key > qi || key >= S) v = -INFINITY;
      }
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float mnew = fmaxf(mrow, pm);  // finite: key 0 is in every query's range
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(mrow - mnew);  // 0 on the first block
    lrow = lrow * corr + ps;
    if (__any(mnew != mrow)) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    }
    mrow = mnew;
    const bf16x8 p0 = bf16x8_of(make_float4(st[0], st[1], st[2], st[3]),
                                make_float4(st[4], st[5], st[6], st[7]));
    const bf16x8 p1 = bf16x8_of(make_float4(st[8], st[9], st[10], st[11]),
                                make_float4(st[12], st[13], st[14], st[15]));
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint16_t* vrow = Vt[32 * t + j];
      o[t] = mfma_bf16(bf16x8_of(*reinterpret_cast<const uint4*>(vrow + 8 * h)), p0, o[t]);
      o[t] = mfma_bf16(bf16x8_of(*reinterpret_cast<const uint4*>(vrow + 16 + 8 * h)), p1, o[t]);
    }
  }

  const float inv = 1.0f / lrow;
  float (*Os)[33] = reinterpret_cast<float (*)[33]>(lds + wave * 32 * 33 * 4);
  uint16_t* op = p.o16 + fs.o + hh * HD;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) Os[j][acc_row(r, h)] = o[t][r] * inv;
    __syncthreads();
    for (int e = lane; e < 32 * 16; e += 64) {
      const int r = e >> 4, c = (e & 15) * 2;
      const int qrow = q0 + wave * 32 + r;
      if (qrow < S)
        *reinterpret_cast<uint32_t*>(op + (size_t)qrow * d + 32 * t + c) =
            pack_bf16x2(Os[r][c], Os[r][c + 1]);
    }
  }
}

// Causal flash attention (head_dim 64 or 128) in fp32 accuracy on
// v_mfma_f32_32x32x16_bf16: k_flash_bf16's structure (block = 4 waves x 32
// queries, 32-key blocks, S^T = K Q^T so each lane owns one query, P^T fed
// from the accumulators) with every fp32 operand split exactly into three
// bfloat16 terms (split3_rne): Q once into registers, K and V^T into three
// LDS planes per key block, the probabilities P per key block.  Both
// contractions accumulate the six products down to 2^-16 of each full
// product (as k_gemm_x6), so scores and outputs carry fp32-level error.
// Softmax statistics, the output and lse are fp32, as in k_flash_mfma,
// whose per-shader meta handling (row_offset) this follows.  UA: the head
// size is not a multiple of 4, so head rows lack 16-byte alignment and are
// loaded element by element (a separate instantiation: the aligned kernels
// keep their code).
// LDS of a 128-query tile: K's KPLANES planes and V^T's three, or the four
// waves' 32 x 33 output transposes.
template <int HD, int KPLANES>
constexpr int flash_q128_lds() {
  constexpr int KB = 32, KV_BYTES = (KPLANES * KB * (HD + 8) + 3 * HD * (KB + 8)) * 2;
  constexpr int O_BYTES = 4 * 32 * 33 * 4;
  return KV_BYTES > O_BYTES ? KV_BYTES : O_BYTES;
}

template <int HD, bool UA>
__device__ __forceinline__ void flash_x6_tile(const FlashParams& p, unsigned char* lds) {
  constexpr int QB = 128, KB = 32, NT = HD / 32, NQ = HD / 16;
  constexpr int KP = HD + 8;   // K row stride (bf16)
  constexpr int VP = KB + 8;   // V^T row stride (bf16)
  constexpr int CPR = HD / 4;  // float4 per K/V row
  constexpr int KPT = KB * CPR / 256;  // consecutive keys staged per thread
  static_assert(KPT == 2 || KPT == 4, "staging covers 2 or 4 keys per thread");
  constexpr int K_PLANE = KB * KP, V_PLANE = HD * VP;  // bf16 elements
  auto Ks = [&](int pl) { return reinterpret_cast<uint16_t (*)[KP]>(lds) + pl * KB; };
  auto Vt = [&](int pl) {
    return reinterpret_cast<uint16_t (*)[VP]>(lds + 3 * K_PLANE * 2) + pl * HD;
  };

  const int qblk = gridDim.z - 1 - blockIdx.z, hh = blockIdx.x, b = blockIdx.y;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return;
  const int S = fs.S, d = fs.d, hd = p.hd;  // head size hd <= HD
  const float scale = fs.scale;
  const int H = d / hd;
  // Scores in the log2 domain: exp(scale x - m) = exp2(scale log2(e) x - m').
  const float qscale = scale * 1.44269504088896341f;
  const int q0 = qblk * QB;
  if (q0 >= S) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  const float* qp = p.q + fs.q + hh * hd;
  const float* kp = p.k + fs.kv + hh * hd;
  const float* vp = p.v + fs.kv + hh * hd;
  // Columns past the head size read as zero.  A head size that is not a
  // multiple of 4 (UA) leaves head rows without 16-byte alignment, and its
  // last quad reaches into the next head: element by element.
  auto col4 = [hd](const float* src, int c) {
    if constexpr (!UA)
      return c < hd ? *reinterpret_cast<const float4*>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
    return make_float4(c < hd ? src[0] : 0.f, c + 1 < hd ? src[1] : 0.f,
                       c + 2 < hd ? src[2] : 0.f, c + 3 < hd ? src[3] : 0.f);
  };

  const int qi = q0 + wave * 32 + j;
  uint4 qf[3][NQ];  // the three planes of dims 16 s + 8 h .. + 7 of query qi
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + 8 * h;
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      split3_rne(col4(qr + 16 * s, 16 * s + 8 * h), col4(qr + 16 * s + 4, 16 * s + 8 * h + 4),
                 qf[0][s], qf[1][s], qf[2][s]);
  }
  f32x16 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = zero16();
  float mrow = -INFINITY, lrow = 0.f;

  const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
  const int kend = min(S, q0 + QB);
  const int nkb = (kend + KB - 1) / KB;

  // Staging: thread t takes dims 4 (t % CPR) .. + 3 of KPT consecutive keys
  // from KPT (t / CPR), so K rows and V^T rows are both written 4 or 8 bytes
  // at a time per plane.
  const int sc = (tid % CPR) * 4, sk = (tid / CPR) * KPT;
  float4 kr[KPT], vr[KPT];
  auto load_kv = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int key = kb * KB + sk + i;
      const size_t off = (size_t)(key < S ? key : 0) * d + sc;
      kr[i] = col4(kp + off, sc);
      vr[i] = col4(vp + off, sc);
    }
  };
  // Three bfloat16 terms of a and b, packed as pairs (a_pl, b_pl).
  auto split_pair = [](float a, float b, uint32_t (&t)[3]) {
    t[0] = cvt_pk_bf16(a, b);
    const float ra = a - __uint_as_float(t[0] << 16), rb = b - __uint_as_float(t[0] & 0xFFFF0000u);
    t[1] = cvt_pk_bf16(ra, rb);
    t[2] = cvt_pk_bf16(ra - __uint_as_float(t[1] << 16), rb - __uint_as_float(t[1] & 0xFFFF0000u));
  };
  load_kv(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      uint32_t lo[3], hi[3];
      split_pair(kr[i].x, kr[i].y, lo);
      split_pair(kr[i].z, kr[i].w, hi);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        *reinterpret_cast<uint2*>(&Ks(pl)[sk + i][sc]) = make_uint2(lo[pl], hi[pl]);
    }
    // V^T: dim row sc + c, keys sk .. sk + KPT - 1 at their permuted
    // positions (bits 2 and 3 of the key swapped, so the eight keys an MFMA
    // lane takes, acc_row(8 half .. 8 half + 7, h), are one 16-byte run).
    const int vk = (sk & ~12) | ((sk >> 1) & 4) | ((sk << 1) & 8);
    const float vc[4][4] = {
#define AKH_VCOL(f) {vr[0].f, vr[1].f, KPT == 4 ? vr[KPT - 2].f : 0.f, KPT == 4 ? vr[KPT - 1].f : 0.f}
        AKH_VCOL(x), AKH_VCOL(y), AKH_VCOL(z), AKH_VCOL(w)
#undef AKH_VCOL
    };
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t t01[3], t23[3];
      split_pair(vc[c][0], vc[c][1], t01);
      if constexpr (KPT == 4) {
        split_pair(vc[c][2], vc[c][3], t23);
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint2*>(&Vt(pl)[sc + c][vk]) = make_uint2(t01[pl], t23[pl]);
      } else {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint32_t*>(&Vt(pl)[sc + c][vk]) = t01[pl];
      }
    }
    __syncthreads();
    load_kv(kb + 1);  // rows past S read row 0: harmless, never used
    const int j0 = kb * KB;
    if (j0 > wave_qmax) continue;

    f32x16 st = zero16();
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      bf16x8 kf[3];
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        kf[pl] = bf16x8_of(*reinterpret_cast<const uint4*>(&Ks(pl)[j][16 * s + 8 * h]));
      // Smallest terms first.
      st = mfma_bf16(kf[2], bf16x8_of(qf[0][s]), st);
      st = mfma_bf16(kf[1], bf16x8_of(qf[1][s]), st);
      st = mfma_bf16(kf[0], bf16x8_of(qf[2][s]), st);
      st = mfma_bf16(kf[1], bf16x8_of(qf[0][s]), st);
      st = mfma_bf16(kf[0], bf16x8_of(qf[1][s]), st);
      st = mfma_bf16(kf[0], bf16x8_of(qf[0][s]), st);
    }

    // Keys above a query (the diagonal block) or past S are masked.
    const bool masked = j0 + KB - 1 > wave_qmin || j0 + KB > S;
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * qscale;
      if (masked) {
        const int key = j0 + acc_row(r, h);
        if (key > qi || key >= S) v = -INFINITY;
      }
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float mnew = fmaxf(mrow, pm);  // finite: key 0 is in every query's range
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(mrow - mnew);  // 0 on the first block
    lrow = lrow * corr + ps;
    if (__any(mnew != mrow)) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    }
    mrow = mnew;
    // P^T planes: MFMA 0 of the block takes entries 0..7 of each lane (keys
    // acc_row(0..7, h)), MFMA 1 entries 8..15.
    uint4 pf[2][3];
#pragma unroll
    for (int half = 0; half < 2; ++half)
      split3_rne(make_float4(st[8 * half], st[8 * half + 1], st[8 * half + 2], st[8 * half + 3]),
                 make_float4(st[8 * half + 4], st[8 * half + 5], st[8 * half + 6],
                             st[8 * half + 7]),
                 pf[half][0], pf[half][1], pf[half][2]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // V^T rows of the same keys: one 16-byte run at their permuted positions.
        bf16x8 vf[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          vf[pl] = bf16x8_of(
              *reinterpret_cast<const uint4*>(Vt(pl)[32 * t + j] + 16 * half + 8 * h));
        o[t] = mfma_bf16(vf[2], bf16x8_of(pf[half][0]), o[t]);
        o[t] = mfma_bf16(vf[1], bf16x8_of(pf[half][1]), o[t]);
        o[t] = mfma_bf16(vf[0], bf16x8_of(pf[half][2]), o[t]);
        o[t] = mfma_bf16(vf[1], bf16x8_of(pf[half][0]), o[t]);
        o[t] = mfma_bf16(vf[0], bf16x8_of(pf[half][1]), o[t]);
        o[t] = mfma_bf16(vf[0], bf16x8_of(pf[half][0]), o[t]);
      }
    }
  }

  // O^T (rows = dims) -> LDS, one 32-dim tile at a time -> coalesced rows.
  const float inv = 1.0f / lrow;
  float (*Os)[33] = reinterpret_cast<float (*)[33]>(lds + wave * 32 * 33 * 4);
  float* op = p.o + fs.o + hh * hd;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) Os[j][acc_row(r, h)] = o[t][r] * inv;
    __syncthreads();
    for (int e = lane; e < 32 * 32; e += 64) {
      const int r = e >> 5, c = e & 31;
      const int qrow = q0 + wave * 32 + r;
      if (qrow < S && 32 * t + c < hd) op[(size_t)qrow * d + 32 * t + c] = Os[r][c];
    }
  }
  if (p.lse && h == 0 && qi < S)  // max + ln(sum), back in natural units
    p.lse[fs.l + (size_t)qi * H + hh] =
        mrow * 0.69314718055994531f + logf(lrow);
}

template <int HD, bool UA = false>
__global__ __launch_bounds__(256, 2) void k_flash_x6(FlashParams p) {
  __shared__ __align__(16) unsigned char lds[flash_q128_lds<HD, 3>()];
  flash_x6_tile<HD, UA>(p, lds);
}

// Causal flash attention in fp32 accuracy on fp16 MFMAs, the structure of
// k_flash_x6 with two-term fp16 splits (split2_f16: x = hi + 2^-11 lo) and
// three products per contraction instead of six.  Scores: Q and K split,
// hi.hi in one accumulator and the two cross terms in another (the
// k_gemm_h3 scheme).  Output: P split the same way and V^T staged as hi, the
// unscaled remainder v - hi and hi 2^-11, so one accumulator takes
// p0 v0 + p0 v1 + p1 (2^-11 v0): the remainder and the scaled hi can be
// subnormal, but each loses at most 2^-25 absolute, weighted by the
// probabilities (sum 1).  Output, lse and softmax statistics stay fp32.  A
// non-finite output (an operand beyond fp16's range) sets *p.range_flag.
// FALLBACK: a tile with a non-finite output stores nothing and returns false
// (the caller recomputes it); otherwise it sets *p.range_flag, if given, and
// stores.
template <int HD, bool FALLBACK>
__device__ __forceinline__ bool flash_h3_tile(const FlashParams& p, unsigned char* lds) {
  constexpr int QB = 128, KB = 32, NT = HD / 32, NQ = HD / 16;
  constexpr int KP = HD + 8;   // K row stride (fp16)
  constexpr int VP = KB + 8;   // V^T row stride (fp16)
  constexpr int CPR = HD / 4;  // float4 per K/V row
  constexpr int KPT = KB * CPR / 256;  // consecutive keys staged per thread
  static_assert(KPT == 2 || KPT == 4, "staging covers 2 or 4 keys per thread");
  constexpr int K_PLANE = KB * KP, V_PLANE = HD * VP;  // fp16 elements
  auto Ks = [&](int pl) { return reinterpret_cast<uint16_t (*)[KP]>(lds) + pl * KB; };
  auto Vt = [&](int pl) {
    return reinterpret_cast<uint16_t (*)[VP]>(lds + 2 * K_PLANE * 2) + pl * HD;
  };

  const int qblk = gridDim.z - 1 - blockIdx.z, hh = blockIdx.x, b = blockIdx.y;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return true;
  const int S = fs.S, d = fs.d, hd = p.hd;  // head size hd <= HD
  const float scale = fs.scale;
  const int H = d / hd;
  // Scores in the log2 domain: exp(scale x - m) = exp2(scale log2(e) x - m').
  const float qscale = scale * 1.44269504088896341f;
  const int q0 = qblk * QB;
  if (q0 >= S) return true;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  const float* qp = p.q + fs.q + hh * hd;
  const float* kp = p.k + fs.kv + hh * hd;
  const float* vp = p.v + fs.kv + hh * hd;
  // Columns past the head size (hd a multiple of 4 below HD) read as zero.
  auto col4 = [hd](const float* src, int c) {
    return c < hd ? *reinterpret_cast<const float4*>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
  };

  const int qi = q0 + wave * 32 + j;
  uint4 qf[2][NQ];  // hi and scaled lo of dims 16 s + 8 h .. + 7 of query qi
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + 8 * h;
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      split2_f16(col4(qr + 16 * s, 16 * s + 8 * h), col4(qr + 16 * s + 4, 16 * s + 8 * h + 4),
                 qf[0][s], qf[1][s]);
  }
  f32x16 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = zero16();
  float mrow = -INFINITY, lrow = 0.f;

  const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
  const int kend = min(S, q0 + QB);
  const int nkb = (kend + KB - 1) / KB;

  // Staging: thread t takes dims 4 (t % CPR) .. + 3 of KPT consecutive keys
  // from KPT (t / CPR), so K rows and V^T rows are both written 4 or 8 bytes
  // at a time per plane.
  const int sc = (tid % CPR) * 4, sk = (tid / CPR) * KPT;
  float4 kr[KPT], vr[KPT];
  auto load_kv = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int key = kb * KB + sk + i;
      const size_t off = (size_t)(key < S ? key : 0) * d + sc;
      kr[i] = col4(kp + off, sc);
      vr[i] = col4(vp + off, sc);
    }
  };
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  // K: hi and scaled lo (split2_f16) of a and b, packed as pairs.
  auto split_k = [](float a, float b, uint32_t (&t)[2]) {
    t[0] = cvt_pk_f16(a, b);
    const h2 hv = __builtin_bit_cast(h2, t[0]);
    t[1] = cvt_pk_f16((a - (float)hv[0]) * 2048.f, (b - (float)hv[1]) * 2048.f);
  };
  // V: hi, the unscaled remainder, and hi 2^-11, so that with P split as
  // p0 + 2^-11 p1 one accumulator takes p0 v0 + p0 v1 + p1 (2^-11 v0).
  auto split_v = [](float a, float b, uint32_t (&t)[3]) {
    t[0] = cvt_pk_f16(a, b);
    const h2 hv = __builtin_bit_cast(h2, t[0]);
    const float ha = (float)hv[0], hb = (float)hv[1];
    t[1] = cvt_pk_f16(a - ha, b - hb);
    t[2] = cvt_pk_f16(ha * 0x1p-11f, hb * 0x1p-11f);
  };
  load_kv(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      uint32_t lo[2], hi[2];
      split_k(kr[i].x, kr[i].y, lo);
      split_k(kr[i].z, kr[i].w, hi);
#pragma unroll
      for (int pl = 0; pl < 2; ++pl)
        *reinterpret_cast<uint2*>(&Ks(pl)[sk + i][sc]) = make_uint2(lo[pl], hi[pl]);
    }
    // V^T: dim row sc + c, keys sk .. sk + KPT - 1 at their permuted
    // positions (bits 2 and 3 of the key swapped, so the eight keys an MFMA
    // lane takes, acc_row(8 half .. 8 half + 7, h), are one 16-byte run).
    const int vk = (sk & ~12) | ((sk >> 1) & 4) | ((sk << 1) & 8);
    const float vc[4][4] = {
#define AKH_VCOL(f) {vr[0].f, vr[1].f, KPT == 4 ? vr[KPT - 2].f : 0.f, KPT == 4 ? vr[KPT - 1].f : 0.f}
        AKH_VCOL(x), AKH_VCOL(y), AKH_VCOL(z), AKH_VCOL(w)
#undef AKH_VCOL
    };
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t t01[3], t23[3];
      split_v(vc[c][0], vc[c][1], t01);
      if constexpr (KPT == 4) {
        split_v(vc[c][2], vc[c][3], t23);
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint2*>(&Vt(pl)[sc + c][vk]) = make_uint2(t01[pl], t23[pl]);
      } else {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint32_t*>(&Vt(pl)[sc + c][vk]) = t01[pl];
      }
    }
    __syncthreads();
    load_kv(kb + 1);  // rows past S read row 0: harmless, never used
    const int j0 = kb * KB;
    if (j0 > wave_qmax) continue;

    // Scores: hi.hi in st, the cross terms in sc, st + 2^-11 sc.
    f32x16 st = zero16(), scr = zero16();
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      f16x8 kf[2];
#pragma unroll
      for (int pl = 0; pl < 2; ++pl)
        kf[pl] = f16x8_of(*reinterpret_cast<const uint4*>(&Ks(pl)[j][16 * s + 8 * h]));
      scr = mfma_f16(kf[1], f16x8_of(qf[0][s]), scr);
      scr = mfma_f16(kf[0], f16x8_of(qf[1][s]), scr);
      st = mfma_f16(kf[0], f16x8_of(qf[0][s]), st);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] += scr[r] * 0x1p-11f;

    // Keys above a query (the diagonal block) or past S are masked.
    const bool masked = j0 + KB - 1 > wave_qmin || j0 + KB > S;
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * qscale;
      if (masked) {
        const int key = j0 + acc_row(r, h);
        if (key > qi || key >= S) v = -INFINITY;
      }
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float mnew = fmaxf(mrow, pm);  // finite: key 0 is in every query's range
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(mrow - mnew);  // 0 on the first block
    lrow = lrow * corr + ps;
    if (__any(mnew != mrow)) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    }
    mrow = mnew;
    // P^T planes: MFMA 0 of the block takes entries 0..7 of each lane (keys
    // acc_row(0..7, h)), MFMA 1 entries 8..15.
    uint4 pf[2][2];
#pragma unroll
    for (int half = 0; half < 2; ++half)
      split2_f16(make_float4(st[8 * half], st[8 * half + 1], st[8 * half + 2], st[8 * half + 3]),
                 make_float4(st[8 * half + 4], st[8 * half + 5], st[8 * half + 6],
                             st[8 * half + 7]),
                 pf[half][0], pf[half][1]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // V^T rows of the same keys: one 16-byte run at their permuted positions.
        f16x8 vf[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
          vf[pl] = f16x8_of(
              *reinterpret_cast<const uint4*>(Vt(pl)[32 * t + j] + 16 * half + 8 * h));
        }
        // Smallest terms first: p1 (2^-11 v0), p0 v1, then p0 v0.
        o[t] = mfma_f16(vf[2], f16x8_of(pf[half][1]), o[t]);
        o[t] = mfma_f16(vf[1], f16x8_of(pf[half][0]), o[t]);
        o[t] = mfma_f16(vf[0], f16x8_of(pf[half][0]), o[t]);
      }
    }
  }

  // O^T (rows = dims) -> LDS, one 32-dim tile at a time -> coalesced rows.
  const float inv = 1.0f / lrow;
  // An operand beyond fp16's range (|x| >= 65520) makes the output or the
  // softmax state non-finite: give the tile back to the caller (FALLBACK),
  // or flag it for the caller's fp32 rerun.
  {
    bool finite = __builtin_isfinite(inv);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) finite = finite && __builtin_isfinite(o[t][r]);
    if constexpr (FALLBACK) {
      if (__syncthreads_or(!finite)) return false;
    } else if (!finite && p.range_flag) {
      *p.range_flag = 1;
    }
  }
  float (*Os)[33] = reinterpret_cast<float (*)[33]>(lds + wave * 32 * 33 * 4);
  float* op = p.o + fs.o + hh * hd;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) Os[j][acc_row(r, h)] = o[t][r] * inv;
    __syncthreads();
    for (int e = lane; e < 32 * 32; e += 64) {
      const int r = e >> 5, c = e & 31;
      const int qrow = q0 + wave * 32 + r;
      if (qrow < S && 32 * t + c < hd) op[(size_t)qrow * d + 32 * t + c] = Os[r][c];
    }
  }
  if (p.lse && h == 0 && qi < S)  // max + ln(sum), back in natural units
    p.lse[fs.l + (size_t)qi * H + hh] =
        mrow * 0.69314718055994531f + logf(lrow);
  return true;
}

template <int HD>
__global__ __launch_bounds__(256, 2) void k_flash_h3(FlashParams p) {
  __shared__ __align__(16) unsigned char lds[flash_q128_lds<HD, 2>()];
  flash_h3_tile<HD, false>(p, lds);
}

// The 128-query tile on split-fp16 products, recomputed on split-bf16
// products when an operand is beyond fp16's range (a non-finite output):
// fp32 accuracy for any finite input, with no flag for the caller to read.
// Head size 64 only: at 128 the two paths in one kernel spill registers.
template <int HD>
__global__ __launch_bounds__(256, 2) void k_flash_h3x(FlashParams p) {
  static_assert(HD == 64, "k_flash_x6 serves head size 128");
  constexpr int L2 = flash_q128_lds<HD, 2>(), L3 = flash_q128_lds<HD, 3>();
  __shared__ __align__(16) unsigned char lds[L2 > L3 ? L2 : L3];
  if (!flash_h3_tile<HD, true>(p, lds)) {
    __syncthreads();
    flash_x6_tile<HD, false>(p, lds);
  }
}

// k_flash_x6 for grids too small to fill the part (a single sequence's
// FLASH_ATTENTION node): one 32-query tile per block, its key blocks dealt
// round-robin to the block's NW waves.  Each wave stages its own key block
// in a private LDS region and keeps its own softmax state, so the key loop
// has no block barrier; at the end the partial states merge through LDS:
// M = max m_w, O = sum O_w 2^(m_w - M) / sum l_w 2^(m_w - M).  A wave stages
// K's three planes, takes the scores, then stages V^T's three planes in the
// same region for the output products, so a region holds one of the two
// (HD 64: 15 KB, eight waves in 123 KB; HD 128: 31 KB, four waves).  The
// next key block's K rows are loaded while the wave works on this one's
// scores and its V rows while it takes this one's output.  The heaviest
// tile walks 1 / NW of the key blocks on its critical path.  Scores,
// products and statistics are those of k_flash_x6.
//
// LDS of a key-split tile: NW per-wave regions holding K's KPLANES planes or
// V^T's three (whichever is larger), or the merge's NW partial states.
template <int HD, int NW, int KPLANES>
constexpr int flash_w_lds() {
  constexpr int KB = 32, K_BYTES = KPLANES * KB * (HD + 8) * 2, V_BYTES = 3 * HD * (KB + 8) * 2;
  constexpr int W_BYTES = K_BYTES > V_BYTES ? K_BYTES : V_BYTES;
  constexpr int M_BYTES = NW * (HD * 33 + 64) * 4;
  return NW * W_BYTES > M_BYTES ? NW * W_BYTES : M_BYTES;
}

template <int HD, int NW>
__device__ __forceinline__ void flash_x6w_tile(const FlashParams& p, unsigned char* lds) {
  constexpr int KB = 32, NT = HD / 32, NQ = HD / 16;
  constexpr int KP = HD + 8, VP = KB + 8, CPR = HD / 4;
  constexpr int KPT = KB * CPR / 64;  // consecutive keys staged per lane
  static_assert(KPT == 8 || KPT == 16, "a wave stages 32 keys in runs of 8 or 16");
  constexpr int K_PLANE = KB * KP, V_PLANE = HD * VP;  // bf16 elements
  constexpr int K_BYTES = 3 * K_PLANE * 2, V_BYTES = 3 * V_PLANE * 2;
  constexpr int W_BYTES = K_BYTES > V_BYTES ? K_BYTES : V_BYTES;
  constexpr int OS = 33;                                // merge row stride

  const int qblk = gridDim.z - 1 - blockIdx.z, hh = blockIdx.x, b = blockIdx.y;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return;
  const int S = fs.S, d = fs.d;
  const float scale = fs.scale;
  const int H = d / HD;
  const float qscale = scale * 1.44269504088896341f;
  const int q0 = qblk * 32;
  if (q0 >= S) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  unsigned char* wl = lds + wave * W_BYTES;
  auto Ks = [&](int pl) { return reinterpret_cast<uint16_t (*)[KP]>(wl) + pl * KB; };
  auto Vt = [&](int pl) { return reinterpret_cast<uint16_t (*)[VP]>(wl) + pl * HD; };

  const float* qp = p.q + fs.q + hh * HD;
  const float* kp = p.k + fs.kv + hh * HD;
  const float* vp = p.v + fs.kv + hh * HD;

  const int qi = q0 + j;
  const int kend = min(S, q0 + 32);
  const int nkb = (kend + KB - 1) / KB;

  // Staging: lane l takes dims 4 (l % CPR) .. + 3 of keys KPT (l / CPR) ..
  // + KPT - 1.
  const int sc = (lane % CPR) * 4, sk = (lane / CPR) * KPT;
  float4 kr[KPT], vr[KPT];
  auto load_rows = [&](const float* src, int kb, float4 (&r)[KPT]) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int key = kb * KB + sk + i;
      r[i] = *reinterpret_cast<const float4*>(src + (size_t)(key < S ? key : 0) * d + sc);
    }
  };
  auto split_pair = [](float a, float c, uint32_t (&t)[3]) {
    t[0] = cvt_pk_bf16(a, c);
    const float ra = a - __uint_as_float(t[0] << 16), rc = c - __uint_as_float(t[0] & 0xFFFF0000u);
    t[1] = cvt_pk_bf16(ra, rc);
    t[2] = cvt_pk_bf16(ra - __uint_as_float(t[1] << 16), rc - __uint_as_float(t[1] & 0xFFFF0000u));
  };
  // The query rows, then the first key block's K and V rows, all in flight
  // before the wave waits on any of them.
  float4 qr4[2 * NQ];
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + 8 * h;
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      qr4[2 * s] = *reinterpret_cast<const float4*>(qr + 16 * s);
      qr4[2 * s + 1] = *reinterpret_cast<const float4*>(qr + 16 * s + 4);
    }
  }
  if (wave < nkb) {
    load_rows(kp, wave, kr);
    load_rows(vp, wave, vr);
  }
  uint4 qf[3][NQ];
#pragma unroll
  for (int s = 0; s < NQ; ++s)
    split3_rne(qr4[2 * s], qr4[2 * s + 1], qf[0][s], qf[1][s], qf[2][s]);
  f32x16 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = zero16();
  float mrow = -INFINITY, lrow = 0.f;
  for (int kb = wave; kb < nkb; kb += NW) {
    const bool more = kb + NW < nkb;
    // The wave's own region: its reads of the previous key block's V^T were
    // issued before these writes, and one wave's LDS operations complete in
    // order; the wave barrier keeps the compiler from moving them across.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      uint32_t lo[3], hi[3];
      split_pair(kr[i].x, kr[i].y, lo);
      split_pair(kr[i].z, kr[i].w, hi);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        *reinterpret_cast<uint2*>(&Ks(pl)[sk + i][sc]) = make_uint2(lo[pl], hi[pl]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the writes have landed
    __builtin_amdgcn_wave_barrier();
    if (more) load_rows(kp, kb + NW, kr);
    const int j0 = kb * KB;

    f32x16 st = zero16();
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      bf16x8 kf[3];
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        kf[pl] = bf16x8_of(*reinterpret_cast<const uint4*>(&Ks(pl)[j][16 * s + 8 * h]));
      st = mfma_bf16(kf[2], bf16x8_of(qf[0][s]), st);
      st = mfma_bf16(kf[1], bf16x8_of(qf[1][s]), st);
      st = mfma_bf16(kf[0], bf16x8_of(qf[2][s]), st);
      st = mfma_bf16(kf[1], bf16x8_of(qf[0][s]), st);
      st = mfma_bf16(kf[0], bf16x8_of(qf[1][s]), st);
      st = mfma_bf16(kf[0], bf16x8_of(qf[0][s]), st);
    }
    // The score MFMAs consumed every K fragment read, so those reads have
    // completed: V^T may overwrite the region.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int run = 0; run < KPT / 8; ++run) {
        uint32_t t[4][3];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 a = vr[8 * run + 2 * g], e = vr[8 * run + 2 * g + 1];
          const float x0 = c == 0 ? a.x : c == 1 ? a.y : c == 2 ? a.z : a.w;
          const float x1 = c == 0 ? e.x : c == 1 ? e.y : c == 2 ? e.z : e.w;
          split_pair(x0, x1, t[g]);
        }
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint4*>(&Vt(pl)[sc + c][sk + 8 * run]) =
              make_uint4(t[0][pl], t[1][pl], t[2][pl], t[3][pl]);
      }
    }
    if (more) load_rows(vp, kb + NW, vr);
    const bool masked = j0 + KB - 1 > q0 || j0 + KB > S;
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * qscale;
      if (masked) {
        const int key = j0 + acc_row(r, h);
        if (key > qi || key >= S) v = -INFINITY;
      }
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    // Every block this wave takes has a key at or below each query of the
    // tile except on the diagonal, where key j0 <= q0 <= qi: pm is finite.
    const float mnew = fmaxf(mrow, pm);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(mrow - mnew);
    lrow = lrow * corr + ps;
    if (__any(mnew != mrow)) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    }
    mrow = mnew;
    uint4 pf[2][3];
#pragma unroll
    for (int half = 0; half < 2; ++half)
      split3_rne(make_float4(st[8 * half], st[8 * half + 1], st[8 * half + 2], st[8 * half + 3]),
                 make_float4(st[8 * half + 4], st[8 * half + 5], st[8 * half + 6],
                             st[8 * half + 7]),
                 pf[half][0], pf[half][1], pf[half][2]);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the V^T writes have landed
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // V^T rows of the same keys: two runs of four (the staging writes
        // eight consecutive keys per store; k_flash_x6's permuted layout,
        // which would split them, measured slower here).
        bf16x8 vf[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
          const uint16_t* vrow = Vt(pl)[32 * t + j] + 16 * half;
          const uint2 a0 = *reinterpret_cast<const uint2*>(vrow + 4 * h);
          const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + 8 + 4 * h);
          vf[pl] = bf16x8_of(make_uint4(a0.x, a0.y, a1.x, a1.y));
        }
        o[t] = mfma_bf16(vf[2], bf16x8_of(pf[half][0]), o[t]);
        o[t] = mfma_bf16(vf[1], bf16x8_of(pf[half][1]), o[t]);
        o[t] = mfma_bf16(vf[0], bf16x8_of(pf[half][2]), o[t]);
        o[t] = mfma_bf16(vf[1], bf16x8_of(pf[half][0]), o[t]);
        o[t] = mfma_bf16(vf[0], bf16x8_of(pf[half][1]), o[t]);
        o[t] = mfma_bf16(vf[0], bf16x8_of(pf[half][0]), o[t]);
      }
    }
  }

  // Merge.  Wave w's O^T goes to Om[w][dim][query] and its (m, l) per query
  // to ML[w]; a wave that took no key block holds m = -inf, l = 0, O = 0.
  __syncthreads();
  float* Om = reinterpret_cast<float*>(lds);
  float2* ML = reinterpret_cast<float2*>(lds + NW * HD * OS * 4);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) Om[(wave * HD + 32 * t + acc_row(r, h)) * OS + j] = o[t][r];
  if (h == 0) ML[wave * 32 + j] = make_float2(mrow, lrow);
  __syncthreads();
  float* op = p.o + fs.o + hh * HD;
  for (int e = tid; e < 32 * HD; e += 64 * NW) {
    const int qr = e / HD, dim = e % HD, qrow = q0 + qr;
    if (qrow >= S) continue;
    float2 ml[NW];
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      ml[w] = ML[w * 32 + qr];
      mx = fmaxf(mx, ml[w].x);  // finite: wave 0 took key block 0
    }
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __builtin_amdgcn_exp2f(ml[w].x - mx);
      num += Om[(w * HD + dim) * OS + qr] * f;
      den += ml[w].y * f;
    }
    op[(size_t)qrow * d + dim] = num / den;
    if (p.lse && dim == 0)
      p.lse[fs.l + (size_t)qrow * H + hh] = mx * 0.69314718055994531f + logf(den);
  }
}

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void k_flash_x6w(FlashParams p) {
  __shared__ __align__(16) unsigned char lds[flash_w_lds<HD, NW, 3>()];
  flash_x6w_tile<HD, NW>(p, lds);
}

// The key-split tile on split-fp16 products (k_flash_h3's arithmetic: Q and
// K as two fp16 terms, three products per score contraction; P as two terms
// and V^T as hi, remainder and hi 2^-11, three products per output), with
// k_flash_x6w's layout: K's two planes or V^T's three in a wave's region,
// partial states merged through LDS.  Fewer planes and half the MFMAs of the
// split-bf16 tile.  An operand beyond fp16's range makes some output of the
// tile NaN (its infinite hi meets the opposite infinity of its remainder in
// every sum it enters), so the merge computes the tile's outputs, and stores
// them only if all are finite; otherwise it returns false having stored
// nothing, and the caller recomputes the tile on split-bf16 products.
template <int HD, int NW>
__device__ __forceinline__ bool flash_h3w_tile(const FlashParams& p, unsigned char* lds) {
  constexpr int KB = 32, NT = HD / 32, NQ = HD / 16;
  constexpr int KP = HD + 8, VP = KB + 8, CPR = HD / 4;
  constexpr int KPT = KB * CPR / 64;  // consecutive keys staged per lane
  static_assert(KPT == 8 || KPT == 16, "a wave stages 32 keys in runs of 8 or 16");
  constexpr int K_PLANE = KB * KP, V_PLANE = HD * VP;  // fp16 elements
  constexpr int K_BYTES = 2 * K_PLANE * 2, V_BYTES = 3 * V_PLANE * 2;
  constexpr int W_BYTES = K_BYTES > V_BYTES ? K_BYTES : V_BYTES;
  constexpr int OS = 33;                          // merge row stride
  constexpr int PER = 32 * HD / (64 * NW);        // merged outputs per lane
  static_assert(PER * 64 * NW == 32 * HD, "the merge deals whole rounds");

  const int qblk = gridDim.z - 1 - blockIdx.z, hh = blockIdx.x, b = blockIdx.y;
  FlashSeq fs;
  if (!flash_seq<HD>(p, hh, b, fs)) return true;
  const int S = fs.S, d = fs.d;
  const float scale = fs.scale;
  const int H = d / HD;
  const float qscale = scale * 1.44269504088896341f;
  const int q0 = qblk * 32;
  if (q0 >= S) return true;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  unsigned char* wl = lds + wave * W_BYTES;
  auto Ks = [&](int pl) { return reinterpret_cast<uint16_t (*)[KP]>(wl) + pl * KB; };
  auto Vt = [&](int pl) { return reinterpret_cast<uint16_t (*)[VP]>(wl) + pl * HD; };

  const float* qp = p.q + fs.q + hh * HD;
  const float* kp = p.k + fs.kv + hh * HD;
  const float* vp = p.v + fs.kv + hh * HD;

  const int qi = q0 + j;
  const int kend = min(S, q0 + 32);
  const int nkb = (kend + KB - 1) / KB;

  // Staging: lane l takes dims 4 (l % CPR) .. + 3 of keys KPT (l / CPR) ..
  // + KPT - 1.
  const int sc = (lane % CPR) * 4, sk = (lane / CPR) * KPT;
  float4 kr[KPT], vr[KPT];
  auto load_rows = [&](const float* src, int kb, float4 (&r)[KPT]) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int key = kb * KB + sk + i;
      r[i] = *reinterpret_cast<const float4*>(src + (size_t)(key < S ? key : 0) * d + sc);
    }
  };
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  // K: hi and scaled lo (x = hi + 2^-11 lo), packed as pairs.
  auto split_k = [](float a, float c, uint32_t (&t)[2]) {
    t[0] = cvt_pk_f16(a, c);
    const h2 hv = __builtin_bit_cast(h2, t[0]);
    t[1] = cvt_pk_f16((a - (float)hv[0]) * 2048.f, (c - (float)hv[1]) * 2048.f);
  };
  // V: hi, the unscaled remainder, and hi 2^-11, so that with P split as
  // p0 + 2^-11 p1 one accumulator takes p0 v0 + p0 v1 + p1 (2^-11 v0).
  auto split_v = [](float a, float c, uint32_t (&t)[3]) {
    t[0] = cvt_pk_f16(a, c);
    const h2 hv = __builtin_bit_cast(h2, t[0]);
    const float ha = (float)hv[0], hc = (float)hv[1];
    t[1] = cvt_pk_f16(a - ha, c - hc);
    t[2] = cvt_pk_f16(ha * 0x1p-11f, hc * 0x1p-11f);
  };
  // The query rows, then the first key block's K and V rows, all in flight
  // before the wave waits on any of them.
  float4 qr4[2 * NQ];
  {
    const float* qr = qp + (size_t)(qi < S ? qi : 0) * d + 8 * h;
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      qr4[2 * s] = *reinterpret_cast<const float4*>(qr + 16 * s);
      qr4[2 * s + 1] = *reinterpret_cast<const float4*>(qr + 16 * s + 4);
    }
  }
  if (wave < nkb) {
    load_rows(kp, wave, kr);
    load_rows(vp, wave, vr);
  }
  uint4 qf[2][NQ];
#pragma unroll
  for (int s = 0; s < NQ; ++s) split2_f16(qr4[2 * s], qr4[2 * s + 1], qf[0][s], qf[1][s]);
  f32x16 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = zero16();
  float mrow = -INFINITY, lrow = 0.f;
  for (int kb = wave; kb < nkb; kb += NW) {
    const bool more = kb + NW < nkb;
    // The wave's own region: its reads of the previous key block's V^T were
    // issued before these writes, and one wave's LDS operations complete in
    // order; the wave barrier keeps the compiler from moving them across.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      uint32_t lo[2], hi[2];
      split_k(kr[i].x, kr[i].y, lo);
      split_k(kr[i].z, kr[i].w, hi);
#pragma unroll
      for (int pl = 0; pl < 2; ++pl)
        *reinterpret_cast<uint2*>(&Ks(pl)[sk + i][sc]) = make_uint2(lo[pl], hi[pl]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the writes have landed
    __builtin_amdgcn_wave_barrier();
    if (more) load_rows(kp, kb + NW, kr);
    const int j0 = kb * KB;

    // Scores: hi.hi in st, the cross terms in scr, st + 2^-11 scr.
    f32x16 st = zero16(), scr = zero16();
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      f16x8 kf[2];
#pragma unroll
      for (int pl = 0; pl < 2; ++pl)
        kf[pl] = f16x8_of(*reinterpret_cast<const uint4*>(&Ks(pl)[j][16 * s + 8 * h]));
      scr = mfma_f16(kf[1], f16x8_of(qf[0][s]), scr);
      scr = mfma_f16(kf[0], f16x8_of(qf[1][s]), scr);
      st = mfma_f16(kf[0], f16x8_of(qf[0][s]), st);
    }
    // The score MFMAs consumed every K fragment read, so those reads have
    // completed: V^T may overwrite the region.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int run = 0; run < KPT / 8; ++run) {
        uint32_t t[4][3];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 a = vr[8 * run + 2 * g], e = vr[8 * run + 2 * g + 1];
          const float x0 = c == 0 ? a.x : c == 1 ? a.y : c == 2 ? a.z : a.w;
          const float x1 = c == 0 ? e.x : c == 1 ? e.y : c == 2 ? e.z : e.w;
          split_v(x0, x1, t[g]);
        }
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint4*>(&Vt(pl)[sc + c][sk + 8 * run]) =
              make_uint4(t[0][pl], t[1][pl], t[2][pl], t[3][pl]);
      }
    }
    if (more) load_rows(vp, kb + NW, vr);
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] += scr[r] * 0x1p-11f;
    const bool masked = j0 + KB - 1 > q0 || j0 + KB > S;
    float pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * qscale;
      if (masked) {
        const int key = j0 + acc_row(r, h);
        if (key > qi || key >= S) v = -INFINITY;
      }
      st[r] = v;
      pm = fmaxf(pm, v);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    // Every block this wave takes has a key at or below each query of the
    // tile except on the diagonal, where key j0 <= q0 <= qi: pm is finite
    // unless a score is +inf.
    const float mnew = fmaxf(mrow, pm);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(st[r] - mnew);
      st[r] = e;
      ps += e;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(mrow - mnew);
    lrow = lrow * corr + ps;
    if (__any(mnew != mrow)) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    }
    mrow = mnew;
    uint4 pf[2][2];
#pragma unroll
    for (int half = 0; half < 2; ++half)
      split2_f16(make_float4(st[8 * half], st[8 * half + 1], st[8 * half + 2], st[8 * half + 3]),
                 make_float4(st[8 * half + 4], st[8 * half + 5], st[8 * half + 6],
                             st[8 * half + 7]),
                 pf[half][0], pf[half][1]);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the V^T writes have landed
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // V^T rows of the same keys: two runs of four (acc_row(8 half ..
        // 8 half + 7, h)).
        f16x8 vf[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
          const uint16_t* vrow = Vt(pl)[32 * t + j] + 16 * half;
          const uint2 a0 = *reinterpret_cast<const uint2*>(vrow + 4 * h);
          const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + 8 + 4 * h);
          vf[pl] = f16x8_of(make_uint4(a0.x, a0.y, a1.x, a1.y));
        }
        // Smallest terms first: p1 (2^-11 v0), p0 v1, then p0 v0.
        o[t] = mfma_f16(vf[2], f16x8_of(pf[half][1]), o[t]);
        o[t] = mfma_f16(vf[1], f16x8_of(pf[half][0]), o[t]);
        o[t] = mfma_f16(vf[0], f16x8_of(pf[half][0]), o[t]);
      }
    }
  }

  // Merge as in flash_x6w_tile, into registers first.
  __syncthreads();
  float* Om = reinterpret_cast<float*>(lds);
  float2* ML = reinterpret_cast<float2*>(lds + NW * HD * OS * 4);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) Om[(wave * HD + 32 * t + acc_row(r, h)) * OS + j] = o[t][r];
  if (h == 0) ML[wave * 32 + j] = make_float2(mrow, lrow);
  __syncthreads();
  float res[PER], lse[PER];
  bool finite = true;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid + i * 64 * NW;
    const int qr = e / HD, dim = e % HD;
    float2 ml[NW];
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      ml[w] = ML[w * 32 + qr];
      mx = fmaxf(mx, ml[w].x);
    }
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __builtin_amdgcn_exp2f(ml[w].x - mx);
      num += Om[(w * HD + dim) * OS + qr] * f;
      den += ml[w].y * f;
    }
    res[i] = num / den;
    lse[i] = mx * 0.69314718055994531f + logf(den);
    // Rows past S hold no keys' weights: not stored, not checked.
    if (q0 + qr < S) finite = finite && __builtin_isfinite(res[i]) && __builtin_isfinite(lse[i]);
  }
  if (__syncthreads_or(!finite)) return false;
  float* op = p.o + fs.o + hh * HD;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid + i * 64 * NW;
    const int qr = e / HD, dim = e % HD, qrow = q0 + qr;
    if (qrow >= S) continue;
    op[(size_t)qrow * d + dim] = res[i];
    if (p.lse && dim == 0) p.lse[fs.l + (size_t)qrow * H + hh] = lse[i];
  }
  return true;
}

// The key-split tile on split-fp16 products, recomputed on split-bf16
// products when an operand is beyond fp16's range: fp32 accuracy for any
// finite input, with no flag for the caller to read.
template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void k_flash_h3w(FlashParams p) {
  constexpr int L2 = flash_w_lds<HD, NW, 2>(), L3 = flash_w_lds<HD, NW, 3>();
  __shared__ __align__(16) unsigned char lds[L2 > L3 ? L2 : L3];
  if (!flash_h3w_tile<HD, NW>(p, lds)) {
    __syncthreads();
    flash_x6w_tile<HD, NW>(p, lds);
  }
}

// ---------------------------------------------------------------------------

hipError_t launch_gemm(const GemmParams& p, int epi, hipStream_t s) {
  dim3 g((p.N + 127) / 128, (p.M + 127) / 128), b(256);
  GemmParams q = p;
  q.split_kc = p.K;
  if (p.split_ws && p.split_cnt && (epi == GEMM_STORE || epi == GEMM_ADD)) {
    // Fewer tiles than the part has CUs: K split over up to 16 blocks per
    // tile (at least 64 rows each), about 256 blocks in all, within the
    // workspace (one 128 x 128 partial per tile and split).
    const long tiles = (long)g.x * g.y, ws_tiles = (long)(kGemvWsFloats / (128 * 128));
    int splits = 1;
    if (tiles < 256 && tiles <= kGemvSlabs)
      splits = (int)std::min<long>({16, (256 + tiles - 1) / tiles, std::max(1, p.K / 64),
                                    ws_tiles / tiles});
    if (splits > 1) {
      q.split_kc = ((p.K + splits - 1) / splits + 15) / 16 * 16;
      g.z = (p.K + q.split_kc - 1) / q.split_kc;
    }
  }
  if (g.z <= 1) q.split_ws = nullptr;
  switch (epi) {
    case GEMM_STORE:
      if (q.split_ws) hipLaunchKernelGGL((k_gemm<GEMM_STORE, true>), g, b, 0, s, q);
      else hipLaunchKernelGGL((k_gemm<GEMM_STORE>), g, b, 0, s, q);
      break;
    case GEMM_ADD:
      if (q.split_ws) hipLaunchKernelGGL((k_gemm<GEMM_ADD, true>), g, b, 0, s, q);
      else hipLaunchKernelGGL((k_gemm<GEMM_ADD>), g, b, 0, s, q);
      break;
    case GEMM_SILU: hipLaunchKernelGGL(k_gemm<GEMM_SILU>, g, b, 0, s, q); break;
    case GEMM_QKV: hipLaunchKernelGGL(k_gemm<GEMM_QKV>, g, b, 0, s, q); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The part's CU count: below it, a 128-query flash grid leaves CUs idle.
static int flash_small_grid() {
  static int n = 0;
  if (!n) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus > 0)
      n = cus;
    else
      n = 256;
  }
  return n;
}

hipError_t launch_flash(const FlashParams& p, int batch, int max_rows,
                        hipStream_t s) {
  if (p.hd <= 0 || p.d % p.hd != 0) return hipErrorInvalidValue;
  const int H = p.d / p.hd;
  if (p.hd > 32 && p.hd < 128 && p.hd != 64) {
    // A head size between the MFMA kernels': the split-bf16 kernel of the
    // next larger size, columns past hd zero (fp32-accurate, whatever p.x6
    // asks); heads that are not a multiple of 4 load element by element.
    const dim3 g(H, batch, (max_rows + 127) / 128);
    const bool ua = p.hd % 4 != 0;
    if (p.hd < 64) {
      if (ua)
        hipLaunchKernelGGL((k_flash_x6<64, true>), g, dim3(256), 0, s, p);
      else
        hipLaunchKernelGGL((k_flash_x6<64, false>), g, dim3(256), 0, s, p);
    } else if (ua) {
      hipLaunchKernelGGL((k_flash_x6<128, true>), g, dim3(256), 0, s, p);
    } else {
      hipLaunchKernelGGL((k_flash_x6<128, false>), g, dim3(256), 0, s, p);
    }
    return hipGetLastError();
  }
  if (p.hd == 64 || p.hd == 128) {
    // Query blocks slowest and last-first: every (sequence, head)'s longest
    // causal block is dispatched before any shorter one, so the grid ends on
    // short blocks (longest-first scheduling).
    const dim3 g(H, batch, (max_rows + 127) / 128);
    if (p.x6 && (long)g.x * g.y * g.z < flash_small_grid()) {
      // Fewer 128-query blocks than CUs: 32-query tiles, keys split over
      // the block's waves; split-fp16 tiles that recompute themselves on
      // split-bf16 when an operand is out of fp16's range (k_flash_h3w),
      // or split-bf16 throughout for FLASH_X6.
      const dim3 gw(H, batch, (max_rows + 31) / 32);
      if (p.x6 == FLASH_X6) {
        if (p.hd == 64)
          hipLaunchKernelGGL((k_flash_x6w<64, 8>), gw, dim3(512), 0, s, p);
        else
          hipLaunchKernelGGL((k_flash_x6w<128, 4>), gw, dim3(256), 0, s, p);
      } else if (p.hd == 64) {
        hipLaunchKernelGGL((k_flash_h3w<64, 8>), gw, dim3(512), 0, s, p);
      } else {
        hipLaunchKernelGGL((k_flash_h3w<128, 4>), gw, dim3(256), 0, s, p);
      }
    } else if (p.x6 == FLASH_H3) {
      if (p.hd == 64)
        hipLaunchKernelGGL(k_flash_h3<64>, g, dim3(256), 0, s, p);
      else
        hipLaunchKernelGGL(k_flash_h3<128>, g, dim3(256), 0, s, p);
    } else if (p.x6 == FLASH_FP32 && p.hd == 64) {
      hipLaunchKernelGGL(k_flash_h3x<64>, g, dim3(256), 0, s, p);
    } else if (p.x6) {
      if (p.hd == 64)
        hipLaunchKernelGGL(k_flash_x6<64>, g, dim3(256), 0, s, p);
      else
        hipLaunchKernelGGL(k_flash_x6<128>, g, dim3(256), 0, s, p);
    } else if (p.hd == 64) {
      hipLaunchKernelGGL(k_flash_mfma<64>, g, dim3(256), 0, s, p);
    } else {
      hipLaunchKernelGGL(k_flash_mfma<128>, g, dim3(256), 0, s, p);
    }
    return hipGetLastError();
  }
  // Head sizes up to 32: the scalar kernel of the next power of two.
  dim3 g((max_rows + 63) / 64, H, batch), b(64);
  if (p.hd <= 2)
    hipLaunchKernelGGL(k_flash_generic<2>, g, b, 0, s, p);
  else if (p.hd <= 4)
    hipLaunchKernelGGL(k_flash_generic<4>, g, b, 0, s, p);
  else if (p.hd <= 8)
    hipLaunchKernelGGL(k_flash_generic<8>, g, b, 0, s, p);
  else if (p.hd <= 16)
    hipLaunchKernelGGL(k_flash_generic<16>, g, b, 0, s, p);
  else if (p.hd <= 32)
    hipLaunchKernelGGL(k_flash_generic<32>, g, b, 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_gemm_bf16(const GemmParams& p, int epi, hipStream_t s) {
  // K bounded so a block's 256 rows fit a buffer resource's byte range.
  if (p.K % 8 != 0 || p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K > (1 << 20))
    return hipErrorInvalidValue;
  if (!p.a == !p.a16) return hipErrorInvalidValue;
  dim3 g((p.N + 255) / 256, (p.M + 255) / 256), b(512);
#define AKH_GO(E)                                                 \
  if (p.a && p.a_hi_only)                                         \
    hipLaunchKernelGGL((k_gemm_bf16<E, 2>), g, b, 0, s, p);       \
  else if (p.a)                                                   \
    hipLaunchKernelGGL((k_gemm_bf16<E, 1>), g, b, 0, s, p);       \
  else                                                            \
    hipLaunchKernelGGL((k_gemm_bf16<E, 0>), g, b, 0, s, p);
  switch (epi) {
    case GEMM_ADD: AKH_GO(GEMM_ADD) break;
    case GEMM_SILU: AKH_GO(GEMM_SILU) break;
    case GEMM_QKV: AKH_GO(GEMM_QKV) break;
    default: return hipErrorInvalidValue;
  }
#undef AKH_GO
  return hipGetLastError();
}

hipError_t launch_gemm_x6(const GemmParams& p, int epi, hipStream_t s) {
  // K bounded so a block's rows (at most 256 of K floats) fit a buffer
  // resource's 32-bit byte range.
  if (p.K % 8 != 0 || p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K > (1 << 20) || !p.a || !p.bt)
    return hipErrorInvalidValue;
  // 256x256 tiles when they fill the chip twice over, else 128x128 (fewer
  // idle CUs on the last round of tiles); measured on MI355X.
  const bool big = (long)((p.M + 255) / 256) * ((p.N + 255) / 256) >= 512;
  // 128 x 128 tiles interleave MFMAs with the split where K is short.
  const bool il = p.K <= 1024;
#define AKH_X6_GO(E)                                                                        \
  if (big)                                                                                  \
    hipLaunchKernelGGL((k_gemm_x6<E, 256, 256, 2, 4, false>),                               \
                       dim3((p.N + 255) / 256, (p.M + 255) / 256), dim3(512), 0, s, p);      \
  else if (il)                                                                              \
    hipLaunchKernelGGL((k_gemm_x6<E, 128, 128, 2, 2, true>),                                \
                       dim3((p.N + 127) / 128, (p.M + 127) / 128), dim3(256), 0, s, p);      \
  else                                                                                      \
    hipLaunchKernelGGL((k_gemm_x6<E, 128, 128, 2, 2, false>),                               \
                       dim3((p.N + 127) / 128, (p.M + 127) / 128), dim3(256), 0, s, p);
  switch (epi) {
    case GEMM_STORE: AKH_X6_GO(GEMM_STORE) break;
    case GEMM_ADD: AKH_X6_GO(GEMM_ADD) break;
    case GEMM_SILU: AKH_X6_GO(GEMM_SILU) break;
    case GEMM_QKV: AKH_X6_GO(GEMM_QKV) break;
    default: return hipErrorInvalidValue;
  }
#undef AKH_X6_GO
  return hipGetLastError();
}

hipError_t launch_gemm_h3(const GemmParams& p, int epi, hipStream_t s) {
  // K bounded so a block's rows (at most 256 of K floats) fit a buffer
  // resource's 32-bit byte range.
  if (p.K % 8 != 0 || p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K > (1 << 20) || !p.a || !p.bp16 ||
      !p.range_flag)
    return hipErrorInvalidValue;
  // 256 x 128 tiles when there are at least four per CU, else 128 x 128
  // (fewer idle CUs on the last round); measured on MI355X.
  const bool big = (long)((p.M + 255) / 256) * ((p.N + 127) / 128) >= 1024;
#define AKH_H3_GO(E)                                                                        \
  if (big)                                                                                  \
    hipLaunchKernelGGL((k_gemm_h3<E, 256, 128, 4, 2>),                                      \
                       dim3((p.N + 127) / 128, (p.M + 255) / 256), dim3(512), 0, s, p);      \
  else                                                                                      \
    hipLaunchKernelGGL((k_gemm_h3<E, 128, 128, 2, 2>),                                      \
                       dim3((p.N + 127) / 128, (p.M + 127) / 128), dim3(256), 0, s, p);
  switch (epi) {
    case GEMM_STORE: AKH_H3_GO(GEMM_STORE) break;
    case GEMM_ADD: AKH_H3_GO(GEMM_ADD) break;
    case GEMM_SILU: AKH_H3_GO(GEMM_SILU) break;
    case GEMM_QKV: AKH_H3_GO(GEMM_QKV) break;
    default: return hipErrorInvalidValue;
  }
#undef AKH_H3_GO
  return hipGetLastError();
}

hipError_t launch_transpose_f32(const float* w, int K, int N, float* wt, hipStream_t s) {
  if (K <= 0 || N <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_transpose_f32, dim3((N + 31) / 32, (K + 31) / 32), dim3(256), 0, s, w, K,
                     N, wt);
  return hipGetLastError();
}

hipError_t launch_split_weights_f16(const float* w, int K, int N, uint16_t* wp, hipStream_t s) {
  if (K <= 0 || N <= 0 || K % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_split_weights_f16, dim3((N + 31) / 32, (K + 31) / 32), dim3(256), 0, s, w,
                     K, N, wp);
  return hipGetLastError();
}

hipError_t launch_transpose_bf16(const float* w, int K, int N, uint16_t* wt, hipStream_t s) {
  if (K <= 0 || N <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_transpose_bf16, dim3((N + 31) / 32, (K + 31) / 32), dim3(256), 0, s, w,
                     K, N, wt);
  return hipGetLastError();
}

hipError_t launch_flash_bf16(const FlashParams& p, int batch, int max_rows, hipStream_t s) {
  if (p.meta || !p.o16) return hipErrorInvalidValue;
  const dim3 g(p.d / p.hd, batch, (max_rows + 127) / 128);  // as launch_flash
  if (p.hd == 64)
    hipLaunchKernelGGL(k_flash_bf16<64>, g, dim3(256), 0, s, p);
  else if (p.hd == 128)
    hipLaunchKernelGGL(k_flash_bf16<128>, g, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_rows_rmsnorm(const float* x, const float* w, float* out,
                               int rows, int size, float eps, hipStream_t s) {
  const dim3 g((rows + 3) / 4);
  if (size % 4 != 0 || size > 4096)
    hipLaunchKernelGGL(k_rows_rmsnorm<0>, dim3(rows), dim3(256), 0, s, x, w, out, rows, size, eps);
  else if (size <= 1024)
    hipLaunchKernelGGL(k_rows_rmsnorm<4>, g, dim3(256), 0, s, x, w, out, rows, size, eps);
  else if (size <= 2048)
    hipLaunchKernelGGL(k_rows_rmsnorm<8>, g, dim3(256), 0, s, x, w, out, rows, size, eps);
  else
    hipLaunchKernelGGL(k_rows_rmsnorm<16>, g, dim3(256), 0, s, x, w, out, rows, size, eps);
  return hipGetLastError();
}

hipError_t launch_embedding_rows(const uint32_t* tokens, const float* table,
                                 float* out, int rows, int d, uint32_t vocab,
                                 hipStream_t s) {
  hipLaunchKernelGGL(k_embedding_rows, dim3(rows), dim3(256), 0, s, tokens,
                     table, out, d, vocab);
  return hipGetLastError();
}

}  // namespace akh
