// Batched decode kernels: every sequence of a step is one row of a 32-row
// MFMA tile, so each weight byte is read once per step for the whole batch.
//
// Activations that feed a GEMM (the residual stream, the attention output
// and the SiLU'd ffn hidden state) live in the k-quad layout [K/4][32][4]:
// the MFMA A operand of a half-wave is one contiguous 512-byte float4 load
// per four k.  RMSNorm is folded into its consumer GEMM: the gain is applied
// to the A operand, the sum of squares of the same operand is accumulated
// in the main loop, and 1/rms scales the output rows (the norm is a per-row
// scale, so it commutes with the contraction).  Nothing synchronises across
// work-groups inside a kernel; the residual GEMMs split K across
// work-groups and add their partial tiles into the residual stream with
// device-scope atomics.
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels.h"

namespace akh {

// Y[M, N] (epilogue) A[M, K] . W[K, N] for M <= 32.
//
// Grid (N tiles of NT = 32*C columns, ksplit), W waves per block.  A pass of
// the block covers KC = 2*W*HL rows of K: wave w takes 2*HL of them and half
// h of its lanes HL, lane (j, h) supplying A[j][k] (a float4 of the k-quad
// tile covers four k) and W[k][n0 + C*j + c] for MFMA tile c, so a wave load
// covers two row segments of 128*C contiguous bytes.  All of a pass's loads
// are issued before its first MFMA, so each wave keeps HL weight rows in
// flight.  The waves' tiles are reduced in LDS as a binary tree (fixed
// order) and wave 0 runs the epilogue.
template <int C, int W, int HL, int EPI, bool NORM>
__global__ __launch_bounds__(64 * W) void k_dec_gemm(DecGemmParams p) {
  constexpr int NT = 32 * C;
  constexpr int RH = W > 1 ? W / 2 : 1;
  constexpr int KC = 2 * W * HL;
  static_assert(HL % 4 == 0, "HL must cover whole k-quads");
  __shared__ float red[RH][32][NT + 1];
  __shared__ float ssw[W][32];
  __shared__ float rs_s[32];

  const int M = p.M, N = p.N, K = p.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int tile = blockIdx.x, n0 = tile * NT;
  const int per = (K + (int)gridDim.y - 1) / (int)gridDim.y;
  const int rows = (per + KC - 1) / KC * KC;  // whole passes per block
  const int kb = blockIdx.y * rows;
  if (kb >= K) return;
  const int ke = min(K, kb + rows);
  const int ncol = n0 + C * j;
  bool cok[C];
#pragma unroll
  for (int c = 0; c < C; ++c) cok[c] = ncol + c < N;
  const bool vec = C > 1 && (N % C) == 0 && ncol + C <= N;

  f32x16 acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) acc[c] = zero16();
  float ss = 0.f;
  for (int k0 = kb; k0 < ke; k0 += KC) {
    const int kr = k0 + wave * 2 * HL + h * HL;  // first row of this half
    float a[HL];
    float wv[HL][C];
#pragma unroll
    for (int u = 0; u < HL; ++u) {
      const int k = kr + u;
      const bool ok = k < ke;
      const float* wr = p.w + (size_t)(ok ? k : kb) * N + ncol;
      if (C == 4 && vec) {
        const float4 t = ok ? *reinterpret_cast<const float4*>(wr)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[u][0] = t.x;
        wv[u][C > 1 ? 1 : 0] = t.y;
        wv[u][C > 2 ? 2 : 0] = t.z;
        wv[u][C > 3 ? 3 : 0] = t.w;
      } else if (C == 2 && vec) {
        const float2 t = ok ? *reinterpret_cast<const float2*>(wr)
                            : make_float2(0.f, 0.f);
        wv[u][0] = t.x;
        wv[u][C > 1 ? 1 : 0] = t.y;
      } else {
#pragma unroll
        for (int c = 0; c < C; ++c) wv[u][c] = (ok && cok[c]) ? wr[c] : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < HL / 4; ++q) {
      const int kq = (kr >> 2) + q;
      float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
      if (4 * kq < ke)
        t = *reinterpret_cast<const float4*>(p.xt + ((size_t)kq * 32 + j) * 4);
      a[4 * q] = t.x;
      a[4 * q + 1] = t.y;
      a[4 * q + 2] = t.z;
      a[4 * q + 3] = t.w;
    }
    if (NORM) {
#pragma unroll
      for (int q = 0; q < HL / 4; ++q) {
        float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
        if (kr + 4 * q < ke) g = *reinterpret_cast<const float4*>(p.gain + kr + 4 * q);
        const float gg[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = a[4 * q + e];
          ss += x * x;
          a[4 * q + e] = __fmul_rn(x, gg[e]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < HL; ++u)
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] = mfma32(a[u], wv[u][c], acc[c]);
  }

  if (W > 1) {
    for (int half = RH; half >= 1; half >>= 1) {
      __syncthreads();
      if (wave >= half && wave < 2 * half)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            red[wave - half][acc_row(r, h)][C * j + c] = acc[c][r];
      __syncthreads();
      if (wave < half)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            acc[c][r] += red[wave][acc_row(r, h)][C * j + c];
    }
  }
  if (NORM) {
    // Whole rows are in this block (the host never splits K of a
    // normalising GEMM): finish sum(x^2) and turn it into 1/rms.
    ss += __shfl_xor(ss, 32, 64);
    if (h == 0) ssw[wave][j] = ss;
    __syncthreads();
    if (threadIdx.x < 32) {
      float t = 0.f;
      for (int w = 0; w < W; ++w) t += ssw[w][threadIdx.x];
      rs_s[threadIdx.x] = 1.0f / sqrtf(t / (float)K + p.eps);
    }
    __syncthreads();
  }
  if (wave != 0) return;

#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = acc_row(r, h);
    float v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = NORM ? __fmul_rn(acc[c][r], rs_s[m]) : acc[c][r];
    if (EPI == DEC_RESID) {
#pragma unroll
      for (int c = 0; c < C; ++c)
        if (m < M && cok[c]) {
          float* y = p.yt + kq_index(m, ncol + c);
          if (gridDim.y > 1)
            atomicAdd(y, v[c]);
          else
            *y = *y + v[c];
        }
    } else if (EPI == DEC_SILU_T) {
#pragma unroll
      for (int c = 0; c < C; ++c)
        if (m < M && cok[c]) p.yt[kq_index(m, ncol + c)] = v[c] / (1.0f + expf(-v[c]));
    } else if (EPI == DEC_QKV) {
      static_assert(EPI != DEC_QKV || C == 1, "QKV epilogue pairs lanes");
      // RoPE pairs (2i, 2i+1) sit in lanes j and j^1 of the same half.
      const float partner = __shfl_xor(v[0], 1, 64);
      if (m < M && cok[0]) {
        const int dim = p.dim;
        const int region = ncol / dim, cc = ncol - region * dim;
        const int pos = p.pos[m];
        float out = v[0];
        if (region < 2) {
          const int i = (cc % p.head_dim) >> 1;
          const float2 cs = p.rope[(size_t)pos * (p.head_dim >> 1) + i];
          const bool odd = ncol & 1;
          float x0 = odd ? partner : v[0], x1 = odd ? v[0] : partner;
          rope_pair(x0, x1, cs.x, cs.y);
          out = odd ? x1 : x0;
        }
        if (region == 0)
          p.q_out[(size_t)m * dim + cc] = out;
        else
          (region == 1 ? p.kcache : p.vcache)[(size_t)m * p.seq_stride +
                                              (size_t)pos * dim + cc] = out;
      }
    } else if (EPI == DEC_LOGITS) {
      // Logits, and the first maximum of the row over this tile's columns.
      float bv = -INFINITY;
      uint32_t bi = (uint32_t)ncol;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const bool ok = m < M && cok[c];
        if (ok) {
          p.y[(size_t)m * N + ncol + c] = v[c];
          amax_merge(bv, bi, v[c], (uint32_t)(ncol + c));
        }
      }
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        amax_merge(bv, bi, ov, oi);
      }
      if (j == 0 && m < M) {
        const int ntiles = (N + NT - 1) / NT;
        p.amax[(size_t)m * ntiles + tile] = make_uint2(__float_as_uint(bv), bi);
      }
    }
  }
}

// Single-query attention over the KV cache for one (sequence, head) per
// block: AW waves split the live rows 0..pos, each streams its rows with
// HD/4 lanes per row (a float4 each) and RB row groups of K and V in flight,
// keeps an online softmax, and the waves' (max, sum, o) are merged in LDS.
// The output row is written in the k-quad layout for the out_proj GEMM.
template <int HD, int AW>
__global__ __launch_bounds__(64 * AW) void k_dec_attn(DecAttnParams p) {
  constexpr int LPR = HD / 4;    // lanes per row
  constexpr int RPW = 64 / LPR;  // rows per wave per load
  constexpr int RB = 8;          // row groups per batch
  __shared__ float wm_s[AW], wl_s[AW];
  __shared__ float4 wo_s[AW][LPR];

  const int bh = blockIdx.x, b = bh / p.H, hh = bh - b * p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane % LPR, rl = lane / LPR;
  const int T = p.pos[b] + 1;
  const int ch = ((T + AW - 1) / AW + RPW - 1) / RPW * RPW;
  const int r0 = wave * ch, r1 = min(T, r0 + ch);

  const float4 q4 =
      *reinterpret_cast<const float4*>(p.q + (size_t)b * p.d + hh * HD + 4 * g);
  const float* kbase = p.kc + (size_t)b * p.seq_stride + hh * HD + 4 * g;
  const float* vbase = p.vc + (size_t)b * p.seq_stride + hh * HD + 4 * g;

  float m = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int base = r0; base < r1; base += RPW * RB) {
    float4 kv[RB], vv[RB];
    bool ok[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int r = base + i * RPW + rl;
      ok[i] = r < r1;
      const size_t off = (size_t)(ok[i] ? r : r0) * p.d;
      kv[i] = *reinterpret_cast<const float4*>(kbase + off);
      vv[i] = *reinterpret_cast<const float4*>(vbase + off);
    }
    float t[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      float s = q4.x * kv[i].x + q4.y * kv[i].y + q4.z * kv[i].z + q4.w * kv[i].w;
#pragma unroll
      for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      t[i] = ok[i] ? s * p.scale : -INFINITY;
    }
    float bm = t[0];
#pragma unroll
    for (int i = 1; i < RB; ++i) bm = fmaxf(bm, t[i]);
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) bm = fmaxf(bm, __shfl_xor(bm, o, 64));
    const float mn = fmaxf(m, bm);
    const float corr = m == -INFINITY ? 0.f : expf(m - mn);
    float ps = 0.f;
    float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const float e = ok[i] ? expf(t[i] - mn) : 0.f;
      ps += e;
      pv.x += e * vv[i].x;
      pv.y += e * vv[i].y;
      pv.z += e * vv[i].z;
      pv.w += e * vv[i].w;
    }
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) ps += __shfl_xor(ps, o, 64);
    l = l * corr + ps;
    acc.x = acc.x * corr + pv.x;
    acc.y = acc.y * corr + pv.y;
    acc.z = acc.z * corr + pv.z;
    acc.w = acc.w * corr + pv.w;
    m = mn;
  }
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) {
    acc.x += __shfl_xor(acc.x, o, 64);
    acc.y += __shfl_xor(acc.y, o, 64);
    acc.z += __shfl_xor(acc.z, o, 64);
    acc.w += __shfl_xor(acc.w, o, 64);
  }
  if (rl == 0) wo_s[wave][g] = acc;
  if (lane == 0) {
    wm_s[wave] = m;
    wl_s[wave] = l;
  }
  __syncthreads();
  if (threadIdx.x < LPR) {
    const int t = threadIdx.x;
    float M = -INFINITY;
    for (int w = 0; w < AW; ++w) M = fmaxf(M, wm_s[w]);
    float L = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = 0; w < AW; ++w) {
      const float wg = wm_s[w] == -INFINITY ? 0.f : expf(wm_s[w] - M);
      L += wg * wl_s[w];
      o.x += wg * wo_s[w][t].x;
      o.y += wg * wo_s[w][t].y;
      o.z += wg * wo_s[w][t].z;
      o.w += wg * wo_s[w][t].w;
    }
    const float inv = 1.0f / L;
    *reinterpret_cast<float4*>(p.out_t + ((size_t)(hh * (HD / 4) + t) * 32 + b) * 4) =
        make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
  }
}

// Rows into the k-quad layout: an embedding lookup (EMBEDDING semantics,
// cpu.rs:25-41) or the last row of every prefilled sequence.
__global__ void k_rows_to_kq(const float* table, const uint32_t* ids,
                             uint32_t vocab, const float* src, long row0,
                             long row_stride, float* xt, int d) {
  const int m = blockIdx.x;
  const float* row;
  if (ids) {
    const uint32_t id = ids[m];
    row = id < vocab ? table + (size_t)id * d : nullptr;
  } else {
    row = src + (size_t)(row0 + (long)m * row_stride) * d;
  }
  for (int q = threadIdx.x; q < d / 4; q += blockDim.x) {
    const float4 v = row ? *reinterpret_cast<const float4*>(row + 4 * q)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
    *reinterpret_cast<float4*>(xt + ((size_t)q * 32 + m) * 4) = v;
  }
}

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
      const int p0 = pos[m];
      if (hrow) {
        hrow[p0] = tok[m];
        hrow[p0 + 1] = id;
      }
      pos[m] = p0 + 1;
    } else if (hrow) {
      hrow[next_pos] = id;
    }
    tok[m] = id;
  }
}

// ---------------------------------------------------------------------------

template <int C, int W, int HL, int EPI, bool NORM>
static hipError_t dec_go(const DecGemmParams& p, int ksplit, hipStream_t s) {
  hipLaunchKernelGGL((k_dec_gemm<C, W, HL, EPI, NORM>),
                     dim3((p.N + 32 * C - 1) / (32 * C), ksplit), dim3(64 * W), 0,
                     s, p);
  return hipGetLastError();
}

// Launch shapes per role (N tile, waves, rows in flight per half-wave):
//   QKV, UP    32 cols, 16 waves, 24 rows: one block per N tile owns the
//              whole K = dim (needed by the folded RMSNorm);
//   OUT, DOWN  32 cols,  4 waves, 16 rows: K split in chunks of 128 rows,
//              partial tiles added atomically into the residual stream;
//   LM         64 cols,  8 waves, 24 rows: whole K in two passes.
int dec_gemm_rows_per_block(int cfg) {
  switch (cfg) {
    case DEC_CFG_QKV:
    case DEC_CFG_UP: return 2 * 16 * 24;
    case DEC_CFG_OUT:
    case DEC_CFG_DOWN: return 2 * 4 * 16;
    default: return 2 * 8 * 24;
  }
}

hipError_t launch_dec_gemm(const DecGemmParams& p, int cfg, int ksplit,
                           hipStream_t s) {
  switch (cfg) {
    case DEC_CFG_QKV: return dec_go<1, 16, 24, DEC_QKV, true>(p, 1, s);
    case DEC_CFG_UP: return dec_go<1, 16, 24, DEC_SILU_T, true>(p, 1, s);
    case DEC_CFG_OUT:
    case DEC_CFG_DOWN: return dec_go<1, 4, 16, DEC_RESID, false>(p, ksplit, s);
    case DEC_CFG_LM: return dec_go<2, 8, 24, DEC_LOGITS, true>(p, 1, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dec_attn(const DecAttnParams& p, int batch, int hd,
                           hipStream_t s) {
  constexpr int AW = 8;
  dim3 g(batch * p.H), b(64 * AW);
  switch (hd) {
    case 4: hipLaunchKernelGGL((k_dec_attn<4, AW>), g, b, 0, s, p); break;
    case 8: hipLaunchKernelGGL((k_dec_attn<8, AW>), g, b, 0, s, p); break;
    case 16: hipLaunchKernelGGL((k_dec_attn<16, AW>), g, b, 0, s, p); break;
    case 32: hipLaunchKernelGGL((k_dec_attn<32, AW>), g, b, 0, s, p); break;
    case 64: hipLaunchKernelGGL((k_dec_attn<64, AW>), g, b, 0, s, p); break;
    case 128: hipLaunchKernelGGL((k_dec_attn<128, AW>), g, b, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rows_to_kq(const float* table, const uint32_t* ids,
                             uint32_t vocab, const float* src, long row0,
                             long row_stride, float* xt, int M, int d,
                             hipStream_t s) {
  hipLaunchKernelGGL(k_rows_to_kq, dim3(M), dim3(256), 0, s, table, ids,
                     vocab, src, row0, row_stride, xt, d);
  return hipGetLastError();
}

hipError_t launch_argmax_final(const uint2* part, int ntiles, int M,
                               uint32_t* tok, int* pos, uint32_t* hist,
                               int hist_stride, int next_pos, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_final, dim3(M), dim3(256), 0, s, part, ntiles,
                     tok, pos, hist, hist_stride, next_pos);
  return hipGetLastError();
}

}  // namespace akh
