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
// Grid (N / 32 tiles, ksplit), W waves per block.  The block's K chunk is
// split over its waves, and within a wave half h of the lanes walks rows
// kbase_h + s: lane (j, h) supplies A[j][k] (a float4 of the k-quad tile
// covers four steps) and W[k][n0 + j] (a wave load covers two 128-byte row
// segments), and v_mfma_f32_32x32x2f32 accumulates the 32x32 output tile.
// The waves' tiles are reduced in LDS as a binary tree (fixed order) and
// wave 0 runs the epilogue.
template <int W, int EPI, bool NORM>
__global__ __launch_bounds__(64 * W) void k_dec_gemm(DecGemmParams p) {
  constexpr int U = 8;
  constexpr int RH = W > 1 ? W / 2 : 1;
  __shared__ float red[RH][32][33];
  __shared__ float ssw[W][32];
  __shared__ float rs_s[32];

  const int M = p.M, N = p.N, K = p.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int tile = blockIdx.x, n0 = tile * 32;
  constexpr int STEP = 16 * W;  // chunk granularity: 8 k per half-wave
  const int kc = ((K + (int)gridDim.y - 1) / (int)gridDim.y + STEP - 1) / STEP * STEP;
  const int kb = blockIdx.y * kc;
  if (kb >= K) return;
  const int ke = min(K, kb + kc);
  const int kw = kc / W, hl = kw / 2;
  const int kbase = kb + wave * kw + h * hl;
  const int ncol = n0 + j;
  const bool col_ok = ncol < N;

  f32x16 acc = zero16();
  float ss = 0.f;
  for (int s0 = 0; s0 < hl; s0 += U) {
    const int k0 = kbase + s0;
    float a[U], wv[U];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int kq = (k0 >> 2) + q;
      float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
      if (4 * kq < ke)
        t = *reinterpret_cast<const float4*>(p.xt + ((size_t)kq * 32 + j) * 4);
      a[4 * q] = t.x;
      a[4 * q + 1] = t.y;
      a[4 * q + 2] = t.z;
      a[4 * q + 3] = t.w;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + u;
      wv[u] = (k < ke && col_ok) ? p.w[(size_t)k * N + ncol] : 0.f;
    }
    if (NORM) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k0 + 4 * q < ke) g = *reinterpret_cast<const float4*>(p.gain + k0 + 4 * q);
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
    for (int u = 0; u < U; ++u) acc = mfma32(a[u], wv[u], acc);
  }

  if (W > 1) {
    for (int half = RH; half >= 1; half >>= 1) {
      __syncthreads();
      if (wave >= half && wave < 2 * half)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave - half][acc_row(r, h)][j] = acc[r];
      __syncthreads();
      if (wave < half)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += red[wave][acc_row(r, h)][j];
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
    float v = acc[r];
    if (NORM) v = __fmul_rn(v, rs_s[m]);
    if (EPI == DEC_RESID) {
      if (m < M && col_ok) {
        float* y = p.yt + kq_index(m, ncol);
        if (gridDim.y > 1)
          atomicAdd(y, v);
        else
          *y = *y + v;
      }
    } else if (EPI == DEC_SILU_T) {
      if (m < M && col_ok) p.yt[kq_index(m, ncol)] = v / (1.0f + expf(-v));
    } else if (EPI == DEC_QKV) {
      // RoPE pairs (2i, 2i+1) sit in lanes j and j^1 of the same half.
      const float partner = __shfl_xor(v, 1, 64);
      if (m < M && col_ok) {
        const int dim = p.dim;
        const int region = ncol / dim, c = ncol - region * dim;
        const int pos = p.pos[m];
        float out = v;
        if (region < 2) {
          const int i = (c % p.head_dim) >> 1;
          const float2 cs = p.rope[(size_t)pos * (p.head_dim >> 1) + i];
          const bool odd = ncol & 1;
          float x0 = odd ? partner : v, x1 = odd ? v : partner;
          rope_pair(x0, x1, cs.x, cs.y);
          out = odd ? x1 : x0;
        }
        if (region == 0)
          p.q_out[(size_t)m * dim + c] = out;
        else
          (region == 1 ? p.kcache : p.vcache)[(size_t)m * p.seq_stride +
                                              (size_t)pos * dim + c] = out;
      }
    } else if (EPI == DEC_LOGITS) {
      const bool ok = m < M && col_ok;
      if (ok) p.y[(size_t)m * N + ncol] = v;
      // First maximum of the row over this tile's 32 columns.
      float bv = ok ? v : -INFINITY;
      uint32_t bi = (uint32_t)ncol;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        amax_merge(bv, bi, ov, oi);
      }
      if (j == 0 && m < M) {
        const int ntiles = (N + 31) / 32;
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

template <int W, int EPI, bool NORM>
static hipError_t dec_go(const DecGemmParams& p, int ksplit, hipStream_t s) {
  hipLaunchKernelGGL((k_dec_gemm<W, EPI, NORM>), dim3((p.N + 31) / 32, ksplit),
                     dim3(64 * W), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_dec_gemm(const DecGemmParams& p, int epi, bool norm,
                           int ksplit, hipStream_t s) {
  if (ksplit < 1 || (ksplit > 1 && (epi != DEC_RESID || norm)))
    return hipErrorInvalidValue;
  switch (epi) {
    case DEC_RESID:
      return norm ? hipErrorInvalidValue : dec_go<4, DEC_RESID, false>(p, ksplit, s);
    case DEC_SILU_T:
      return norm ? dec_go<8, DEC_SILU_T, true>(p, 1, s)
                  : dec_go<8, DEC_SILU_T, false>(p, 1, s);
    case DEC_QKV:
      return norm ? dec_go<8, DEC_QKV, true>(p, 1, s)
                  : dec_go<8, DEC_QKV, false>(p, 1, s);
    case DEC_LOGITS:
      return norm ? dec_go<4, DEC_LOGITS, true>(p, 1, s)
                  : dec_go<4, DEC_LOGITS, false>(p, 1, s);
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
