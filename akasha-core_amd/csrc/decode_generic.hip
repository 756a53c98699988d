// Decode step for model shapes the batched decode kernels do not take: a
// head size that is not a multiple of 4 (their lanes read four columns at
// a time), a dim that is not a multiple of 32 or above 4096, an ffn_hidden
// that is not a multiple of 32.  The reference decodes any shape that
// ModelConfig::new accepts (src/config.rs:15-30; the CPU decode kernels take
// any head size, src/shaders/cpu.rs:144-178), so these sessions decode too,
// with the activations in plain row-major rows:
//
//   x = embedding(tok); xn = norm_1(x)
//   per layer: qkv = xn W_qkv; attention (RoPE, KV append, softmax(scale
//     q K^T) V) -> a; x += a W_o; xn = norm_2(x); f = silu(xn W_up);
//     x += f W_down; xn = next norm(x)
//   logits = xn W_lm; first-max partial per row
//
// The GEMMs are the fp32-MFMA prefill GEMM (any M, N, K) and the norms the
// prefill's row RMSNorm; the attention below is scalar and takes any head
// size up to 128.  Numerics follow the reference's CPU kernels to rounding
// (fp32 throughout).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace akh {

namespace {

constexpr int kGenChunk = 1024;  // scores held in LDS per pass over the keys

__device__ __forceinline__ float kv_load(const void* base, size_t i, bool kv16) {
  if (kv16) return __uint_as_float((uint32_t) static_cast<const uint16_t*>(base)[i] << 16);
  return static_cast<const float*>(base)[i];
}

// One block of 256 threads per (head, sequence).  Sequence b's token sits at
// position t = pos[b]: q and k of its head are rotated by RoPE at t
// (cpu.rs:111-142: pairs (2i, 2i + 1), the session's table of cos / sin),
// k and v are appended to the cache at row t (cpu.rs:224-236), and the
// output is softmax(scale q K^T) V over rows 0..t (cpu.rs:144-203; the
// scores are scaled inside the softmax, its maximum taken over the scaled
// scores).  Keys run in chunks of kGenChunk scores held in LDS, the running
// maximum and sum rescaled per chunk; thread c < hd accumulates output
// column c.  Rows with active[b] == 0 (a finished generate row) do nothing.
template <bool KV16>
__global__ __launch_bounds__(256) void k_gen_attn(GenAttnParams p) {
  __shared__ float qs[128], ks[128], vs[128];
  __shared__ float sc[kGenChunk];
  __shared__ float red[4];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  if (p.active && !p.active[b]) return;
  const int d = p.d, hd = p.hd, half = hd / 2;
  const int t = p.pos[b];
  const float* row = p.qkv + (size_t)b * 3 * d + (size_t)h * hd;
  for (int i = tid; i < half; i += 256) {
    const float2 cs = p.rope[(size_t)t * half + i];
    float q0 = row[2 * i], q1 = row[2 * i + 1];
    float k0 = row[d + 2 * i], k1 = row[d + 2 * i + 1];
    rope_pair(q0, q1, cs.x, cs.y);
    rope_pair(k0, k1, cs.x, cs.y);
    qs[2 * i] = q0;
    qs[2 * i + 1] = q1;
    ks[2 * i] = k0;
    ks[2 * i + 1] = k1;
  }
  for (int c = tid; c < hd; c += 256) vs[c] = row[2 * d + c];
  __syncthreads();
  const size_t base = (size_t)b * p.seq_stride + (size_t)h * hd;
  for (int c = tid; c < hd; c += 256) {
    const size_t at = base + (size_t)t * d + c;
    if (KV16) {
      static_cast<uint16_t*>(p.kc)[at] = (uint16_t)bf16_bits(ks[c]);
      static_cast<uint16_t*>(p.vc)[at] = (uint16_t)bf16_bits(vs[c]);
    } else {
      static_cast<float*>(p.kc)[at] = ks[c];
      static_cast<float*>(p.vc)[at] = vs[c];
    }
  }
  // Row t is read back from LDS (as the cache holds it), not from memory.
  if (KV16) {
    __syncthreads();
    for (int c = tid; c < hd; c += 256) {
      ks[c] = __uint_as_float(bf16_bits(ks[c]) << 16);
      vs[c] = __uint_as_float(bf16_bits(vs[c]) << 16);
    }
    __syncthreads();
  }
  float m = -INFINITY, l = 0.f, o = 0.f;
  for (int j0 = 0; j0 <= t; j0 += kGenChunk) {
    const int n = min(kGenChunk, t + 1 - j0);
    float cmax = -INFINITY;
    for (int jj = tid; jj < n; jj += 256) {
      const int j = j0 + jj;
      float s = 0.f;
      if (j == t) {
        for (int c = 0; c < hd; ++c) s += qs[c] * ks[c];
      } else {
        const size_t kr = base + (size_t)j * d;
        for (int c = 0; c < hd; ++c) s += qs[c] * kv_load(p.kc, kr + c, KV16);
      }
      s *= p.scale;
      sc[jj] = s;
      cmax = fmaxf(cmax, s);
    }
    cmax = block_max256(cmax, red);
    const float mnew = fmaxf(m, cmax);
    const float corr = m == -INFINITY ? 0.f : expf(m - mnew);
    float csum = 0.f;
    for (int jj = tid; jj < n; jj += 256) {
      const float e = expf(sc[jj] - mnew);
      sc[jj] = e;
      csum += e;
    }
    csum = block_sum256(csum, red);  // its barriers publish sc
    l = l * corr + csum;
    if (tid < hd) {
      float acc = o * corr;
      for (int jj = 0; jj < n; ++jj) {
        const int j = j0 + jj;
        acc += sc[jj] * (j == t ? vs[tid] : kv_load(p.vc, base + (size_t)j * d + tid, KV16));
      }
      o = acc;
    }
    m = mnew;
    __syncthreads();  // sc is rewritten by the next chunk
  }
  if (tid < hd) p.out[(size_t)b * d + (size_t)h * hd + tid] = o / l;
}

// Per-row first maximum of logits [rows, n] (sampling.rs:83-91), stored as
// the single argmax partial of the row: (value bits, index).
__global__ __launch_bounds__(256) void k_gen_argmax_part(const float* logits, int n,
                                                         uint2* part) {
  const int r = blockIdx.x;
  const float* x = logits + (size_t)r * n;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (int i = threadIdx.x; i < n; i += 256) amax_merge(bv, bi, x[i], (uint32_t)i);
  block_amax256(bv, bi);
  if (threadIdx.x == 0) part[r] = make_uint2(__float_as_uint(bv), bi);
}

// dst row m = src row (src_rows ? src_rows[m] : row0 + m * row_stride).
__global__ __launch_bounds__(256) void k_gen_gather_rows(const float* src, float* dst, int d,
                                                         long row0, long row_stride,
                                                         const int* src_rows) {
  const int m = blockIdx.x;
  const long r = src_rows ? (long)src_rows[m] : row0 + (long)m * row_stride;
  for (int c = threadIdx.x; c < d; c += 256) dst[(size_t)m * d + c] = src[(size_t)r * d + c];
}

}  // namespace

hipError_t launch_gen_attn(const GenAttnParams& p, int batch, hipStream_t s) {
  if (p.hd <= 0 || p.hd > 128 || p.hd % 2 != 0 || p.d % p.hd != 0) return hipErrorInvalidValue;
  const dim3 g(p.d / p.hd, batch);
  if (p.kv16)
    hipLaunchKernelGGL(k_gen_attn<true>, g, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(k_gen_attn<false>, g, dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_gen_argmax_part(const float* logits, int rows, int n, uint2* part,
                                  hipStream_t s) {
  if (rows <= 0 || n <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gen_argmax_part, dim3(rows), dim3(256), 0, s, logits, n, part);
  return hipGetLastError();
}

hipError_t launch_gen_gather_rows(const float* src, float* dst, int rows, int d, long row0,
                                  long row_stride, const int* src_rows, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gen_gather_rows, dim3(rows), dim3(256), 0, s, src, dst, d, row0,
                     row_stride, src_rows);
  return hipGetLastError();
}

}  // namespace akh
