// Device helpers shared by the kernel files (CDNA4 / gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace akh {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x2f32.  Operand layout: lane l supplies A[l % 32][l / 32]
// and B[l / 32][l % 32]; accumulator register r of lane l holds
// D[acc_row(r, l / 32)][l % 32].
__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// bfloat16 operands of v_mfma_f32_32x32x16_bf16: lane l supplies
// A[l % 32][8 * (l / 32) + i] and B[8 * (l / 32) + i][l % 32], i = 0..7; the
// accumulator layout is mfma32's.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// float -> bfloat16 bits, round to nearest even.
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return bf16_bits(lo) | (bf16_bits(hi) << 16);
}
__device__ __forceinline__ bf16x8 bf16x8_of(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// Eight floats (x0, x1) as three bfloat16 octets with x = hi + mid + lo
// exactly: hi keeps the top 8 significant bits (truncation), mid the top 8
// of the exact remainder x - hi (at most 16 bits), and the last remainder
// has at most 8 significant bits, so lo holds it without rounding.  With
// bfloat16 weights every product of a term with a weight is exact in fp32,
// so three bf16 MFMAs give an fp32-accurate A . W.
__device__ __forceinline__ void split3_bf16(float4 x0, float4 x1, uint4& hi, uint4& mid,
                                            uint4& lo) {
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  uint32_t ph[4], pm[4], pl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ua = __float_as_uint(v[2 * i]), ub = __float_as_uint(v[2 * i + 1]);
    const float ra = v[2 * i] - __uint_as_float(ua & 0xFFFF0000u);
    const float rb = v[2 * i + 1] - __uint_as_float(ub & 0xFFFF0000u);
    const uint32_t sa = __float_as_uint(ra), sb = __float_as_uint(rb);
    const uint32_t la = __float_as_uint(ra - __uint_as_float(sa & 0xFFFF0000u));
    const uint32_t lb = __float_as_uint(rb - __uint_as_float(sb & 0xFFFF0000u));
    ph[i] = (ua >> 16) | (ub & 0xFFFF0000u);
    pm[i] = (sa >> 16) | (sb & 0xFFFF0000u);
    pl[i] = (la >> 16) | (lb & 0xFFFF0000u);
  }
  hi = make_uint4(ph[0], ph[1], ph[2], ph[3]);
  mid = make_uint4(pm[0], pm[1], pm[2], pm[3]);
  lo = make_uint4(pl[0], pl[1], pl[2], pl[3]);
}
__device__ __forceinline__ bf16x8 bf16x8_of(float4 a, float4 b) {
  return bf16x8_of(make_uint4(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w),
                              pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)));
}

// Two floats as packed bfloat16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
}

// Eight floats as three bfloat16 octets with x = hi + mid + lo exactly,
// rounding to nearest: |x - hi| <= 2^-8 |x| and the remainder x - hi is
// exact (Sterbenz) with at most 16 significant bits; mid rounds it the same
// way, and the last remainder (at most 8 significant bits, |lo| <= 2^-16 |x|)
// converts without rounding.
__device__ __forceinline__ void split3_rne(float4 x0, float4 x1, uint4& hi, uint4& mid,
                                           uint4& lo) {
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  uint32_t ph[4], pm[4], pl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = v[2 * i], b = v[2 * i + 1];
    ph[i] = cvt_pk_bf16(a, b);
    const float ra = a - __uint_as_float(ph[i] << 16);
    const float rb = b - __uint_as_float(ph[i] & 0xFFFF0000u);
    pm[i] = cvt_pk_bf16(ra, rb);
    pl[i] = cvt_pk_bf16(ra - __uint_as_float(pm[i] << 16), rb - __uint_as_float(pm[i] & 0xFFFF0000u));
  }
  hi = make_uint4(ph[0], ph[1], ph[2], ph[3]);
  mid = make_uint4(pm[0], pm[1], pm[2], pm[3]);
  lo = make_uint4(pl[0], pl[1], pl[2], pl[3]);
}

// fp16 operands of v_mfma_f32_32x32x16_f16, laid out as mfma_bf16's.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x16 mfma_f16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x8 f16x8_of(uint4 v) { return __builtin_bit_cast(f16x8, v); }

// Two floats as packed fp16, round to nearest even.
__device__ __forceinline__ uint32_t cvt_pk_f16(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
}

// Eight floats as two fp16 octets with x = hi + 2^-11 lo to within 2^-22 |x|
// (the scaled-residual split of Ootomo and Yokota, IJHPCA 2022): hi rounds x
// to 11 significant bits, the remainder x - hi is exact and at most 2^-11 |x|,
// and lo rounds it scaled by 2^11.  Below fp16's normal range (|x| < 2^-14)
// hi is subnormal, which the fp16 MFMAs take exactly (checked on gfx950), and
// lo still carries the remainder, so the error stays below 2^-36 there;
// |x| >= 65520 gives an infinite hi.
__device__ __forceinline__ void split2_f16(float4 x0, float4 x1, uint4& hi, uint4& lo) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  uint32_t ph[4], pl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ph[i] = cvt_pk_f16(v[2 * i], v[2 * i + 1]);
    const h2 hv = __builtin_bit_cast(h2, ph[i]);
    pl[i] = cvt_pk_f16((v[2 * i] - (float)hv[0]) * 2048.f, (v[2 * i + 1] - (float)hv[1]) * 2048.f);
  }
  hi = make_uint4(ph[0], ph[1], ph[2], ph[3]);
  lo = make_uint4(pl[0], pl[1], pl[2], pl[3]);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ int acc_row(int r, int h) {
  return (r >> 2) * 8 + h * 4 + (r & 3);
}


// x of the lane that DPP control CTRL selects within the lane's 16-lane row
// (a VALU operand modifier: no LDS crossbar traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// x[lane] + x[lane ^ O] and max(x[lane], x[lane ^ O]) for O = 16 or 32, on
// gfx950's permlane swaps (VALU, no LDS crossbar).  Swapping x with itself
// leaves, across the two results, x of the lane and of its partner in an
// order that depends on the lane: v_permlane16_swap exchanges the odd
// 16-lane rows of its first operand with the even rows of its second,
// v_permlane32_swap the upper 32 lanes of the first with the lower 32 of
// the second.  The sum and max of the pair are commutative, so both
// partners get the same value.
template <int O>
__device__ __forceinline__ void xor_pair(float x, float& a, float& b) {
  static_assert(O == 16 || O == 32, "permlane swaps pair lanes 16 or 32 apart");
  const uint32_t u = __float_as_uint(x);
  if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  }
}
template <int O>
__device__ __forceinline__ float xor_sum(float x) {
  float a, b;
  xor_pair<O>(x, a, b);
  return a + b;
}
template <int O>
__device__ __forceinline__ float xor_max(float x) {
  float a, b;
  xor_pair<O>(x, a, b);
  return fmaxf(a, b);
}

// Sum over aligned groups of N lanes (N a power of two <= 64); every lane of
// a group receives the same total.  Within a 16-lane row the partners come
// from DPP: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (lane 7 - i of each 8, pairing the two quads) and
// row_mirror (lane 15 - i, pairing the two halves); each step adds two
// partial sums that already agree across the lanes being paired.  Wider
// groups add lane ^ 16 and lane ^ 32 by permlane swaps.  Every lane of the
// wave must be active (the callers reduce in uniform control flow).
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N is a power of two <= 64");
  if constexpr (N >= 2) v += dpp_f32<0xB1>(v);
  if constexpr (N >= 4) v += dpp_f32<0x4E>(v);
  if constexpr (N >= 8) v += dpp_f32<0x141>(v);
  if constexpr (N >= 16) v += dpp_f32<0x140>(v);
  if constexpr (N >= 32) v = xor_sum<16>(v);
  if constexpr (N >= 64) v = xor_sum<32>(v);
  return v;
}

// Maximum over aligned groups of N lanes, the partners of group_sum.
template <int N>
__device__ __forceinline__ float group_max(float v) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N is a power of two <= 64");
  if constexpr (N >= 2) v = fmaxf(v, dpp_f32<0xB1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp_f32<0x4E>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp_f32<0x141>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp_f32<0x140>(v));
  if constexpr (N >= 32) v = xor_max<16>(v);
  if constexpr (N >= 64) v = xor_max<32>(v);
  return v;
}

// Sum and maximum over the wave; every lane receives the result.
#ifndef AKH_WAVE_DPP
#define AKH_WAVE_DPP 1
#endif
__device__ __forceinline__ float wave_sum(float v) {
  if constexpr (AKH_WAVE_DPP) return group_sum<64>(v);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  if constexpr (AKH_WAVE_DPP) return group_max<64>(v);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}


// Reductions over a 256-thread block; every thread gets the result.  The
// order is fixed (butterfly in waves, then waves 0..3), so results are
// reproducible run to run.
__device__ __forceinline__ float block_sum256(float v, float* red4) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  return ((red4[0] + red4[1]) + red4[2]) + red4[3];
}

__device__ __forceinline__ float block_max256(float v, float* red4) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
}

// (x0*c - x1*s, x0*s + x1*c) with every product rounded separately, as the
// reference's CPU RoPE computes it (src/shaders/cpu.rs:102-103).
__device__ __forceinline__ void rope_pair(float& x0, float& x1, float c,
                                          float s) {
  const float a = __fmul_rn(x0, c), b = __fmul_rn(x1, s);
  const float e = __fmul_rn(x0, s), f = __fmul_rn(x1, c);
  x0 = __fsub_rn(a, b);
  x1 = __fadd_rn(e, f);
}

// Greedy-argmax merge (src/nn/sampling.rs:83-91 picks the first index of
// the maximum): larger value wins, equal values keep the lower index, which
// equals the sequential strict-> scan for any split of the row.
__device__ __forceinline__ void amax_merge(float& bv, uint32_t& bi, float v,
                                           uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__device__ __forceinline__ void block_amax256(float& bv, uint32_t& bi) {
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

// Index of element (row m, column k) of a 32-row activation tile stored in
// the k-quad layout [K/4][32][4]: a half-wave reading four consecutive k of
// its 32 rows touches 512 contiguous bytes.
__device__ __forceinline__ size_t kq_index(int m, int k) {
  return ((size_t)(k >> 2) * 32 + m) * 4 + (k & 3);
}

__device__ __forceinline__ void add4(float4& a, const float4 b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

// acc + p[0] + p[stride] + ... + p[(n - 1) * stride], added in index order.
// The loads are issued NB at a time, the remainder (fewer than NB) as one
// more batch, so up to NB partials cost one memory latency instead of NB
// dependent ones.
template <int NB>
__device__ __forceinline__ float4 sum_parts4(float4 acc, const float* p,
                                             size_t stride, int n) {
  int s = 0;
  for (; s + NB <= n; s += NB) {
    float4 t[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
      t[i] = *reinterpret_cast<const float4*>(p + (size_t)(s + i) * stride);
#pragma unroll
    for (int i = 0; i < NB; ++i) add4(acc, t[i]);
  }
  if (s < n) {
    float4 t[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
      if (s + i < n) t[i] = *reinterpret_cast<const float4*>(p + (size_t)(s + i) * stride);
#pragma unroll
    for (int i = 0; i < NB; ++i)
      if (s + i < n) add4(acc, t[i]);
  }
  return acc;
}

// sum_parts4 issuing NB1 loads at a time while at least NB1 remain, then NB2.
template <int NB1, int NB2>
__device__ __forceinline__ float4 sum_parts4_2(float4 acc, const float* p, size_t stride,
                                               int n) {
  int s = 0;
  for (; s + NB1 <= n; s += NB1) {
    float4 t[NB1];
#pragma unroll
    for (int i = 0; i < NB1; ++i)
      t[i] = *reinterpret_cast<const float4*>(p + (size_t)(s + i) * stride);
#pragma unroll
    for (int i = 0; i < NB1; ++i) add4(acc, t[i]);
  }
  return sum_parts4<NB2>(acc, p + (size_t)s * stride, stride, n - s);
}

}  // namespace akh
