// Batched decode kernels: every sequence of a step is one row of a 32-row
// MFMA tile (two tiles for 33..64 sequences), so each weight byte is read
// once per step for the whole batch.
//
// Dataflow of one layer (B <= 64 rows):
//
//   xn_t --qkv GEMM--> P_qkv --attention (sum, RoPE, KV append)--> attn_t
//   attn_t --out GEMM--> P_out --rows_norm (x += sum, RMSNorm)--> x_t, xn_t
//   xn_t --up GEMM--> P_up_t --down GEMM (A = silu(sum))--> P_down
//   P_down --rows_norm (x += sum, next RMSNorm)--> x_t, xn_t
//
// Activations that feed a GEMM live in the k-quad layout [R/32][K/4][32][4]:
// the MFMA A operand of a half-wave is one contiguous 512-byte float4 load
// per four k.  A decode GEMM moves only a few MB, so the kernels split K
// over many small blocks (the whole GPU works on each GEMM) and store
// partial tiles; the consumer of each GEMM sums the partials in a fixed
// order, so results are deterministic.  In this default dataflow nothing
// synchronises across work-groups inside a kernel.  The optional fused norm
// (DEC_RESID / PRO_NORM) folds each rows_norm into the GEMMs around it; its
// residual epilogue counts finished blocks with one atomic per block and
// sums the partials in split order, so it is deterministic too.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace akh {

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// SiLU where ffn_down loads its A operand: each of its column tiles evaluates
// it again over its whole K chunk, so it must be cheap in VALU issue.
// x / (1 + e^-x) as x * rcp(1 + 2^(-x log2 e)) on the hardware exp2 and
// reciprocal: five instructions instead of about 35 for expf and an IEEE
// division, within a few ulp of it (the decode parity bar is 1e-3 on logits).
__device__ __forceinline__ float silu_fast(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.44269504088896341f));
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

// One-time packing of a [K, N] row-major matrix into 32-column tiles of
// Kp rows in the k-quad order (see launch_pack_tiles in kernels.h).
__global__ __launch_bounds__(256) void k_pack_tiles(const float* __restrict__ w, int K,
                                                    int N, int Kp, float* __restrict__ out) {
  const int j = threadIdx.x & 31;
  const int q = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int t = blockIdx.y;
  if (4 * q >= Kp) return;
  const int n = t * 32 + j;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < N) {
    const int k = 4 * q;
    if (k < K) v.x = w[(size_t)k * N + n];
    if (k + 1 < K) v.y = w[(size_t)(k + 1) * N + n];
    if (k + 2 < K) v.z = w[(size_t)(k + 2) * N + n];
    if (k + 3 < K) v.w = w[(size_t)(k + 3) * N + n];
  }
  *reinterpret_cast<float4*>(out + (((size_t)t * (Kp / 4) + q) * 32 + j) * 4) = v;
}

// Split-fp16 lm_head tiles (launch_pack_lm_h3): one thread per (k-octet,
// column), 32 bytes out (hi octet, then lo octet).
__global__ __launch_bounds__(256) void k_pack_lm_h3(const float* __restrict__ w, int K, int N,
                                                    int Kp, uint16_t* __restrict__ out,
                                                    int* __restrict__ flag) {
  const int j = threadIdx.x & 31;
  const int o = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int t = blockIdx.y;
  if (8 * o >= Kp) return;
  const int n = t * 32 + j;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * o + e;
    x[e] = n < N && k < K ? w[(size_t)k * N + n] : 0.f;
  }
  uint4 hi, lo;
  split2_f16(make_float4(x[0], x[1], x[2], x[3]), make_float4(x[4], x[5], x[6], x[7]), hi, lo);
  bool ok = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) ok = ok && fabsf(x[e]) < 65504.f;
  if (!ok) *flag = 1;
  uint4* dst = reinterpret_cast<uint4*>(out + (((size_t)t * (Kp / 8) + o) * 32 + j) * 16);
  dst[0] = hi;
  dst[1] = lo;
}

// The same tiles with bfloat16 elements in k-octets: element (k, n) of tile
// t = n / 32 at ((k / 8) * 32 + n % 32) * 8 + k % 8, so a lane's 16-byte load
// holds eight consecutive k of its column.  Used only for matrices whose
// every value is a bfloat16 (low 16 bits zero), so the conversion is exact.
__global__ __launch_bounds__(256) void k_pack_tiles_bf16(const float* __restrict__ w, int K,
                                                         int N, int Kp,
                                                         uint16_t* __restrict__ out) {
  const int j = threadIdx.x & 31;
  const int o = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int t = blockIdx.y;
  if (8 * o >= Kp) return;
  const int n = t * 32 + j;
  uint32_t v[4] = {0u, 0u, 0u, 0u};
  if (n < N) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = 8 * o + e;
      const uint32_t bits = k < K ? __float_as_uint(w[(size_t)k * N + n]) >> 16 : 0u;
      v[e / 2] |= bits << (16 * (e % 2));
    }
  }
  *reinterpret_cast<uint4*>(out + (((size_t)t * (Kp / 8) + o) * 32 + j) * 8) =
      make_uint4(v[0], v[1], v[2], v[3]);
}

// flag = 1 if any of the n values has nonzero low 16 bits (not a bfloat16).
__global__ __launch_bounds__(256) void k_check_bf16(const uint32_t* __restrict__ w, size_t n,
                                                    int* flag) {
  uint32_t any = 0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    any |= w[i] & 0xFFFFu;
  if (__any(any != 0) && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

__device__ __forceinline__ float4 bf16x4(uint32_t lo, uint32_t hi) {
  return make_float4(__uint_as_float(lo << 16), __uint_as_float(lo & 0xFFFF0000u),
                     __uint_as_float(hi << 16), __uint_as_float(hi & 0xFFFF0000u));
}

// Y (epilogue) A[M, K] . W[K, N] for M <= 32 * MT, W packed in 32-column
// tiles.  The rows are MT tiles of 32 (activations [MT][K/4][32][4], row m
// in tile m / 32); each weight load feeds the MFMAs of every row tile, so
// the weights are read once for up to 64 rows.
//
// Grid (N / 32 tiles, K chunks), W waves per block.  Lane (j, h) owns column
// 32 * tile + j.  A pass covers KC = 2*W*HL rows of K: wave w takes 2*HL of
// them and half h of its lanes HL, loading, per four rows, one float4 of the
// packed weight tile (its column, four consecutive k) and one float4 of the
// k-quad activation (its row m = j, the same four k); a half-wave's load is
// 512 contiguous bytes.  All loads of a pass are issued before its first
// MFMA.  A block runs one pass when K is split over the grid, and loops over
// all of K otherwise.  Partial-tile epilogues write every wave's 32x32 tile
// to LDS behind one barrier, then wave w sums rows [w * 32 / W, (w + 1) *
// 32 / W) over the waves in index order; the logits epilogue reduces the
// waves' tiles as a binary tree (fixed order) and wave 0 finishes it.
//
// PRO_SILU_SUM: A = silu(sum of p.nparts k-quad partial tiles at p.xt).
// PRO_NORM: A = RMSNorm of the residual rows at p.xt (see DecGemmParams).
// DEC_RESID: k-quad partial tiles, then the last block of each column tile
// adds their sum to the residual p.res and writes the per-row sums of
// squares of its 32 columns (one split: done directly in the epilogue).
// BF: W is packed in bfloat16 k-octets (k_pack_tiles_bf16); a lane loads
// eight k per 16 bytes.  Its octet and the same eight k of its row of A are
// the operands of v_mfma_f32_32x32x16_bf16, with A split exactly into three
// bfloat16 terms (split3_bf16): every product is exact, so the result has
// fp32 accuracy at 3 x 32 instead of 8 x 64 MFMA cycles per 16 k.
#ifndef AKH_GEMM_NT
#define AKH_GEMM_NT 1
#endif
#ifndef AKH_DEC_PIPE
#define AKH_DEC_PIPE 1
#endif
#ifndef AKH_LM_GEMM_NT
#define AKH_LM_GEMM_NT 0
#endif
// The attention's softmax runs in the log2 domain: scores scaled by
// scale * log2(e), weights from the hardware 2^x (one v_exp_f32 against
// about 35 instructions for expf).  The split states (max, sum) it hands to
// out_proj's merge are in the same units.
#ifndef AKH_ATTN_EXP2
#define AKH_ATTN_EXP2 1
#endif
__device__ __forceinline__ float attn_exp(float x) {
  if constexpr (AKH_ATTN_EXP2)
    return __builtin_amdgcn_exp2f(x);
  else
    return expf(x);
}
__device__ __forceinline__ float attn_score_scale(float scale) {
  return AKH_ATTN_EXP2 ? scale * 1.44269504088896341f : scale;
}

//
// VB > 0: at most VB live rows (small batches), on the VALU instead of the
// MFMAs.  A 32-row MFMA tile spends the same matrix-pipe time on one live
// row as on 32, and that time sits on the decode step's critical path
// (ffn_up's 96 blocks: ~2.6 us of fp32 MFMAs per CU); the VALU computes only
// the live rows.  Lane (j, h) takes the dot products of rows 0..VB-1 with
// its column over its k-quads, the two halves are added, and the sums enter
// the MFMA accumulator layout (row h*4 + r in entry r) so the epilogues are
// unchanged.
template <int W, int HL, int EPI, int PRO, bool BF, int MT, int NT = 1, int VB = 0>
__global__ __launch_bounds__(64 * W) void k_dec_gemm(DecGemmParams p) {
  constexpr int KC = 2 * W * HL;
  constexpr int HQ = HL / 4;
  constexpr int R = 32 * MT;  // rows of the activation and partial tiles
  static_assert(HL % 4 == 0, "HL must cover whole k-quads");
  static_assert(!BF || HL % 8 == 0, "bfloat16 tiles need whole k-octets");
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16, "W must be a power of 2 <= 16");
  static_assert(MT == 1 || MT == 2, "one or two row tiles");
  static_assert(EPI != DEC_RESID || W > 1, "the residual epilogue reduces across waves");
  static_assert(NT == 1 || NT == 2, "one or two column tiles");
  static_assert(NT == 1 || (EPI != DEC_RESID && PRO != PRO_NORM),
                "the residual epilogue and the norm prologue work per column tile");
  __shared__ float red[W][32][33];
  // PRO_NORM: per-row sums of four column tiles, and the rows' scales.
  __shared__ float nsum[PRO == PRO_NORM ? R : 1][33];
  __shared__ float nrs[PRO == PRO_NORM ? R : 1];
  __shared__ int last_block;

  const int M = p.M, N = p.N, K = p.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  // The block's column tiles: tile, tile + 1, ... tile + NT - 1.
  const int ntiles = (N + 31) / 32;
  const int tile = blockIdx.x * NT;
  const int rows = p.kpass * KC;  // whole passes per block
  const int kb = blockIdx.y * rows;
  if (kb >= K) return;
  const int ke = min(K, kb + rows);
  const float* wt = p.w + (size_t)tile * p.Kp * 32 + j * 4;
  const uint16_t* wh = reinterpret_cast<const uint16_t*>(p.w) + (size_t)tile * p.Kp * 32 + j * 8;
  // Offset of column tile tile + nt's weights from wt / wh (elements); a
  // tile past the last reads the last one's and stores nothing.
  auto wofs = [&](int nt) { return (size_t)(min(tile + nt, ntiles - 1) - tile) * p.Kp * 32; };

  f32x16 acc[MT * NT];  // [row tile][column tile]
#pragma unroll
  for (int i = 0; i < MT * NT; ++i) acc[i] = zero16();
  if constexpr (VB > 0) {
    static_assert(VB <= 8 && MT == 1 && NT == 1 && !BF && PRO != PRO_NORM,
                  "the VALU rows serve one tile of float weights");
    constexpr bool kNT = AKH_GEMM_NT && EPI != DEC_LOGITS;
    typedef float f4 __attribute__((ext_vector_type(4)));
    // A's four k of row `row` at k-quad kq (in range).
    auto a_quad = [&](int kq, int row) -> float4 {
      const size_t off = ((size_t)kq * 32 + row) * 4;
      float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (PRO == PRO_SILU_SUM) {
        t = sum_parts4<4>(t, p.xt + off, (size_t)R * K, p.nparts);
        t = make_float4(silu_fast(t.x), silu_fast(t.y), silu_fast(t.z), silu_fast(t.w));
      } else if constexpr (PRO == PRO_ATTN_MERGE) {
        // The attention splits' softmax states of (row, head (4 kq) / hd),
        // merged as in the MFMA path.
        const int H = K / p.hd, hq = (4 * kq) / p.hd;
        float mx = -INFINITY;
        float2 ml[kMaxAttnSplits];
#pragma unroll
        for (int sp = 0; sp < kMaxAttnSplits; ++sp) {
          ml[sp] = sp < p.nparts ? p.ml[((size_t)sp * H + hq) * R + row]
                                 : make_float2(-INFINITY, 0.f);
          mx = fmaxf(mx, ml[sp].x);
        }
        float L = 0.f;
#pragma unroll
        for (int sp = 0; sp < kMaxAttnSplits; ++sp) {
          if (sp >= p.nparts) continue;
          const float4 o = *reinterpret_cast<const float4*>(p.xt + (size_t)sp * R * K + off);
          const float w = ml[sp].x == -INFINITY ? 0.f : attn_exp(ml[sp].x - mx);
          L += w * ml[sp].y;
          t.x += w * o.x;
          t.y += w * o.y;
          t.z += w * o.z;
          t.w += w * o.w;
        }
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        t = make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv);
      } else {
        t = *reinterpret_cast<const float4*>(p.xt + off);
      }
      return t;
    };
    float sum[VB];
#pragma unroll
    for (int b = 0; b < VB; ++b) sum[b] = 0.f;
    for (int k0 = kb; k0 < ke; k0 += KC) {
      const int kq0 = (k0 + wave * 2 * HL + h * HL) >> 2;
      float4 wq[HQ], aq[VB][HQ];
#pragma unroll
      for (int q = 0; q < HQ; ++q) {
        const int kq = kq0 + q;
        const f4* src = reinterpret_cast<const f4*>(wt + (size_t)kq * 128);
        const f4 t = 4 * kq < ke ? (kNT ? __builtin_nontemporal_load(src) : *src)
                                 : f4{0.f, 0.f, 0.f, 0.f};
        wq[q] = make_float4(t.x, t.y, t.z, t.w);
      }
#pragma unroll
      for (int q = 0; q < HQ; ++q)
#pragma unroll
        for (int b = 0; b < VB; ++b)
          aq[b][q] = 4 * (kq0 + q) < ke ? a_quad(kq0 + q, b) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int q = 0; q < HQ; ++q)
#pragma unroll
        for (int b = 0; b < VB; ++b) {
          sum[b] = fmaf(aq[b][q].x, wq[q].x, sum[b]);
          sum[b] = fmaf(aq[b][q].y, wq[q].y, sum[b]);
          sum[b] = fmaf(aq[b][q].z, wq[q].z, sum[b]);
          sum[b] = fmaf(aq[b][q].w, wq[q].w, sum[b]);
        }
    }
    // The two halves of the wave took different k: add them, then lane
    // (j, h) holds rows h*4 .. h*4 + 3 in accumulator entries 0..3.
#pragma unroll
    for (int b = 0; b < VB; ++b) sum[b] += __shfl_xor(sum[b], 32, 64);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v0 = r < VB ? sum[r < VB ? r : 0] : 0.f;
      const float v1 = 4 + r < VB ? sum[4 + r < VB ? 4 + r : 0] : 0.f;
      acc[0][r] = h == 0 ? v0 : v1;
    }
  } else if constexpr (PRO == PRO_NONE && MT == 1 && NT == 1 && AKH_DEC_PIPE) {
    // Plain A, one row tile: the loads of pass i + 1 are issued before the
    // MFMAs of pass i, so a block waits on one memory round trip, not one per
    // pass.  Loads past K read the block's last valid quad (clamped, always
    // issued, so the wait counts are static) and are zeroed where they are
    // used.  Measured on MI355X: config 4's qkv 5.5 -> 4.9 us, ffn_up 5.7 ->
    // 5.3 us, its step 0.641 -> 0.632 ms.  With two row tiles the second
    // register set costs occupancy: config 5's qkv went 13.7 -> 15.4 us and
    // its lm_head 82 -> 97 us, so two-tile blocks keep the loop below.
    constexpr bool kNT = AKH_GEMM_NT && (AKH_LM_GEMM_NT || EPI != DEC_LOGITS);
    using WRaw = typename std::conditional<BF, uint4, float4>::type;
    constexpr int NW = BF ? HQ / 2 : HQ;
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int kqe = (ke >> 2) - 1;  // last valid k-quad
    WRaw wc[2][NW];
    float4 a[2][MT][HQ];
    auto load_pass = [&](int k0, int set) {
      const int kq0 = (k0 + wave * 2 * HL + h * HL) >> 2;
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const int kq = min(kq0 + (BF ? 2 * i : i), BF ? (kqe & ~1) : kqe);
        const f4* src = reinterpret_cast<const f4*>(
            BF ? static_cast<const void*>(wh + (size_t)kq * 128)
               : static_cast<const void*>(wt + (size_t)kq * 128));
        wc[set][i] = __builtin_bit_cast(WRaw, kNT ? __builtin_nontemporal_load(src) : *src);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < HQ; ++q) {
          const int kq = min(kq0 + q, kqe);
          a[set][mt][q] = *reinterpret_cast<const float4*>(
              p.xt + (size_t)mt * 32 * K + ((size_t)kq * 32 + j) * 4);
        }
    };
    auto mma_pass = [&](int k0, int set) {
      const int kq0 = (k0 + wave * 2 * HL + h * HL) >> 2;
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (BF) {
#pragma unroll
          for (int q = 0; q < HQ; q += 2) {
            const bool in = 4 * (kq0 + q) < ke, in1 = 4 * (kq0 + q + 1) < ke;
            const bf16x8 w8 = bf16x8_of(in ? wc[set][q / 2] : make_uint4(0u, 0u, 0u, 0u));
            uint4 hi, mid, lo;
            split3_bf16(in ? a[set][mt][q] : z, in1 ? a[set][mt][q + 1] : z, hi, mid, lo);
            acc[mt] = mfma_bf16(bf16x8_of(hi), w8, acc[mt]);
            acc[mt] = mfma_bf16(bf16x8_of(mid), w8, acc[mt]);
            acc[mt] = mfma_bf16(bf16x8_of(lo), w8, acc[mt]);
          }
        } else {
#pragma unroll
          for (int q = 0; q < HQ; ++q) {
            const bool in = 4 * (kq0 + q) < ke;
            const float4 x = in ? a[set][mt][q] : z, w = in ? wc[set][q] : z;
            acc[mt] = mfma32(x.x, w.x, acc[mt]);
            acc[mt] = mfma32(x.y, w.y, acc[mt]);
            acc[mt] = mfma32(x.z, w.z, acc[mt]);
            acc[mt] = mfma32(x.w, w.w, acc[mt]);
          }
        }
      }
    };
    const int np = (ke - kb + KC - 1) / KC;  // passes of this block
    load_pass(kb, 0);
    int i = 0;
    for (; i + 2 <= np; i += 2) {
      load_pass(kb + (i + 1) * KC, 1);
      mma_pass(kb + i * KC, 0);
      if (i + 2 < np) load_pass(kb + (i + 2) * KC, 0);
      mma_pass(kb + (i + 1) * KC, 1);
    }
    if (i < np) mma_pass(kb + i * KC, 0);
  } else
  for (int k0 = kb; k0 < ke; k0 += KC) {
    const int kq0 = (k0 + wave * 2 * HL + h * HL) >> 2;  // first k-quad of this half
    // PRO_NORM: the RMSNorm scale of every row from the residual's
    // per-column-tile sums of squares [R][K / 32].  The block loads them in
    // one batch (a float4 of four tiles per thread) ahead of the pass's
    // weights: memory counters retire in order, so waiting for them does
    // not wait for the weights.
    constexpr int NL = PRO == PRO_NORM ? (R * 32 + 64 * W - 1) / (64 * W) : 1;
    const int nq = K >> 7;  // float4 of sums per row (K % 128 == 0, K <= 4096)
    float4 v[NL];
    if constexpr (PRO == PRO_NORM) {
      if (k0 == kb) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
          const int e = threadIdx.x + i * 64 * W;
          v[i] = e < R * nq ? *reinterpret_cast<const float4*>(p.ssq + 4 * (size_t)e)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
    // The pass's weights: bfloat16 octets or float quads, read once per
    // step, so non-temporal in the layer GEMMs (a measured 2 % per decode
    // step, though each GEMM alone is a little slower).  The lm_head (many
    // passes per block) streams better through the caches.
    constexpr bool kNT = AKH_GEMM_NT && (AKH_LM_GEMM_NT || EPI != DEC_LOGITS);
    using WRaw = typename std::conditional<BF, uint4, float4>::type;
    constexpr int NW = BF ? HQ / 2 : HQ;
    typedef float f4 __attribute__((ext_vector_type(4)));
    WRaw wc[NT][NW];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int kq = kq0 + (BF ? 2 * i : i);  // BF: even, HL is a multiple of 8
      const size_t wo = wofs(nt) + (size_t)kq * 128;
      const f4* src = reinterpret_cast<const f4*>(BF ? static_cast<const void*>(wh + wo)
                                                     : static_cast<const void*>(wt + wo));
      const f4 t = 4 * kq < ke ? (kNT ? __builtin_nontemporal_load(src) : *src)
                               : f4{0.f, 0.f, 0.f, 0.f};
      wc[nt][i] = __builtin_bit_cast(WRaw, t);
    }
    float4 g[HQ];  // PRO_NORM: the gain of the pass's k
    if constexpr (PRO == PRO_NORM) {
#pragma unroll
      for (int q = 0; q < HQ; ++q) {
        const int kq = kq0 + q;
        g[q] = 4 * kq < ke ? *reinterpret_cast<const float4*>(p.gain + 4 * kq)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float4 a[MT][HQ];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
      const int kq = kq0 + q;
      float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
      if (4 * kq < ke) {
        // Row 32 mt + j of the k-quad tiles; partial tiles / splits R * K apart.
        const size_t off = (size_t)mt * 32 * K + ((size_t)kq * 32 + j) * 4;
        if (PRO == PRO_SILU_SUM) {
          t = sum_parts4<4>(t, p.xt + off, (size_t)R * K, p.nparts);
          t = make_float4(silu_fast(t.x), silu_fast(t.y), silu_fast(t.z), silu_fast(t.w));
        } else if (PRO == PRO_ATTN_MERGE) {
          // Softmax states (max, sum, unnormalised o) of the attention
          // splits of row 32 mt + j, head (4 kq) / hd:
          // o = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(max_s - max)
          // (2^(max_s - max): the attention keeps its maxima in log2 units).
          const int H = K / p.hd, hq = (4 * kq) / p.hd;
          float2 ml[kMaxAttnSplits];
          float4 o[kMaxAttnSplits];
#pragma unroll
          for (int sp = 0; sp < kMaxAttnSplits; ++sp) {
            const bool in = sp < p.nparts;
            ml[sp] = in ? p.ml[((size_t)sp * H + hq) * R + mt * 32 + j]
                        : make_float2(-INFINITY, 0.f);
            o[sp] = in ? *reinterpret_cast<const float4*>(p.xt + (size_t)sp * R * K + off)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
          }
          float mx = ml[0].x;
#pragma unroll
          for (int sp = 1; sp < kMaxAttnSplits; ++sp) mx = fmaxf(mx, ml[sp].x);
          float L = 0.f;
#pragma unroll
          for (int sp = 0; sp < kMaxAttnSplits; ++sp) {
            const float w = ml[sp].x == -INFINITY ? 0.f : attn_exp(ml[sp].x - mx);
            L += w * ml[sp].y;
            t.x += w * o[sp].x;
            t.y += w * o[sp].y;
            t.z += w * o[sp].z;
            t.w += w * o[sp].w;
          }
          const float inv = L > 0.f ? 1.0f / L : 0.f;
          t = make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv);
        } else {
          t = *reinterpret_cast<const float4*>(p.xt + off);  // PRO_NORM: the residual
        }
      }
      a[mt][q] = t;
    }
    if constexpr (PRO == PRO_NORM) {
      if (k0 == kb) {
        // Each float4 summed, then one thread per row adds its row's K / 128
        // sums in order.
#pragma unroll
        for (int i = 0; i < NL; ++i) {
          const int e = threadIdx.x + i * 64 * W;
          if (e < R * nq) nsum[e / nq][e % nq] = ((v[i].x + v[i].y) + v[i].z) + v[i].w;
        }
        __syncthreads();
        if (threadIdx.x < R) {
          float ss = 0.f;
          for (int c = 0; c < nq; ++c) ss += nsum[threadIdx.x][c];
          nrs[threadIdx.x] = 1.0f / sqrtf(ss / (float)K + p.eps);
        }
        __syncthreads();
      }
      // A = (x * rs) * gain, as the RMSNorm kernel rounds it.
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float rs = nrs[mt * 32 + j];
#pragma unroll
        for (int q = 0; q < HQ; ++q) {
          const float4 x = a[mt][q];
          a[mt][q] = make_float4(__fmul_rn(__fmul_rn(x.x, rs), g[q].x),
                                 __fmul_rn(__fmul_rn(x.y, rs), g[q].y),
                                 __fmul_rn(__fmul_rn(x.z, rs), g[q].z),
                                 __fmul_rn(__fmul_rn(x.w, rs), g[q].w));
        }
      }
    }
    // Each split of A feeds the MFMAs of all NT column tiles.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (BF) {
#pragma unroll
        for (int q = 0; q < HQ; q += 2) {
          uint4 hi, mid, lo;
          split3_bf16(a[mt][q], a[mt][q + 1], hi, mid, lo);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            f32x16& c = acc[mt * NT + nt];
            const bf16x8 w8 = bf16x8_of(wc[nt][q / 2]);
            c = mfma_bf16(bf16x8_of(hi), w8, c);
            c = mfma_bf16(bf16x8_of(mid), w8, c);
            c = mfma_bf16(bf16x8_of(lo), w8, c);
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < HQ; ++q)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            f32x16& c = acc[mt * NT + nt];
            c = mfma32(a[mt][q].x, wc[nt][q].x, c);
            c = mfma32(a[mt][q].y, wc[nt][q].y, c);
            c = mfma32(a[mt][q].z, wc[nt][q].z, c);
            c = mfma32(a[mt][q].w, wc[nt][q].w, c);
          }
      }
    }
  }

  if (W > 1 && EPI != DEC_LOGITS) {
    // Partial tiles: every wave's 32x32 tile goes to LDS behind one barrier,
    // then wave w sums rows [w * 32 / W, (w + 1) * 32 / W) over the waves in
    // index order and stores them (lane: column j, rows h, h + 2, ...).
    // Tile by tile (row tiles, then column tiles within each), one barrier
    // before each tile's reads and one before the next tile overwrites the
    // LDS.
    constexpr int RW = 32 / W;
#pragma unroll
    for (int pi = 0; pi < MT * NT; ++pi) {
      const int mt = pi / NT, ct = tile + pi % NT, cl = ct * 32 + j;
      if (pi > 0) __syncthreads();
#pragma unroll
      for (int r = 0; r < 16; ++r) red[wave][acc_row(r, h)][j] = acc[pi][r];
      __syncthreads();
      if (cl < N) {
#pragma unroll
        for (int i = 0; i < RW / 2; ++i) {
          const int ml = wave * RW + h + 2 * i, m = mt * 32 + ml;
          float v = red[0][ml][j];
#pragma unroll
          for (int w = 1; w < W; ++w) v += red[w][ml][j];
          if (EPI == DEC_RESID && rows >= K) {
            // One split: the block holds whole sums.  Residual add, and the
            // row's sum of squares over the tile's 32 columns (a butterfly
            // over the half-wave; lane 0's result is stored).
            float* rp = p.res + (size_t)mt * 32 * N + kq_index(ml, cl);
            const float r = *rp + v;
            *rp = r;
            float q2 = r * r;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) q2 += __shfl_xor(q2, o, 64);
            if (j == 0) p.ssq_out[(size_t)m * (N >> 5) + ct] = q2;
          } else if (EPI == DEC_PART)
            p.y[((size_t)blockIdx.y * R + m) * N + cl] = v;
          else if (EPI == DEC_PART_T)
            p.y[((size_t)blockIdx.y * R + mt * 32) * N + kq_index(ml, cl)] = v;
          else if (EPI == DEC_RESID)
            // Written through to device scope (a relaxed agent-scope atomic
            // store): no cache write-back is needed before the count below.
            __hip_atomic_store(p.y + ((size_t)blockIdx.y * R + mt * 32) * N + kq_index(ml, cl),
                               v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            p.y[(size_t)mt * 32 * N + kq_index(ml, cl)] = silu(v);
        }
      }
    }
    if constexpr (EPI == DEC_RESID) {
      if (rows >= K) return;  // one split: done above
      // The last of the column tile's blocks to finish adds the tile's
      // partials, in split order, to the residual, and writes the per-row
      // sums of squares of the tile's 32 new columns.  Each wave waits until
      // its device-scope stores have completed, the block meets, then one
      // thread counts the block; the last block reads the partials with
      // device-scope loads.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      const int nsplit = (K + rows - 1) / rows;
      if (threadIdx.x == 0) {
        const int done =
            __hip_atomic_fetch_add(p.count + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_block = done == nsplit - 1;
        if (last_block)  // zero for the next launch
          __hip_atomic_store(p.count + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!last_block) return;
      // One float4 (four columns of one row) per thread: row ml of row tile
      // mt, column quad cq of the tile; k-quad offsets equal in the partial
      // tiles (R * N apart) and the residual.
      constexpr int NE = R * 8;
      constexpr int NI = (NE + 64 * W - 1) / (64 * W);
      auto ld = [](const float* q) {
        return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      };
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int e = threadIdx.x + i * 64 * W;
        if (e < NE) {
          const int ml = e & 31, cq = (e >> 5) & 7, mt = e >> 8;
          const size_t off = (size_t)mt * 32 * N + ((size_t)(tile * 8 + cq) * 32 + ml) * 4;
          float4 v = *reinterpret_cast<const float4*>(p.res + off);
          for (int s0 = 0; s0 < nsplit; s0 += 8) {
            float4 t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const float* q = p.y + (size_t)(s0 + u) * R * N + off;
              t[u] = s0 + u < nsplit ? make_float4(ld(q), ld(q + 1), ld(q + 2), ld(q + 3))
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
              if (s0 + u < nsplit) add4(v, t[u]);
          }
          *reinterpret_cast<float4*>(p.res + off) = v;
          // e = (mt * 8 + cq) * 32 + ml: red viewed as [R / 32][8][32].
          (&red[0][0][0])[e] = ((v.x * v.x + v.y * v.y) + v.z * v.z) + v.w * v.w;
        }
      }
      __syncthreads();
      if (threadIdx.x < R) {
        const int mt = threadIdx.x >> 5, ml = threadIdx.x & 31;
        const float* sq = &red[0][0][0] + mt * 256 + ml;
        float ss = 0.f;
#pragma unroll
        for (int cq = 0; cq < 8; ++cq) ss += sq[cq * 32];
        p.ssq_out[(size_t)threadIdx.x * (N >> 5) + tile] = ss;
      }
    }
    return;
  }
#pragma unroll
  for (int pi = 0; pi < MT * NT; ++pi) {
    const int mt = pi / NT, ct = tile + pi % NT, cl = ct * 32 + j;
    const bool ck = cl < N;
    if (W > 1) {
      for (int half = W / 2; half >= 1; half >>= 1) {
        __syncthreads();
        if (wave >= half && wave < 2 * half)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[wave - half][acc_row(r, h)][j] = acc[pi][r];
        __syncthreads();
        if (wave < half)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[pi][r] += red[wave][acc_row(r, h)][j];
      }
    }
    if (wave != 0) continue;

    float bv = -INFINITY;
    uint32_t bi = (uint32_t)cl;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ml = acc_row(r, h), m = mt * 32 + ml;
      if (EPI == DEC_PART) {
        if (ck) p.y[((size_t)blockIdx.y * R + m) * N + cl] = acc[pi][r];
      } else if (EPI == DEC_PART_T) {
        if (ck) p.y[((size_t)blockIdx.y * R + mt * 32) * N + kq_index(ml, cl)] = acc[pi][r];
      } else if (EPI == DEC_SILU_T) {
        if (ck) p.y[(size_t)mt * 32 * N + kq_index(ml, cl)] = silu(acc[pi][r]);
      } else if (EPI == DEC_LOGITS) {
        // Logits, and the first maximum of the row over this tile's columns.
        bv = -INFINITY;
        bi = (uint32_t)cl;
        if (m < M && ck) {
          p.y[(size_t)m * N + cl] = acc[pi][r];
          bv = acc[pi][r];
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
          const float ov = __shfl_xor(bv, o, 64);
          const uint32_t oi = __shfl_xor(bi, o, 64);
          amax_merge(bv, bi, ov, oi);
        }
        if (j == 0 && m < M && ct < ntiles)
          p.amax[(size_t)m * ntiles + ct] = make_uint2(__float_as_uint(bv), bi);
      }
    }
  }
}

// lm_head (logits = A . W, K <= Kp = 2*W*HL) and the first maximum of every
// row, W packed in 32-column tiles of Kp rows (zero beyond K).
//
// A persistent grid of G blocks (one per CU): block b owns the tiles b, b+G,
// b+2G, ... in increasing order.  Wave w covers rows [2*HL*w, 2*HL*(w+1))
// and half h of its lanes HL of them, so its A operand (HL floats per lane)
// is loaded once and stays in registers.  The weights of the block's next
// tile are loaded while the MFMAs of the current one run, through a buffer
// resource: the lane's offset in the tile is one VGPR, the tile and k-quad
// offsets are scalar, and a tile past the end gets an offset outside the
// resource, which reads as zero without touching memory.  The W per-wave
// 32x32 tiles are summed in LDS (waves in order), each wave finishing 32/W
// rows: it stores their logits and keeps a running (value, index) maximum
// per row.  amax[m, b] is the first maximum of row m over block b's columns.
#ifndef AKH_LM_CPOL
#define AKH_LM_CPOL 0
#endif
template <int HQ>
__device__ __forceinline__ void lm_load_b(float4 (&bb)[HQ], __amdgpu_buffer_rsrc_t w,
                                          uint32_t voff, int ntiles, int Kp, int tile) {
  const uint32_t vo = tile < ntiles ? voff : 0x80000000u;
  const int so = tile * Kp * 128;
#pragma unroll
  for (int q = 0; q < HQ; ++q) {
    // Cache policy AKH_LM_CPOL: 0 (cached) measured faster per decode step
    // than 2 (non-temporal) here.
    const f32x4v v = __builtin_bit_cast(
        f32x4v, __builtin_amdgcn_raw_buffer_load_b128(w, (int)vo, so + q * 512, AKH_LM_CPOL));
    bb[q] = make_float4(v.x, v.y, v.z, v.w);
  }
}

// One row tile's logits of one column tile: the waves' 32x32 tiles are
// summed in LDS (waves in order), each wave finishing 32 / W rows.
template <int W>
__device__ __forceinline__ void lm_finish(const f32x16& acc, float (*red)[32][33], int tile,
                                          int row0, const DecGemmParams& p, float& bv,
                                          uint32_t& bi) {
  constexpr int RW = 32 / W;     // rows finished per wave
  constexpr int LPR = 64 / RW;   // lanes per finished row
  constexpr int E = 32 / LPR;    // columns per lane
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
#pragma unroll
  for (int r = 0; r < 16; ++r) red[wave][acc_row(r, h)][j] = acc[r];
  __syncthreads();
  const int ml = wave * RW + lane / LPR, m = row0 + ml;
  const int c0 = (lane % LPR) * E;
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = red[0][ml][c0 + e];
#pragma unroll
  for (int w = 1; w < W; ++w)
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] += red[w][ml][c0 + e];
  if (m < p.M) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int col = tile * 32 + c0 + e;
      if (col < p.N) {
        p.y[(size_t)m * p.N + col] = v[e];
        amax_merge(bv, bi, v[e], (uint32_t)col);
      }
    }
  }
}

// MT row tiles: A for all of them stays in registers and each weight tile
// feeds the MFMAs of every row tile, so the weights are read once.  The LDS
// buffers alternate per (column tile, row tile), so one barrier per row tile
// orders each buffer's reads before its next writes.
template <int W, int HL, int MT>
__global__ __launch_bounds__(64 * W) void k_dec_lm(DecGemmParams p) {
  constexpr int RW = 32 / W;
  constexpr int LPR = 64 / RW;
  constexpr int HQ = HL / 4;
  static_assert(W * RW == 32 && LPR <= 64, "W must divide 32");
  static_assert(HL % 4 == 0, "HL must cover whole k-quads");
  static_assert(MT == 1 || MT == 2, "one or two row tiles");
  __shared__ float red[2][W][32][33];
  const int N = p.N, K = p.K, Kp = p.Kp;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int ntiles = (N + 31) / 32;
  const int G = gridDim.x;
  const int kq0 = (wave * 2 * HL + h * HL) >> 2;  // first k-quad of this half
  const uint32_t voff = (uint32_t)(kq0 * 32 + j) * 16u;
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.w), (short)0, ntiles * Kp * 128, 0x00020000);

  float4 a[MT][HQ];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
      const int kq = kq0 + q;
      a[mt][q] = 4 * kq < K ? *reinterpret_cast<const float4*>(
                                  p.xt + (size_t)mt * 32 * K + ((size_t)kq * 32 + j) * 4)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    }

  float bv[MT];
  uint32_t bi[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    bv[mt] = -INFINITY;
    bi[mt] = 0xFFFFFFFFu;
  }
  // cur holds this tile's weights; nxt receives the next tile's while the
  // MFMAs run, and is handed over after the epilogue.
  float4 cur[HQ], nxt[HQ];
  lm_load_b(cur, wres, voff, ntiles, Kp, blockIdx.x);
  int par = 0;
#pragma unroll 1
  for (int tile = blockIdx.x; tile < ntiles; tile += G) {
    lm_load_b(nxt, wres, voff, ntiles, Kp, tile + G);
    // Compiler-only barrier: the prefetch stays issued here instead of being
    // sunk to its first use after the MFMAs (which would serialise it).
    asm volatile("" ::: "memory");
    f32x16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt] = zero16();
#pragma unroll
      for (int q = 0; q < HQ; ++q) {
        acc[mt] = mfma32(a[mt][q].x, cur[q].x, acc[mt]);
        acc[mt] = mfma32(a[mt][q].y, cur[q].y, acc[mt]);
        acc[mt] = mfma32(a[mt][q].z, cur[q].z, acc[mt]);
        acc[mt] = mfma32(a[mt][q].w, cur[q].w, acc[mt]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      lm_finish<W>(acc[mt], red[par], tile, 32 * mt, p, bv[mt], bi[mt]);
      par ^= 1;
    }
#pragma unroll
    for (int q = 0; q < HQ; ++q) cur[q] = nxt[q];
  }
  // First maximum of each finished row over this block's columns.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv[mt], o, 64);
      const uint32_t oi = __shfl_xor(bi[mt], o, 64);
      amax_merge(bv[mt], bi[mt], ov, oi);
    }
    const int m = 32 * mt + wave * RW + lane / LPR;
    if (lane % LPR == 0 && m < p.M)
      p.amax[(size_t)m * G + blockIdx.x] = make_uint2(__float_as_uint(bv[mt]), bi[mt]);
  }
}

// k_dec_lm on split-fp16 tiles (k_pack_lm_h3): the same persistent grid,
// prefetch and epilogue, with each 16-k step of a row tile three
// v_mfma_f32_32x32x16_f16 products (hi.hi into acc, hi.lo and lo.hi into
// cor; the result is acc + 2^-11 cor, error ~2^-22 relative) instead of
// sixteen fp32 MFMAs of twice the cycles.  The weights take the same 4
// bytes per element.  A is split once: the block scales it by 2^-S, S the
// smallest shift that brings max |A| under 2^15 (0 for any ordinary row),
// so its fp16 terms cannot overflow, and scales the results back by 2^S
// (both exact).  Half h of a wave's lanes covers k [2 HL w + HL h, + HL) as
// in k_dec_lm, eight k per step.
template <int W, int HL, int MT>
__global__ __launch_bounds__(64 * W) void k_dec_lm_h3(DecGemmParams p) {
  constexpr int RW = 32 / W;
  constexpr int LPR = 64 / RW;
  constexpr int NS = HL / 8;  // 16-k MFMA steps per tile
  static_assert(W * RW == 32 && LPR <= 64, "W must divide 32");
  static_assert(HL % 8 == 0, "HL must cover whole k-octets");
  static_assert(MT == 1 || MT == 2, "one or two row tiles");
  __shared__ float red[2][W][32][33];
  __shared__ float amx[W];
  const int N = p.N, K = p.K, Kp = p.Kp;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int ntiles = (N + 31) / 32;
  const int G = gridDim.x;
  const int k0 = wave * 2 * HL + h * HL;  // first k of this half
  // Lane offset within a tile: octet k0 / 8 + s, column j, 32 bytes each.
  const uint32_t voff = (uint32_t)((k0 / 8) * 32 + j) * 32u;
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.w), (short)0, ntiles * Kp * 128, 0x00020000);

  float4 af[MT][2 * NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 2 * NS; ++q) {
      const int kq = k0 / 4 + q;
      af[mt][q] = 4 * kq < K ? *reinterpret_cast<const float4*>(
                                   p.xt + (size_t)mt * 32 * K + ((size_t)kq * 32 + j) * 4)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  // Block scale: max |A| over the block (every block holds all of A).
  float mx = 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 2 * NS; ++q)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(af[mt][q].x), fabsf(af[mt][q].y)),
                           fmaxf(fabsf(af[mt][q].z), fabsf(af[mt][q].w))));
  mx = wave_max(mx);
  if (lane == 0) amx[wave] = mx;
  __syncthreads();
  mx = amx[0];
#pragma unroll
  for (int w = 1; w < W; ++w) mx = fmaxf(mx, amx[w]);
  float down = 1.f, up = 1.f;
  if (mx >= 32768.f && mx <= 3.0e38f) {
    int e;
    frexpf(mx, &e);  // mx < 2^e
    down = ldexpf(1.f, 15 - e);
    up = ldexpf(1.f, e - 15);
  }
  uint4 ah[MT][NS], al[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float4 x0 = af[mt][2 * s], x1 = af[mt][2 * s + 1];
      split2_f16(make_float4(x0.x * down, x0.y * down, x0.z * down, x0.w * down),
                 make_float4(x1.x * down, x1.y * down, x1.z * down, x1.w * down), ah[mt][s],
                 al[mt][s]);
    }

  float bv[MT];
  uint32_t bi[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    bv[mt] = -INFINITY;
    bi[mt] = 0xFFFFFFFFu;
  }
  auto load_b = [&](uint4 (&bb)[2 * NS], int tile) {
    const uint32_t vo = tile < ntiles ? voff : 0x80000000u;
    const int so = tile * Kp * 128;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      bb[2 * s] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, (int)vo, so + s * 1024, AKH_LM_CPOL));
      bb[2 * s + 1] = __builtin_bit_cast(
          uint4,
          __builtin_amdgcn_raw_buffer_load_b128(wres, (int)vo, so + s * 1024 + 16, AKH_LM_CPOL));
    }
  };
  uint4 cur[2 * NS], nxt[2 * NS];
  load_b(cur, blockIdx.x);
  int par = 0;
#pragma unroll 1
  for (int tile = blockIdx.x; tile < ntiles; tile += G) {
    load_b(nxt, tile + G);
    asm volatile("" ::: "memory");  // keep the prefetch issued here
    f32x16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x16 c = zero16(), cor = zero16();
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const f16x8 bh = f16x8_of(cur[2 * s]), bl = f16x8_of(cur[2 * s + 1]);
        const f16x8 xh = f16x8_of(ah[mt][s]), xl = f16x8_of(al[mt][s]);
        cor = mfma_f16(xl, bh, cor);
        cor = mfma_f16(xh, bl, cor);
        c = mfma_f16(xh, bh, c);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][r] = (c[r] + cor[r] * 0x1p-11f) * up;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      lm_finish<W>(acc[mt], red[par], tile, 32 * mt, p, bv[mt], bi[mt]);
      par ^= 1;
    }
#pragma unroll
    for (int q = 0; q < 2 * NS; ++q) cur[q] = nxt[q];
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv[mt], o, 64);
      const uint32_t oi = __shfl_xor(bi[mt], o, 64);
      amax_merge(bv[mt], bi[mt], ov, oi);
    }
    const int m = 32 * mt + wave * RW + lane / LPR;
    if (lane % LPR == 0 && m < p.M)
      p.amax[(size_t)m * G + blockIdx.x] = make_uint2(__float_as_uint(bv[mt]), bi[mt]);
  }
}

// Single-query attention over the KV cache, one (sequence, head, split) per
// block, with the fused head of the layer's attention:
//   q, k, v of the new token = the sum of the QKV GEMM's partial tiles, with
//   RoPE on q and k at position pos; k and v appended to the cache at row
//   pos (inference_graphs.rs:398-426);
//   softmax(scale * q . K[0..pos]) . V[0..pos] (attn_qk_cached + softmax_rect
//   + attn_av_cached, inference_graphs.rs:428-456), computed as SP partial
//   softmax states over SP ranges of the rows.
// Split sp takes cached rows [sp*per, (sp+1)*per) of 0..pos-1; the last
// split also folds in the new row and appends it to the cache.  AW waves
// divide the split's rows; each streams its rows with HD/4 lanes per row (a
// float4 each) and RB row groups of K and V in flight, keeping an online
// softmax.  The waves' (max, sum, o) are merged in LDS and the split writes
// its unnormalised o (k-quad layout, one tile per split) and (max, sum);
// the out_proj GEMM merges the splits when it loads its A operand.
//
// KV16: the cache holds bfloat16 rows (a lane loads 8 bytes per row and
// widens them); the new row is rounded to bfloat16 before it is used and
// appended, so every step sees the cache's values.
// A row's score: the sum of its LPR lanes' partial dot products.
#ifndef AKH_ATTN_DPP
#define AKH_ATTN_DPP 1
#endif
template <int LPR>
__device__ __forceinline__ float row_dot_sum(float s) {
  if constexpr (AKH_ATTN_DPP) {
    return group_sum<LPR>(s);
  } else {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    return s;
  }
}

// Sum and max over a wave's row slots: lanes LPR, 2 LPR, ... apart (each
// lane pairs with the lane of the same column in the other slot; slots
// under 16 lanes apart by bpermute).
template <int LPR>
__device__ __forceinline__ float slots_sum(float v) {
  if constexpr (AKH_ATTN_DPP) {
#pragma unroll
    for (int o = LPR; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
    if constexpr (LPR <= 16) v = xor_sum<16>(v);
    if constexpr (LPR <= 32) v = xor_sum<32>(v);
  } else {
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  }
  return v;
}
template <int LPR>
__device__ __forceinline__ float slots_max(float v) {
  if constexpr (AKH_ATTN_DPP) {
#pragma unroll
    for (int o = LPR; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if constexpr (LPR <= 16) v = xor_max<16>(v);
    if constexpr (LPR <= 32) v = xor_max<32>(v);
  } else {
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  }
  return v;
}

template <int HD, int AW, int RB, int SP, bool KV16>
__global__ __launch_bounds__(64 * AW) void k_dec_attn(DecAttnParams p) {
  constexpr int LPR = HD / 4;    // lanes per row
  constexpr int RPW = 64 / LPR;  // rows per wave per load
  __shared__ float wm_s[AW], wl_s[AW];
  __shared__ float4 wo_s[AW][LPR];

  const int sp = blockIdx.x % SP, bh = blockIdx.x / SP;
  const int b = bh / p.H, hh = bh - b * p.H;
  if (p.active && !p.active[b]) return;  // a finished sequence: cache untouched
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane % LPR, rl = lane / LPR;
  const int pos = p.pos[b];
  const int d = p.d;
  const bool last = sp == SP - 1;
  // The head size hd <= HD (a multiple of 4): lanes whose four columns lie
  // past it load zeros and store nothing.
  const int hd = d / p.H;
  const bool gin = 4 * g < hd;

  const size_t hoff = (size_t)b * p.seq_stride + hh * hd + (gin ? 4 * g : 0);
  using KT = typename std::conditional<KV16, uint16_t, float>::type;
  const KT* kbase = static_cast<const KT*>(p.kc) + hoff;
  const KT* vbase = static_cast<const KT*>(p.vc) + hoff;

  // This split's share of the cached rows 0..pos-1, divided over the waves.
  const int per = (pos + SP - 1) / SP;
  const int t0 = min(pos, sp * per), t1 = min(pos, t0 + per);
  const int ch = ((t1 - t0 + AW - 1) / AW + RPW - 1) / RPW * RPW;
  const int r0 = t0 + wave * ch, r1 = min(t1, r0 + ch);

  // The first row batch is requested before the new token's q, k, v, so the
  // two memory round trips overlap.
  // Rows are held as loaded (bfloat16 pairs stay packed until used).
  // The rows are read once per step: non-temporal loads keep them from
  // displacing the caches' other contents (measured ~10 % faster streaming).
  using Raw = typename std::conditional<KV16, uint2, float4>::type;
  Raw kv[RB], vv[RB];
  bool ok[RB];
  auto nt_load = [](const KT* p) -> Raw {
    if constexpr (KV16) {
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      const u2 t = __builtin_nontemporal_load(reinterpret_cast<const u2*>(p));
      return make_uint2(t.x, t.y);
    } else {
      typedef float f4 __attribute__((ext_vector_type(4)));
      const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
      return make_float4(t.x, t.y, t.z, t.w);
    }
  };
  auto load_batch = [&](int base) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int r = base + i * RPW + rl;
      ok[i] = r < r1;
      const size_t off = (size_t)(ok[i] ? r : r0) * d;
      kv[i] = ok[i] && gin ? nt_load(kbase + off) : Raw{};
      vv[i] = ok[i] && gin ? nt_load(vbase + off) : Raw{};
    }
  };
  auto wide = [](const Raw& x) -> float4 {
    if constexpr (KV16)
      return bf16x4(x.x, x.y);
    else
      return x;
  };
  load_batch(r0);
  asm volatile("" ::: "memory");

  // The new token's q, k, v (columns hh*hd + 4g .. +3 of each role).
  float4 q4 = make_float4(0.f, 0.f, 0.f, 0.f), kn = q4, vn = q4;
  if (gin) {
    const float* row = p.qkv + (size_t)b * 3 * d + (size_t)hh * hd + 4 * g;
    const size_t ps = (size_t)p.rows * 3 * d;
    q4 = sum_parts4<4>(q4, row, ps, p.nparts);
    if (last) {
      kn = sum_parts4<4>(kn, row + d, ps, p.nparts);
      vn = sum_parts4<4>(vn, row + 2 * d, ps, p.nparts);
    }
    // Pairs (4g, 4g+1) and (4g+2, 4g+3) of the head: rope entries 2g, 2g+1.
    const float2 c0 = p.rope[(size_t)pos * (hd / 2) + 2 * g];
    const float2 c1 = p.rope[(size_t)pos * (hd / 2) + 2 * g + 1];
    rope_pair(q4.x, q4.y, c0.x, c0.y);
    rope_pair(q4.z, q4.w, c1.x, c1.y);
    rope_pair(kn.x, kn.y, c0.x, c0.y);
    rope_pair(kn.z, kn.w, c1.x, c1.y);
  }
  if constexpr (KV16) {
    const uint2 ku = make_uint2(pack_bf16x2(kn.x, kn.y), pack_bf16x2(kn.z, kn.w));
    const uint2 vu = make_uint2(pack_bf16x2(vn.x, vn.y), pack_bf16x2(vn.z, vn.w));
    kn = bf16x4(ku.x, ku.y);
    vn = bf16x4(vu.x, vu.y);
    if (last && wave == 0 && rl == 0 && gin) {
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.kc) + hoff + (size_t)pos * d) = ku;
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.vc) + hoff + (size_t)pos * d) = vu;
    }
  } else if (last && wave == 0 && rl == 0 && gin) {
    *reinterpret_cast<float4*>(static_cast<float*>(p.kc) + hoff + (size_t)pos * d) = kn;
    *reinterpret_cast<float4*>(static_cast<float*>(p.vc) + hoff + (size_t)pos * d) = vn;
  }

  const float qs = attn_score_scale(p.scale);
  float m = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (last && wave == 0) {
    // The new row; every lane of a row group holds its full score, and only
    // row slot 0 adds it so the slot sum below counts it once.
    float s = q4.x * kn.x + q4.y * kn.y + q4.z * kn.z + q4.w * kn.w;
    s = row_dot_sum<LPR>(s);
    m = s * qs;
    l = rl == 0 ? 1.f : 0.f;
    acc = rl == 0 ? vn : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int base = r0; base < r1; base += RPW * RB) {
    if (base != r0) load_batch(base);
    float t[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const float4 kk = wide(kv[i]);
      float s = q4.x * kk.x + q4.y * kk.y + q4.z * kk.z + q4.w * kk.w;
      s = row_dot_sum<LPR>(s);
      t[i] = ok[i] ? s * qs : -INFINITY;
    }
    float bm = t[0];
#pragma unroll
    for (int i = 1; i < RB; ++i) bm = fmaxf(bm, t[i]);
    bm = slots_max<LPR>(bm);
    const float mn = fmaxf(m, bm);
    const float corr = m == -INFINITY ? 0.f : attn_exp(m - mn);
    float ps = 0.f;
    float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const float e = ok[i] ? attn_exp(t[i] - mn) : 0.f;
      const float4 vw = wide(vv[i]);
      ps += e;
      pv.x += e * vw.x;
      pv.y += e * vw.y;
      pv.z += e * vw.z;
      pv.w += e * vw.w;
    }
    l = l * corr + ps;
    acc.x = acc.x * corr + pv.x;
    acc.y = acc.y * corr + pv.y;
    acc.z = acc.z * corr + pv.z;
    acc.w = acc.w * corr + pv.w;
    m = mn;
  }
  // Sum the wave's row slots (they share the running max m).
  l = slots_sum<LPR>(l);
  acc = make_float4(slots_sum<LPR>(acc.x), slots_sum<LPR>(acc.y), slots_sum<LPR>(acc.z),
                    slots_sum<LPR>(acc.w));
  if (rl == 0) wo_s[wave][g] = acc;
  if (lane == 0) {
    wm_s[wave] = m;
    wl_s[wave] = l;
  }
  __syncthreads();
  if (threadIdx.x < LPR && 4 * (int)threadIdx.x < hd) {
    const int t = threadIdx.x;
    float M = -INFINITY;
    for (int w = 0; w < AW; ++w) M = fmaxf(M, wm_s[w]);
    float L = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = 0; w < AW; ++w) {
      const float wg = wm_s[w] == -INFINITY ? 0.f : attn_exp(wm_s[w] - M);
      L += wg * wl_s[w];
      o.x += wg * wo_s[w][t].x;
      o.y += wg * wo_s[w][t].y;
      o.z += wg * wo_s[w][t].z;
      o.w += wg * wo_s[w][t].w;
    }
    *reinterpret_cast<float4*>(p.out_t + (size_t)sp * p.rows * d + (size_t)(b >> 5) * 32 * d +
                               ((size_t)(hh * (hd / 4) + t) * 32 + (b & 31)) * 4) = o;
    if (t == 0) p.ml[((size_t)sp * p.H + hh) * p.rows + b] = make_float2(M, L);
  }
}

// One block per row m: the row's new residual value (an embedding lookup,
// a gathered row, or x + the sum of a GEMM's partial tiles) is stored in the
// k-quad residual stream, and its RMSNorm with `gain` (cpu.rs:205-222:
// x * (1 / sqrt(sum(x^2)/d + eps)) * w) as the next GEMM's input.
// Partial tiles summed per batch of loads (24: ffn_down's whole split count
// in one memory round trip; measured 0.5 % faster per decode step than 8).
#ifndef AKH_NORM_NB1
#define AKH_NORM_NB1 24
#endif
#ifndef AKH_NORM_WIDE
#define AKH_NORM_WIDE 1
#endif
template <int QPT, int NTH>
__global__ __launch_bounds__(NTH) void k_rows_norm(RowsNormParams p) {
  static_assert(NTH == 256 || NTH == 512, "256 or 512 threads per row");
  __shared__ float redw[NTH / 64];
  const int m = blockIdx.x, d = p.d, nq = d / 4;
  const size_t tile_off = (size_t)(m >> 5) * 32 * d;  // row m's 32-row k-quad tile
  // The gain does not depend on the row: request it first, so its memory
  // round trip overlaps the row's.
  float4 g[QPT];
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int q = threadIdx.x + NTH * i;
    g[i] = q < nq ? *reinterpret_cast<const float4*>(p.gain + 4 * q)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float* row = nullptr;
  if (p.ids) {
    const uint32_t id = p.ids[m];
    row = id < p.vocab ? p.table + (size_t)id * d : nullptr;
  } else if (p.src) {
    row = p.src + (size_t)(p.src_rows ? (long)p.src_rows[m] : p.row0 + (long)m * p.row_stride) * d;
  }
  const bool gather = p.ids || p.src;
  float4 x[QPT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int q = threadIdx.x + NTH * i;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < nq) {
      float* xq = p.xt + tile_off + ((size_t)q * 32 + (m & 31)) * 4;
      if (p.ssq) {
        v = *reinterpret_cast<const float4*>(xq);
      } else {
        if (gather) {
          if (row) v = *reinterpret_cast<const float4*>(row + 4 * q);
        } else {
          v = sum_parts4_2<AKH_NORM_NB1, 8>(*reinterpret_cast<const float4*>(xq),
                                            p.parts + (size_t)m * d + 4 * q, (size_t)p.rows * d,
                                            p.nparts);
        }
        *reinterpret_cast<float4*>(xq) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
    }
    x[i] = v;
  }
  if (p.ssq) {
    // The residual's per-column-tile sums of squares, added as the decode
    // GEMMs' RMSNorm prologue adds them (four tiles, then in order).
    const float4* sq = reinterpret_cast<const float4*>(p.ssq + (size_t)m * (d >> 5));
    for (int c = 0; c < (d >> 7); ++c) {
      const float4 v = sq[c];
      ss += ((v.x + v.y) + v.z) + v.w;
    }
  } else {
    // The waves' sums, added in wave order.
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) redw[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = redw[0];
#pragma unroll
    for (int w = 1; w < NTH / 64; ++w) ss += redw[w];
  }
  const float rs = 1.0f / sqrtf(ss / (float)d + p.eps);
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int q = threadIdx.x + NTH * i;
    if (q < nq) {
      const float4 v = x[i];
      *reinterpret_cast<float4*>(p.xnt + tile_off + ((size_t)q * 32 + (m & 31)) * 4) = make_float4(
          __fmul_rn(__fmul_rn(v.x, rs), g[i].x), __fmul_rn(__fmul_rn(v.y, rs), g[i].y),
          __fmul_rn(__fmul_rn(v.z, rs), g[i].z), __fmul_rn(__fmul_rn(v.w, rs), g[i].w));
    }
  }
}

__global__ __launch_bounds__(256) void k_argmax_final(
    const uint2* part, int ntiles, uint32_t* tok, int* pos, uint32_t* hist,
    int hist_stride, int next_pos, const int* at, const float* logits, long lstride) {
  const int m = blockIdx.x;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (int t = threadIdx.x; t < ntiles; t += 256) {
    const uint2 v = part[(size_t)m * ntiles + t];
    amax_merge(bv, bi, __uint_as_float(v.x), v.y);
  }
  block_amax256(bv, bi);
  if (threadIdx.x == 0) {
    // The reference's scan (sampling.rs:83-91) starts from index 0; a NaN
    // logit there never loses a comparison, so it stays the answer.
    const bool nan0 = logits && __builtin_isnan(logits[(size_t)m * lstride]);
    const uint32_t id = bi == 0xFFFFFFFFu || nan0 ? 0u : bi;
    uint32_t* hrow = hist ? hist + (size_t)m * hist_stride : nullptr;
    if (pos) {
      const int p0 = pos[m];
      if (hrow) {
        hrow[p0] = tok[m];
        hrow[p0 + 1] = id;
      }
      pos[m] = p0 + 1;
    } else if (hrow) {
      hrow[at ? at[m] : next_pos] = id;
    }
    tok[m] = id;
  }
}

// ---------------------------------------------------------------------------

namespace {

// Launch shapes per role (W waves, HL rows per half-wave), chosen by timing
// whole decode steps on MI355X, one set for matrices under AKH_LARGE_GEMM
// elements (hall-1.0's) and one for larger (the scaled configuration's);
// each can be overridden at build time, e.g. -DAKH_SHAPE_QKV=4,24 or
// -DAKH_SHAPE_L_OUT=4,16.  The four layer GEMMs split K into chunks of
// whole passes: one pass per block while the grid stays within the role's
// block cap (AKH_GEMM_BLOCKS_*), more passes per block (fewer partial tiles
// for the consumer to sum) beyond; the generic lm_head (K beyond the
// persistent kernel's reach) runs whole-K blocks.  The caps bind only for
// the scaled configuration's matrices (config 5, one 64-row session: qkv
// 1024, out 1024, up 256 -- one K split, so ffn_up applies SiLU itself and
// the separate SiLU kernel goes -- and down 512 measured best per role,
// 6.52 -> 6.13 ms per bf16-KV step); hall-1.0's grids stay below every cap.
// hall-1.0's shapes, re-swept with the pipelined passes and the attention
// and norm changes: qkv 16,8 (three K splits) and up 16,24 (one K split, so
// ffn_up applies SiLU and ffn_down reads plain rows) took the step from
// 0.593 to 0.588 ms; out 4,12 and down 16,12 stayed best.
#ifndef AKH_SHAPE_QKV
#define AKH_SHAPE_QKV 16, 8
#endif
#ifndef AKH_SHAPE_OUT
#define AKH_SHAPE_OUT 4, 12
#endif
#ifndef AKH_SHAPE_UP
#define AKH_SHAPE_UP 16, 24
#endif
#ifndef AKH_SHAPE_DOWN
#define AKH_SHAPE_DOWN 16, 12
#endif
#ifndef AKH_SHAPE_LM
#define AKH_SHAPE_LM 4, 16
#endif
#ifndef AKH_SHAPE_L_QKV
#define AKH_SHAPE_L_QKV 4, 24
#endif
#ifndef AKH_SHAPE_L_OUT
#define AKH_SHAPE_L_OUT 4, 16
#endif
#ifndef AKH_SHAPE_L_UP
#define AKH_SHAPE_L_UP 8, 32
#endif
#ifndef AKH_SHAPE_L_DOWN
#define AKH_SHAPE_L_DOWN 8, 8
#endif
#ifndef AKH_SHAPE_L_LM
#define AKH_SHAPE_L_LM 4, 16
#endif
#ifndef AKH_LARGE_GEMM
#define AKH_LARGE_GEMM (1l << 22)
#endif
#ifndef AKH_GEMM_BLOCKS_QKV
#define AKH_GEMM_BLOCKS_QKV 1024
#endif
#ifndef AKH_GEMM_BLOCKS_OUT
#define AKH_GEMM_BLOCKS_OUT 1024
#endif
#ifndef AKH_GEMM_BLOCKS_UP
#define AKH_GEMM_BLOCKS_UP 256
#endif
#ifndef AKH_GEMM_BLOCKS_DOWN
#define AKH_GEMM_BLOCKS_DOWN 512
#endif

template <int ROLE, bool LARGE>
struct RoleShape;
#define AKH_ROLE_SHAPE(R, L, w, hl) \
  template <> struct RoleShape<R, L> { static constexpr int W = w, HL = hl; };
#define AKH_ROLE_SHAPE_(...) AKH_ROLE_SHAPE(__VA_ARGS__)
AKH_ROLE_SHAPE_(DEC_CFG_QKV, false, AKH_SHAPE_QKV)
AKH_ROLE_SHAPE_(DEC_CFG_OUT, false, AKH_SHAPE_OUT)
AKH_ROLE_SHAPE_(DEC_CFG_UP, false, AKH_SHAPE_UP)
AKH_ROLE_SHAPE_(DEC_CFG_DOWN, false, AKH_SHAPE_DOWN)
AKH_ROLE_SHAPE_(DEC_CFG_LM, false, AKH_SHAPE_LM)
AKH_ROLE_SHAPE_(DEC_CFG_QKV, true, AKH_SHAPE_L_QKV)
AKH_ROLE_SHAPE_(DEC_CFG_OUT, true, AKH_SHAPE_L_OUT)
AKH_ROLE_SHAPE_(DEC_CFG_UP, true, AKH_SHAPE_L_UP)
AKH_ROLE_SHAPE_(DEC_CFG_DOWN, true, AKH_SHAPE_L_DOWN)
AKH_ROLE_SHAPE_(DEC_CFG_LM, true, AKH_SHAPE_L_LM)

bool large_gemm(int K, int N) { return (long)K * N >= AKH_LARGE_GEMM; }

// K passes (of KC rows) per block; every one of the role_splits blocks of
// a column tile gets at least one pass.
template <int ROLE, bool LARGE>
int role_kpass(int K, int N) {
  constexpr int KC = 2 * RoleShape<ROLE, LARGE>::W * RoleShape<ROLE, LARGE>::HL;
  const int passes = (K + KC - 1) / KC;
  if (ROLE == DEC_CFG_LM) return passes;
  constexpr int cap = ROLE == DEC_CFG_QKV  ? AKH_GEMM_BLOCKS_QKV
                      : ROLE == DEC_CFG_OUT ? AKH_GEMM_BLOCKS_OUT
                      : ROLE == DEC_CFG_UP  ? AKH_GEMM_BLOCKS_UP
                                            : AKH_GEMM_BLOCKS_DOWN;
  const int want = std::max(1, std::min(passes, cap / ((N + 31) / 32)));
  return (passes + want - 1) / want;
}

template <int ROLE, bool LARGE>
int role_splits(int K, int N) {
  constexpr int KC = 2 * RoleShape<ROLE, LARGE>::W * RoleShape<ROLE, LARGE>::HL;
  const int passes = (K + KC - 1) / KC, kp = role_kpass<ROLE, LARGE>(K, N);
  return (passes + kp - 1) / kp;
}

template <int ROLE>
int role_splits(int K, int N) {
  return large_gemm(K, N) ? role_splits<ROLE, true>(K, N) : role_splits<ROLE, false>(K, N);
}

template <int ROLE>
bool role_bf16(int K, int N) {
  // A k-octet shape exists (dec_go_shape): HL a multiple of 8, or an even W.
  using S = RoleShape<ROLE, false>;
  using SL = RoleShape<ROLE, true>;
  return large_gemm(K, N) ? SL::HL % 8 == 0 || SL::W % 2 == 0
                          : S::HL % 8 == 0 || S::W % 2 == 0;
}

#ifndef AKH_DEC_NT2
#define AKH_DEC_NT2 2
#endif
#ifndef AKH_DEC_VALU
#define AKH_DEC_VALU 1
#endif
template <int ROLE, bool LARGE, int EPI, int PRO>
hipError_t dec_go_shape(DecGemmParams p, hipStream_t s) {
  using S = RoleShape<ROLE, LARGE>;
  // bfloat16 tiles need whole k-octets per half-wave: a shape whose HL is
  // not a multiple of 8 runs them as W / 2 waves of 2 HL rows, the same pass
  // length KC and so the same partial tiles.
  constexpr bool kOct = S::HL % 8 == 0;
  static_assert(kOct || S::W % 2 == 0, "no k-octet shape with the same pass length");
  constexpr int WB = kOct ? S::W : S::W / 2, HLB = kOct ? S::HL : 2 * S::HL;
  p.kpass = role_kpass<ROLE, LARGE>(p.K, p.N);
  const int ntiles = (p.N + 31) / 32, splits = role_splits<ROLE, LARGE>(p.K, p.N);
  const dim3 g(ntiles, splits);
#define AKH_DEC_GO(MT)                                                                        \
  if (p.wbf16)                                                                                \
    hipLaunchKernelGGL((k_dec_gemm<WB, HLB, EPI, PRO, true, MT>), g, dim3(64 * WB), 0, s, p); \
  else                                                                                        \
    hipLaunchKernelGGL((k_dec_gemm<S::W, S::HL, EPI, PRO, false, MT>), g, dim3(64 * S::W), 0, \
                       s, p);
  if (p.mt == 1) {
    // A single sequence of float tiles on the VALU.  Measured on MI355X at
    // hall-1.0: one live row, qkv 4.08 -> 3.71 us, ffn_up 6.75 -> 5.11 us,
    // ffn_down 4.86 -> 4.00 us, config 1 0.406 -> 0.376 ms per token; four
    // live rows lost (out_proj 4.1 -> 7.0 us, ffn_up 6.8 -> 9.4 us: every
    // lane loads, and for out_proj merges, each row's A), so those keep the
    // MFMAs.
    constexpr bool kValu = AKH_DEC_VALU && EPI != DEC_RESID && EPI != DEC_LOGITS &&
                           PRO != PRO_NORM;
    if constexpr (kValu) {
      if (!p.wbf16 && p.M == 1) {
        hipLaunchKernelGGL((k_dec_gemm<S::W, S::HL, EPI, PRO, false, 1, 1, 1>), g,
                           dim3(64 * S::W), 0, s, p);
        return hipGetLastError();
      }
    }
    AKH_DEC_GO(1)
  } else if (p.mt == 2) {
    // Two row tiles of bfloat16 weights: each block of the K-split roles
    // (qkv, out, down) takes two column tiles, so every A operand it loads
    // (4x the bytes of a tile's weights per pass) and every split of it
    // feeds twice the MFMAs.  Config 5, A/B on one box: out 13.7 -> 11.0 us,
    // down 15.1 -> 14.0 us, qkv 13.7 -> 13.4 us.  ffn_up (one K split, 128
    // blocks left) went 15.9 -> 19.9 us and the lm_head 82 -> 111 us, so
    // they keep one column tile.
    constexpr bool kNT2 =
        ROLE == DEC_CFG_QKV || ROLE == DEC_CFG_OUT || ROLE == DEC_CFG_DOWN;
    if constexpr (AKH_DEC_NT2 == 2 && kNT2 && EPI != DEC_RESID && PRO != PRO_NORM) {
      if (p.wbf16) {
        hipLaunchKernelGGL((k_dec_gemm<WB, HLB, EPI, PRO, true, 2, 2>),
                           dim3((ntiles + 1) / 2, splits), dim3(64 * WB), 0, s, p);
        return hipGetLastError();
      }
    }
    AKH_DEC_GO(2)
  } else {
    return hipErrorInvalidValue;
  }
#undef AKH_DEC_GO
  return hipGetLastError();
}

template <int ROLE, int EPI, int PRO>
hipError_t dec_go(const DecGemmParams& p, hipStream_t s) {
  return large_gemm(p.K, p.N) ? dec_go_shape<ROLE, true, EPI, PRO>(p, s)
                              : dec_go_shape<ROLE, false, EPI, PRO>(p, s);
}

// The persistent lm_head covers K <= 2 * 8 * 64 (A held in registers; for
// two row tiles K <= 768) and packed weights under 2 GiB (32-bit buffer
// offsets); its tiles are padded to exactly 2 * 8 * HL rows.
int lm_rows(int K) { return K <= 256 ? 256 : K <= 768 ? 768 : 1024; }
bool lm_persistent(int N, int K, int mt) {
  return K <= (mt == 1 ? 1024 : 768) &&
         (long)((N + 31) / 32) * lm_rows(K) * 128 < (1l << 31);
}

}  // namespace

hipError_t launch_pack_tiles(const float* w, int K, int N, int Kp, float* out, bool bf16,
                             hipStream_t s) {
  if (K <= 0 || N <= 0 || Kp < K || Kp % (bf16 ? 8 : 4) != 0) return hipErrorInvalidValue;
  if (bf16)
    hipLaunchKernelGGL(k_pack_tiles_bf16, dim3((Kp / 8 + 7) / 8, (N + 31) / 32), dim3(256), 0,
                       s, w, K, N, Kp, reinterpret_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(k_pack_tiles, dim3((Kp / 4 + 7) / 8, (N + 31) / 32), dim3(256), 0, s,
                       w, K, N, Kp, out);
  return hipGetLastError();
}

hipError_t launch_pack_lm_h3(const float* w, int K, int N, int Kp, uint16_t* out, int* flag,
                             hipStream_t s) {
  if (K <= 0 || N <= 0 || Kp < K || Kp % 8 != 0 || !flag) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pack_lm_h3, dim3((Kp / 8 + 7) / 8, (N + 31) / 32), dim3(256), 0, s, w, K,
                     N, Kp, out, flag);
  return hipGetLastError();
}

// Sessions of one and two row tiles both run the persistent kernel (K <= 768).
bool dec_lm_h3_capable(int K, int N) { return lm_persistent(N, K, 2); }

hipError_t launch_check_bf16(const float* w, size_t n, int* flag, hipStream_t s) {
  const size_t blocks = std::min<size_t>(2048, (n + 255) / 256);
  hipLaunchKernelGGL(k_check_bf16, dim3((unsigned)std::max<size_t>(1, blocks)), dim3(256), 0,
                     s, reinterpret_cast<const uint32_t*>(w), n, flag);
  return hipGetLastError();
}

int dec_packed_rows(int role, int K) {
  if (role == DEC_CFG_LM && K <= 1024) return lm_rows(K);
  return (K + 7) / 8 * 8;  // whole k-octets, for either element type
}

bool dec_bf16_capable(int role, int K, int N) {
  switch (role) {
    case DEC_CFG_QKV: return role_bf16<DEC_CFG_QKV>(K, N);
    case DEC_CFG_OUT: return role_bf16<DEC_CFG_OUT>(K, N);
    case DEC_CFG_UP: return role_bf16<DEC_CFG_UP>(K, N);
    case DEC_CFG_DOWN: return role_bf16<DEC_CFG_DOWN>(K, N);
    // Tiles whose lm_head runs the persistent kernel at one row tile stay
    // float (that kernel reads float quads).
    default: return !lm_persistent(N, K, 1) && role_bf16<DEC_CFG_LM>(K, N);
  }
}

int dec_gemm_splits(int role, int K, int N) {
  switch (role) {
    case DEC_CFG_QKV: return role_splits<DEC_CFG_QKV>(K, N);
    case DEC_CFG_OUT: return role_splits<DEC_CFG_OUT>(K, N);
    case DEC_CFG_UP: return role_splits<DEC_CFG_UP>(K, N);
    case DEC_CFG_DOWN: return role_splits<DEC_CFG_DOWN>(K, N);
    default: return 1;
  }
}

#ifndef AKH_LM_BLOCKS_PER_CU
#define AKH_LM_BLOCKS_PER_CU 2  // float tiles: 2 beat 1 and 3 (config 4: 34.7 us vs 39.6)
#endif
#ifndef AKH_LM_H3_BLOCKS_PER_CU
#define AKH_LM_H3_BLOCKS_PER_CU 1  // split tiles (one block fits per CU): 27.4 us vs 30.0 for 2
#endif
int dec_lm_parts(int N, int K, int num_cus, int mt, bool h3) {
  // Two row tiles hold twice the A registers: one block per CU fits.
  const int per_cu = mt == 1 ? (h3 ? AKH_LM_H3_BLOCKS_PER_CU : AKH_LM_BLOCKS_PER_CU) : 1;
  if (lm_persistent(N, K, mt)) return std::max(1, std::min((N + 31) / 32, per_cu * num_cus));
  return (N + 31) / 32;
}

hipError_t launch_dec_lm(const DecGemmParams& p, int num_cus, hipStream_t s) {
  if (p.mt != 1 && p.mt != 2) return hipErrorInvalidValue;
  if (!lm_persistent(p.N, p.K, p.mt)) {
    if (p.wh3) return hipErrorInvalidValue;  // split tiles serve the persistent kernel only
    return dec_go<DEC_CFG_LM, DEC_LOGITS, PRO_NONE>(p, s);
  }
  if (p.Kp != lm_rows(p.K)) return hipErrorInvalidValue;
  const dim3 g(dec_lm_parts(p.N, p.K, num_cus, p.mt, p.wh3 != 0));
  if (p.wh3) {
    if (p.Kp != 256 && p.Kp != 768) return hipErrorInvalidValue;
#define AKH_LM_H3_GO(MT)                                                    \
  if (p.Kp == 256)                                                          \
    hipLaunchKernelGGL((k_dec_lm_h3<8, 16, MT>), g, dim3(512), 0, s, p);    \
  else                                                                      \
    hipLaunchKernelGGL((k_dec_lm_h3<8, 48, MT>), g, dim3(512), 0, s, p);
    if (p.mt == 1) {
      AKH_LM_H3_GO(1)
    } else {
      AKH_LM_H3_GO(2)
    }
#undef AKH_LM_H3_GO
    return hipGetLastError();
  }
#define AKH_LM_GO(MT)                                           \
  if (p.Kp == 256)                                              \
    hipLaunchKernelGGL((k_dec_lm<8, 16, MT>), g, dim3(512), 0, s, p); \
  else if (p.Kp == 768)                                         \
    hipLaunchKernelGGL((k_dec_lm<8, 48, MT>), g, dim3(512), 0, s, p); \
  else if (MT == 1)                                             \
    hipLaunchKernelGGL((k_dec_lm<8, 64, 1>), g, dim3(512), 0, s, p);
  if (p.mt == 1) {
    AKH_LM_GO(1)
  } else {
    AKH_LM_GO(2)
  }
#undef AKH_LM_GO
  return hipGetLastError();
}

bool dec_norm_fusable(int K) { return K % 128 == 0 && K <= 4096; }

// The shapes the batched decode kernels take: lanes read head rows four
// columns at a time (k_dec_attn), activations are whole 32-column k-quad
// tiles of at most 4096 columns (k_rows_norm, k_dec_gemm).
bool dec_fast_shape(int d, int hd, int F) {
  return hd >= 4 && hd <= 128 && hd % 4 == 0 && d % 32 == 0 && d <= 4096 && F % 32 == 0;
}

hipError_t launch_dec_gemm(const DecGemmParams& p, int role, hipStream_t s) {
  // PRO_NORM reads [rows][K / 32] sums of squares four tiles at a time;
  // DEC_RESID writes them for N / 32 column tiles.
  if (p.ssq && !dec_norm_fusable(p.K)) return hipErrorInvalidValue;
  if (p.res && (!p.ssq_out || !p.count || !dec_norm_fusable(p.N))) return hipErrorInvalidValue;
  switch (role) {
    case DEC_CFG_QKV:
      return p.ssq ? dec_go<DEC_CFG_QKV, DEC_PART, PRO_NORM>(p, s)
                   : dec_go<DEC_CFG_QKV, DEC_PART, PRO_NONE>(p, s);
    case DEC_CFG_OUT:
      return p.res ? dec_go<DEC_CFG_OUT, DEC_RESID, PRO_ATTN_MERGE>(p, s)
                   : dec_go<DEC_CFG_OUT, DEC_PART, PRO_ATTN_MERGE>(p, s);
    case DEC_CFG_UP:
      // One split: the whole sum is in the block, so SiLU is applied here.
      if (dec_gemm_splits(DEC_CFG_UP, p.K, p.N) == 1)
        return p.ssq ? dec_go<DEC_CFG_UP, DEC_SILU_T, PRO_NORM>(p, s)
                     : dec_go<DEC_CFG_UP, DEC_SILU_T, PRO_NONE>(p, s);
      return p.ssq ? dec_go<DEC_CFG_UP, DEC_PART_T, PRO_NORM>(p, s)
                   : dec_go<DEC_CFG_UP, DEC_PART_T, PRO_NONE>(p, s);
    case DEC_CFG_DOWN:
      if (p.res)
        return p.nparts ? dec_go<DEC_CFG_DOWN, DEC_RESID, PRO_SILU_SUM>(p, s)
                        : dec_go<DEC_CFG_DOWN, DEC_RESID, PRO_NONE>(p, s);
      return p.nparts ? dec_go<DEC_CFG_DOWN, DEC_PART, PRO_SILU_SUM>(p, s)
                      : dec_go<DEC_CFG_DOWN, DEC_PART, PRO_NONE>(p, s);
  }
  return hipErrorInvalidValue;
}

// Attention launch shapes: AW waves, RB row groups in flight, SP splits.
// The default serves short contexts and small grids (hall-1.0 at batch 32:
// 384 (sequence, head) pairs over 449..512 rows).  Long contexts with at
// least 512 pairs take 8 waves per block: with the f32 cache in 2 splits,
// with the bfloat16 cache in 1 split of 4 row groups (config 5, 64 x 16
// pairs at 2048 rows: 10.11 -> 9.58 and 6.15 -> 6.06 ms per step).
#ifndef AKH_SHAPE_ATTN
#define AKH_SHAPE_ATTN 4, 8, 2
#endif
#ifndef AKH_SHAPE_ATTN_LONG
#define AKH_SHAPE_ATTN_LONG 8, 8, 2
#endif
#ifndef AKH_SHAPE_ATTN_LONG16
#define AKH_SHAPE_ATTN_LONG16 8, 4, 1
#endif
namespace {
template <int AW_, int RB_, int SP_>
struct AttnShape {
  static constexpr int AW = AW_, RB = RB_, SP = SP_;
};
using AttnCfg = AttnShape<AKH_SHAPE_ATTN>;
using AttnLong = AttnShape<AKH_SHAPE_ATTN_LONG>;
using AttnLong16 = AttnShape<AKH_SHAPE_ATTN_LONG16>;
static_assert(AttnCfg::SP <= kMaxAttnSplits && AttnLong::SP <= kMaxAttnSplits &&
                  AttnLong16::SP <= kMaxAttnSplits,
              "too many attention splits");
bool attn_long(int batch, int heads, long max_ctx) {
  return max_ctx >= 1024 && (long)batch * heads >= 512;
}
}  // namespace

int dec_attn_splits(int batch, int heads, long max_ctx, bool kv16) {
  if (!attn_long(batch, heads, max_ctx)) return AttnCfg::SP;
  return kv16 ? AttnLong16::SP : AttnLong::SP;
}
int dec_attn_max_splits() {
  return std::max(AttnCfg::SP, std::max(AttnLong::SP, AttnLong16::SP));
}

namespace {
template <class SH>
hipError_t launch_dec_attn_shape(const DecAttnParams& p, int batch, int hd,
                                 hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  constexpr int AW = SH::AW, RB = SH::RB, SP = SH::SP;
  // Row groups in flight for a bfloat16 cache (config 5: 8 beat 16, 24, 32).
#ifndef AKH_ATTN_KV16_RB
#define AKH_ATTN_KV16_RB RB
#endif
  constexpr int RB16 = AKH_ATTN_KV16_RB;
  dim3 g(batch * p.H * SP), b(64 * AW);
  // With events, the dispatch itself carries their timestamps
  // (hipExtLaunchKernelGGL): t0 to t1 spans the kernel alone.
#define AKH_ATTN_GO(K)                                                             \
  if (t0)                                                                          \
    hipExtLaunchKernelGGL(K, g, b, 0, s, t0, t1, 0, p);                             \
  else                                                                             \
    hipLaunchKernelGGL(K, g, b, 0, s, p);
#define AKH_ATTN(HD)                                                               \
  if (p.kv16) {                                                                    \
    AKH_ATTN_GO((k_dec_attn<HD, AW, RB16, SP, true>))                              \
  } else {                                                                         \
    AKH_ATTN_GO((k_dec_attn<HD, AW, RB, SP, false>))                               \
  }
  // The kernel of the next power of two; its lanes past hd stay idle.
  if (hd < 4 || hd > 128 || hd % 4 != 0 || p.d != hd * p.H) return hipErrorInvalidValue;
  if (hd <= 4) {
    AKH_ATTN(4)
  } else if (hd <= 8) {
    AKH_ATTN(8)
  } else if (hd <= 16) {
    AKH_ATTN(16)
  } else if (hd <= 32) {
    AKH_ATTN(32)
  } else if (hd <= 64) {
    AKH_ATTN(64)
  } else {
    AKH_ATTN(128)
  }
#undef AKH_ATTN
#undef AKH_ATTN_GO
  return hipGetLastError();
}
}  // namespace

hipError_t launch_dec_attn(const DecAttnParams& p, int batch, int hd,
                           hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  if (p.d <= 0 || p.H <= 0) return hipErrorInvalidValue;
  if (!attn_long(batch, p.H, p.seq_stride / p.d))
    return launch_dec_attn_shape<AttnCfg>(p, batch, hd, s, t0, t1);
  return p.kv16 ? launch_dec_attn_shape<AttnLong16>(p, batch, hd, s, t0, t1)
                : launch_dec_attn_shape<AttnLong>(p, batch, hd, s, t0, t1);
}

// act = silu(sum of the partial tiles), four elements per thread.
__global__ void k_silu_sum(const float* __restrict__ parts, int nparts, float* __restrict__ act,
                           size_t n4) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (size_t)gridDim.x * blockDim.x) {
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    t = sum_parts4<4>(t, parts + 4 * i, 4 * n4, nparts);
    reinterpret_cast<float4*>(act)[i] = make_float4(silu(t.x), silu(t.y), silu(t.z), silu(t.w));
  }
}

hipError_t launch_silu_sum(const float* parts, int nparts, float* act, size_t n,
                           hipStream_t s) {
  if (n % 4 != 0 || nparts < 1) return hipErrorInvalidValue;
  const size_t n4 = n / 4;
  const size_t blocks = std::min<size_t>((n4 + 255) / 256, 65535u * 16u);
  hipLaunchKernelGGL(k_silu_sum, dim3((unsigned)std::max<size_t>(1, blocks)), dim3(256), 0, s,
                     parts, nparts, act, n4);
  return hipGetLastError();
}

// Prefill's fp32 K/V rows into a bfloat16 cache, four elements per thread.
__global__ void k_kv_store_bf16(const float* __restrict__ k, const float* __restrict__ v,
                                uint16_t* kc, uint16_t* vc, int S, int d, long seq_stride,
                                const int2* __restrict__ rowmap, size_t n4) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t row = i / (d / 4), c = (i % (d / 4)) * 4;
    size_t b, t;
    if (rowmap) {
      const int2 st = rowmap[row];
      b = (size_t)st.x;
      t = (size_t)st.y;
    } else {
      b = row / S;
      t = row % S;
    }
    const size_t dst = b * seq_stride + t * d + c;
    const float4 a = *reinterpret_cast<const float4*>(k + row * d + c);
    const float4 e = *reinterpret_cast<const float4*>(v + row * d + c);
    *reinterpret_cast<uint2*>(kc + dst) = make_uint2(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w));
    *reinterpret_cast<uint2*>(vc + dst) = make_uint2(pack_bf16x2(e.x, e.y), pack_bf16x2(e.z, e.w));
  }
}

// The same store element by element, for a dim that is not a multiple of 4.
__global__ void k_kv_store_bf16_1(const float* __restrict__ k, const float* __restrict__ v,
                                  uint16_t* kc, uint16_t* vc, int S, int d, long seq_stride,
                                  const int2* __restrict__ rowmap, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t row = i / d, c = i % d;
    size_t b, t;
    if (rowmap) {
      const int2 st = rowmap[row];
      b = (size_t)st.x;
      t = (size_t)st.y;
    } else {
      b = row / S;
      t = row % S;
    }
    const size_t dst = b * seq_stride + t * d + c;
    kc[dst] = (uint16_t)bf16_bits(k[row * d + c]);
    vc[dst] = (uint16_t)bf16_bits(v[row * d + c]);
  }
}

hipError_t launch_kv_store_bf16(const float* k, const float* v, uint16_t* kc, uint16_t* vc,
                                size_t rows, int S, int d, long seq_stride,
                                const int2* rowmap, hipStream_t s) {
  if (d <= 0 || (!rowmap && S <= 0)) return hipErrorInvalidValue;
  if (d % 4 != 0) {
    const size_t n = rows * d;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 65535u * 16u);
    hipLaunchKernelGGL(k_kv_store_bf16_1, dim3((unsigned)std::max<size_t>(1, blocks)), dim3(256),
                       0, s, k, v, kc, vc, S, d, seq_stride, rowmap, n);
    return hipGetLastError();
  }
  const size_t n4 = rows * (d / 4);
  const size_t blocks = std::min<size_t>((n4 + 255) / 256, 65535u * 16u);
  hipLaunchKernelGGL(k_kv_store_bf16, dim3((unsigned)std::max<size_t>(1, blocks)), dim3(256), 0,
                     s, k, v, kc, vc, S, d, seq_stride, rowmap, n4);
  return hipGetLastError();
}

// Synthetic KV rows for timing decode over a filled cache: rows [0, len) of
// every (layer, K/V, sequence) plane get N(0, 1) values from a counter-based
// hash of (seed, plane, row, column) (splitmix64 finaliser, then Box-Muller
// on two 24-bit uniforms).  Planes are max_ctx * d apart; kv16 stores
// bfloat16 rounded to nearest even.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_fill_kv_synthetic(void* kv, bool kv16, size_t planes,
                                                           int len, int d, long max_ctx,
                                                           uint64_t seed) {
  const size_t n = planes * (size_t)len * d;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t c = i % d, r = (i / d) % len, pl = i / ((size_t)d * len);
    const size_t dst = (pl * max_ctx + r) * d + c;
    const uint64_t h = mix64(seed * 0x9E3779B97F4A7C15ull + dst);
    const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    const float v = sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958648f * u2);
    if (kv16)
      static_cast<uint16_t*>(kv)[dst] = (uint16_t)bf16_bits(v);
    else
      static_cast<float*>(kv)[dst] = v;
  }
}

hipError_t launch_fill_kv_synthetic(void* kv, bool kv16, size_t planes, int len, int d,
                                    long max_ctx, uint64_t seed, hipStream_t s) {
  const size_t n = planes * (size_t)len * d;
  if (n == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(k_fill_kv_synthetic, dim3((unsigned)blocks), dim3(256), 0, s, kv, kv16,
                     planes, len, d, max_ctx, seed);
  return hipGetLastError();
}

hipError_t launch_rows_norm(const RowsNormParams& p, int M, hipStream_t s) {
  const int nq = p.d / 4;
  if (nq <= 256)
    hipLaunchKernelGGL((k_rows_norm<1, 256>), dim3(M), dim3(256), 0, s, p);
  else if (nq <= 512)
    hipLaunchKernelGGL((k_rows_norm<AKH_NORM_WIDE ? 1 : 2, AKH_NORM_WIDE ? 512 : 256>), dim3(M),
                       dim3(AKH_NORM_WIDE ? 512 : 256), 0, s, p);
  else if (nq <= 1024)
    hipLaunchKernelGGL((k_rows_norm<AKH_NORM_WIDE ? 2 : 4, AKH_NORM_WIDE ? 512 : 256>), dim3(M),
                       dim3(AKH_NORM_WIDE ? 512 : 256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_argmax_final(const uint2* part, int ntiles, int M,
                               uint32_t* tok, int* pos, uint32_t* hist,
                               int hist_stride, int next_pos, hipStream_t s, const int* at,
                               const float* logits, long lstride) {
  hipLaunchKernelGGL(k_argmax_final, dim3(M), dim3(256), 0, s, part, ntiles,
                     tok, pos, hist, hist_stride, next_pos, at, logits, lstride);
  return hipGetLastError();
}

}  // namespace akh
