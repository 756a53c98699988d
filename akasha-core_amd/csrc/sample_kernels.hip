// Device-side token choice: sample_token of src/nn/sampling.rs:3-81 for a
// batch of rows, one 1024-thread block per row (or per part of a row, below).
//
// The reference copies the logits, applies the repetition penalty to every
// distinct seen id, and then either takes the argmax (temperature <= 0) or
// sorts all ids by logit (descending), keeps the top_k, turns them into f64
// probabilities exp((l - max) / T) / sum, keeps the smallest prefix whose
// cumulative probability reaches top_p (renormalised), and walks the prefix
// with r = rand::random() until r < p.
//
// On the general path nothing is sorted.  Every cut the reference makes
// along the sorted order -- the k-th element, the top_p crossing, the
// element where the walk stops -- is found by a radix select over 32-bit
// order-preserving keys of the penalised logits: three histogram passes
// (11, 11 and 10 bits) narrow the key, counting elements (top_k) or summing
// their f64 weights (top_p, the walk), and the elements that share the
// final key are resolved in index order (the
// reference's unstable sort leaves that order unspecified; lower index first
// is this implementation's choice).  The per-element weights live in a
// scratch row; the repetition penalty is applied on the fly through a bitmap
// of the seen ids in LDS.
//
// With 0 < top_k <= 1024 (run_chat's 40) only the top_k elements matter:
// a cut on d = max - l admitting between top_k and 2048 elements is found
// by counting against 16 thresholds per pass (powers of four, then 16-way
// refinements), those elements are gathered to LDS and each takes its place
// in the order (logit descending, index ascending) by counting the entries
// above it; the first top_k then go through the reference's own sequence:
// f64 probabilities summed in order, the top_p prefix, the walk r -= p.
// With top_k <= 256 a row is split over several blocks (parts of the
// vocabulary), whose top_k the row's last block merges.  NaN or infinite
// maxima, fewer than top_k finite elements and ties too wide for the cut
// take the radix path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace akh {

namespace {

#ifndef AKH_SAMPLE_NT
#define AKH_SAMPLE_NT 1024
#endif
#ifndef AKH_SAMPLE_BLOCKS
#define AKH_SAMPLE_BLOCKS 256
#endif
constexpr int NT = AKH_SAMPLE_NT;  // threads per row (per part of a split row)
constexpr int NW = NT / 64;     // waves per block

// Radix digits of the order keys: 11, 11 and 10 bits (three passes).
constexpr int kBins = 2048;
struct SampleShared {
  // One radix pass's bins: counts or f64 weight sums (a select uses one).
  union {
    uint32_t hist_n[kBins];
    double hist_w[kBins];
  };
  // The last pass's bins (kBins / 2): members of nonzero weight, lowest index.
  uint32_t last_n[kBins / 2];
  uint32_t last_i[kBins / 2];
  double wave_d[NW];
  uint32_t wave_u[NW];
  float wave_f[NW];
  uint32_t bcast_u[4];
  double bcast_d[2];
};

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Penalised logit (sampling.rs:3-16): every distinct seen id once.
__device__ __forceinline__ float pen_logit(const float* row, int i, const uint32_t* bm,
                                           float penalty) {
  float l = row[i];
  if (bm && (bm[i >> 5] >> (i & 31) & 1u)) l = l > 0.0f ? __fdiv_rn(l, penalty) : __fmul_rn(l, penalty);
  return l;
}

__device__ __forceinline__ double block_sum_d(double v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_d[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int k = 0; k < NW; ++k) t += sh.wave_d[k];
  return t;
}

__device__ __forceinline__ uint32_t block_sum_u(uint32_t v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_u[w] = v;
  __syncthreads();
  uint32_t t = 0;
  for (int k = 0; k < NW; ++k) t += sh.wave_u[k];
  return t;
}

__device__ __forceinline__ uint32_t block_min_u(uint32_t v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_u[w] = v;
  __syncthreads();
  uint32_t t = 0xFFFFFFFFu;
  for (int k = 0; k < NW; ++k) t = min(t, sh.wave_u[k]);
  return t;
}

__device__ __forceinline__ float block_max_f(float v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_f[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int k = 0; k < NW; ++k) t = fmaxf(t, sh.wave_f[k]);
  return t;
}

// Exclusive prefix sum over the block in thread order (0 for thread 0).
template <typename T>
__device__ T block_scan_excl(T v, T* wave_tot) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const T u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  T ex = __shfl_up(v, 1, 64);
  if (lane == 0) ex = 0;
  __syncthreads();
  if (lane == 63) wave_tot[w] = v;
  __syncthreads();
  T off = 0;
  for (int k = 0; k < w; ++k) off += wave_tot[k];
  return ex + off;
}

// The element of the descending order at which a cumulative quantity
// crosses `target`: counts of elements (weights == nullptr, crossing when
// the count reaches target) or sums of weights[i] (crossing at >= target if
// inclusive, > target otherwise).  Returns the index, or n if the total
// never crosses.  `key_of(i)` gives element i's order key.
template <typename KeyFn>
__device__ __forceinline__ uint32_t select_desc(int n, KeyFn key_of, const double* weights,
                                                double target, bool inclusive,
                                                SampleShared& sh) {
  uint32_t prefix = 0, mask = 0;
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : pass == 1 ? 10 : 0;
    const int nb = pass < 2 ? kBins : kBins / 2;
    for (int b = threadIdx.x; b < kBins; b += NT) {
      if (weights) sh.hist_w[b] = 0.0;
      else sh.hist_n[b] = 0u;
      if (pass == 2 && b < kBins / 2) {
        sh.last_n[b] = 0u;
        sh.last_i[b] = 0xFFFFFFFFu;
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += NT) {
      const uint32_t k = key_of(i);
      if ((k & mask) == prefix) {
        const int bin = (k >> shift) & (nb - 1);
        const double w = weights ? weights[i] : 1.0;
        if (weights) {
          if (w != 0.0) atomicAdd(&sh.hist_w[bin], w);
        } else {
          atomicAdd(&sh.hist_n[bin], 1u);
        }
        if (pass == 2 && w != 0.0) {
          atomicAdd(&sh.last_n[bin], 1u);
          atomicMin(&sh.last_i[bin], (uint32_t)i);
        }
      }
    }
    __syncthreads();
    // The first bin in descending order whose cumulative total crosses
    // target: thread t holds bins nb - 1 - 2t and nb - 2 - 2t, one block scan
    // gives the total before them, and the lowest crossing thread wins.
    const int t = threadIdx.x, b1 = nb - 1 - 2 * t, b0 = b1 - 1;
    auto val = [&](int b) {
      return b < 0 ? 0.0 : weights ? sh.hist_w[b] : (double)sh.hist_n[b];
    };
    const double v1 = val(b1), v0 = val(b0);
    const double before = block_scan_excl<double>(v1 + v0, sh.wave_d);
    auto crosses = [&](double nxt) {
      return weights ? (inclusive ? nxt >= target : nxt > target) : nxt >= target;
    };
    const double n1 = before + v1;
    const int mine = b1 < 0 ? -1 : crosses(n1) ? b1 : (b0 >= 0 && crosses(n1 + v0)) ? b0 : -1;
    const uint32_t win = block_min_u(mine >= 0 ? (uint32_t)t : 0xFFFFFFFFu, sh);
    if (win == 0xFFFFFFFFu) return (uint32_t)n;
    if ((uint32_t)t == win) {
      sh.bcast_u[0] = (uint32_t)mine;
      sh.bcast_d[0] = target - (mine == b1 ? before : n1);
    }
    __syncthreads();
    const uint32_t sel = sh.bcast_u[0];
    prefix |= sel << shift;
    mask |= (uint32_t)(nb - 1) << shift;
    target = sh.bcast_d[0];
    // One member of nonzero weight with the final key (distinct logits):
    // the crossing is in its bin, so it is the answer.
    const bool only = pass == 2 && sh.last_n[sel] == 1u;
    const uint32_t at = only ? sh.last_i[sel] : 0u;
    __syncthreads();
    if (only) return at;
  }
  // Elements with the final key, in index order: each thread sums its
  // members over a contiguous run of the row, one block scan gives every run
  // the total before it, and each thread walks its run again from there
  // (two barriers, where 1024-element chunks of the row took three block
  // reductions each).
  const int run = (n + NT - 1) / NT;
  const int i0 = min(n, (int)threadIdx.x * run), i1 = min(n, i0 + run);
  double own = 0.0;
  for (int i = i0; i < i1; ++i)
    if (key_of(i) == prefix) own += weights ? weights[i] : 1.0;
  double incl = block_scan_excl<double>(own, sh.wave_d);
  uint32_t first = 0xFFFFFFFFu;
  for (int i = i0; i < i1; ++i) {
    if (key_of(i) != prefix) continue;
    const double v = weights ? weights[i] : 1.0;
    if (v == 0.0) continue;
    incl += v;
    if (weights ? (inclusive ? incl >= target : incl > target) : incl >= target) {
      first = (uint32_t)i;
      break;
    }
  }
  first = block_min_u(first, sh);
  return first == 0xFFFFFFFFu ? (uint32_t)n : first;
}

constexpr int KCAP = 1024;  // largest top_k of the candidate path
constexpr int CCAP = 2048;  // candidates gathered for the sort
constexpr int NTH = 16;     // thresholds counted per pass

struct TopKShared {
  unsigned long long comp[CCAP];  // key << 32 | ~index: descending = the order
  unsigned long long top[KCAP];   // the first entries of that order
  double prob[KCAP];
  double norm;
  int keep;
  uint32_t wcnt[NW][NTH];
  uint32_t cnt[NTH];
  uint32_t n_cand;
  uint32_t pick;
};

// The float whose order_key is k.
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// tk.top[0 .. min(nc, K)) = the first entries of tk.comp[0 .. nc) in
// descending order (nc <= CCAP, K <= KCAP).  The entries are distinct (each
// holds its element's index), so an entry's place is the number of entries
// above it: every thread counts for its own entries, reading the others as
// LDS broadcasts, with no barrier in between.
__device__ __forceinline__ int rank_top(int nc, int K, TopKShared& tk) {
  for (int e = threadIdx.x; e < nc; e += NT) {
    const unsigned long long x = tk.comp[e];
    int above = 0;
#pragma unroll 8
    for (int f = 0; f < nc; ++f) above += tk.comp[f] > x ? 1 : 0;
    if (above < K) tk.top[above] = x;
  }
  __syncthreads();
  return min(nc, K);
}

// sampling.rs:45-80 over tk.top[0 .. top_k) in the reference's order: f64
// probabilities, their sum folded in order (one thread), each divided by it,
// the top_p prefix by the in-order running sum, its sum folded in order and
// divided out, and the walk r -= p.  The divisions, independent per element,
// run in parallel; the folds and the walk, whose order fixes the bits, on one
// thread.
__device__ __forceinline__ uint32_t tail_topk(uint32_t top_k, float temperature, float top_p,
                                              double r, TopKShared& tk) {
  const int K = (int)top_k;
  const double mxd = (double)key_value((uint32_t)(tk.top[0] >> 32));
  for (int t = threadIdx.x; t < K; t += NT)
    tk.prob[t] = exp(((double)key_value((uint32_t)(tk.top[t] >> 32)) - mxd) / (double)temperature);
  __syncthreads();
  if (threadIdx.x == 0) {
    double sum = 0.0;
    for (int t = 0; t < K; ++t) sum += tk.prob[t];
    tk.norm = sum;
  }
  __syncthreads();
  const double sum = tk.norm;
  for (int t = threadIdx.x; t < K; t += NT) tk.prob[t] /= sum;
  __syncthreads();
  int len = K;
  if (top_p < 1.0f) {
    if (threadIdx.x == 0) {
      double cum = 0.0;
      int keep = K;
      for (int t = 0; t < K; ++t) {
        cum += tk.prob[t];
        if (cum >= (double)top_p) {
          keep = t + 1;
          break;
        }
      }
      double s2 = 0.0;
      for (int t = 0; t < keep; ++t) s2 += tk.prob[t];
      tk.keep = keep;
      tk.norm = s2;
    }
    __syncthreads();
    len = tk.keep;
    const double s2 = tk.norm;
    for (int t = threadIdx.x; t < len; t += NT) tk.prob[t] /= s2;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    auto idx_of = [&](int t) { return 0xFFFFFFFFu - (uint32_t)(tk.top[t] & 0xFFFFFFFFull); };
    uint32_t pk = idx_of(len - 1);
    double rr = r;
    for (int t = 0; t < len; ++t) {
      if (rr < tk.prob[t]) {
        pk = idx_of(t);
        break;
      }
      rr -= tk.prob[t];
    }
    tk.pick = pk;
  }
  __syncthreads();
  return tk.pick;
}

// Calls f(l, i, live) for every index of the row in chunks of U elements per
// thread, the chunk's loads issued before any is used; every thread makes
// the same number of calls (live = i < n), so f may use wave-wide votes.
constexpr int U = 8;
template <typename LFn, typename F>
__device__ __forceinline__ void for_row(int n, LFn l_of, F f) {
  for (int c0 = 0; c0 < n; c0 += NT * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = c0 + u * NT + (int)threadIdx.x;
      v[u] = i < n ? l_of(i) : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = c0 + u * NT + (int)threadIdx.x;
      f(v[u], i, i < n);
    }
  }
}

// Block sums of per-thread counts c[j] (plus base) -> tk.cnt.
__device__ void reduce_counts(const uint32_t (&c)[NTH], uint32_t base, TopKShared& tk) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < NTH; ++j) {
    uint32_t x = c[j];
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    if (lane == 0) tk.wcnt[w][j] = x;
  }
  __syncthreads();
  if (threadIdx.x < NTH) {
    uint32_t t = base;
    for (int k = 0; k < NW; ++k) t += tk.wcnt[k][threadIdx.x];
    tk.cnt[threadIdx.x] = t;
  }
  __syncthreads();
}

// The top_k elements of l_of(0 .. n) (0 < top_k <= KCAP) in order in
// tk.top (index idx0 + i), from at most CCAP candidates gathered to tk.comp:
// returns how many (top_k, or fewer with all_finite), or -1 where the radix path must decide instead
// (NaN, an infinite maximum, fewer than top_k finite elements near the
// maximum, ties too wide to cut).  With all_finite, fewer than top_k finite
// elements near the maximum gathers every finite element instead (a part
// of a row, which may hold fewer than top_k).  Every thread of the block
// calls it; the outcome is the same for all.  The first count bins d =
// max - l by its binary exponent (d < 2^(2j - 12) exactly when its
// exponent is below 2j - 12), four packed 8-bit counters per chunk;
// refinements compare only the elements inside the narrowed interval.
template <typename LFn>
__device__ __forceinline__ int topk_candidates(int n, LFn l_of, uint32_t idx0, uint32_t top_k,
                                              bool all_finite, SampleShared& sh, TopKShared& tk) {
  float mxv = -INFINITY;
  uint32_t nan = 0;
  for_row(n, l_of, [&](float l, int, bool) {
    if (l != l) nan = 1;
    else mxv = fmaxf(mxv, l);
  });
  const float mx = block_max_f(mxv, sh);
  if (block_sum_u(nan, sh) != 0) return -1;
  if (mx == -INFINITY && all_finite) return 0;  // a part with no finite element
  if (!isfinite(mx)) return -1;

  // Threshold t: 2^(2t - 12) in the first count, then (lo, hi] cut in NTH.
  bool linear = false;
  float lo = 0.0f, hi = 0.0f;
  auto thr = [&](int t) {
    return !linear ? ldexpf(1.0f, 2 * t - 12)
                   : (t == NTH - 1 ? hi : lo + (hi - lo) * (float)(t + 1) / NTH);
  };
  {
    uint32_t c[NTH];
#pragma unroll
    for (int j = 0; j < NTH; ++j) c[j] = 0u;
    uint32_t h[4] = {0u, 0u, 0u, 0u};  // this chunk's bins (at most U per field)
    int k = 0;
    for_row(n, l_of, [&](float l, int, bool) {
      const float d = mx - l;
      int j0 = 0;
      if (!(d < ldexpf(1.0f, -12))) j0 = ((int)((__float_as_uint(d) >> 23) & 255u) - 127 + 12) / 2 + 1;
      if (j0 < NTH) {
        const uint32_t inc = 1u << ((j0 & 3) * 8);
#pragma unroll
        for (int q = 0; q < 4; ++q) h[q] += (j0 >> 2) == q ? inc : 0u;
      }
      if (++k == U) {  // fold the chunk's bins into the cumulative counts
        uint32_t run = 0;
#pragma unroll
        for (int j = 0; j < NTH; ++j) {
          run += (h[j >> 2] >> ((j & 3) * 8)) & 255u;
          c[j] += run;
        }
        h[0] = h[1] = h[2] = h[3] = 0u;
        k = 0;
      }
    });
    reduce_counts(c, 0u, tk);
  }
  float cut = 0.0f;
  for (int round = 0; round < 4; ++round) {
    int j = 0;
    while (j < NTH && tk.cnt[j] < top_k) ++j;
    if (j == NTH) {  // fewer than top_k finite elements near the max
      if (!all_finite) return -1;
      cut = INFINITY;
      break;
    }
    if (tk.cnt[j] <= (uint32_t)(round == 0 ? CCAP / 4 : CCAP)) {
      cut = thr(j);
      break;
    }
    if (round == 3) return -1;  // ties too wide to cut
    const uint32_t base = j > 0 ? tk.cnt[j - 1] : 0u;
    const float nlo = j > 0 ? thr(j - 1) : lo, nhi = thr(j);
    lo = nlo;
    hi = nhi;
    linear = true;
    float tv[NTH];
#pragma unroll
    for (int t = 0; t < NTH; ++t) tv[t] = thr(t);
    uint32_t c[NTH];
#pragma unroll
    for (int t = 0; t < NTH; ++t) c[t] = 0u;
    for_row(n, l_of, [&](float l, int, bool) {
      const float d = mx - l;
      if (!(d < lo) && d < hi) {
#pragma unroll
        for (int t = 0; t < NTH; ++t) c[t] += d < tv[t] ? 1u : 0u;
      }
    });
    __syncthreads();  // every thread has read cnt
    reduce_counts(c, base, tk);
  }

  // Gather the elements under the cut.
  if (threadIdx.x == 0) tk.n_cand = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  for_row(n, l_of, [&](float l, int i, bool live) {
    const bool take = live && mx - l < cut;
    const unsigned long long mask = __ballot(take);
    if (mask) {
      const int lead = __ffsll((long long)mask) - 1;
      uint32_t base = 0;
      if (lane == lead) base = atomicAdd(&tk.n_cand, (uint32_t)__popcll(mask));
      base = __shfl(base, lead, 64);
      const uint32_t slot = base + __popcll(mask & ((1ull << lane) - 1ull));
      if (take && slot < (uint32_t)CCAP)
        tk.comp[slot] = ((unsigned long long)order_key(l) << 32) | (0xFFFFFFFFu - (idx0 + (uint32_t)i));
    }
  });
  __syncthreads();
  const int nc = (int)tk.n_cand;
  if (nc > CCAP || (!all_finite && nc < (int)top_k)) return -1;
  return rank_top(nc, (int)top_k, tk);
}

__global__ __launch_bounds__(NT) void k_sample_rows(SampleArgs a) {
  extern __shared__ uint32_t bitmap[];
  __shared__ SampleShared sh;
  __shared__ TopKShared tk;
  const int m = blockIdx.x, n = a.n;
  const float* row = a.logits + (size_t)m * a.row_stride;
  double* w = a.wbuf + (size_t)m * n;

  // This row's seen ids (positions [s_lo, s_hi) of ids, a row of id_len
  // entries) and draw, their loads issued together.
  const uint32_t* ids = nullptr;
  long id_len = 0;
  int s_lo = 0, s_hi = 0;
  double r = 0.0;
  if (a.tok) {
    const int dn = a.done[m], st = a.start[m], p = a.pos[m];
    const uint32_t c = a.count[m];
    if (dn) {
      if (threadIdx.x == 0) a.active[m] = 0;
      return;
    }
    ids = a.hist + (size_t)m * a.hist_stride;
    id_len = a.hist_stride;
    s_lo = st;
    s_hi = p > st ? p : st;
    if (a.uniform) r = a.uniform[(size_t)c * gridDim.x + m];
  } else {
    if (a.seen) {
      ids = a.seen + (size_t)m * a.seen_stride;
      id_len = a.seen_stride;
      s_hi = a.seen_len ? (int)min(a.seen_len[m], (uint32_t)a.seen_stride) : 0;
    }
    if (a.uniform) r = a.uniform[m];
  }

  // Bitmap of this row's seen ids (only if the penalty changes anything).
  // The ids are read from their whole row (its extent is known) while the
  // range is still being loaded.
  const uint32_t* bm = nullptr;
  if (a.penalty != 1.0f && ids) {
    const int words = (n + 31) / 32;
    for (long s0 = 0; s0 < id_len; s0 += 4 * NT) {
      uint32_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long q = s0 + u * NT + threadIdx.x;
        v[u] = q < id_len ? ids[q] : 0u;
      }
      if (s0 == 0) {
        for (int k = threadIdx.x; k < words; k += NT) bitmap[k] = 0;
        __syncthreads();
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long q = s0 + u * NT + threadIdx.x;
        if (q >= s_lo && q < s_hi && v[u] < (uint32_t)n) atomicOr(&bitmap[v[u] >> 5], 1u << (v[u] & 31));
      }
    }
    if (id_len <= 0) {
      for (int k = threadIdx.x; k < words; k += NT) bitmap[k] = 0;
    }
    __syncthreads();
    bm = bitmap;
  }
  auto key_of = [&](int i) { return order_key(pen_logit(row, i, bm, a.penalty)); };

  uint32_t pick;
  bool picked = false;
  const bool topk = a.temperature > 0.0f && a.top_k > 0 && a.top_k < n && a.top_k <= KCAP;
  auto l_at = [&](int i) { return pen_logit(row, i, bm, a.penalty); };
  const int S = gridDim.y;
  int nc = 0;
  if (topk) {
    // With S > 1 (the host splits only rows with topk, a.cnt, and
    // S * (top_k + 1) <= n) this block takes part blockIdx.y of the row.
    const int per = (n + S - 1) / S;
    const int lo = min(n, (int)blockIdx.y * per), hi = min(n, lo + per);
    if (lo < hi)
      nc = topk_candidates(hi - lo, [&](int i) { return l_at(lo + i); }, (uint32_t)lo,
                           (uint32_t)a.top_k, S > 1, sh, tk);
  }
  if (S > 1) {
    // Its top_k (at most) to the row's workspace, then the row's last part
    // to arrive merges them.
    const int part = blockIdx.y;
    const int L = nc;
    unsigned long long* cand = reinterpret_cast<unsigned long long*>(w);
    int* status = reinterpret_cast<int*>(cand + (size_t)S * a.top_k);
    for (int t = threadIdx.x; t < L; t += NT)
      __hip_atomic_store(cand + (size_t)part * a.top_k + t, tk.top[t], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x == 0)
      __hip_atomic_store(status + part, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int done = __hip_atomic_fetch_add(a.cnt + m, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.bcast_u[1] = done == S - 1;
      if (done == S - 1)  // zero for the next launch
        __hip_atomic_store(a.cnt + m, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!sh.bcast_u[1]) return;
    // Every part's status in one batch of loads (at most 16 parts).
    int Lp[16];
#pragma unroll
    for (int q = 0; q < 16; ++q)
      Lp[q] = q < S ? __hip_atomic_load(status + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    int total = 0;
    bool fail = false;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      fail = fail || Lp[q] < 0;
      total += Lp[q] > 0 ? Lp[q] : 0;
    }
    if (!fail && total >= a.top_k && total <= CCAP) {
      // Entry e of the merged list: part q (the one whose prefix covers e),
      // position e - prefix; a thread's entries (at most two) load at once.
      unsigned long long got[CCAP / NT];
#pragma unroll
      for (int u = 0; u < CCAP / NT; ++u) {
        const int e = threadIdx.x + u * NT;
        int q = -1, base = 0, run = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int len = Lp[k] > 0 ? Lp[k] : 0;
          if (q < 0 && e < run + len) {
            q = k;
            base = run;
          }
          run += len;
        }
        got[u] = q >= 0 ? __hip_atomic_load(cand + (size_t)q * a.top_k + (e - base),
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : 0ull;
      }
#pragma unroll
      for (int u = 0; u < CCAP / NT; ++u) {
        const int e = threadIdx.x + u * NT;
        if (e < total) tk.comp[e] = got[u];
      }
      __syncthreads();
      rank_top(total, a.top_k, tk);
      pick = tail_topk((uint32_t)a.top_k, a.temperature, a.top_p, r, tk);
      picked = true;
    }
    // Otherwise this block takes the whole row on the radix path below.
  } else if (topk && nc >= 0) {
    pick = tail_topk((uint32_t)a.top_k, a.temperature, a.top_p, r, tk);
    picked = true;
  }
  if (picked) {
  } else if (a.temperature <= 0.0f) {
    // sampling.rs:30-32, 83-91: first index of the maximum.
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for_row(n, l_at, [&](float l, int i, bool live) {
      if (live) amax_merge(bv, bi, l, (uint32_t)i);
    });
    const float mx = block_max_f(bv, sh);
    pick = block_min_u(bv == mx ? bi : 0xFFFFFFFFu, sh);
    // The reference's scan starts from index 0 and a NaN there never loses
    // a comparison: it stays the answer.
    if (pick == 0xFFFFFFFFu || __builtin_isnan(pen_logit(row, 0, bm, a.penalty))) pick = 0;
  } else {
    float mxv = -INFINITY;
    for (int i = threadIdx.x; i < n; i += NT) mxv = fmaxf(mxv, pen_logit(row, i, bm, a.penalty));
    const double mx = (double)block_max_f(mxv, sh);
    const double T = (double)a.temperature;

    // top_k (sampling.rs:41-43): the k-th element of the descending order.
    uint32_t kth = (uint32_t)n;
    if (a.top_k > 0 && a.top_k < n) kth = select_desc(n, key_of, nullptr, (double)a.top_k, true, sh);
    const uint32_t kkey = kth < (uint32_t)n ? key_of((int)kth) : 0u;
    // Members: key above the k-th element's, or equal and not after it.
    auto in_k = [&](int i) {
      if (kth >= (uint32_t)n) return true;
      const uint32_t k = key_of(i);
      return k > kkey || (k == kkey && (uint32_t)i <= kth);
    };

    // Probabilities (sampling.rs:45-53).
    double part = 0.0;
    for (int i = threadIdx.x; i < n; i += NT) {
      const double e = in_k(i) ? exp(((double)pen_logit(row, i, bm, a.penalty) - mx) / T) : 0.0;
      w[i] = e;
      part += e;
    }
    // The reference divides every weight by their sum (sampling.rs:50-52),
    // and by the kept sum after the top_p cut, before comparing cumulative
    // sums with top_p and r.  The weights stay unnormalised here and those
    // targets are scaled by the sums instead: the same comparisons up to
    // rounding, without a pass over the row for each division.
    const double sum = block_sum_d(part, sh);
    double total = sum;

    // top_p (sampling.rs:55-70): the smallest prefix reaching top_p, renormalised.
    uint32_t last = kth < (uint32_t)n ? kth : (uint32_t)n;  // last kept element, n = unknown
    if (a.top_p < 1.0f) {
      // No crossing keeps every element (and still renormalises).
      const uint32_t cut = select_desc(n, key_of, w, (double)a.top_p * sum, true, sh);
      const uint32_t ckey = cut < (uint32_t)n ? key_of((int)cut) : 0u;
      double kept = 0.0;
      for (int i = threadIdx.x; i < n; i += NT) {
        if (cut < (uint32_t)n) {
          const uint32_t k = key_of(i);
          if (k < ckey || (k == ckey && (uint32_t)i > cut)) w[i] = 0.0;
        }
        kept += w[i];
      }
      total = block_sum_d(kept, sh);
      if (cut < (uint32_t)n) last = cut;
    }

    // The walk (sampling.rs:72-80): first element whose cumulative
    // probability exceeds r; the last kept element if none does.
    pick = select_desc(n, key_of, w, r * total, false, sh);
    if (pick >= (uint32_t)n) {
      if (last >= (uint32_t)n) {
        // Every element is kept: the last of the descending order is the
        // minimum, the highest index among equal minima.
        float mn = INFINITY;
        for (int i = threadIdx.x; i < n; i += NT) mn = fminf(mn, pen_logit(row, i, bm, a.penalty));
        const float lo = -block_max_f(-mn, sh);
        uint32_t hi = 0;
        for (int i = threadIdx.x; i < n; i += NT)
          if (pen_logit(row, i, bm, a.penalty) == lo) hi = max(hi, (uint32_t)i);
        pick = ~block_min_u(~hi, sh);
      } else {
        pick = last;
      }
    }
  }
  if (threadIdx.x == 0) {
    if (a.out) a.out[m] = pick;
    if (a.tok) {
      const int p = a.pos[m];
      const uint32_t c = a.count[m];
      a.gen[(size_t)m * a.max_new + c] = pick;
      a.count[m] = c + 1;
      a.hist[(size_t)m * a.hist_stride + p] = pick;
      a.tok[m] = pick;
      const bool stop = pick == a.eos || p >= a.max_ctx;
      a.active[m] = stop ? 0 : 1;
      a.done[m] = stop || (int)c + 1 >= a.max_new ? 1 : 0;
    }
  }
}

__global__ void k_advance(int* pos, const int* active, int rows, const uint32_t* tok,
                          uint32_t* hist, long hist_stride) {
  const int m = threadIdx.x;
  if (m >= rows || !active[m]) return;
  if (tok) hist[(size_t)m * hist_stride + pos[m]] = tok[m];
  pos[m] += 1;
}

}  // namespace

size_t sample_scratch_bytes(int rows, int n) { return (size_t)rows * n * sizeof(double); }

// Workspace of the allocation-free sampler entry point (the per-row f64
// weights, kNoAllocSampleElems doubles = 16 MiB).  Every GPU the library
// runs on holds its own copy until the process ends.  In host code the
// array's name is not a device address: kernels get the address from
// sample_noalloc_scratch().  k_sample_rows writes every weight it reads
// within the same launch, so the array needs no clearing between calls.
namespace {
__device__ __align__(256) double scratch[kNoAllocSampleElems];
std::mutex g_scratch_mu;
double* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t sample_noalloc_scratch(int device, double** ptr) {
  if (device < 0 || device >= kMaxDevices || !ptr) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    // The caller made `device` current: its copy of the array is resolved.
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = static_cast<double*>(p);
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

hipError_t launch_advance(int* pos, const int* active, int rows, hipStream_t s,
                          const uint32_t* tok, uint32_t* hist, long hist_stride) {
  if (rows <= 0 || rows > 1024 || (tok && !hist)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_advance, dim3(1), dim3(64 * ((rows + 63) / 64)), 0, s, pos, active, rows,
                     tok, hist, hist_stride);
  return hipGetLastError();
}

hipError_t launch_sample_rows(const SampleArgs& a, int rows, hipStream_t s) {
  if (a.n <= 0 || a.n > kMaxSampleVocab || rows <= 0) return hipErrorInvalidValue;
  if (a.tok && (!a.pos || !a.hist || !a.start || !a.active || !a.done || !a.count || !a.gen ||
                a.max_new <= 0))
    return hipErrorInvalidValue;
  const size_t lds = a.penalty != 1.0f && (a.seen || a.tok) ? (size_t)(a.n + 31) / 32 * 4 : 0;
  // Rows sampled with 0 < top_k <= 256 over parts of the vocabulary: about
  // 256 blocks in all, at most 16 parts, each part's top_k and status within
  // the row's workspace of n doubles, and all parts' top_k within CCAP.
  int parts = 1;
  if (a.cnt && rows <= kSampleCounters && a.temperature > 0.0f && a.top_k > 0 &&
      a.top_k <= 256 && a.top_k < a.n) {
    parts = std::min(AKH_SAMPLE_BLOCKS / 16, std::max(1, AKH_SAMPLE_BLOCKS / rows));
    // The last block merges parts * top_k entries in its CCAP-entry buffer.
    while (parts > 1 && ((long)parts * (a.top_k + 1) > a.n || (long)parts * a.top_k > CCAP)) --parts;
  }
  hipLaunchKernelGGL(k_sample_rows, dim3(rows, parts), dim3(NT), lds, s, a);
  return hipGetLastError();
}

}  // namespace akh
