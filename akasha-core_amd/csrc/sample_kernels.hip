// Device-side token choice: sample_token of src/nn/sampling.rs:3-81 for a
// batch of rows, one 1024-thread block per row.
//
// The reference copies the logits, applies the repetition penalty to every
// distinct seen id, and then either takes the argmax (temperature <= 0) or
// sorts all ids by logit (descending), keeps the top_k, turns them into f64
// probabilities exp((l - max) / T) / sum, keeps the smallest prefix whose
// cumulative probability reaches top_p (renormalised), and walks the prefix
// with r = rand::random() until r < p.
//
// Here nothing is sorted.  Every cut the reference makes along the sorted
// order -- the k-th element, the top_p crossing, the element where the walk
// stops -- is found by a radix select over 32-bit order-preserving keys of
// the penalised logits: four 8-bit histogram passes narrow the key, counting
// elements (top_k) or summing their f64 weights (top_p, the walk), and the
// elements that share the final key are resolved in index order (the
// reference's unstable sort leaves that order unspecified; lower index first
// is this implementation's choice).  The per-element weights live in a
// scratch row; the repetition penalty is applied on the fly through a bitmap
// of the seen ids in LDS.
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.h"
#include "kernels.h"

namespace akh {

namespace {

constexpr int NT = 1024;        // threads per row
constexpr int NW = NT / 64;     // waves per block

struct SampleShared {
  uint32_t hist_n[256];
  double hist_w[256];
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

__device__ double block_sum_d(double v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_d[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int k = 0; k < NW; ++k) t += sh.wave_d[k];
  return t;
}

__device__ uint32_t block_sum_u(uint32_t v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_u[w] = v;
  __syncthreads();
  uint32_t t = 0;
  for (int k = 0; k < NW; ++k) t += sh.wave_u[k];
  return t;
}

__device__ uint32_t block_min_u(uint32_t v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_u[w] = v;
  __syncthreads();
  uint32_t t = 0xFFFFFFFFu;
  for (int k = 0; k < NW; ++k) t = min(t, sh.wave_u[k]);
  return t;
}

__device__ float block_max_f(float v, SampleShared& sh) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wave_f[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int k = 0; k < NW; ++k) t = fmaxf(t, sh.wave_f[k]);
  return t;
}

// Inclusive prefix sum over the block in thread order.
template <typename T>
__device__ T block_scan(T v, T* wave_tot) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const T u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  __syncthreads();
  if (lane == 63) wave_tot[w] = v;
  __syncthreads();
  T off = 0;
  for (int k = 0; k < w; ++k) off += wave_tot[k];
  return v + off;
}

// The element of the descending order at which a cumulative quantity
// crosses `target`: counts of elements (weights == nullptr, crossing when
// the count reaches target) or sums of weights[i] (crossing at >= target if
// inclusive, > target otherwise).  Returns the index, or n if the total
// never crosses.  `key_of(i)` gives element i's order key.
template <typename KeyFn>
__device__ uint32_t select_desc(int n, KeyFn key_of, const double* weights, double target,
                                bool inclusive, SampleShared& sh) {
  uint32_t prefix = 0, mask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += NT) {
      sh.hist_n[b] = 0;
      sh.hist_w[b] = 0.0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += NT) {
      const uint32_t k = key_of(i);
      if ((k & mask) == prefix) {
        const int bin = (k >> shift) & 255;
        if (weights) {
          const double w = weights[i];
          if (w != 0.0) atomicAdd(&sh.hist_w[bin], w);
        } else {
          atomicAdd(&sh.hist_n[bin], 1u);
        }
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      double acc = 0.0;
      int sel = -1;
      for (int b = 255; b >= 0; --b) {
        const double v = weights ? sh.hist_w[b] : (double)sh.hist_n[b];
        const double nxt = acc + v;
        if (weights ? (inclusive ? nxt >= target : nxt > target) : nxt >= target) {
          sel = b;
          break;
        }
        acc = nxt;
      }
      sh.bcast_u[0] = (uint32_t)sel;
      sh.bcast_d[0] = target - acc;
    }
    __syncthreads();
    const int sel = (int)sh.bcast_u[0];
    if (sel < 0) return (uint32_t)n;
    prefix |= (uint32_t)sel << shift;
    mask |= 0xFFu << shift;
    target = sh.bcast_d[0];
    __syncthreads();
  }
  // Elements with the final key, in index order.
  double base = 0.0;
  for (int c = 0; c < n; c += NT) {
    const int i = c + threadIdx.x;
    double v = 0.0;
    if (i < n && key_of(i) == prefix) v = weights ? weights[i] : 1.0;
    const double incl = block_scan<double>(v, sh.wave_d) + base;
    const bool hit = v != 0.0 && (weights ? (inclusive ? incl >= target : incl > target)
                                          : incl >= target);
    const uint32_t first = block_min_u(hit ? (uint32_t)i : 0xFFFFFFFFu, sh);
    if (first != 0xFFFFFFFFu) return first;
    base = block_sum_d(v, sh) + base;
  }
  return (uint32_t)n;
}

__global__ __launch_bounds__(NT) void k_sample_rows(SampleArgs a) {
  extern __shared__ uint32_t bitmap[];
  __shared__ SampleShared sh;
  const int m = blockIdx.x, n = a.n;
  const float* row = a.logits + (size_t)m * a.row_stride;
  double* w = a.wbuf + (size_t)m * n;

  // This row's seen ids and draw.
  const uint32_t* sr = nullptr;
  uint32_t cnt = 0;
  double r = 0.0;
  if (a.tok) {
    if (a.done[m]) {
      if (threadIdx.x == 0) a.active[m] = 0;
      return;
    }
    const int st = a.start[m], p = a.pos[m];
    sr = a.hist + (size_t)m * a.hist_stride + st;
    cnt = p > st ? (uint32_t)(p - st) : 0u;
    if (a.uniform) r = a.uniform[(size_t)a.count[m] * gridDim.x + m];
  } else {
    if (a.seen) {
      sr = a.seen + (size_t)m * a.seen_stride;
      cnt = a.seen_len ? min(a.seen_len[m], (uint32_t)a.seen_stride) : 0u;
    }
    if (a.uniform) r = a.uniform[m];
  }

  // Bitmap of this row's seen ids (only if the penalty changes anything).
  const uint32_t* bm = nullptr;
  if (a.penalty != 1.0f && sr) {
    const int words = (n + 31) / 32;
    for (int k = threadIdx.x; k < words; k += NT) bitmap[k] = 0;
    __syncthreads();
    for (uint32_t s = threadIdx.x; s < cnt; s += NT) {
      const uint32_t id = sr[s];
      if (id < (uint32_t)n) atomicOr(&bitmap[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    bm = bitmap;
  }
  auto key_of = [&](int i) { return order_key(pen_logit(row, i, bm, a.penalty)); };

  uint32_t pick;
  if (a.temperature <= 0.0f) {
    // sampling.rs:30-32, 83-91: first index of the maximum.
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int i = threadIdx.x; i < n; i += NT) amax_merge(bv, bi, pen_logit(row, i, bm, a.penalty), (uint32_t)i);
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
    const double sum = block_sum_d(part, sh);
    for (int i = threadIdx.x; i < n; i += NT) w[i] = w[i] / sum;
    __syncthreads();

    // top_p (sampling.rs:55-70): the smallest prefix reaching top_p, renormalised.
    uint32_t last = kth < (uint32_t)n ? kth : (uint32_t)n;  // last kept element, n = unknown
    if (a.top_p < 1.0f) {
      // No crossing keeps every element (and still renormalises).
      const uint32_t cut = select_desc(n, key_of, w, (double)a.top_p, true, sh);
      const uint32_t ckey = cut < (uint32_t)n ? key_of((int)cut) : 0u;
      double kept = 0.0;
      for (int i = threadIdx.x; i < n; i += NT) {
        if (cut < (uint32_t)n) {
          const uint32_t k = key_of(i);
          if (k < ckey || (k == ckey && (uint32_t)i > cut)) w[i] = 0.0;
        }
        kept += w[i];
      }
      const double s = block_sum_d(kept, sh);
      for (int i = threadIdx.x; i < n; i += NT) w[i] = w[i] / s;
      __syncthreads();
      if (cut < (uint32_t)n) last = cut;
    }

    // The walk (sampling.rs:72-80): first element whose cumulative
    // probability exceeds r; the last kept element if none does.
    pick = select_desc(n, key_of, w, r, false, sh);
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
  hipLaunchKernelGGL(k_sample_rows, dim3(rows), dim3(NT), lds, s, a);
  return hipGetLastError();
}

}  // namespace akh
