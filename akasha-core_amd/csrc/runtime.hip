// Runtime behind include/akasha_hip.h: backend, tensors, graphs, the
// per-shader launchers, ModelWeights and the batched InferenceSession.
//
// Reference interfaces mirrored here (paths relative to akasha-core's root):
//   InferenceSession      src/nn/inference.rs:13-326
//   DecodeScratch / Cache src/nn/inference_graphs.rs:13-196, 511-543
//   ModelWeights          src/nn/weights.rs:32-47, 158-171
//   AkashaError           src/lib.rs:10-37
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <cstring>
#include <unordered_map>
#include <vector>

#include "akasha_hip.h"
#include "checkpoint.h"
#include "kernels.h"

using namespace akh;

namespace {

thread_local std::string g_err;

akh_status fail(akh_status st, const std::string& msg) {
  g_err = msg;
  return st;
}

#define HIP_TRY(expr)                                                    \
  do {                                                                   \
    hipError_t e_ = (expr);                                              \
    if (e_ != hipSuccess)                                                \
      return fail(AKH_E_HIP, std::string(#expr) + ": " +                 \
                                 hipGetErrorString(e_));                 \
  } while (0)

#define CHECK_ARG(cond, msg)                                   \
  do {                                                         \
    if (!(cond)) return fail(AKH_E_INVALID, std::string(msg)); \
  } while (0)

// Head sizes the flash kernels take: any head_dim up to 128 dividing dim,
// as the reference's FLASH_ATTENTION (emit.rs:564-572).  Up to 32 the
// scalar kernel of the next power of two; beyond that the MFMA kernel of 64
// or 128 columns, the columns past the head size zero.
bool supported_head_dim(uint32_t hd) { return hd >= 1 && hd <= 128; }

}  // namespace

// ---------------------------------------------------------------------------
// Backend
// ---------------------------------------------------------------------------

struct akh_backend {
  int device = 0;
  int num_cus = 256;
  hipStream_t stream = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  bool capturing = false;
  void* scratch = nullptr;  // launcher scratch, grown on demand outside capture
  size_t scratch_bytes = 0;
  double* noalloc_scratch = nullptr;  // the device's fixed sampler workspace
  // The small-m MATMUL launchers' K-split partials and per-slab counters
  // (allocated with the backend, so graph capture never has to).
  float* gemv_ws = nullptr;
  int* gemv_cnt = nullptr;
  // The sampler's per-row arrival counters (zero between launches).
  int* sample_cnt = nullptr;
  // Tensor memory.  Every use of a tensor is on the backend's one stream, so
  // allocation, upload and free are ordered on it instead of waiting for it:
  // a freed block is kept (up to kPoolCap bytes) and handed out again zeroed
  // by a fill queued behind the work that used it before; an upload of up to
  // kStageSlot bytes is copied into a pinned slot and queued, the slot reused
  // once its copy has run.
  static constexpr size_t kPoolCap = (size_t)8 << 30;
  static constexpr int kStageSlots = 64;
  static constexpr size_t kStageSlot = 64 << 10;
  std::multimap<size_t, void*> pool;        // capacity -> free block
  std::unordered_map<void*, size_t> owned;  // block handed out -> capacity
  size_t pool_bytes = 0;
  char* stage = nullptr;
  hipEvent_t stage_done[kStageSlots] = {};
  bool stage_busy[kStageSlots] = {};
  int stage_next = 0;
};

namespace {

// Scratch of at least `bytes` on the backend's device.
akh_status backend_scratch(akh_backend* be, size_t bytes, void** out) {
  if (be->scratch_bytes < bytes) {
    CHECK_ARG(!be->capturing, "scratch must grow outside graph capture (run once eagerly first)");
    HIP_TRY(hipStreamSynchronize(be->stream));
    if (be->scratch) HIP_TRY(hipFree(be->scratch));
    be->scratch = nullptr;
    be->scratch_bytes = 0;
    HIP_TRY(hipMalloc(&be->scratch, bytes));
    be->scratch_bytes = bytes;
  }
  *out = be->scratch;
  return AKH_OK;
}

// Returns the pooled blocks to HIP (after the stream has drained).
hipError_t pool_release(akh_backend* be) {
  hipError_t e = hipStreamSynchronize(be->stream);
  for (auto& kv : be->pool) {
    hipError_t f = hipFree(kv.second);
    if (e == hipSuccess) e = f;
  }
  be->pool.clear();
  be->pool_bytes = 0;
  return e;
}

}  // namespace

struct akh_graph {
  akh_backend* be = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

extern "C" const char* akh_last_error(void) { return g_err.c_str(); }
extern "C" int akh_abi_version(void) { return AKH_ABI_VERSION; }

extern "C" akh_status akh_backend_new(int device, akh_backend** out) {
  CHECK_ARG(out, "akh_backend_new: out is NULL");
  *out = nullptr;
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  CHECK_ARG(device >= 0 && device < n, "akh_backend_new: no such device");
  HIP_TRY(hipSetDevice(device));
  akh_backend* be = new akh_backend();
  be->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess &&
      prop.multiProcessorCount > 0)
    be->num_cus = prop.multiProcessorCount;
  hipError_t e = hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&be->t0);
  if (e == hipSuccess) e = hipEventCreate(&be->t1);
  // The device's copy of the allocation-free sampler's workspace (device
  // current above).
  if (e == hipSuccess) e = sample_noalloc_scratch(device, &be->noalloc_scratch);
  if (e == hipSuccess) e = hipMalloc(&be->gemv_ws, kGemvWsFloats * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&be->gemv_cnt, kGemvSlabs * sizeof(int));
  if (e == hipSuccess) e = hipMemset(be->gemv_cnt, 0, kGemvSlabs * sizeof(int));
  if (e == hipSuccess) e = hipMalloc(&be->sample_cnt, kSampleCounters * sizeof(int));
  if (e == hipSuccess) e = hipMemset(be->sample_cnt, 0, kSampleCounters * sizeof(int));
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&be->stage),
                      akh_backend::kStageSlots * akh_backend::kStageSlot, hipHostMallocDefault);
  for (int i = 0; e == hipSuccess && i < akh_backend::kStageSlots; ++i)
    e = hipEventCreateWithFlags(&be->stage_done[i], hipEventDisableTiming);
  if (e != hipSuccess) {
    akh_backend_free(be);
    return fail(AKH_E_HIP, std::string("akh_backend_new: ") + hipGetErrorString(e));
  }
  *out = be;
  return AKH_OK;
}

extern "C" void akh_backend_free(akh_backend* be) {
  if (!be) return;
  hipSetDevice(be->device);
  if (be->stream) hipStreamSynchronize(be->stream);
  if (be->t0) hipEventDestroy(be->t0);
  if (be->t1) hipEventDestroy(be->t1);
  if (be->scratch) hipFree(be->scratch);
  if (be->gemv_ws) hipFree(be->gemv_ws);
  if (be->gemv_cnt) hipFree(be->gemv_cnt);
  if (be->sample_cnt) hipFree(be->sample_cnt);
  if (be->stream) pool_release(be);
  for (hipEvent_t ev : be->stage_done)
    if (ev) hipEventDestroy(ev);
  if (be->stage) hipHostFree(be->stage);
  if (be->stream) hipStreamDestroy(be->stream);
  delete be;
}

extern "C" akh_status akh_synchronize(akh_backend* be) {
  CHECK_ARG(be, "akh_synchronize: backend is NULL");
  CHECK_ARG(!be->capturing, "akh_synchronize: graph capture in progress");
  HIP_TRY(hipStreamSynchronize(be->stream));
  return AKH_OK;
}

namespace {

// A device block of `want` bytes from the backend's pool (one of at least
// `want` and at most twice that) or from HIP, its capacity in *cap.
akh_status tensor_block(akh_backend* be, size_t want, void** out, size_t* cap) {
  auto it = be->pool.lower_bound(want);
  if (it != be->pool.end() && it->first <= 2 * want) {
    *cap = it->first;
    *out = it->second;
    be->pool_bytes -= it->first;
    be->pool.erase(it);
    return AKH_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess && !be->pool.empty()) {  // give the pool back, retry
    (void)hipGetLastError();
    HIP_TRY(pool_release(be));
    e = hipMalloc(&p, want);
  }
  if (e != hipSuccess) return fail(AKH_E_HIP, std::string("tensor allocation: ") + hipGetErrorString(e));
  *cap = want;
  *out = p;
  return AKH_OK;
}

}  // namespace

extern "C" akh_status akh_tensor_alloc(akh_backend* be, size_t bytes,
                                       void** dev) {
  CHECK_ARG(be && dev, "akh_tensor_alloc: NULL argument");
  CHECK_ARG(!be->capturing, "akh_tensor_alloc: graph capture in progress");
  *dev = nullptr;
  const size_t want = bytes ? bytes : 4;
  void* p = nullptr;
  size_t cap = 0;
  akh_status st = tensor_block(be, want, &p, &cap);
  if (st != AKH_OK) return st;
  hipError_t e = hipMemsetAsync(p, 0, want, be->stream);
  if (e != hipSuccess) {
    hipFree(p);
    return fail(AKH_E_HIP, std::string("akh_tensor_alloc: ") + hipGetErrorString(e));
  }
  be->owned[p] = cap;
  *dev = p;
  return AKH_OK;
}

extern "C" akh_status akh_tensor_from_host(akh_backend* be, const void* host, size_t bytes,
                                           void** dev) {
  CHECK_ARG(be && dev && (host || !bytes), "akh_tensor_from_host: NULL argument");
  CHECK_ARG(!be->capturing, "akh_tensor_from_host: graph capture in progress");
  if (!bytes) return akh_tensor_alloc(be, 0, dev);
  *dev = nullptr;
  void* p = nullptr;
  size_t cap = 0;
  akh_status st = tensor_block(be, bytes, &p, &cap);
  if (st != AKH_OK) return st;
  be->owned[p] = cap;
  st = akh_tensor_upload(be, p, host, bytes);  // every byte written: no zero fill
  if (st != AKH_OK) {
    akh_tensor_free(be, p);
    return st;
  }
  *dev = p;
  return AKH_OK;
}

extern "C" akh_status akh_tensor_free(akh_backend* be, void* dev) {
  CHECK_ARG(be, "akh_tensor_free: backend is NULL");
  CHECK_ARG(!be->capturing, "akh_tensor_free: graph capture in progress");
  if (!dev) return AKH_OK;
  auto it = be->owned.find(dev);
  if (it != be->owned.end() && be->pool_bytes + it->second <= akh_backend::kPoolCap) {
    be->pool.emplace(it->second, dev);
    be->pool_bytes += it->second;
    be->owned.erase(it);
    return AKH_OK;
  }
  if (it != be->owned.end()) {
    be->owned.erase(it);
  } else {
    for (const auto& kv : be->pool)
      CHECK_ARG(kv.second != dev, "akh_tensor_free: tensor already freed");
  }
  HIP_TRY(hipStreamSynchronize(be->stream));
  HIP_TRY(hipFree(dev));
  return AKH_OK;
}

extern "C" akh_status akh_tensor_upload(akh_backend* be, void* dev,
                                        const void* host, size_t bytes) {
  CHECK_ARG(be && (dev || !bytes) && (host || !bytes),
            "akh_tensor_upload: NULL argument");
  CHECK_ARG(!be->capturing, "akh_tensor_upload: graph capture in progress");
  if (!bytes) return AKH_OK;
  if (bytes <= akh_backend::kStageSlot) {
    const int i = be->stage_next;
    be->stage_next = (i + 1) % akh_backend::kStageSlots;
    if (be->stage_busy[i]) HIP_TRY(hipEventSynchronize(be->stage_done[i]));
    char* slot = be->stage + (size_t)i * akh_backend::kStageSlot;
    memcpy(slot, host, bytes);
    HIP_TRY(hipMemcpyAsync(dev, slot, bytes, hipMemcpyHostToDevice, be->stream));
    HIP_TRY(hipEventRecord(be->stage_done[i], be->stream));
    be->stage_busy[i] = true;
    return AKH_OK;
  }
  HIP_TRY(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, be->stream));
  HIP_TRY(hipStreamSynchronize(be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_tensor_download(akh_backend* be, void* host,
                                          const void* dev, size_t bytes) {
  CHECK_ARG(be && (dev || !bytes) && (host || !bytes),
            "akh_tensor_download: NULL argument");
  CHECK_ARG(!be->capturing, "akh_tensor_download: graph capture in progress");
  if (!bytes) return AKH_OK;
  HIP_TRY(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, be->stream));
  HIP_TRY(hipStreamSynchronize(be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_graph_begin(akh_backend* be) {
  CHECK_ARG(be, "akh_graph_begin: backend is NULL");
  CHECK_ARG(!be->capturing, "akh_graph_begin: capture already in progress");
  HIP_TRY(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal));
  be->capturing = true;
  return AKH_OK;
}

extern "C" akh_status akh_graph_end(akh_backend* be, akh_graph** out) {
  CHECK_ARG(be && out, "akh_graph_end: NULL argument");
  CHECK_ARG(be->capturing, "akh_graph_end: no capture in progress");
  *out = nullptr;
  be->capturing = false;
  akh_graph* g = new akh_graph();
  g->be = be;
  hipError_t e = hipStreamEndCapture(be->stream, &g->graph);
  if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    akh_graph_free(g);
    return fail(AKH_E_HIP, std::string("akh_graph_end: ") + hipGetErrorString(e));
  }
  *out = g;
  return AKH_OK;
}

extern "C" akh_status akh_graph_execute(akh_graph* g) {
  CHECK_ARG(g && g->exec, "akh_graph_execute: invalid graph");
  CHECK_ARG(!g->be->capturing, "akh_graph_execute: capture in progress");
  HIP_TRY(hipGraphLaunch(g->exec, g->be->stream));
  return AKH_OK;
}

extern "C" void akh_graph_free(akh_graph* g) {
  if (!g) return;
  if (g->exec) hipGraphExecDestroy(g->exec);
  if (g->graph) hipGraphDestroy(g->graph);
  delete g;
}

extern "C" akh_status akh_timer_start(akh_backend* be) {
  CHECK_ARG(be && !be->capturing, "akh_timer_start: invalid backend state");
  HIP_TRY(hipEventRecord(be->t0, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_timer_stop(akh_backend* be, float* ms) {
  CHECK_ARG(be && ms && !be->capturing, "akh_timer_stop: invalid argument");
  HIP_TRY(hipEventRecord(be->t1, be->stream));
  HIP_TRY(hipEventSynchronize(be->t1));
  HIP_TRY(hipEventElapsedTime(ms, be->t0, be->t1));
  return AKH_OK;
}

// ---------------------------------------------------------------------------
// Per-shader launchers
// ---------------------------------------------------------------------------

#define BE_CHECK(be) CHECK_ARG(be, "backend is NULL")

extern "C" akh_status akh_embedding(akh_backend* be, const uint32_t* tokens,
                                    const float* table, float* out,
                                    akh_embedding_meta shape,
                                    const akh_embedding_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(tokens && table && out && meta, "akh_embedding: NULL buffer");
  HIP_TRY(shader_embedding(tokens, table, out, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_rmsnorm(akh_backend* be, const float* input,
                                  const float* weight, float* output,
                                  akh_norm_meta shape,
                                  const akh_norm_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(input && weight && output && meta, "akh_rmsnorm: NULL buffer");
  HIP_TRY(shader_rmsnorm(input, weight, output, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_matmul(akh_backend* be, const float* a,
                                 const float* b, float* c,
                                 akh_matmul_meta shape,
                                 const akh_matmul_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(a && b && c && meta, "akh_matmul: NULL buffer");
  HIP_TRY(shader_matmul(a, b, c, shape, meta, 0, be->gemv_ws, be->gemv_cnt, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_matmul_add(akh_backend* be, const float* a,
                                     const float* b, float* c,
                                     akh_matmul_meta shape,
                                     const akh_matmul_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(a && b && c && meta, "akh_matmul_add: NULL buffer");
  HIP_TRY(shader_matmul(a, b, c, shape, meta, 1, be->gemv_ws, be->gemv_cnt, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_head_gather(akh_backend* be, const float* src,
                                      float* dst, akh_head_move_meta shape,
                                      const akh_head_move_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(src && dst && meta, "akh_head_gather: NULL buffer");
  HIP_TRY(shader_head_gather(src, dst, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_rope(akh_backend* be, float* buf,
                               akh_rope_meta shape,
                               const akh_rope_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(buf && meta, "akh_rope: NULL buffer");
  CHECK_ARG(shape.head_dim && shape.dim % shape.head_dim == 0 &&
                shape.head_dim % 2 == 0,
            "akh_rope: head_dim must be even and divide dim");
  HIP_TRY(shader_rope(buf, shape.seq_len, shape.dim,
                      reinterpret_cast<const uint32_t*>(meta), 0, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_rope_offset(akh_backend* be, float* buf,
                                      akh_rope_offset_meta shape,
                                      const akh_rope_offset_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(buf && meta, "akh_rope_offset: NULL buffer");
  CHECK_ARG(shape.head_dim && shape.dim % shape.head_dim == 0 &&
                shape.head_dim % 2 == 0,
            "akh_rope_offset: head_dim must be even and divide dim");
  HIP_TRY(shader_rope(buf, shape.seq_len, shape.dim,
                      reinterpret_cast<const uint32_t*>(meta), 1, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_cache_write(akh_backend* be, const float* src,
                                      float* cache,
                                      akh_cache_write_meta shape,
                                      const akh_cache_write_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(src && cache && meta, "akh_cache_write: NULL buffer");
  HIP_TRY(shader_cache_write(src, cache, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_flash_attention(akh_backend* be, const float* q,
                                          const float* k, const float* v,
                                          float* out, float* l_cache,
                                          akh_flash_attn_meta shape,
                                          const akh_flash_attn_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(q && k && v && out && meta, "akh_flash_attention: NULL buffer");
  // emit.rs:564-572: head_dim <= 128 and dim % head_dim == 0.
  CHECK_ARG(shape.head_dim > 0 && shape.head_dim <= 128,
            "flash_attention: head_dim must be <= 128");
  CHECK_ARG(shape.dim % shape.head_dim == 0,
            "flash_attention: dim must be divisible by head_dim");
  HIP_TRY(shader_flash_attention(q, k, v, out, l_cache, shape, meta, 1, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_flash_attention_batched(akh_backend* be, const float* q,
                                                  const float* k, const float* v, float* out,
                                                  float* l_cache, akh_flash_attn_meta shape,
                                                  const akh_flash_attn_meta* meta,
                                                  uint32_t batch) {
  BE_CHECK(be);
  CHECK_ARG(q && k && v && out && meta, "akh_flash_attention_batched: NULL buffer");
  CHECK_ARG(shape.head_dim > 0 && shape.head_dim <= 128,
            "flash_attention: head_dim must be <= 128");
  CHECK_ARG(shape.dim % shape.head_dim == 0,
            "flash_attention: dim must be divisible by head_dim");
  HIP_TRY(shader_flash_attention(q, k, v, out, l_cache, shape, meta, batch, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_attn_qk_cached(akh_backend* be, const float* q,
                                         const float* k_cache, float* scores,
                                         uint32_t num_heads,
                                         uint32_t max_attn_len,
                                         const akh_attn_cached_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(q && k_cache && scores && meta, "akh_attn_qk_cached: NULL buffer");
  if (!num_heads || !max_attn_len) return AKH_OK;
  HIP_TRY(shader_attn_qk_cached(q, k_cache, scores, num_heads, max_attn_len,
                                meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_softmax_rect(akh_backend* be, float* scores,
                                       akh_softmax_rect_meta shape,
                                       const akh_softmax_rect_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(scores && meta, "akh_softmax_rect: NULL buffer");
  HIP_TRY(shader_softmax_rect(scores, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_attn_av_cached(akh_backend* be, const float* scores,
                                         const float* v_cache, float* out,
                                         uint32_t dim,
                                         const akh_attn_cached_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(scores && v_cache && out && meta, "akh_attn_av_cached: NULL buffer");
  if (!dim) return AKH_OK;
  HIP_TRY(shader_attn_av_cached(scores, v_cache, out, dim, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_silu(akh_backend* be, float* buf, uint32_t len) {
  BE_CHECK(be);
  CHECK_ARG(buf || !len, "akh_silu: NULL buffer");
  HIP_TRY(shader_silu(buf, len, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_qkv_split(akh_backend* be, const float* src, float* q, float* k,
                                    float* v, akh_head_move_meta shape,
                                    const akh_head_move_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(src && q && k && v && meta, "akh_qkv_split: NULL buffer");
  CHECK_ARG(shape.full_dim >= 3 * shape.head_dim, "akh_qkv_split: full_dim < 3 * head_dim");
  HIP_TRY(shader_qkv_split(src, q, k, v, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_rope_qk(akh_backend* be, float* q, float* k, akh_rope_meta shape,
                                  const akh_rope_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(q && k && meta, "akh_rope_qk: NULL buffer");
  CHECK_ARG(shape.head_dim && shape.dim % shape.head_dim == 0 && shape.head_dim % 2 == 0,
            "akh_rope_qk: head_dim must be even and divide dim");
  HIP_TRY(shader_rope_qk(q, k, shape, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_add(akh_backend* be, const float* a, const float* b, float* out,
                              uint32_t len) {
  BE_CHECK(be);
  CHECK_ARG((a && b && out) || !len, "akh_add: NULL buffer");
  HIP_TRY(shader_add(a, b, out, len, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_residual_add(akh_backend* be, float* target, const float* source,
                                       uint32_t len) {
  BE_CHECK(be);
  CHECK_ARG((target && source) || !len, "akh_residual_add: NULL buffer");
  HIP_TRY(shader_add(target, source, target, len, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_silu_out(akh_backend* be, const float* input, float* out,
                                   uint32_t len) {
  BE_CHECK(be);
  CHECK_ARG((input && out) || !len, "akh_silu_out: NULL buffer");
  HIP_TRY(shader_silu_out(input, out, len, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_cross_entropy(akh_backend* be, float* logits, const uint32_t* targets,
                                        float* losses, akh_cross_entropy_meta shape,
                                        const akh_cross_entropy_meta* meta) {
  BE_CHECK(be);
  CHECK_ARG(logits && targets && losses && meta, "akh_cross_entropy: NULL buffer");
  CHECK_ARG(shape.vocab_size > 0, "akh_cross_entropy: empty rows");
  HIP_TRY(launch_cross_entropy(logits, targets, losses, shape.num_rows, meta, be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_argmax_rows(akh_backend* be, const float* logits,
                                      uint32_t rows, uint32_t n,
                                      uint32_t* out) {
  BE_CHECK(be);
  CHECK_ARG(logits && out, "akh_argmax_rows: NULL buffer");
  CHECK_ARG(n > 0, "akh_argmax_rows: empty rows");
  HIP_TRY(shader_argmax_rows(logits, rows, n, out, be->stream));
  return AKH_OK;
}

namespace {
akh_status sample_rows_into(akh_backend* be, const float* logits, uint32_t rows, uint32_t n,
                            akh_sampling params, const uint32_t* seen, uint32_t seen_stride,
                            const uint32_t* seen_len, const double* uniforms, uint32_t* out,
                            double* wbuf, int* cnt);
}  // namespace

extern "C" akh_status akh_sample_rows(akh_backend* be, const float* logits, uint32_t rows,
                                      uint32_t n, akh_sampling params, const uint32_t* seen,
                                      uint32_t seen_stride, const uint32_t* seen_len,
                                      const double* uniforms, uint32_t* out) {
  CHECK_ARG(be && logits && out && rows > 0 && n > 0, "akh_sample_rows: bad argument");
  CHECK_ARG(n <= (uint32_t)kMaxSampleVocab, "akh_sample_rows: n exceeds 2^20");
  CHECK_ARG(params.temperature <= 0.0f || uniforms,
            "akh_sample_rows: sampling (temperature > 0) needs uniforms");
  CHECK_ARG(!seen || (seen_len && seen_stride > 0), "akh_sample_rows: seen needs seen_len");
  void* wb = nullptr;
  akh_status st = backend_scratch(be, sample_scratch_bytes((int)rows, (int)n), &wb);
  if (st != AKH_OK) return st;
  return sample_rows_into(be, logits, rows, n, params, seen, seen_stride, seen_len, uniforms,
                          out, static_cast<double*>(wb), be->sample_cnt);
}

extern "C" akh_status akh_sample_rows_noalloc(akh_backend* be, const float* logits,
                                              uint32_t rows, uint32_t n, akh_sampling params,
                                              const uint32_t* seen, uint32_t seen_stride,
                                              const uint32_t* seen_len, const double* uniforms,
                                              uint32_t* out) {
  CHECK_ARG(be && logits && out && rows > 0 && n > 0, "akh_sample_rows_noalloc: bad argument");
  CHECK_ARG(n <= (uint32_t)kMaxSampleVocab, "akh_sample_rows_noalloc: n exceeds 2^20");
  CHECK_ARG((size_t)rows * n <= kNoAllocSampleElems,
            "akh_sample_rows_noalloc: rows * n exceeds 2^21, the fixed workspace");
  CHECK_ARG(params.temperature <= 0.0f || uniforms,
            "akh_sample_rows_noalloc: sampling (temperature > 0) needs uniforms");
  CHECK_ARG(!seen || (seen_len && seen_stride > 0),
            "akh_sample_rows_noalloc: seen needs seen_len");
  CHECK_ARG(be->noalloc_scratch, "akh_sample_rows_noalloc: no workspace on this device");
  return sample_rows_into(be, logits, rows, n, params, seen, seen_stride, seen_len, uniforms,
                          out, be->noalloc_scratch, nullptr);
}

namespace {

// The sampler launch of akh_sample_rows / akh_sample_rows_noalloc, on the
// workspace `wbuf` (rows * n doubles); allocates nothing.
akh_status sample_rows_into(akh_backend* be, const float* logits, uint32_t rows, uint32_t n,
                            akh_sampling params, const uint32_t* seen, uint32_t seen_stride,
                            const uint32_t* seen_len, const double* uniforms, uint32_t* out,
                            double* wbuf, int* cnt) {
  SampleArgs a{};
  a.logits = logits;
  a.n = (int)n;
  a.row_stride = n;
  a.temperature = params.temperature;
  a.top_k = (int)std::min<uint32_t>(params.top_k, 0x7FFFFFFFu);
  a.top_p = params.top_p;
  a.penalty = params.repetition_penalty;
  a.seen = seen;
  a.seen_stride = seen_stride;
  a.seen_len = seen_len;
  a.uniform = uniforms;
  a.wbuf = wbuf;
  a.out = out;
  a.cnt = cnt;
  HIP_TRY(launch_sample_rows(a, (int)rows, be->stream));
  return AKH_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Model weights
// ---------------------------------------------------------------------------

// A weight matrix as the decode kernels read it: packed 32-column tiles of
// `rows` k (launch_pack_tiles), float or bfloat16, refreshed whenever the
// parameter is uploaded.
struct PackedMatrix {
  float* w = nullptr;
  int K = 0, N = 0, rows = 0, role = 0;
  bool bf16 = false;  // tiles hold bfloat16 (every value of the matrix is one)
  bool h3 = false;    // lm_head tiles hold fp16 hi/lo terms (launch_pack_lm_h3)
};

struct akh_model {
  akh_backend* be = nullptr;
  akh_model_config cfg{};
  std::vector<float*> params;  // ModelWeights::params() order
  std::vector<size_t> counts;
  std::vector<PackedMatrix> packed;  // per parameter; w == nullptr if not a decode matrix
  int* bf16_flag = nullptr;          // device scratch of the bfloat16 check
  bool allow_bf16 = true;            // bfloat16 tiles where every value is one
  bool prefill_bf16 = false;         // the optional bfloat16-MFMA prefill
  std::vector<uint16_t*> wt16;       // per parameter: bf16 [N, K] copy (layer matrices)
  // The f32 prefill's layer GEMMs (and the trainer forward's lm_head) on
  // split operands, fp32-accurate: SPLIT_NONE runs the fp32-MFMA kernels,
  // SPLIT_X6 three bfloat16 terms per operand (k_gemm_x6, on transposed fp32
  // [N, K] copies), SPLIT_H3 two fp16 terms (k_gemm_h3, on fp16 planes), the
  // default where dim and ffn_hidden are multiples of 8.  wsplit holds the
  // copies per parameter (layer matrices and lm_head).  Flash attention
  // follows the split: split-fp16 (k_flash_h3, flagged and rerun like the
  // GEMMs) under SPLIT_H3, split-bfloat16 (k_flash_x6) under SPLIT_X6.
  int prefill_split = AKH_SPLIT_NONE;
  std::vector<void*> wsplit;
  int* range_flag = nullptr;  // set by k_gemm_h3 on a non-finite result
  uint64_t layout_gen = 0;           // bumped when a packed matrix changes element type

  float* embedding() const { return params[0]; }
  float* layer(uint32_t l, int which) const { return params[1 + 6 * l + which]; }
  float* final_norm() const { return params[1 + 6 * cfg.num_layers]; }
  float* lm_head() const { return params[2 + 6 * cfg.num_layers]; }
  const PackedMatrix& packed_layer(uint32_t l, int which) const {
    return packed[1 + 6 * l + which];
  }
  const PackedMatrix& packed_lm_head() const { return packed[2 + 6 * cfg.num_layers]; }
};

enum { W_NORM1 = 0, W_QKV = 1, W_OUT = 2, W_NORM2 = 3, W_UP = 4, W_DOWN = 5 };

extern "C" void akh_model_free(akh_model* m) {
  if (!m) return;
  hipSetDevice(m->be->device);
  hipStreamSynchronize(m->be->stream);
  for (float* p : m->params)
    if (p) hipFree(p);
  for (const PackedMatrix& pm : m->packed)
    if (pm.w) hipFree(pm.w);
  if (m->bf16_flag) hipFree(m->bf16_flag);
  for (uint16_t* p : m->wt16)
    if (p) hipFree(p);
  for (void* p : m->wsplit)
    if (p) hipFree(p);
  delete m;
}

namespace {

bool split_capable(const akh_model_config& c) { return c.dim % 8 == 0 && c.ffn_hidden % 8 == 0; }

// The split kernels' copy of parameter `index` from the parameter itself.
hipError_t fill_split(akh_model* m, uint32_t index, hipStream_t st) {
  const PackedMatrix& pm = m->packed[index];
  if (m->prefill_split == AKH_SPLIT_X6)
    return launch_transpose_f32(m->params[index], pm.K, pm.N, static_cast<float*>(m->wsplit[index]),
                                st);
  return launch_split_weights_f16(m->params[index], pm.K, pm.N,
                                  static_cast<uint16_t*>(m->wsplit[index]), st);
}

// Frees the split copies and allocates (zeroed) those of `kind`; `fill`
// fills them from the parameters (else their uploads do).
akh_status set_split(akh_model* m, int kind, bool fill) {
  HIP_TRY(hipSetDevice(m->be->device));
  HIP_TRY(hipStreamSynchronize(m->be->stream));
  for (void*& p : m->wsplit)
    if (p) {
      HIP_TRY(hipFree(p));
      p = nullptr;
    }
  m->prefill_split = AKH_SPLIT_NONE;
  if (kind == AKH_SPLIT_NONE) return AKH_OK;
  m->wsplit.assign(m->params.size(), nullptr);
  m->prefill_split = kind;
  for (uint32_t i = 0; i < m->packed.size(); ++i) {
    const PackedMatrix& pm = m->packed[i];
    if (!pm.rows) continue;
    // Both copies take 4 bytes per element: an fp32 value, or two fp16 terms.
    void* p = nullptr;
    akh_status st = akh_tensor_alloc(m->be, (size_t)pm.K * pm.N * 4, &p);
    if (st != AKH_OK) {
      set_split(m, AKH_SPLIT_NONE, false);
      return st;
    }
    m->wsplit[i] = p;
    if (fill) HIP_TRY(fill_split(m, i, m->be->stream));
  }
  HIP_TRY(hipStreamSynchronize(m->be->stream));
  return AKH_OK;
}

}  // namespace

extern "C" akh_status akh_model_new(akh_backend* be,
                                    const akh_model_config* cfg,
                                    akh_model** out) {
  CHECK_ARG(be && cfg && out, "akh_model_new: NULL argument");
  *out = nullptr;
  const akh_model_config c = *cfg;
  // config.rs:15-17: at least one layer, dim divisible by heads.
  CHECK_ARG(c.num_layers >= 1, "At least one layer is required!");
  CHECK_ARG(c.num_heads > 0 && c.dim % c.num_heads == 0,
            "dim must be divisible by num_heads");
  CHECK_ARG(c.vocab_size > 0 && c.ffn_hidden > 0, "empty vocab or ffn");
  akh_model* m = new akh_model();
  m->be = be;
  m->cfg = c;
  const size_t d = c.dim, V = c.vocab_size, F = c.ffn_hidden;
  m->counts.push_back(V * d);
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    m->counts.push_back(d);
    m->counts.push_back(d * 3 * d);
    m->counts.push_back(d * d);
    m->counts.push_back(d);
    m->counts.push_back(d * F);
    m->counts.push_back(F * d);
  }
  m->counts.push_back(d);
  m->counts.push_back(d * V);
  for (size_t n : m->counts) {
    void* p = nullptr;
    akh_status st = akh_tensor_alloc(be, n * sizeof(float), &p);
    if (st != AKH_OK) {
      akh_model_free(m);
      return st;
    }
    m->params.push_back(static_cast<float*>(p));
  }
  // Packed copies of the decode matrices (zero until their upload).
  m->packed.resize(m->params.size());
  auto plan = [&](size_t index, int role, size_t K, size_t N) {
    PackedMatrix& pm = m->packed[index];
    pm.K = (int)K;
    pm.N = (int)N;
    pm.rows = dec_packed_rows(role, (int)K);
    pm.role = role;
  };
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    plan(1 + 6 * l + W_QKV, DEC_CFG_QKV, d, 3 * d);
    plan(1 + 6 * l + W_OUT, DEC_CFG_OUT, d, d);
    plan(1 + 6 * l + W_UP, DEC_CFG_UP, d, F);
    plan(1 + 6 * l + W_DOWN, DEC_CFG_DOWN, F, d);
  }
  plan(2 + 6 * c.num_layers, DEC_CFG_LM, d, V);
  for (PackedMatrix& pm : m->packed) {
    if (!pm.rows) continue;
    void* p = nullptr;
    const size_t n = (size_t)(pm.N + 31) / 32 * 32 * pm.rows;
    akh_status st = akh_tensor_alloc(be, n * sizeof(float), &p);
    if (st != AKH_OK) {
      akh_model_free(m);
      return st;
    }
    pm.w = static_cast<float*>(p);
  }
  {
    void* p = nullptr;
    akh_status st = akh_tensor_alloc(be, 2 * sizeof(int), &p);
    if (st != AKH_OK) {
      akh_model_free(m);
      return st;
    }
    m->bf16_flag = static_cast<int*>(p);
    m->range_flag = m->bf16_flag + 1;
  }
  if (split_capable(c)) {
    akh_status st = set_split(m, AKH_SPLIT_H3, false);  // filled as parameters are uploaded
    if (st != AKH_OK) {
      akh_model_free(m);
      return st;
    }
  }
  *out = m;
  return AKH_OK;
}

extern "C" uint32_t akh_model_num_params(const akh_model* m) {
  return m ? (uint32_t)m->params.size() : 0u;
}

extern "C" akh_status akh_model_param(akh_model* m, uint32_t index,
                                      float** dev, size_t* count) {
  CHECK_ARG(m && index < m->params.size(), "akh_model_param: bad index");
  if (dev) *dev = m->params[index];
  if (count) *count = m->counts[index];
  return AKH_OK;
}

namespace {

#ifndef AKH_LM_H3
#define AKH_LM_H3 1
#endif
// Rebuilds the packed decode copy of parameter `index` from its rows: in
// bfloat16 when the role's kernel supports it and every value is a
// bfloat16, else in float.
akh_status repack(akh_model* m, uint32_t index) {
  PackedMatrix& pm = m->packed[index];
  if (!pm.w) return AKH_OK;
  hipStream_t st = m->be->stream;
  bool bf16 = false;
  if (m->allow_bf16 && dec_bf16_capable(pm.role, pm.K, pm.N)) {
    int flag = 0;
    HIP_TRY(hipMemcpyAsync(m->bf16_flag, &flag, sizeof(int), hipMemcpyHostToDevice, st));
    HIP_TRY(launch_check_bf16(m->params[index], (size_t)pm.K * pm.N, m->bf16_flag, st));
    HIP_TRY(hipMemcpyAsync(&flag, m->bf16_flag, sizeof(int), hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    bf16 = flag == 0;
  }
  // The persistent lm_head reads split-fp16 tiles (the same bytes as float
  // ones, a fifth of the MFMA cycles) unless a weight is beyond fp16's range.
  bool h3 = false;
  if (AKH_LM_H3 && pm.role == DEC_CFG_LM && !bf16 && dec_lm_h3_capable(pm.K, pm.N)) {
    int flag = 0;
    HIP_TRY(hipMemcpyAsync(m->bf16_flag, &flag, sizeof(int), hipMemcpyHostToDevice, st));
    HIP_TRY(launch_pack_lm_h3(m->params[index], pm.K, pm.N, pm.rows,
                              reinterpret_cast<uint16_t*>(pm.w), m->bf16_flag, st));
    HIP_TRY(hipMemcpyAsync(&flag, m->bf16_flag, sizeof(int), hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    h3 = flag == 0;
  }
  if (!h3) HIP_TRY(launch_pack_tiles(m->params[index], pm.K, pm.N, pm.rows, pm.w, bf16, st));
  if (index < m->wt16.size() && m->wt16[index])
    HIP_TRY(launch_transpose_bf16(m->params[index], pm.K, pm.N, m->wt16[index], st));
  if (index < m->wsplit.size() && m->wsplit[index]) HIP_TRY(fill_split(m, index, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (bf16 != pm.bf16 || h3 != pm.h3) {
    pm.bf16 = bf16;
    pm.h3 = h3;
    ++m->layout_gen;  // captured decode graphs chose kernels by element type
  }
  return AKH_OK;
}

}  // namespace

extern "C" akh_status akh_model_set_prefill_bf16(akh_model* m, int enable) {
  CHECK_ARG(m && (enable == 0 || enable == 1), "akh_model_set_prefill_bf16: bad argument");
  CHECK_ARG(!m->be->capturing, "akh_model_set_prefill_bf16: graph capture in progress");
  const akh_model_config& c = m->cfg;
  const uint32_t hd = c.dim / c.num_heads;
  CHECK_ARG(!enable || ((hd == 64 || hd == 128) && c.dim % 8 == 0 && c.ffn_hidden % 8 == 0),
            "akh_model_set_prefill_bf16: needs head_dim 64 or 128 and dim, ffn_hidden "
            "multiples of 8");
  HIP_TRY(hipSetDevice(m->be->device));
  HIP_TRY(hipStreamSynchronize(m->be->stream));
  for (uint16_t*& p : m->wt16)
    if (p) {
      HIP_TRY(hipFree(p));
      p = nullptr;
    }
  m->prefill_bf16 = false;
  if (!enable) return AKH_OK;
  m->wt16.assign(m->params.size(), nullptr);
  for (uint32_t l = 0; l < c.num_layers; ++l)
    for (int which : {W_QKV, W_OUT, W_UP, W_DOWN}) {
      const uint32_t i = 1 + 6 * l + which;
      const PackedMatrix& pm = m->packed[i];
      void* p = nullptr;
      akh_status st = akh_tensor_alloc(m->be, (size_t)pm.K * pm.N * sizeof(uint16_t), &p);
      if (st != AKH_OK) return st;
      m->wt16[i] = static_cast<uint16_t*>(p);
      HIP_TRY(launch_transpose_bf16(m->params[i], pm.K, pm.N, m->wt16[i], m->be->stream));
    }
  HIP_TRY(hipStreamSynchronize(m->be->stream));
  m->prefill_bf16 = true;
  return AKH_OK;
}

extern "C" akh_status akh_model_set_prefill_split(akh_model* m, int kind) {
  CHECK_ARG(m && (kind == AKH_SPLIT_NONE || kind == AKH_SPLIT_X6 || kind == AKH_SPLIT_H3),
            "akh_model_set_prefill_split: bad argument");
  CHECK_ARG(!m->be->capturing, "akh_model_set_prefill_split: graph capture in progress");
  CHECK_ARG(kind == AKH_SPLIT_NONE || split_capable(m->cfg),
            "akh_model_set_prefill_split: needs dim and ffn_hidden multiples of 8");
  if (kind == m->prefill_split) return AKH_OK;
  return set_split(m, kind, true);
}

extern "C" int akh_model_prefill_split(const akh_model* m) {
  return m ? m->prefill_split : AKH_SPLIT_NONE;
}

extern "C" akh_status akh_model_set_prefill_x6(akh_model* m, int enable) {
  CHECK_ARG(m && (enable == 0 || enable == 1), "akh_model_set_prefill_x6: bad argument");
  return akh_model_set_prefill_split(m, enable ? AKH_SPLIT_X6 : AKH_SPLIT_NONE);
}

extern "C" akh_status akh_model_set_bf16_tiles(akh_model* m, int allow, uint32_t* n_bf16) {
  CHECK_ARG(m && (allow == 0 || allow == 1), "akh_model_set_bf16_tiles: bad argument");
  CHECK_ARG(!m->be->capturing, "akh_model_set_bf16_tiles: graph capture in progress");
  m->allow_bf16 = allow != 0;
  uint32_t n = 0;
  for (uint32_t i = 0; i < m->packed.size(); ++i) {
    akh_status st = repack(m, i);
    if (st != AKH_OK) return st;
    n += m->packed[i].bf16 ? 1u : 0u;
  }
  if (n_bf16) *n_bf16 = n;
  return AKH_OK;
}

extern "C" akh_status akh_model_upload_param(akh_model* m, uint32_t index,
                                             const float* host, size_t count) {
  CHECK_ARG(m && index < m->params.size(), "akh_model_upload_param: bad index");
  CHECK_ARG(count == m->counts[index], "akh_model_upload_param: size mismatch");
  akh_status st = akh_tensor_upload(m->be, m->params[index], host, count * sizeof(float));
  if (st != AKH_OK) return st;
  return repack(m, index);
}

// ---------------------------------------------------------------------------
// Checkpoints (src/nn/checkpoint.rs)
// ---------------------------------------------------------------------------

namespace {

// Walks the tensor lists of an opened file (structure only).
akh_status ckpt_walk(CkptReader& r, uint64_t* total, uint64_t* pairs) {
  uint64_t t = 0, p = 0;
  for (uint64_t i = 0; i < r.head.num_params; ++i) {
    uint64_t n = 0;
    if (!r.tensor_len(n) || !r.skip_floats(n)) return fail(AKH_E_IO, r.err);
    t += n;
  }
  if (!r.u64(p)) return fail(AKH_E_IO, r.err);
  for (uint64_t i = 0; i < 2 * p; ++i) {
    uint64_t n = 0;
    if (!r.tensor_len(n) || !r.skip_floats(n)) return fail(AKH_E_IO, r.err);
  }
  if (total) *total = t;
  if (pairs) *pairs = p;
  return AKH_OK;
}

akh_status ckpt_open(CkptReader& r, const char* path) {
  if (!r.open(path)) return fail(r.io_error ? AKH_E_IO : AKH_E_INVALID, r.err);
  return AKH_OK;
}

}  // namespace

extern "C" akh_status akh_checkpoint_info(const char* path, akh_checkpoint_info_t* info) {
  CHECK_ARG(path && info, "akh_checkpoint_info: NULL argument");
  memset(info, 0, sizeof(*info));
  CkptReader r;
  akh_status st = ckpt_open(r, path);
  if (st != AKH_OK) return st;
  info->vocab_size = r.head.vocab_size;
  info->dim = r.head.dim;
  info->num_heads = r.head.num_heads;
  info->num_layers = r.head.num_layers;
  info->seq_len = r.head.seq_len;
  info->ffn_hidden = r.head.ffn_hidden;
  info->train_step = r.head.train_step;
  info->schedule_step = r.head.schedule_step;
  info->num_params = r.head.num_params;
  return ckpt_walk(r, &info->total_param_floats, &info->num_moment_pairs);
}

extern "C" akh_status akh_model_load_checkpoint(akh_model* m, const char* path,
                                                uint64_t* train_step,
                                                int* has_optimizer) {
  CHECK_ARG(m && path, "akh_model_load_checkpoint: NULL argument");
  // bincode::deserialize_from reads the whole body before any check.
  uint64_t pairs = 0;
  {
    CkptReader r;
    akh_status st = ckpt_open(r, path);
    if (st == AKH_OK) st = ckpt_walk(r, nullptr, &pairs);
    if (st != AKH_OK) return st;
  }
  CkptReader r;
  akh_status st = ckpt_open(r, path);
  if (st != AKH_OK) return st;
  const akh_model_config& c = m->cfg;
  const CkptHeader& h = r.head;
  if (h.vocab_size != c.vocab_size || h.dim != c.dim || h.num_heads != c.num_heads ||
      h.num_layers != (uint64_t)c.num_layers || h.ffn_hidden != c.ffn_hidden) {
    char msg[512];  // checkpoint.rs:111-129
    snprintf(msg, sizeof msg,
             "checkpoint architecture mismatch: file (%u, %u, %u, %llu, %u) vs model "
             "(%u, %u, %u, %u, %u) (vocab_size, dim, num_heads, num_layers, ffn_hidden)",
             h.vocab_size, h.dim, h.num_heads, (unsigned long long)h.num_layers,
             h.ffn_hidden, c.vocab_size, c.dim, c.num_heads, c.num_layers, c.ffn_hidden);
    return fail(AKH_E_INVALID, msg);
  }
  if (h.num_params != m->params.size())  // checkpoint.rs:162-168
    return fail(AKH_E_INVALID, "checkpoint has " + std::to_string(h.num_params) +
                                   " parameter tensors, model expects " +
                                   std::to_string(m->params.size()));
  std::vector<float> host;
  for (uint32_t i = 0; i < m->params.size(); ++i) {
    uint64_t n = 0;
    if (!r.tensor_len(n)) return fail(AKH_E_IO, r.err);
    if (n != m->counts[i])  // checkpoint.rs:173-181
      return fail(AKH_E_INVALID, "checkpoint tensor " + std::to_string(i) + " has " +
                                     std::to_string(n) + " elements, model expects " +
                                     std::to_string(m->counts[i]));
    host.resize((size_t)n);
    if (!r.floats(host.data(), n)) return fail(AKH_E_IO, r.err);
    st = akh_model_upload_param(m, i, host.data(), (size_t)n);
    if (st != AKH_OK) return st;
  }
  if (pairs != 0 && pairs != m->params.size())  // checkpoint.rs:137-145
    return fail(AKH_E_INVALID, "checkpoint has " + std::to_string(pairs) +
                                   " moment pairs, model expects " +
                                   std::to_string(m->params.size()));
  if (train_step) *train_step = h.train_step;
  if (has_optimizer) *has_optimizer = pairs != 0;
  return AKH_OK;
}

// ---------------------------------------------------------------------------
// Batched session
// ---------------------------------------------------------------------------

struct akh_session {
  akh_model* m = nullptr;
  akh_backend* be = nullptr;
  uint32_t max_ctx = 0, B = 0;
  std::vector<uint32_t> cur_len;
  std::vector<uint8_t> has_cache;  // InferenceSession::cache is Some (per sequence)

  // Cache: per layer, K then V, each [B, max_ctx, dim]; sequence b's slice
  // is exactly the reference's per-session Cache tensor [max_ctx, dim].
  float* kv = nullptr;
  float2* rope = nullptr;  // [max_ctx, head_dim / 2] (cos, sin)

  // Decode-step state, 32 rows (the MFMA tile height).  *_t buffers are in
  // the k-quad layout [K/4][32][4]; p_* hold a GEMM's partial tiles.
  float* xt = nullptr;      // residual stream
  float* xnt = nullptr;     // RMSNorm of the residual stream (GEMM input)
  float* attn_t = nullptr;  // attention splits: unnormalised o [splits][32][dim]
  float2* attn_ml = nullptr;  // attention splits: (max, sum) [splits][heads][32]
  float* p_qkv = nullptr;   // [ks_qkv][32][3*dim]
  float* p_out = nullptr;   // [ks_out] partial tiles of [32, dim] (k-quad when fused)
  float* p_up = nullptr;    // [ks_up] k-quad tiles of [32, ffn]
  float* up_act = nullptr;  // silu(ffn_up) when summed by its own kernel
  float* p_down = nullptr;  // [ks_down] partial tiles of [32, dim] (k-quad when fused)
  // With the RMSNorm folded into the GEMMs (akh_session_set_fused_norm):
  // out_proj (fuse_out) and ffn_down (fuse_down) add their sums to xt
  // themselves and write ssq [32][dim / 32], the new residual's sums of
  // squares per 32-column tile, which ffn_up, qkv_proj and the final norm
  // turn into each row's scale: 5 launches per layer instead of 7.  Off by
  // default: the cross-block handoff in those epilogues costs more than the
  // two kernel boundaries it removes.  rcount holds the per-column-tile
  // block counters of the epilogues (zero between launches).
  bool fuse_out = false, fuse_down = false;
  float* ssq = nullptr;
  int* rcount = nullptr;
  float* logits = nullptr;  // [32, vocab]
  uint2* amax = nullptr;    // [32, lm tiles] argmax partials
  uint32_t* tok = nullptr;  // tokens fed to the next step
  int* pos = nullptr;       // per-sequence position of the next token
  uint32_t* hist = nullptr; // [B, max_ctx + 1] token at each position

  int ks_qkv = 1, ks_out = 1, ks_up = 1, ks_down = 1;
  // A shape the batched decode kernels do not take (dec_fast_shape): the
  // step runs on decode_generic.hip's kernels over row-major activations
  // (residual, normed rows, qkv, attention output, ffn), and the lm_head
  // leaves one argmax partial per row.
  bool generic = false;
  float *gx = nullptr, *gxn = nullptr, *gqkv = nullptr, *gattn = nullptr, *gffn = nullptr;
  // 32-row tiles of the decode rows (B <= 32 * mt): activations are
  // [mt][K/4][32][4], partial tiles [splits][32 * mt][N].
  int mt = 1;
  size_t rows() const { return (size_t)32 * mt; }

  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  hipGraph_t graph_n = nullptr;       // kStepsPerGraph decode steps in one graph
  hipGraphExec_t gexec_n = nullptr;
  uint64_t glayout = 0;  // model layout_gen the graphs were captured for

  // Prefill buffers, grown on demand to the prompt rows (B * prompt_len, or
  // the sum of ragged prompt lengths).
  size_t prows = 0;
  float *px = nullptr, *pxn = nullptr, *pq = nullptr, *pattn = nullptr,
        *pffn = nullptr;
  uint32_t* ptok = nullptr;
  // Ragged prompts packed back to back: sequence b's rows [p_at[b],
  // p_at[b + 1]), row r = position p_map[r].y of sequence p_map[r].x, its
  // last row p_last[b] and its length p_len[b].
  int* p_at = nullptr;
  int2* p_map = nullptr;
  int *p_last = nullptr, *p_len = nullptr;

  // InferenceSession::generate on the device: per-row state of the rounds.
  int* active = nullptr;   // row is decoded this round (attention skips others)
  int* done = nullptr;     // row stopped sampling
  int* gstart = nullptr;   // position of the call's first prompt token
  uint32_t* gcount = nullptr;  // tokens generated so far
  uint32_t* ggen = nullptr;    // [B, gcap] generated tokens
  double* guni = nullptr;      // [gcap, B] draws
  double* gwbuf = nullptr;     // sampler scratch
  uint32_t gcap = 0;
  hipGraph_t ggraph = nullptr;
  hipGraphExec_t ggexec = nullptr;
  akh_sampling gparams{};
  uint32_t gmax_new = 0;

  // KV cache: [L][K,V][B][max_ctx][d] elements, fp32 or (kv16) bfloat16.
  bool kv16 = false;
  float *pk = nullptr, *pv = nullptr;  // kv16 prefill: K/V rows in fp32 [rows, d]
  size_t kv_elem() const { return kv16 ? 2 : 4; }
  size_t layer_stride() const { return (size_t)2 * B * max_ctx * m->cfg.dim; }
  void* kv_at(uint32_t l, int which) {
    const size_t e = l * layer_stride() + (size_t)which * B * max_ctx * m->cfg.dim;
    return reinterpret_cast<char*>(kv) + e * kv_elem();
  }
  float* kcache(uint32_t l) { return static_cast<float*>(kv_at(l, 0)); }  // fp32 caches
  float* vcache(uint32_t l) { return static_cast<float*>(kv_at(l, 1)); }
  long seq_stride() const { return (long)max_ctx * m->cfg.dim; }
};

namespace {

// The lm_head's argmax partials per row for the model's current tiles, and
// the most any tiles need (the size of amax).
int lm_parts(const akh_session* s) {
  return dec_lm_parts((int)s->m->cfg.vocab_size, (int)s->m->cfg.dim, s->be->num_cus, s->mt,
                      s->m->packed_lm_head().h3);
}
int lm_parts_max(const akh_session* s) {
  return dec_lm_parts((int)s->m->cfg.vocab_size, (int)s->m->cfg.dim, s->be->num_cus, s->mt,
                      false);
}
// The argmax partials per row the step's lm_head leaves.
int argmax_parts(const akh_session* s) { return s->generic ? 1 : lm_parts(s); }

void free_prefill(akh_session* s) {
  for (float* p : {s->px, s->pxn, s->pq, s->pattn, s->pffn, s->pk, s->pv})
    if (p) hipFree(p);
  for (void* p : {(void*)s->ptok, (void*)s->p_at, (void*)s->p_map, (void*)s->p_last,
                  (void*)s->p_len})
    if (p) hipFree(p);
  s->px = s->pxn = s->pq = s->pattn = s->pffn = s->pk = s->pv = nullptr;
  s->ptok = nullptr;
  s->p_at = s->p_last = s->p_len = nullptr;
  s->p_map = nullptr;
  s->prows = 0;
}

akh_status ensure_prefill(akh_session* s, size_t rows) {
  if (rows <= s->prows) return AKH_OK;
  free_prefill(s);
  const size_t d = s->m->cfg.dim, F = s->m->cfg.ffn_hidden;
  HIP_TRY(hipMalloc(&s->px, rows * d * 4));
  HIP_TRY(hipMalloc(&s->pxn, rows * d * 4));
  HIP_TRY(hipMalloc(&s->pq, rows * d * 4));
  HIP_TRY(hipMalloc(&s->pattn, rows * d * 4));
  HIP_TRY(hipMalloc(&s->pffn, rows * F * 4));
  HIP_TRY(hipMalloc(&s->ptok, rows * 4));
  HIP_TRY(hipMalloc(&s->p_at, (s->B + 1) * sizeof(int)));
  HIP_TRY(hipMalloc(&s->p_map, rows * sizeof(int2)));
  HIP_TRY(hipMalloc(&s->p_last, s->B * sizeof(int)));
  HIP_TRY(hipMalloc(&s->p_len, s->B * sizeof(int)));
  if (s->kv16) {
    HIP_TRY(hipMalloc(&s->pk, rows * d * 4));
    HIP_TRY(hipMalloc(&s->pv, rows * d * 4));
  }
  s->prows = rows;
  return AKH_OK;
}

// AkashaError::NoCache if a sequence's cache was taken (inference.rs:72, 180).
akh_status need_caches(const akh_session* s) {
  if (!s->kv) return fail(AKH_E_HIP, "session has no KV cache allocation");
  for (uint32_t b = 0; b < s->B; ++b)
    if (!s->has_cache[b])
      return fail(AKH_E_NO_CACHE, "sequence " + std::to_string(b) + " has no cache");
  return AKH_OK;
}

akh_status upload_positions(akh_session* s) {
  std::vector<int> p(kMaxBatch, 0);
  for (uint32_t b = 0; b < s->B; ++b) p[b] = (int)s->cur_len[b];
  HIP_TRY(hipMemcpyAsync(s->pos, p.data(), kMaxBatch * sizeof(int),
                         hipMemcpyHostToDevice, s->be->stream));
  HIP_TRY(hipStreamSynchronize(s->be->stream));
  return AKH_OK;
}

DecGemmParams dec_base(akh_session* s) {
  DecGemmParams p{};
  p.M = (int)s->B;
  p.mt = s->mt;
  return p;
}

void use_packed(DecGemmParams& p, const PackedMatrix& pm) {
  p.w = pm.w;
  p.Kp = pm.rows;
  p.wbf16 = pm.bf16 ? 1 : 0;
  p.wh3 = pm.h3 ? 1 : 0;
}

RowsNormParams norm_base(akh_session* s, const float* gain) {
  RowsNormParams r{};
  r.xt = s->xt;
  r.xnt = s->xnt;
  r.gain = gain;
  r.eps = s->m->cfg.norm_eps;
  r.d = (int)s->m->cfg.dim;
  r.rows = (int)s->rows();
  return r;
}

// A GEMM whose A operand is the RMSNorm of the residual with `gain`: the
// normed rows xnt, or with the fused norm the residual and its sums of
// squares (layer 0's qkv_proj reads the embedding kernel's xnt).
void norm_operand(akh_session* s, DecGemmParams& p, const float* gain, bool fused) {
  if (!fused) {
    p.xt = s->xnt;
    return;
  }
  p.xt = s->xt;
  p.ssq = s->ssq;
  p.gain = gain;
  p.eps = s->m->cfg.norm_eps;
}

// The residual-add epilogue of out_proj and ffn_down when the norm is fused.
void resid_epilogue(akh_session* s, DecGemmParams& p, bool fused) {
  if (!fused) return;
  p.res = s->xt;
  p.ssq_out = s->ssq;
  p.count = s->rcount;
}

// qkv_proj on the normalised residual (inference_graphs.rs:363-384):
// partial tiles, summed by the attention kernel.
hipError_t enqueue_qkv(akh_session* s, uint32_t l) {
  const akh_model_config& c = s->m->cfg;
  DecGemmParams p = dec_base(s);
  norm_operand(s, p, s->m->layer(l, W_NORM1), s->fuse_down && l > 0);
  use_packed(p, s->m->packed_layer(l, W_QKV));
  p.y = s->p_qkv;
  p.N = 3 * c.dim;
  p.K = c.dim;
  return launch_dec_gemm(p, DEC_CFG_QKV, s->be->stream);
}

// q/k/v split + RoPE + cache append + cached attention
// (inference_graphs.rs:385-456): one kernel.
hipError_t enqueue_attn(akh_session* s, uint32_t l, hipEvent_t t0 = nullptr,
                        hipEvent_t t1 = nullptr) {
  const akh_model_config& c = s->m->cfg;
  DecAttnParams p{};
  p.qkv = s->p_qkv;
  p.nparts = s->ks_qkv;
  p.rope = s->rope;
  p.kc = s->kv_at(l, 0);
  p.vc = s->kv_at(l, 1);
  p.kv16 = s->kv16 ? 1 : 0;
  p.out_t = s->attn_t;
  p.ml = s->attn_ml;
  p.active = s->active;
  p.pos = s->pos;
  p.seq_stride = s->seq_stride();
  p.H = (int)c.num_heads;
  p.d = (int)c.dim;
  const uint32_t hd = c.dim / c.num_heads;
  p.scale = 1.0f / sqrtf((float)hd);
  p.rows = (int)s->rows();
  return launch_dec_attn(p, (int)s->B, (int)hd, s->be->stream, t0, t1);
}

// out_proj (inference_graphs.rs:458-470): partial tiles, or with the fused
// norm the residual add (inference_graphs.rs:471) as well.
hipError_t enqueue_out(akh_session* s, uint32_t l) {
  const akh_model_config& c = s->m->cfg;
  DecGemmParams p = dec_base(s);
  p.xt = s->attn_t;
  p.nparts = dec_attn_splits((int)s->B, (int)c.num_heads, (long)s->max_ctx, s->kv16);
  p.ml = s->attn_ml;
  p.hd = (int)(c.dim / c.num_heads);
  use_packed(p, s->m->packed_layer(l, W_OUT));
  p.y = s->p_out;
  p.N = c.dim;
  p.K = c.dim;
  resid_epilogue(s, p, s->fuse_out);
  return launch_dec_gemm(p, DEC_CFG_OUT, s->be->stream);
}

// Residual add of a GEMM's partial tiles + the next RMSNorm (unfused norm).
hipError_t enqueue_resid_norm(akh_session* s, const float* parts, int nparts,
                              const float* gain) {
  RowsNormParams r = norm_base(s, gain);
  r.parts = parts;
  r.nparts = nparts;
  return launch_rows_norm(r, (int)s->B, s->be->stream);
}

// The RMSNorm of the residual rows alone, from the sums of squares the
// fused epilogue wrote (the final norm before lm_head).
hipError_t enqueue_norm_only(akh_session* s, const float* gain) {
  RowsNormParams r = norm_base(s, gain);
  r.ssq = s->ssq;
  return launch_rows_norm(r, (int)s->B, s->be->stream);
}

// ffn_up on norm_2 of the residual (inference_graphs.rs:472-493).
hipError_t enqueue_up(akh_session* s, uint32_t l) {
  const akh_model_config& c = s->m->cfg;
  DecGemmParams p = dec_base(s);
  norm_operand(s, p, s->m->layer(l, W_NORM2), s->fuse_out);
  use_packed(p, s->m->packed_layer(l, W_UP));
  p.y = s->p_up;
  p.N = c.ffn_hidden;
  p.K = c.dim;
  return launch_dec_gemm(p, DEC_CFG_UP, s->be->stream);
}

// SiLU + ffn_down (inference_graphs.rs:495-508): partial tiles.  The
// SiLU of the summed ffn_up partials is computed while down loads its A
// operand, once per column tile of down; where that re-reads the partials
// too often (config 5: 64 tiles x 4 splits, 268 MB of L2 reads per call)
// one small kernel computes it first.
hipError_t enqueue_down(akh_session* s, uint32_t l) {
  const akh_model_config& c = s->m->cfg;
  DecGemmParams p = dec_base(s);
  if (s->ks_up == 1) {
    p.xt = s->p_up;  // ffn_up applied SiLU to its whole sums
  } else if (s->up_act) {
    hipError_t e = launch_silu_sum(s->p_up, s->ks_up, s->up_act, s->rows() * c.ffn_hidden,
                                   s->be->stream);
    if (e != hipSuccess) return e;
    p.xt = s->up_act;
  } else {
    p.xt = s->p_up;
    p.nparts = s->ks_up;
  }
  use_packed(p, s->m->packed_layer(l, W_DOWN));
  p.y = s->p_down;
  p.N = c.dim;
  p.K = c.ffn_hidden;
  resid_epilogue(s, p, s->fuse_down);
  return launch_dec_gemm(p, DEC_CFG_DOWN, s->be->stream);
}

// lm_head on the final-normed residual + per-tile argmax (inference.rs:
// 228-252).
hipError_t enqueue_lm_head(akh_session* s) {
  const akh_model_config& c = s->m->cfg;
  DecGemmParams p = dec_base(s);
  p.xt = s->xnt;
  use_packed(p, s->m->packed_lm_head());
  p.y = s->logits;
  p.amax = s->amax;
  p.N = c.vocab_size;
  p.K = c.dim;
  return launch_dec_lm(p, s->be->num_cus, s->be->stream);
}

// One decode step of build_decode_layer (inference_graphs.rs:339-509) for
// every sequence: embedding + norm_1, then per layer qkv GEMM, attention,
// out GEMM, residual + norm_2, up GEMM, down GEMM, residual + next norm;
// lm_head, greedy argmax + position advance.  Reads tok/pos from the
// device, so it can be replayed step after step with no host work.
hipError_t enqueue_decode_generic(akh_session* s);

hipError_t enqueue_decode_body(akh_session* s) {
  if (s->generic) return enqueue_decode_generic(s);
  const akh_model_config& c = s->m->cfg;
  hipStream_t st = s->be->stream;
  RowsNormParams emb = norm_base(s, s->m->layer(0, W_NORM1));
  emb.table = s->m->embedding();
  emb.ids = s->tok;
  emb.vocab = c.vocab_size;
  hipError_t e = launch_rows_norm(emb, (int)s->B, st);
  for (uint32_t l = 0; l < c.num_layers && e == hipSuccess; ++l) {
    const float* next_gain =
        l + 1 < c.num_layers ? s->m->layer(l + 1, W_NORM1) : s->m->final_norm();
    e = enqueue_qkv(s, l);
    if (e == hipSuccess) e = enqueue_attn(s, l);
    if (e == hipSuccess) e = enqueue_out(s, l);
    if (e == hipSuccess && !s->fuse_out)
      e = enqueue_resid_norm(s, s->p_out, s->ks_out, s->m->layer(l, W_NORM2));
    if (e == hipSuccess) e = enqueue_up(s, l);
    if (e == hipSuccess) e = enqueue_down(s, l);
    if (e == hipSuccess && !s->fuse_down)
      e = enqueue_resid_norm(s, s->p_down, s->ks_down, next_gain);
  }
  // Fused: the last ffn_down left the residual and its sums of squares.
  if (e == hipSuccess && s->fuse_down) e = enqueue_norm_only(s, s->m->final_norm());
  if (e == hipSuccess) e = enqueue_lm_head(s);
  return e;
}

// A GEMM of the generic step: y (epi) a[B, K] w[K, N], on the fp32-MFMA
// prefill GEMM (any M, N, K).
hipError_t gen_gemm(akh_session* s, const float* a, const float* w, float* y, uint32_t N,
                    uint32_t K, int epi) {
  GemmParams g{};
  g.a = a;
  g.b = w;
  g.c = y;
  g.M = (int)s->B;
  g.N = (int)N;
  g.K = (int)K;
  return launch_gemm(g, epi, s->be->stream);
}

// The final RMSNorm of the rows in gx, the lm_head and each row's first-max
// partial (the generic step's and the generic prefill's tail).
hipError_t gen_lm_tail(akh_session* s) {
  const akh_model_config& c = s->m->cfg;
  hipStream_t st = s->be->stream;
  hipError_t e = launch_rows_rmsnorm(s->gx, s->m->final_norm(), s->gxn, (int)s->B,
                                     (int)c.dim, c.norm_eps, st);
  if (e == hipSuccess)
    e = gen_gemm(s, s->gxn, s->m->lm_head(), s->logits, c.vocab_size, c.dim, GEMM_STORE);
  if (e == hipSuccess)
    e = launch_gen_argmax_part(s->logits, (int)s->B, (int)c.vocab_size, s->amax, st);
  return e;
}

// build_decode_layer's step (inference_graphs.rs:339-509) on the generic
// kernels, every sequence at its own position (pos on the device).
hipError_t enqueue_decode_generic(akh_session* s) {
  const akh_model_config& c = s->m->cfg;
  hipStream_t st = s->be->stream;
  const int B = (int)s->B, d = (int)c.dim;
  const uint32_t hd = c.dim / c.num_heads;
  hipError_t e = launch_embedding_rows(s->tok, s->m->embedding(), s->gx, B, d, c.vocab_size, st);
  if (e == hipSuccess)
    e = launch_rows_rmsnorm(s->gx, s->m->layer(0, W_NORM1), s->gxn, B, d, c.norm_eps, st);
  for (uint32_t l = 0; l < c.num_layers && e == hipSuccess; ++l) {
    e = gen_gemm(s, s->gxn, s->m->layer(l, W_QKV), s->gqkv, 3 * c.dim, c.dim, GEMM_STORE);
    if (e == hipSuccess) {
      GenAttnParams a{};
      a.qkv = s->gqkv;
      a.rope = s->rope;
      a.kc = s->kv_at(l, 0);
      a.vc = s->kv_at(l, 1);
      a.seq_stride = s->seq_stride();
      a.pos = s->pos;
      a.active = s->active;
      a.out = s->gattn;
      a.d = d;
      a.hd = (int)hd;
      a.scale = 1.0f / sqrtf((float)hd);
      a.kv16 = s->kv16 ? 1 : 0;
      e = launch_gen_attn(a, B, st);
    }
    if (e == hipSuccess)
      e = gen_gemm(s, s->gattn, s->m->layer(l, W_OUT), s->gx, c.dim, c.dim, GEMM_ADD);
    if (e == hipSuccess)
      e = launch_rows_rmsnorm(s->gx, s->m->layer(l, W_NORM2), s->gxn, B, d, c.norm_eps, st);
    if (e == hipSuccess)
      e = gen_gemm(s, s->gxn, s->m->layer(l, W_UP), s->gffn, c.ffn_hidden, c.dim, GEMM_SILU);
    if (e == hipSuccess)
      e = gen_gemm(s, s->gffn, s->m->layer(l, W_DOWN), s->gx, c.dim, c.ffn_hidden, GEMM_ADD);
    if (e == hipSuccess && l + 1 < c.num_layers)
      e = launch_rows_rmsnorm(s->gx, s->m->layer(l + 1, W_NORM1), s->gxn, B, d, c.norm_eps, st);
  }
  if (e == hipSuccess) e = gen_lm_tail(s);
  return e;
}

hipError_t enqueue_decode(akh_session* s) {
  hipError_t e = enqueue_decode_body(s);
  if (e == hipSuccess)
    e = launch_argmax_final(s->amax, argmax_parts(s), (int)s->B, s->tok, s->pos, s->hist,
                            (int)s->max_ctx + 1, 0, s->be->stream, nullptr, s->logits,
                            (long)s->m->cfg.vocab_size);
  return e;
}

// One round of InferenceSession::generate (inference.rs:303-323) for every
// sequence: sample_token on the current logits over the sequence's history,
// record the token (stopping at eos or a full context), then decode the
// sampled tokens of the rows still going and advance their positions.
hipError_t enqueue_generate_round(akh_session* s) {
  const akh_model_config& c = s->m->cfg;
  SampleArgs a{};
  a.logits = s->logits;
  a.n = (int)c.vocab_size;
  a.row_stride = c.vocab_size;
  a.temperature = s->gparams.temperature;
  a.top_k = (int)std::min<uint32_t>(s->gparams.top_k, 0x7FFFFFFFu);
  a.top_p = s->gparams.top_p;
  a.penalty = s->gparams.repetition_penalty;
  a.uniform = s->gparams.temperature > 0.0f ? s->guni : nullptr;
  a.wbuf = s->gwbuf;
  a.cnt = s->be->sample_cnt;
  a.tok = s->tok;
  a.pos = s->pos;
  a.hist = s->hist;
  a.hist_stride = (long)s->max_ctx + 1;
  a.start = s->gstart;
  a.active = s->active;
  a.done = s->done;
  a.count = s->gcount;
  a.gen = s->ggen;
  a.max_new = (int)s->gmax_new;
  a.max_ctx = (int)s->max_ctx;
  a.eos = c.eos_token;
  hipError_t e = launch_sample_rows(a, (int)s->B, s->be->stream);
  if (e == hipSuccess) e = enqueue_decode_body(s);
  if (e == hipSuccess) e = launch_advance(s->pos, s->active, (int)s->B, s->be->stream);
  return e;
}

akh_status capture(akh_session* s, hipError_t (*enqueue)(akh_session*), hipGraph_t* graph,
                   hipGraphExec_t* exec, const char* what) {
  hipStream_t st = s->be->stream;
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  hipError_t e = enqueue(s);
  hipGraph_t g = nullptr;
  hipError_t e2 = hipStreamEndCapture(st, &g);
  if (e != hipSuccess || e2 != hipSuccess) {
    if (g) hipGraphDestroy(g);
    return fail(AKH_E_HIP, std::string(what) + " capture: " +
                               hipGetErrorString(e != hipSuccess ? e : e2));
  }
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g);
    return fail(AKH_E_HIP, std::string(what) + " instantiate: " + hipGetErrorString(e));
  }
  *graph = g;
  *exec = ex;
  return AKH_OK;
}

akh_status set_active(akh_session* s, bool all_rows) {
  std::vector<int> v(kMaxBatch, 0);
  for (uint32_t b = 0; b < s->B; ++b) v[b] = all_rows ? 1 : 0;
  HIP_TRY(hipMemcpyAsync(s->active, v.data(), kMaxBatch * sizeof(int), hipMemcpyHostToDevice,
                         s->be->stream));
  HIP_TRY(hipStreamSynchronize(s->be->stream));
  return AKH_OK;
}

void drop_graphs(akh_session* s) {
  for (hipGraphExec_t* e : {&s->gexec, &s->gexec_n, &s->ggexec})
    if (*e) {
      hipGraphExecDestroy(*e);
      *e = nullptr;
    }
  for (hipGraph_t* g : {&s->graph, &s->graph_n, &s->ggraph})
    if (*g) {
      hipGraphDestroy(*g);
      *g = nullptr;
    }
}

// Captured graphs hold the kernels chosen for the packed weights' element
// types: drop them when an upload changed one.
void drop_stale_graphs(akh_session* s) {
  if (s->glayout == s->m->layout_gen) return;
  drop_graphs(s);
  s->glayout = s->m->layout_gen;
}

#ifndef AKH_STEPS_PER_GRAPH
#define AKH_STEPS_PER_GRAPH 8
#endif
constexpr uint32_t kStepsPerGraph = AKH_STEPS_PER_GRAPH;

hipError_t enqueue_decode_n(akh_session* s) {
  for (uint32_t i = 0; i < kStepsPerGraph; ++i) {
    const hipError_t e = enqueue_decode(s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// The one-step decode graph and, when steps are batched, the
// kStepsPerGraph-step one (positions and tokens live on the device, so
// consecutive steps replay without the host).
akh_status ensure_decode_graph(akh_session* s) {
  drop_stale_graphs(s);
  if (!s->gexec) {
    akh_status st = capture(s, enqueue_decode, &s->graph, &s->gexec, "decode graph");
    if (st != AKH_OK) return st;
  }
  if (kStepsPerGraph > 1 && !s->gexec_n)
    return capture(s, enqueue_decode_n, &s->graph_n, &s->gexec_n, "decode graph");
  return AKH_OK;
}

akh_status download_outputs(akh_session* s, float* logits, uint32_t* next) {
  const akh_model_config& c = s->m->cfg;
  hipStream_t st = s->be->stream;
  if (logits)
    HIP_TRY(hipMemcpyAsync(logits, s->logits,
                           (size_t)s->B * c.vocab_size * sizeof(float),
                           hipMemcpyDeviceToHost, st));
  if (next)
    HIP_TRY(hipMemcpyAsync(next, s->tok, (size_t)s->B * sizeof(uint32_t),
                           hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return AKH_OK;
}

}  // namespace

extern "C" void akh_session_free(akh_session* s) {
  if (!s) return;
  hipSetDevice(s->be->device);
  hipStreamSynchronize(s->be->stream);
  drop_graphs(s);
  free_prefill(s);
  void* bufs[] = {s->kv,     s->rope,   s->xt,     s->xnt,    s->attn_t, s->attn_ml,
                  s->p_qkv,  s->p_out,  s->p_up,   s->up_act, s->p_down,
                  s->logits, s->amax,   s->ssq,    s->rcount,
                  s->tok,    s->pos,    s->hist,   s->active, s->done,   s->gstart,
                  s->gcount, s->ggen,   s->guni,   s->gwbuf,  s->gx,     s->gxn,
                  s->gqkv,   s->gattn,  s->gffn};
  for (void* p : bufs)
    if (p) hipFree(p);
  delete s;
}

namespace {

#ifndef AKH_SILU_KERNEL_READS
#define AKH_SILU_KERNEL_READS 128
#endif
// Whether down's SiLU runs as its own kernel: when down's column tiles
// times ffn_up's splits (partial re-reads per element) reach
// AKH_SILU_KERNEL_READS.
bool silu_own_kernel(const akh_session* s) {
  const akh_model_config& c = s->m->cfg;
  return s->ks_up > 1 && (long)(c.dim / 32) * s->ks_up >= AKH_SILU_KERNEL_READS;
}

// A session's buffers.  With decode false only what prefill needs (KV
// cache, RoPE table) is allocated, and the decode kernels' shape limits do
// not apply: the trainer's forward uses such a session.
akh_status session_create(akh_model* m, uint32_t max_context_len, uint32_t batch, bool decode,
                          akh_session** out) {
  CHECK_ARG(m && out, "akh_session_new: NULL argument");
  *out = nullptr;
  const akh_model_config& c = m->cfg;
  CHECK_ARG(batch >= 1 && (!decode || batch <= (uint32_t)kMaxBatch),
            "akh_session_new: batch must be in 1..64");
  CHECK_ARG(max_context_len >= 1, "akh_session_new: max_context_len is 0");
  const uint32_t hd = c.dim / c.num_heads;
  // RoPE rotates pairs inside a head (cpu.rs:84-109): an even head size, at
  // most 128 (FLASH_ATTENTION's limit, emit.rs:564-567).
  CHECK_ARG(supported_head_dim(hd) && hd % 2 == 0,
            "akh_session_new: head_dim must be even and at most 128");

  akh_session* s = new akh_session();
  // Shapes outside the batched decode kernels decode on the generic ones.
  s->generic = decode && !dec_fast_shape(c.dim, hd, c.ffn_hidden);
  s->m = m;
  s->be = m->be;
  s->max_ctx = max_context_len;
  s->B = batch;
  s->cur_len.assign(batch, 0);
  s->has_cache.assign(batch, 1);
  if (!s->generic) {
    s->ks_qkv = dec_gemm_splits(DEC_CFG_QKV, c.dim, 3 * c.dim);
    s->ks_out = dec_gemm_splits(DEC_CFG_OUT, c.dim, c.dim);
    s->ks_up = dec_gemm_splits(DEC_CFG_UP, c.dim, c.ffn_hidden);
    s->ks_down = dec_gemm_splits(DEC_CFG_DOWN, c.ffn_hidden, c.dim);
  }

  s->mt = batch > 32 ? 2 : 1;
  // Activation and partial tiles hold R rows; the per-row step state holds
  // kMaxBatch entries (it is uploaded and downloaded whole).
  const size_t d = c.dim, V = c.vocab_size, F = c.ffn_hidden, R = s->rows(), RB = kMaxBatch;
  hipError_t e = hipSetDevice(s->be->device);
  auto alloc = [&](void** p, size_t bytes) {
    if (e == hipSuccess) e = hipMalloc(p, bytes);
    if (e == hipSuccess) e = hipMemset(*p, 0, bytes);
  };
  alloc((void**)&s->kv, (size_t)c.num_layers * 2 * batch * max_context_len * d * 4);
  alloc((void**)&s->rope, (size_t)max_context_len * (hd / 2) * sizeof(float2));
  if (decode && s->generic) {
    const size_t Bs = batch;
    alloc((void**)&s->gx, Bs * d * 4);
    alloc((void**)&s->gxn, Bs * d * 4);
    alloc((void**)&s->gqkv, Bs * 3 * d * 4);
    alloc((void**)&s->gattn, Bs * d * 4);
    alloc((void**)&s->gffn, Bs * F * 4);
  }
  if (decode && !s->generic) {
  alloc((void**)&s->xt, R * d * 4);
  alloc((void**)&s->xnt, R * d * 4);
  alloc((void**)&s->attn_t, (size_t)dec_attn_max_splits() * R * d * 4);
  alloc((void**)&s->attn_ml, (size_t)dec_attn_max_splits() * c.num_heads * R * sizeof(float2));
  alloc((void**)&s->p_qkv, (size_t)s->ks_qkv * R * 3 * d * 4);
  alloc((void**)&s->p_out, (size_t)s->ks_out * R * d * 4);
  alloc((void**)&s->p_up, (size_t)s->ks_up * R * F * 4);
  if (silu_own_kernel(s)) alloc((void**)&s->up_act, R * F * 4);
  alloc((void**)&s->p_down, (size_t)s->ks_down * R * d * 4);
  if (dec_norm_fusable((int)d)) {  // for akh_session_set_fused_norm
    alloc((void**)&s->ssq, R * (d / 32) * 4);
    alloc((void**)&s->rcount, (d / 32) * sizeof(int));  // zeroed by alloc
  }
  }
  if (decode) {
  alloc((void**)&s->logits, R * V * 4);
  alloc((void**)&s->amax, R * (size_t)(s->generic ? 1 : lm_parts_max(s)) * sizeof(uint2));
  alloc((void**)&s->tok, RB * 4);
  alloc((void**)&s->pos, RB * 4);
  alloc((void**)&s->hist, (size_t)batch * (max_context_len + 1) * 4);
  alloc((void**)&s->active, RB * sizeof(int));
  alloc((void**)&s->done, RB * sizeof(int));
  alloc((void**)&s->gstart, RB * sizeof(int));
  alloc((void**)&s->gcount, RB * sizeof(uint32_t));
  alloc((void**)&s->gwbuf, sample_scratch_bytes((int)batch, (int)V));
  }
  if (e == hipSuccess) {
    // RoPE table in f32 exactly as src/shaders/cpu.rs:98-100 forms it:
    // freq = 1 / 10000^(2i / head_dim), angle = pos * freq, then sin/cos.
    std::vector<float2> tab((size_t)max_context_len * (hd / 2));
    for (uint32_t t = 0; t < max_context_len; ++t)
      for (uint32_t i = 0; i < hd / 2; ++i) {
        const float freq = 1.0f / powf(10000.0f, (float)(2 * i) / (float)hd);
        const float angle = (float)t * freq;
        tab[(size_t)t * (hd / 2) + i] = make_float2(cosf(angle), sinf(angle));
      }
    e = hipMemcpy(s->rope, tab.data(), tab.size() * sizeof(float2),
                  hipMemcpyHostToDevice);
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    akh_session_free(s);
    return fail(AKH_E_HIP, std::string("akh_session_new: ") + hipGetErrorString(e));
  }
  akh_status st = decode ? set_active(s, true) : AKH_OK;
  if (st != AKH_OK) {
    akh_session_free(s);
    return st;
  }
  *out = s;
  return AKH_OK;
}

}  // namespace

extern "C" akh_status akh_session_new(akh_model* m, uint32_t max_context_len,
                                      uint32_t batch, akh_session** out) {
  return session_create(m, max_context_len, batch, true, out);
}

extern "C" akh_status akh_session_reset(akh_session* s) {
  CHECK_ARG(s, "akh_session_reset: NULL session");
  std::fill(s->cur_len.begin(), s->cur_len.end(), 0u);
  return upload_positions(s);
}

extern "C" akh_status akh_session_cur_len(const akh_session* s, uint32_t* out) {
  CHECK_ARG(s && out, "akh_session_cur_len: NULL argument");
  std::copy(s->cur_len.begin(), s->cur_len.end(), out);
  return AKH_OK;
}

extern "C" akh_status akh_session_set_len(akh_session* s, uint32_t len) {
  CHECK_ARG(s && len <= s->max_ctx, "akh_session_set_len: bad argument");
  akh_status nc = need_caches(s);
  if (nc != AKH_OK) return nc;
  std::fill(s->cur_len.begin(), s->cur_len.end(), len);
  return upload_positions(s);
}

extern "C" akh_status akh_session_fill_cache_synthetic(akh_session* s, uint32_t len,
                                                       uint64_t seed) {
  CHECK_ARG(s && len <= s->max_ctx, "akh_session_fill_cache_synthetic: bad argument");
  CHECK_ARG(!s->be->capturing, "akh_session_fill_cache_synthetic: graph capture in progress");
  akh_status nc = need_caches(s);
  if (nc != AKH_OK) return nc;
  HIP_TRY(hipSetDevice(s->be->device));
  const akh_model_config& c = s->m->cfg;
  HIP_TRY(launch_fill_kv_synthetic(s->kv, s->kv16, (size_t)c.num_layers * 2 * s->B, (int)len,
                                   (int)c.dim, (long)s->max_ctx, seed, s->be->stream));
  std::fill(s->cur_len.begin(), s->cur_len.end(), len);
  return upload_positions(s);
}

extern "C" akh_status akh_session_truncate(akh_session* s, uint32_t len) {
  CHECK_ARG(s, "akh_session_truncate: NULL session");
  for (uint32_t b = 0; b < s->B; ++b)
    CHECK_ARG(len <= s->cur_len[b], "akh_session_truncate: len > cur_len");
  // The next step feeds the token that occupied position `len`.
  HIP_TRY(hipMemcpy2DAsync(s->tok, sizeof(uint32_t), s->hist + len,
                           (size_t)(s->max_ctx + 1) * sizeof(uint32_t),
                           sizeof(uint32_t), s->B, hipMemcpyDeviceToDevice,
                           s->be->stream));
  std::fill(s->cur_len.begin(), s->cur_len.end(), len);
  return upload_positions(s);
}

namespace {

// A prefill GEMM on parameter `index`: the model's split kernel on its copy
// of the matrix, or the fp32-MFMA kernel (no copy, or `exact`).
hipError_t prefill_gemm(const akh_model* m, GemmParams& g, uint32_t index, int epi,
                        hipStream_t st, bool exact) {
  if (!exact && index < m->wsplit.size() && m->wsplit[index]) {
    if (m->prefill_split == AKH_SPLIT_X6) {
      g.bt = static_cast<const float*>(m->wsplit[index]);
      return launch_gemm_x6(g, epi, st);
    }
    g.bp16 = static_cast<const uint16_t*>(m->wsplit[index]);
    g.range_flag = m->range_flag;
    return launch_gemm_h3(g, epi, st);
  }
  return launch_gemm(g, epi, st);
}

// Whether the f32 prefill runs k_gemm_h3, whose range flag then needs a
// check (and, if set, an exact rerun).
bool h3_prefill(const akh_model* m) {
  return m->prefill_split == AKH_SPLIT_H3 && !m->prefill_bf16;
}

hipError_t clear_range_flag(const akh_model* m, hipStream_t st) {
  return hipMemsetAsync(m->range_flag, 0, sizeof(int), st);
}

// Waits for the stream and reads the range flag.
hipError_t range_flag_set(const akh_model* m, hipStream_t st, bool* set) {
  int v = 0;
  hipError_t e = hipMemcpyAsync(&v, m->range_flag, sizeof(int), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  *set = v != 0;
  return e;
}

// The rows of one prefill.  Uniform prompts of length S keep the layout
// row = b * S + t and need no tables; ragged prompts are packed back to back
// with the session's tables (p_at, p_map) on the device.
struct PrefillRows {
  size_t rows = 0;
  uint32_t S = 0;  // the longest prompt
  bool ragged = false;
};

// The prefill layers in fp32 (build_prefill_layer's node order); `exact`
// runs them on the fp32-MFMA kernels whatever the model's split kernels.
hipError_t prefill_layers_f32(akh_session* s, const PrefillRows& pr, bool exact) {
  const akh_model_config& c = s->m->cfg;
  const uint32_t d = c.dim, hd = d / c.num_heads, S = pr.S;
  const size_t rows = pr.rows;
  hipStream_t st = s->be->stream;
#define TRY_HIP(x)                      \
  do {                                  \
    const hipError_t e_ = (x);          \
    if (e_ != hipSuccess) return e_;    \
  } while (0)
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    TRY_HIP(launch_rows_rmsnorm(s->px, s->m->layer(l, W_NORM1), s->pxn,
                                (int)rows, (int)d, c.norm_eps, st));
    GemmParams g{};
    g.a = s->pxn;
    g.b = s->m->layer(l, W_QKV);
    g.M = (int)rows;
    g.N = 3 * d;
    g.K = d;
    g.q_out = s->pq;
    // With a bfloat16 cache, K and V go to fp32 rows (packed like the
    // prompt's) for this prompt's attention and are stored into the cache
    // after it.
    g.kcache = s->kv16 ? s->pk : s->kcache(l);
    g.vcache = s->kv16 ? s->pv : s->vcache(l);
    g.kv_packed = s->kv16 ? 1 : 0;
    g.seq_stride = s->seq_stride();
    g.S = (int)S;
    g.rowmap = pr.ragged ? s->p_map : nullptr;
    g.rope = s->rope;
    g.dim = d;
    g.head_dim = hd;
    const uint32_t base = 1 + 6 * l;
    TRY_HIP(prefill_gemm(s->m, g, base + W_QKV, GEMM_QKV, st, exact));
    if (s->kv16)
      TRY_HIP(launch_kv_store_bf16(s->pk, s->pv, static_cast<uint16_t*>(s->kv_at(l, 0)),
                                   static_cast<uint16_t*>(s->kv_at(l, 1)), rows, (int)S,
                                   (int)d, s->seq_stride(), g.rowmap, st));

    FlashParams f{};
    f.q = s->pq;
    f.k = g.kcache;
    f.v = g.vcache;
    f.o = s->pattn;
    f.q_bs = (long)S * d;
    f.kv_bs = s->kv16 ? (long)S * d : s->seq_stride();
    f.o_bs = (long)S * d;
    f.rows_at = pr.ragged ? s->p_at : nullptr;
    f.kv_packed = s->kv16 ? 1 : 0;
    f.S = (int)S;
    f.d = (int)d;
    f.hd = (int)hd;
    f.scale = 1.0f / sqrtf((float)hd);
    f.x6 = exact || s->m->prefill_split == AKH_SPLIT_NONE ? 0
           : s->m->prefill_split == AKH_SPLIT_H3          ? FLASH_H3
                                                          : FLASH_X6;
    f.range_flag = s->m->range_flag;
    TRY_HIP(launch_flash(f, (int)s->B, (int)S, st));

    GemmParams o{};
    o.a = s->pattn;
    o.b = s->m->layer(l, W_OUT);
    o.c = s->px;
    o.M = (int)rows;
    o.N = d;
    o.K = d;
    TRY_HIP(prefill_gemm(s->m, o, base + W_OUT, GEMM_ADD, st, exact));

    TRY_HIP(launch_rows_rmsnorm(s->px, s->m->layer(l, W_NORM2), s->pxn,
                                (int)rows, (int)d, c.norm_eps, st));
    GemmParams u{};
    u.a = s->pxn;
    u.b = s->m->layer(l, W_UP);
    u.c = s->pffn;
    u.M = (int)rows;
    u.N = c.ffn_hidden;
    u.K = d;
    TRY_HIP(prefill_gemm(s->m, u, base + W_UP, GEMM_SILU, st, exact));

    GemmParams w{};
    w.a = s->pffn;
    w.b = s->m->layer(l, W_DOWN);
    w.c = s->px;
    w.M = (int)rows;
    w.N = d;
    w.K = c.ffn_hidden;
    TRY_HIP(prefill_gemm(s->m, w, base + W_DOWN, GEMM_ADD, st, exact));
  }
#undef TRY_HIP
  return hipSuccess;
}

// The prefill layers on the bfloat16 MFMAs (akh_model_set_prefill_bf16),
// in build_prefill_layer's node order.  Weights come from the model's
// transposed bfloat16 copies.  The QKV, ffn_up and ffn_down GEMMs take their
// fp32 A operand (normed rows, SiLU output) as bfloat16 hi + lo parts, two
// MFMAs per product: with bfloat16 weights those GEMMs are then accurate to
// about 2^-16.  Flash attention runs on bfloat16 Q, K, V and P and writes
// a bfloat16 output, which out_proj takes as is.  The residual stream px
// and the KV cache stay fp32.
hipError_t prefill_layers_bf16(akh_session* s, const PrefillRows& pr) {
  const akh_model_config& c = s->m->cfg;
  const uint32_t d = c.dim, hd = d / c.num_heads, S = pr.S;
  const size_t rows = pr.rows;
  hipStream_t st = s->be->stream;
  uint16_t* attn16 = reinterpret_cast<uint16_t*>(s->pattn);
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    const uint32_t base = 1 + 6 * l;
    hipError_t e = launch_rows_rmsnorm(s->px, s->m->layer(l, W_NORM1), s->pxn, (int)rows,
                                       (int)d, c.norm_eps, st);
    if (e != hipSuccess) return e;
    GemmParams g{};
    g.a = s->pxn;
    g.bt16 = s->m->wt16[base + W_QKV];
    g.M = (int)rows;
    g.N = 3 * d;
    g.K = d;
    g.q_out = s->pq;
    // With a bfloat16 cache, K and V go to fp32 rows (packed like the
    // prompt's) for this prompt's attention and are stored into the cache
    // after it.
    g.kcache = s->kv16 ? s->pk : s->kcache(l);
    g.vcache = s->kv16 ? s->pv : s->vcache(l);
    g.kv_packed = s->kv16 ? 1 : 0;
    g.seq_stride = s->seq_stride();
    g.S = (int)S;
    g.rowmap = pr.ragged ? s->p_map : nullptr;
    g.rope = s->rope;
    g.dim = d;
    g.head_dim = hd;
    // QKV rounds its input rows to bfloat16 (one product); ffn_up and
    // ffn_down keep the hi + lo split, which holds most of the accuracy
    // (config 5's logits 0.0139 from the f32 oracle against 0.0212 with
    // every input rounded, the bar being 2e-2).
    g.a_hi_only = 1;
    if ((e = launch_gemm_bf16(g, GEMM_QKV, st)) != hipSuccess) return e;
    if (s->kv16 &&
        (e = launch_kv_store_bf16(s->pk, s->pv, static_cast<uint16_t*>(s->kv_at(l, 0)),
                                  static_cast<uint16_t*>(s->kv_at(l, 1)), rows, (int)S,
                                  (int)d, s->seq_stride(), g.rowmap, st)) != hipSuccess)
      return e;

    FlashParams f{};
    f.q = s->pq;
    f.k = g.kcache;
    f.v = g.vcache;
    f.o16 = attn16;
    f.q_bs = (long)S * d;
    f.kv_bs = s->kv16 ? (long)S * d : s->seq_stride();
    f.o_bs = (long)S * d;
    f.rows_at = pr.ragged ? s->p_at : nullptr;
    f.kv_packed = s->kv16 ? 1 : 0;
    f.S = (int)S;
    f.d = (int)d;
    f.hd = (int)hd;
    f.scale = 1.0f / sqrtf((float)hd);
    if ((e = launch_flash_bf16(f, (int)s->B, (int)S, st)) != hipSuccess) return e;

    GemmParams o{};
    o.a16 = attn16;
    o.bt16 = s->m->wt16[base + W_OUT];
    o.c = s->px;
    o.M = (int)rows;
    o.N = d;
    o.K = d;
    if ((e = launch_gemm_bf16(o, GEMM_ADD, st)) != hipSuccess) return e;

    if ((e = launch_rows_rmsnorm(s->px, s->m->layer(l, W_NORM2), s->pxn, (int)rows, (int)d,
                                 c.norm_eps, st)) != hipSuccess)
      return e;
    GemmParams u{};
    u.a = s->pxn;
    u.bt16 = s->m->wt16[base + W_UP];
    u.c = s->pffn;
    u.M = (int)rows;
    u.N = c.ffn_hidden;
    u.K = d;
    if ((e = launch_gemm_bf16(u, GEMM_SILU, st)) != hipSuccess) return e;

    GemmParams w{};
    w.a = s->pffn;
    w.bt16 = s->m->wt16[base + W_DOWN];
    w.c = s->px;
    w.M = (int)rows;
    w.N = d;
    w.K = c.ffn_hidden;
    if ((e = launch_gemm_bf16(w, GEMM_ADD, st)) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

// InferenceSession::prefill (inference.rs:61-176) for all sequences, with
// build_prefill_layer's node order (inference_graphs.rs:198-337): 7 kernels
// per layer (RMSNorm, QKV GEMM + RoPE + cache append, flash attention,
// out_proj + residual, RMSNorm, ffn_up + SiLU, ffn_down + residual).
namespace {

// InferenceSession::prefill for every sequence, sequence b with lens[b]
// tokens (tokens packed back to back).  The reference checks each prompt
// (inference.rs:61-75): empty, longer than the context, or a cache that is
// not empty fail with its errors before any work.
akh_status prefill_impl(akh_session* s, const uint32_t* tokens, const uint32_t* lens,
                        float* logits, uint32_t* next) {
  uint32_t S = 0;
  size_t rows = 0;
  bool ragged = false;
  for (uint32_t b = 0; b < s->B; ++b) {
    if (lens[b] == 0) return fail(AKH_E_EMPTY_PROMPT, "prompt is empty");
    if (lens[b] > s->max_ctx)
      return fail(AKH_E_PROMPT_TOO_LONG,
                  "prompt is " + std::to_string(lens[b]) +
                      " tokens, context window is " + std::to_string(s->max_ctx));
    S = std::max(S, lens[b]);
    ragged = ragged || lens[b] != lens[0];
    rows += lens[b];
  }
  akh_status nc = need_caches(s);
  if (nc != AKH_OK) return nc;
  for (uint32_t b = 0; b < s->B; ++b)
    if (s->cur_len[b] != 0)
      return fail(AKH_E_CACHE_NOT_EMPTY,
                  "prefill needs an empty cache, this one holds " +
                      std::to_string(s->cur_len[b]) + " tokens");
  const akh_model_config& c = s->m->cfg;
  const uint32_t d = c.dim;
  akh_status st0 = ensure_prefill(s, rows);
  if (st0 != AKH_OK) return st0;
  hipStream_t st = s->be->stream;
  HIP_TRY(hipMemcpyAsync(s->ptok, tokens, rows * 4, hipMemcpyHostToDevice, st));
  // Ragged prompts: the row tables (first row and length per sequence,
  // (sequence, position) per row, last row per sequence).
  std::vector<int> at(s->B + 1, 0), last(s->B), len(s->B);
  for (uint32_t b = 0; b < s->B; ++b) {
    at[b + 1] = at[b] + (int)lens[b];
    last[b] = at[b + 1] - 1;
    len[b] = (int)lens[b];
  }
  if (ragged) {
    std::vector<int2> map(rows);
    for (uint32_t b = 0; b < s->B; ++b)
      for (uint32_t t = 0; t < lens[b]; ++t) map[at[b] + t] = make_int2((int)b, (int)t);
    HIP_TRY(hipMemcpyAsync(s->p_at, at.data(), at.size() * sizeof(int), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->p_map, map.data(), rows * sizeof(int2), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->p_last, last.data(), s->B * sizeof(int), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->p_len, len.data(), s->B * sizeof(int), hipMemcpyHostToDevice, st));
    // The host tables are read by the copies above before they go away.
    HIP_TRY(hipStreamSynchronize(st));
  }
  // Token history: each prompt occupies positions 0..len-1 of its sequence.
  if (ragged) {
    for (uint32_t b = 0; b < s->B; ++b)
      HIP_TRY(hipMemcpyAsync(s->hist + (size_t)b * (s->max_ctx + 1), s->ptok + at[b],
                             (size_t)lens[b] * 4, hipMemcpyDeviceToDevice, st));
  } else {
    HIP_TRY(hipMemcpy2DAsync(s->hist, (size_t)(s->max_ctx + 1) * 4, s->ptok,
                             (size_t)S * 4, (size_t)S * 4, s->B,
                             hipMemcpyDeviceToDevice, st));
  }

  PrefillRows pr;
  pr.rows = rows;
  pr.S = S;
  pr.ragged = ragged;
  const bool h3 = h3_prefill(s->m);
  // Last row of every sequence -> final RMSNorm -> lm_head -> greedy token
  // (inference.rs:120-168).
  auto tail = [&]() -> hipError_t {
    if (s->generic) {
      hipError_t e = launch_gen_gather_rows(s->px, s->gx, (int)s->B, (int)d, (long)S - 1,
                                            (long)S, ragged ? s->p_last : nullptr, st);
      if (e == hipSuccess) e = gen_lm_tail(s);
      if (e == hipSuccess)
        e = launch_argmax_final(s->amax, 1, (int)s->B, s->tok, nullptr, s->hist,
                                (int)s->max_ctx + 1, (int)S, st, ragged ? s->p_len : nullptr,
                                s->logits, (long)c.vocab_size);
      return e;
    }
    RowsNormParams r = norm_base(s, s->m->final_norm());
    r.src = s->px;
    r.row0 = (long)S - 1;
    r.row_stride = (long)S;
    r.src_rows = ragged ? s->p_last : nullptr;
    hipError_t e = launch_rows_norm(r, (int)s->B, st);
    if (e == hipSuccess) e = enqueue_lm_head(s);
    if (e == hipSuccess)
      e = launch_argmax_final(s->amax, lm_parts(s), (int)s->B, s->tok, nullptr, s->hist,
                              (int)s->max_ctx + 1, (int)S, st, ragged ? s->p_len : nullptr,
                              s->logits, (long)c.vocab_size);
    return e;
  };
  if (h3) HIP_TRY(clear_range_flag(s->m, st));
  HIP_TRY(launch_embedding_rows(s->ptok, s->m->embedding(), s->px, (int)rows,
                                (int)d, c.vocab_size, st));
  HIP_TRY(s->m->prefill_bf16 ? prefill_layers_bf16(s, pr) : prefill_layers_f32(s, pr, false));
  // The tail is queued before the range flag is read, so the stream does not
  // wait for the host in the middle of the prefill; the flag is almost never
  // set.
  HIP_TRY(tail());
  bool redo = false;
  if (h3) HIP_TRY(range_flag_set(s->m, st, &redo));
  if (redo) {
    // An operand beyond fp16's range: the same layers on the fp32 kernels
    // (they rewrite every row and cache entry the first pass wrote), then
    // the tail again.
    HIP_TRY(launch_embedding_rows(s->ptok, s->m->embedding(), s->px, (int)rows,
                                  (int)d, c.vocab_size, st));
    HIP_TRY(prefill_layers_f32(s, pr, true));
    HIP_TRY(tail());
  }
  for (uint32_t b = 0; b < s->B; ++b) s->cur_len[b] = lens[b];
  akh_status ps = upload_positions(s);
  if (ps != AKH_OK) return ps;
  return download_outputs(s, logits, next);
}

}  // namespace

extern "C" akh_status akh_session_prefill(akh_session* s,
                                          const uint32_t* tokens,
                                          uint32_t prompt_len, float* logits,
                                          uint32_t* next) {
  CHECK_ARG(s && (tokens || !prompt_len), "akh_session_prefill: NULL argument");
  const std::vector<uint32_t> lens(s->B, prompt_len);
  return prefill_impl(s, tokens, lens.data(), logits, next);
}

extern "C" akh_status akh_session_prefill_ragged(akh_session* s, const uint32_t* tokens,
                                                 const uint32_t* prompt_lens, float* logits,
                                                 uint32_t* next) {
  CHECK_ARG(s && prompt_lens, "akh_session_prefill_ragged: NULL argument");
  size_t n = 0;
  for (uint32_t b = 0; b < s->B; ++b) n += prompt_lens[b];
  CHECK_ARG(tokens || n == 0, "akh_session_prefill_ragged: NULL tokens");
  return prefill_impl(s, tokens, prompt_lens, logits, next);
}

extern "C" akh_status akh_session_decode_step(akh_session* s,
                                              const uint32_t* tokens,
                                              float* logits, uint32_t* next) {
  CHECK_ARG(s, "akh_session_decode_step: NULL session");
  akh_status nc = need_caches(s);
  if (nc != AKH_OK) return nc;
  for (uint32_t b = 0; b < s->B; ++b)
    if (s->cur_len[b] >= s->max_ctx)
      return fail(AKH_E_CONTEXT_FULL, "context window is full (" +
                                          std::to_string(s->max_ctx) +
                                          " tokens)");
  akh_status st0 = ensure_decode_graph(s);
  if (st0 != AKH_OK) return st0;
  hipStream_t st = s->be->stream;
  if (tokens)
    HIP_TRY(hipMemcpyAsync(s->tok, tokens, (size_t)s->B * 4,
                           hipMemcpyHostToDevice, st));
  HIP_TRY(hipGraphLaunch(s->gexec, st));
  for (uint32_t b = 0; b < s->B; ++b) s->cur_len[b] += 1;
  return download_outputs(s, logits, next);
}

extern "C" akh_status akh_session_decode_greedy(akh_session* s,
                                                uint32_t steps,
                                                uint32_t* out_tokens) {
  CHECK_ARG(s, "akh_session_decode_greedy: NULL session");
  akh_status nc = need_caches(s);
  if (nc != AKH_OK) return nc;
  for (uint32_t b = 0; b < s->B; ++b)
    if (s->cur_len[b] + steps > s->max_ctx)
      return fail(AKH_E_CONTEXT_FULL, "context window is full (" +
                                          std::to_string(s->max_ctx) +
                                          " tokens)");
  if (steps == 0) return AKH_OK;
  akh_status st0 = ensure_decode_graph(s);
  if (st0 != AKH_OK) return st0;
  hipStream_t st = s->be->stream;
  std::vector<uint32_t> start(s->cur_len);
  uint32_t i = 0;
  if (kStepsPerGraph > 1)
    for (; i + kStepsPerGraph <= steps; i += kStepsPerGraph)
      HIP_TRY(hipGraphLaunch(s->gexec_n, st));
  for (; i < steps; ++i) HIP_TRY(hipGraphLaunch(s->gexec, st));
  for (uint32_t b = 0; b < s->B; ++b) s->cur_len[b] += steps;
  if (out_tokens) {
    std::vector<uint32_t> h((size_t)s->B * (s->max_ctx + 1));
    HIP_TRY(hipMemcpyAsync(h.data(), s->hist, h.size() * 4,
                           hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    for (uint32_t i = 0; i < steps; ++i)
      for (uint32_t b = 0; b < s->B; ++b)
        out_tokens[(size_t)i * s->B + b] =
            h[(size_t)b * (s->max_ctx + 1) + start[b] + 1 + i];
  }
  return AKH_OK;
}

namespace {

// Buffers and graph of generate rounds for `max_new` tokens with `params`.
akh_status ensure_generate(akh_session* s, uint32_t max_new, const akh_sampling& params) {
  drop_stale_graphs(s);
  if (max_new > s->gcap) {
    if (s->ggexec) hipGraphExecDestroy(s->ggexec);
    if (s->ggraph) hipGraphDestroy(s->ggraph);
    s->ggexec = nullptr;
    s->ggraph = nullptr;
    if (s->ggen) HIP_TRY(hipFree(s->ggen));
    if (s->guni) HIP_TRY(hipFree(s->guni));
    s->ggen = nullptr;
    s->guni = nullptr;
    HIP_TRY(hipMalloc(&s->ggen, (size_t)s->B * max_new * sizeof(uint32_t)));
    HIP_TRY(hipMalloc(&s->guni, (size_t)max_new * s->B * sizeof(double)));
    s->gcap = max_new;
  }
  const bool same = s->ggexec && s->gmax_new == max_new &&
                    s->gparams.temperature == params.temperature &&
                    s->gparams.top_k == params.top_k && s->gparams.top_p == params.top_p &&
                    s->gparams.repetition_penalty == params.repetition_penalty;
  if (same) return AKH_OK;
  if (s->ggexec) hipGraphExecDestroy(s->ggexec);
  if (s->ggraph) hipGraphDestroy(s->ggraph);
  s->ggexec = nullptr;
  s->ggraph = nullptr;
  s->gparams = params;
  s->gmax_new = max_new;
  return capture(s, enqueue_generate_round, &s->ggraph, &s->ggexec, "generate graph");
}

}  // namespace

namespace {

// Prompts of different lengths fed to sequences that hold caches
// (inference.rs:290-299: one decode step per prompt token), right-aligned:
// in step i of L = the longest prompt, sequence b decodes its token
// i - (L - lens[b]) if that is >= 0 and is left out otherwise (attention
// skips it, its cache and position stay).  Every sequence decodes its last
// prompt token in the final step, so the logits then are each sequence's
// own.  ContextFull as decode_step raises it (inference.rs:179-187): the
// steps before the first token some context cannot take are decoded, then
// the call fails.
akh_status feed_ragged(akh_session* s, const uint32_t* tokens, const uint32_t* lens) {
  const uint32_t B = s->B;
  uint32_t L = 0;
  std::vector<size_t> at(B + 1, 0);
  for (uint32_t b = 0; b < B; ++b) {
    L = std::max(L, lens[b]);
    at[b + 1] = at[b] + lens[b];
  }
  hipStream_t st = s->be->stream;
  // Every step's tokens and rows, kept until the stream has read them.
  std::vector<uint32_t> cols((size_t)L * kMaxBatch, 0u);
  std::vector<int> acts((size_t)L * kMaxBatch, 0);
  for (uint32_t i = 0; i < L; ++i)
    for (uint32_t b = 0; b < B; ++b) {
      const uint32_t lead = L - lens[b];
      if (i < lead) continue;
      cols[(size_t)i * kMaxBatch + b] = tokens[at[b] + (i - lead)];
      acts[(size_t)i * kMaxBatch + b] = 1;
    }
  bool full = false;
  for (uint32_t i = 0; i < L && !full; ++i) {
    for (uint32_t b = 0; b < B; ++b)
      full = full || (acts[(size_t)i * kMaxBatch + b] && s->cur_len[b] >= s->max_ctx);
    if (full) break;
    HIP_TRY(hipMemcpyAsync(s->tok, cols.data() + (size_t)i * kMaxBatch, B * sizeof(uint32_t),
                           hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->active, acts.data() + (size_t)i * kMaxBatch,
                           kMaxBatch * sizeof(int), hipMemcpyHostToDevice, st));
    HIP_TRY(enqueue_decode_body(s));
    HIP_TRY(launch_advance(s->pos, s->active, (int)B, st, s->tok, s->hist,
                           (long)s->max_ctx + 1));
    for (uint32_t b = 0; b < B; ++b) s->cur_len[b] += acts[(size_t)i * kMaxBatch + b];
  }
  HIP_TRY(hipStreamSynchronize(st));
  akh_status sa = set_active(s, true);
  if (full)
    return fail(AKH_E_CONTEXT_FULL,
                "context window is full (" + std::to_string(s->max_ctx) + " tokens)");
  return sa;
}

akh_status generate_impl(akh_session* s, const uint32_t* tokens, const uint32_t* lens,
                         uint32_t max_new_tokens, akh_sampling params,
                         const double* uniforms, uint32_t* out_tokens,
                         uint32_t* out_counts) {
  bool uniform = true;
  for (uint32_t b = 0; b < s->B; ++b) {
    if (lens[b] == 0) return fail(AKH_E_EMPTY_PROMPT, "prompt is empty");
    uniform = uniform && lens[b] == lens[0];
  }
  const uint32_t prompt_len = lens[0];
  CHECK_ARG(params.temperature <= 0.0f || uniforms || max_new_tokens == 0,
            "akh_session_generate: sampling (temperature > 0) needs uniforms");
  // A sequence without a cache gets a fresh one (inference.rs:278-287).
  for (uint32_t b = 0; b < s->B; ++b)
    if (!s->has_cache[b]) {
      s->has_cache[b] = 1;
      s->cur_len[b] = 0;
    }
  bool all_empty = true, all_resumed = true;
  for (uint32_t b = 0; b < s->B; ++b) {
    all_empty = all_empty && s->cur_len[b] == 0;
    all_resumed = all_resumed && s->cur_len[b] > 0;
  }
  CHECK_ARG(all_empty || all_resumed,
            "akh_session_generate: sequences must all be empty or all hold a cache");
  const uint32_t B = s->B;
  std::vector<int> start(kMaxBatch, 0);
  for (uint32_t b = 0; b < B; ++b) start[b] = (int)s->cur_len[b];
  // The prompt: prefill on empty caches, else one decode step per token
  // (inference.rs:290-299).
  akh_status st = AKH_OK;
  if (all_empty) {
    st = prefill_impl(s, tokens, lens, nullptr, nullptr);
  } else if (uniform) {
    std::vector<uint32_t> col(B);
    for (uint32_t i = 0; i < prompt_len && st == AKH_OK; ++i) {
      for (uint32_t b = 0; b < B; ++b) col[b] = tokens[(size_t)b * prompt_len + i];
      st = akh_session_decode_step(s, col.data(), nullptr, nullptr);
    }
  } else {
    st = feed_ragged(s, tokens, lens);
  }
  if (st != AKH_OK) return st;
  std::fill(out_counts, out_counts + B, 0u);
  if (max_new_tokens == 0) return AKH_OK;

  st = ensure_generate(s, max_new_tokens, params);
  if (st != AKH_OK) return st;
  hipStream_t hs = s->be->stream;
  std::vector<int> zero(kMaxBatch, 0), done(kMaxBatch, 1);
  for (uint32_t b = 0; b < B; ++b) done[b] = 0;
  HIP_TRY(hipMemcpyAsync(s->gstart, start.data(), kMaxBatch * sizeof(int), hipMemcpyHostToDevice, hs));
  HIP_TRY(hipMemcpyAsync(s->gcount, zero.data(), kMaxBatch * sizeof(int), hipMemcpyHostToDevice, hs));
  HIP_TRY(hipMemcpyAsync(s->done, done.data(), kMaxBatch * sizeof(int), hipMemcpyHostToDevice, hs));
  if (params.temperature > 0.0f)
    HIP_TRY(hipMemcpyAsync(s->guni, uniforms, (size_t)max_new_tokens * B * sizeof(double),
                           hipMemcpyHostToDevice, hs));
  for (uint32_t i = 0; i < max_new_tokens; ++i) HIP_TRY(hipGraphLaunch(s->ggexec, hs));

  std::vector<uint32_t> cnt(kMaxBatch), gen((size_t)B * max_new_tokens);
  std::vector<int> pos(kMaxBatch);
  HIP_TRY(hipMemcpyAsync(cnt.data(), s->gcount, kMaxBatch * sizeof(uint32_t), hipMemcpyDeviceToHost, hs));
  HIP_TRY(hipMemcpyAsync(gen.data(), s->ggen, gen.size() * sizeof(uint32_t), hipMemcpyDeviceToHost, hs));
  HIP_TRY(hipMemcpyAsync(pos.data(), s->pos, kMaxBatch * sizeof(int), hipMemcpyDeviceToHost, hs));
  HIP_TRY(hipStreamSynchronize(hs));
  for (uint32_t b = 0; b < B; ++b) {
    out_counts[b] = cnt[b];
    for (uint32_t i = 0; i < cnt[b]; ++i)
      out_tokens[(size_t)b * max_new_tokens + i] = gen[(size_t)b * max_new_tokens + i];
    s->cur_len[b] = (uint32_t)pos[b];
  }
  return set_active(s, true);
}

}  // namespace

extern "C" akh_status akh_session_generate(akh_session* s, const uint32_t* tokens,
                                           uint32_t prompt_len, uint32_t max_new_tokens,
                                           akh_sampling params, const double* uniforms,
                                           uint32_t* out_tokens, uint32_t* out_counts) {
  CHECK_ARG(s && (tokens || !prompt_len) && out_counts && (out_tokens || !max_new_tokens),
            "akh_session_generate: NULL argument");
  const std::vector<uint32_t> lens(s->B, prompt_len);
  return generate_impl(s, tokens, lens.data(), max_new_tokens, params, uniforms, out_tokens,
                       out_counts);
}

extern "C" akh_status akh_session_generate_ragged(akh_session* s, const uint32_t* tokens,
                                                  const uint32_t* prompt_lens,
                                                  uint32_t max_new_tokens, akh_sampling params,
                                                  const double* uniforms, uint32_t* out_tokens,
                                                  uint32_t* out_counts) {
  CHECK_ARG(s && prompt_lens && out_counts && (out_tokens || !max_new_tokens),
            "akh_session_generate_ragged: NULL argument");
  size_t n = 0;
  for (uint32_t b = 0; b < s->B; ++b) n += prompt_lens[b];
  CHECK_ARG(tokens || n == 0, "akh_session_generate_ragged: NULL tokens");
  return generate_impl(s, tokens, prompt_lens, max_new_tokens, params, uniforms, out_tokens,
                       out_counts);
}

namespace {

// One sequence's [max_ctx, d] rows of layer l, K (which 0) or V (1), to or
// from host fp32, widening or rounding (to nearest even) a bfloat16 cache.
akh_status cache_rows_out(akh_session* s, uint32_t l, int which, uint32_t seq, float* host) {
  const size_t n = (size_t)s->seq_stride();
  const char* src = static_cast<const char*>(s->kv_at(l, which)) + seq * n * s->kv_elem();
  if (!s->kv16) {
    HIP_TRY(hipMemcpyAsync(host, src, n * 4, hipMemcpyDeviceToHost, s->be->stream));
    HIP_TRY(hipStreamSynchronize(s->be->stream));
    return AKH_OK;
  }
  std::vector<uint16_t> t(n);
  HIP_TRY(hipMemcpyAsync(t.data(), src, n * 2, hipMemcpyDeviceToHost, s->be->stream));
  HIP_TRY(hipStreamSynchronize(s->be->stream));
  for (size_t i = 0; i < n; ++i) {
    const uint32_t u = (uint32_t)t[i] << 16;
    std::memcpy(host + i, &u, 4);
  }
  return AKH_OK;
}

akh_status cache_rows_in(akh_session* s, uint32_t l, int which, uint32_t seq, const float* host) {
  const size_t n = (size_t)s->seq_stride();
  char* dst = static_cast<char*>(s->kv_at(l, which)) + seq * n * s->kv_elem();
  if (!s->kv16) {
    HIP_TRY(hipMemcpyAsync(dst, host, n * 4, hipMemcpyHostToDevice, s->be->stream));
    HIP_TRY(hipStreamSynchronize(s->be->stream));
    return AKH_OK;
  }
  std::vector<uint16_t> t(n);
  for (size_t i = 0; i < n; ++i) {
    uint32_t u;
    std::memcpy(&u, host + i, 4);
    t[i] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
  HIP_TRY(hipMemcpyAsync(dst, t.data(), n * 2, hipMemcpyHostToDevice, s->be->stream));
  HIP_TRY(hipStreamSynchronize(s->be->stream));
  return AKH_OK;
}

}  // namespace

extern "C" akh_status akh_session_set_kv_bf16(akh_session* s, int enable) {
  CHECK_ARG(s && (enable == 0 || enable == 1), "akh_session_set_kv_bf16: bad argument");
  CHECK_ARG(!s->be->capturing, "akh_session_set_kv_bf16: graph capture in progress");
  for (uint32_t b = 0; b < s->B; ++b)
    if (s->cur_len[b] != 0)
      return fail(AKH_E_CACHE_NOT_EMPTY, "akh_session_set_kv_bf16 needs empty caches, sequence " +
                                             std::to_string(b) + " holds " +
                                             std::to_string(s->cur_len[b]) + " tokens");
  if ((enable != 0) == s->kv16) return AKH_OK;
  const akh_model_config& c = s->m->cfg;
  const size_t elems = (size_t)c.num_layers * s->layer_stride();
  HIP_TRY(hipSetDevice(s->be->device));
  HIP_TRY(hipStreamSynchronize(s->be->stream));
  // Graphs hold the attention kernel of the old element type.
  drop_graphs(s);
  free_prefill(s);
  // The new cache is allocated before the old one is freed: on failure the
  // session keeps its old cache and element type unchanged.
  const size_t bytes = elems * (enable ? 2 : 4);
  void* nkv = nullptr;
  HIP_TRY(hipMalloc(&nkv, bytes));
  hipError_t e = hipMemset(nkv, 0, bytes);
  if (e != hipSuccess) {
    hipFree(nkv);
    return fail(AKH_E_HIP, std::string("akh_session_set_kv_bf16: ") + hipGetErrorString(e));
  }
  hipFree(s->kv);
  s->kv = static_cast<float*>(nkv);
  s->kv16 = enable != 0;
  return AKH_OK;
}

extern "C" akh_status akh_session_take_cache(akh_session* s, uint32_t seq, float* k,
                                             float* v, uint32_t* cur_len, int* had_cache) {
  CHECK_ARG(s && seq < s->B, "akh_session_take_cache: bad argument");
  const bool had = s->has_cache[seq] != 0;
  if (had_cache) *had_cache = had ? 1 : 0;
  if (cur_len) *cur_len = had ? s->cur_len[seq] : 0;
  if (!had) return AKH_OK;
  const size_t n = (size_t)s->seq_stride();
  for (uint32_t l = 0; l < s->m->cfg.num_layers; ++l) {
    akh_status st = k ? cache_rows_out(s, l, 0, seq, k + l * n) : AKH_OK;
    if (st == AKH_OK && v) st = cache_rows_out(s, l, 1, seq, v + l * n);
    if (st != AKH_OK) return st;
  }
  s->has_cache[seq] = 0;
  s->cur_len[seq] = 0;
  return upload_positions(s);
}

extern "C" akh_status akh_session_replace_cache(akh_session* s, uint32_t seq, const float* k,
                                                const float* v, uint32_t cur_len) {
  CHECK_ARG(s && seq < s->B && k && v, "akh_session_replace_cache: bad argument");
  CHECK_ARG(cur_len <= s->max_ctx, "Cache/session max_context_len mismatch");
  const size_t n = (size_t)s->seq_stride();
  hipStream_t st = s->be->stream;
  for (uint32_t l = 0; l < s->m->cfg.num_layers; ++l) {
    akh_status cs = cache_rows_in(s, l, 0, seq, k + l * n);
    if (cs == AKH_OK) cs = cache_rows_in(s, l, 1, seq, v + l * n);
    if (cs != AKH_OK) return cs;
  }
  // The installed cache carries no token history.
  HIP_TRY(hipMemsetAsync(s->hist + (size_t)seq * (s->max_ctx + 1), 0,
                         (size_t)(s->max_ctx + 1) * sizeof(uint32_t), st));
  HIP_TRY(hipMemsetAsync(s->tok + seq, 0, sizeof(uint32_t), st));
  s->has_cache[seq] = 1;
  s->cur_len[seq] = cur_len;
  return upload_positions(s);
}

extern "C" akh_status akh_session_download_cache(akh_session* s,
                                                 uint32_t layer, uint32_t seq,
                                                 int which, float* host) {
  CHECK_ARG(s && host && layer < s->m->cfg.num_layers && seq < s->B &&
                (which == 0 || which == 1),
            "akh_session_download_cache: bad argument");
  return cache_rows_out(s, layer, which, seq, host);
}

extern "C" akh_status akh_session_time_decode_kernel(akh_session* s,
                                                     int kernel,
                                                     uint32_t reps,
                                                     float* avg_ms) {
  CHECK_ARG(s && avg_ms && reps > 0, "akh_session_time_decode_kernel: bad argument");
  CHECK_ARG(kernel >= 0 && kernel <= 6, "akh_session_time_decode_kernel: bad kernel");
  CHECK_ARG(!s->generic, "akh_session_time_decode_kernel: times the batched decode kernels, "
                         "which this session's shape does not run");
  for (uint32_t b = 0; b < s->B; ++b)
    CHECK_ARG(s->cur_len[b] >= 1 && s->cur_len[b] < s->max_ctx,
              "akh_session_time_decode_kernel: needs 1 <= cur_len < max_ctx");
  akh_backend* be = s->be;
  const uint32_t L = s->m->cfg.num_layers;
  auto one = [&](uint32_t i) -> hipError_t {
    const uint32_t l = i % L;
    switch (kernel) {
      case 0: return enqueue_attn(s, l);
      case 1: return enqueue_qkv(s, l);
      case 2: return enqueue_out(s, l);
      case 3: return enqueue_up(s, l);
      case 4: return enqueue_down(s, l);
      case 5: return enqueue_lm_head(s);
      default:
        // The step's RMSNorm kernel: the residual add + norm after each
        // GEMM pair, or with the norm fused, the final norm alone.
        return s->fuse_out && s->fuse_down
                   ? enqueue_norm_only(s, s->m->final_norm())
                   : enqueue_resid_norm(s, s->p_out, s->ks_out, s->m->layer(l, W_NORM2));
    }
  };
  for (uint32_t l = 0; l < L; ++l) HIP_TRY(one(l));  // warm
  HIP_TRY(hipEventRecord(be->t0, be->stream));
  for (uint32_t i = 0; i < reps; ++i) HIP_TRY(one(i));
  HIP_TRY(hipEventRecord(be->t1, be->stream));
  HIP_TRY(hipEventSynchronize(be->t1));
  float ms = 0.f;
  HIP_TRY(hipEventElapsedTime(&ms, be->t0, be->t1));
  *avg_ms = ms / (float)reps;
  return AKH_OK;
}

extern "C" akh_status akh_session_time_decode_attn(akh_session* s, uint32_t reps,
                                                   float* avg_ms) {
  CHECK_ARG(s && avg_ms && reps > 0 && reps <= 4096,
            "akh_session_time_decode_attn: bad argument");
  CHECK_ARG(!s->generic, "akh_session_time_decode_attn: times the batched decode kernels, "
                         "which this session's shape does not run");
  for (uint32_t b = 0; b < s->B; ++b)
    CHECK_ARG(s->cur_len[b] >= 1 && s->cur_len[b] < s->max_ctx,
              "akh_session_time_decode_attn: needs 1 <= cur_len < max_ctx");
  const uint32_t L = s->m->cfg.num_layers;
  std::vector<hipEvent_t> ev(2 * (size_t)reps, nullptr);
  hipError_t e = hipSuccess;
  for (size_t i = 0; i < ev.size() && e == hipSuccess; ++i) e = hipEventCreate(&ev[i]);
  for (uint32_t l = 0; l < L && e == hipSuccess; ++l) e = enqueue_attn(s, l);  // warm
  for (uint32_t i = 0; i < reps && e == hipSuccess; ++i)
    e = enqueue_attn(s, i % L, ev[2 * i], ev[2 * i + 1]);
  if (e == hipSuccess) e = hipStreamSynchronize(s->be->stream);
  double total = 0.0;
  for (uint32_t i = 0; i < reps && e == hipSuccess; ++i) {
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]);
    total += ms;
  }
  for (hipEvent_t x : ev)
    if (x) hipEventDestroy(x);
  HIP_TRY(e);
  *avg_ms = (float)(total / reps);
  return AKH_OK;
}

extern "C" akh_status akh_session_decode_launches(akh_session* s, uint32_t* launches) {
  CHECK_ARG(s && launches, "akh_session_decode_launches: bad argument");
  CHECK_ARG(!s->be->capturing, "akh_session_decode_launches: graph capture in progress");
  HIP_TRY(hipSetDevice(s->be->device));
  akh_status st = ensure_decode_graph(s);
  if (st != AKH_OK) return st;
  size_t n = 0;
  HIP_TRY(hipGraphGetNodes(s->graph, nullptr, &n));
  std::vector<hipGraphNode_t> nodes(n);
  HIP_TRY(hipGraphGetNodes(s->graph, nodes.data(), &n));
  uint32_t k = 0;
  for (hipGraphNode_t node : nodes) {
    hipGraphNodeType t;
    HIP_TRY(hipGraphNodeGetType(node, &t));
    if (t == hipGraphNodeTypeKernel) ++k;
  }
  *launches = k;
  return AKH_OK;
}

extern "C" akh_status akh_session_set_fused_norm(akh_session* s, int enable) {
  CHECK_ARG(s, "akh_session_set_fused_norm: NULL session");
  CHECK_ARG(!s->be->capturing, "akh_session_set_fused_norm: graph capture in progress");
  CHECK_ARG(!enable || s->ssq,
            "akh_session_set_fused_norm: needs a decode session on the batched kernels "
            "whose dim is a multiple of "
            "128, at most 4096");
  if (s->fuse_out != (enable != 0)) {
    HIP_TRY(hipSetDevice(s->be->device));
    HIP_TRY(hipStreamSynchronize(s->be->stream));
    drop_graphs(s);  // captured with the other kernels
    s->fuse_out = s->fuse_down = enable != 0;
  }
  return AKH_OK;
}

// ---------------------------------------------------------------------------
// The trainer's fused forward (Trainer::forward + CrossEntropy)
// ---------------------------------------------------------------------------

struct akh_forward {
  akh_model* m = nullptr;
  akh_session* s = nullptr;  // prefill buffers; its KV cache is scratch
  uint32_t B = 0, S = 0;
  float* logits = nullptr;    // [rows, vocab]: logits, then probabilities
  float* losses = nullptr;    // [rows]
  uint32_t* targets = nullptr;
  akh_cross_entropy_meta* ce = nullptr;  // device meta
};

extern "C" void akh_forward_free(akh_forward* f) {
  if (!f) return;
  if (f->s) akh_session_free(f->s);
  void* bufs[] = {f->logits, f->losses, f->targets, f->ce};
  for (void* p : bufs)
    if (p) hipFree(p);
  delete f;
}

extern "C" akh_status akh_forward_new(akh_model* m, uint32_t batch, uint32_t seq_len,
                                      akh_forward** out) {
  CHECK_ARG(m && out, "akh_forward_new: NULL argument");
  CHECK_ARG(batch >= 1 && seq_len >= 1, "akh_forward_new: needs batch >= 1 and seq_len >= 1");
  *out = nullptr;
  akh_forward* f = new akh_forward();
  f->m = m;
  f->B = batch;
  f->S = seq_len;
  akh_status st = session_create(m, seq_len, batch, false, &f->s);
  if (st != AKH_OK) {
    akh_forward_free(f);
    return st;
  }
  const size_t rows = (size_t)batch * seq_len, V = m->cfg.vocab_size;
  hipError_t e = hipMalloc(&f->logits, rows * V * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&f->losses, rows * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&f->targets, rows * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMalloc(&f->ce, sizeof(akh_cross_entropy_meta));
  akh_cross_entropy_meta ce{(uint32_t)V, (uint32_t)rows};
  if (e == hipSuccess) e = hipMemcpy(f->ce, &ce, sizeof ce, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    akh_forward_free(f);
    return fail(AKH_E_HIP, std::string("akh_forward_new: ") + hipGetErrorString(e));
  }
  *out = f;
  return AKH_OK;
}

extern "C" akh_status akh_forward_loss(akh_forward* f, const uint32_t* tokens,
                                       const uint32_t* targets, float* losses,
                                       float* mean_loss) {
  CHECK_ARG(f && tokens && targets && mean_loss, "akh_forward_loss: NULL argument");
  akh_session* s = f->s;
  const akh_model_config& c = f->m->cfg;
  const uint32_t S = f->S, d = c.dim, V = c.vocab_size;
  const size_t rows = (size_t)f->B * S;
  for (size_t r = 0; r < rows; ++r)
    CHECK_ARG(targets[r] < V, "akh_forward_loss: target token " + std::to_string(targets[r]) +
                                  " is out of the vocabulary");
  akh_status st0 = ensure_prefill(s, rows);
  if (st0 != AKH_OK) return st0;
  hipStream_t st = s->be->stream;
  HIP_TRY(hipMemcpyAsync(s->ptok, tokens, rows * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(f->targets, targets, rows * 4, hipMemcpyHostToDevice, st));
  PrefillRows pr;
  pr.rows = rows;
  pr.S = S;
  // The range flag needs a check whenever a GEMM may run k_gemm_h3: the
  // layers under the split-fp16 prefill, and the lm_head whenever the model
  // keeps its split-fp16 copy, also under the bf16-MFMA layers.
  const bool h3 = f->m->prefill_split == AKH_SPLIT_H3;
  // The layers, final_norm and lm_head on every row (train.rs:154-177).
  auto forward = [&](bool exact) -> hipError_t {
    hipError_t e = launch_embedding_rows(s->ptok, f->m->embedding(), s->px, (int)rows, (int)d,
                                         V, st);
    if (e == hipSuccess)
      e = f->m->prefill_bf16 ? prefill_layers_bf16(s, pr) : prefill_layers_f32(s, pr, exact);
    if (e == hipSuccess)
      e = launch_rows_rmsnorm(s->px, f->m->final_norm(), s->pxn, (int)rows, (int)d, c.norm_eps,
                              st);
    GemmParams g{};
    g.a = s->pxn;
    g.b = f->m->lm_head();
    g.c = f->logits;
    g.M = (int)rows;
    g.N = (int)V;
    g.K = (int)d;
    if (e == hipSuccess) e = prefill_gemm(f->m, g, 2 + 6 * c.num_layers, GEMM_STORE, st, exact);
    return e;
  };
  // The forward and the loss, whose copy to the host is queued before the
  // range flag is read (one wait for both).
  std::vector<float> l(rows);
  auto forward_loss = [&](bool exact) -> hipError_t {
    hipError_t e = forward(exact);
    if (e == hipSuccess)
      e = launch_cross_entropy(f->logits, f->targets, f->losses, (uint32_t)rows, f->ce, st);
    if (e == hipSuccess)
      e = hipMemcpyAsync(l.data(), f->losses, rows * 4, hipMemcpyDeviceToHost, st);
    return e;
  };
  if (h3) HIP_TRY(clear_range_flag(f->m, st));
  HIP_TRY(forward_loss(false));
  bool redo = false;
  if (h3) HIP_TRY(range_flag_set(f->m, st, &redo));
  if (redo) HIP_TRY(forward_loss(true));  // an operand beyond fp16's range
  HIP_TRY(hipStreamSynchronize(st));
  // CrossEntropy::loss (layers.rs:512-515): sequential f32 sum over rows.
  float sum = 0.f;
  for (float v : l) sum += v;
  *mean_loss = sum / (float)rows;
  if (losses) std::copy(l.begin(), l.end(), losses);
  return AKH_OK;
}

extern "C" akh_status akh_forward_probs(akh_forward* f, uint32_t row0, uint32_t n, float* host) {
  CHECK_ARG(f && (host || !n), "akh_forward_probs: NULL argument");
  CHECK_ARG((size_t)row0 + n <= (size_t)f->B * f->S, "akh_forward_probs: rows out of range");
  const size_t V = f->m->cfg.vocab_size;
  HIP_TRY(hipMemcpyAsync(host, f->logits + (size_t)row0 * V, (size_t)n * V * 4,
                         hipMemcpyDeviceToHost, f->s->be->stream));
  HIP_TRY(hipStreamSynchronize(f->s->be->stream));
  return AKH_OK;
}

extern "C" akh_status akh_forward_hidden(akh_forward* f, float* host) {
  CHECK_ARG(f && host, "akh_forward_hidden: NULL argument");
  CHECK_ARG(f->s->px, "akh_forward_hidden: no forward has run");
  HIP_TRY(hipMemcpyAsync(host, f->s->px, (size_t)f->B * f->S * f->m->cfg.dim * 4,
                         hipMemcpyDeviceToHost, f->s->be->stream));
  HIP_TRY(hipStreamSynchronize(f->s->be->stream));
  return AKH_OK;
}
