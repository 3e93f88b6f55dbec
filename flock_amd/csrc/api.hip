// C ABI of libflock_attn.so: argument checks, error reporting, streams,
// memory helpers and the entry points declared in include/flock_attn.h.
//
// Every entry point validates its arguments on the host before touching the
// device, so a rejected call has no side effect -- the reference's Layer
// throws before encoding anything (kernels/layer.ts:575, 689-698; lib.ts:504-506).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "common.hpp"

namespace flk {

// The error text and the current stream belong to the calling host thread:
// two threads can drive two streams without one's flk_set_stream retargeting
// the other's launches. g_left_streams: this thread switched away from a
// non-null stream, which may still hold work that reads buffers (flk_free
// then waits for the whole device).
static thread_local char g_err[512] = "";
static thread_local hipStream_t g_stream = nullptr;
static thread_local bool g_left_streams = false;

hipStream_t Stream::get() { return g_stream; }

static int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

static int32_t hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FLK_OK;
  return fail(FLK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

static int32_t check_heads(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim) {
  if (n_heads == 0 || n_kv_heads == 0)
    return fail(FLK_ERR_ARG, "n_heads (%u) and n_kv_heads (%u) must be >= 1", n_heads, n_kv_heads);
  if (n_heads % n_kv_heads != 0)
    return fail(FLK_ERR_ARG, "n_heads %u is not a multiple of n_kv_heads %u", n_heads, n_kv_heads);
  if (n_heads / n_kv_heads > 8)
    return fail(FLK_ERR_UNSUPPORTED, "GQA group %u > 8 is not supported", n_heads / n_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return fail(FLK_ERR_UNSUPPORTED, "head_dim %u not supported (64 or 128)", head_dim);
  return FLK_OK;
}

static int32_t check_ws(void* ws, uint64_t ws_bytes, uint64_t need) {
  if (need == 0) return FLK_OK;  // single-split launch: no partials
  if (ws == nullptr || ws_bytes < need)
    return fail(FLK_ERR_WORKSPACE, "workspace of %llu bytes needed, got %llu%s",
                (unsigned long long)need, (unsigned long long)ws_bytes,
                ws == nullptr ? " (null)" : "");
  if (reinterpret_cast<uintptr_t>(ws) % 256 != 0)
    return fail(FLK_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return FLK_OK;
}

// The attention kernels move 16-byte vectors (float4) of q, o and the caches.
static int32_t check_vec4(const void* p, const char* name) {
  if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
    return fail(FLK_ERR_ARG, "%s must be 16-byte aligned", name);
  return FLK_OK;
}

#define FLK_ALIGNED(p)                                                  \
  do {                                                                  \
    int32_t rc_ = check_vec4((p), #p);                                  \
    if (rc_) return rc_;                                                \
  } while (0)

#define FLK_NONNULL(p)                                                  \
  do {                                                                  \
    if ((p) == nullptr) return fail(FLK_ERR_ARG, "%s is null", #p);     \
  } while (0)

}  // namespace flk

using namespace flk;

extern "C" {

const char* flk_last_error(void) { return g_err; }

const char* flk_version(void) { return "flock_attn 0.1 (gfx950)"; }

int32_t flk_device_count(int32_t* count) {
  FLK_NONNULL(count);
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return FLK_OK;
}

int32_t flk_set_stream(void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (g_stream != nullptr && g_stream != s) g_left_streams = true;
  g_stream = s;
  return FLK_OK;
}

int32_t flk_alloc(void** dptr, uint64_t bytes) {
  FLK_NONNULL(dptr);
  if (bytes == 0) return fail(FLK_ERR_ARG, "flk_alloc of 0 bytes");
  return hip_status(hipMalloc(dptr, bytes), "hipMalloc");
}

int32_t flk_free(void* dptr) {
  if (dptr == nullptr) return FLK_OK;
  // A free cannot be recorded into a graph, and hipFree would end a capture
  // in progress: refuse it while the library stream is capturing.
  if (g_stream != nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(FLK_ERR_ARG, "flk_free while the library stream is capturing a graph");
  }
  // Work queued on the library stream may still read this buffer (a caller
  // can drop its last reference right after a launch): wait for that stream,
  // and for the whole device when this thread has launched on other streams
  // since (streams from flk_stream_create do not synchronise with the null
  // stream, so the null stream's wait alone would not cover them).
  hipError_t e = hipStreamSynchronize(g_stream);
  if (e == hipSuccess && g_left_streams) {
    e = hipDeviceSynchronize();
    if (e == hipSuccess) g_left_streams = false;
  }
  if (e == hipSuccess) e = hipFree(dptr);
  return hip_status(e, "hipFree");
}

int32_t flk_h2d(void* dst, const void* host_src, uint64_t bytes, uint64_t dst_off) {
  FLK_NONNULL(dst);
  FLK_NONNULL(host_src);
  if (bytes == 0) return FLK_OK;
  hipError_t e = hipMemcpyAsync(static_cast<char*>(dst) + dst_off, host_src, bytes,
                                hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  return hip_status(e, "flk_h2d");
}

int32_t flk_d2h(void* host_dst, const void* src, uint64_t bytes, uint64_t src_off) {
  FLK_NONNULL(host_dst);
  FLK_NONNULL(src);
  if (bytes == 0) return FLK_OK;
  hipError_t e = hipMemcpyAsync(host_dst, static_cast<const char*>(src) + src_off, bytes,
                                hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  return hip_status(e, "flk_d2h");
}

int32_t flk_memset(void* dst, int32_t value, uint64_t bytes) {
  FLK_NONNULL(dst);
  if (bytes == 0) return FLK_OK;
  return hip_status(hipMemsetAsync(dst, value, bytes, g_stream), "hipMemsetAsync");
}

int32_t flk_sync(void) { return hip_status(hipStreamSynchronize(g_stream), "flk_sync"); }

uint64_t flk_workspace_bytes(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                             uint32_t max_keys, uint32_t max_queries, uint32_t max_seqs) {
  if (n_heads == 0 || n_kv_heads == 0 || n_heads % n_kv_heads != 0 || head_dim == 0) return 0;
  if (max_keys == 0) max_keys = 1;
  if (max_seqs == 0) max_seqs = 1;
  const DecodeShape ds{n_heads, n_kv_heads, head_dim, max_seqs, max_keys};
  uint64_t need = decode_ws_bound(ds);
  // A single-sequence decode plans its splits on its own, so cover it too.
  const DecodeShape ds1{n_heads, n_kv_heads, head_dim, 1, max_keys};
  const uint64_t d1 = decode_ws_bound(ds1);
  if (d1 > need) need = d1;
  if (max_queries > 0) {
    const uint32_t nq = max_queries < max_keys ? max_queries : max_keys;
    const uint64_t b = prefill_ws_bound(n_heads, n_kv_heads, head_dim, nq, max_keys);
    if (b > need) need = b;
  }
  return ws_align(need > 0 ? need : 1);
}

uint64_t flk_call_workspace_bytes(int32_t kind, uint32_t n_heads, uint32_t n_kv_heads,
                                  uint32_t head_dim, uint32_t n, uint32_t pos0, uint32_t n_seqs) {
  if (n_heads == 0 || n_kv_heads == 0 || n_heads % n_kv_heads != 0 || head_dim == 0 || n == 0)
    return 0;
  switch (kind) {
    case FLK_CALL_DECODE:
      return decode_ws_bytes(DecodeShape{n_heads, n_kv_heads, head_dim, 1, n});
    case FLK_CALL_RAGGED:
      return decode_ws_bytes(DecodeShape{n_heads, n_kv_heads, head_dim, n_seqs ? n_seqs : 1, n});
    case FLK_CALL_PREFILL:
      return prefill_ws_bytes(prefill_plan(n_heads, n_kv_heads, head_dim, n, pos0), head_dim);
    default:
      return 0;
  }
}

int32_t flk_rmsnorm(const float* x, const float* g, float* o, uint32_t n, uint32_t n_vecs,
                    float eps) {
  FLK_NONNULL(x);
  FLK_NONNULL(g);
  FLK_NONNULL(o);
  if (n == 0 || n_vecs == 0) return fail(FLK_ERR_ARG, "rmsnorm n=%u n_vecs=%u", n, n_vecs);
  if (!(eps >= 0.f)) return fail(FLK_ERR_ARG, "rmsnorm eps must be >= 0");
  return hip_status(launch_rmsnorm(x, g, o, n, n_vecs, eps, g_stream), "flk_rmsnorm");
}

int32_t flk_rope(float* x, const float* inv_freq, uint32_t n_tokens, uint32_t n_heads,
                 uint32_t head_dim, uint32_t pos0, int32_t pairing) {
  FLK_NONNULL(x);
  FLK_NONNULL(inv_freq);
  if (n_tokens == 0 || n_heads == 0 || head_dim == 0 || head_dim % 2 != 0)
    return fail(FLK_ERR_ARG, "rope n_tokens=%u n_heads=%u head_dim=%u", n_tokens, n_heads,
                head_dim);
  if (pairing != FLK_ROPE_NEOX && pairing != FLK_ROPE_NORM)
    return fail(FLK_ERR_ARG, "rope pairing %d (0 = neox, 1 = norm)", pairing);
  return hip_status(launch_rope(x, inv_freq, n_tokens, n_heads, head_dim, pos0, pairing, g_stream),
                    "flk_rope");
}

int32_t flk_kv_append(const float* kn, const float* v, float* kcache, float* vcache,
                      uint32_t n_tokens, uint32_t pos0, uint32_t n_kv_heads, uint32_t head_dim,
                      uint32_t max_keys) {
  FLK_NONNULL(kn);
  FLK_NONNULL(v);
  FLK_NONNULL(kcache);
  FLK_NONNULL(vcache);
  if (n_tokens == 0 || n_kv_heads == 0 || head_dim == 0)
    return fail(FLK_ERR_ARG, "kv_append n_tokens=%u n_kv_heads=%u head_dim=%u", n_tokens,
                n_kv_heads, head_dim);
  if ((uint64_t)pos0 + n_tokens > max_keys)
    return fail(FLK_ERR_CACHE_FULL, "KV cache would exceed %u keys (%u + %u)", max_keys, pos0,
                n_tokens);
  return hip_status(
      launch_kv_append(kn, v, kcache, vcache, n_tokens, pos0, n_kv_heads, head_dim, g_stream),
      "flk_kv_append");
}

static int32_t qk_prologue_common(const float* q_raw, const float* k_raw, const float* v_raw,
                                  uint32_t in_stride, const float* gq, const float* gk,
                                  const float* inv_freq, float eps, int32_t pairing, float* qn_out,
                                  float* kcache, float* vcache, uint32_t n_tokens, uint32_t pos0,
                                  uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                  uint32_t max_keys, const char* what) {
  FLK_NONNULL(q_raw);
  FLK_NONNULL(k_raw);
  FLK_NONNULL(v_raw);
  FLK_NONNULL(gq);
  FLK_NONNULL(gk);
  FLK_NONNULL(inv_freq);
  FLK_NONNULL(qn_out);
  FLK_NONNULL(kcache);
  FLK_NONNULL(vcache);
  int32_t rc = check_heads(n_heads, n_kv_heads, head_dim);
  if (rc) return rc;
  if (n_tokens == 0) return fail(FLK_ERR_ARG, "n_tokens must be >= 1, got 0");
  if (pairing != FLK_ROPE_NEOX && pairing != FLK_ROPE_NORM)
    return fail(FLK_ERR_ARG, "rope pairing %d (0 = neox, 1 = norm)", pairing);
  if (in_stride != 0 && in_stride < n_heads * head_dim)
    return fail(FLK_ERR_ARG, "in_stride %u is shorter than a q row (%u floats)", in_stride,
                n_heads * head_dim);
  if ((uint64_t)pos0 + n_tokens > max_keys)
    return fail(FLK_ERR_CACHE_FULL, "KV cache would exceed %u keys (%u + %u)", max_keys, pos0,
                n_tokens);
  return hip_status(launch_qk_prologue(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps, pairing, qn_out,
                                       kcache, vcache, n_tokens, pos0, n_heads, n_kv_heads,
                                       head_dim, g_stream, in_stride),
                    what);
}

int32_t flk_qk_prologue(const float* q_raw, const float* k_raw, const float* v_raw,
                        const float* gq, const float* gk, const float* inv_freq, float eps,
                        int32_t pairing, float* qn_out, float* kcache, float* vcache,
                        uint32_t n_tokens, uint32_t pos0, uint32_t n_heads, uint32_t n_kv_heads,
                        uint32_t head_dim, uint32_t max_keys) {
  return qk_prologue_common(q_raw, k_raw, v_raw, 0, gq, gk, inv_freq, eps, pairing, qn_out,
                            kcache, vcache, n_tokens, pos0, n_heads, n_kv_heads, head_dim,
                            max_keys, "flk_qk_prologue");
}

int32_t flk_qk_prologue_strided(const float* q_raw, const float* k_raw, const float* v_raw,
                                uint32_t in_stride, const float* gq, const float* gk,
                                const float* inv_freq, float eps, int32_t pairing,
                                float* qn_out, float* kcache, float* vcache, uint32_t n_tokens,
                                uint32_t pos0, uint32_t n_heads, uint32_t n_kv_heads,
                                uint32_t head_dim, uint32_t max_keys) {
  return qk_prologue_common(q_raw, k_raw, v_raw, in_stride, gq, gk, inv_freq, eps, pairing,
                            qn_out, kcache, vcache, n_tokens, pos0, n_heads, n_kv_heads, head_dim,
                            max_keys, "flk_qk_prologue_strided");
}

int32_t flk_attn_decode(const float* q, const float* kcache, const float* vcache, float* o,
                        uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t n_keys,
                        void* ws, uint64_t ws_bytes) {
  FLK_NONNULL(q);
  FLK_NONNULL(kcache);
  FLK_NONNULL(vcache);
  FLK_NONNULL(o);
  FLK_ALIGNED(q);
  FLK_ALIGNED(kcache);
  FLK_ALIGNED(vcache);
  FLK_ALIGNED(o);
  int32_t rc = check_heads(n_heads, n_kv_heads, head_dim);
  if (rc) return rc;
  if (n_keys == 0) return fail(FLK_ERR_ARG, "decode n_keys must be >= 1");
  const DecodeShape s{n_heads, n_kv_heads, head_dim, 1, n_keys};
  rc = check_ws(ws, ws_bytes, decode_ws_bytes(s));
  if (rc) return rc;
  return hip_status(launch_decode(q, kcache, vcache, o, nullptr, nullptr, s, nullptr, ws, g_stream),
                    "flk_attn_decode");
}

int32_t flk_attn_prefill(const float* q, const float* kcache, const float* vcache, float* o,
                         uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t n_queries, uint32_t pos0, void* ws, uint64_t ws_bytes) {
  FLK_NONNULL(q);
  FLK_NONNULL(kcache);
  FLK_NONNULL(vcache);
  FLK_NONNULL(o);
  FLK_ALIGNED(q);
  FLK_ALIGNED(kcache);
  FLK_ALIGNED(vcache);
  FLK_ALIGNED(o);
  int32_t rc = check_heads(n_heads, n_kv_heads, head_dim);
  if (rc) return rc;
  if (n_queries == 0) return fail(FLK_ERR_ARG, "prefill n_queries must be >= 1");
  if ((uint64_t)pos0 + n_queries > 0xFFFFFFFFull)
    return fail(FLK_ERR_ARG, "pos0 + n_queries overflows");
  // The kernel addresses a 64-row key tile with 32-bit byte offsets.
  if ((uint64_t)n_kv_heads * head_dim * 4 * 64 > 0x7FFFFFFFull)
    return fail(FLK_ERR_UNSUPPORTED, "prefill: %u kv heads x %u dims exceed a 64-row tile's 2 GiB",
                n_kv_heads, head_dim);
  const PrefillPlan p = prefill_plan(n_heads, n_kv_heads, head_dim, n_queries, pos0);
  rc = check_ws(ws, ws_bytes, prefill_ws_bytes(p, head_dim));
  if (rc) return rc;
  return hip_status(launch_prefill(q, kcache, vcache, o, n_heads, n_kv_heads, head_dim, n_queries,
                                   pos0, ws, g_stream),
                    "flk_attn_prefill");
}

}  // extern "C"

// ---------------------------------------------------- static split-K scratch ---
// flk_decode_layer_noalloc takes its split-K partials from this array instead
// of a caller workspace, for callers that cannot allocate. Every device the
// library runs on holds its own copy until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in):
// the device address comes from hipGetSymbolAddress, once per device, with
// that device current.
constexpr uint64_t kScratchBytes = 8ull << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
static void* g_scratch_ptr[kScratchDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch array.
static int32_t scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kScratchDevices)
    return fail(FLK_ERR_UNSUPPORTED, "device %d: static scratch is kept for devices 0..%d", dev,
                kScratchDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FLK_OK;
}

// ws == nullptr with use_scratch: the partials go to the static scratch array
// (after every argument check has passed).
static int32_t decode_layer_common(const float* q_raw, const float* k_raw, const float* v_raw,
                                   const float* gq, const float* gk, const float* inv_freq,
                                   float eps, int32_t pairing, float* qn_out, float* kcache,
                                   float* vcache, float* o, uint32_t n_keys,
                                   const uint32_t* n_keys_dev, uint32_t n_heads,
                                   uint32_t n_kv_heads, uint32_t head_dim, void* ws,
                                   uint64_t ws_bytes, const char* what,
                                   bool use_scratch = false) {
  FLK_NONNULL(q_raw);
  FLK_NONNULL(k_raw);
  FLK_NONNULL(v_raw);
  FLK_NONNULL(gq);
  FLK_NONNULL(gk);
  FLK_NONNULL(inv_freq);
  FLK_NONNULL(qn_out);
  FLK_NONNULL(kcache);
  FLK_NONNULL(vcache);
  FLK_NONNULL(o);
  FLK_ALIGNED(q_raw);  // the raw q, k, v rows are read as float4s too
  FLK_ALIGNED(k_raw);
  FLK_ALIGNED(v_raw);
  FLK_ALIGNED(qn_out);
  FLK_ALIGNED(kcache);
  FLK_ALIGNED(vcache);
  FLK_ALIGNED(o);
  int32_t rc = check_heads(n_heads, n_kv_heads, head_dim);
  if (rc) return rc;
  if (pairing != FLK_ROPE_NEOX && pairing != FLK_ROPE_NORM)
    return fail(FLK_ERR_ARG, "rope pairing %d (0 = neox, 1 = norm)", pairing);
  const DecodeShape s{n_heads, n_kv_heads, head_dim, 1, n_keys};
  const uint64_t need = decode_ws_bytes(s);
  if (use_scratch) {
    if (need > kScratchBytes)
      return fail(FLK_ERR_WORKSPACE,
                  "%s: %u heads over %u keys need %llu bytes of split-K scratch; the static "
                  "scratch holds %llu (use flk_decode_layer with a workspace)",
                  what, n_heads, n_keys, (unsigned long long)need,
                  (unsigned long long)kScratchBytes);
    ws_bytes = kScratchBytes;
    if (need > 0) {
      rc = scratch_ptr(&ws);
      if (rc) return rc;
    }
  }
  rc = check_ws(ws, ws_bytes, need);
  if (rc) return rc;
  DecodeFused f;
  f.q_raw = q_raw;
  f.k_raw = k_raw;
  f.v_raw = v_raw;
  f.gq = gq;
  f.gk = gk;
  f.inv_freq = inv_freq;
  f.eps = eps;
  f.pairing = pairing;
  f.qn_out = qn_out;
  f.kcache_w = kcache;
  f.vcache_w = vcache;
  return hip_status(launch_decode(qn_out, kcache, vcache, o, nullptr, n_keys_dev, s, &f, ws,
                                  g_stream),
                    what);
}

extern "C" {

int32_t flk_decode_layer(const float* q_raw, const float* k_raw, const float* v_raw,
                         const float* gq, const float* gk, const float* inv_freq, float eps,
                         int32_t pairing, float* qn_out, float* kcache, float* vcache, float* o,
                         uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t max_keys, void* ws, uint64_t ws_bytes) {
  if (pos >= max_keys) return fail(FLK_ERR_CACHE_FULL, "KV cache full at %u keys", max_keys);
  return decode_layer_common(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps, pairing, qn_out, kcache,
                             vcache, o, pos + 1, nullptr, n_heads, n_kv_heads, head_dim, ws,
                             ws_bytes, "flk_decode_layer");
}

int32_t flk_decode_layer_noalloc(const float* q_raw, const float* k_raw, const float* v_raw,
                                 const float* gq, const float* gk, const float* inv_freq,
                                 float eps, int32_t pairing, float* qn_out, float* kcache,
                                 float* vcache, float* o, uint32_t pos, uint32_t n_heads,
                                 uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_keys) {
  if (pos >= max_keys) return fail(FLK_ERR_CACHE_FULL, "KV cache full at %u keys", max_keys);
  return decode_layer_common(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps, pairing, qn_out, kcache,
                             vcache, o, pos + 1, nullptr, n_heads, n_kv_heads, head_dim, nullptr,
                             0, "flk_decode_layer_noalloc", true);
}

int32_t flk_decode_layer_dev(const float* q_raw, const float* k_raw, const float* v_raw,
                             const float* gq, const float* gk, const float* inv_freq, float eps,
                             int32_t pairing, float* qn_out, float* kcache, float* vcache,
                             float* o, const uint32_t* n_keys_dev, uint32_t n_heads,
                             uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_keys, void* ws,
                             uint64_t ws_bytes) {
  FLK_NONNULL(n_keys_dev);
  if (reinterpret_cast<uintptr_t>(n_keys_dev) % alignof(uint32_t) != 0)
    return fail(FLK_ERR_ARG, "decode_layer_dev: n_keys_dev must be 4-byte aligned");
  if (max_keys == 0) return fail(FLK_ERR_ARG, "decode_layer_dev max_keys 0");
  return decode_layer_common(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps, pairing, qn_out, kcache,
                             vcache, o, max_keys, n_keys_dev, n_heads, n_kv_heads, head_dim, ws,
                             ws_bytes, "flk_decode_layer_dev");
}

}  // extern "C"

// Checks shared by the two ragged entry points (before any launch).
static int32_t check_ragged(const float* kcache, const float* vcache, const uint64_t* seq_row_off,
                            const uint32_t* n_keys, const float* o, uint32_t n_seqs,
                            uint32_t max_n_keys, uint32_t n_heads, uint32_t n_kv_heads,
                            uint32_t head_dim, void* ws, uint64_t ws_bytes, const char* what) {
  FLK_NONNULL(kcache);
  FLK_NONNULL(vcache);
  FLK_NONNULL(seq_row_off);
  FLK_NONNULL(n_keys);
  FLK_NONNULL(o);
  FLK_ALIGNED(kcache);
  FLK_ALIGNED(vcache);
  FLK_ALIGNED(o);
  // The kernels read seq_row_off[b] and n_keys[b] as naturally aligned words.
  if (reinterpret_cast<uintptr_t>(seq_row_off) % alignof(uint64_t) != 0 ||
      reinterpret_cast<uintptr_t>(n_keys) % alignof(uint32_t) != 0)
    return fail(FLK_ERR_ARG, "%s: seq_row_off must be 8-byte aligned and n_keys 4-byte aligned",
                what);
  int32_t rc = check_heads(n_heads, n_kv_heads, head_dim);
  if (rc) return rc;
  if (n_seqs == 0 || max_n_keys == 0)
    return fail(FLK_ERR_ARG, "%s n_seqs=%u max_n_keys=%u", what, n_seqs, max_n_keys);
  if (n_seqs > 65535)
    return fail(FLK_ERR_UNSUPPORTED, "%s n_seqs %u exceeds 65535 (grid z)", what, n_seqs);
  const DecodeShape s{n_heads, n_kv_heads, head_dim, n_seqs, max_n_keys};
  return check_ws(ws, ws_bytes, decode_ws_bytes(s));
}

extern "C" {

int32_t flk_attn_decode_ragged(const float* q, const float* kcache, const float* vcache,
                               const uint64_t* seq_row_off, const uint32_t* n_keys, float* o,
                               uint32_t n_seqs, uint32_t max_n_keys, uint32_t n_heads,
                               uint32_t n_kv_heads, uint32_t head_dim, void* ws,
                               uint64_t ws_bytes) {
  FLK_NONNULL(q);
  FLK_ALIGNED(q);
  int32_t rc = check_ragged(kcache, vcache, seq_row_off, n_keys, o, n_seqs, max_n_keys, n_heads,
                            n_kv_heads, head_dim, ws, ws_bytes, "ragged decode");
  if (rc) return rc;
  const DecodeShape s{n_heads, n_kv_heads, head_dim, n_seqs, max_n_keys};
  return hip_status(
      launch_decode(q, kcache, vcache, o, seq_row_off, n_keys, s, nullptr, ws, g_stream),
      "flk_attn_decode_ragged");
}

int32_t flk_decode_layer_ragged(const float* q_raw, const float* k_raw, const float* v_raw,
                                const float* gq, const float* gk, const float* inv_freq,
                                float eps, int32_t pairing, float* qn_out, float* kcache,
                                float* vcache, const uint64_t* seq_row_off,
                                const uint32_t* n_keys, float* o, uint32_t n_seqs,
                                uint32_t max_n_keys, uint32_t n_heads, uint32_t n_kv_heads,
                                uint32_t head_dim, void* ws, uint64_t ws_bytes) {
  FLK_NONNULL(q_raw);
  FLK_NONNULL(k_raw);
  FLK_NONNULL(v_raw);
  FLK_NONNULL(gq);
  FLK_NONNULL(gk);
  FLK_NONNULL(inv_freq);
  FLK_NONNULL(qn_out);
  FLK_ALIGNED(qn_out);  // the attention launch reads qn as float4s
  if (pairing != FLK_ROPE_NEOX && pairing != FLK_ROPE_NORM)
    return fail(FLK_ERR_ARG, "rope pairing %d (0 = neox, 1 = norm)", pairing);
  int32_t rc = check_ragged(kcache, vcache, seq_row_off, n_keys, o, n_seqs, max_n_keys, n_heads,
                            n_kv_heads, head_dim, ws, ws_bytes, "ragged decode layer");
  if (rc) return rc;
  const DecodeShape s{n_heads, n_kv_heads, head_dim, n_seqs, max_n_keys};
  DecodeFused f;
  f.q_raw = q_raw;
  f.k_raw = k_raw;
  f.v_raw = v_raw;
  f.gq = gq;
  f.gk = gk;
  f.inv_freq = inv_freq;
  f.eps = eps;
  f.pairing = pairing;
  f.qn_out = qn_out;
  f.kcache_w = kcache;
  f.vcache_w = vcache;
  return hip_status(
      launch_decode(qn_out, kcache, vcache, o, seq_row_off, n_keys, s, &f, ws, g_stream),
      "flk_decode_layer_ragged");
}

}  // extern "C"

// ------------------------------------------------------------- Q8_0 -------
int32_t flk_q8_matvec(const int8_t* qs, const uint16_t* scales, const float* x, float* o,
                      uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens) {
  FLK_NONNULL(qs);
  FLK_NONNULL(scales);
  FLK_NONNULL(x);
  FLK_NONNULL(o);
  if (n_rows == 0 || n_cols == 0 || n_tokens == 0)
    return fail(FLK_ERR_ARG, "q8_matvec n_rows=%u n_cols=%u n_tokens=%u", n_rows, n_cols,
                n_tokens);
  if (n_cols % 32 != 0) return fail(FLK_ERR_ARG, "q8_matvec n_cols %u is not a multiple of 32", n_cols);
  if (n_tokens > 65535) return fail(FLK_ERR_UNSUPPORTED, "q8_matvec n_tokens %u > 65535", n_tokens);
  FLK_ALIGNED(qs);
  FLK_ALIGNED(x);
  if (reinterpret_cast<uintptr_t>(scales) % 2 != 0)
    return fail(FLK_ERR_ARG, "scales must be 2-byte aligned");
  return hip_status(launch_q8_matvec(reinterpret_cast<const uint8_t*>(qs), scales, x, o, n_rows,
                                     n_cols, n_tokens, g_stream),
                    "flk_q8_matvec");
}

// ------------------------------------------------------------------ head ---
uint64_t flk_argmax_ws_bytes(uint32_t n) { return argmax_ws_bytes(n > 0 ? n : 1); }

int32_t flk_argmax(const float* x, uint32_t n, float* oval, uint32_t* oidx, void* ws,
                   uint64_t ws_bytes) {
  FLK_NONNULL(x);
  FLK_NONNULL(oval);
  FLK_NONNULL(oidx);
  if (n == 0) return fail(FLK_ERR_ARG, "argmax of an empty vector");
  if (int32_t rc = check_ws(ws, ws_bytes, argmax_ws_bytes(n))) return rc;
  return hip_status(launch_argmax(x, n, oval, oidx, ws, g_stream), "flk_argmax");
}

uint64_t flk_lm_head_ws_bytes(uint32_t vocab, uint32_t hidden) {
  if (vocab == 0 || hidden == 0 || hidden % 32 != 0) return 0;
  return lm_head_ws_bytes(vocab, hidden);
}

int32_t flk_lm_head(const float* x, const float* norm_gain, float eps, const int8_t* qs,
                    const uint16_t* scales, uint32_t vocab, uint32_t hidden, float* normed,
                    float* logits, float* oval, uint32_t* oidx, void* ws, uint64_t ws_bytes) {
  FLK_NONNULL(x);
  FLK_NONNULL(norm_gain);
  FLK_NONNULL(qs);
  FLK_NONNULL(scales);
  FLK_NONNULL(normed);
  FLK_NONNULL(oval);
  FLK_NONNULL(oidx);
  if (vocab == 0 || hidden == 0 || hidden % 32 != 0)
    return fail(FLK_ERR_ARG, "lm_head vocab=%u hidden=%u (hidden a multiple of 32)", vocab, hidden);
  if (!(eps >= 0.f)) return fail(FLK_ERR_ARG, "lm_head eps must be >= 0");
  FLK_ALIGNED(qs);
  FLK_ALIGNED(normed);
  if (reinterpret_cast<uintptr_t>(scales) % 2 != 0)
    return fail(FLK_ERR_ARG, "scales must be 2-byte aligned");
  if (int32_t rc = check_ws(ws, ws_bytes, lm_head_ws_bytes(vocab, hidden))) return rc;
  return hip_status(launch_lm_head(x, norm_gain, eps, reinterpret_cast<const uint8_t*>(qs), scales,
                                   vocab, hidden, normed, logits, oval, oidx, ws, g_stream),
                    "flk_lm_head");
}

int32_t flk_q8_matvec_ex(const int8_t* qs, const uint16_t* scales, const float* x, float* o,
                         uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens,
                         const float* norm_gain, float norm_eps, const float* up,
                         const float* res) {
  FLK_NONNULL(qs);
  FLK_NONNULL(scales);
  FLK_NONNULL(x);
  FLK_NONNULL(o);
  if (n_rows == 0 || n_cols == 0 || n_tokens == 0)
    return fail(FLK_ERR_ARG, "q8_matvec n_rows=%u n_cols=%u n_tokens=%u", n_rows, n_cols,
                n_tokens);
  if (n_cols % 32 != 0) return fail(FLK_ERR_ARG, "q8_matvec n_cols %u is not a multiple of 32", n_cols);
  if (n_tokens > 65535) return fail(FLK_ERR_UNSUPPORTED, "q8_matvec n_tokens %u > 65535", n_tokens);
  if (norm_gain != nullptr && up != nullptr)
    return fail(FLK_ERR_ARG, "q8_matvec_ex: norm_gain and up are exclusive");
  if (norm_gain != nullptr && !(norm_eps >= 0.f))
    return fail(FLK_ERR_ARG, "q8_matvec_ex: eps must be >= 0");
  FLK_ALIGNED(qs);
  FLK_ALIGNED(x);
  if (norm_gain != nullptr) FLK_ALIGNED(norm_gain);
  if (up != nullptr) FLK_ALIGNED(up);
  if (reinterpret_cast<uintptr_t>(scales) % 2 != 0)
    return fail(FLK_ERR_ARG, "scales must be 2-byte aligned");
  Q8Fuse f;
  f.norm_gain = norm_gain;
  f.norm_eps = norm_eps;
  f.up = up;
  f.res = res;
  return hip_status(launch_q8_matvec(reinterpret_cast<const uint8_t*>(qs), scales, x, o, n_rows,
                                     n_cols, n_tokens, g_stream, nullptr, nullptr, nullptr, &f),
                    "flk_q8_matvec_ex");
}

int32_t flk_q8_gate_up_swiglu(const int8_t* qs, const uint16_t* scales, const float* x,
                              float* act, uint32_t n_ffn, uint32_t n_cols, uint32_t n_tokens,
                              const float* norm_gain, float norm_eps) {
  FLK_NONNULL(qs);
  FLK_NONNULL(scales);
  FLK_NONNULL(x);
  FLK_NONNULL(act);
  if (n_ffn == 0 || n_cols == 0 || n_tokens == 0 || n_cols % 32 != 0)
    return fail(FLK_ERR_ARG, "gate_up_swiglu n_ffn=%u n_cols=%u n_tokens=%u", n_ffn, n_cols,
                n_tokens);
  if (n_cols > 1024)
    return fail(FLK_ERR_UNSUPPORTED, "gate_up_swiglu needs n_cols <= 1024 (got %u)", n_cols);
  if (n_tokens > 65535) return fail(FLK_ERR_UNSUPPORTED, "q8_matvec n_tokens %u > 65535", n_tokens);
  if (norm_gain != nullptr && !(norm_eps >= 0.f))
    return fail(FLK_ERR_ARG, "gate_up_swiglu: eps must be >= 0");
  FLK_ALIGNED(qs);
  FLK_ALIGNED(x);
  if (norm_gain != nullptr) FLK_ALIGNED(norm_gain);
  if (reinterpret_cast<uintptr_t>(scales) % 2 != 0)
    return fail(FLK_ERR_ARG, "scales must be 2-byte aligned");
  Q8Fuse f;
  f.norm_gain = norm_gain;
  f.norm_eps = norm_eps;
  f.act = act;
  return hip_status(launch_q8_matvec(reinterpret_cast<const uint8_t*>(qs), scales, x, nullptr,
                                     2 * n_ffn, n_cols, n_tokens, g_stream, nullptr, nullptr,
                                     nullptr, &f),
                    "flk_q8_gate_up_swiglu");
}

int32_t flk_swiglu(const float* gate, const float* up, float* o, uint32_t n) {
  FLK_NONNULL(gate);
  FLK_NONNULL(up);
  FLK_NONNULL(o);
  if (n == 0) return fail(FLK_ERR_ARG, "swiglu of 0 elements");
  return hip_status(launch_elementwise(0, gate, up, o, n, g_stream), "flk_swiglu");
}

int32_t flk_add(const float* a, const float* b, float* o, uint32_t n) {
  FLK_NONNULL(a);
  FLK_NONNULL(b);
  FLK_NONNULL(o);
  if (n == 0) return fail(FLK_ERR_ARG, "add of 0 elements");
  return hip_status(launch_elementwise(1, a, b, o, n, g_stream), "flk_add");
}

// splitQ8, kernels/lib.ts:141-156 (host memory only).
int32_t flk_q8_split(const uint8_t* packed, uint32_t n_rows, uint32_t n_cols, int8_t* qs,
                     uint16_t* scales) {
  FLK_NONNULL(packed);
  FLK_NONNULL(qs);
  FLK_NONNULL(scales);
  if (n_rows == 0 || n_cols == 0 || n_cols % 32 != 0)
    return fail(FLK_ERR_ARG, "q8_split n_rows=%u n_cols=%u (n_cols a multiple of 32)", n_rows,
                n_cols);
  const uint32_t nb = n_cols / 32;
  for (uint32_t r = 0; r < n_rows; r++)
    for (uint32_t b = 0; b < nb; b++) {
      const uint8_t* src = packed + ((uint64_t)r * nb + b) * 34;
      scales[(uint64_t)r * nb + b] = (uint16_t)(src[0] | (src[1] << 8));
      memcpy(qs + (uint64_t)r * n_cols + (uint64_t)b * 32, src + 2, 32);
    }
  return FLK_OK;
}

// ------------------------------------------------------------------ wire ---
int32_t flk_f32_to_f16(const float* in, uint16_t* out, uint64_t n) {
  FLK_NONNULL(in);
  FLK_NONNULL(out);
  if (n == 0) return FLK_OK;
  return hip_status(launch_wire(0, in, out, n, g_stream), "flk_f32_to_f16");
}

int32_t flk_f16_to_f32(const uint16_t* in, float* out, uint64_t n) {
  FLK_NONNULL(in);
  FLK_NONNULL(out);
  if (n == 0) return FLK_OK;
  return hip_status(launch_wire(1, in, out, n, g_stream), "flk_f16_to_f32");
}

static void put_u32(uint8_t* p, uint32_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
  p[2] = (uint8_t)(v >> 16);
  p[3] = (uint8_t)(v >> 24);
}

static uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// pack (wire.mjs:66-78): magic, seq, hidden, offset, flags, little-endian.
int32_t flk_wire_header_pack(uint32_t seq, uint32_t hidden, uint32_t offset, uint32_t flags,
                             void* out20) {
  FLK_NONNULL(out20);
  uint8_t* p = static_cast<uint8_t*>(out20);
  put_u32(p, FLK_WIRE_MAGIC);
  put_u32(p + 4, seq);
  put_u32(p + 8, hidden);
  put_u32(p + 12, offset);
  put_u32(p + 16, flags & (FLK_WIRE_RESET | FLK_WIRE_REPLAY));
  return FLK_OK;
}

// unpack's header (wire.mjs:80-88).
int32_t flk_wire_header_unpack(const void* frame, uint64_t frame_bytes, uint32_t* seq,
                               uint32_t* hidden, uint32_t* offset, uint32_t* flags,
                               uint64_t* n_values) {
  FLK_NONNULL(frame);
  const uint8_t* p = static_cast<const uint8_t*>(frame);
  if (frame_bytes < FLK_WIRE_HEADER_BYTES || get_u32(p) != FLK_WIRE_MAGIC)
    return fail(FLK_ERR_ARG, "not a flock frame");
  if (seq) *seq = get_u32(p + 4);
  if (hidden) *hidden = get_u32(p + 8);
  if (offset) *offset = get_u32(p + 12);
  if (flags) *flags = get_u32(p + 16);
  if (n_values) *n_values = (frame_bytes - FLK_WIRE_HEADER_BYTES) / 2;
  return FLK_OK;
}

// ----------------------------------------------------------------- graph ---
int32_t flk_embed(const int8_t* qs, const uint16_t* scales, const uint32_t* ids,
                  uint32_t n_tokens, uint32_t vocab, uint32_t hidden, float* out) {
  FLK_NONNULL(qs);
  FLK_NONNULL(scales);
  FLK_NONNULL(ids);
  FLK_NONNULL(out);
  if (n_tokens == 0 || vocab == 0 || hidden == 0 || hidden % 32 != 0)
    return fail(FLK_ERR_ARG, "embed n_tokens=%u vocab=%u hidden=%u (a multiple of 32)", n_tokens,
                vocab, hidden);
  if (reinterpret_cast<uintptr_t>(qs) % 4 != 0 || reinterpret_cast<uintptr_t>(scales) % 2 != 0)
    return fail(FLK_ERR_ARG, "embed: qs must be 4-byte and scales 2-byte aligned");
  FLK_ALIGNED(out);
  return hip_status(launch_embed(qs, scales, ids, n_tokens, vocab, hidden, out, g_stream),
                    "flk_embed");
}

int32_t flk_advance(uint32_t* state, uint32_t delta, const uint32_t* value, uint32_t* log,
                    uint32_t log_len) {
  FLK_NONNULL(state);
  return hip_status(launch_advance(state, delta, value, log, log_len, g_stream), "flk_advance");
}

int32_t flk_stream_create(void** stream) {
  FLK_NONNULL(stream);
  hipStream_t s = nullptr;
  int32_t rc = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = rc ? nullptr : s;
  return rc;
}

int32_t flk_stream_destroy(void* stream) {
  if (stream == nullptr) return FLK_OK;
  if (g_stream == static_cast<hipStream_t>(stream)) g_stream = nullptr;
  return hip_status(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
}

int32_t flk_capture_begin(void) {
  if (g_stream == nullptr)
    return fail(FLK_ERR_ARG, "capture needs a stream (flk_set_stream), not the null stream");
  return hip_status(hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed),
                    "hipStreamBeginCapture");
}

int32_t flk_capture_end(void** graph) {
  FLK_NONNULL(graph);
  *graph = nullptr;
  hipGraph_t g = nullptr;
  int32_t rc = hip_status(hipStreamEndCapture(g_stream, &g), "hipStreamEndCapture");
  if (rc) return rc;
  hipGraphExec_t exec = nullptr;
  rc = hip_status(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  (void)hipGraphDestroy(g);  // the executable graph keeps what it needs
  if (rc) return rc;
  *graph = exec;
  return FLK_OK;
}

int32_t flk_graph_launch(void* graph) {
  FLK_NONNULL(graph);
  return hip_status(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), g_stream),
                    "hipGraphLaunch");
}

int32_t flk_graph_destroy(void* graph) {
  if (graph == nullptr) return FLK_OK;
  return hip_status(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)), "hipGraphExecDestroy");
}
