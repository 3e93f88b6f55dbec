// Per-head RMSNorm + RoPE + K/V append, and the unfused rmsnorm / rope / append
// ops. These are bytes-trivial kernels (a few KB per token); their job is to
// be bit-exact with the CPU oracle so that the KV cache a prefill writes is the
// cache N decode steps write (test_prefill.ts:119-132).
#include "common.hpp"

namespace flk {

// ------------------------------------------------------------ rmsnorm (any n)
// rmsnorm.wgsl:41-73: one 128-thread workgroup per vector; thread t sums a
// stride-128 slice with fma32, then a pairwise LDS tree (strides 64 .. 1).
__global__ __launch_bounds__(128) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ g,
                                                      float* __restrict__ o, uint32_t n,
                                                      uint32_t n_vecs, float eps) {
  __shared__ float part[128];
  const uint32_t vec = blockIdx.x;
  const uint32_t t = threadIdx.x;
  if (vec >= n_vecs) return;  // uniform per block
  const float* xv = x + (size_t)vec * n;
  float acc = 0.f;
  // Eight elements are loaded before any is used; past the end they read 0,
  // which adds exactly nothing to the partial.
  for (uint32_t base = t; base < n; base += 128 * 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t i = base + 128 * k;
      v[k] = xv[min(i, n - 1)];
      v[k] = i < n ? v[k] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; k++) acc = fma32(v[k], v[k], acc);
  }
  part[t] = acc;
  __syncthreads();
  for (uint32_t stride = 64; stride > 0; stride >>= 1) {
    if (t < stride) part[t] = part[t] + part[t + stride];
    __syncthreads();
  }
  const float mean = part[0] / (float)n;
  const float scale = rsqrt_once(mean + eps);
  float* ov = o + (size_t)vec * n;
  for (uint32_t i = t; i < n; i += 128) ov[i] = (xv[i] * scale) * g[i];
}

hipError_t launch_rmsnorm(const float* x, const float* g, float* o, uint32_t n, uint32_t n_vecs,
                          float eps, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_vecs), dim3(128), 0, st, x, g, o, n, n_vecs, eps);
  return hipGetLastError();
}

// ------------------------------------------------------------- rope (any d)
// rope.wgsl:50-78: one thread per rotated pair, in place.
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ x,
                                                   const float* __restrict__ inv_freq,
                                                   uint32_t n_tokens, uint32_t n_heads,
                                                   uint32_t head_dim, uint32_t pos0,
                                                   int32_t pairing) {
  const uint32_t half = head_dim / 2;
  const uint64_t total = (uint64_t)n_tokens * n_heads * half;
  const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= total) return;
  const uint32_t j = (uint32_t)(gid % half);
  const uint32_t head = (uint32_t)((gid / half) % n_heads);
  const uint32_t token = (uint32_t)(gid / ((uint64_t)half * n_heads));
  const size_t base = ((size_t)token * n_heads + head) * head_dim;
  const size_t ia = base + (pairing == FLK_ROPE_NORM ? 2 * j : j);
  const size_t ib = base + (pairing == FLK_ROPE_NORM ? 2 * j + 1 : j + half);
  const float a = x[ia], b = x[ib];
  const uint32_t pos = pos0 + token;
  const float2 cs = rope_cos_sin(inv_freq[j], pos);
  x[ia] = rope_rot(a, b, true, cs);
  x[ib] = rope_rot(b, a, false, cs);
}

hipError_t launch_rope(float* x, const float* inv_freq, uint32_t n_tokens, uint32_t n_heads,
                       uint32_t head_dim, uint32_t pos0, int32_t pairing, hipStream_t st) {
  const uint64_t total = (uint64_t)n_tokens * n_heads * (head_dim / 2);
  const uint32_t blocks = (uint32_t)((total + 255) / 256);
  hipLaunchKernelGGL(rope_kernel, dim3(blocks), dim3(256), 0, st, x, inv_freq, n_tokens, n_heads,
                     head_dim, pos0, pairing);
  return hipGetLastError();
}

// ---------------------------------------------------------------- append ----
// layer.ts:616-622 / 737-741: both caches are [key][kv_head][head_dim], so n
// tokens of new rows are one contiguous run at row pos0.
hipError_t launch_kv_append(const float* kn, const float* v, float* kcache, float* vcache,
                            uint32_t n_tokens, uint32_t pos0, uint32_t n_kv_heads,
                            uint32_t head_dim, hipStream_t st) {
  const size_t row = (size_t)n_kv_heads * head_dim;
  const size_t bytes = (size_t)n_tokens * row * sizeof(float);
  hipError_t e = hipMemcpyAsync(kcache + (size_t)pos0 * row, kn, bytes, hipMemcpyDeviceToDevice, st);
  if (e != hipSuccess) return e;
  return hipMemcpyAsync(vcache + (size_t)pos0 * row, v, bytes, hipMemcpyDeviceToDevice, st);
}

// --------------------------------------------------------- fused prologue ----
// One workgroup per token (every head of a token shares its position): the
// first D/2 threads put cos/sin of the token's D/2 RoPE angles in LDS, then
// each wave takes head vectors. Vector id -> kind: the first n_heads are q
// heads (norm + rope -> qn_out), the next n_kv_heads are k heads (norm + rope
// -> kcache row pos0 + token), the last n_kv_heads are v heads (copied raw to
// vcache). Identical arithmetic to rmsnorm_kernel + rope_kernel for head_dim
// vectors, so the caches match the unfused path bit for bit.
//
// Ragged batches (RAGGED, flk_decode_layer_ragged): "token" b is sequence b's
// new token. Its position is n_keys[b] - 1 and its cache row is seq_row_off[b]
// + n_keys[b] - 1. A sequence with n_keys[b] == 0 is idle (its qn rows are
// zeroed, nothing is appended); one with n_keys[b] > max_n_keys is refused on
// the device (qn rows NaN, nothing appended: the attention launch after it
// fills that sequence's o with NaN too). Workgroup 0 also zeroes the
// n_queue item counters of the batch decode kernel that follows on the
// stream, so the ragged step needs no separate reset launch.
constexpr int kPrologueThreads = 256;

struct RaggedTokens {
  const uint32_t* n_keys = nullptr;       // [n_seqs]
  const uint64_t* seq_row_off = nullptr;  // [n_seqs]
  uint32_t max_n_keys = 0;
  uint32_t* queue = nullptr;              // item counters to zero (or null)
  uint32_t n_queue = 0;
};

template <int D, bool RAGGED>
__global__ __launch_bounds__(kPrologueThreads) void qk_prologue_kernel(
    const float* __restrict__ q_raw, const float* __restrict__ k_raw,
    const float* __restrict__ v_raw, const float* __restrict__ gq, const float* __restrict__ gk,
    const float* __restrict__ inv_freq, float eps, int32_t pairing, float* __restrict__ qn_out,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t pos0, uint32_t n_heads,
    uint32_t n_kv_heads, uint32_t q_stride, uint32_t kv_stride, RaggedTokens rt) {
  __shared__ float2 s_cs[D / 2];
  const int lane = threadIdx.x & 63;
  // The wave index in a scalar register: the compiler then knows each vector
  // index is wave-uniform, so locate()'s branches and row addresses are scalar
  // work instead of exec-masked vector code.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t tok = blockIdx.x;
  uint32_t pos = pos0 + tok;
  uint64_t cache_row = pos;
  if constexpr (RAGGED) {
    if (tok == 0 && threadIdx.x < rt.n_queue) rt.queue[threadIdx.x] = 0u;
    const uint32_t nk = rt.n_keys[tok];
    if (nk == 0 || nk > rt.max_n_keys) {  // idle (zeros) or refused (NaN): no append
      const float fill = nk == 0 ? 0.f : __builtin_nanf("");
      float* dq = qn_out + (size_t)tok * n_heads * D;
      for (uint32_t i = threadIdx.x; i < n_heads * D; i += kPrologueThreads) dq[i] = fill;
      return;  // uniform per workgroup
    }
    pos = nk - 1;
    cache_row = rt.seq_row_off[tok] + pos;
  }
  const uint32_t per_tok = n_heads + 2 * n_kv_heads;
  const size_t kv_row = (size_t)n_kv_heads * D;
  // Vector idx -> (source, destination, gain): q heads, then k heads, then v.
  auto locate = [&](uint32_t idx, const float*& src, float*& dst, const float*& g) {
    g = nullptr;
    if (idx < n_heads) {
      src = q_raw + (size_t)tok * q_stride + (size_t)idx * D;
      dst = qn_out + ((size_t)tok * n_heads + idx) * D;
      g = gq;
    } else if (idx < n_heads + n_kv_heads) {
      const uint32_t h = idx - n_heads;
      src = k_raw + (size_t)tok * kv_stride + (size_t)h * D;
      dst = kcache + cache_row * kv_row + (size_t)h * D;
      g = gk;
    } else {
      const uint32_t h = idx - n_heads - n_kv_heads;
      src = v_raw + (size_t)tok * kv_stride + (size_t)h * D;
      dst = vcache + cache_row * kv_row + (size_t)h * D;
    }
  };
  // Each wave takes vectors wave, wave + 4, ...; a batch of kBatch vectors is
  // loaded before any is used, so their memory latency overlaps. The first
  // batch is requested before the cos/sin table is computed.
  constexpr int kWaves = kPrologueThreads / 64;
  constexpr int kBatch = 8;
  float e0[kBatch], e1[kBatch];
  auto load_batch = [&](uint32_t base) {
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const uint32_t idx = min(base + kWaves * b, per_tok - 1);  // extras reload the last
      const float* src;
      float* dst;
      const float* g;
      locate(idx, src, dst, g);
      e0[b] = src[lane];
      e1[b] = D == 128 ? src[lane + 64] : 0.f;
    }
  };
  // Loads retire in issue order: inv_freq first, so the table waits for it alone.
  const float invf = inv_freq[min((int)threadIdx.x, D / 2 - 1)];
  load_batch(wave);
  const float gq0 = gq[lane], gq1 = D == 128 ? gq[lane + 64] : 0.f;
  const float gk0 = gk[lane], gk1 = D == 128 ? gk[lane + 64] : 0.f;
  if (threadIdx.x < D / 2) s_cs[threadIdx.x] = rope_cos_sin(invf, pos);
  __syncthreads();

  for (uint32_t base = wave; base < per_tok; base += kWaves * kBatch) {
    if (base != (uint32_t)wave) load_batch(base);
    // The batch's norm scales (head_rmsnorm's arithmetic): every vector's
    // sum of squares by the tree, then lane b evaluates vector b's
    // 1 / sqrt(mean + eps) -- one f64 sequence for the batch instead of one
    // per vector -- and each vector reads its scale back from lane b.
    float mine = 0.f;
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      float p = e0[b] * e0[b];
      if (D == 128) p = p + e1[b] * e1[b];
      p = tree_sum64(p);
      mine = (lane & (kBatch - 1)) == b ? p : mine;
    }
    const float scale_mine = rsqrt_once(mine / (float)D + eps);
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const uint32_t idx = base + kWaves * b;
      if (idx >= per_tok) continue;  // uniform per wave
      const float* src;
      float* dst;
      const float* g;
      locate(idx, src, dst, g);
      float x0 = e0[b], x1 = e1[b];
      if (g != nullptr) {  // uniform per wave
        const bool is_q = idx < n_heads;
        const float scale =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, scale_mine), b));
        x0 = (x0 * scale) * (is_q ? gq0 : gk0);
        if (D == 128) x1 = (x1 * scale) * (is_q ? gq1 : gk1);
        head_rope<D>(x0, x1, s_cs, pairing, lane);
      }
      dst[lane] = x0;
      if (D == 128) dst[lane + 64] = x1;
    }
  }
}

hipError_t launch_qk_prologue(const float* q_raw, const float* k_raw, const float* v_raw,
                              const float* gq, const float* gk, const float* inv_freq, float eps,
                              int32_t pairing, float* qn_out, float* kcache, float* vcache,
                              uint32_t n_tokens, uint32_t pos0, uint32_t n_heads,
                              uint32_t n_kv_heads, uint32_t head_dim, hipStream_t st,
                              uint32_t in_stride) {
  // Raw rows of consecutive tokens: packed, or in_stride floats apart.
  const uint32_t q_stride = in_stride ? in_stride : n_heads * head_dim;
  const uint32_t kv_stride = in_stride ? in_stride : n_kv_heads * head_dim;
  const RaggedTokens none{};
  if (head_dim == 128)
    hipLaunchKernelGGL((qk_prologue_kernel<128, false>), dim3(n_tokens), dim3(kPrologueThreads), 0,
                       st, q_raw, k_raw, v_raw, gq, gk, inv_freq, eps, pairing, qn_out, kcache,
                       vcache, pos0, n_heads, n_kv_heads, q_stride, kv_stride, none);
  else
    hipLaunchKernelGGL((qk_prologue_kernel<64, false>), dim3(n_tokens), dim3(kPrologueThreads), 0,
                       st, q_raw, k_raw, v_raw, gq, gk, inv_freq, eps, pairing, qn_out, kcache,
                       vcache, pos0, n_heads, n_kv_heads, q_stride, kv_stride, none);
  return hipGetLastError();
}

hipError_t launch_ragged_prologue(const DecodeFused& f, const uint64_t* seq_row_off,
                                  const uint32_t* n_keys, uint32_t n_seqs, uint32_t max_n_keys,
                                  uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                  uint32_t* queue, uint32_t n_queue, hipStream_t st) {
  RaggedTokens rt;
  rt.n_keys = n_keys;
  rt.seq_row_off = seq_row_off;
  rt.max_n_keys = max_n_keys;
  rt.queue = queue;
  rt.n_queue = queue != nullptr ? n_queue : 0;
  const uint32_t q_stride = n_heads * head_dim, kv_stride = n_kv_heads * head_dim;
  if (head_dim == 128)
    hipLaunchKernelGGL((qk_prologue_kernel<128, true>), dim3(n_seqs), dim3(kPrologueThreads), 0,
                       st, f.q_raw, f.k_raw, f.v_raw, f.gq, f.gk, f.inv_freq, f.eps, f.pairing,
                       f.qn_out, f.kcache_w, f.vcache_w, 0u, n_heads, n_kv_heads, q_stride,
                       kv_stride, rt);
  else
    hipLaunchKernelGGL((qk_prologue_kernel<64, true>), dim3(n_seqs), dim3(kPrologueThreads), 0,
                       st, f.q_raw, f.k_raw, f.v_raw, f.gq, f.gk, f.inv_freq, f.eps, f.pairing,
                       f.qn_out, f.kcache_w, f.vcache_w, 0u, n_heads, n_kv_heads, q_stride,
                       kv_stride, rt);
  return hipGetLastError();
}

}  // namespace flk
