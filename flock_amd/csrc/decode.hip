// GQA decode attention (one query per head) as split-K flash-decoding.
//
// The reference kernel (attention.wgsl:58-122) runs one 128-thread workgroup
// per q-head and holds every score in workgroup memory, which caps context at
// $MAX_KEYS and leaves the GPU with 16 workgroups. Here two launches:
//
// decode_split_kernel  grid (n_kv_heads, n_splits, n_seqs), 256 threads.
//   One workgroup streams keys [t0, t1) of one kv head and serves all G =
//   n_heads / n_kv_heads query heads that read it, so each K/V byte is read
//   from HBM once. Each K/V row of one kv head (D floats) is loaded by D/4
//   lanes as float4 -- one coalesced 512 B segment for D = 128 -- so a
//   workgroup has 256 / (D/4) "slots", slot s taking keys t0 + s, t0 + s +
//   SLOTS, ..., and U keys per slot are in flight per iteration.
//   Scores: per-lane float4 dot, then a DPP/swizzle sum over the row's lanes;
//   online softmax (running max m, denominator l, unnormalised accumulator)
//   per slot; the slots merge through LDS. A single-split row writes o
//   directly, otherwise the workgroup writes its (m, l, acc) partial.
// decode_merge_kernel  grid (n_heads, n_seqs), 256 threads: combines the
//   partials of one head with log-sum-exp weights (rows of a single split exit).
// The two launches are ordered by the stream: no atomics or device-scope fences
// inside a launch.
//
// Fused mode (flk_decode_layer) prepends Layer.encode's prologue
// (layer.ts:598-622): every workgroup recomputes q's per-head RMSNorm + RoPE
// for its G heads (a few hundred flops), and the workgroup whose key range
// holds position pos also normalises/rotates the new k row and writes k and v
// into the cache before streaming keys.
#include <float.h>

#include "common.hpp"

namespace flk {

struct DecodeArgs {
  const float* q;
  const float* kcache;
  const float* vcache;
  float* o;
  const uint64_t* seq_row_off;  // ragged only
  const uint32_t* n_keys_dev;   // ragged only
  uint32_t n_keys;              // single sequence (ragged: the bound max_n_keys)
  uint32_t n_heads, n_kv_heads;
  uint32_t kps;                 // keys per split
  uint32_t max_splits;
  float scale;
  float2* part_ml;              // [seq][head][split] (m, l)
  float* part_acc;              // [seq][head][split][D]
  // fused prologue (q_raw != nullptr)
  const float* q_raw;
  const float* k_raw;
  const float* v_raw;
  const float* gq;
  const float* gk;
  const float* inv_freq;
  float eps;
  int32_t pairing;
  float* qn_out;
  float* kcache_w;
  float* vcache_w;
};

// Launch-shape tunables (compile-time; the defaults are the measured choice).
#ifndef FLK_DECODE_UNROLL
#define FLK_DECODE_UNROLL 8
#endif
#ifndef FLK_DECODE_TARGET_WG
#define FLK_DECODE_TARGET_WG 1024
#endif
constexpr int kDecodeThreads = 256;
constexpr int kDecodeUnroll = FLK_DECODE_UNROLL;
constexpr int kMergeThreads = 256;

// Keys sequence `seq` attends: the argument for one sequence; for a ragged
// batch its n_keys entry, clamped to the planned bound so that the grid covers
// every split (n_keys == 0 marks an empty sequence).
__device__ __forceinline__ uint32_t seq_keys(const DecodeArgs& a, uint32_t seq) {
  return a.n_keys_dev != nullptr ? min(a.n_keys_dev[seq], a.n_keys) : a.n_keys;
}

template <int D, int G>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_kernel(DecodeArgs a) {
  constexpr int LPK = D / 4;                    // lanes per key row
  constexpr int SLOTS = kDecodeThreads / LPK;   // concurrent keys per workgroup
  constexpr int U = kDecodeUnroll;
  constexpr int NT = G * LPK;                   // (head, float4 column) items

  __shared__ float4 s_q[G][LPK];
  __shared__ float s_m[SLOTS][G];
  __shared__ float s_l[SLOTS][G];
  __shared__ float4 s_acc[SLOTS][G][LPK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slot = tid / LPK;
  const int sl = tid % LPK;
  const uint32_t kvh = blockIdx.x;
  const uint32_t split = blockIdx.y;
  const uint32_t seq = blockIdx.z;
  const uint32_t h0 = kvh * G;  // first q head of this group

  const uint32_t n_keys = seq_keys(a, seq);
  const uint64_t row0 = a.seq_row_off != nullptr ? a.seq_row_off[seq] : 0;
  if (n_keys == 0) {  // empty ragged sequence: zero output rows
    if (split == 0)
      for (int i = tid; i < G * D; i += kDecodeThreads)
        a.o[((size_t)seq * a.n_heads + h0) * D + i] = 0.f;
    return;
  }
  const uint32_t n_splits = (n_keys + a.kps - 1) / a.kps;
  if (split >= n_splits) return;  // uniform per workgroup
  const uint32_t t0 = split * a.kps;
  const uint32_t t1 = min(t0 + a.kps, n_keys);
  const size_t row = (size_t)a.n_kv_heads * D;  // floats per cache row

  // ---- q for the G heads (fused: prologue computed here) -------------------
  if (a.q_raw != nullptr) {
    const uint32_t pos = n_keys - 1;
    const bool owns_pos = pos >= t0 && pos < t1;
    const int n_vec = G + (owns_pos ? 2 : 0);
    for (int vi = wave; vi < n_vec; vi += kDecodeThreads / 64) {
      float e0, e1;
      if (vi < G) {  // q head h0 + vi
        const float* src = a.q_raw + (size_t)(h0 + vi) * D;
        e0 = lane < D ? src[lane] : 0.f;
        e1 = D == 128 ? src[lane + 64] : 0.f;
        head_rmsnorm<D>(e0, e1, a.gq, lane, a.eps);
        head_rope<D>(e0, e1, a.inv_freq, (int)pos, a.pairing, lane);
        float* sq = reinterpret_cast<float*>(&s_q[vi][0]);
        if (lane < D) sq[lane] = e0;
        if (D == 128) sq[lane + 64] = e1;
        if (split == 0) {
          float* dq = a.qn_out + (size_t)(h0 + vi) * D;
          if (lane < D) dq[lane] = e0;
          if (D == 128) dq[lane + 64] = e1;
        }
      } else if (vi == G) {  // new k row of this kv head -> kcache[pos]
        const float* src = a.k_raw + (size_t)kvh * D;
        e0 = lane < D ? src[lane] : 0.f;
        e1 = D == 128 ? src[lane + 64] : 0.f;
        head_rmsnorm<D>(e0, e1, a.gk, lane, a.eps);
        head_rope<D>(e0, e1, a.inv_freq, (int)pos, a.pairing, lane);
        float* dk = a.kcache_w + (size_t)pos * row + (size_t)kvh * D;
        if (lane < D) dk[lane] = e0;
        if (D == 128) dk[lane + 64] = e1;
      } else {  // new v row, raw
        const float* src = a.v_raw + (size_t)kvh * D;
        float* dv = a.vcache_w + (size_t)pos * row + (size_t)kvh * D;
        if (lane < D) dv[lane] = src[lane];
        if (D == 128) dv[lane + 64] = src[lane + 64];
      }
    }
  } else {
    for (int i = tid; i < NT; i += kDecodeThreads) {
      const int g = i / LPK, c = i % LPK;
      s_q[g][c] = reinterpret_cast<const float4*>(a.q + ((size_t)seq * a.n_heads + h0 + g) * D)[c];
    }
  }
  __syncthreads();  // s_q ready; fused cache writes visible to this workgroup

  float4 qv[G];
#pragma unroll
  for (int g = 0; g < G; g++) qv[g] = s_q[g][sl];

  float m[G], l[G];
  float4 acc[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.f;
    acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const float4* kb = reinterpret_cast<const float4*>(a.kcache + row0 * row + (size_t)kvh * D) + sl;
  const float4* vb = reinterpret_cast<const float4*>(a.vcache + row0 * row + (size_t)kvh * D) + sl;
  const size_t row4 = row / 4;

  for (uint32_t base = t0; base < t1; base += SLOTS * U) {
    float4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t t = base + u * SLOTS + slot;
      if (t < t1) {
        kr[u] = kb[(size_t)t * row4];
        vr[u] = vb[(size_t)t * row4];
      } else {
        kr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        vr[u] = kr[u];
      }
    }
    float s[G][U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const bool valid = base + u * SLOTS + slot < t1;
#pragma unroll
      for (int g = 0; g < G; g++) {
        float d = qv[g].x * kr[u].x;
        d = fmaf(qv[g].y, kr[u].y, d);
        d = fmaf(qv[g].z, kr[u].z, d);
        d = fmaf(qv[g].w, kr[u].w, d);
        d = group_sum<LPK>(d);
        s[g][u] = valid ? d * a.scale : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      float cm = s[g][0];
#pragma unroll
      for (int u = 1; u < U; u++) cm = fmaxf(cm, s[g][u]);
      const float mn = fmaxf(m[g], cm);
      if (mn == -INFINITY) continue;  // no valid key yet in this slot
      const float corr = expf(m[g] - mn);
      l[g] *= corr;
      acc[g].x *= corr;
      acc[g].y *= corr;
      acc[g].z *= corr;
      acc[g].w *= corr;
#pragma unroll
      for (int u = 0; u < U; u++) {
        const float e = expf(s[g][u] - mn);
        l[g] += e;
        acc[g].x = fmaf(e, vr[u].x, acc[g].x);
        acc[g].y = fmaf(e, vr[u].y, acc[g].y);
        acc[g].z = fmaf(e, vr[u].z, acc[g].z);
        acc[g].w = fmaf(e, vr[u].w, acc[g].w);
      }
      m[g] = mn;
    }
  }

  // ---- merge the slots of this workgroup --------------------------------
  if (sl == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      s_m[slot][g] = m[g];
      s_l[slot][g] = l[g];
    }
  }
#pragma unroll
  for (int g = 0; g < G; g++) s_acc[slot][g][sl] = acc[g];
  __syncthreads();

  for (int i = tid; i < NT; i += kDecodeThreads) {
    const int g = i / LPK, c = i % LPK;
    float M = -INFINITY;
    for (int s = 0; s < SLOTS; s++) M = fmaxf(M, s_m[s][g]);
    float L = 0.f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < SLOTS; s++) {
      const float ms = s_m[s][g];
      const float w = ms == -INFINITY ? 0.f : expf(ms - M);
      L = fmaf(s_l[s][g], w, L);
      const float4 as = s_acc[s][g][c];
      A.x = fmaf(as.x, w, A.x);
      A.y = fmaf(as.y, w, A.y);
      A.z = fmaf(as.z, w, A.z);
      A.w = fmaf(as.w, w, A.w);
    }
    if (n_splits == 1) {
      const float4 r = make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
      reinterpret_cast<float4*>(a.o + ((size_t)seq * a.n_heads + h0 + g) * D)[c] = r;
    } else {
      const size_t p = ((size_t)seq * a.n_heads + h0 + g) * a.max_splits + split;
      if (c == 0) a.part_ml[p] = make_float2(M, L);
      reinterpret_cast<float4*>(a.part_acc + p * D)[c] = A;
    }
  }
}

// One workgroup per (head, sequence). Thread -> (group, float4 column): group
// r folds splits r, r + GROUPS, ... with weights exp(m_s - M) against the
// global max M; the groups then add up through LDS in a fixed order, so the
// result does not depend on scheduling.
template <int D>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(DecodeArgs a) {
  constexpr int LPK = D / 4;
  constexpr int GROUPS = kMergeThreads / LPK;
  __shared__ float s_max[GROUPS];
  __shared__ float s_l[GROUPS];
  __shared__ float4 s_acc[GROUPS][LPK];

  const uint32_t head = blockIdx.x;
  const uint32_t seq = blockIdx.y;
  const uint32_t n_keys = seq_keys(a, seq);
  const uint32_t n_splits = (n_keys + a.kps - 1) / a.kps;
  if (n_splits <= 1) return;  // written by the split kernel (or empty)
  const int tid = threadIdx.x;
  const int grp = tid / LPK, c = tid % LPK;
  const size_t p0 = ((size_t)seq * a.n_heads + head) * a.max_splits;

  float M = -INFINITY;
  for (uint32_t s = grp; s < n_splits; s += GROUPS) M = fmaxf(M, a.part_ml[p0 + s].x);
  if (c == 0) s_max[grp] = M;
  __syncthreads();
  M = s_max[0];
#pragma unroll
  for (int r = 1; r < GROUPS; r++) M = fmaxf(M, s_max[r]);

  float L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s = grp; s < n_splits; s += GROUPS) {
    const float2 ml = a.part_ml[p0 + s];
    const float w = ml.x == -INFINITY ? 0.f : expf(ml.x - M);
    const float4 p = reinterpret_cast<const float4*>(a.part_acc + (p0 + s) * D)[c];
    L = fmaf(ml.y, w, L);
    A.x = fmaf(p.x, w, A.x);
    A.y = fmaf(p.y, w, A.y);
    A.z = fmaf(p.z, w, A.z);
    A.w = fmaf(p.w, w, A.w);
  }
  if (c == 0) s_l[grp] = L;
  s_acc[grp][c] = A;
  __syncthreads();
  if (grp != 0) return;
  L = s_l[0];
  A = s_acc[0][c];
#pragma unroll
  for (int r = 1; r < GROUPS; r++) {
    L += s_l[r];
    const float4 p = s_acc[r][c];
    A.x += p.x;
    A.y += p.y;
    A.z += p.z;
    A.w += p.w;
  }
  reinterpret_cast<float4*>(a.o + ((size_t)seq * a.n_heads + head) * D)[c] =
      make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
}

// ------------------------------------------------------------------ plan ----
// Keys per split: aim for ~kTargetWG split workgroups in total (several per CU
// so that enough 512 B rows are in flight to cover HBM latency), in multiples
// of one loop iteration (SLOTS * U keys), and at least kMinKps keys.
constexpr uint32_t kTargetWG = FLK_DECODE_TARGET_WG;
constexpr uint32_t kMinKps = 128;

uint32_t decode_keys_per_split(const DecodeShape& s) {
  const uint64_t work = (uint64_t)s.max_n_keys * s.n_kv_heads * s.n_seqs;
  uint64_t kps = (work + kTargetWG - 1) / kTargetWG;
  const uint64_t q = 64;  // SLOTS * U for D = 128 (and a divisor of it for 64)
  kps = (kps + q - 1) / q * q;
  if (kps < kMinKps) kps = kMinKps;
  return (uint32_t)kps;
}

static uint32_t max_splits_for(const DecodeShape& s) {
  const uint32_t kps = decode_keys_per_split(s);
  return (s.max_n_keys + kps - 1) / kps;
}

// Partials of `slots` (sequence, head, split) triples.
static uint64_t ws_for_slots(uint64_t slots, uint32_t head_dim) {
  return ws_align(slots * sizeof(float2)) + slots * head_dim * sizeof(float);
}

uint64_t decode_ws_bytes(const DecodeShape& s) {
  const uint32_t splits = max_splits_for(s);
  if (splits <= 1) return 0;
  return ws_for_slots((uint64_t)s.n_seqs * s.n_heads * splits, s.head_dim);
}

// Bound over every call with n_keys <= s.max_n_keys and n_seqs <= s.n_seqs:
// kps >= kMinKps and kps >= n_keys * n_kv_heads * n / kTargetWG for a call
// with n sequences, so it has at most min(ceil(max / kMinKps), ceil(kTargetWG
// / (n_kv_heads * n))) splits per sequence; take the largest n * splits.
uint64_t decode_ws_bound(const DecodeShape& s) {
  const uint64_t by_len = (s.max_n_keys + kMinKps - 1) / kMinKps;
  uint64_t best = 0;
  for (uint64_t n = 1; n <= s.n_seqs; n++) {
    const uint64_t per = (uint64_t)s.n_kv_heads * n;
    const uint64_t by_wg = (kTargetWG + per - 1) / per;
    const uint64_t slots = n * (by_len < by_wg ? by_len : by_wg);
    if (slots > best) best = slots;
  }
  return ws_for_slots(best * s.n_heads, s.head_dim);
}

template <int D>
static hipError_t launch_split_d(const DecodeArgs& a, dim3 grid, uint32_t G, hipStream_t st) {
  switch (G) {
#define FLK_CASE(g)                                                                         \
  case g:                                                                                   \
    hipLaunchKernelGGL((decode_split_kernel<D, g>), grid, dim3(kDecodeThreads), 0, st, a); \
    break;
    FLK_CASE(1)
    FLK_CASE(2)
    FLK_CASE(3)
    FLK_CASE(4)
    FLK_CASE(5)
    FLK_CASE(6)
    FLK_CASE(7)
    FLK_CASE(8)
#undef FLK_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const float* q, const float* kcache, const float* vcache, float* o,
                         const uint64_t* seq_row_off, const uint32_t* n_keys_dev,
                         const DecodeShape& s, const DecodeFused* fused, void* ws,
                         hipStream_t st) {
  DecodeArgs a{};
  a.q = q;
  a.kcache = kcache;
  a.vcache = vcache;
  a.o = o;
  a.seq_row_off = seq_row_off;
  a.n_keys_dev = n_keys_dev;
  a.n_keys = s.max_n_keys;
  a.n_heads = s.n_heads;
  a.n_kv_heads = s.n_kv_heads;
  a.kps = decode_keys_per_split(s);
  a.max_splits = max_splits_for(s);
  a.scale = (float)(1.0 / sqrt((double)s.head_dim));
  if (a.max_splits > 1) {
    char* w = static_cast<char*>(ws);
    const uint64_t slots = (uint64_t)s.n_seqs * s.n_heads * a.max_splits;
    a.part_ml = reinterpret_cast<float2*>(w);
    a.part_acc = reinterpret_cast<float*>(w + ws_align(slots * sizeof(float2)));
  }
  if (fused != nullptr) {
    a.q_raw = fused->q_raw;
    a.k_raw = fused->k_raw;
    a.v_raw = fused->v_raw;
    a.gq = fused->gq;
    a.gk = fused->gk;
    a.inv_freq = fused->inv_freq;
    a.eps = fused->eps;
    a.pairing = fused->pairing;
    a.qn_out = fused->qn_out;
    a.kcache_w = fused->kcache_w;
    a.vcache_w = fused->vcache_w;
  }
  const dim3 grid(s.n_kv_heads, a.max_splits, s.n_seqs);
  const uint32_t G = s.n_heads / s.n_kv_heads;
  hipError_t e = s.head_dim == 128 ? launch_split_d<128>(a, grid, G, st)
                                   : launch_split_d<64>(a, grid, G, st);
  if (e != hipSuccess || a.max_splits <= 1) return e;
  const dim3 mgrid(s.n_heads, s.n_seqs);
  if (s.head_dim == 128)
    hipLaunchKernelGGL(decode_merge_kernel<128>, mgrid, dim3(kMergeThreads), 0, st, a);
  else
    hipLaunchKernelGGL(decode_merge_kernel<64>, mgrid, dim3(kMergeThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace flk
