// GQA decode attention (one query per head) as split-K flash-decoding.
//
// The reference kernel (attention.wgsl:58-122) runs one 128-thread workgroup
// per q-head and holds every score in workgroup memory, which caps context at
// $MAX_KEYS and leaves the GPU with 16 workgroups. Here two launches (three
// for a ragged batch):
//
// decode_split_kernel<D, G, KH, RAGGED>  grid (n_kv_heads / KH, n_splits, n_seqs),
//   512 threads. A workgroup streams a share of the keys of KH adjacent kv heads and
//   serves the KH * G query heads that read them (G = n_heads / n_kv_heads),
//   so each K/V byte is read from HBM once. The cache row of one (key, kv head)
//   is D floats, loaded by D/4 lanes as float4: a "slot". The 512 / (D/4)
//   slots are KH kv heads x PH key phases; with KH = n_kv_heads (8 for
//   Qwen3-0.6B) and D = 128 a workgroup reads whole 4 KB cache rows, two keys
//   at a time, as one contiguous stream per K and V. Loads carry the
//   non-temporal hint: each row is read once.
//   Keys go to workgroups in blocks of PH * U, dealt round-robin over the
//   splits, so the launch sweeps the cache front to back as one window.
//   Per iteration a slot holds U keys in registers, and the next iteration's
//   keys are loaded before the current ones are used (two register sets). The
//   first set is requested before the prologue runs, so HBM latency overlaps
//   it. Scores: per-lane float4 dot, then a DPP/swizzle sum over the slot's
//   lanes; online softmax (running max m, denominator l, unnormalised
//   accumulator) per slot; phases of one kv head merge through LDS. A
//   single-split sequence writes o directly, otherwise each head writes its
//   (m, l, acc) partial.
// decode_batch_kernel<D, G, KH>  (ragged batches of up to 2048 sequences, after
//   queue_zero_kernel): the same splits and partials, run by one persistent
//   workgroup per CU that claims (sequence, split) items from a counter.
// decode_merge_kernel  grid (n_heads, D / 32, n_seqs): combines the partials of
//   one head with log-sum-exp weights in one round of loads.
// The launches are ordered by the stream: no device-scope fences inside a
// launch (the batch kernel's only atomics are its item claims).
//
// Fused mode (flk_decode_layer) prepends Layer.encode's prologue
// (layer.ts:598-622): every workgroup computes q's per-head RMSNorm + RoPE for
// its KH * G heads, and the workgroup whose key range holds position pos also
// normalises/rotates the new k rows and writes k and v into the cache row pos;
// it uses those rows from LDS rather than reading them back.
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
  uint32_t strict;              // ragged layer step: n_keys[b] > n_keys is refused (NaN rows)
  uint32_t n_heads, n_kv_heads;
  uint32_t kpi;                 // keys per block (one loop iteration of a slot group)
  uint32_t bps;                 // blocks per split (a sequence's split count divisor)
  uint32_t max_splits;          // cap on splits per sequence (= grid y)
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
#ifndef FLK_DECODE_TARGET_WG
#define FLK_DECODE_TARGET_WG 256
#endif
// Ragged batches: splits planned as if the longest sequence filled the batch
// with this many split workgroups. On the persistent batch kernel, 64
// sequences of 1025..16385 keys: 1024 739 us, 1536 690, 2048 676-677, 2560
// 669-671, 3072 671-676, 4096 682, 6144 701-702, 8192 703, 12288 730 (more
// items cost more per item than they save at the end of the queue).
#ifndef FLK_DECODE_RAGGED_TARGET_WG
#define FLK_DECODE_RAGGED_TARGET_WG 3072
#endif
#ifndef FLK_DECODE_NT
#define FLK_DECODE_NT 1  // K/V rows are read with the non-temporal hint (0: plain loads)
#endif
#ifndef FLK_DECODE_UNROLL
#define FLK_DECODE_UNROLL 2
#endif
#ifndef FLK_DECODE_THREADS
#define FLK_DECODE_THREADS 512
#endif
constexpr int kDecodeThreads = FLK_DECODE_THREADS;
constexpr int kMergeThreads = 256;
constexpr int kMergeNarrow = 64;  // one wave: batches whose heads have few splits
constexpr int kMergeCols = 8;    // float4 columns per merge workgroup (32 channels)
constexpr int kMergeBatch = 8;   // splits per thread per round of loads
constexpr uint32_t kMergeNarrowSplits = kMergeNarrow / kMergeCols * kMergeBatch;  // 64

// Keys per slot per iteration: fewer when G is large, to bound registers.
// Ragged batches (many shorter-lived workgroups, each paying its first rows'
// latency) keep more rows in flight: 64 sequences, 1025..16385 keys, 731 ->
// 712 us per call with 4 instead of 2 (on the persistent batch kernel: 2
// 688 us, 4 667, 8 792); one 32769-key sequence is slower with 4 (45.4 ->
// 47.2 us per fused call).
#ifndef FLK_DECODE_BATCH
#define FLK_DECODE_BATCH 1  // ragged batches of up to kBatchMaxSeqs: persistent decode_batch_kernel
#endif
#ifndef FLK_DECODE_RAGGED_UNROLL
#define FLK_DECODE_RAGGED_UNROLL 4
#endif
__host__ __device__ constexpr int decode_unroll(int G, bool ragged) {
  return ragged ? (G <= 4 ? FLK_DECODE_RAGGED_UNROLL
                          : (FLK_DECODE_RAGGED_UNROLL > 1 ? FLK_DECODE_RAGGED_UNROLL / 2 : 1))
                : (G <= 4 ? FLK_DECODE_UNROLL : (FLK_DECODE_UNROLL > 1 ? FLK_DECODE_UNROLL / 2 : 1));
}

// Splits of a sequence with n_keys keys: ceil(blocks / bps), at most
// max_splits. Both launches evaluate it identically.
__device__ __forceinline__ uint32_t seq_splits(const DecodeArgs& a, uint32_t n_keys) {
  const uint32_t nb = (n_keys + a.kpi - 1) / a.kpi;
  return min(a.max_splits, (nb + a.bps - 1) / a.bps);
}

// Keys sequence `seq` attends: the argument for one sequence; for a ragged
// batch its n_keys entry, clamped to the planned bound so that the grid covers
// every split (n_keys == 0 marks an empty sequence). The fused layer call with
// the key count in device memory (flk_decode_layer_dev) accepts only 1 ..
// max_keys there: any other value gives 0, and the split kernel then fills o
// with NaN and appends nothing (the reference throws "KV cache full" on the
// host, layer.ts:575; a replayed graph has no host step to throw from). The
// ragged layer step (strict) likewise refuses n_keys[b] > max_n_keys, whose
// prologue appended nothing; its n_keys[b] == 0 is an idle sequence.
__device__ __forceinline__ uint32_t seq_keys(const DecodeArgs& a, uint32_t seq) {
  if (a.n_keys_dev == nullptr) return a.n_keys;
  const uint32_t v = a.n_keys_dev[seq];
  if (a.q_raw != nullptr || a.strict) return v <= a.n_keys ? v : 0u;
  return min(v, a.n_keys);
}

// o rows of a sequence with no keys to attend: zeros for an empty (idle)
// sequence, NaN for a key count the device refused.
__device__ __forceinline__ float empty_fill(const DecodeArgs& a, uint32_t seq) {
  if (a.q_raw != nullptr) return __builtin_nanf("");
  if (a.strict && a.n_keys_dev[seq] != 0u) return __builtin_nanf("");
  return 0.f;
}

// U keys of one slot: rows base + u * PH + ph. Past the end of the split the
// last row (t1 - 1) is loaded again instead, so every load is unconditional;
// attend_keys masks those keys out.
template <int U, int PH>
__device__ __forceinline__ void load_keys(float4 (&kr)[U], float4 (&vr)[U], const float4* kb,
                                          const float4* vb, size_t row4, uint32_t base, int ph,
                                          uint32_t t1) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t t = min(base + u * PH + ph, t1 - 1);
#if FLK_DECODE_NT
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v k4 = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(kb + (size_t)t * row4));
    const f4v v4 = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(vb + (size_t)t * row4));
    kr[u] = make_float4(k4.x, k4.y, k4.z, k4.w);
    vr[u] = make_float4(v4.x, v4.y, v4.z, v4.w);
#else
    kr[u] = kb[(size_t)t * row4];
    vr[u] = vb[(size_t)t * row4];
#endif
  }
}

// Online-softmax update of one slot's G heads with U keys. The row at `pos`
// (when this workgroup appended it) is taken from knew / vnew.
template <int D, int G, int U, int PH>
__device__ __forceinline__ void attend_keys(const float4 (&kr_in)[U], const float4 (&vr_in)[U],
                                            const float4 (&qv)[G], float (&m)[G], float (&l)[G],
                                            float4 (&acc)[G], uint32_t base, int ph, uint32_t t1,
                                            bool owns_pos, uint32_t pos, float4 knew, float4 vnew,
                                            float scale) {
  constexpr int LPK = D / 4;
  float4 kr[U], vr[U];
  float s[G][U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t t = base + u * PH + ph;
    const bool mine = owns_pos && t == pos;
    const bool valid = t < t1;
    kr[u] = mine ? knew : kr_in[u];
    // A key past the end re-read row t1 - 1; its weight is exactly 0, but
    // 0 * v is NaN if that row holds a NaN pattern -- and in the fused layer
    // call row t1 - 1 is the row being appended in this launch, so other
    // workgroups may read it before it is written. Such v are zeroed (a bit
    // mask, so the row's contents never reach the sum).
    const uint32_t keep = valid ? 0xffffffffu : 0u;
    const float4 vv = mine ? vnew : vr_in[u];
    vr[u] = make_float4(__uint_as_float(__float_as_uint(vv.x) & keep),
                        __uint_as_float(__float_as_uint(vv.y) & keep),
                        __uint_as_float(__float_as_uint(vv.z) & keep),
                        __uint_as_float(__float_as_uint(vv.w) & keep));
#pragma unroll
    for (int g = 0; g < G; g++) {
      float d = qv[g].x * kr[u].x;
      d = fmaf(qv[g].y, kr[u].y, d);
      d = fmaf(qv[g].z, kr[u].z, d);
      d = fmaf(qv[g].w, kr[u].w, d);
      d = group_sum<LPK>(d);
      s[g][u] = valid ? d * scale : -INFINITY;
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

// The key phases of each kv head combined through LDS (PH > 1), then emit(hq,
// c, M, L, A) for every (q head of the workgroup, float4 column). Every
// thread of the workgroup calls it.
template <int D, int G, int KH, int PH, class EMIT>
__device__ __forceinline__ void combine_phases(const float (&m)[G], const float (&l)[G],
                                               const float4 (&acc)[G], int slot, int sl, int kh,
                                               int tid, float (*s_m)[G], float (*s_l)[G],
                                               float4 (*s_acc)[G][D / 4], EMIT emit) {
  constexpr int LPK = D / 4;
  constexpr int HG = KH * G;
  if constexpr (PH == 1) {
#pragma unroll
    for (int g = 0; g < G; g++) emit(kh * G + g, sl, m[g], l[g], acc[g]);
    return;
  }
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
  for (int i = tid; i < HG * LPK; i += kDecodeThreads) {
    const int hq = i / LPK, c = i % LPK;  // hq = kv-head-in-group * G + g
    const int j = hq / G, g = hq % G;
    float M = -INFINITY;
#pragma unroll
    for (int p = 0; p < PH; p++) M = fmaxf(M, s_m[j + KH * p][g]);
    float L = 0.f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int p = 0; p < PH; p++) {
      const int sidx = j + KH * p;
      const float ms = s_m[sidx][g];
      const float w = ms == -INFINITY ? 0.f : expf(ms - M);
      L = fmaf(s_l[sidx][g], w, L);
      const float4 as = s_acc[sidx][g][c];
      A.x = fmaf(as.x, w, A.x);
      A.y = fmaf(as.y, w, A.y);
      A.z = fmaf(as.z, w, A.z);
      A.w = fmaf(as.w, w, A.w);
    }
    emit(hq, c, M, L, A);
  }
}

template <int D, int G, int KH, bool RAGGED>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_kernel(DecodeArgs a) {
  constexpr int LPK = D / 4;                    // lanes per (key, kv head) row
  constexpr int SLOTS = kDecodeThreads / LPK;   // 16 (D = 128) or 32 (D = 64) at 512 threads
  static_assert(SLOTS % KH == 0, "KH must divide the slot count");
  constexpr int PH = SLOTS / KH;                // key phases
  constexpr int U = decode_unroll(G, RAGGED);
  constexpr int KPI = PH * U;                   // keys per iteration
  constexpr int HG = KH * G;                    // q heads of this workgroup

  __shared__ float4 s_q[HG][LPK];
  __shared__ float4 s_knew[KH][LPK];
  __shared__ float4 s_vnew[KH][LPK];
  __shared__ float2 s_cs[D / 2];  // fused: RoPE cos/sin at the new position
  __shared__ float s_m[PH > 1 ? SLOTS : 1][G];
  __shared__ float s_l[PH > 1 ? SLOTS : 1][G];
  __shared__ float4 s_acc[PH > 1 ? SLOTS : 1][G][LPK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slot = tid / LPK;
  const int sl = tid % LPK;
  const int kh = slot % KH;
  const int ph = slot / KH;
  const uint32_t kvh0 = blockIdx.x * KH;
  const uint32_t kvh = kvh0 + kh;
  const uint32_t split = blockIdx.y;
  const uint32_t seq = blockIdx.z;
  const uint32_t h0 = kvh0 * G;  // first q head of this workgroup

  const uint32_t n_keys = seq_keys(a, seq);
  const uint64_t row0 = a.seq_row_off != nullptr ? a.seq_row_off[seq] : 0;
  if (n_keys == 0) {  // empty ragged sequence: zero rows; refused key count: NaN rows
    if (split == 0) {
      const float fill = empty_fill(a, seq);
      for (int i = tid; i < HG * D; i += kDecodeThreads)
        a.o[((size_t)seq * a.n_heads + h0) * D + i] = fill;
    }
    return;
  }
  const uint32_t n_splits = seq_splits(a, n_keys);
  if (split >= n_splits) return;  // uniform per workgroup
  // Blocks of KPI keys are dealt round-robin: split s takes blocks s, s +
  // n_splits, ..., so at any time the workgroups of a launch read neighbouring
  // blocks (one moving window of the cache rather than n_splits streams).
  const uint32_t n_blocks = (n_keys + KPI - 1) / KPI;
  const uint32_t t1 = n_keys;
  const size_t row4 = (size_t)a.n_kv_heads * (D / 4);  // float4 per cache row

  // vmcnt retires loads in issue order, so everything the prologue reads is
  // requested BEFORE the first K/V rows: the prologue then waits only for its
  // own inputs while the rows stream in. Inputs are staged through LDS.
  constexpr int QLD = (HG * LPK + kDecodeThreads - 1) / kDecodeThreads;  // q float4 / thread
  constexpr int KLD = (KH * LPK + kDecodeThreads - 1) / kDecodeThreads;  // new-row float4
  const bool fused = a.q_raw != nullptr;
  const uint32_t pos = n_keys - 1;  // the appended row (fused)
  const bool owns_pos = fused && (pos / KPI) % n_splits == split;
  float4 qld[QLD], kld[KLD], vld[KLD];
  float gq0 = 0.f, gq1 = 0.f, gk0 = 0.f, gk1 = 0.f, invf = 0.f;
  {
    const float4* qs = reinterpret_cast<const float4*>(
        fused ? a.q_raw + (size_t)h0 * D : a.q + ((size_t)seq * a.n_heads + h0) * D);
#pragma unroll
    for (int i = 0; i < QLD; i++) qld[i] = qs[min(tid + kDecodeThreads * i, HG * LPK - 1)];
  }
  if (fused) {
    const float4* ks = reinterpret_cast<const float4*>(a.k_raw + (size_t)kvh0 * D);
    const float4* vs = reinterpret_cast<const float4*>(a.v_raw + (size_t)kvh0 * D);
#pragma unroll
    for (int i = 0; i < KLD; i++) {
      const int f = min(tid + kDecodeThreads * i, KH * LPK - 1);
      kld[i] = ks[f];
      vld[i] = vs[f];
    }
    gq0 = a.gq[lane];
    gk0 = a.gk[lane];
    if (D == 128) {
      gq1 = a.gq[lane + 64];
      gk1 = a.gk[lane + 64];
    }
    invf = a.inv_freq[min(tid, D / 2 - 1)];
  }

  const float4* kb = reinterpret_cast<const float4*>(a.kcache) + row0 * row4 + (size_t)kvh * LPK + sl;
  const float4* vb = reinterpret_cast<const float4*>(a.vcache) + row0 * row4 + (size_t)kvh * LPK + sl;
  float4 ka[U], va[U], kn[U], vn[U];
  load_keys<U, PH>(ka, va, kb, vb, row4, split * KPI, ph, t1);

  // ---- q for the KH * G heads (fused: prologue computed here) --------------
  // Unconditional stores (clamped index: surplus threads rewrite the last
  // element with the value they loaded from it), so the loads above have no
  // conditional use to be sunk into, past the row loads.
#pragma unroll
  for (int i = 0; i < QLD; i++) {
    const int f = min(tid + kDecodeThreads * i, HG * LPK - 1);
    s_q[f / LPK][f % LPK] = qld[i];
  }
  if (fused) {
#pragma unroll
    for (int i = 0; i < KLD; i++) {
      const int f = min(tid + kDecodeThreads * i, KH * LPK - 1);
      s_knew[f / LPK][f % LPK] = kld[i];
      s_vnew[f / LPK][f % LPK] = vld[i];
    }
    if (tid < D / 2) s_cs[tid] = rope_cos_sin(invf, pos);
    __syncthreads();
    for (int vi = wave; vi < HG; vi += kDecodeThreads / 64) {  // q head h0 + vi
      float* sq = reinterpret_cast<float*>(&s_q[vi][0]);
      float e0 = sq[lane], e1 = D == 128 ? sq[lane + 64] : 0.f;
      head_rmsnorm<D>(e0, e1, gq0, gq1, a.eps);
      head_rope<D>(e0, e1, s_cs, a.pairing, lane);
      sq[lane] = e0;
      if (D == 128) sq[lane + 64] = e1;
      if (split == 0) {
        float* dq = a.qn_out + (size_t)(h0 + vi) * D;
        dq[lane] = e0;
        if (D == 128) dq[lane + 64] = e1;
      }
    }
    if (owns_pos) {  // append row pos: k normed + rotated, v raw (layer.ts:616-622)
      const size_t row = (size_t)a.n_kv_heads * D;
      for (int j = wave; j < KH; j += kDecodeThreads / 64) {
        float* lk = reinterpret_cast<float*>(&s_knew[j][0]);
        const float* lv = reinterpret_cast<const float*>(&s_vnew[j][0]);
        float e0 = lk[lane], e1 = D == 128 ? lk[lane + 64] : 0.f;
        head_rmsnorm<D>(e0, e1, gk0, gk1, a.eps);
        head_rope<D>(e0, e1, s_cs, a.pairing, lane);
        float* dk = a.kcache_w + (size_t)pos * row + (size_t)(kvh0 + j) * D;
        float* dv = a.vcache_w + (size_t)pos * row + (size_t)(kvh0 + j) * D;
        dk[lane] = lk[lane] = e0;
        dv[lane] = lv[lane];
        if (D == 128) {
          dk[lane + 64] = lk[lane + 64] = e1;
          dv[lane + 64] = lv[lane + 64];
        }
      }
    }
  }
  __syncthreads();  // s_q (and the new k/v rows) ready

  float4 qv[G];
#pragma unroll
  for (int g = 0; g < G; g++) qv[g] = s_q[kh * G + g][sl];
  const float4 knew = s_knew[kh][sl];
  const float4 vnew = s_vnew[kh][sl];

  float m[G], l[G];
  float4 acc[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.f;
    acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Two register sets: the next block's loads are issued before the current
  // block's arithmetic. Loads are unconditional, so the compiler can count
  // them: past the split's last block a slot loads block 0 instead, which
  // the tails of all splits request, so after the first request on an XCD it
  // comes from L2 (the split's own last block, read with the non-temporal
  // hint, need not still be there); those rows are never used.
  for (uint32_t b = split; b < n_blocks; b += 2 * n_splits) {
    const uint32_t b1 = b + n_splits;
    const uint32_t b2 = b1 + n_splits;
    load_keys<U, PH>(kn, vn, kb, vb, row4, (b1 < n_blocks ? b1 : 0) * KPI, ph, t1);
    attend_keys<D, G, U, PH>(ka, va, qv, m, l, acc, b * KPI, ph, t1, owns_pos, pos, knew, vnew,
                             a.scale);
    load_keys<U, PH>(ka, va, kb, vb, row4, (b2 < n_blocks ? b2 : 0) * KPI, ph, t1);
    if (b1 < n_blocks)
      attend_keys<D, G, U, PH>(kn, vn, qv, m, l, acc, b1 * KPI, ph, t1, owns_pos, pos, knew,
                               vnew, a.scale);
  }

  // ---- combine the phases of each kv head, write o or the partial ---------
  // hq: q head within the workgroup (kv head j = hq / G, group member hq % G).
  auto emit = [&](int hq, int c, float M, float L, float4 A) {
    const uint32_t h = h0 + (uint32_t)hq;
    if (n_splits == 1) {
      reinterpret_cast<float4*>(a.o + ((size_t)seq * a.n_heads + h) * D)[c] =
          make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
    } else {
      const size_t p = ((size_t)seq * a.n_heads + h) * a.max_splits + split;
      if (c == 0) a.part_ml[p] = make_float2(M, L);
      reinterpret_cast<float4*>(a.part_acc + p * D)[c] = A;
    }
  };
  combine_phases<D, G, KH, PH>(m, l, acc, slot, sl, kh, tid, s_m, s_l, s_acc, emit);
}

// ------------------------------------------------------- ragged batches ----
// decode_batch_kernel<D, G, KH>  grid (n_kv_heads / KH, kBatchWG / groups),
//   512 threads: the same splits, partials and merge as decode_split_kernel's
//   ragged instance, run by one long-lived workgroup per CU instead of one
//   workgroup per split (a bare read of 4 GiB in this shape: 610 us, against
//   660-664 us as ~4000 one-shot workgroups). The batch's (sequence, split)
//   items are numbered sequence by sequence (an empty sequence has one item,
//   which zeroes its rows) and claimed in order from a counter (one per kv
//   head group, zeroed by queue_zero_kernel at the start of the call), so at
//   any time the workgroups sweep a few sequences, each as a moving window,
//   and a faster XCD simply claims more items (a fixed stride of items per
//   workgroup measured 728-733 us, slower than one-shot workgroups at 710, as
//   the slowest XCD then sets the end). Which workgroup runs an item does not
//   change its partial, so results are bit-reproducible. Each workgroup first
//   builds, in LDS, the first item of every sequence (a prefix sum of the
//   split counts) and the sequences' key counts and row offsets.
#ifndef FLK_DECODE_BATCH_WG
#define FLK_DECODE_BATCH_WG 256
#endif
constexpr uint32_t kBatchWG = FLK_DECODE_BATCH_WG;
constexpr uint32_t kBatchMaxSeqs = 2048;

constexpr uint32_t kBatchMaxGroups = 64;  // item counters in the workspace
constexpr uint64_t kQueueBytes = 256;      // kBatchMaxGroups counters, 256-byte aligned

// Whether a batch of n_seqs sequences in `groups` kv-head groups takes
// decode_batch_kernel (its tables fit in LDS, its counters in kQueueBytes).
static bool use_batch(uint32_t n_seqs, uint32_t groups) {
  return FLK_DECODE_BATCH && n_seqs <= kBatchMaxSeqs && groups <= kBatchMaxGroups;
}

__global__ void queue_zero_kernel(uint32_t* queue, uint32_t n) {
  if (threadIdx.x < n) queue[threadIdx.x] = 0u;
}

template <int D, int G, int KH>
__global__ __launch_bounds__(kDecodeThreads) void decode_batch_kernel(DecodeArgs a,
                                                                      uint32_t n_seqs,
                                                                      uint32_t* queue) {
  constexpr int LPK = D / 4;
  constexpr int SLOTS = kDecodeThreads / LPK;
  static_assert(SLOTS % KH == 0, "KH must divide the slot count");
  constexpr int PH = SLOTS / KH;
  constexpr int U = decode_unroll(G, true);
  constexpr int KPI = PH * U;
  constexpr int HG = KH * G;
  constexpr int WAVES = kDecodeThreads / kWave;

  __shared__ float4 s_q[HG][LPK];
  __shared__ float s_m[PH > 1 ? SLOTS : 1][G];
  __shared__ float s_l[PH > 1 ? SLOTS : 1][G];
  __shared__ float4 s_acc[PH > 1 ? SLOTS : 1][G][LPK];
  __shared__ uint32_t s_first[kBatchMaxSeqs + 1];  // first item of each sequence
  __shared__ uint32_t s_nk[kBatchMaxSeqs];
  __shared__ uint64_t s_row[kBatchMaxSeqs];
  __shared__ uint32_t s_wsum[WAVES];
  __shared__ uint32_t s_item;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slot = tid / LPK;
  const int sl = tid % LPK;
  const int kh = slot % KH;
  const int ph = slot / KH;
  const uint32_t kvh0 = blockIdx.x * KH;
  const uint32_t kvh = kvh0 + kh;
  const uint32_t h0 = kvh0 * G;
  const size_t row4 = (size_t)a.n_kv_heads * (D / 4);

  // ---- item table: exclusive prefix of items per sequence, 512 at a time --
  uint32_t carry = 0;
  for (uint32_t c0 = 0; c0 < n_seqs; c0 += kDecodeThreads) {
    const uint32_t sq = c0 + tid;
    uint32_t items = 0;
    if (sq < n_seqs) {
      const uint32_t nk = seq_keys(a, sq);
      s_nk[sq] = nk;
      s_row[sq] = a.seq_row_off[sq];
      items = nk == 0 ? 1u : seq_splits(a, nk);
    }
    uint32_t incl = items;  // inclusive scan over the wave
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, d, kWave);
      if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) s_wsum[wave] = incl;
    __syncthreads();
    uint32_t before = carry;
    for (int w = 0; w < wave; w++) before += s_wsum[w];
    if (sq < n_seqs) s_first[sq] = before + incl - items;
    for (int w = 0; w < WAVES; w++) carry += s_wsum[w];
    __syncthreads();
  }
  if (tid == 0) s_first[n_seqs] = carry;
  __syncthreads();
  const uint32_t n_items = carry;

  // Item -> (sequence, split, keys): the last sequence whose first item is
  // at or before it (every sequence has at least one item).
  auto locate = [&](uint32_t item, uint32_t& seq, uint32_t& split, uint32_t& n_keys) {
    uint32_t lo = 0, hi = n_seqs;  // s_first[lo] <= item < s_first[hi]
    while (hi - lo > 1) {
      const uint32_t mid = (lo + hi) / 2;
      if (s_first[mid] <= item) lo = mid; else hi = mid;
    }
    seq = lo;
    split = item - s_first[lo];
    n_keys = s_nk[lo];
  };
  const size_t col = (size_t)kvh * LPK + sl;
  auto k_base = [&](uint32_t seq) {
    return reinterpret_cast<const float4*>(a.kcache) + s_row[seq] * row4 + col;
  };
  auto v_base = [&](uint32_t seq) {
    return reinterpret_cast<const float4*>(a.vcache) + s_row[seq] * row4 + col;
  };
  constexpr int QLD = (HG * LPK + kDecodeThreads - 1) / kDecodeThreads;
  auto load_q = [&](uint32_t seq, float4 (&qld)[QLD]) {
    const float4* qs = reinterpret_cast<const float4*>(a.q + ((size_t)seq * a.n_heads + h0) * D);
#pragma unroll
    for (int i = 0; i < QLD; i++) qld[i] = qs[min(tid + kDecodeThreads * i, HG * LPK - 1)];
  };

  // Items are claimed one ahead: the claim of the next item is issued as an
  // item starts and published at its first barrier; the item's last
  // iteration then loads the next item's first block (in place of the
  // unused reload every split's last iteration makes) and its q is requested
  // before the combine, so a new item starts with its data in registers.
  uint32_t* counter = queue + blockIdx.x;
  if (tid == 0)
    s_item = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  uint32_t it = s_item;
  __syncthreads();  // every thread has read s_item before the first item writes it
  bool pre = false;  // ka, va and qld hold item it's first block and q
  float4 ka[U], va[U], kn[U], vn[U];
  float4 qld[QLD];
  const float4 none = make_float4(0.f, 0.f, 0.f, 0.f);
  while (it < n_items) {
    uint32_t claim = 0;
    if (tid == 0)
      claim = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t seq, split, n_keys;
    locate(it, seq, split, n_keys);
    if (n_keys == 0) {  // empty sequence: zero rows (refused key count: NaN)
      const float fill = empty_fill(a, seq);
      for (int i = tid; i < HG * D; i += kDecodeThreads)
        a.o[((size_t)seq * a.n_heads + h0) * D + i] = fill;
      if (tid == 0) s_item = claim;
      __syncthreads();
      it = s_item;
      pre = false;
      __syncthreads();  // every thread has read s_item before it is written again
      continue;         // uniform
    }
    const uint32_t n_splits = s_first[seq + 1] - s_first[seq];
    const uint32_t n_blocks = (n_keys + KPI - 1) / KPI;
    const uint32_t t1 = n_keys;
    const float4* kb = k_base(seq);
    const float4* vb = v_base(seq);
    if (!pre) {
      load_q(seq, qld);
      load_keys<U, PH>(ka, va, kb, vb, row4, split * KPI, ph, t1);
    }
#pragma unroll
    for (int i = 0; i < QLD; i++) {
      const int f = min(tid + kDecodeThreads * i, HG * LPK - 1);
      s_q[f / LPK][f % LPK] = qld[i];
    }
    if (tid == 0) s_item = claim;
    __syncthreads();  // s_q and the next item ready (the previous item's LDS reads are done)
    const uint32_t nit = s_item;
    float4 qv[G];
#pragma unroll
    for (int g = 0; g < G; g++) qv[g] = s_q[kh * G + g][sl];
    // The next item, if it has keys: where its first block is.
    uint32_t nseq = seq, nsplit = 0, nkeys = 0;
    if (nit < n_items) locate(nit, nseq, nsplit, nkeys);
    const bool pf = nit < n_items && nkeys > 0;
    const float4* nkb = pf ? k_base(nseq) : kb;
    const float4* nvb = pf ? v_base(nseq) : vb;
    const uint32_t nbase = pf ? nsplit * KPI : 0;
    const uint32_t nt1 = pf ? nkeys : t1;

    float m[G], l[G];
    float4 acc[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      m[g] = -INFINITY;
      l[g] = 0.f;
      acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (uint32_t b = split; b < n_blocks; b += 2 * n_splits) {
      const uint32_t b1 = b + n_splits;
      const uint32_t b2 = b1 + n_splits;
      load_keys<U, PH>(kn, vn, kb, vb, row4, (b1 < n_blocks ? b1 : 0) * KPI, ph, t1);
      attend_keys<D, G, U, PH>(ka, va, qv, m, l, acc, b * KPI, ph, t1, false, 0, none, none,
                               a.scale);
      if (b2 < n_blocks)
        load_keys<U, PH>(ka, va, kb, vb, row4, b2 * KPI, ph, t1);
      else  // the last iteration: the next item's first block (or a reload)
        load_keys<U, PH>(ka, va, nkb, nvb, row4, nbase, ph, nt1);
      if (b1 < n_blocks)
        attend_keys<D, G, U, PH>(kn, vn, qv, m, l, acc, b1 * KPI, ph, t1, false, 0, none, none,
                                 a.scale);
    }
    if (pf) load_q(nseq, qld);
    auto emit = [&](int hq, int c, float M, float L, float4 A) {
      const uint32_t h = h0 + (uint32_t)hq;
      if (n_splits == 1) {
        reinterpret_cast<float4*>(a.o + ((size_t)seq * a.n_heads + h) * D)[c] =
            make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
      } else {
        const size_t p = ((size_t)seq * a.n_heads + h) * a.max_splits + split;
        if (c == 0) a.part_ml[p] = make_float2(M, L);
        reinterpret_cast<float4*>(a.part_acc + p * D)[c] = A;
      }
    };
    combine_phases<D, G, KH, PH>(m, l, acc, slot, sl, kh, tid, s_m, s_l, s_acc, emit);
    __syncthreads();  // LDS (s_q, s_item, the combine) free for the next item
    it = nit;
    pre = pf;
  }
}

// grid (head, column chunk, sequence); thread -> (group r, float4 column c),
// lane = 8 * (r mod 8) + c. Group r takes splits r, r + GROUPS, ...: each
// round issues up to kMergeBatch independent loads per thread and folds them
// with weights against the running max. The groups then combine in a fixed
// order (the result does not depend on scheduling): the workgroup's maximum
// (lane butterfly, then the waves through LDS), one rescale per thread, and a
// sum butterfly over the lanes of a column (strides 8, 16, 32) followed by
// the waves in order.
template <int D, int THREADS>
__global__ __launch_bounds__(THREADS) void decode_merge_kernel(DecodeArgs a) {
  constexpr int GROUPS = THREADS / kMergeCols;
  constexpr int WAVES = THREADS / kWave;
  static_assert(kMergeCols == 8 && kWave == 64, "lane = 8 * (group mod 8) + column");
  __shared__ float s_m[WAVES];
  __shared__ float s_l[WAVES];
  __shared__ float4 s_acc[WAVES][kMergeCols];

  const uint32_t head = blockIdx.x;
  const uint32_t seq = blockIdx.z;
  const uint32_t n_keys = seq_keys(a, seq);
  const uint32_t n_splits = seq_splits(a, n_keys);
  if (n_splits <= 1) return;  // written by the split kernel (or empty)
  const int tid = threadIdx.x;
  const int grp = tid / kMergeCols;
  const int c = blockIdx.y * kMergeCols + tid % kMergeCols;  // float4 column
  const size_t p0 = ((size_t)seq * a.n_heads + head) * a.max_splits;

  float M = -INFINITY, L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s0 = grp; s0 < n_splits; s0 += GROUPS * kMergeBatch) {
    // Unconditional loads (indices past the last split reload it and are
    // given weight 0), so the wait counts stay exact.
    float2 ml[kMergeBatch];
    float4 pa[kMergeBatch];
#pragma unroll
    for (int i = 0; i < kMergeBatch; i++) {
      const uint32_t s = min(s0 + GROUPS * i, n_splits - 1);
      ml[i] = a.part_ml[p0 + s];
      pa[i] = reinterpret_cast<const float4*>(a.part_acc + (p0 + s) * D)[c];
    }
#pragma unroll
    for (int i = 0; i < kMergeBatch; i++)
      if (s0 + GROUPS * i >= n_splits) ml[i].x = -INFINITY;
    float mx = M;
#pragma unroll
    for (int i = 0; i < kMergeBatch; i++) mx = fmaxf(mx, ml[i].x);
    if (mx == -INFINITY) continue;
    const float wo = M == -INFINITY ? 0.f : expf(M - mx);
    L *= wo;
    A.x *= wo;
    A.y *= wo;
    A.z *= wo;
    A.w *= wo;
#pragma unroll
    for (int i = 0; i < kMergeBatch; i++) {
      const float w = ml[i].x == -INFINITY ? 0.f : expf(ml[i].x - mx);
      L = fmaf(ml[i].y, w, L);
      A.x = fmaf(pa[i].x, w, A.x);
      A.y = fmaf(pa[i].y, w, A.y);
      A.z = fmaf(pa[i].z, w, A.z);
      A.w = fmaf(pa[i].w, w, A.w);
    }
    M = mx;
  }
  const int wave = tid / kWave, lane = tid % kWave;
  float MM = fmaxf(M, xor_lane<8>(M));
  MM = max_xor<16>(MM);
  MM = max_xor<32>(MM);
  if (lane == 0) s_m[wave] = MM;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < WAVES; w++) MM = fmaxf(MM, s_m[w]);
  const float wt = M == -INFINITY ? 0.f : expf(M - MM);
  float v[5] = {L * wt, A.x * wt, A.y * wt, A.z * wt, A.w * wt};
#pragma unroll
  for (int k = 0; k < 5; k++) {
    v[k] = v[k] + xor_lane<8>(v[k]);
    v[k] = sum_xor<16>(v[k]);
    v[k] = sum_xor<32>(v[k]);
  }
  if (lane < kMergeCols) {
    if (lane == 0) s_l[wave] = v[0];
    s_acc[wave][lane] = make_float4(v[1], v[2], v[3], v[4]);
  }
  __syncthreads();
  if (tid >= kMergeCols) return;
  L = s_l[0];
  A = s_acc[0][tid];
#pragma unroll
  for (int w = 1; w < WAVES; w++) {
    L += s_l[w];
    const float4 p = s_acc[w][tid];
    A.x += p.x;
    A.y += p.y;
    A.z += p.z;
    A.w += p.w;
  }
  reinterpret_cast<float4*>(a.o + ((size_t)seq * a.n_heads + head) * D)[c] =
      make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
}

// ------------------------------------------------------------------ plan ----
// KH: kv heads per workgroup, the largest of 8, 4, 2, 1 dividing n_kv_heads.
static uint32_t kv_heads_per_wg(uint32_t n_kv_heads) {
  for (uint32_t kh = 8; kh > 1; kh >>= 1)
    if (n_kv_heads % kh == 0) return kh;
  return 1;
}

// Keys per loop iteration of one workgroup (PH * U) for calls of n_seqs
// sequences (more than one: the ragged instance).
static uint32_t keys_per_iter(const DecodeShape& s, uint32_t n_seqs) {
  const uint32_t slots = kDecodeThreads / (s.head_dim / 4);
  const uint32_t U = decode_unroll((int)(s.n_heads / s.n_kv_heads), n_seqs > 1);
  return slots / kv_heads_per_wg(s.n_kv_heads) * U;
}

// Split plan. A single sequence gets one split workgroup per CU group:
// kTargetWG / (n_kv_heads / KH) splits (256 for Qwen3: one per CU, each
// taking every 256th block), fewer when there are under kMinBps blocks per
// split. A ragged batch plans from its longest sequence: bps blocks per
// split, chosen so the longest batch of that length would give about
// kRaggedTargetWG workgroups, and each sequence gets ceil(blocks / bps).
constexpr uint32_t kTargetWG = FLK_DECODE_TARGET_WG;
constexpr uint32_t kRaggedTargetWG = FLK_DECODE_RAGGED_TARGET_WG;
#ifndef FLK_DECODE_MIN_BPS
#define FLK_DECODE_MIN_BPS 1
#endif
constexpr uint32_t kMinBps = FLK_DECODE_MIN_BPS;

struct SplitPlan {
  uint32_t kpi, bps, max_splits;
};

static SplitPlan split_plan(const DecodeShape& s) {
  SplitPlan p{};
  p.kpi = keys_per_iter(s, s.n_seqs);
  const uint64_t groups = s.n_kv_heads / kv_heads_per_wg(s.n_kv_heads);
  const uint64_t nb = ((uint64_t)s.max_n_keys + p.kpi - 1) / p.kpi;
  if (s.n_seqs == 1) {
    const uint64_t by_wg = kTargetWG / groups > 0 ? kTargetWG / groups : 1;
    const uint64_t by_len = (nb + kMinBps - 1) / kMinBps;
    p.bps = kMinBps;
    p.max_splits = (uint32_t)(by_wg < by_len ? by_wg : by_len);
  } else {
    uint64_t bps = (nb * groups * s.n_seqs + kRaggedTargetWG - 1) / kRaggedTargetWG;
    if (bps < kMinBps) bps = kMinBps;
    p.bps = (uint32_t)bps;
    p.max_splits = (uint32_t)((nb + bps - 1) / bps);
  }
  return p;
}

// Partials of `slots` (sequence, head, split) triples.
static uint64_t ws_for_slots(uint64_t slots, uint32_t head_dim) {
  return ws_align(slots * sizeof(float2)) + slots * head_dim * sizeof(float);
}

uint64_t decode_ws_bytes(const DecodeShape& s) {
  const SplitPlan p = split_plan(s);
  if (p.max_splits <= 1) return 0;
  const uint32_t groups = s.n_kv_heads / kv_heads_per_wg(s.n_kv_heads);
  const uint64_t queue = s.n_seqs > 1 && use_batch(s.n_seqs, groups) ? kQueueBytes : 0;
  return queue + ws_for_slots((uint64_t)s.n_seqs * s.n_heads * p.max_splits, s.head_dim);
}

// Bound over every call with n_keys <= s.max_n_keys and n_seqs <= s.n_seqs
// (single-sequence calls included). One sequence: max_splits <= kTargetWG /
// groups. n > 1 sequences: bps >= nb * groups * n / kRaggedTargetWG, so
// max_splits = ceil(nb / bps) <= kRaggedTargetWG / (groups * n) + 1; both
// also <= ceil(nb / kMinBps). Take the largest n * splits.
uint64_t decode_ws_bound(const DecodeShape& s) {
  const uint64_t groups = s.n_kv_heads / kv_heads_per_wg(s.n_kv_heads);
  uint64_t best = 0;
  for (uint64_t n = 1; n <= s.n_seqs; n++) {
    const uint64_t kpi = keys_per_iter(s, (uint32_t)n);
    const uint64_t nb = ((uint64_t)s.max_n_keys + kpi - 1) / kpi;
    const uint64_t by_len = (nb + kMinBps - 1) / kMinBps;
    const uint64_t by_wg = n == 1 ? (kTargetWG / groups > 0 ? kTargetWG / groups : 1)
                                  : kRaggedTargetWG / (groups * n) + 1;
    const uint64_t splits = by_len < by_wg ? by_len : by_wg;
    if (splits > 1 && n * splits > best) best = n * splits;
  }
  // (+ the batch kernel's counters, which only calls of 2+ sequences use)
  return best ? kQueueBytes + ws_for_slots(best * s.n_heads, s.head_dim) : 0;
}

template <int D, int KH, bool RAGGED>
static hipError_t launch_split_kh(const DecodeArgs& a, dim3 grid, uint32_t G, hipStream_t st) {
  switch (G) {
#define FLK_CASE(g)                                                                      \
  case g:                                                                                \
    hipLaunchKernelGGL((decode_split_kernel<D, g, KH, RAGGED>), grid, dim3(kDecodeThreads), 0, \
                       st, a);                                                           \
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

template <int D, int KH>
static hipError_t launch_batch_kh(const DecodeArgs& a, dim3 grid, uint32_t G, uint32_t n_seqs,
                                  uint32_t* queue, hipStream_t st) {
  switch (G) {
#define FLK_CASE(g)                                                                          \
  case g:                                                                                    \
    hipLaunchKernelGGL((decode_batch_kernel<D, g, KH>), grid, dim3(kDecodeThreads), 0, st, a, \
                       n_seqs, queue);                                                       \
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

template <int D>
static hipError_t launch_batch_d(const DecodeArgs& a, dim3 grid, uint32_t G, uint32_t KH,
                                 uint32_t n_seqs, uint32_t* queue, hipStream_t st) {
  switch (KH) {
    case 8: return launch_batch_kh<D, 8>(a, grid, G, n_seqs, queue, st);
    case 4: return launch_batch_kh<D, 4>(a, grid, G, n_seqs, queue, st);
    case 2: return launch_batch_kh<D, 2>(a, grid, G, n_seqs, queue, st);
    default: return launch_batch_kh<D, 1>(a, grid, G, n_seqs, queue, st);
  }
}

template <int D>
static hipError_t launch_split_d(const DecodeArgs& a, dim3 grid, uint32_t G, uint32_t KH,
                                 bool ragged, hipStream_t st) {
  if (ragged) {
    switch (KH) {
      case 8: return launch_split_kh<D, 8, true>(a, grid, G, st);
      case 4: return launch_split_kh<D, 4, true>(a, grid, G, st);
      case 2: return launch_split_kh<D, 2, true>(a, grid, G, st);
      default: return launch_split_kh<D, 1, true>(a, grid, G, st);
    }
  }
  switch (KH) {
    case 8: return launch_split_kh<D, 8, false>(a, grid, G, st);
    case 4: return launch_split_kh<D, 4, false>(a, grid, G, st);
    case 2: return launch_split_kh<D, 2, false>(a, grid, G, st);
    default: return launch_split_kh<D, 1, false>(a, grid, G, st);
  }
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
  const SplitPlan plan = split_plan(s);
  a.kpi = plan.kpi;
  a.bps = plan.bps;
  a.max_splits = plan.max_splits;
  a.scale = (float)(1.0 / sqrt((double)s.head_dim));
  const uint32_t KH = kv_heads_per_wg(s.n_kv_heads);
  const uint32_t groups = s.n_kv_heads / KH;
  const bool ragged = s.n_seqs > 1;  // the plan's kpi assumes the same instance
  // Batches take the claimed-item kernel when they have partials (so a
  // workspace, whose first kQueueBytes hold its counters).
  const bool batch = ragged && use_batch(s.n_seqs, groups) && a.max_splits > 1;
  uint32_t* queue = batch ? static_cast<uint32_t*>(ws) : nullptr;
  if (a.max_splits > 1) {
    char* w = static_cast<char*>(ws) + (batch ? kQueueBytes : 0);
    const uint64_t slots = (uint64_t)s.n_seqs * s.n_heads * a.max_splits;
    a.part_ml = reinterpret_cast<float2*>(w);
    a.part_acc = reinterpret_cast<float*>(w + ws_align(slots * sizeof(float2)));
  }
  // The ragged layer step: its prologue launch (norm + RoPE of every
  // sequence's q and k, the append, and the batch kernel's counter reset)
  // writes qn and the new cache rows, then the batch runs as plain ragged
  // decode over qn, refusing key counts past the bound.
  const bool ragged_layer = fused != nullptr && seq_row_off != nullptr;
  if (ragged_layer) {
    a.q = fused->qn_out;
    a.strict = 1;
  } else if (fused != nullptr) {
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
  const dim3 grid(groups, a.max_splits, s.n_seqs);
  const uint32_t G = s.n_heads / s.n_kv_heads;
  hipError_t e;
  if (ragged_layer) {
    e = launch_ragged_prologue(*fused, seq_row_off, n_keys_dev, s.n_seqs, s.max_n_keys,
                               s.n_heads, s.n_kv_heads, s.head_dim, queue, groups, st);
    if (e != hipSuccess) return e;
  }
  if (batch) {
    // The counters start at zero: a kernel, not a memset, so that a captured
    // graph replays it (the ragged layer step's prologue zeroes them).
    if (!ragged_layer)
      hipLaunchKernelGGL(queue_zero_kernel, dim3(1), dim3(kBatchMaxGroups), 0, st, queue, groups);
    const dim3 bgrid(groups, kBatchWG / groups > 0 ? kBatchWG / groups : 1);
    e = s.head_dim == 128 ? launch_batch_d<128>(a, bgrid, G, KH, s.n_seqs, queue, st)
                          : launch_batch_d<64>(a, bgrid, G, KH, s.n_seqs, queue, st);
  } else {
    e = s.head_dim == 128 ? launch_split_d<128>(a, grid, G, KH, ragged, st)
                          : launch_split_d<64>(a, grid, G, KH, ragged, st);
  }
  if (e != hipSuccess || a.max_splits <= 1) return e;
  const dim3 mgrid(s.n_heads, s.head_dim / 4 / kMergeCols, s.n_seqs);
  // A batch's heads have few splits each (~24 for 64 sequences): one wave
  // per (sequence, head, column chunk) folds up to 64 in one round, and all
  // of them are resident at once (64 sequences: 10.7 -> 5.1 us, the call 671
  // -> 666 us).
  const bool narrow = ragged && a.max_splits <= kMergeNarrowSplits;
  if (s.head_dim == 128) {
    if (narrow)
      hipLaunchKernelGGL((decode_merge_kernel<128, kMergeNarrow>), mgrid, dim3(kMergeNarrow), 0,
                         st, a);
    else
      hipLaunchKernelGGL((decode_merge_kernel<128, kMergeThreads>), mgrid, dim3(kMergeThreads),
                         0, st, a);
  } else {
    if (narrow)
      hipLaunchKernelGGL((decode_merge_kernel<64, kMergeNarrow>), mgrid, dim3(kMergeNarrow), 0,
                         st, a);
    else
      hipLaunchKernelGGL((decode_merge_kernel<64, kMergeThreads>), mgrid, dim3(kMergeThreads), 0,
                         st, a);
  }
  return hipGetLastError();
}

}  // namespace flk
