// Prefill kernel pieces: arguments, key-tile counts, and the staging of one
// 64-key K/V tile through registers into LDS.
#pragma once

#include "common.hpp"

namespace flk {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 64;    // query-head rows per q tile
constexpr int kBK = 64;      // keys per tile
constexpr int kPThreads = 512;  // 8 waves: 4 row blocks x 2 key halves
constexpr int kHalfKB = 2;      // 16-key blocks per wave per tile
constexpr uint32_t kMinPairedWG = 192;    // paired mode when it yields this many
constexpr uint32_t kTargetSplitWG = 256;  // split mode aims at one workgroup per CU
constexpr uint32_t kMinKtPerSplit = 2;
#ifndef FLK_PREFILL_OPAD
#define FLK_PREFILL_OPAD 4  // padding of the combine's o rows in LDS (floats)
#endif
#ifndef FLK_PREFILL_AHEAD
#define FLK_PREFILL_AHEAD 1  // operand groups read from LDS ahead of their MFMAs
#endif

struct PrefillArgs {
  const float* q;
  const float* kcache;
  const float* vcache;
  float* o;
  float2* part_ml;   // [slot][kRows]
  float* part_acc;   // [slot][kRows][D]
  uint32_t n_heads, n_kv_heads, group;
  uint32_t n_queries, pos0;
  uint32_t q_per_tile, n_qtiles;
  uint32_t paired, work_per_kvh;
  uint32_t kt_per_split, max_splits;
  float scale_log2e;  // fr(1/sqrt(d) * log2(e)): scores in base-2 units
};

__host__ __device__ __forceinline__ uint32_t qtile_kt(uint32_t qt, uint32_t q_per_tile,
                                                      uint32_t n_queries, uint32_t pos0) {
  const uint32_t q_end = (qt + 1) * q_per_tile < n_queries ? (qt + 1) * q_per_tile : n_queries;
  return (pos0 + q_end + kBK - 1) / kBK;
}

// gfx9 buffer-descriptor word 3 for untyped 32-bit-element loads.
constexpr int kBufferWord3 = 0x00020000;

// Rows of key tile kt of `cache` (K or V) into registers: NPF float4 per
// thread. The descriptor covers the tile's live rows only (rows from kt * kBK,
// at most kBK, at most up to the last key), so a row past the last key reads
// as 0.
template <int D, int NPF = kBK * D / 4 / kPThreads>
__device__ __forceinline__ void load_rows(float4 (&pr)[NPF], const float* cache,
                                          const PrefillArgs& a, uint32_t kvh, uint32_t kt,
                                          uint32_t n_keys_total, int tid) {
  const uint32_t key0 = kt * kBK;
  const uint32_t rows = min(n_keys_total - key0, (uint32_t)kBK);
  const uint32_t row_bytes = a.n_kv_heads * D * 4;
  const size_t base = (size_t)key0 * row_bytes + (size_t)kvh * D * 4;
  const uint32_t n_bytes = (rows - 1) * row_bytes + D * 4;
  const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(reinterpret_cast<const char*>(cache) + base), 0, n_bytes, kBufferWord3);
  typedef float f4v __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int i = 0; i < NPF; i++) {
    const int f = tid + kPThreads * i;
    const int r = f / (D / 4), c4 = f % (D / 4);
    const f4v x = __builtin_bit_cast(
        f4v, __builtin_amdgcn_raw_buffer_load_b128(rr, r * (int)row_bytes + 16 * c4, 0, 0));
    pr[i] = make_float4(x.x, x.y, x.z, x.w);
  }
}

// K and V rows of key tile kt into registers.
template <int D, int NPF = kBK * D / 4 / kPThreads>
__device__ __forceinline__ void load_tile(float4 (&pk)[NPF], float4 (&pv)[NPF],
                                          const PrefillArgs& a, uint32_t kvh, uint32_t kt,
                                          uint32_t n_keys_total, int tid) {
  load_rows<D>(pk, a.kcache, a, kvh, kt, n_keys_total, tid);
  load_rows<D>(pv, a.vcache, a, kvh, kt, n_keys_total, tid);
}

// Position of float4 chunk c within a K row in LDS. PERM (head_dim 128)
// swaps chunks 8..15 with 16..23, so that 32 lanes reading 16 key rows at
// chunks g and 8 + g (or 16 + g and 24 + g) hit distinct banks of the 128.
template <int D, bool PERM>
__device__ __forceinline__ int k_chunk_pos(int c) {
  if constexpr (PERM && D == 128) return (c >= 8 && c < 24) ? (c ^ 24) : c;
  return c;
}

template <int D, bool PERM = false, int NPF = kBK * D / 4 / kPThreads>
__device__ __forceinline__ void store_k(const float4 (&pk)[NPF], float* k_lds, int tid) {
#pragma unroll
  for (int i = 0; i < NPF; i++) {
    const int f = tid + kPThreads * i;
    *reinterpret_cast<float4*>(&k_lds[(f / (D / 4)) * (D + 4) +
                                      4 * k_chunk_pos<D, PERM>(f % (D / 4))]) = pk[i];
  }
}
template <int D, int NPF = kBK * D / 4 / kPThreads>
__device__ __forceinline__ void store_v(const float4 (&pv)[NPF], float* v_lds, int tid) {
#pragma unroll
  for (int i = 0; i < NPF; i++) {
    const int f = tid + kPThreads * i;
    *reinterpret_cast<float4*>(&v_lds[(f / (D / 4)) * D + 4 * (f % (D / 4))]) = pv[i];
  }
}

// Registers of one key tile into one LDS buffer (K rows padded to D + 4).
template <int D, bool PERM = false, int NPF = kBK * D / 4 / kPThreads>
__device__ __forceinline__ void store_tile(const float4 (&pk)[NPF], const float4 (&pv)[NPF],
                                           float* k_lds, float* v_lds, int tid) {
  store_k<D, PERM>(pk, k_lds, tid);
  store_v<D>(pv, v_lds, tid);
}

}  // namespace flk
