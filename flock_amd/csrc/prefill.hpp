// Prefill kernel pieces: arguments, key-tile counts, and the loads that bring
// one 64-key K/V tile from HBM straight into LDS.
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
#ifndef FLK_PREFILL_KPERM
#define FLK_PREFILL_KPERM 1  // K rows stored with chunks 8..15 and 16..23 swapped (D = 128)
#endif
constexpr bool kKPerm = FLK_PREFILL_KPERM != 0;

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

// Position of float4 chunk c within a K row in LDS (an involution). PERM
// (head_dim 128) swaps chunks 8..15 with 16..23, so that 32 lanes reading 16
// key rows at chunks g and 8 + g (or 16 + g and 24 + g) hit distinct banks of
// the 128.
template <int D, bool PERM>
__device__ __forceinline__ int k_chunk_pos(int c) {
  if constexpr (PERM && D == 128) return (c >= 8 && c < 24) ? (c ^ 24) : c;
  return c;
}

// ---- key tiles straight into LDS -------------------------------------------
// A key tile goes from HBM to LDS with buffer_load_dwordx4 ... lds: each such
// wave instruction writes 64 consecutive 16-byte LDS slots, lane l into slot
// l, from the address lane l names, so the LDS layout is set by which float4
// of the tile each lane fetches. The K tile is kBK rows of D + 4 floats (D/4 +
// 1 slots; the last slot of a row is padding, fetched from an offset past the
// descriptor's end, which writes zeros), its chunks placed by k_chunk_pos; the
// V tile is kBK rows of D floats in natural order. Wave w issues the wave
// instructions w, w + 8, ...: D/4 + 1 of them for K, D/4 for V. The descriptor
// covers the tile's live rows only, so rows past the last key arrive as zeros
// too. The loads count on vmcnt: a wait for vmcnt(0) and then a barrier make
// a tile visible to every wave.
constexpr uint32_t kPastEnd = 0x7ffffff0u;  // an offset beyond every descriptor

template <int D>
struct TileOffsets {
  static constexpr int KS = D / 4 + 1;         // slots of a K row
  static constexpr int KW = kBK * KS / 64;     // K wave instructions per tile
  static constexpr int VW = kBK * D / 4 / 64;  // V wave instructions per tile
  static constexpr int KI = (KW + 7) / 8;      // per wave (the last one for wave 0 only)
  static constexpr int VI = VW / 8;            // per wave
  static_assert(KW == 8 * (KI - 1) + 1 && VW == 8 * VI, "wave instructions per tile");
  uint32_t k[KI];
  uint32_t v[VI];
};

// This lane's byte offsets within a tile's descriptor: the same for every
// tile of every q tile.
template <int D>
__device__ __forceinline__ void tile_offsets(TileOffsets<D>& t, uint32_t row_bytes, int wave,
                                             int lane) {
  using T = TileOffsets<D>;
#pragma unroll
  for (int i = 0; i < T::KI; i++) {
    const int s = 64 * (wave + 8 * i) + lane;
    const int row = s / T::KS, pos = s % T::KS;
    t.k[i] = pos < D / 4 && row < kBK ? row * row_bytes + 16 * k_chunk_pos<D, kKPerm>(pos)
                                      : kPastEnd;
  }
#pragma unroll
  for (int i = 0; i < T::VI; i++) {
    const int s = 64 * (wave + 8 * i) + lane;
    t.v[i] = (s / (D / 4)) * row_bytes + 16 * (s % (D / 4));
  }
}

#define FLK_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// Requests key tile kt of kv head kvh into one K and one V buffer. `wave`
// must be wave-uniform: it selects the LDS addresses.
template <int D>
__device__ __forceinline__ void request_tile(const PrefillArgs& a, float* k_buf, float* v_buf,
                                             uint32_t kvh, uint32_t kt, uint32_t n_keys_total,
                                             const TileOffsets<D>& t, int wave) {
  using T = TileOffsets<D>;
  const uint32_t key0 = kt * kBK;
  const uint32_t rows = min(n_keys_total - key0, (uint32_t)kBK);
  const uint32_t row_bytes = a.n_kv_heads * D * 4;
  const size_t base = (size_t)key0 * row_bytes + (size_t)kvh * D * 4;
  const uint32_t n_bytes = (rows - 1) * row_bytes + D * 4;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(reinterpret_cast<const char*>(a.kcache) + base), 0, n_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(reinterpret_cast<const char*>(a.vcache) + base), 0, n_bytes, kBufferWord3);
#pragma unroll
  for (int i = 0; i < T::KI; i++) {
    const int j = wave + 8 * i;
    if (i + 1 < T::KI || j < T::KW)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, FLK_LDS_PTR(k_buf + 256 * j), 16, t.k[i], 0, 0,
                                               0);
  }
#pragma unroll
  for (int i = 0; i < T::VI; i++)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, FLK_LDS_PTR(v_buf + 256 * (wave + 8 * i)), 16,
                                             t.v[i], 0, 0, 0);
}

// The two LDS buffer pairs as four distinct LDS objects: the compiler then
// sees that reads of one pair do not depend on loads in flight into the other.
struct TileBuffers {
  float* k0;
  float* k1;
  float* v0;
  float* v1;
};

// s_waitcnt vmcnt(0), with expcnt and lgkmcnt left at their maxima.
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0f70); }

}  // namespace flk
