// Shared device helpers and launch plumbing for libflock_attn (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flock_attn.h"
#include "../../include/flock_q8.h"
#include "../../include/flock_wire.h"
#include "../../include/flock_graph.h"
#include "trig.hpp"

namespace flk {

constexpr int kWave = 64;

// ---------------------------------------------------------------- rounding --
// The CPU oracle evaluates in f64 and rounds to f32 at fixed points. For +, -,
// *, / and sqrt of two f32 operands, rounding the f64 result to f32 equals the
// f32 operation itself (53 >= 2*24 + 2), so plain f32 arithmetic matches it.
// Two compound forms need f64 on the device to match bit for bit:
//   fma32(a, b, c) = f32(f64(a*b) + c): the f64 sum rounds before the f32 one.
//   1/sqrt(y)      = f32(1 / sqrt(f64 y)): one f32 rounding of the compound.
__device__ __forceinline__ float fma32(float a, float b, float c) {
  return (float)((double)a * (double)b + (double)c);
}
__device__ __forceinline__ float rsqrt_once(float y) { return (float)(1.0 / sqrt((double)y)); }

// ------------------------------------------------------------- lane shuffles --
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// Data-parallel-primitive move: lane i reads lane f(i) of v within its row of
// 16 lanes (CTRL is the DPP control word). Runs as a VALU modifier, no LDS.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124;       // row_ror:4, lane i <- (i - 4) mod 16 within its row
constexpr int kDppRor8 = 0x128;       // row_ror:8, lane i <- i ^ 8 within its row
constexpr int kDppRor12 = 0x12C;      // row_ror:12, lane i <- (i + 4) mod 16 within its row
constexpr int kDppHalfMirror = 0x141; // lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <- 15 - i within 16

// v of lane i ^ M, for M = 1, 2, 4, 8, on DPP (no LDS traffic): quad_perm for
// 1 and 2, row_ror:8 (exactly i ^ 8) for 8, row_ror:12 or :4 for 4 (lane i
// with bit 2 clear reads i + 4, with it set i - 4). (row_ror:n hands lane i
// the value of lane (i - n) mod 16 of its row.) Strides 16 and 32 leave the
// row: see swap_pair.
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "xor_lane");
  if constexpr (M == 1) {
    return dpp<kDppXor1>(v);
  } else if constexpr (M == 2) {
    return dpp<kDppXor2>(v);
  } else if constexpr (M == 8) {
    return dpp<kDppRor8>(v);
  } else {
    const float up = dpp<kDppRor12>(v), down = dpp<kDppRor4>(v);  // lanes i + 4, i - 4
    return (threadIdx.x & 4) ? down : up;
  }
}

// gfx950 v_permlane16_swap / v_permlane32_swap with v in both operands: the
// two results hold, in every lane i, v of lane i and of lane i ^ M (one of
// each; which one is which depends on bit log2(M) of i). For a commutative op
// op(lo, hi) is therefore the xor-M butterfly step in every lane, computed on
// the VALU instead of through the LDS pipeline (ds_swizzle, ds_bpermute).
// Needs every lane of the wave active.
template <int M>
__device__ __forceinline__ void swap_pair(float v, float& lo, float& hi) {
  static_assert(M == 16 || M == 32, "swap_pair");
  const int x = __builtin_bit_cast(int, v);
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    lo = __builtin_bit_cast(float, (int)r[0]);
    hi = __builtin_bit_cast(float, (int)r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    lo = __builtin_bit_cast(float, (int)r[0]);
    hi = __builtin_bit_cast(float, (int)r[1]);
  }
}
// v + (v of lane i ^ M); the same float in both lanes (a + b == b + a).
template <int M>
__device__ __forceinline__ float sum_xor(float v) {
  float lo, hi;
  swap_pair<M>(v, lo, hi);
  return lo + hi;
}
template <int M>
__device__ __forceinline__ float max_xor(float v) {
  float lo, hi;
  swap_pair<M>(v, lo, hi);
  return fmaxf(lo, hi);
}

// The pairwise tree over P lanes (P a power of two <= 64) as an xor
// butterfly, strides P/2 .. 1: every lane of an aligned group of P ends with
// the group's tree total.
template <int P>
__device__ __forceinline__ float lane_tree(float v) {
  if constexpr (P >= 64) v = sum_xor<32>(v);
  if constexpr (P >= 32) v = sum_xor<16>(v);
  if constexpr (P >= 16) v = v + xor_lane<8>(v);
  // After the stride-8 step lanes j and j ^ 8 hold the same float, so one
  // row_ror:4 (lane i - 4, i.e. i ^ 4 or (i ^ 4) ^ 8) serves as xor 4.
  if constexpr (P >= 16) v = v + dpp<kDppRor4>(v);
  else if constexpr (P >= 8) v = v + xor_lane<4>(v);
  if constexpr (P >= 4) v = v + xor_lane<2>(v);
  if constexpr (P >= 2) v = v + xor_lane<1>(v);
  return v;
}

// Sum over aligned groups of `width` lanes (a power of two <= 64); every lane
// of a group ends with the same total (each step adds a pair of equal-shaped
// partial sums, so both partners compute the same float). Must be called with
// all lanes of the wave active.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(width >= 1 && width <= 64 && (width & (width - 1)) == 0, "width");
  if (width >= 2) v += dpp<kDppXor1>(v);
  if (width >= 4) v += dpp<kDppXor2>(v);
  if (width >= 8) v += dpp<kDppHalfMirror>(v);
  if (width >= 16) v += dpp<kDppMirror>(v);
  if (width >= 32) v = sum_xor<16>(v);  // the two 16-lane halves of each 32-lane group
  if (width >= 64) v = sum_xor<32>(v);
  return v;
}

// --------------------------------------------------------- RoPE + RMSNorm ----
// One wave owns one head vector of D (64 or 128) floats: lane l holds element
// l and, for D = 128, element l + 64; g0, g1 are the gains of those elements. The sum of squares follows the reference
// kernel's order exactly (rmsnorm.wgsl:45-66, rmsnormRef ops_ref.ts:20-49 with
// wg = 128): partial[t] = x_t^2 (one element per partial), then a pairwise
// tree with strides 64, 32, ..., 1. Stride 64 is in-lane; the rest is an xor
// butterfly, after which every lane holds the tree total (each level's value
// in lane i equals tree[i mod stride], and addition is commutative).
//
// tree_sum64 is that butterfly (strides 32, 16, ..., 1, every lane adding its
// partner i ^ stride) with 32 and 16 on the permlane swaps and the in-row
// strides on DPP: 8 is row_ror:8 (exactly
// i ^ 8); 4 is row_ror:4, which reads lane (i - 4) mod 16 -- that is i ^ 4
// or (i ^ 4) ^ 8, and after the stride-8 step lanes j and j ^ 8 hold the same
// float (a + b and b + a), so it is the same value; 2 and 1 are quad_perm.
__device__ __forceinline__ float tree_sum64(float p) {
  p = sum_xor<32>(p);
  p = sum_xor<16>(p);
  p = p + dpp<kDppRor8>(p);
  p = p + dpp<kDppRor4>(p);
  p = p + dpp<kDppXor2>(p);
  p = p + dpp<kDppXor1>(p);
  return p;
}

template <int D>
__device__ __forceinline__ void head_rmsnorm(float& e0, float& e1, float g0, float g1, float eps) {
  float p = e0 * e0;
  if (D == 128) p = p + e1 * e1;
  p = tree_sum64(p);
  // rmsnorm.wgsl:68 with the reference's rounding: fr(fr(sum / n) + eps), then
  // 1/sqrt as one rounding (ops_ref.ts:39-45).
  const float mean = p / (float)D;
  const float scale = rsqrt_once(mean + eps);
  e0 = (e0 * scale) * g0;
  if (D == 128) e1 = (e1 * scale) * g1;
}

// cos/sin of RoPE angle theta = fr(pos * inv_freq[j]) (ops_ref.ts:75-76): the
// product of an f32 and an integer position is formed exactly in f64 and
// rounded once, and cos/sin are rounded once to f32 like fr(Math.cos(theta)).
__device__ __forceinline__ float2 rope_cos_sin(float inv_f, uint32_t pos) {
  const float theta = (float)((double)pos * (double)inv_f);
  float s, c;
  sincos_f32_exact(theta, s, c);
  return make_float2(c, s);
}

// One rotated element: `x` is this element, `y` its pair partner, `first`
// says whether this element is the pair's a (else b); cs = (cos, sin).
// a' = fr(-b*s + fr(a*c)) and b' = fr(b*c + fr(a*s)), the f64 sum rounding
// before the f32 one (ops_ref.ts:80-88).
__device__ __forceinline__ float rope_rot(float x, float y, bool first, float2 cs) {
  if (first) return (float)(-(double)y * (double)cs.y + (double)(x * cs.x));
  return (float)((double)x * (double)cs.x + (double)(y * cs.y));
}

// RoPE on one head vector held as above (rope.wgsl:50-78, ropeRef
// ops_ref.ts:65-92), with cs[j] = rope_cos_sin(inv_freq[j], pos) for the
// vector's position precomputed in LDS (one table per position, shared by
// all heads of a token). NEOX pairs (j, j + D/2): for D = 128 both halves sit
// in the same lane; for D = 64 the partner is lane l ^ 32. NORM pairs (2j,
// 2j+1): the partner is lane l ^ 1.
template <int D>
__device__ __forceinline__ void head_rope(float& e0, float& e1, const float2* cs, int pairing,
                                          int lane) {
  constexpr int half = D / 2;
  if (pairing == FLK_ROPE_NORM) {
    const float p0 = shfl_xor(e0, 1);
    const float p1 = (D == 128) ? shfl_xor(e1, 1) : 0.f;
    const bool first = (lane & 1) == 0;
    if (lane < D) e0 = rope_rot(e0, p0, first, cs[lane >> 1]);
    if (D == 128) e1 = rope_rot(e1, p1, first, cs[(lane + 64) >> 1]);
  } else if (D == 128) {
    const float a = e0, b = e1;  // elements j = lane and j + 64
    const float2 c = cs[lane];
    e0 = rope_rot(a, b, true, c);
    e1 = rope_rot(b, a, false, c);
  } else {
    const float p0 = shfl_xor(e0, 32);
    const bool first = lane < half;
    e0 = rope_rot(e0, p0, first, cs[first ? lane : lane - half]);
  }
}

// ---------------------------------------------------------------- launches --
struct Stream {
  static hipStream_t get();
};

// Internal launchers (return a hipError_t; the C ABI maps it to FLK_ERR_HIP).
hipError_t launch_rmsnorm(const float* x, const float* g, float* o, uint32_t n, uint32_t n_vecs,
                          float eps, hipStream_t st);
hipError_t launch_rope(float* x, const float* inv_freq, uint32_t n_tokens, uint32_t n_heads,
                       uint32_t head_dim, uint32_t pos0, int32_t pairing, hipStream_t st);
hipError_t launch_kv_append(const float* kn, const float* v, float* kcache, float* vcache,
                            uint32_t n_tokens, uint32_t pos0, uint32_t n_kv_heads,
                            uint32_t head_dim, hipStream_t st);
hipError_t launch_qk_prologue(const float* q_raw, const float* k_raw, const float* v_raw,
                              const float* gq, const float* gk, const float* inv_freq, float eps,
                              int32_t pairing, float* qn_out, float* kcache, float* vcache,
                              uint32_t n_tokens, uint32_t pos0, uint32_t n_heads,
                              uint32_t n_kv_heads, uint32_t head_dim, hipStream_t st,
                              uint32_t in_stride = 0);

// Decode: plan + launch. `fused` carries the prologue inputs for
// flk_decode_layer (null q_raw means plain decode).
struct DecodeFused {
  const float* q_raw = nullptr;
  const float* k_raw = nullptr;
  const float* v_raw = nullptr;
  const float* gq = nullptr;
  const float* gk = nullptr;
  const float* inv_freq = nullptr;
  float eps = 0.f;
  int32_t pairing = 0;
  float* qn_out = nullptr;
  float* kcache_w = nullptr;
  float* vcache_w = nullptr;
};

struct DecodeShape {
  uint32_t n_heads, n_kv_heads, head_dim;
  uint32_t n_seqs;      // 1 unless ragged
  uint32_t max_n_keys;  // n_keys for a single sequence
};

// The ragged layer step's prologue: per sequence b, norm + RoPE of q and k at
// position n_keys[b] - 1, qn_out rows and the append at row seq_row_off[b] +
// n_keys[b] - 1; also zeroes n_queue counters at `queue` (when not null).
hipError_t launch_ragged_prologue(const DecodeFused& f, const uint64_t* seq_row_off,
                                  const uint32_t* n_keys, uint32_t n_seqs, uint32_t max_n_keys,
                                  uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                  uint32_t* queue, uint32_t n_queue, hipStream_t st);

uint64_t decode_ws_bytes(const DecodeShape& s);
uint64_t decode_ws_bound(const DecodeShape& s);
hipError_t launch_decode(const float* q, const float* kcache, const float* vcache, float* o,
                         const uint64_t* seq_row_off, const uint32_t* n_keys_dev,
                         const DecodeShape& s, const DecodeFused* fused, void* ws, hipStream_t st);

struct PrefillPlan {
  uint32_t rows_per_tile;   // query-head rows of one work item (all share a kv head)
  uint32_t q_per_tile;      // rows_per_tile / group
  uint32_t n_qtiles;
  uint32_t paired;          // 1: each workgroup runs q tiles t and n_qtiles-1-t whole
  uint32_t work_per_kvh;    // workgroups per kv head
  uint32_t ktiles_per_split;
  uint32_t max_splits;      // splits of the heaviest q tile (split mode)
  uint64_t partial_slots;   // n_qtiles * max_splits * n_kv_heads when splitting
};
PrefillPlan prefill_plan(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t n_queries, uint32_t pos0);
uint64_t prefill_ws_bytes(const PrefillPlan& p, uint32_t head_dim);
uint64_t prefill_ws_bound(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t max_queries, uint32_t max_keys);
hipError_t launch_prefill(const float* q, const float* kcache, const float* vcache, float* o,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t n_queries, uint32_t pos0, void* ws, hipStream_t st);

// ------------------------------------------------------------------ argmax --
// argmax.wgsl's contract: (va, ia) beats (vb, ib) if va > vb, or va == vb and
// ia < ib; the empty result is (-3.4028235e38, 0xffffffff), and a NaN never
// wins (every comparison with it is false). The order of comparisons does not
// change the result, so any reduction tree gives the reference's answer.
constexpr float kArgmaxNoVal = -3.40282347e38f;
constexpr uint32_t kArgmaxNoIdx = 0xffffffffu;

__device__ __forceinline__ bool argmax_better(float va, uint32_t ia, float vb, uint32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// Reduces every thread's (v, i) of the workgroup (blockDim.x a multiple of 64,
// at most 1024) and writes the winner to val[blockIdx.x], idx[blockIdx.x].
// Every thread of the workgroup must call it.
__device__ __forceinline__ void argmax_block_store(float v, uint32_t i, float* val, uint32_t* idx) {
  __shared__ float s_v[16];
  __shared__ uint32_t s_i[16];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(v, m, kWave);
    const uint32_t oi = (uint32_t)__shfl_xor((int)i, m, kWave);
    if (argmax_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[wave] = v;
    s_i[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); w++)
      if (argmax_better(s_v[w], s_i[w], v, i)) {
        v = s_v[w];
        i = s_i[w];
      }
    val[blockIdx.x] = v;
    idx[blockIdx.x] = i;
  }
}

// ------------------------------------------------------------- Q8_0 matvec --
// best_val / best_idx: per-workgroup argmax partials (null for a plain
// matvec); *n_workgroups receives the launch's workgroup count.
struct Q8Fuse {
  const float* norm_gain = nullptr;  // x <- rmsnorm(x) (per token, n = n_cols)
  float norm_eps = 0.f;
  const float* up = nullptr;         // x <- swiglu(x, up)
  const float* res = nullptr;        // o <- res + W x
  float* act = nullptr;              // (gate, up) row pairs -> act = swiglu (<= 1024 columns)
};
hipError_t launch_q8_matvec(const uint8_t* qs, const uint16_t* scales, const float* x, float* o,
                            uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens, hipStream_t st,
                            float* best_val = nullptr, uint32_t* best_idx = nullptr,
                            uint32_t* n_workgroups = nullptr, const Q8Fuse* fuse = nullptr);
uint32_t q8_max_workgroups(uint32_t n_rows, uint32_t n_cols);

// op 0: swiglu(a, b); op 1: a + b (elementwise.wgsl).
hipError_t launch_elementwise(int op, const float* a, const float* b, float* o, uint32_t n,
                              hipStream_t st);

hipError_t launch_embed(const int8_t* qs, const uint16_t* scales, const uint32_t* ids,
                        uint32_t n_tokens, uint32_t vocab, uint32_t hidden, float* out,
                        hipStream_t st);
hipError_t launch_advance(uint32_t* state, uint32_t delta, const uint32_t* value, uint32_t* log,
                          uint32_t log_len, hipStream_t st);

// dir 0: f32 -> f16 (wire pack), 1: f16 -> f32 (wire unpack).
hipError_t launch_wire(int dir, const void* in, void* out, uint64_t n, hipStream_t st);

// ------------------------------------------------------------------- head ----
uint64_t argmax_ws_bytes(uint32_t n);
hipError_t launch_argmax(const float* x, uint32_t n, float* oval, uint32_t* oidx, void* ws,
                         hipStream_t st);
uint64_t lm_head_ws_bytes(uint32_t vocab, uint32_t hidden);
hipError_t launch_lm_head(const float* x, const float* gain, float eps, const uint8_t* qs,
                          const uint16_t* scales, uint32_t vocab, uint32_t hidden, float* normed,
                          float* logits, float* oval, uint32_t* oidx, void* ws, hipStream_t st);

// Workspace layout (split-K partials): [(m, l) pairs][pad to 256 B][acc rows].
constexpr uint64_t kWsAlign = 256;
__host__ __device__ constexpr uint64_t ws_align(uint64_t n) {
  return (n + kWsAlign - 1) / kWsAlign * kWsAlign;
}

}  // namespace flk
