// Causal GQA prefill attention on v_mfma_f32_32x32x2f32, 128-row q tiles
// (head_dim 128). Same algorithm and results contract as prefill.hip's
// 64-row kernel (attention_prefill.wgsl:75-175: query pos0 + i attends keys
// 0 .. pos0 + i, online softmax over 64-key tiles); the tile shape is what
// changes:
//
// A q tile is 128 query-head rows sharing one kv head ((128 / G) queries x
// the G heads). 8 waves: wave w owns rows 32 (w & 3) .. + 31 and key half
// w >> 2 (32 keys) of every 64-key K/V tile staged in LDS.
//   S^T = K Q^T     32x32x2: A = K [32 keys x 2 dims] from LDS (lane l: key
//                   l % 32), B = Q^T [2 dims x 32 rows] from registers (lane
//                   l: row l % 32), loaded once per q tile. k-step 4g + u
//                   reads dim 8g + 4(l / 32) + u, so a lane reads its K
//                   operands of 4 steps as one float4. Out: lane l, register
//                   i holds S^T[key 8(i / 4) + 4(l / 32) + i % 4][row l % 32].
//   softmax         a row lives in lanes l and l ^ 32 (16 keys each).
//   O^T += V^T P^T  B = P^T straight from the S^T registers: k-step s uses
//                   register s, i.e. keys 8(s / 4) + s % 4 (lanes < 32) and
//                   that + 4 (lanes >= 32); A = V^T read with the same key
//                   order. Output channel block c (32 channels), row i holds
//                   channel 4i + c, so one float4 of a V row (channels 4j ..
//                   4j + 3) feeds the four blocks' MFMAs of a k-step, and the
//                   16 lanes of a read group take 256 contiguous bytes.
// Per flop this reads half the LDS operands of the 16x16x4 kernel (each
// 32x32x2 MFMA does twice the work of a 16x16x4 one per operand float) and
// stages each K/V tile once for 128 rows instead of 64.
//
// Work split ("pair pieces"). Q tiles are paired high with low (hi = n - 1 -
// p, lo = p; the middle tile of an odd count is its own pair), so a pair's
// causal key tiles add up to about the same for every p. The pair's units
// (hi's key tiles, then lo's) are cut into m equal pieces; workgroup (p, k,
// kv head) runs piece k: a segment of hi's key tiles and/or of lo's. A
// segment that is a whole q tile writes o; otherwise it writes an (m, l, acc)
// partial that prefill32_merge_kernel folds in piece order. m = 1 is the
// plain pairing (no partials); m = 2 splits the 2048-token prompt's pairs
// into 256 equal workgroups; a single q tile (a 64-token chunk onto a long
// cache) is m pieces of its keys.
#include "prefill.hpp"

namespace flk {

typedef float floatx16 __attribute__((ext_vector_type(16)));

#ifndef FLK_P32_AHEAD
#define FLK_P32_AHEAD 1  // LDS operands read one group / k-step ahead of their MFMAs
#endif
#ifndef FLK_P32_SCHAINS
#define FLK_P32_SCHAINS 1  // accumulation chains of the S MFMAs per wave
#endif

constexpr int kRows32 = 128;       // query-head rows per q tile
constexpr uint32_t kMaxPieces = 64;
constexpr uint32_t kMaxItems = 512;  // cap on workgroups when pairs are cut into pieces

// Start (in units of the pair's sequence) of piece k of m over u units.
__host__ __device__ __forceinline__ uint32_t piece_start(uint32_t k, uint32_t u, uint32_t m) {
  return (uint32_t)((uint64_t)k * u / m);
}
// The non-empty piece that holds unit x (< u).
__host__ __device__ __forceinline__ uint32_t piece_of(uint32_t x, uint32_t u, uint32_t m) {
  const uint32_t k = (uint32_t)(((uint64_t)(x + 1) * m + u - 1) / u) - 1;
  return k < m ? k : m - 1;
}
// Partial slot of (tile t of pair p: 0 = hi, 1 = lo; piece k) for kv head kvh.
__host__ __device__ __forceinline__ size_t piece_slot(const PrefillArgs& a, uint32_t t,
                                                      uint32_t p, uint32_t k, uint32_t kvh) {
  const uint32_t n_pairs = (a.n_qtiles + 1) / 2;
  return (((size_t)t * n_pairs + p) * a.pieces + k) * a.n_kv_heads + kvh;
}

// q rows of tile qt in the B-operand layout: lane l (row l % 32 of the wave's
// block, half hl = l / 32) holds dims 8g + 4hl .. + 3 for every g, scaled by
// scale * log2(e) so that S^T comes out in base-2 units.
template <int D>
__device__ __forceinline__ void load_q32(float (&qreg)[D / 2], const PrefillArgs& a,
                                         uint32_t kvh, uint32_t qt) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, hl = lane >> 5;
  const uint32_t q0 = qt * a.q_per_tile;
  const uint32_t r = (wave & 3) * 32 + j;
  const uint32_t qi = q0 + r / a.group;
  const uint32_t h = kvh * a.group + r % a.group;
  const bool row_ok = r < a.q_per_tile * a.group && qi < a.n_queries;
  const float* src =
      a.q + ((size_t)(row_ok ? qi : q0) * a.n_heads + (row_ok ? h : kvh * a.group)) * D + 4 * hl;
#pragma unroll
  for (int g = 0; g < D / 8; g++) {
    const float4 v = *reinterpret_cast<const float4*>(src + 8 * g);
    qreg[4 * g + 0] = v.x * a.scale_log2e;
    qreg[4 * g + 1] = v.y * a.scale_log2e;
    qreg[4 * g + 2] = v.z * a.scale_log2e;
    qreg[4 * g + 3] = v.w * a.scale_log2e;
  }
}

// Key tiles [kt0, kt1) of q tile qt; writes o rows (normalised) when `final`,
// else partial slot `slot`. With nxt_qt >= 0 the next segment's first key
// tile (nxt_kt0) is requested into pk/pv during the last key tile and its q
// rows into qreg after the loop; that segment then runs with preloaded.
template <int D, int NPF = kBK * D / 4 / kPThreads>
__device__ __forceinline__ void run_seg32(const PrefillArgs& a, float* k_lds, float* v_lds,
                                          uint32_t kvh, uint32_t qt, uint32_t kt0, uint32_t kt1,
                                          bool final, size_t slot, float (&qreg)[D / 2],
                                          float4 (&pk)[NPF], float4 (&pv)[NPF], bool preloaded,
                                          int nxt_qt, uint32_t nxt_kt0) {
  constexpr int LDK = D + 4;  // padded K row in LDS (floats)
  constexpr int NG = D / 8;   // S: groups of 4 k-steps (8 dims)
  constexpr int NST = 16;     // PV: k-steps of 2 keys over the wave's 32 keys
  constexpr int CB = D / 32;  // O^T channel blocks of 32 channels
  static_assert(CB == 4, "one float4 of a V row feeds the four channel blocks");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = wave >> 2;  // which 32 keys of every tile this wave takes
  const int j = lane & 31;     // row within the wave's 32-row block
  const int hl = lane >> 5;
  const uint32_t n_keys_total = a.pos0 + a.n_queries;
  const uint32_t q0 = qt * a.q_per_tile;

  const uint32_t r = (wave & 3) * 32 + j;
  const uint32_t qi = q0 + r / a.group;
  const uint32_t h = kvh * a.group + r % a.group;
  const bool row_ok = r < a.q_per_tile * a.group && qi < a.n_queries;
  const uint32_t qpos = a.pos0 + qi;

  if (!preloaded) {
    load_tile<D>(pk, pv, a, kvh, kt0, n_keys_total, tid);
    load_q32<D>(qreg, a, kvh, qt);
  }
  floatx16 oacc[CB];
#pragma unroll
  for (int c = 0; c < CB; c++)
#pragma unroll
    for (int i = 0; i < 16; i++) oacc[c][i] = 0.f;
  // Running reference (log2 units, finite) and this lane's share of the
  // denominator (its 16 keys of each tile; the row's two lanes are summed at
  // the end).
  float m_run = -1e30f, l_run = 0.f;

  const bool all_rows = a.q_per_tile * a.group == kRows32 && q0 + a.q_per_tile <= a.n_queries;
  auto full_tile = [&](uint32_t key0) { return all_rows && key0 + kBK - 1 <= a.pos0 + q0; };

  __syncthreads();  // LDS may still hold the previous segment's combine data
  store_tile<D>(pk, pv, k_lds, v_lds, tid);
  load_tile<D>(pk, pv, a, kvh, kt0 + 1 < kt1 ? kt0 + 1 : kt0, n_keys_total, tid);
  __syncthreads();

  const float* kr0 = &k_lds[(half * 32 + j) * LDK + 4 * hl];
  const float* vr0 = &v_lds[(half * 32 + 4 * hl) * D + 4 * j];
  auto k_group = [&](const float* kb, int g) {
    return *reinterpret_cast<const floatx4*>(kb + 8 * g);
  };
  // V row of k-step s: key 8(s / 4) + s % 4 (+ 4 for lanes >= 32, in vr0).
  auto v_step = [&](const float* vb, int s) {
    return *reinterpret_cast<const floatx4*>(vb + (8 * (s / 4) + (s % 4)) * D);
  };

  for (uint32_t kt = kt0; kt < kt1; kt++) {
    const uint32_t key0 = kt * kBK;
    const int buf = (kt - kt0) & 1;
    const float* kb = kr0 + buf * (kBK * LDK);
    const float* vb = vr0 + buf * (kBK * D);

    floatx4 kg[2];
    if (FLK_P32_AHEAD) kg[0] = k_group(kb, 0);
    __builtin_amdgcn_sched_barrier(0);

    // ---- S^T = K Q^T ----------------------------------------------------------
    // FLK_P32_SCHAINS accumulation chains (groups dealt round-robin), added
    // at the end.
    floatx16 sch[FLK_P32_SCHAINS];
#pragma unroll
    for (int c = 0; c < FLK_P32_SCHAINS; c++)
#pragma unroll
      for (int i = 0; i < 16; i++) sch[c][i] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; g++) {
      if (FLK_P32_AHEAD && g + 1 < NG) kg[(g + 1) & 1] = k_group(kb, g + 1);
      if (!FLK_P32_AHEAD) kg[g & 1] = k_group(kb, g);
      __builtin_amdgcn_sched_barrier(0);
      // The next tile goes from registers into the free buffers, K a quarter
      // and V three quarters of the way through S; the tile after it is
      // requested right after each half.
      if (g == NG / 4 && kt + 1 < kt1) {
        store_k<D>(pk, k_lds + (buf ^ 1) * (kBK * LDK), tid);
        load_rows<D>(pk, a.kcache, a, kvh, kt + 2 < kt1 ? kt + 2 : kt + 1, n_keys_total, tid);
      }
      if (g == 3 * NG / 4 && kt + 1 < kt1) {
        store_v<D>(pv, v_lds + (buf ^ 1) * (kBK * D), tid);
        load_rows<D>(pv, a.vcache, a, kvh, kt + 2 < kt1 ? kt + 2 : kt + 1, n_keys_total, tid);
      }
      // During the last tile, the next segment's first key tile is requested.
      if (g == NG / 2 && kt + 1 == kt1 && nxt_qt >= 0)
        load_tile<D>(pk, pv, a, kvh, nxt_kt0, n_keys_total, tid);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; u++)
        sch[g % FLK_P32_SCHAINS] = __builtin_amdgcn_mfma_f32_32x32x2f32(
            kg[g & 1][u], qreg[4 * g + u], sch[g % FLK_P32_SCHAINS], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    floatx16 sacc = sch[0];
#pragma unroll
    for (int c = 1; c < FLK_P32_SCHAINS; c++) sacc += sch[c];

    floatx4 vg[2];
    if (FLK_P32_AHEAD) vg[0] = v_step(vb, 0);  // before the softmax, which does not need it
    __builtin_amdgcn_sched_barrier(0);

    // ---- online softmax of this lane's row (base 2) ---------------------------
    // As in the 64-row kernel: the reference m_run moves only when some
    // score of the wave exceeds it by more than 8, and then only for the rows
    // that passed; other rows are multiplied by exactly 1.
    if (!full_tile(key0)) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t key = key0 + half * 32 + 8 * (i / 4) + 4 * hl + (i % 4);
        if (!(row_ok && key <= qpos)) sacc[i] = -INFINITY;
      }
    }
    float lmx = sacc[0];
#pragma unroll
    for (int i = 1; i < 16; i++) lmx = fmaxf(lmx, sacc[i]);
    if (__builtin_amdgcn_ballot_w64(lmx > m_run + 8.f) != 0) {  // uniform branch
      const float mx = max_xor<32>(lmx);
      const bool up = mx > m_run + 8.f;
      const float corr = up ? __builtin_amdgcn_exp2f(m_run - mx) : 1.f;
      l_run *= corr;
#pragma unroll
      for (int c = 0; c < CB; c++) oacc[c] *= corr;
      m_run = up ? mx : m_run;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float p = __builtin_amdgcn_exp2f(sacc[i] - m_run);
      sacc[i] = p;
      l_run += p;
    }

    // ---- O^T += V^T P^T --------------------------------------------------------
#pragma unroll
    for (int s = 0; s < NST; s++) {
      if (FLK_P32_AHEAD && s + 1 < NST) vg[(s + 1) & 1] = v_step(vb, s + 1);
      if (!FLK_P32_AHEAD) vg[s & 1] = v_step(vb, s);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CB; c++)
        oacc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(vg[s & 1][c], sacc[s], oacc[c], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // tile kt + 1 stored; buffer of tile kt free again
  }

  if (nxt_qt >= 0) load_q32<D>(qreg, a, kvh, (uint32_t)nxt_qt);  // the next segment's rows
  l_run = sum_xor<32>(l_run);  // the row's denominator: its two lanes

  // ---- combine the two key halves of each row through LDS --------------------
  // Register i of block c holds channel 4 * ch(i) + c, ch(i) = 8(i / 4) +
  // 4hl + i % 4, so the four blocks' values of one i are a float4 of
  // contiguous channels. Every wave has passed the last tile's barrier: the
  // whole LDS (K and V buffers) is free for the upper waves' (m, l, acc).
  constexpr int LDO = D + FLK_PREFILL_OPAD;
  static_assert(2 * kRows32 + kRows32 * LDO <= 2 * kBK * LDK + 2 * kBK * D,
                "combine data exceeds the LDS tile buffers");
  float* m_lds = k_lds;                // [kRows32] m, then [kRows32] l
  float* o_lds = k_lds + 2 * kRows32;  // [kRows32][LDO], over the K and V buffers
  if (half == 1) {
    float* dst = o_lds + r * LDO;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int ch = 8 * (i / 4) + 4 * hl + (i % 4);
      *reinterpret_cast<float4*>(dst + 4 * ch) =
          make_float4(oacc[0][i], oacc[1][i], oacc[2][i], oacc[3][i]);
    }
    if (hl == 0) {
      m_lds[r] = m_run;
      m_lds[kRows32 + r] = l_run;
    }
  }
  __syncthreads();
  if (half == 1) return;
  const float m2 = m_lds[r], l2 = m_lds[kRows32 + r];
  const float M = fmaxf(m_run, m2);
  const float w1 = __builtin_amdgcn_exp2f(m_run - M);
  const float w2 = __builtin_amdgcn_exp2f(m2 - M);
  const float L = l_run * w1 + l2 * w2;
  const float* o2 = o_lds + r * LDO;
  float* dst;
  if (final) {
    if (!row_ok) return;
    dst = a.o + ((size_t)qi * a.n_heads + h) * D;
  } else {
    dst = a.part_acc + (slot * kRows32 + r) * D;
    if (hl == 0) a.part_ml[slot * kRows32 + r] = make_float2(M, L);
  }
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int ch = 8 * (i / 4) + 4 * hl + (i % 4);
    const float4 p = *reinterpret_cast<const float4*>(o2 + 4 * ch);
    float4 v = make_float4(oacc[0][i] * w1 + p.x * w2, oacc[1][i] * w1 + p.y * w2,
                           oacc[2][i] * w1 + p.z * w2, oacc[3][i] * w1 + p.w * w2);
    if (final) v = make_float4(v.x / L, v.y / L, v.z / L, v.w / L);
    *reinterpret_cast<float4*>(dst + 4 * ch) = v;
  }
}

// Pair p's tiles and units: hi = n - 1 - p, lo = p (none for the middle tile).
struct PairUnits {
  uint32_t hi, lo, kth, ktl, u;
};
__host__ __device__ __forceinline__ PairUnits pair_units(const PrefillArgs& a, uint32_t p) {
  PairUnits pu;
  pu.hi = a.n_qtiles - 1 - p;
  pu.lo = p;
  pu.kth = qtile_kt(pu.hi, a.q_per_tile, a.n_queries, a.pos0);
  pu.ktl = pu.lo < pu.hi ? qtile_kt(pu.lo, a.q_per_tile, a.n_queries, a.pos0) : 0;
  pu.u = pu.kth + pu.ktl;
  return pu;
}

template <int D>
__global__ __launch_bounds__(kPThreads) void prefill32_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[2 * kBK * (D + 4) + 2 * kBK * D];
  float* k_lds = lds;
  float* v_lds = lds + 2 * kBK * (D + 4);
  const uint32_t kvh = blockIdx.x % a.n_kv_heads;
  const uint32_t item = blockIdx.x / a.n_kv_heads;
  const uint32_t p = item / a.pieces, k = item % a.pieces;
  const PairUnits pu = pair_units(a, p);
  const uint32_t u0 = piece_start(k, pu.u, a.pieces), u1 = piece_start(k + 1, pu.u, a.pieces);
  if (u0 == u1) return;  // an empty piece (fewer units than pieces); uniform
  const bool has_hi = u0 < pu.kth, has_lo = u1 > pu.kth;
  const uint32_t lo0 = u0 > pu.kth ? u0 - pu.kth : 0;
  constexpr int NPF = kBK * D / 4 / kPThreads;
  float qreg[D / 2];
  float4 pk[NPF], pv[NPF];
  if (has_hi)
    run_seg32<D>(a, k_lds, v_lds, kvh, pu.hi, u0, u1 < pu.kth ? u1 : pu.kth,
                 u0 == 0 && u1 >= pu.kth, piece_slot(a, 0, p, k, kvh), qreg, pk, pv, false,
                 has_lo ? (int)pu.lo : -1, lo0);
  if (has_lo)
    run_seg32<D>(a, k_lds, v_lds, kvh, pu.lo, lo0, u1 - pu.kth, u0 <= pu.kth && u1 == pu.u,
                 piece_slot(a, 1, p, k, kvh), qreg, pk, pv, has_hi, -1, 0);
}

// grid (kv head, q tile, 128 / RPB row chunks); D/4 lanes per row, each owning
// a float4 of channels. Folds the partials of a q tile cut over several
// pieces, in piece order, with log-sum-exp weights; a tile run whole by one
// piece was written by the kernel and exits here.
constexpr int kP32MergeBatch = 8;
template <int D>
__global__ __launch_bounds__(256) void prefill32_merge_kernel(PrefillArgs a) {
  constexpr int LPR = D / 4;
  constexpr int RPB = 256 / LPR;
  const uint32_t kvh = blockIdx.x;
  const uint32_t qt = blockIdx.y;
  const uint32_t hi_side = qt >= a.n_qtiles - 1 - qt;
  const uint32_t p = hi_side ? a.n_qtiles - 1 - qt : qt;
  const PairUnits pu = pair_units(a, p);
  const uint32_t t = hi_side ? 0 : 1;
  const uint32_t s = t == 0 ? 0 : pu.kth, e = t == 0 ? pu.kth : pu.u;
  const uint32_t k0 = piece_of(s, pu.u, a.pieces), k1 = piece_of(e - 1, pu.u, a.pieces);
  if (k0 == k1) return;
  const uint32_t r = blockIdx.z * RPB + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  const uint32_t qi = qt * a.q_per_tile + r / a.group;
  if (r >= a.q_per_tile * a.group || qi >= a.n_queries) return;
  const uint32_t h = kvh * a.group + r % a.group;
  float M = -INFINITY, L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t b0 = k0; b0 <= k1; b0 += kP32MergeBatch) {
    float2 ml[kP32MergeBatch];
    float4 pa[kP32MergeBatch];
    // Unconditional loads: pieces past k1 reload k1 and, like empty pieces
    // (which wrote nothing), get weight 0.
#pragma unroll
    for (int i = 0; i < kP32MergeBatch; i++) {
      const uint32_t kk = min(b0 + i, k1);
      const size_t slot = piece_slot(a, t, p, kk, kvh);
      ml[i] = a.part_ml[slot * kRows32 + r];
      pa[i] = reinterpret_cast<const float4*>(a.part_acc + (slot * kRows32 + r) * D)[c];
    }
#pragma unroll
    for (int i = 0; i < kP32MergeBatch; i++) {
      const uint32_t kk = b0 + i;
      const bool live = kk <= k1 && piece_start(kk, pu.u, a.pieces) <
                                        piece_start(kk + 1, pu.u, a.pieces);
      if (!live) ml[i].x = -INFINITY;
    }
    float mx = M;
#pragma unroll
    for (int i = 0; i < kP32MergeBatch; i++) mx = fmaxf(mx, ml[i].x);  // piece b0 is live
    const float wo = __builtin_amdgcn_exp2f(M - mx);  // m in log2 units; exp2(-inf) = 0
    L *= wo;
    A.x *= wo;
    A.y *= wo;
    A.z *= wo;
    A.w *= wo;
#pragma unroll
    for (int i = 0; i < kP32MergeBatch; i++) {
      const float w = __builtin_amdgcn_exp2f(ml[i].x - mx);
      L = fmaf(ml[i].y, w, L);
      A.x = fmaf(pa[i].x, w, A.x);
      A.y = fmaf(pa[i].y, w, A.y);
      A.z = fmaf(pa[i].z, w, A.z);
      A.w = fmaf(pa[i].w, w, A.w);
    }
    M = mx;
  }
  float4* dst = reinterpret_cast<float4*>(a.o + ((size_t)qi * a.n_heads + h) * D);
  dst[c] = make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
}

// ------------------------------------------------------------------ plan ----
// Pieces per pair: the m in 1 .. kMaxPieces that minimises the makespan
// estimate rounds(m) * u / m (+1 unit when there are partials to merge),
// where rounds(m) = ceil(items / kTargetSplitWG) and items = pairs * kv heads
// * m <= kMaxItems; u is pair 0's unit count (the pairs' counts differ by at
// most a few units).
static uint32_t choose_pieces(uint32_t n_pairs, uint32_t n_kv_heads, uint32_t u) {
  const uint64_t base = (uint64_t)n_pairs * n_kv_heads;
  uint32_t best = 1;
  double best_span = 0;
  for (uint32_t m = 1; m <= kMaxPieces && m <= u; m++) {
    const uint64_t items = base * m;
    if (m > 1 && items > kMaxItems) break;
    const uint64_t rounds = (items + kTargetSplitWG - 1) / kTargetSplitWG;
    const double span = (double)rounds * u / m + (m > 1 ? 1.0 : 0.0);
    if (m == 1 || span < best_span) {
      best = m;
      best_span = span;
    }
  }
  return best;
}

#ifndef FLK_PREFILL32
#define FLK_PREFILL32 1  // 0: every call takes the 64-row kernel
#endif

bool prefill32_fits(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                    uint32_t n_queries) {
  return FLK_PREFILL32 && head_dim == 128 && (uint64_t)n_queries * (n_heads / n_kv_heads) > (uint64_t)kRows;
}

PrefillPlan prefill32_plan(uint32_t n_heads, uint32_t n_kv_heads, uint32_t n_queries,
                           uint32_t pos0) {
  PrefillPlan p{};
  const uint32_t group = n_heads / n_kv_heads;
  p.x32 = 1;
  p.rows_per_tile = kRows32;
  p.q_per_tile = kRows32 / group;
  p.n_qtiles = (n_queries + p.q_per_tile - 1) / p.q_per_tile;
  const uint32_t n_pairs = (p.n_qtiles + 1) / 2;
  const uint32_t kth = qtile_kt(p.n_qtiles - 1, p.q_per_tile, n_queries, pos0);
  const uint32_t u = kth + (p.n_qtiles > 1 ? qtile_kt(0, p.q_per_tile, n_queries, pos0) : 0);
  p.pieces = choose_pieces(n_pairs, n_kv_heads, u);
  p.paired = p.pieces == 1;
  p.work_per_kvh = n_pairs * p.pieces;
  p.max_splits = p.pieces;
  p.partial_slots =
      p.pieces > 1 ? (uint64_t)(p.n_qtiles > 1 ? 2 : 1) * n_pairs * p.pieces * n_kv_heads : 0;
  return p;
}

// Partial slots of any plan with n_queries <= max_queries, pos0 + n_queries
// <= max_keys: per q-tile count, pieces are at most min(kMaxPieces,
// kMaxItems / (pairs * kv heads), units) and units at most two tiles' worth
// of the longest cache.
uint64_t prefill32_slots_bound(uint32_t n_heads, uint32_t n_kv_heads, uint32_t max_queries,
                               uint32_t max_keys) {
  const uint32_t qpt = kRows32 / (n_heads / n_kv_heads);
  const uint64_t max_qt = (max_queries + qpt - 1) / qpt;
  const uint64_t max_u = 2 * (((uint64_t)max_keys + kBK - 1) / kBK);
  uint64_t best = 0;
  for (uint64_t nqt = 1; nqt <= max_qt; nqt++) {
    const uint64_t pairs = (nqt + 1) / 2;
    const uint64_t base = pairs * n_kv_heads;
    uint64_t m = kMaxPieces;
    if (kMaxItems / base < m) m = kMaxItems / base;
    if (max_u < m) m = max_u;
    if (m <= 1) continue;
    const uint64_t slots = (nqt > 1 ? 2 : 1) * pairs * m * n_kv_heads;
    if (slots > best) best = slots;
  }
  return best;
}

template <int D>
static hipError_t launch_prefill32_d(const PrefillArgs& a, const PrefillPlan& p, hipStream_t st) {
  const dim3 grid(a.n_kv_heads * p.work_per_kvh);
  hipLaunchKernelGGL(prefill32_kernel<D>, grid, dim3(kPThreads), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.pieces <= 1) return e;
  constexpr int RPB = 256 / (D / 4);
  const dim3 mgrid(a.n_kv_heads, p.n_qtiles, kRows32 / RPB);
  hipLaunchKernelGGL(prefill32_merge_kernel<D>, mgrid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_prefill32(const PrefillArgs& a, const PrefillPlan& p, hipStream_t st) {
  return launch_prefill32_d<128>(a, p, st);
}

}  // namespace flk
