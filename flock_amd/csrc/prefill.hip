// Causal GQA prefill attention as tiled flash attention on fp32 MFMA.
//
// The reference (attention_prefill.wgsl:75-175) runs one workgroup per
// (query, head), streams every key of that query through scalar FMAs and two
// barrier-heavy tree reductions per 64-key tile. Here a work item is a "q
// tile" of 64 query-head rows that share one kv head ((64 / G) queries x the
// G heads of the group), so every 64-key K/V tile staged in LDS serves 64
// rows, and both products run on v_mfma_f32_16x16x4f32 (f32 in, f32 out).
//
// Per 64-key tile, each of 8 waves owns 16 rows (one 16-column block) and one
// half (32 keys) of the tile; the two halves of a row keep separate online-
// softmax states and are combined through LDS when the q tile is done:
//   S^T = K Q^T     A = K block [16 keys x 4 dims] from LDS, B = Q^T from
//                   registers (loaded once); out lane l, reg i holds
//                   S^T[key 4(l/16)+i][row l%16].
//   softmax         every column (one query-head row) lives in lanes with the
//                   same l%16: in-lane max/sum over 16 values, then lane xor
//                   16 and 32 (permlane swaps). Running (m, l) per lane, no
//                   LDS.
//   O^T += V^T P^T  B = P^T taken directly from the S^T registers (the key
//                   order inside a k-step is permuted identically on both
//                   operands); A = V^T read from LDS. Output row m of channel
//                   block c is channel CB*m + c (CB = D/16), so a lane reads
//                   its CB values of a key as contiguous float4s and, at the
//                   end, holds 4*CB contiguous output channels.
// The d-summation of S uses dim (D/4)*(l/16) + s at step s (any permutation
// of the summed index is the same dot product), so each lane reads D/4
// contiguous floats of a K row from LDS.
//
// Each tile's K/V rows go from HBM straight into LDS (buffer_load_dwordx4
// ... lds) while the previous tile is computed: no registers, no LDS store
// instructions, and one wait + barrier per tile. The loads go through a
// buffer descriptor made per tile (scalar registers): a lane's offsets within
// the tile are the same for every tile, so the fetch costs no per-tile
// address arithmetic, and rows past the last key arrive as 0. Causal bound:
// query at absolute position p sees keys 0..p (attention_prefill.wgsl:90),
// applied per element.
//
// Scheduling (1-D grid, workgroup id = kv head + n_kv_heads * work item, so
// with 8 kv heads the workgroups of one kv head share an XCD and its L2):
//   paired: work item w runs q tiles n_qtiles-1-w and w whole (their causal
//           key counts add up to about the same for every w); writes o.
//   split:  too few q tiles to fill the GPU (chunked prefill onto a long
//           cache): work item (q tile, split) runs a range of key tiles and
//           writes an (m, l, acc) partial that prefill_merge_kernel combines.
#include <type_traits>

#include "prefill.hpp"

namespace flk {

// Requests this lane's row of q tile qt in the B-operand layout of S^T = K
// Q^T: D/4 floats from dim (D/4) * lg.
template <int D>
__device__ __forceinline__ void fetch_q(float4 (&qraw)[D / 16], const PrefillArgs& a,
                                        uint32_t kvh, uint32_t qt) {
  constexpr int DS = D / 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const uint32_t q0 = qt * a.q_per_tile;
  const uint32_t r = (wave & 3) * 16 + lc;
  const uint32_t qi = q0 + r / a.group;
  const uint32_t h = kvh * a.group + r % a.group;
  const bool row_ok = r < a.q_per_tile * a.group && qi < a.n_queries;
  const float4* src = reinterpret_cast<const float4*>(
      a.q + ((size_t)(row_ok ? qi : q0) * a.n_heads + (row_ok ? h : kvh * a.group)) * D + DS * lg);
#pragma unroll
  for (int s4 = 0; s4 < DS / 4; s4++) qraw[s4] = src[s4];
}

// The fetched row pre-multiplied by scale * log2(e), so that S^T comes out in
// base-2 units.
template <int D>
__device__ __forceinline__ void scale_q(float (&qreg)[D / 4], const float4 (&qraw)[D / 16],
                                        const PrefillArgs& a) {
#pragma unroll
  for (int s4 = 0; s4 < D / 16; s4++) {
    qreg[4 * s4 + 0] = qraw[s4].x * a.scale_log2e;
    qreg[4 * s4 + 1] = qraw[s4].y * a.scale_log2e;
    qreg[4 * s4 + 2] = qraw[s4].z * a.scale_log2e;
    qreg[4 * s4 + 3] = qraw[s4].w * a.scale_log2e;
  }
}

// Runs key tiles [kt0, kt1) for q tile qt of kv head kvh; writes o rows
// (normalised) when `final`, else the partial of `slot`. Tile kt0 is (or, with
// preloaded, already was) requested into LDS buffer pair p0, and this lane's
// q row into qraw (the caller's). With nxt_qt >= 0, the first key tile of q
// tile nxt_qt (key tile 0) is requested into the free buffer pair, and its q
// rows into qraw, at the start of the last key tile, so that their latency
// overlaps that tile and the combine; the next call passes preloaded = true
// and that pair as its p0.
template <int D>
__device__ __forceinline__ void run_qtile(const PrefillArgs& a, const TileBuffers& lb,
                                          uint32_t kvh, uint32_t qt, uint32_t kt0, uint32_t kt1,
                                          bool final, size_t slot, float4 (&qraw)[D / 16],
                                          const TileOffsets<D>& toff, uint32_t p0, bool preloaded,
                                          int nxt_qt) {
  constexpr int LDK = D + 4;        // padded K row in LDS (floats)
  constexpr int DS = D / 4;         // k-steps of 4 dims for S
  constexpr int CB = D / 16;        // channel blocks of O^T

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = wave >> 2;  // which 32 keys of every tile this wave takes
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int lc = lane & 15;    // column within the 16-block = row of this lane
  const int lg = lane >> 4;    // lane group 0..3
  // V-read swizzle (D = 128): A-operand lane lc supplies channel 8*lc + (c ^
  // 4*sw(lc)) of block c with sw(m) = ((m >> 2) ^ (m >> 3)) & 1, so the two
  // float4s of a key row are read in swapped order by lanes lc and lc ^ 4 and
  // by lanes lc and lc ^ 8: any 8 consecutive lanes cover 32 distinct banks
  // and any 16 cover 64. Output row m of the O^T accumulators then holds
  // channel 8*m + (c ^ 4*sw(m)); for this lane's rows m = 4*lg + j that is
  // sw_wr.
  const int sw_rd = CB == 8 ? ((lc >> 2) ^ (lc >> 3)) & 1 : 0;
  const int sw_wr = CB == 8 ? (lg ^ (lg >> 1)) & 1 : 0;
  const uint32_t n_keys_total = a.pos0 + a.n_queries;
  const uint32_t q0 = qt * a.q_per_tile;

  // ---- this lane's row: r -> (query, head) -----------------------------------
  const uint32_t r = (wave & 3) * 16 + lc;
  const uint32_t qi = q0 + r / a.group;
  const uint32_t h = kvh * a.group + r % a.group;
  const bool row_ok = r < a.q_per_tile * a.group && qi < a.n_queries;
  const uint32_t qpos = a.pos0 + qi;

  auto k_buf = [&](int b) { return b ? lb.k1 : lb.k0; };
  auto v_buf = [&](int b) { return b ? lb.v1 : lb.v0; };
  if (!preloaded) {
    request_tile<D>(a, k_buf(p0), v_buf(p0), kvh, kt0, n_keys_total, toff, wave_u);
    fetch_q<D>(qraw, a, kvh, qt);
  }
  float qreg[D / 4];
  scale_q<D>(qreg, qraw, a);
  wait_vm0();       // this wave's share of tile kt0 is in LDS
  __syncthreads();  // every wave's; the previous q tile's combine is done
  // The next q tile's rows: in flight during the first key tile, then held.
  if (nxt_qt >= 0) fetch_q<D>(qraw, a, kvh, (uint32_t)nxt_qt);
  floatx4 oacc[CB];
#pragma unroll
  for (int c = 0; c < CB; c++) oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Running reference m_run (log2 units; finite, so that a masked key's
  // weight exp2(-inf - m_run) is exactly 0) and this lane's share of the
  // denominator (its keys only; summed over the row's lanes at the end).
  float m_run = -1e30f, l_run = 0.f;

  // A tile needs no causal mask when its last key is at or before the q
  // tile's first query position and every row of the q tile is live.
  const bool all_rows = a.q_per_tile * a.group == kRows && q0 + a.q_per_tile <= a.n_queries;
  auto full_tile = [&](uint32_t key0) { return all_rows && key0 + kBK - 1 <= a.pos0 + q0; };

  // Two LDS buffer pairs: tile kt is computed from pair (p0 + kt - kt0) & 1
  // while tile kt + 1 loads into the other one; a wait + barrier ends each
  // tile.

  // Operands are read from LDS kAhead groups ahead of the MFMAs that use
  // them; sched_barrier keeps the compiler from sinking each read next to its
  // first use, where every group's LDS latency would stall the wave.
  constexpr int kAhead = FLK_PREFILL_AHEAD;
  constexpr int NG = DS / 4;        // S: groups of 4 k-steps (one float4 per chain)
  constexpr int NST = kHalfKB * 4;  // PV: k-steps of 4 keys
  // Lane group lg reads chunks 8 lg .. 8 lg + 7 (D = 128) of its key rows.
  const int kr0 = ((half * kHalfKB) * 16 + lc) * LDK + 4 * k_chunk_pos<D, kKPerm>((DS / 4) * lg);
  const int vr0 = ((half * kHalfKB) * 16 + 4 * lg) * D + CB * lc;
  auto k_group = [&](const float* kt_lds_base, int g, int b) {
    return *reinterpret_cast<const floatx4*>(kt_lds_base + b * 16 * LDK + 4 * g);
  };
  auto v_step = [&](const float* vt_lds_base, int st, int c4) {
    const int b = st / 4, i = st % 4;
    return *reinterpret_cast<const floatx4*>(vt_lds_base + (b * 16 + i) * D + 4 * (c4 ^ sw_rd));
  };

  // The buffer of every tile is a compile-time choice (B), so that the
  // compiler sees that the operand reads of one buffer do not depend on the
  // loads in flight into the other and places no wait for them.
  auto tile = [&](uint32_t kt, auto bc) {
    constexpr int B = decltype(bc)::value;
    float* const k_cur = B ? lb.k1 : lb.k0;
    float* const v_cur = B ? lb.v1 : lb.v0;
    float* const k_nxt = B ? lb.k0 : lb.k1;
    float* const v_nxt = B ? lb.v0 : lb.v1;
    const uint32_t key0 = kt * kBK;
    if (kt + 1 < kt1)
      request_tile<D>(a, k_nxt, v_nxt, kvh, kt + 1, n_keys_total, toff, wave_u);
    else if (nxt_qt >= 0)  // the next q tile's first key tile
      request_tile<D>(a, k_nxt, v_nxt, kvh, 0, n_keys_total, toff, wave_u);
    const float* kb = k_cur + kr0;
    const float* vb = v_cur + vr0;

    // The first K groups of this tile (in LDS since the barrier).
    floatx4 kg[kAhead + 1][kHalfKB];
#pragma unroll
    for (int g = 0; g < kAhead; g++)
#pragma unroll
      for (int b = 0; b < kHalfKB; b++) kg[g][b] = k_group(kb, g, b);
    __builtin_amdgcn_sched_barrier(0);

    // ---- S^T = K Q^T ------------------------------------------------------------
    // Each MFMA depends on the previous one of its block's chain, so the
    // blocks' chains are issued interleaved, step by step.
    floatx4 sacc[kHalfKB];
#pragma unroll
    for (int b = 0; b < kHalfKB; b++) sacc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < NG; g++) {
      if (g + kAhead < NG) {
#pragma unroll
        for (int b = 0; b < kHalfKB; b++) kg[(g + kAhead) % (kAhead + 1)][b] = k_group(kb, g + kAhead, b);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int b = 0; b < kHalfKB; b++)
          sacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kg[g % (kAhead + 1)][b][j], qreg[4 * g + j],
                                                         sacc[b], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }

    // The first V steps go out before the softmax, which does not need them.
    floatx4 vg[kAhead + 1][CB / 4];
#pragma unroll
    for (int st = 0; st < kAhead; st++)
#pragma unroll
      for (int c4 = 0; c4 < CB / 4; c4++) vg[st][c4] = v_step(vb, st, c4);
    __builtin_amdgcn_sched_barrier(0);

    // ---- online softmax of this lane's row (base 2) ----------------------------
    // Scores are base-2 already (q carries scale * log2(e)), so every weight is
    // one v_exp_f32 against the reference m_run. The reference moves only when
    // some score of the wave exceeds it by more than 8 (a factor 256): the
    // check needs only each lane's own 8 scores, and the row's maximum across
    // its four lane groups is formed only then (rarely after the first tile).
    // Otherwise the weights are taken against the old reference -- each at
    // most 256 -- and nothing is rescaled. Tiles wholly below the causal
    // diagonal with every row live skip the mask.
    if (!full_tile(key0)) {
#pragma unroll
      for (int b = 0; b < kHalfKB; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t key = key0 + (half * kHalfKB + b) * 16 + 4 * lg + i;
          sacc[b][i] = row_ok && key <= qpos ? sacc[b][i] : -INFINITY;
        }
    }
    float lmx = sacc[0][0];
#pragma unroll
    for (int b = 0; b < kHalfKB; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) lmx = fmaxf(lmx, sacc[b][i]);
    if (__builtin_amdgcn_ballot_w64(lmx > m_run + 8.f) != 0) {  // uniform branch
      // Only rows whose own maximum passed the threshold move their reference;
      // the others keep it and are multiplied by exactly 1, so a row's result
      // depends on its own keys only (causality holds bit for bit).
      float mx = max_xor<16>(lmx);
      mx = max_xor<32>(mx);
      const bool up = mx > m_run + 8.f;
      const float corr = up ? __builtin_amdgcn_exp2f(m_run - mx) : 1.f;
      l_run *= corr;
#pragma unroll
      for (int c = 0; c < CB; c++) oacc[c] *= corr;
      m_run = up ? mx : m_run;
    }
#pragma unroll
    for (int b = 0; b < kHalfKB; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float p = __builtin_amdgcn_exp2f(sacc[b][i] - m_run);
        sacc[b][i] = p;
        l_run += p;
      }

    // ---- O^T += V^T P^T ---------------------------------------------------------
#pragma unroll
    for (int st = 0; st < NST; st++) {
      if (st + kAhead < NST) {
#pragma unroll
        for (int c4 = 0; c4 < CB / 4; c4++)
          vg[(st + kAhead) % (kAhead + 1)][c4] = v_step(vb, st + kAhead, c4);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CB; c++)
        oacc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vg[st % (kAhead + 1)][c / 4][c % 4],
                                                       sacc[st / 4][st % 4], oacc[c], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm0();       // this wave's share of the next tile is in LDS
    __syncthreads();  // every wave's; every wave is done with this tile's buffers
  };
  uint32_t kt = kt0;
  if (p0 != 0 && kt < kt1) tile(kt++, std::integral_constant<int, 1>{});
  for (; kt + 1 < kt1; kt += 2) {
    tile(kt, std::integral_constant<int, 0>{});
    tile(kt + 1, std::integral_constant<int, 1>{});
  }
  if (kt < kt1) tile(kt, std::integral_constant<int, 0>{});

  l_run = sum_xor<16>(l_run);  // the row's denominator: its four lane groups
  l_run = sum_xor<32>(l_run);
  // ---- combine the two key halves of each row through LDS --------------------
  // Lane holds channels 4*CB*lg + CB*j + c of its row. The upper waves park
  // their acc in the last tile's K buffer and (m, l) in its V buffer; the
  // lower waves fold them in and write the row.
  // The last tile's buffers are free (the other pair may hold the next q
  // tile's first key tile).
  // o rows padded to D + FLK_PREFILL_OPAD floats: the 16 lanes of a group
  // hold 16 different rows, which then fall in distinct bank groups.
  constexpr int LDO = D + FLK_PREFILL_OPAD;
  static_assert(kRows * LDO <= kBK * LDK && 2 * kRows <= kBK * D, "combine data exceeds a buffer");
  const int buf_last = (p0 + kt1 - 1 - kt0) & 1;
  float* m_lds = v_buf(buf_last);  // [kRows] m, then [kRows] l
  float* o_lds = k_buf(buf_last);  // [kRows][LDO]
  if (half == 1) {
    float* dst = o_lds + r * LDO + 4 * CB * lg;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int c4 = 0; c4 < CB / 4; c4++)
        *reinterpret_cast<float4*>(dst + CB * j + 4 * (c4 ^ sw_wr)) =
            make_float4(oacc[4 * c4 + 0][j], oacc[4 * c4 + 1][j], oacc[4 * c4 + 2][j],
                        oacc[4 * c4 + 3][j]);
    if (lg == 0) {
      m_lds[r] = m_run;
      m_lds[kRows + r] = l_run;
    }
  }
  __syncthreads();
  if (half == 1) return;
  const float m2 = m_lds[r], l2 = m_lds[kRows + r];
  const float M = fmaxf(m_run, m2);
  // A half that saw no key of this row still holds the initial reference
  // (-1e30, l = 0): its weight exp2(-1e30 - M) is 0.
  const float w1 = __builtin_amdgcn_exp2f(m_run - M);
  const float w2 = __builtin_amdgcn_exp2f(m2 - M);
  const float L = l_run * w1 + l2 * w2;
  const float* o2 = o_lds + r * LDO + 4 * CB * lg;
  float* dst;
  if (final) {
    if (!row_ok) return;
    dst = a.o + ((size_t)qi * a.n_heads + h) * D + 4 * CB * lg;
  } else {
    dst = a.part_acc + (slot * kRows + r) * D + 4 * CB * lg;
    if (lg == 0) a.part_ml[slot * kRows + r] = make_float2(M, L);
  }
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int c4 = 0; c4 < CB / 4; c4++) {
      const float4 p = *reinterpret_cast<const float4*>(o2 + CB * j + 4 * (c4 ^ sw_wr));
      float4 v = make_float4(oacc[4 * c4 + 0][j] * w1 + p.x * w2,
                             oacc[4 * c4 + 1][j] * w1 + p.y * w2,
                             oacc[4 * c4 + 2][j] * w1 + p.z * w2,
                             oacc[4 * c4 + 3][j] * w1 + p.w * w2);
      if (final) v = make_float4(v.x / L, v.y / L, v.z / L, v.w / L);
      *reinterpret_cast<float4*>(dst + CB * j + 4 * (c4 ^ sw_wr)) = v;
    }
}

template <int D>
__global__ __launch_bounds__(kPThreads) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) float k_lds0[kBK * (D + 4)];
  __shared__ __attribute__((aligned(16))) float k_lds1[kBK * (D + 4)];
  __shared__ __attribute__((aligned(16))) float v_lds0[kBK * D];
  __shared__ __attribute__((aligned(16))) float v_lds1[kBK * D];
  const TileBuffers lb{k_lds0, k_lds1, v_lds0, v_lds1};
  const uint32_t kvh = blockIdx.x % a.n_kv_heads;
  const uint32_t w = blockIdx.x / a.n_kv_heads;
  float4 qraw[D / 16];
  TileOffsets<D> toff;
  tile_offsets<D>(toff, a.n_kv_heads * D * 4, threadIdx.x >> 6, threadIdx.x & 63);
  if (a.paired) {
    const uint32_t qt_hi = a.n_qtiles - 1 - w;
    const uint32_t n_hi = qtile_kt(qt_hi, a.q_per_tile, a.n_queries, a.pos0);
    run_qtile<D>(a, lb, kvh, qt_hi, 0, n_hi, true, 0, qraw, toff, 0, false,
                 w < qt_hi ? (int)w : -1);
    if (w < qt_hi)
      run_qtile<D>(a, lb, kvh, w, 0, qtile_kt(w, a.q_per_tile, a.n_queries, a.pos0),
                   true, 0, qraw, toff, n_hi & 1, true, -1);
    return;
  }
  const uint32_t qt = a.n_qtiles - 1 - w / a.max_splits;  // heaviest q tile first
  const uint32_t split = w % a.max_splits;
  const uint32_t n_kt = qtile_kt(qt, a.q_per_tile, a.n_queries, a.pos0);
  const uint32_t ns = (n_kt + a.kt_per_split - 1) / a.kt_per_split;
  if (split >= ns) return;  // uniform per workgroup
  const uint32_t kt0 = split * n_kt / ns;
  const uint32_t kt1 = (split + 1) * n_kt / ns;
  const size_t slot = ((size_t)qt * a.max_splits + split) * a.n_kv_heads + kvh;
  run_qtile<D>(a, lb, kvh, qt, kt0, kt1, ns == 1, slot, qraw, toff, 0, false, -1);
}

// One workgroup per (kv head, q tile, 256 / (D/4) rows); D/4 lanes per row,
// each owning a float4 of channels. Combines the splits of a multi-split q
// tile with log-sum-exp weights in one pass: the splits go in rounds of
// kPMergeBatch whose loads are all issued first (indices past the last split
// reload it and get weight 0, so every load is unconditional), then folded
// against a running maximum. Single-split tiles exit.
constexpr int kPMergeBatch = 8;
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  constexpr int LPR = D / 4;
  constexpr int RPB = 256 / LPR;   // rows per block
  const uint32_t kvh = blockIdx.x;
  const uint32_t qt = blockIdx.y;
  const uint32_t n_kt = qtile_kt(qt, a.q_per_tile, a.n_queries, a.pos0);
  const uint32_t ns = (n_kt + a.kt_per_split - 1) / a.kt_per_split;
  if (ns == 1) return;
  const uint32_t r = blockIdx.z * RPB + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  const uint32_t qi = qt * a.q_per_tile + r / a.group;
  if (r >= a.q_per_tile * a.group || qi >= a.n_queries) return;
  const uint32_t h = kvh * a.group + r % a.group;
  float M = -INFINITY, L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s0 = 0; s0 < ns; s0 += kPMergeBatch) {
    float2 ml[kPMergeBatch];
    float4 pa[kPMergeBatch];
#pragma unroll
    for (int i = 0; i < kPMergeBatch; i++) {
      const uint32_t sp = min(s0 + i, ns - 1);
      const size_t slot = ((size_t)qt * a.max_splits + sp) * a.n_kv_heads + kvh;
      ml[i] = a.part_ml[slot * kRows + r];
      pa[i] = reinterpret_cast<const float4*>(a.part_acc + (slot * kRows + r) * D)[c];
    }
#pragma unroll
    for (int i = 0; i < kPMergeBatch; i++)
      if (s0 + i >= ns) ml[i].x = -INFINITY;  // a reloaded split: weight 0
    float mx = M;
#pragma unroll
    for (int i = 0; i < kPMergeBatch; i++) mx = fmaxf(mx, ml[i].x);  // finite: split s0 is live
    const float wo = __builtin_amdgcn_exp2f(M - mx);  // m is in log2 units; exp2(-inf) = 0
    L *= wo;
    A.x *= wo;
    A.y *= wo;
    A.z *= wo;
    A.w *= wo;
#pragma unroll
    for (int i = 0; i < kPMergeBatch; i++) {
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
PrefillPlan prefill_plan(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t n_queries, uint32_t pos0) {
  PrefillPlan p{};
  const uint32_t group = n_heads / n_kv_heads;
  p.rows_per_tile = kRows;
  p.q_per_tile = kRows / group;
  p.n_qtiles = (n_queries + p.q_per_tile - 1) / p.q_per_tile;
  const uint32_t pairs = (p.n_qtiles + 1) / 2;
  if ((uint64_t)pairs * n_kv_heads >= kMinPairedWG) {
    p.paired = 1;
    p.work_per_kvh = pairs;
    p.ktiles_per_split = 0;
    p.max_splits = 1;
    p.partial_slots = 0;
    return p;
  }
  uint64_t total = 0;
  for (uint32_t qt = 0; qt < p.n_qtiles; qt++) total += qtile_kt(qt, p.q_per_tile, n_queries, pos0);
  total *= n_kv_heads;
  uint64_t ch = (total + kTargetSplitWG - 1) / kTargetSplitWG;
  if (ch < kMinKtPerSplit) ch = kMinKtPerSplit;
  const uint32_t max_kt = qtile_kt(p.n_qtiles - 1, p.q_per_tile, n_queries, pos0);
  const uint64_t ms = (max_kt + ch - 1) / ch;
  p.paired = 0;
  p.ktiles_per_split = (uint32_t)ch;
  p.max_splits = (uint32_t)ms;
  p.work_per_kvh = p.n_qtiles * p.max_splits;
  p.partial_slots = ms > 1 ? (uint64_t)p.n_qtiles * ms * n_kv_heads : 0;
  return p;
}

uint64_t prefill_ws_bytes(const PrefillPlan& p, uint32_t head_dim) {
  if (p.partial_slots == 0) return 0;
  return ws_align(p.partial_slots * kRows * sizeof(float2)) +
         p.partial_slots * kRows * head_dim * sizeof(float);
}

// Upper bound over every plan with n_queries <= max_queries and pos0 +
// n_queries <= max_keys. Only split plans have partials, and only while
// ceil(n_qtiles / 2) * n_kv_heads < kMinPairedWG. In a split plan the last q
// tile alone gives total >= n_kv_heads * max_kt key tiles, so ch >= n_kv_heads
// * max_kt / kTargetSplitWG and ms = ceil(max_kt / ch) <= ceil(kTargetSplitWG /
// n_kv_heads); also ms <= ceil(max_kt / kMinKtPerSplit) with max_kt <=
// ceil(max_keys / kBK).
uint64_t prefill_ws_bound(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t max_queries, uint32_t max_keys) {
  const uint32_t qpt = kRows / (n_heads / n_kv_heads);
  const uint64_t max_qt = (max_queries + qpt - 1) / qpt;
  uint64_t nqt = 0;  // most q tiles a split plan can have
  for (uint64_t t = 1; t <= max_qt && (t + 1) / 2 * n_kv_heads < kMinPairedWG; t++) nqt = t;
  if (nqt == 0) return 0;
  const uint64_t max_kt = ((uint64_t)max_keys + kBK - 1) / kBK;
  const uint64_t by_wg = (kTargetSplitWG + n_kv_heads - 1) / n_kv_heads;
  const uint64_t by_kt = (max_kt + kMinKtPerSplit - 1) / kMinKtPerSplit;
  const uint64_t ms = by_wg < by_kt ? by_wg : by_kt;
  if (ms <= 1) return 0;
  PrefillPlan p{};
  p.partial_slots = nqt * ms * n_kv_heads;
  return prefill_ws_bytes(p, head_dim);
}

template <int D>
static hipError_t launch_prefill_d(const PrefillArgs& a, const PrefillPlan& p, hipStream_t st) {
  const dim3 grid(a.n_kv_heads * p.work_per_kvh);
  hipLaunchKernelGGL(prefill_kernel<D>, grid, dim3(kPThreads), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.paired || p.max_splits <= 1) return e;
  constexpr int RPB = 256 / (D / 4);
  const dim3 mgrid(a.n_kv_heads, p.n_qtiles, kRows / RPB);
  hipLaunchKernelGGL(prefill_merge_kernel<D>, mgrid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_prefill(const float* q, const float* kcache, const float* vcache, float* o,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t n_queries, uint32_t pos0, void* ws, hipStream_t st) {
  const PrefillPlan p = prefill_plan(n_heads, n_kv_heads, head_dim, n_queries, pos0);
  PrefillArgs a{};
  a.q = q;
  a.kcache = kcache;
  a.vcache = vcache;
  a.o = o;
  if (p.partial_slots > 0) {
    char* w = static_cast<char*>(ws);
    a.part_ml = reinterpret_cast<float2*>(w);
    a.part_acc = reinterpret_cast<float*>(w + ws_align(p.partial_slots * kRows * sizeof(float2)));
  }
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.group = n_heads / n_kv_heads;
  a.n_queries = n_queries;
  a.pos0 = pos0;
  a.q_per_tile = p.q_per_tile;
  a.n_qtiles = p.n_qtiles;
  a.paired = p.paired;
  a.work_per_kvh = p.work_per_kvh;
  a.kt_per_split = p.ktiles_per_split;
  a.max_splits = p.max_splits;
  a.scale_log2e = (float)(1.4426950408889634 / sqrt((double)head_dim));
  if (head_dim == 128) return launch_prefill_d<128>(a, p, st);
  return launch_prefill_d<64>(a, p, st);
}

}  // namespace flk
