// Causal GQA prefill attention as tiled flash attention on fp32 MFMA.
//
// The reference (attention_prefill.wgsl:75-175) runs one workgroup per
// (query, head), streams every key of that query through scalar FMAs and two
// barrier-heavy tree reductions per 64-key tile. Here one workgroup owns a
// tile of 128 query-head rows that share one kv head -- (128 / G) queries x
// the G heads of the group -- so every K/V tile staged in LDS is used by 128
// rows, and both products run on v_mfma_f32_16x16x4f32 (f32 in, f32 out).
//
// Per 64-key tile and wave (32 rows = two 16-column blocks):
//   S^T = K Q^T     A = K block [16 keys x 4 dims] from LDS, B = Q^T from
//                   registers (loaded once); out lane l, reg i holds
//                   S^T[key 4(l/16)+i][row l%16].
//   softmax         every column (one query-head row) lives in lanes with the
//                   same l%16: in-lane max/sum over 16 values, then lane xor
//                   16 and 32. Running (m, l) per lane, no LDS.
//   O^T += V^T P^T  B = P^T taken directly from the S^T registers (the key
//                   order inside a k-step is permuted consistently on both
//                   operands), A = V^T read from LDS; out lane l, reg j holds
//                   O^T[channel 4(l/16)+j][row l%16], so the online-softmax
//                   rescale of O is per lane as well.
// The d-summation of S uses dim 32*(l/16) + s at step s (any permutation of the
// summed index is the same dot product), so each lane reads 32 contiguous
// floats of a K row from LDS.
//
// Causal bound: query at absolute position p sees keys 0..p (the reference's
// loop bound, attention_prefill.wgsl:90); applied per element.
// Long rows are split over keys: the grid is (kv head, split, q tile, heaviest
// tile first); single-split tiles normalise and store o, multi-split tiles
// store (m, l, acc) partials that prefill_merge_kernel combines.
#include "common.hpp"

namespace flk {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 128;   // query-head rows per workgroup
constexpr int kBK = 64;      // keys per tile
constexpr int kPThreads = 256;
constexpr uint32_t kMinKtPerSplit = 4;
constexpr uint32_t kTargetItems = 1024;
constexpr uint64_t kMaxSlots = 2048;

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
  uint32_t kt_per_split, max_splits;
  float scale;
};

__device__ __forceinline__ uint32_t tile_kt(const PrefillArgs& a, uint32_t qt) {
  const uint32_t q_end = min((qt + 1) * a.q_per_tile, a.n_queries);
  return (a.pos0 + q_end + kBK - 1) / kBK;
}

__device__ __forceinline__ uint32_t tile_splits(const PrefillArgs& a, uint32_t n_kt) {
  return (n_kt + a.kt_per_split - 1) / a.kt_per_split;
}

template <int D>
__global__ __launch_bounds__(kPThreads) void prefill_kernel(PrefillArgs a) {
  constexpr int LDK = D + 4;        // padded LDS row (floats)
  constexpr int DS = D / 4;         // k-steps of 4 dims
  constexpr int CHB = D / 16;       // 16-channel blocks of O^T
  __shared__ __attribute__((aligned(16))) float k_lds[kBK * LDK];
  __shared__ __attribute__((aligned(16))) float v_lds[kBK * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lc = lane & 15;   // column within a 16-block
  const int lg = lane >> 4;   // lane group 0..3

  const uint32_t kvh = blockIdx.x;
  const uint32_t split = blockIdx.y;
  const uint32_t qt = a.n_qtiles - 1 - blockIdx.z;
  const uint32_t n_kt = tile_kt(a, qt);
  const uint32_t ns = tile_splits(a, n_kt);
  if (split >= ns) return;
  const uint32_t kt0 = split * n_kt / ns;
  const uint32_t kt1 = (split + 1) * n_kt / ns;
  const uint32_t n_keys_total = a.pos0 + a.n_queries;
  const size_t row = (size_t)a.n_kv_heads * D;
  const uint32_t q0 = qt * a.q_per_tile;

  // ---- this lane's two columns: row r -> (query, head) ----------------------
  uint32_t qpos[2];
  bool col_ok[2];
  float qreg[2][DS];
#pragma unroll
  for (int cb = 0; cb < 2; cb++) {
    const uint32_t r = wave * 32 + cb * 16 + lc;
    const uint32_t qi = q0 + r / a.group;
    const uint32_t h = kvh * a.group + r % a.group;
    col_ok[cb] = r < a.q_per_tile * a.group && qi < a.n_queries;
    qpos[cb] = a.pos0 + qi;
    const float4* src = reinterpret_cast<const float4*>(
        a.q + ((size_t)(col_ok[cb] ? qi : 0) * a.n_heads + h) * D + DS * lg);
#pragma unroll
    for (int s4 = 0; s4 < DS / 4; s4++) {
      const float4 v = col_ok[cb] ? src[s4] : make_float4(0.f, 0.f, 0.f, 0.f);
      qreg[cb][4 * s4 + 0] = v.x;
      qreg[cb][4 * s4 + 1] = v.y;
      qreg[cb][4 * s4 + 2] = v.z;
      qreg[cb][4 * s4 + 3] = v.w;
    }
  }

  floatx4 oacc[CHB][2];
#pragma unroll
  for (int c = 0; c < CHB; c++)
#pragma unroll
    for (int cb = 0; cb < 2; cb++) oacc[c][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};

  for (uint32_t kt = kt0; kt < kt1; kt++) {
    const uint32_t key0 = kt * kBK;
    // ---- stage K and V tiles in LDS ------------------------------------------
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int i = 0; i < (kBK * D / 4) / kPThreads; i++) {
      const int f = tid + kPThreads * i;
      const int r = f / (D / 4), c4 = f % (D / 4);
      const uint32_t key = key0 + r;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (key < n_keys_total) {
        const size_t off = (size_t)key * row + (size_t)kvh * D + 4 * c4;
        kv = *reinterpret_cast<const float4*>(a.kcache + off);
        vv = *reinterpret_cast<const float4*>(a.vcache + off);
      }
      *reinterpret_cast<float4*>(&k_lds[r * LDK + 4 * c4]) = kv;
      *reinterpret_cast<float4*>(&v_lds[r * LDK + 4 * c4]) = vv;
    }
    __syncthreads();

    // ---- S^T = K Q^T ------------------------------------------------------------
    floatx4 sacc[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      float kf[DS];
      const float* kr = &k_lds[(kb * 16 + lc) * LDK + DS * lg];
#pragma unroll
      for (int s4 = 0; s4 < DS / 4; s4++) {
        const float4 v = *reinterpret_cast<const float4*>(kr + 4 * s4);
        kf[4 * s4 + 0] = v.x;
        kf[4 * s4 + 1] = v.y;
        kf[4 * s4 + 2] = v.z;
        kf[4 * s4 + 3] = v.w;
      }
#pragma unroll
      for (int cb = 0; cb < 2; cb++) {
        floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < DS; s++) c = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[s], qreg[cb][s], c, 0, 0, 0);
        sacc[kb][cb] = c;
      }
    }

    // ---- online softmax per column ---------------------------------------------
#pragma unroll
    for (int cb = 0; cb < 2; cb++) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t key = key0 + kb * 16 + 4 * lg + i;
          const bool ok = col_ok[cb] && key <= qpos[cb];
          const float s = ok ? sacc[kb][cb][i] * a.scale : -INFINITY;
          sacc[kb][cb][i] = s;
          mx = fmaxf(mx, s);
        }
      mx = fmaxf(mx, shfl_xor(mx, 16));
      mx = fmaxf(mx, shfl_xor(mx, 32));
      const float mn = fmaxf(m_run[cb], mx);
      float corr = 1.f, rs = 0.f;
      if (mn != -INFINITY) {
        corr = expf(m_run[cb] - mn);
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float p = expf(sacc[kb][cb][i] - mn);
            sacc[kb][cb][i] = p;
            rs += p;
          }
      } else {
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int i = 0; i < 4; i++) sacc[kb][cb][i] = 0.f;
      }
      rs += shfl_xor(rs, 16);
      rs += shfl_xor(rs, 32);
      l_run[cb] = l_run[cb] * corr + rs;
      m_run[cb] = mn;
#pragma unroll
      for (int c = 0; c < CHB; c++) oacc[c][cb] *= corr;
    }

    // ---- O^T += V^T P^T -------------------------------------------------------
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float* vr = &v_lds[(kb * 16 + 4 * lg + i) * LDK + lc];
#pragma unroll
        for (int c = 0; c < CHB; c++) {
          const float av = vr[16 * c];
#pragma unroll
          for (int cb = 0; cb < 2; cb++)
            oacc[c][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, sacc[kb][cb][i], oacc[c][cb], 0, 0, 0);
        }
      }
  }

  // ---- epilogue ------------------------------------------------------------------
  const bool single = ns == 1;
  const size_t slot = ((size_t)qt * a.max_splits + split) * a.n_kv_heads + kvh;
#pragma unroll
  for (int cb = 0; cb < 2; cb++) {
    const uint32_t r = wave * 32 + cb * 16 + lc;
    if (single) {
      if (!col_ok[cb]) continue;
      const uint32_t qi = q0 + r / a.group;
      const uint32_t h = kvh * a.group + r % a.group;
      float* dst = a.o + ((size_t)qi * a.n_heads + h) * D + 4 * lg;
      const float L = l_run[cb];
#pragma unroll
      for (int c = 0; c < CHB; c++) {
        const float4 v = make_float4(oacc[c][cb][0] / L, oacc[c][cb][1] / L, oacc[c][cb][2] / L,
                                     oacc[c][cb][3] / L);
        *reinterpret_cast<float4*>(dst + 16 * c) = v;
      }
    } else {
      float* dst = a.part_acc + (slot * kRows + r) * D + 4 * lg;
#pragma unroll
      for (int c = 0; c < CHB; c++)
        *reinterpret_cast<float4*>(dst + 16 * c) =
            make_float4(oacc[c][cb][0], oacc[c][cb][1], oacc[c][cb][2], oacc[c][cb][3]);
      if (lg == 0) a.part_ml[slot * kRows + r] = make_float2(m_run[cb], l_run[cb]);
    }
  }
}

// One workgroup per (kv head, q tile, 8 rows); 32 lanes per row (D = 128) or
// 16 (D = 64), each owning a float4 of channels. Combines the splits of a
// multi-split tile with log-sum-exp weights; single-split tiles exit.
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  constexpr int LPR = D / 4;
  constexpr int RPB = 256 / LPR;   // rows per block
  const uint32_t kvh = blockIdx.x;
  const uint32_t qt = blockIdx.y;
  const uint32_t n_kt = tile_kt(a, qt);
  const uint32_t ns = tile_splits(a, n_kt);
  if (ns == 1) return;
  const uint32_t r = blockIdx.z * RPB + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  const uint32_t qi = qt * a.q_per_tile + r / a.group;
  if (r >= a.q_per_tile * a.group || qi >= a.n_queries) return;
  const uint32_t h = kvh * a.group + r % a.group;
  float M = -INFINITY;
  for (uint32_t s = 0; s < ns; s++) {
    const size_t slot = ((size_t)qt * a.max_splits + s) * a.n_kv_heads + kvh;
    M = fmaxf(M, a.part_ml[slot * kRows + r].x);
  }
  float L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s = 0; s < ns; s++) {
    const size_t slot = ((size_t)qt * a.max_splits + s) * a.n_kv_heads + kvh;
    const float2 ml = a.part_ml[slot * kRows + r];
    if (ml.x == -INFINITY) continue;
    const float w = expf(ml.x - M);
    const float4 p = reinterpret_cast<const float4*>(a.part_acc + (slot * kRows + r) * D)[c];
    L = fmaf(ml.y, w, L);
    A.x = fmaf(p.x, w, A.x);
    A.y = fmaf(p.y, w, A.y);
    A.z = fmaf(p.z, w, A.z);
    A.w = fmaf(p.w, w, A.w);
  }
  float4* dst = reinterpret_cast<float4*>(a.o + ((size_t)qi * a.n_heads + h) * D);
  dst[c] = make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
}

// ------------------------------------------------------------------ plan ----
PrefillPlan prefill_plan(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t n_queries, uint32_t pos0) {
  (void)head_dim;
  PrefillPlan p{};
  const uint32_t group = n_heads / n_kv_heads;
  p.rows_per_tile = kRows;
  p.q_per_tile = kRows / group;
  p.n_qtiles = (n_queries + p.q_per_tile - 1) / p.q_per_tile;
  auto n_kt = [&](uint32_t qt) {
    const uint32_t q_end = (qt + 1) * p.q_per_tile < n_queries ? (qt + 1) * p.q_per_tile : n_queries;
    return (pos0 + q_end + kBK - 1) / kBK;
  };
  uint64_t total = 0;
  for (uint32_t qt = 0; qt < p.n_qtiles; qt++) total += n_kt(qt);
  total *= n_kv_heads;
  uint64_t ch = (total + kTargetItems - 1) / kTargetItems;
  if (ch < kMinKtPerSplit) ch = kMinKtPerSplit;
  const uint32_t max_kt = n_kt(p.n_qtiles - 1);
  for (;;) {
    const uint64_t ms = (max_kt + ch - 1) / ch;
    const uint64_t slots = (uint64_t)p.n_qtiles * ms * n_kv_heads;
    if (ms <= 1 || slots <= kMaxSlots) {
      p.ktiles_per_split = (uint32_t)ch;
      p.max_splits = (uint32_t)ms;
      p.partial_slots = ms > 1 ? slots : 0;
      break;
    }
    ch++;
  }
  return p;
}

// Upper bound over every plan with n_queries <= max_queries and pos0 +
// n_queries <= max_keys: splits per tile never exceed ceil(kt / kMinKtPerSplit)
// and the planner never exceeds kMaxSlots when it splits at all.
uint64_t prefill_ws_bound(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t max_queries, uint32_t max_keys) {
  const uint32_t q_per_tile = kRows / (n_heads / n_kv_heads);
  const uint64_t n_qt = (max_queries + q_per_tile - 1) / q_per_tile;
  const uint64_t max_kt = (max_keys + kBK - 1) / kBK;
  const uint64_t ms = (max_kt + kMinKtPerSplit - 1) / kMinKtPerSplit;
  uint64_t slots = ms > 1 ? n_qt * ms * n_kv_heads : 0;
  if (slots > kMaxSlots) slots = kMaxSlots;
  PrefillPlan p{};
  p.partial_slots = slots;
  return prefill_ws_bytes(p, head_dim);
}

uint64_t prefill_ws_bytes(const PrefillPlan& p, uint32_t head_dim) {
  if (p.partial_slots == 0) return 0;
  return ws_align(p.partial_slots * kRows * sizeof(float2)) +
         p.partial_slots * kRows * head_dim * sizeof(float);
}

template <int D>
static hipError_t launch_prefill_d(const PrefillArgs& a, const PrefillPlan& p, hipStream_t st) {
  const dim3 grid(a.n_kv_heads, p.max_splits, p.n_qtiles);
  hipLaunchKernelGGL(prefill_kernel<D>, grid, dim3(kPThreads), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.max_splits <= 1) return e;
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
  char* w = static_cast<char*>(ws);
  if (p.partial_slots > 0) {
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
  a.kt_per_split = p.ktiles_per_split;
  a.max_splits = p.max_splits;
  a.scale = (float)(1.0 / sqrt((double)head_dim));
  if (head_dim == 128) return launch_prefill_d<128>(a, p, st);
  return launch_prefill_d<64>(a, p, st);
}

}  // namespace flk
