// Q8_0 dequantizing matvec: the projections on either side of attention.
//
// Weights arrive in the reference's split layout (kernels/lib.ts:141-156):
// `qs` holds each row's int8 quants contiguously, `scales` one f16 per 32
// quants. out[t][r] = sum_c W[r][c] * x[t][c] with W[r][c] = scale * q.
//
// Summation order is the reference's cooperative one (q8_coop.wgsl:96-140,
// cpuMatmulQ8F32 with coop(64), kernels/lib.ts:196-278), so results are
// identical to it, not merely close:
//   logical lane l (0..63) of a row owns blocks l, l + 64, ... in order;
//   per block and word pair g: d0 = dot4(q[8g..8g+3], x), d1 = dot4(q[8g+4..
//   8g+7], x) with dot4 = one rounded product then three FMAs, and
//   part = fma(scale, d0 + d1, part);
//   the 64 partials are summed by the pairwise tree (stride 32, 16, ..., 1),
//   done here as an xor butterfly (f32 addition is commutative).
//
// Layout on the GPU: a row needs P = min(64, pow2 >= blocks per row) logical
// lanes (lanes past the row's block count hold 0 and the tree adds them as
// exact zeros), so a wave covers 64 / P rows at once (2 for 1024 columns).
// Lane l's x slice (blocks l, l + 64, ...) is the same for every row: it is
// loaded into registers once per wave and the row loop streams only the
// weights, several row groups in flight. Tokens of a small batch ride on grid
// y (q8_coop.wgsl:28-35) and each re-reads the weights; batches of 8 or more
// tokens take the tile kernels further down, which reuse every weight block
// for 8 tokens.
#include "common.hpp"

namespace flk {

constexpr int kQ8Lanes = 64;      // the reference's LANES (q8_coop.wgsl:58)
constexpr int kQ8Threads = 256;   // 4 waves
// Row groups whose loads are in flight together (fewer when x takes more
// registers). 151936 x 1024 (the LM head): 32.3 us with 4, 30.7 with 2, 30.6
// with 1, 32.5 with 3; a second register set requesting the next groups before
// the current ones are folded, 32.3 (2 + 2) to 34.1 (4 + 4); the weights read
// with the non-temporal hint, 32.2. A greedy token at 513 keys (graph replay):
// 0.999 ms with 4 everywhere, 0.982 with 2, 0.969 with 2 here and 4 where an
// input fusion is compiled in (FLK_Q8_UNROLL_FUSED).
#ifndef FLK_Q8_UNROLL
#define FLK_Q8_UNROLL 2
#endif
#ifndef FLK_Q8_WG_PER_CU
#define FLK_Q8_WG_PER_CU 0  // 0: as many as fit (occupancy query)
#endif
// Batches of at least this many tokens take the weight-reusing tile kernel.
#ifndef FLK_Q8_MM_MIN_TOKENS
#define FLK_Q8_MM_MIN_TOKENS 8
#endif
// Waves per SIMD the tile kernel's registers are limited to (rows of more
// than 1024 columns keep a second set of partials).
#ifndef FLK_Q8_MM_WAVES
#define FLK_Q8_MM_WAVES 2
#endif
#ifndef FLK_Q8_MM_WAVES1
#define FLK_Q8_MM_WAVES1 3  // rows of at most 1024 columns
#endif
// With an input fusion every wave recomputes the fused input's norm, so fewer
// waves (more row groups each) pay it fewer times.
#ifndef FLK_Q8_UNROLL_FUSED
#define FLK_Q8_UNROLL_FUSED 4
#endif
// Request order (0 for the older orders, kept for A/B builds). A greedy token
// at 513 keys, graph replay, ms per 32 tokens: residuals read after each
// row's sum and the norm's loads after the weights 30.98-31.00; residuals
// requested with the weights 30.22-30.26; and the norm's first batch ahead of
// the weights 29.40-29.51; the fused x and gain also requested before the
// norm's reduction (one round trip fewer, 32 more registers) 29.65, not kept.
#ifndef FLK_Q8_RES_EARLY
#define FLK_Q8_RES_EARLY 1
#endif
#ifndef FLK_Q8_NORM_FIRST
#define FLK_Q8_NORM_FIRST 1
#endif
template <int NB, bool FUSE>
constexpr int q8_unroll() {
  return NB == 1 ? (FUSE ? FLK_Q8_UNROLL_FUSED : FLK_Q8_UNROLL) : (NB == 2 ? 2 : 1);
}
#ifndef FLK_Q8_1K
#define FLK_Q8_1K 1  // rows of 1024 columns take q8_matvec1k_kernel (contiguous row reads)
#endif
constexpr int kQ8MaxRegBlocks = 4;  // x blocks per lane kept in registers (8192 columns)
#ifndef FLK_Q8_LDS_TREE_ROWS
#define FLK_Q8_LDS_TREE_ROWS 65536
#endif
constexpr uint32_t kQ8LdsTreeRows = FLK_Q8_LDS_TREE_ROWS;  // rows from which the lane tree uses the LDS unit

struct Q8Args {
  const uint8_t* qs;
  const uint16_t* scales;
  const float* x;
  float* o;                 // may be null when best_val is set (argmax only)
  uint32_t n_rows, n_cols, n_tokens;
  float* best_val;          // per-workgroup argmax partials (null: none)
  uint32_t* best_idx;
  // Input and output fusions (all null: plain W x):
  const float* norm_gain;   // x <- rmsnorm(x) with this gain (rmsnorm.wgsl:41-73), eps below
  float norm_eps;
  const float* up;          // x <- swiglu(x, up) (elementwise.wgsl:24-30; x is the gate)
  const float* res;         // o <- res + W x (elementwise.wgsl:32-37, the residual add)
  // Rows in (gate, up) pairs: 2i = gate row i, 2i + 1 = up row i. Instead of
  // o, act[t][i] = swiglu(gate_i, up_i) (elementwise.wgsl:24-30). Needs two
  // or more rows per wave (at most 1024 columns).
  float* act;
};

// swigluRef (ops_ref.ts:103-110): fr(fr(g / fr(1 + fr(exp(-g)))) * up).
__device__ __forceinline__ float q8_swiglu(float g, float u) {
  const float e = (float)exp(-(double)g);
  return (g / (1.f + e)) * u;
}

// Loads of fused inputs c0 .. c0 + 31 of one token (xt: the token's x,
// tok_off: its offset in x and up): x, and the norm gain or the up values.
__device__ __forceinline__ void q8_fused_load(const Q8Args& a, const float* xt, size_t tok_off,
                                              uint32_t c0, float4 (&xv)[8], float4 (&yv)[8]) {
  const float4* xs = reinterpret_cast<const float4*>(xt + c0);
  const float4* ys = reinterpret_cast<const float4*>(
      a.norm_gain != nullptr ? a.norm_gain + c0 : a.up + tok_off + c0);
#pragma unroll
  for (int i = 0; i < 8; i++) xv[i] = xs[i];
#pragma unroll
  for (int i = 0; i < 8; i++) yv[i] = ys[i];
}

// The fused inputs from those loads (scale: the token's rmsnorm scale).
__device__ __forceinline__ void q8_fused_apply(const Q8Args& a, float scale, const float4 (&xv)[8],
                                               const float4 (&yv)[8], float (&out)[32]) {
  if (a.norm_gain != nullptr) {  // uniform
#pragma unroll
    for (int i = 0; i < 8; i++) {
      out[4 * i + 0] = (xv[i].x * scale) * yv[i].x;
      out[4 * i + 1] = (xv[i].y * scale) * yv[i].y;
      out[4 * i + 2] = (xv[i].z * scale) * yv[i].z;
      out[4 * i + 3] = (xv[i].w * scale) * yv[i].w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      out[4 * i + 0] = q8_swiglu(xv[i].x, yv[i].x);
      out[4 * i + 1] = q8_swiglu(xv[i].y, yv[i].y);
      out[4 * i + 2] = q8_swiglu(xv[i].z, yv[i].z);
      out[4 * i + 3] = q8_swiglu(xv[i].w, yv[i].w);
    }
  }
}

// Both steps (x read straight from memory).
__device__ __forceinline__ void q8_fused_block(const Q8Args& a, const float* xt, size_t tok_off,
                                               uint32_t c0, float scale, float (&out)[32]) {
  float4 xv[8], yv[8];
  q8_fused_load(a, xt, tok_off, c0, xv, yv);
  q8_fused_apply(a, scale, xv, yv, out);
}

// rmsnorm scale of a token's n elements, read through ld(i) from any memory
// (rmsnorm.wgsl:45-66), per wave and without a barrier: lane l holds the
// reference's partials l and l + 64 (stride-128 fma32 sums), their sum is the
// tree's stride-64 step, and the xor butterfly over the wave is its strides
// 32 .. 1; scale = 1 / sqrt(mean + eps) rounded once. (A workgroup barrier
// would also wait for the weight loads already in flight.)
#ifndef FLK_Q8_NORM_BATCH
#define FLK_Q8_NORM_BATCH 16
#endif
constexpr int kQ8NormBatch = FLK_Q8_NORM_BATCH;

// One batch: elements base + 64k, k < kQ8NormBatch (0 past the end).
template <class LOAD>
__device__ __forceinline__ void q8_rms_load(uint32_t base, uint32_t n, LOAD ld,
                                            float (&v)[kQ8NormBatch]) {
#pragma unroll
  for (int k = 0; k < kQ8NormBatch; k++) {
    const uint32_t i = base + 64 * k;
    v[k] = ld(min(i, n - 1));
    v[k] = i < n ? v[k] : 0.f;
  }
}

__device__ __forceinline__ void q8_rms_fold(const float (&v)[kQ8NormBatch], float& p0, float& p1) {
#pragma unroll
  for (int k = 0; k < kQ8NormBatch; k += 2) {
    p0 = fma32(v[k], v[k], p0);
    p1 = fma32(v[k + 1], v[k + 1], p1);
  }
}

// Batches after the first (elements from 64 * kQ8NormBatch on), folded, then
// the tree and the scale.
template <class LOAD>
__device__ __forceinline__ float q8_rms_rest(float p0, float p1, uint32_t n, float eps, LOAD ld) {
  const uint32_t l = threadIdx.x & 63;
  for (uint32_t base = l + 64 * kQ8NormBatch; base < n; base += 64 * kQ8NormBatch) {
    float v[kQ8NormBatch];
    q8_rms_load(base, n, ld, v);
    q8_rms_fold(v, p0, p1);
  }
  const float sum = tree_sum64(p0 + p1);
  const float mean = sum / (float)n;
  return rsqrt_once(mean + eps);
}

template <class LOAD>
__device__ __forceinline__ float q8_rms_scale(uint32_t n, float eps, LOAD ld) {
  // Elements l + 64k: even k feed partial l, odd k partial l + 64. A batch of
  // kQ8NormBatch is loaded before any is used (a load-use loop would
  // serialise the latencies; 16 cover a 1024-wide row in one round trip);
  // past the end they read 0, which adds exactly nothing.
  float v[kQ8NormBatch];
  q8_rms_load(threadIdx.x & 63, n, ld, v);
  float p0 = 0.f, p1 = 0.f;
  q8_rms_fold(v, p0, p1);
  return q8_rms_rest(p0, p1, n, eps, ld);
}

// The scale of token row xt in global memory; 1 when there is no norm.
__device__ __forceinline__ float q8_norm_scale(const Q8Args& a, const float* xt) {
  if (a.norm_gain == nullptr) return 1.f;
  return q8_rms_scale(a.n_cols, a.norm_eps, [xt](uint32_t i) { return xt[i]; });
}

// halfToF32 (kernels/lib.ts:28-33): exact for every finite f16 (subnormals
// included); exponent 31 (inf, nan) becomes +-3.4028235e38, the largest f32.
__device__ __forceinline__ float q8_scale(uint16_t h) {
  if ((h & 0x7c00u) == 0x7c00u) return (h & 0x8000u) ? -3.40282347e38f : 3.40282347e38f;
  return (float)__builtin_bit_cast(_Float16, h);
}

// int8 quant k (0..3) of a little-endian word as f32.
__device__ __forceinline__ float q8_quant(uint32_t w, int k) {
  return (float)((int32_t)(w << (24 - 8 * k)) >> 24);
}

// dot(vec4, vec4) as the reference's GPU evaluates it: the first product
// rounded, the other three fused.
__device__ __forceinline__ float q8_dot4(uint32_t w, const float* x) {
  float s = q8_quant(w, 0) * x[0];
  s = __builtin_fmaf(q8_quant(w, 1), x[1], s);
  s = __builtin_fmaf(q8_quant(w, 2), x[2], s);
  s = __builtin_fmaf(q8_quant(w, 3), x[3], s);
  return s;
}

// One 32-quant block folded into a lane's partial (q8_coop.wgsl:105-112).
__device__ __forceinline__ float q8_block(float part, float scale, uint4 w0, uint4 w1,
                                          const float* x) {
  const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const float d0 = q8_dot4(w[2 * g], x + 8 * g);
    const float d1 = q8_dot4(w[2 * g + 1], x + 8 * g + 4);
    part = __builtin_fmaf(scale, d0 + d1, part);
  }
  return part;
}

// Weights of kQ8Unroll row groups g0, g0 + waves, ... for logical lane ll of
// row slot sub (rows past the end re-read the last row, so every load is
// unconditional).
template <int P, int NB, int UR>
__device__ __forceinline__ void q8_load_rows(const Q8Args& a, uint32_t g0, uint32_t waves, int ll,
                                             int sub, uint32_t nb, uint4 (&w0)[UR][NB],
                                             uint4 (&w1)[UR][NB], uint16_t (&hs)[UR][NB]) {
  constexpr int R = kWave / P;
#pragma unroll
  for (int u = 0; u < UR; u++) {
    const uint32_t row = min((g0 + waves * u) * R + sub, a.n_rows - 1);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const uint32_t b = min((uint32_t)(ll + kQ8Lanes * j), nb - 1);
      const uint4* src = reinterpret_cast<const uint4*>(a.qs + (size_t)row * a.n_cols + 32 * (size_t)b);
      w0[u][j] = src[0];
      w1[u][j] = src[1];
      hs[u][j] = a.scales[(size_t)row * nb + b];
    }
  }
}

// Residuals of the same row groups (o <- res + W x), requested with their
// weights rather than after the row's sum, which would add a memory round
// trip to the end of every group. Rows past the end re-read the last row.
template <int P, int UR>
__device__ __forceinline__ void q8_load_res(const Q8Args& a, uint32_t tok, uint32_t g0,
                                            uint32_t waves, int sub, float (&rv)[UR]) {
  constexpr int R = kWave / P;
  if (a.res == nullptr) return;  // uniform
#pragma unroll
  for (int u = 0; u < UR; u++) {
    const uint32_t row = min((g0 + waves * u) * R + sub, a.n_rows - 1);
    rv[u] = a.res[(size_t)tok * a.n_rows + row];
  }
}

// P logical lanes per row, NB x blocks per lane in registers (NB * 64 >= the
// row's block count). Grid: (workgroups over row groups, tokens).
// FUSE: the input fusions (rmsnorm / swiglu) are compiled in.
// LDS_TREE: the lane tree's exchanges through ds_bpermute (the LDS unit)
// instead of DPP (the VALU): for very tall matrices (the LM head), where the
// VALU is the busier unit and latency is hidden by many row groups.
template <int P, int NB, bool FUSE, bool LDS_TREE = false>
__global__ __launch_bounds__(kQ8Threads) void q8_matvec_kernel(Q8Args a) {
  constexpr int R = kWave / P;  // rows per wave per step
  constexpr int kQ8Unroll = q8_unroll<NB, FUSE>();
  const int lane = threadIdx.x & 63;
  const int ll = lane % P;      // logical lane
  const int sub = lane / P;     // which row of the group
  const uint32_t tok = blockIdx.y;
  const uint32_t nb = a.n_cols / 32;
  const uint32_t waves = gridDim.x * (kQ8Threads / kWave);
  // Read through readfirstlane, the wave index is known to be wave-uniform:
  // the row loop's control and row addresses are then scalar work.
  const uint32_t wave =
      blockIdx.x * (kQ8Threads / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // The first row groups' weights (and residuals) are requested before x is
  // prepared, so the input fusion's latency overlaps their fetch.
  const size_t tok_off = (size_t)tok * a.n_cols;
  const float* xt = a.x + tok_off;
  auto ldx = [xt](uint32_t i) { return xt[i]; };
  // With the norm first, its first batch of x is requested before the
  // weights: loads return in order, so its sum of squares is formed while
  // the weights are still on their way.
  float nv[kQ8NormBatch];
  if (FUSE && FLK_Q8_NORM_FIRST) q8_rms_load(lane, a.n_cols, ldx, nv);
  uint4 w0[kQ8Unroll][NB], w1[kQ8Unroll][NB];
  uint16_t hs[kQ8Unroll][NB];
  float rv[kQ8Unroll] = {};
  q8_load_rows<P, NB, kQ8Unroll>(a, wave, waves, ll, sub, nb, w0, w1, hs);
  if (FLK_Q8_RES_EARLY) q8_load_res<P, kQ8Unroll>(a, tok, wave, waves, sub, rv);

  // x blocks ll, ll + 64, ... of this token (zeros past the row's end),
  // after the optional input fusion.
  float scale = 1.f;
  if (FUSE && FLK_Q8_NORM_FIRST) {
    if (a.norm_gain != nullptr) {  // uniform
      float p0 = 0.f, p1 = 0.f;
      q8_rms_fold(nv, p0, p1);
      scale = q8_rms_rest(p0, p1, a.n_cols, a.norm_eps, ldx);
    }
  } else if (FUSE) {
    scale = q8_norm_scale(a, xt);
  }
  float xr[NB][32];
  bool live[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const uint32_t b = ll + kQ8Lanes * j;
    live[j] = b < nb;
    const uint32_t c0 = 32 * min(b, nb - 1);
    if (!FUSE) {
      const float4* xs = reinterpret_cast<const float4*>(xt + c0);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float4 v = xs[i];
        xr[j][4 * i + 0] = v.x;
        xr[j][4 * i + 1] = v.y;
        xr[j][4 * i + 2] = v.z;
        xr[j][4 * i + 3] = v.w;
      }
    } else {
      // Every load of the block first (float4s), then the arithmetic: a
      // per-element load-then-use sequence serialises 32 memory latencies.
      q8_fused_block(a, xt, tok_off, c0, scale, xr[j]);
    }
  }

  // Running argmax over the rows this lane finishes (argmax.wgsl's sentinel).
  float bv = kArgmaxNoVal;
  uint32_t bi = kArgmaxNoIdx;

  const uint32_t n_groups = (a.n_rows + R - 1) / R;
  for (uint32_t g0 = wave; g0 < n_groups; g0 += waves * kQ8Unroll) {
    // Loads of kQ8Unroll row groups first, then the arithmetic (the first
    // groups were loaded above).
    if (g0 != wave) {
      q8_load_rows<P, NB, kQ8Unroll>(a, g0, waves, ll, sub, nb, w0, w1, hs);
      if (FLK_Q8_RES_EARLY) q8_load_res<P, kQ8Unroll>(a, tok, g0, waves, sub, rv);
    }
#pragma unroll
    for (int u = 0; u < kQ8Unroll; u++) {
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < NB; j++)
        if (live[j]) part = q8_block(part, q8_scale(hs[u][j]), w0[u][j], w1[u][j], xr[j]);
      // The reference's tree over 64 partials; strides >= P add exact zeros.
      if (LDS_TREE) {
#pragma unroll
        for (int m = P / 2; m >= 1; m >>= 1) part = part + shfl_xor(part, m);
      } else {
        part = lane_tree<P>(part);
      }
      const uint32_t row = (g0 + waves * u) * R + sub;
      if (R >= 2 && a.act != nullptr) {  // uniform: (gate, up) row pairs -> SwiGLU
        const float up = shfl_xor(part, R >= 2 ? P : 0);  // the odd row of the pair
        if (ll == 0 && (sub & 1) == 0 && g0 + waves * u < n_groups && row + 1 < a.n_rows)
          a.act[(size_t)tok * (a.n_rows / 2) + row / 2] = q8_swiglu(part, up);
        continue;
      }
      if (ll == 0 && g0 + waves * u < n_groups && row < a.n_rows) {
        const size_t oi = (size_t)tok * a.n_rows + row;
        if (a.res != nullptr) part = (FLK_Q8_RES_EARLY ? rv[u] : a.res[oi]) + part;
        if (a.o != nullptr) a.o[oi] = part;
        if (argmax_better(part, row, bv, bi)) {
          bv = part;
          bi = row;
        }
      }
    }
  }
  if (a.best_val != nullptr) argmax_block_store(bv, bi, a.best_val, a.best_idx);
}

// Rows of exactly 1024 columns (32 blocks; the LM head and most of a layer's
// projections), read contiguously. The kernel above gives lane l block l of a
// row, so each of its two 16-byte loads per block touches every cache line of
// the row at half density (a read probe of that pattern over the LM head's
// bytes: 4.1 TB/s, against 6.0 TB/s when each instruction covers 1 KB
// contiguously). Here a wave takes rows 2g and 2g + 1 whole: lane L loads
// bytes 16 L .. 16 L + 15 of each, i.e. half h = L & 1 of block b = L >> 1.
// The coop(64) order is kept: block b's partial runs through its four word
// pairs in order -- pairs 0, 1 in the even lane, then, handed over by one DPP
// move, pairs 2, 3 in the odd lane -- and the blocks' partials (in the odd
// lanes) meet in the same pairwise tree, logical lane stride m being
// physical lane stride 2m.
__device__ __forceinline__ float q8_even_to_odd(float v) {
  return dpp<0xA0>(v);  // quad_perm [0, 0, 2, 2]: lane 2k + 1 <- lane 2k
}

// The tree over the odd lanes' 32 block partials (logical strides 16 .. 1 =
// physical xor 32 .. 2; strides 32 .. 63 of the reference's 64 lanes add
// exact zeros and are skipped, as in lane_tree).
template <bool LDS_TREE>
__device__ __forceinline__ float q8_tree_odd(float v) {
  if (LDS_TREE) {
#pragma unroll
    for (int m = 32; m >= 2; m >>= 1) v = v + shfl_xor(v, m);
    return v;
  }
  v = sum_xor<32>(v);
  v = sum_xor<16>(v);
  v = v + xor_lane<8>(v);
  v = v + dpp<kDppRor4>(v);  // lanes j and j ^ 8 agree: row_ror:4 serves as xor 4
  v = v + xor_lane<2>(v);
  return v;
}

// One row's half block in this lane: words w (quants 16h .. 16h + 15 of block
// b), x its 16 inputs; returns the block's coop(64) partial in the odd lane.
__device__ __forceinline__ float q8_half_pair(uint4 w, float scale, const float* x) {
  const float c0 = q8_dot4(w.x, x) + q8_dot4(w.y, x + 4);
  const float c1 = q8_dot4(w.z, x + 8) + q8_dot4(w.w, x + 12);
  const float pe = __builtin_fmaf(scale, c1, __builtin_fmaf(scale, c0, 0.f));  // even: pairs 0, 1
  const float pin = q8_even_to_odd(pe);
  return __builtin_fmaf(scale, c1, __builtin_fmaf(scale, c0, pin));  // odd: pairs 2, 3
}

// Row pairs in flight per wave. 151936 x 1024 (the LM head): 30.8 us with 1,
// 32.2 with 2, 34.1 with 4, 40.0 with 8 (the kernel above: 31.2 with 2).
#ifndef FLK_Q8_1K_UNROLL
#define FLK_Q8_1K_UNROLL 1
#endif
#ifndef FLK_Q8_1K_UNROLL_FUSED
#define FLK_Q8_1K_UNROLL_FUSED 2
#endif
template <bool FUSE>
constexpr int q8_unroll_1k() {
  return FUSE ? FLK_Q8_1K_UNROLL_FUSED : FLK_Q8_1K_UNROLL;
}

template <bool FUSE, bool LDS_TREE>
__global__ __launch_bounds__(kQ8Threads) void q8_matvec1k_kernel(Q8Args a) {
  constexpr int UR = q8_unroll_1k<FUSE>();
  constexpr uint32_t kNb = 32;  // blocks per row
  const int lane = threadIdx.x & 63;
  const int b = lane >> 1, h = lane & 1;
  const uint32_t tok = blockIdx.y;
  const uint32_t waves = gridDim.x * (kQ8Threads / kWave);
  const uint32_t wave =
      blockIdx.x * (kQ8Threads / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t tok_off = (size_t)tok * a.n_cols;
  const float* xt = a.x + tok_off;
  auto ldx = [xt](uint32_t i) { return xt[i]; };

  float nv[kQ8NormBatch];
  if (FUSE && FLK_Q8_NORM_FIRST) q8_rms_load(lane, a.n_cols, ldx, nv);
  // Weights, scales and residuals of UR row pairs (rows past the end re-read
  // the last row, so every load is unconditional).
  uint4 wa[UR], wb[UR];
  uint16_t sa[UR], sb[UR];
  float ra[UR] = {}, rb[UR] = {};
  auto load = [&](uint32_t g0) {
#pragma unroll
    for (int u = 0; u < UR; u++) {
      const uint32_t r0 = min(2 * (g0 + waves * u), a.n_rows - 1);
      const uint32_t r1 = min(2 * (g0 + waves * u) + 1, a.n_rows - 1);
      wa[u] = reinterpret_cast<const uint4*>(a.qs + (size_t)r0 * 1024)[lane];
      wb[u] = reinterpret_cast<const uint4*>(a.qs + (size_t)r1 * 1024)[lane];
      sa[u] = a.scales[(size_t)r0 * kNb + b];
      sb[u] = a.scales[(size_t)r1 * kNb + b];
      if (FLK_Q8_RES_EARLY && a.res != nullptr) {  // uniform
        ra[u] = a.res[(size_t)tok * a.n_rows + r0];
        rb[u] = a.res[(size_t)tok * a.n_rows + r1];
      }
    }
  };
  load(wave);

  // This lane's 16 inputs: columns 32 b + 16 h .. + 15, after the fusion.
  float scale = 1.f;
  if (FUSE && FLK_Q8_NORM_FIRST) {
    if (a.norm_gain != nullptr) {  // uniform
      float p0 = 0.f, p1 = 0.f;
      q8_rms_fold(nv, p0, p1);
      scale = q8_rms_rest(p0, p1, a.n_cols, a.norm_eps, ldx);
    }
  } else if (FUSE) {
    scale = q8_norm_scale(a, xt);
  }
  const uint32_t c0 = 32 * b + 16 * h;
  float xr[16];
  {
    float4 xv[4], yv[4];
    const float4* xs = reinterpret_cast<const float4*>(xt + c0);
#pragma unroll
    for (int i = 0; i < 4; i++) xv[i] = xs[i];
    if (FUSE) {
      const float4* ys = reinterpret_cast<const float4*>(
          a.norm_gain != nullptr ? a.norm_gain + c0 : a.up + tok_off + c0);
#pragma unroll
      for (int i = 0; i < 4; i++) yv[i] = ys[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float e[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        float v = e[k];
        if (FUSE) {
          const float y[4] = {yv[i].x, yv[i].y, yv[i].z, yv[i].w};
          v = a.norm_gain != nullptr ? (v * scale) * y[k] : q8_swiglu(v, y[k]);
        }
        xr[4 * i + k] = v;
      }
    }
  }

  float bv = kArgmaxNoVal;
  uint32_t bi = kArgmaxNoIdx;
  const uint32_t n_groups = (a.n_rows + 1) / 2;
  for (uint32_t g0 = wave; g0 < n_groups; g0 += waves * UR) {
    if (g0 != wave) load(g0);
#pragma unroll
    for (int u = 0; u < UR; u++) {
      float pa = q8_half_pair(wa[u], q8_scale(sa[u]), xr);
      float pb = q8_half_pair(wb[u], q8_scale(sb[u]), xr);
      pa = q8_tree_odd<LDS_TREE>(pa);
      pb = q8_tree_odd<LDS_TREE>(pb);
      const uint32_t g = g0 + waves * u;
      const uint32_t r0 = 2 * g;
      if (lane != 1 || g >= n_groups) continue;
      if (a.act != nullptr) {  // (gate, up) row pairs -> SwiGLU
        if (r0 + 1 < a.n_rows) a.act[(size_t)tok * (a.n_rows / 2) + g] = q8_swiglu(pa, pb);
        continue;
      }
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t row = r0 + k;
        if (row >= a.n_rows) break;
        float part = k == 0 ? pa : pb;
        const size_t oi = (size_t)tok * a.n_rows + row;
        if (a.res != nullptr) part = (FLK_Q8_RES_EARLY ? (k == 0 ? ra[u] : rb[u]) : a.res[oi]) + part;
        if (a.o != nullptr) a.o[oi] = part;
        if (argmax_better(part, row, bv, bi)) {
          bv = part;
          bi = row;
        }
      }
    }
  }
  if (a.best_val != nullptr) argmax_block_store(bv, bi, a.best_val, a.best_idx);
}

// Columns past kQ8MaxRegBlocks * 64 blocks: the same arithmetic with x read
// from memory per block (L1/L2-resident), one row per wave.
__global__ __launch_bounds__(kQ8Threads) void q8_matvec_wide_kernel(Q8Args a) {
  const int lane = threadIdx.x & 63;
  const uint32_t tok = blockIdx.y;
  const uint32_t nb = a.n_cols / 32;
  const uint32_t waves = gridDim.x * (kQ8Threads / kWave);
  const uint32_t wave =
      blockIdx.x * (kQ8Threads / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t tok_off = (size_t)tok * a.n_cols;
  const float* xt = a.x + tok_off;
  const float scale = q8_norm_scale(a, xt);
  float bv = kArgmaxNoVal;
  uint32_t bi = kArgmaxNoIdx;
  for (uint32_t row = wave; row < a.n_rows; row += waves) {
    float part = 0.f;
    for (uint32_t b = lane; b < nb; b += kQ8Lanes) {
      const uint4* src = reinterpret_cast<const uint4*>(a.qs + (size_t)row * a.n_cols + 32 * (size_t)b);
      float xb[32];
      if (a.norm_gain == nullptr && a.up == nullptr) {
        const float4* xs = reinterpret_cast<const float4*>(xt + 32 * (size_t)b);
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float4 v = xs[i];
          xb[4 * i + 0] = v.x;
          xb[4 * i + 1] = v.y;
          xb[4 * i + 2] = v.z;
          xb[4 * i + 3] = v.w;
        }
      } else {
        q8_fused_block(a, xt, tok_off, 32 * b, scale, xb);
      }
      part = q8_block(part, q8_scale(a.scales[(size_t)row * nb + b]), src[0], src[1], xb);
    }
    part = lane_tree<64>(part);
    if (lane == 0) {
      const size_t oi = (size_t)tok * a.n_rows + row;
      if (a.res != nullptr) part = a.res[oi] + part;
      if (a.o != nullptr) a.o[oi] = part;
      if (argmax_better(part, row, bv, bi)) {
        bv = part;
        bi = row;
      }
    }
  }
  if (a.best_val != nullptr) argmax_block_store(bv, bi, a.best_val, a.best_idx);
}

// ---------------------------------------------------------------------------
// Many tokens at once (prefill, replay chunks): the same sums, with every
// weight block used for several tokens instead of re-read per token.
//
// A workgroup owns a tile of kMmRows rows x kMmTokens tokens. Each output
// keeps the coop(64) order: 32 physical lanes q hold leaf q (blocks q, q + 64,
// ...) and, when the row has more than 32 blocks, leaf q + 32 (blocks q + 32,
// q + 96, ...) in a second accumulator; their sum is the tree's stride-32
// step, and strides 16 .. 1 run across the 32 lanes. A lane holds
// kMmRowsPerSlot x kMmTokens outputs, so the cross-lane strides use recursive
// halving (each exchange moves half of the lane's values: 31 exchanges for 32
// outputs instead of 5 per output) -- the same pairs are added, only which
// lane keeps which sum differs, and f32 addition is commutative.
//
// x is staged through LDS in chunks of 32 blocks (1024 columns) with any input
// fusion applied there; each lane reads its block of every token (blocks
// padded to 36 floats so the 16 lanes of a read phase hit distinct banks).
// Weights come straight from memory. Rows of one chunk (q/k/v, gate/up at
// hidden 1024) stage their token tile once per workgroup -- rmsnorm scales
// included, computed from the staged rows -- and stream up to kMmRowTiles row
// tiles through it with no barrier in between; longer rows take one tile per
// workgroup and restage per chunk.
constexpr int kMmRowsPerSlot = 4;
constexpr int kMmTokens = 8;  // 4 x 8 = 32 outputs per lane
constexpr int kMmRows = (kQ8Threads / kWave) * 2 * kMmRowsPerSlot;  // 32
constexpr int kMmPad = 36;
constexpr int kMmChunkCols = 1024;
constexpr int kMmTokenStride = 32 * kMmPad;  // floats per staged token
#ifndef FLK_Q8_MM_ROW_TILES
#define FLK_Q8_MM_ROW_TILES 8
#endif
// Row tiles one workgroup streams through its staged tokens (rows of one
// chunk), at most; fewer when the grid would otherwise leave CUs idle.
constexpr uint32_t kMmRowTiles = FLK_Q8_MM_ROW_TILES;
#ifndef FLK_Q8_MM_MIN_WG
#define FLK_Q8_MM_MIN_WG 1024  // 4 per CU
#endif
constexpr uint32_t kMmMinWorkgroups = FLK_Q8_MM_MIN_WG;

// One block of RT rows (weights w0/w1, scales sc) against the staged tokens,
// folded into acc[r][t] (q8_coop.wgsl:105-112 per output). Per word pair g,
// the quants of every row are converted once and used for every token.
template <int RT, int TT>
__device__ __forceinline__ void q8_mm_block(float (&acc)[RT][TT], const uint4 (&w0)[RT],
                                            const uint4 (&w1)[RT], const float (&sc)[RT],
                                            const float* xb) {
#pragma unroll
  for (int g = 0; g < 4; g++) {
    auto quants = [&](int r, float (&qf)[8]) {
      const uint32_t wa = g == 0 ? w0[r].x : g == 1 ? w0[r].z : g == 2 ? w1[r].x : w1[r].z;
      const uint32_t wb = g == 0 ? w0[r].y : g == 1 ? w0[r].w : g == 2 ? w1[r].y : w1[r].w;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        qf[k] = q8_quant(wa, k);
        qf[4 + k] = q8_quant(wb, k);
      }
    };
    auto fold = [&](int r, int t, const float (&qf)[8], float4 xa, float4 xc) {
      float d0 = qf[0] * xa.x;
      d0 = __builtin_fmaf(qf[1], xa.y, d0);
      d0 = __builtin_fmaf(qf[2], xa.z, d0);
      d0 = __builtin_fmaf(qf[3], xa.w, d0);
      float d1 = qf[4] * xc.x;
      d1 = __builtin_fmaf(qf[5], xc.y, d1);
      d1 = __builtin_fmaf(qf[6], xc.z, d1);
      d1 = __builtin_fmaf(qf[7], xc.w, d1);
      acc[r][t] = __builtin_fmaf(sc[r], d0 + d1, acc[r][t]);
    };
    static_assert(TT >= RT, "quants are converted once per row and used for every token");
    float qf[RT][8];
#pragma unroll
    for (int r = 0; r < RT; r++) quants(r, qf[r]);
#pragma unroll
    for (int t = 0; t < TT; t++) {
      const float4 xa = *reinterpret_cast<const float4*>(xb + t * kMmTokenStride + 8 * g);
      const float4 xc = *reinterpret_cast<const float4*>(xb + t * kMmTokenStride + 8 * g + 4);
#pragma unroll
      for (int r = 0; r < RT; r++) fold(r, t, qf[r], xa, xc);
    }
  }
}

// Tile (row tile or row-tile group, token tile) of workgroup `id`. When the
// row tiles split evenly over the 8 XCDs (workgroups go to XCDs round-robin
// by id), XCD x takes a contiguous eighth of the rows and walks it token tile
// by token tile, so its share of the weights stays in its own L2 while x
// streams.
__device__ __forceinline__ void q8_mm_tile(uint32_t id, uint32_t n_rt, uint32_t& rt,
                                           uint32_t& tt) {
  if (n_rt % 8 == 0) {
    const uint32_t per = n_rt / 8, k = id / 8;
    rt = (id % 8) * per + k % per;
    tt = k / per;
  } else {
    rt = id % n_rt;
    tt = id / n_rt;
  }
}

// Input fusions of the tile kernel.
enum Q8MmFuse { kMmPlain = 0, kMmNorm = 1, kMmSwiglu = 2 };

// Lane q's weights of chunk c (block 32c + q; past the row's end the last
// block is re-read and not used) for RT rows.
template <int RT>
struct Q8MmWeights {
  uint4 w0[RT], w1[RT];
  float sc[RT];
};
template <int RT>
__device__ __forceinline__ Q8MmWeights<RT> q8_mm_weights(const Q8Args& a, uint32_t c, int q,
                                                         const uint8_t* const (&wrow)[RT],
                                                         const uint16_t* const (&srow)[RT]) {
  const uint32_t nb = a.n_cols / 32;
  const uint32_t bl = min(32 * c + q, nb - 1);
  Q8MmWeights<RT> w;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    const uint4* src = reinterpret_cast<const uint4*>(wrow[r] + 32 * (size_t)bl);
    w.w0[r] = src[0];
    w.w1[r] = src[1];
    w.sc[r] = q8_scale(srow[r][bl]);
  }
  return w;
}

// Stages x's columns 1024c .. 1024c + 1023 of tokens tok0 .. tok0 + TT - 1
// into xs (with the input fusion) and ends with a barrier; the caller has
// made sure no wave still reads xs. NORM_HERE (rows of one chunk): the
// rmsnorm scales are computed here from the staged raw rows; otherwise
// s_scale already holds them.
template <int FUSE, bool NORM_HERE, int TT>
__device__ __forceinline__ void q8_mm_stage(const Q8Args& a, uint32_t c, uint32_t tok0, float* xs,
                                            float* s_scale) {
  // Thread j stages float4 j (columns 1024c + 4j ..) of every token; every
  // load is issued before any is used. Columns past the row's end are
  // clamped on load and not stored.
  static_assert(kQ8Threads == kMmChunkCols / 4, "one float4 column per thread");
  const uint32_t j = threadIdx.x;
  const uint32_t col = min(kMmChunkCols * c + 4 * j, a.n_cols - 4);
  float* dst = xs + (j / 8) * kMmPad + 4 * (j % 8);
  float4 v[TT], y[TT];
#pragma unroll
  for (int t = 0; t < TT; t++) {
    const size_t off = (size_t)min(tok0 + t, a.n_tokens - 1) * a.n_cols + col;
    v[t] = *reinterpret_cast<const float4*>(a.x + off);
    if (FUSE == kMmSwiglu) y[t] = *reinterpret_cast<const float4*>(a.up + off);
  }
  float4 gn = make_float4(0.f, 0.f, 0.f, 0.f);
  if (FUSE == kMmNorm) gn = *reinterpret_cast<const float4*>(a.norm_gain + col);
  const bool store = kMmChunkCols * c + 4 * j < a.n_cols;
  if (NORM_HERE) {
    // Raw rows first; each wave then takes the scales of TT / 4 tokens.
#pragma unroll
    for (int t = 0; t < TT; t++)
      if (store) *reinterpret_cast<float4*>(dst + t * kMmTokenStride) = v[t];
    __syncthreads();
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < TT / 4; i++) {
      const int t = wave * (TT / 4) + i;
      const float* row = xs + t * kMmTokenStride;
      const float s = q8_rms_scale(a.n_cols, a.norm_eps,
                                   [row](uint32_t e) { return row[(e >> 5) * kMmPad + (e & 31)]; });
      if ((threadIdx.x & 63) == 0) s_scale[t] = s;
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < TT; t++) {
    float4 u = v[t];
    if (FUSE == kMmNorm) {
      const float s = s_scale[t];
      u = make_float4((u.x * s) * gn.x, (u.y * s) * gn.y, (u.z * s) * gn.z, (u.w * s) * gn.w);
    } else if (FUSE == kMmSwiglu) {
      const float4 gy = y[t];
      u = make_float4(q8_swiglu(u.x, gy.x), q8_swiglu(u.y, gy.y), q8_swiglu(u.z, gy.z),
                      q8_swiglu(u.w, gy.w));
    }
    if (store) *reinterpret_cast<float4*>(dst + t * kMmTokenStride) = u;
  }
  __syncthreads();
}

// One recursive-halving step over v[0 .. N): lanes with bit S clear keep
// v[0 .. N/2), the others v[N/2 .. N) moved down; each adds its partner's
// copy. Written with constant indices only (a select between two array
// elements would otherwise become a select of the index and a scan of the
// whole array).
template <int S, int N, int I = 0>
__device__ __forceinline__ void q8_halve_step(float (&v)[32], bool hi) {
  if constexpr (I < N / 2) {
    const float lo = v[I], up = v[I + N / 2];
    if constexpr (S == 16) {
      // v_permlane16_swap(lo, up) trades the odd rows of lo for the even rows
      // of up: a lane with bit 4 clear then holds its own lo and its
      // partner's lo, a lane with it set its partner's up and its own up --
      // exactly the pair the step adds, with no selects.
      const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, lo),
                                                      __builtin_bit_cast(int, up), false, false);
      v[I] = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
    } else {
      v[I] = (hi ? up : lo) + xor_lane<S>(hi ? lo : up);
    }
    q8_halve_step<S, N, I + 1>(v, hi);
  }
}
template <int S, int N>
__device__ __forceinline__ void q8_halve(float (&v)[32], int q) {
  if constexpr (S >= 1) {
    q8_halve_step<S, N>(v, (q & S) != 0);
    q8_halve<S / 2, N / 2>(v, q);
  }
}

// TWO: the rows have more than 32 blocks (leaf q + 32 exists).
// Outputs o = t * RT + r of acc: the tree's strides 16 .. 1 by recursive
// halving (at stride s the lane whose bit s is clear keeps the lower half of
// its list, its partner the upper half, and each adds what the other sends;
// lane q ends with output q), then the epilogue: SwiGLU of (gate, up) row
// pairs into act, or res + sum into o.
template <int RT, int TT>
__device__ __forceinline__ void q8_mm_finish(const Q8Args& a, const float (&acc)[RT][TT], int q,
                                             uint32_t row0, uint32_t tok0) {
  constexpr int NO = RT * TT;
  static_assert(NO == 32, "one output per lane after halving");
  float v[NO];
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) v[t * RT + r] = acc[r][t];
  q8_halve<16, NO>(v, q);
  const uint32_t tok = tok0 + q / RT, row = row0 + q % RT;
  float out = v[0];
  if (a.act != nullptr) {  // (gate, up) row pairs: lanes q, q ^ 1 (row0 is a multiple of 4)
    const float up = xor_lane<1>(out);
    if ((q & 1) == 0 && tok < a.n_tokens && row + 1 < a.n_rows)
      a.act[(size_t)tok * (a.n_rows / 2) + row / 2] = q8_swiglu(out, up);
  } else if (tok < a.n_tokens && row < a.n_rows) {
    const size_t oi = (size_t)tok * a.n_rows + row;
    if (a.res != nullptr) out = a.res[oi] + out;
    a.o[oi] = out;
  }
}

// Row pointers of lane slot (wave, lane >> 5) in row tile rt (rows past the
// end re-read the last row and are not stored).
template <int RT>
__device__ __forceinline__ uint32_t q8_mm_rows(const Q8Args& a, uint32_t rt,
                                               const uint8_t* (&wrow)[RT],
                                               const uint16_t* (&srow)[RT]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t row0 = rt * kMmRows + (uint32_t)(wave * 2 + (lane >> 5)) * RT;
  const uint32_t nb = a.n_cols / 32;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    const uint32_t row = min(row0 + r, a.n_rows - 1);
    wrow[r] = a.qs + (size_t)row * a.n_cols;
    srow[r] = a.scales + (size_t)row * nb;
  }
  return row0;
}

// Rows of one chunk (at most 1024 columns): a workgroup stages its token
// tile once and streams kMmRowTiles row tiles through it, with no barrier
// between them.
template <int FUSE>
__global__ __launch_bounds__(kQ8Threads, FLK_Q8_MM_WAVES1) void q8_mm1_kernel(Q8Args a,
                                                                              uint32_t n_rg,
                                                                              uint32_t rpw) {
  constexpr int RT = kMmRowsPerSlot, TT = kMmTokens;
  __shared__ __align__(16) float xs[TT * kMmTokenStride];
  __shared__ float s_scale[TT];
  uint32_t rg, tt;
  q8_mm_tile(blockIdx.x, n_rg, rg, tt);
  const int q = threadIdx.x & 31;
  const uint32_t tok0 = tt * TT;
  const uint32_t n_rt = (a.n_rows + kMmRows - 1) / kMmRows;
  const uint32_t rt_end = min(n_rt, (rg + 1) * rpw);
  q8_mm_stage<FUSE, FUSE == kMmNorm, TT>(a, 0, tok0, xs, s_scale);
  const bool live = (uint32_t)q < a.n_cols / 32;
  for (uint32_t rt = rg * rpw; rt < rt_end; rt++) {
    const uint8_t* wrow[RT];
    const uint16_t* srow[RT];
    const uint32_t row0 = q8_mm_rows<RT>(a, rt, wrow, srow);
    const Q8MmWeights<RT> w = q8_mm_weights<RT>(a, 0, q, wrow, srow);
    float acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int t = 0; t < TT; t++) acc[r][t] = 0.f;
    if (live) q8_mm_block<RT, TT>(acc, w.w0, w.w1, w.sc, xs + q * kMmPad);
    q8_mm_finish<RT, TT>(a, acc, q, row0, tok0);
  }
}

// Rows of more than one chunk: a workgroup owns one tile; leaf q's blocks
// sit in the even chunks, leaf q + 32's in the odd ones (a second set of
// partials, added at the end: the tree's stride 32).
template <int FUSE>
__global__ __launch_bounds__(kQ8Threads, FLK_Q8_MM_WAVES) void q8_mm_kernel(Q8Args a,
                                                                            uint32_t n_rt) {
  constexpr int RT = kMmRowsPerSlot, TT = kMmTokens;
  __shared__ __align__(16) float xs[TT * kMmTokenStride];
  __shared__ float s_scale[TT];
  uint32_t rt, tt;
  q8_mm_tile(blockIdx.x, n_rt, rt, tt);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 31;
  const uint32_t tok0 = tt * TT;
  const uint32_t nb = a.n_cols / 32;
  const uint32_t n_chunks = (a.n_cols + kMmChunkCols - 1) / kMmChunkCols;
  if (FUSE == kMmNorm) {  // per-token rmsnorm scales, TT / 4 tokens per wave
#pragma unroll
    for (int i = 0; i < TT / 4; i++) {
      const int t = wave * (TT / 4) + i;
      const uint32_t tok = min(tok0 + t, a.n_tokens - 1);
      const float s = q8_norm_scale(a, a.x + (size_t)tok * a.n_cols);
      if (lane == 0) s_scale[t] = s;
    }
  }
  const uint8_t* wrow[RT];
  const uint16_t* srow[RT];
  const uint32_t row0 = q8_mm_rows<RT>(a, rt, wrow, srow);

  float acc[RT][TT], accb[RT][TT];
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = accb[r][t] = 0.f;
  for (uint32_t c = 0; c < n_chunks; c += 2) {
    const Q8MmWeights<RT> w = q8_mm_weights<RT>(a, c, q, wrow, srow);
    __syncthreads();  // the previous chunk's reads are done (and s_scale is visible)
    q8_mm_stage<FUSE, false, TT>(a, c, tok0, xs, s_scale);
    if (32 * c + q < nb) q8_mm_block<RT, TT>(acc, w.w0, w.w1, w.sc, xs + q * kMmPad);
  }
  for (uint32_t c = 1; c < n_chunks; c += 2) {
    const Q8MmWeights<RT> w = q8_mm_weights<RT>(a, c, q, wrow, srow);
    __syncthreads();
    q8_mm_stage<FUSE, false, TT>(a, c, tok0, xs, s_scale);
    if (32 * c + q < nb) q8_mm_block<RT, TT>(accb, w.w0, w.w1, w.sc, xs + q * kMmPad);
  }
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = acc[r][t] + accb[r][t];
  q8_mm_finish<RT, TT>(a, acc, q, row0, tok0);
}

// Workgroups: one resident wave of them (every CU filled to its occupancy
// limit, so no workgroup waits for another to finish), never more than there
// are row groups.
template <int P, int NB, bool FUSE, bool LDS_TREE = false, bool K1 = false>
static uint32_t q8_grid_x(uint32_t n_groups) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    hipError_t e = hipSuccess;
    if (FLK_Q8_WG_PER_CU == 0) {
      if (K1)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, q8_matvec1k_kernel<FUSE, LDS_TREE>,
                                                         kQ8Threads, 0);
      else
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, q8_matvec_kernel<P, NB, FUSE, LDS_TREE>, kQ8Threads, 0);
    }
    if (FLK_Q8_WG_PER_CU > 0 || e != hipSuccess || n < 1)
      n = FLK_Q8_WG_PER_CU > 0 ? FLK_Q8_WG_PER_CU : 2;
    per_cu = n;
  }
  static int cus_of[64] = {0};
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    if (cus_of[dev] == 0 &&
        hipDeviceGetAttribute(&cus_of[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus_of[dev] = 256;
    cus = cus_of[dev];
  }
  const uint32_t per_wg =
      (kQ8Threads / kWave) * (K1 ? q8_unroll_1k<FUSE>() : q8_unroll<NB, FUSE>());
  const uint32_t need = (n_groups + per_wg - 1) / per_wg;
  const uint32_t cap = (uint32_t)(per_cu * cus);
  return need < cap ? (need > 0 ? need : 1) : cap;
}

template <int P, int NB>
static uint32_t launch_q8(const Q8Args& a, hipStream_t st) {
  const uint32_t groups = (a.n_rows + (kWave / P) - 1) / (kWave / P);
  if (a.norm_gain != nullptr || a.up != nullptr) {
    const uint32_t gx = q8_grid_x<P, NB, true>(groups);
    hipLaunchKernelGGL((q8_matvec_kernel<P, NB, true>), dim3(gx, a.n_tokens), dim3(kQ8Threads), 0,
                       st, a);
    return gx;
  }
  if (a.n_rows >= kQ8LdsTreeRows) {
    const uint32_t gx = q8_grid_x<P, NB, false, true>(groups);
    hipLaunchKernelGGL((q8_matvec_kernel<P, NB, false, true>), dim3(gx, a.n_tokens),
                       dim3(kQ8Threads), 0, st, a);
    return gx;
  }
  const uint32_t gx = q8_grid_x<P, NB, false>(groups);
  hipLaunchKernelGGL((q8_matvec_kernel<P, NB, false>), dim3(gx, a.n_tokens), dim3(kQ8Threads), 0,
                     st, a);
  return gx;
}

// Rows of 1024 columns: q8_matvec1k_kernel (same grid rule, two rows per wave).
static uint32_t launch_q8_1k(const Q8Args& a, hipStream_t st) {
  const uint32_t groups = (a.n_rows + 1) / 2;
  auto go = [&](auto kernel, uint32_t gx) {
    hipLaunchKernelGGL(kernel, dim3(gx, a.n_tokens), dim3(kQ8Threads), 0, st, a);
    return gx;
  };
  if (a.norm_gain != nullptr || a.up != nullptr)
    return go(q8_matvec1k_kernel<true, false>, q8_grid_x<32, 1, true, false, true>(groups));
  if (a.n_rows >= kQ8LdsTreeRows)
    return go(q8_matvec1k_kernel<false, true>, q8_grid_x<32, 1, false, true, true>(groups));
  return go(q8_matvec1k_kernel<false, false>, q8_grid_x<32, 1, false, false, true>(groups));
}

// Row groups of the register-x kernel and the workgroups it launches at most
// (the argmax partials of flk_lm_head need one slot per workgroup).
uint32_t q8_max_workgroups(uint32_t n_rows, uint32_t n_cols) {
  const uint32_t nb = n_cols / 32;
  uint32_t P = 1;
  while (P < nb && P < 64) P <<= 1;
  const uint32_t groups = (n_rows + (kWave / P) - 1) / (kWave / P);
  uint32_t ub = nb > 128 ? 1 : (nb > 64 ? 2 : FLK_Q8_UNROLL);
  if (nb == 32 && FLK_Q8_1K && FLK_Q8_1K_UNROLL < (int)ub) ub = FLK_Q8_1K_UNROLL;
  const uint32_t per_wg = (kQ8Threads / kWave) * ub;
  return (groups + per_wg - 1) / per_wg;
}

hipError_t launch_q8_matvec(const uint8_t* qs, const uint16_t* scales, const float* x, float* o,
                            uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens,
                            hipStream_t st, float* best_val, uint32_t* best_idx,
                            uint32_t* n_workgroups, const Q8Fuse* fuse) {
  Q8Args a{qs, scales, x, o, n_rows, n_cols, n_tokens, best_val, best_idx,
           nullptr, 0.f, nullptr, nullptr, nullptr};
  if (fuse != nullptr) {
    a.norm_gain = fuse->norm_gain;
    a.norm_eps = fuse->norm_eps;
    a.up = fuse->up;
    a.res = fuse->res;
    a.act = fuse->act;
  }
  const uint32_t nb = n_cols / 32;
  uint32_t gx;
  const uint32_t n_rt = (n_rows + kMmRows - 1) / kMmRows;
  const uint32_t n_tt = (n_tokens + kMmTokens - 1) / kMmTokens;
  const bool one = n_cols <= (uint32_t)kMmChunkCols;
  // Row tiles per workgroup (rows of one chunk): as many as keep the grid at
  // kMmMinWorkgroups or more, up to kMmRowTiles.
  uint32_t rpw = 1;
  while (one && rpw < kMmRowTiles && (uint64_t)((n_rt + 2 * rpw - 1) / (2 * rpw)) * n_tt >=
                                          kMmMinWorkgroups)
    rpw *= 2;
  const uint32_t n_rg = (n_rt + rpw - 1) / rpw;
  if (n_tokens >= FLK_Q8_MM_MIN_TOKENS && best_val == nullptr &&
      (uint64_t)n_rg * n_tt <= 0x7fffffffu) {
    gx = n_rg * n_tt;
    const int fuse = a.norm_gain != nullptr ? kMmNorm : (a.up != nullptr ? kMmSwiglu : kMmPlain);
    auto go1 = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(gx), dim3(kQ8Threads), 0, st, a, n_rg, rpw);
    };
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(gx), dim3(kQ8Threads), 0, st, a, n_rg);
    };
    if (fuse == kMmNorm)
      one ? go1(q8_mm1_kernel<kMmNorm>) : go(q8_mm_kernel<kMmNorm>);
    else if (fuse == kMmSwiglu)
      one ? go1(q8_mm1_kernel<kMmSwiglu>) : go(q8_mm_kernel<kMmSwiglu>);
    else
      one ? go1(q8_mm1_kernel<kMmPlain>) : go(q8_mm_kernel<kMmPlain>);
  } else if (nb > (uint32_t)kQ8Lanes * kQ8MaxRegBlocks) {
    gx = (n_rows + 3) / 4 < 2048u ? (n_rows + 3) / 4 : 2048u;
    hipLaunchKernelGGL(q8_matvec_wide_kernel, dim3(gx, n_tokens), dim3(kQ8Threads), 0, st, a);
  } else if (nb > 192) {
    gx = launch_q8<64, 4>(a, st);
  } else if (nb > 128) {
    gx = launch_q8<64, 3>(a, st);
  } else if (nb > 64) {
    gx = launch_q8<64, 2>(a, st);
  } else if (nb > 32) {
    gx = launch_q8<64, 1>(a, st);
  } else if (nb == 32 && FLK_Q8_1K) {
    gx = launch_q8_1k(a, st);
  } else if (nb > 16) {
    gx = launch_q8<32, 1>(a, st);
  } else if (nb > 8) {
    gx = launch_q8<16, 1>(a, st);
  } else if (nb > 4) {
    gx = launch_q8<8, 1>(a, st);
  } else if (nb > 2) {
    gx = launch_q8<4, 1>(a, st);
  } else if (nb > 1) {
    gx = launch_q8<2, 1>(a, st);
  } else {
    gx = launch_q8<1, 1>(a, st);
  }
  if (n_workgroups != nullptr) *n_workgroups = gx;
  return hipGetLastError();
}

}  // namespace flk
