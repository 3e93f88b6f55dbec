// The model head after the last layer (model.ts:307-346, encodeHead):
// output RMSNorm of the hidden state, the tied Q8_0 vocab projection, and the
// greedy token = argmax of the logits (argmax.wgsl).
//
// argmax: the reference runs two passes (argmax.wgsl:92-134): n_groups
// workgroups reduce strided slices to (value, index) partials, then one
// workgroup reduces the partials. flk_argmax does the same with wave
// shuffles in place of the LDS tree. flk_lm_head folds pass 1 into the
// projection: each matvec workgroup reduces the logits it produced, so the
// head is three launches (norm, projection, final reduce) instead of four and
// the logits need not be written at all.
#include "common.hpp"

namespace flk {

constexpr int kArgmaxThreads = 256;
constexpr uint32_t kArgmaxMaxGroups = 1024;

// Pass 1: workgroup g reduces elements g*256 + t, + n_groups*256, ...
// (argmax.wgsl:92-111: adjacent threads read adjacent elements).
__global__ __launch_bounds__(kArgmaxThreads) void argmax_pass1_kernel(const float* __restrict__ x,
                                                                      uint32_t n,
                                                                      float* __restrict__ pv,
                                                                      uint32_t* __restrict__ pi) {
  float bv = kArgmaxNoVal;
  uint32_t bi = kArgmaxNoIdx;
  const uint32_t stride = gridDim.x * kArgmaxThreads;
  for (uint32_t i = blockIdx.x * kArgmaxThreads + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    if (argmax_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  argmax_block_store(bv, bi, pv, pi);
}

// Pass 2: one workgroup over the partials (argmax.wgsl:117-134); the indices
// carried with them are the original element indices.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(
    const float* __restrict__ pv, const uint32_t* __restrict__ pi, uint32_t n_parts,
    float* __restrict__ oval, uint32_t* __restrict__ oidx) {
  float bv = kArgmaxNoVal;
  uint32_t bi = kArgmaxNoIdx;
  for (uint32_t j = threadIdx.x; j < n_parts; j += kArgmaxThreads)
    if (argmax_better(pv[j], pi[j], bv, bi)) {
      bv = pv[j];
      bi = pi[j];
    }
  argmax_block_store(bv, bi, oval, oidx);  // blockIdx.x == 0
}

// ------------------------------------------------------------- elementwise --
// elementwise.wgsl:24-37, one thread per element. swiglu's exp is the f64 one
// rounded to f32, as swigluRef (ops_ref.ts:103-110) computes it.
__global__ __launch_bounds__(256) void elementwise_kernel(int op, const float* a, const float* b,
                                                          float* o, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float g = a[i];
  if (op == 0) {
    const float e = (float)exp(-(double)g);
    o[i] = (g / (1.f + e)) * b[i];
  } else {
    o[i] = g + b[i];
  }
}

hipError_t launch_elementwise(int op, const float* a, const float* b, float* o, uint32_t n,
                              hipStream_t st) {
  hipLaunchKernelGGL(elementwise_kernel, dim3((n + 255) / 256), dim3(256), 0, st, op, a, b, o, n);
  return hipGetLastError();
}

static uint32_t argmax_groups(uint32_t n) {
  const uint32_t g = (n + kArgmaxThreads - 1) / kArgmaxThreads;
  return g < kArgmaxMaxGroups ? (g > 0 ? g : 1) : kArgmaxMaxGroups;
}

// Partials: [groups] values, then [groups] indices, 256-byte aligned.
uint64_t argmax_ws_bytes(uint32_t n) {
  const uint64_t g = argmax_groups(n);
  return ws_align(g * sizeof(float)) + g * sizeof(uint32_t);
}

hipError_t launch_argmax(const float* x, uint32_t n, float* oval, uint32_t* oidx, void* ws,
                         hipStream_t st) {
  const uint32_t g = argmax_groups(n);
  float* pv = static_cast<float*>(ws);
  uint32_t* pi = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + ws_align(g * sizeof(float)));
  hipLaunchKernelGGL(argmax_pass1_kernel, dim3(g), dim3(kArgmaxThreads), 0, st, x, n, pv, pi);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, st, pv, pi, g, oval,
                     oidx);
  return hipGetLastError();
}

// One partial per projection workgroup; q8_max_workgroups bounds every grid
// launch_q8_matvec picks for this shape.
static uint64_t lm_head_groups(uint32_t vocab, uint32_t hidden) {
  return q8_max_workgroups(vocab, hidden);
}

uint64_t lm_head_ws_bytes(uint32_t vocab, uint32_t hidden) {
  const uint64_t g = lm_head_groups(vocab, hidden);
  return ws_align(g * sizeof(float)) + g * sizeof(uint32_t);
}

hipError_t launch_lm_head(const float* x, const float* gain, float eps, const uint8_t* qs,
                          const uint16_t* scales, uint32_t vocab, uint32_t hidden, float* normed,
                          float* logits, float* oval, uint32_t* oidx, void* ws, hipStream_t st) {
  const uint64_t g_max = lm_head_groups(vocab, hidden);
  float* pv = static_cast<float*>(ws);
  uint32_t* pi = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) +
                                             ws_align(g_max * sizeof(float)));
  hipError_t e = launch_rmsnorm(x, gain, normed, hidden, 1, eps, st);
  if (e != hipSuccess) return e;
  uint32_t groups = 0;
  e = launch_q8_matvec(qs, scales, normed, logits, vocab, hidden, 1, st, pv, pi, &groups);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, st, pv, pi, groups,
                     oval, oidx);
  return hipGetLastError();
}

}  // namespace flk
