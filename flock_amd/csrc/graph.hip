// Device-side bookkeeping of a replayable decode step: the embedding gather
// (embed.wgsl) and the position / token-log advance.
#include "common.hpp"

namespace flk {

// embed.wgsl:52-75: one workgroup per token, threads over 4-element groups;
// each element is q * scale (one rounding). An id past the vocabulary writes
// zeros instead of reading outside the matrix.
__global__ __launch_bounds__(256) void embed_kernel(const int8_t* __restrict__ qs,
                                                    const uint16_t* __restrict__ scales,
                                                    const uint32_t* __restrict__ ids,
                                                    uint32_t vocab, uint32_t hidden,
                                                    float* __restrict__ out) {
  const uint32_t tok = blockIdx.x;
  const uint32_t row = ids[tok];
  const bool ok = row < vocab;
  const uint32_t r = ok ? row : 0;
  const uint32_t nb = hidden / 32;
  float* o = out + (size_t)tok * hidden;
  for (uint32_t g = threadIdx.x; g < hidden / 4; g += 256) {
    const uint16_t h = scales[(size_t)r * nb + g / 8];
    float s;
    if ((h & 0x7c00u) == 0x7c00u)
      s = (h & 0x8000u) ? -3.40282347e38f : 3.40282347e38f;
    else
      s = (float)__builtin_bit_cast(_Float16, h);
    const uint32_t w = *reinterpret_cast<const uint32_t*>(qs + (size_t)r * hidden + 4 * g);
    float4 v;
    v.x = (float)((int32_t)(w << 24) >> 24) * s;
    v.y = (float)((int32_t)(w << 16) >> 24) * s;
    v.z = (float)((int32_t)(w << 8) >> 24) * s;
    v.w = (float)((int32_t)w >> 24) * s;
    if (!ok) v = make_float4(0.f, 0.f, 0.f, 0.f);
    reinterpret_cast<float4*>(o)[g] = v;
  }
}

hipError_t launch_embed(const int8_t* qs, const uint16_t* scales, const uint32_t* ids,
                        uint32_t n_tokens, uint32_t vocab, uint32_t hidden, float* out,
                        hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(n_tokens), dim3(256), 0, st, qs, scales, ids, vocab,
                     hidden, out);
  return hipGetLastError();
}

// state = {n_keys, cursor}: the position word every captured decode call
// reads, and where the next logged token goes.
__global__ void advance_kernel(uint32_t* state, uint32_t delta, const uint32_t* value,
                               uint32_t* log, uint32_t log_len) {
  state[0] += delta;
  const uint32_t c = state[1];
  if (log != nullptr && value != nullptr && c < log_len) {
    log[c] = *value;
    state[1] = c + 1;
  }
}

hipError_t launch_advance(uint32_t* state, uint32_t delta, const uint32_t* value, uint32_t* log,
                          uint32_t log_len, hipStream_t st) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, st, state, delta, value, log, log_len);
  return hipGetLastError();
}

}  // namespace flk
