// FLK1 frame payloads on the device (web/js/wire.mjs): f32 <-> f16 with the
// reference's rounding and special values, written as integer bit operations
// so the result does not depend on the conversion instruction's NaN rules.
#include <string.h>

#include "common.hpp"

namespace flk {

// f32to16 (wire.mjs:33-53).
__device__ __forceinline__ uint16_t wire_f32_to_f16(float v) {
  const uint32_t x = __float_as_uint(v);
  const uint32_t sign = (x >> 16) & 0x8000u;
  int32_t exp = (int32_t)((x >> 23) & 0xffu);
  uint32_t man = x & 0x7fffffu;
  if (exp == 255) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
  exp = exp - 127 + 15;
  if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - exp;
    const uint32_t sub = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
    return (uint16_t)(sign | (sub + ((rem > half || (rem == half && (sub & 1u))) ? 1u : 0u)));
  }
  uint32_t h = ((uint32_t)exp << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;
  return (uint16_t)(sign | h);
}

// f16to32 (wire.mjs:55-61): every finite f16 is exact in f32.
__device__ __forceinline__ float wire_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 31) return m ? __uint_as_float(0x7fc00000u) : __uint_as_float(sign | 0x7f800000u);
  if (e == 0) {  // m * 2^-24, exact
    const float v = (float)m * 5.9604644775390625e-08f;
    return __uint_as_float(__float_as_uint(v) | sign);
  }
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

__global__ __launch_bounds__(256) void wire_pack_kernel(const float* __restrict__ in,
                                                        uint16_t* __restrict__ out, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
    out[i] = wire_f32_to_f16(in[i]);
}

__global__ __launch_bounds__(256) void wire_unpack_kernel(const uint16_t* __restrict__ in,
                                                          float* __restrict__ out, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
    out[i] = wire_f16_to_f32(in[i]);
}

static uint32_t wire_grid(uint64_t n) {
  const uint64_t g = (n + 255) / 256;
  return (uint32_t)(g < 4096 ? (g > 0 ? g : 1) : 4096);
}

hipError_t launch_wire(int dir, const void* in, void* out, uint64_t n, hipStream_t st) {
  if (dir == 0)
    hipLaunchKernelGGL(wire_pack_kernel, dim3(wire_grid(n)), dim3(256), 0, st,
                       static_cast<const float*>(in), static_cast<uint16_t*>(out), n);
  else
    hipLaunchKernelGGL(wire_unpack_kernel, dim3(wire_grid(n)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(in), static_cast<float*>(out), n);
  return hipGetLastError();
}

}  // namespace flk
