/*
 * flock_oracle_q8.c -- CPU restatement of flock's Q8_0 projection references.
 *
 * TEST INFRASTRUCTURE ONLY (the checker; see flock_oracle.c for the rules).
 *
 * Restates, rounding point for rounding point:
 *   flko_f32_to_f16      f32to16 (web/js/wire.mjs:33-53): f32 bits -> f16 bits,
 *                        round to nearest even, subnormals, inf/nan.
 *   flko_half_to_f32     halfToF32 (kernels/lib.ts:28-33): f16 bits -> value,
 *                        exponent 31 (inf or nan) clamped to +-3.4028235e38.
 *   flko_quant_row_q8    quantRowQ8 (kernels/lib.ts:38-53): d = amax / 127 in
 *                        double, stored as f32to16(d); q = Math.round(v / d)
 *                        (ties toward +inf), clamped to [-128, 127].
 *   flko_split_q8        splitQ8 (kernels/lib.ts:141-156): 34-byte blocks ->
 *                        contiguous int8 quants + f16 scales.
 *   flko_q8_matvec       cpuMatmulQ8F32 + matmulF32 (kernels/lib.ts:196-278):
 *                        lanes == 0 is SERIAL (q8_matmul.wgsl: 32 fma32 per
 *                        block, then fma32 with the scale); lanes > 0 is
 *                        coop(lanes) (q8_coop.wgsl): lane b % lanes owns block
 *                        b; per word pair g, d0 = dot4(q[8g..8g+3], x),
 *                        d1 = dot4(q[8g+4..8g+7], x) (dot4: one rounded
 *                        product then three fma32), part[lane] =
 *                        fma32(scale, fr(d0 + d1), part[lane]); then the
 *                        pairwise treeSum (lib.ts:312-318).
 *   flko_argmax_wgsl     argmax.wgsl's two-pass contract (lowest index among
 *                        equal maxima, NaN never chosen, empty sentinel).
 *   flko_swiglu, flko_add  swigluRef / addRef (kernels/ops_ref.ts:103-117).
 *   flko_f16_to_f32_wire f16to32 (web/js/wire.mjs:55-61), the frame decoder.
 *
 * `fused` selects the FMA model: 0 = the reference's fma32 (f64 a*b + c,
 * then rounded to f32: two roundings), 1 = fmaf (one rounding, what the GPU's
 * v_fma_f32 does). With int8 weights both agree except where a*b + c is not
 * exact in f64; tests count such cases rather than assume there are none.
 *
 * Pinning (tests/test_oracle_q8.py): f32_to_f16 against numpy's IEEE
 * float16 cast on every f32 class (normal, subnormal, overflow, ties);
 * half_to_f32 against numpy on all 65536 patterns (exponent 31 clamped);
 * quant_row_q8 against its definition's invariants (|v - q*d| <= d/2 for
 * the double d, JS tie rule on constructed ties, amax -> +-127); matvec
 * against exact integer arithmetic on integer inputs (every order gives the
 * exact sum, so a wrong index or operand fails), against an f64 sum within
 * the f32 error bound, and coop against serial on integer inputs;
 * argmax_wgsl against numpy's argmax / nanargmax (lowest index of the
 * maximum) and hand-derived sentinel cases; swiglu against numpy f64
 * silu(g) * up within 2 ulp and on exact cases (g = 0, up = 0); add against
 * numpy f32 addition.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float fr64(double x) { return (float)x; }

static inline float fma_model(float a, float b, float c, int fused) {
  return fused ? fmaf(a, b, c) : (float)((double)a * (double)b + (double)c);
}

/* web/js/wire.mjs:33-53. v arrives as an f32 (setFloat32 rounds the JS double
 * to f32 first; callers holding a double round it with (float)). */
uint16_t flko_f32_to_f16(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
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

/* kernels/lib.ts:28-33 (value as a double; callers round with fr). */
double flko_half_to_f32(uint16_t h) {
  const double s = (h & 0x8000u) ? -1.0 : 1.0;
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) return s * m * ldexp(1.0, -24);
  if (e == 31) return s * 3.4028235e38;
  return s * (1.0 + m / 1024.0) * ldexp(1.0, e - 15);
}

/* JS Math.round: nearest integer, ties toward +inf. */
static double js_round(double x) {
  const double r = floor(x);
  return (x - r >= 0.5) ? r + 1.0 : r;
}

/* kernels/lib.ts:38-53. vals: n (a multiple of 32) f32; out: n / 32 * 34 bytes. */
void flko_quant_row_q8(const float* vals, int64_t n, uint8_t* out) {
  const int64_t nb = n / 32;
  for (int64_t b = 0; b < nb; b++) {
    double amax = 0.0;
    for (int i = 0; i < 32; i++) amax = fmax(amax, fabs((double)vals[b * 32 + i]));
    const double d = amax / 127.0;
    const uint16_t h = flko_f32_to_f16((float)d);
    out[b * 34] = (uint8_t)(h & 0xff);
    out[b * 34 + 1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) {
      double q = d == 0.0 ? 0.0 : js_round((double)vals[b * 32 + i] / d);
      q = fmax(-128.0, fmin(127.0, q));
      out[b * 34 + 2 + i] = (uint8_t)((int)q & 0xff);
    }
  }
}

/* kernels/lib.ts:141-156. packed: rows * cols / 32 * 34 bytes; qs: rows * cols
 * int8; scales: rows * cols / 32 f16 (little-endian byte pairs). */
void flko_split_q8(const uint8_t* packed, int rows, int cols, uint8_t* qs, uint8_t* scales) {
  const int nb = cols / 32;
  const size_t row_bytes = (size_t)nb * 34;
  for (int r = 0; r < rows; r++)
    for (int b = 0; b < nb; b++) {
      const uint8_t* src = packed + (size_t)r * row_bytes + (size_t)b * 34;
      const size_t si = ((size_t)r * nb + b) * 2;
      scales[si] = src[0];
      scales[si + 1] = src[1];
      memcpy(qs + (size_t)r * cols + (size_t)b * 32, src + 2, 32);
    }
}

/* dot(vec4, vec4) as kernels/lib.ts:190-196 models it. */
static float dot4(const float* a, const float* b, int fused) {
  float s = fr64((double)a[0] * (double)b[0]);
  s = fma_model(a[1], b[1], s, fused);
  s = fma_model(a[2], b[2], s, fused);
  s = fma_model(a[3], b[3], s, fused);
  return s;
}

/* kernels/lib.ts:196-278 on the 34-byte layout. out[r] = sum_c W[r][c] x[c].
 * lanes: 0 = SERIAL, else coop(lanes) with lanes a power of two <= 1024. */
void flko_q8_matvec(const uint8_t* packed, const float* x, int rows, int cols, int lanes,
                    int fused, float* out) {
  const int nb = cols / 32;
  const size_t row_bytes = (size_t)nb * 34;
  float part[1024];
  const int np = lanes > 0 ? lanes : 1;
  for (int r = 0; r < rows; r++) {
    for (int i = 0; i < np; i++) part[i] = 0.f;
    for (int b = 0; b < nb; b++) {
      const uint8_t* blk = packed + (size_t)r * row_bytes + (size_t)b * 34;
      const float scale = fr64(flko_half_to_f32((uint16_t)(blk[0] | (blk[1] << 8))));
      float q[32];
      for (int i = 0; i < 32; i++) q[i] = (float)(int8_t)blk[2 + i];
      const float* xb = x + (size_t)b * 32;
      if (lanes == 0) {
        float s = 0.f;
        for (int i = 0; i < 32; i++) s = fma_model(q[i], xb[i], s, fused);
        part[0] = fma_model(scale, s, part[0], fused);
      } else {
        const int lane = b % lanes;
        for (int g = 0; g < 4; g++) {
          const float d0 = dot4(q + 8 * g, xb + 8 * g, fused);
          const float d1 = dot4(q + 8 * g + 4, xb + 8 * g + 4, fused);
          part[lane] = fma_model(scale, fr64((double)d0 + (double)d1), part[lane], fused);
        }
      }
    }
    if (lanes == 0) {
      out[r] = part[0];
    } else {
      for (int stride = lanes >> 1; stride > 0; stride >>= 1)
        for (int i = 0; i < stride; i++) part[i] = fr64((double)part[i] + (double)part[i + stride]);
      out[r] = part[0];
    }
  }
}

/* argmax.wgsl's contract (kernels/argmax.wgsl:54-56, 92-134): (va, ia) beats
 * (vb, ib) if va > vb or (va == vb and ia < ib); start from
 * (-3.4028235e38, 0xffffffff). The comparison is a total order on non-NaN
 * pairs, so the scan order does not matter; NaN never wins. argmaxRef
 * (head_ref.ts:65-74) agrees on every input without NaN and with some value
 * >= -3.4028235e38. */
void flko_argmax_wgsl(const float* x, int64_t n, float* oval, uint32_t* oidx) {
  float bv = -3.40282347e38f;
  uint32_t bi = 0xffffffffu;
  for (int64_t i = 0; i < n; i++)
    if (x[i] > bv || (x[i] == bv && (uint32_t)i < bi)) {
      bv = x[i];
      bi = (uint32_t)i;
    }
  *oval = bv;
  *oidx = bi;
}

/* swigluRef (kernels/ops_ref.ts:103-110): fr(fr(g / fr(1 + fr(exp(-g)))) * up). */
void flko_swiglu(const float* gate, const float* up, float* o, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    const float g = gate[i];
    const float e = fr64(exp(-(double)g));
    const float den = fr64(1.0 + (double)e);
    o[i] = fr64((double)fr64((double)g / (double)den) * (double)up[i]);
  }
}

/* addRef (kernels/ops_ref.ts:113-117). */
void flko_add(const float* a, const float* b, float* o, int64_t n) {
  for (int64_t i = 0; i < n; i++) o[i] = fr64((double)a[i] + (double)b[i]);
}

/* f16to32 (web/js/wire.mjs:55-61): exponent 31 is inf or NaN (not clamped). */
double flko_f16_to_f32_wire(uint16_t h) {
  const double s = (h & 0x8000u) ? -1.0 : 1.0;
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) return s * m * ldexp(1.0, -24);
  if (e == 31) return m ? NAN : s * INFINITY;
  return s * (1.0 + m / 1024.0) * ldexp(1.0, e - 15);
}
