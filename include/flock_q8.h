/*
 * flock_q8.h -- C ABI of the Q8_0 projections in libflock_attn.so.
 *
 * The projections immediately before and after the attention path: q/k/v from
 * the hidden state and o back to it (kernels/layer.ts:495-510, Layer.matvec,
 * dispatching kernels/q8_coop.wgsl). Same conventions as flock_attn.h: device
 * pointers for tensors, FLK_OK or a negative FLK_ERR_* code with
 * flk_last_error(), work queued on the stream set by flk_set_stream().
 *
 * Weights use the reference's upload layout (kernels/lib.ts:141-156, splitQ8):
 *   qs     [n_rows][n_cols] int8 quants, row-major;
 *   scales [n_rows][n_cols / 32] f16 bit patterns, one per 32-quant block.
 * flk_q8_split builds both from GGUF's 34-byte Q8_0 blocks on the host.
 */
#ifndef FLOCK_Q8_H
#define FLOCK_Q8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* o[t][r] = sum_c scale(r, c / 32) * qs[r][c] * x[t][c] for t < n_tokens.
 * Replaces Layer.matvec (kernels/layer.ts:495-510) / q8_coop.wgsl:74-140 with
 * Dims {n_rows, n_cols, n_tokens}: x is [n_tokens][n_cols], o is
 * [n_tokens][n_rows]. n_cols must be a multiple of 32; n_tokens <= 65535.
 * qs and x must be 16-byte aligned. Results are bit-identical to
 * cpuMatmulQ8F32(..., coop(64)) (kernels/lib.ts:251-278) with each
 * multiply-add as one rounding; scales with exponent 31 read as +-FLT_MAX
 * (halfToF32, kernels/lib.ts:28-33). */
int32_t flk_q8_matvec(const int8_t* qs, const uint16_t* scales, const float* x, float* o,
                      uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens);

/* flk_q8_matvec with the layer's neighbouring elementwise ops folded in
 * (Layer.encode, layer.ts:590-649, does them as separate dispatches):
 *   norm_gain != NULL: x is first RMS-normalised per token over n_cols with
 *     that gain and eps (rmsnorm.wgsl, one vector per token) -- the
 *     attn_norm / ffn_norm before the q/k/v and gate/up projections;
 *   up != NULL: x is first replaced by swiglu(x, up) elementwise
 *     (elementwise.wgsl swiglu; up is [n_tokens][n_cols]) -- before ffn_down;
 *   res != NULL: o = res + W x (elementwise.wgsl add; res is
 *     [n_tokens][n_rows], may equal o) -- the residual adds.
 * norm_gain and up are exclusive and, like x, 16-byte aligned. Results are
 * bit-identical to the separate ops (rmsnormRef / swigluRef / addRef, then
 * cpuMatmulQ8F32 coop(64)) except that swiglu's exp is evaluated in f64 and
 * rounded once, as the CPU reference does (the WGSL kernel uses f32 exp).
 * Batches of 8 or more tokens reuse each weight block across tokens; the
 * results are the same. */
int32_t flk_q8_matvec_ex(const int8_t* qs, const uint16_t* scales, const float* x, float* o,
                         uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens,
                         const float* norm_gain, float norm_eps, const float* up,
                         const float* res);

/* The FFN's gate and up projections and SwiGLU in one call (layer.ts:644-646:
 * two matvecs and an elementwise dispatch): the weights are 2 * n_ffn rows
 * with gate and up INTERLEAVED (row 2i = ffn_gate row i, row 2i + 1 = ffn_up
 * row i; interleave at upload), and act[t][i] = swiglu(gate_i, up_i) as
 * flk_swiglu computes it. norm_gain (optional, 16-byte aligned) RMS-normalises
 * x first, as in flk_q8_matvec_ex. n_cols <= 1024 (two or more rows per wave). */
int32_t flk_q8_gate_up_swiglu(const int8_t* qs, const uint16_t* scales, const float* x,
                              float* act, uint32_t n_ffn, uint32_t n_cols, uint32_t n_tokens,
                              const float* norm_gain, float norm_eps);

/* elementwise.wgsl (kernels/elementwise.wgsl:24-37) on n floats:
 * swiglu o = silu(gate) * up = fr(fr(g / fr(1 + fr(exp(-g)))) * up) (exp in
 * f64, rounded once, as swigluRef); add o = a + b. o may alias an input. */
int32_t flk_swiglu(const float* gate, const float* up, float* o, uint32_t n);
int32_t flk_add(const float* a, const float* b, float* o, uint32_t n);

/* splitQ8 (kernels/lib.ts:141-156) on the host: packed is n_rows * n_cols / 32
 * blocks of 34 bytes (f16 scale, little-endian, then 32 int8); writes qs
 * [n_rows * n_cols] and scales [n_rows * n_cols / 32]. HOST pointers. */
int32_t flk_q8_split(const uint8_t* packed, uint32_t n_rows, uint32_t n_cols, int8_t* qs,
                     uint16_t* scales);

/* ---- the head after the last layer (model.ts:307-346, encodeHead) ---- */

/* Greedy token: replaces argmax.wgsl pass1 + pass2 (model.ts:337-346).
 * *oval, *oidx (device) receive the largest x[i] and the lowest index holding
 * it; NaN is never chosen; if nothing beats -3.4028235e38 the result is
 * (-3.4028235e38, 0xffffffff), exactly as argmax.wgsl. ws: device workspace
 * of flk_argmax_ws_bytes(n) bytes, 256-byte aligned (argmax.wgsl's
 * amVal/amIdx partial buffers). */
uint64_t flk_argmax_ws_bytes(uint32_t n);
int32_t flk_argmax(const float* x, uint32_t n, float* oval, uint32_t* oidx, void* ws,
                   uint64_t ws_bytes);

/* encodeHead (model.ts:307-346) in one call: normed = rmsnorm(x[hidden],
 * norm_gain, eps) (rmsnorm.wgsl, one vector), logits = W normed with W the
 * vocab x hidden Q8_0 matrix (the tied token_embd), then the argmax of the
 * logits into *oval, *oidx as flk_argmax. logits may be NULL (greedy decode
 * needs only the token); when given it receives what flk_q8_matvec would
 * write. ws: flk_lm_head_ws_bytes(vocab, hidden) bytes, 256-byte aligned. */
uint64_t flk_lm_head_ws_bytes(uint32_t vocab, uint32_t hidden);
int32_t flk_lm_head(const float* x, const float* norm_gain, float eps, const int8_t* qs,
                    const uint16_t* scales, uint32_t vocab, uint32_t hidden, float* normed,
                    float* logits, float* oval, uint32_t* oidx, void* ws, uint64_t ws_bytes);

#ifdef __cplusplus
}
#endif

#endif /* FLOCK_Q8_H */
