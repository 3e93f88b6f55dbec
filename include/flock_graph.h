/*
 * flock_graph.h -- a decode step as a replayable HIP graph.
 *
 * The reference records a step into one WebGPU command buffer so that the
 * queue, not the host, runs the ~170 dispatches of a token (layer.ts:585-590,
 * model.ts:227-262). Here the calls of a step are captured from the library's
 * stream into a HIP graph and replayed; everything that changes from one token
 * to the next is read from device memory: the position (n_keys_dev below), the
 * token id the embedding gathers (the previous argmax), and the token log.
 *
 * No entry point here has a reference counterpart (WebGPU command encoders are
 * the reference's form of it); they are for hosts that drive many tokens.
 */
#ifndef FLOCK_GRAPH_H
#define FLOCK_GRAPH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* flk_decode_layer with the key count in device memory (a 4-byte aligned
 * word): *n_keys_dev = pos + 1, 1 <= *n_keys_dev <= max_keys. The launch shape depends only on max_keys, so
 * the call can be captured once and replayed at every position. ws:
 * flk_workspace_bytes(..., max_keys, 0, 1). The host cannot see the value, so
 * the kernel checks it: 0 or a value above max_keys (a cache that is full,
 * where flk_decode_layer returns FLK_ERR_CACHE_FULL) appends nothing, leaves
 * qn_out as it was and fills o with NaN, which the LM head's argmax never
 * selects (an all-NaN row yields its sentinel index 0xffffffff). */
int32_t flk_decode_layer_dev(const float* q_raw, const float* k_raw, const float* v_raw,
                             const float* gq, const float* gk, const float* inv_freq, float eps,
                             int32_t pairing, float* qn_out, float* kcache, float* vcache,
                             float* o, const uint32_t* n_keys_dev, uint32_t n_heads,
                             uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_keys, void* ws,
                             uint64_t ws_bytes);

/* The embedding gather (embed.wgsl): out[t][c] = scale * q of row ids[t] of a
 * Q8_0 matrix in the split layout (the tied token_embd the LM head reads).
 * ids is a DEVICE array of n_tokens ids; ids >= vocab are rejected on the
 * device by writing zeros. */
int32_t flk_embed(const int8_t* qs, const uint16_t* scales, const uint32_t* ids,
                  uint32_t n_tokens, uint32_t vocab, uint32_t hidden, float* out);

/* One thread of bookkeeping at the end of a captured step. state is two
 * DEVICE words {n_keys, cursor}: n_keys += delta; if value and log are not
 * NULL and cursor < log_len, log[cursor] = *value and cursor += 1. The host
 * sets both words before replaying (the position, and 0 to start a log). */
int32_t flk_advance(uint32_t* state, uint32_t delta, const uint32_t* value, uint32_t* log,
                    uint32_t log_len);

/* A stream of default priority for capture and replay (the null stream
 * cannot be captured); destroy it when done. */
int32_t flk_stream_create(void** stream);
int32_t flk_stream_destroy(void* stream);

/* Capture the library stream's work between begin and end into an executable
 * graph (the stream set with flk_set_stream must not be the null stream).
 * Calls made between the two are recorded, not run. */
int32_t flk_capture_begin(void);
int32_t flk_capture_end(void** graph);
/* Run a captured graph on the library stream; destroy it when done. */
int32_t flk_graph_launch(void* graph);
int32_t flk_graph_destroy(void* graph);

#ifdef __cplusplus
}
#endif

#endif /* FLOCK_GRAPH_H */
