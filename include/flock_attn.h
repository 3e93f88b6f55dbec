/*
 * flock_attn.h -- C ABI of libflock_attn.so, the MI355X (gfx950) attention hot
 * path of flock: per-head q/k RMSNorm + RoPE + K/V-cache append, GQA decode
 * attention, causal prefill attention.
 *
 * In the reference every op below is a WGSL compute dispatch whose "ABI" is a
 * binding list plus a uniform struct, encoded by kernels/layer.ts. Each entry
 * point here replaces one such dispatch (cited per function) with the same
 * buffer layouts and the same position semantics:
 *
 *   q, qn, o (decode)     [n_heads][head_dim]                f32
 *   q, qn, o (prefill)    [n_tokens][n_heads][head_dim]      f32
 *   k, v (new rows)       [n_tokens][n_kv_heads][head_dim]   f32
 *   kcache, vcache        [max_keys][n_kv_heads][head_dim]   f32, row = position
 *   GQA map               query head h reads kv head h / (n_heads / n_kv_heads)
 *
 * Conventions (all entry points):
 *   - Pointers named q/k/v/o/kcache/... are DEVICE pointers (flk_alloc, or any
 *     HIP/torch allocation on the current device). Host pointers appear only in
 *     flk_h2d / flk_d2h.
 *   - Every function returns int32 status: FLK_OK (0) or a negative FLK_ERR_*.
 *     Argument checks run on the host BEFORE any launch, so a rejected call
 *     has no side effect (the reference throws from Layer before encoding:
 *     kernels/layer.ts:575, 689-698; lib.ts:504-506). flk_last_error() gives a
 *     message for the calling thread's most recent failure. Nothing throws.
 *   - Launches are asynchronous and ordered on the library's current stream
 *     (flk_set_stream; default: the null stream). flk_sync() waits for it.
 *     The current stream, like the flk_last_error text, belongs to the
 *     calling host thread.
 *   - Split-K kernels need scratch for per-split partial results. The caller
 *     passes it as (ws, ws_bytes), sized with flk_workspace_bytes; it needs no
 *     initialisation and holds nothing between calls. Calls that share one
 *     workspace must be ordered on one stream (concurrent calls race). A call
 *     whose plan has a single split needs none (ws may then be NULL).
 *   - head_dim must be 64 or 128; n_heads must be a multiple of n_kv_heads
 *     with n_heads / n_kv_heads <= 8.
 *   - The attention kernels move 16-byte vectors: q, qn, o, kcache, vcache and
 *     (flk_decode_layer) q_raw, k_raw, v_raw must be 16-byte aligned; a
 *     misaligned pointer is rejected with FLK_ERR_ARG before any launch.
 */
#ifndef FLOCK_ATTN_H
#define FLOCK_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FLK_OK = 0,
  FLK_ERR_ARG = -1,          /* bad shape, null pointer, n < 1, ...           */
  FLK_ERR_CACHE_FULL = -2,   /* pos + n_tokens > max_keys (layer.ts:575, 693) */
  FLK_ERR_UNSUPPORTED = -3,  /* head_dim / GQA group outside supported set    */
  FLK_ERR_WORKSPACE = -4,    /* ws null or smaller than flk_workspace_bytes   */
  FLK_ERR_HIP = -5,          /* HIP runtime error (message in flk_last_error) */
};

/* RoPE pairing (lib.ts:517-531): NEOX pairs (j, j + d/2), NORM pairs (2j, 2j+1). */
enum { FLK_ROPE_NEOX = 0, FLK_ROPE_NORM = 1 };

/* ---------------------------------------------------------------- runtime -- */

/* Message for the calling thread's last non-zero status ("" if none). */
const char* flk_last_error(void);
/* Library version string. */
const char* flk_version(void);
/* Number of visible devices (0 when no GPU); never fails. */
int32_t flk_device_count(int32_t* count);
/* Stream for all later launches from the calling thread (hipStream_t; NULL =
 * default; each host thread starts on NULL). Replaces the caller-supplied
 * GPUCommandEncoder of Layer.encode (layer.ts:586-589). */
int32_t flk_set_stream(void* stream);

/* Device memory (storageBuffer / createBuffer, lib.ts:548-566; readBack,
 * lib.ts:575-593). flk_h2d/flk_d2h are synchronous with respect to the host.
 * flk_free waits for the calling thread's library stream -- for the whole
 * device when that thread has switched away from a non-null stream since its
 * last such wait -- then releases the memory with hipFree: call it outside
 * loops that must not stall. While the library stream is capturing a graph it returns
 * FLK_ERR_ARG and frees nothing (free after flk_capture_end). */
int32_t flk_alloc(void** dptr, uint64_t bytes);
int32_t flk_free(void* dptr);
int32_t flk_h2d(void* dst, const void* host_src, uint64_t bytes, uint64_t dst_off);
int32_t flk_d2h(void* host_dst, const void* src, uint64_t bytes, uint64_t src_off);
int32_t flk_memset(void* dst, int32_t value, uint64_t bytes);
/* Wait for all work on the current stream (the mapAsync fence, layer.ts:801-816). */
int32_t flk_sync(void);

/* Workspace for the split-K kernels: bytes needed by any call with at most
 * these sizes (max_seqs: sequences of flk_attn_decode_ragged, else 1). */
uint64_t flk_workspace_bytes(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                             uint32_t max_keys, uint32_t max_queries, uint32_t max_seqs);
/* Bytes one call needs. kind: FLK_CALL_DECODE (flk_attn_decode /
 * flk_decode_layer; n = n_keys), FLK_CALL_PREFILL (n = n_queries, pos0),
 * FLK_CALL_RAGGED (n = max_n_keys, n_seqs). 0 when the call needs no workspace
 * (a single-split plan) or the shape is invalid. */
enum { FLK_CALL_DECODE = 0, FLK_CALL_PREFILL = 1, FLK_CALL_RAGGED = 2 };
uint64_t flk_call_workspace_bytes(int32_t kind, uint32_t n_heads, uint32_t n_kv_heads,
                                  uint32_t head_dim, uint32_t n, uint32_t pos0, uint32_t n_seqs);

/* -------------------------------------------------------------- unfused ops -- */

/* rmsnorm.wgsl main (rmsnorm.wgsl:41-73; dispatch layer.ts:601-602, 725-726).
 * o[v][i] = x[v][i] / sqrt(mean(x[v]^2) + eps) * g[i] over n_vecs vectors of
 * width n, with the reference's 128-lane strided partial sums and pairwise tree.
 * Bit-exact with rmsnormRef (ops_ref.ts:20-49). Any n >= 1. */
int32_t flk_rmsnorm(const float* x, const float* g, float* o, uint32_t n, uint32_t n_vecs,
                    float eps);

/* rope.wgsl main (rope.wgsl:50-78 with ropeSource, lib.ts:528-531; dispatch
 * layer.ts:607-613). In place on x [n_tokens][n_heads][head_dim]; token t is
 * rotated by position pos0 + t using inv_freq [head_dim/2] (layer.ts:180-186).
 * Bit-exact with ropeRef (ops_ref.ts:65-92) up to libm's cos/sin last bit. */
int32_t flk_rope(float* x, const float* inv_freq, uint32_t n_tokens, uint32_t n_heads,
                 uint32_t head_dim, uint32_t pos0, int32_t pairing);

/* The two copyBufferToBuffer calls of the K/V append (layer.ts:616-622,
 * 737-741): kcache[pos0 .. pos0+n) <- kn, vcache[pos0 .. pos0+n) <- v. */
int32_t flk_kv_append(const float* kn, const float* v, float* kcache, float* vcache,
                      uint32_t n_tokens, uint32_t pos0, uint32_t n_kv_heads,
                      uint32_t head_dim, uint32_t max_keys);

/* ------------------------------------------------------------ fused prologue -- */

/* layer.ts:598-622 (decode) and 722-741 (prefill) in one launch: per-head
 * RMSNorm of q and k with gains gq, gk [head_dim]; RoPE of both at positions
 * pos0 + t; qn_out <- q; kcache/vcache rows pos0 + t <- (k normed+roped, v raw).
 * Bit-identical to flk_rmsnorm + flk_rope + flk_kv_append. */
int32_t flk_qk_prologue(const float* q_raw, const float* k_raw, const float* v_raw,
                        const float* gq, const float* gk, const float* inv_freq, float eps,
                        int32_t pairing, float* qn_out, float* kcache, float* vcache,
                        uint32_t n_tokens, uint32_t pos0, uint32_t n_heads,
                        uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_keys);

/* Extension, no reference counterpart (layer.ts:722-724 projects q, k and v
 * into three buffers): flk_qk_prologue reading raw rows that lie in_stride
 * floats apart from one token to the next -- e.g. q_raw = qkv, k_raw = qkv +
 * n_heads * head_dim, v_raw = k_raw + n_kv_heads * head_dim, in_stride = (n_heads
 * + 2 * n_kv_heads) * head_dim for the output of ONE projection over q|k|v
 * stacked row-wise. in_stride 0 means packed (flk_qk_prologue); otherwise it
 * must be at least n_heads * head_dim. Same results. */
int32_t flk_qk_prologue_strided(const float* q_raw, const float* k_raw, const float* v_raw,
                                uint32_t in_stride, const float* gq, const float* gk,
                                const float* inv_freq, float eps, int32_t pairing,
                                float* qn_out, float* kcache, float* vcache, uint32_t n_tokens,
                                uint32_t pos0, uint32_t n_heads, uint32_t n_kv_heads,
                                uint32_t head_dim, uint32_t max_keys);

/* -------------------------------------------------------------- attention -- */

/* attention.wgsl main (attention.wgsl:58-122; bindings [q, kcache, vcache, o,
 * Dims{n_heads, n_kv_heads, head_dim, n_keys}], dispatch layer.ts:624-630).
 * One query per head attends keys [0, n_keys). No cap on n_keys beyond the
 * cache (the reference's $MAX_KEYS workgroup array, lib.ts:503-508, is gone):
 * split-K flash-decoding -- a split kernel, then a log-sum-exp merge launch
 * ordered after it on the same stream (one launch when the plan has a single
 * split). */
int32_t flk_attn_decode(const float* q, const float* kcache, const float* vcache, float* o,
                        uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                        uint32_t n_keys, void* ws, uint64_t ws_bytes);

/* attention_prefill.wgsl main (attention_prefill.wgsl:75-175; bindings [q,
 * kcache, vcache, o, Dims{n_heads, n_kv_heads, head_dim, n_queries, pos0}],
 * dispatch layer.ts:743-750). Query i (absolute position pos0 + i) attends
 * keys [0, pos0 + i]; the chunk's own rows must already be in the cache.
 * Tiled flash attention on fp32 MFMA, split over keys for long caches. */
int32_t flk_attn_prefill(const float* q, const float* kcache, const float* vcache, float* o,
                         uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         uint32_t n_queries, uint32_t pos0, void* ws, uint64_t ws_bytes);

/* Layer.encode's attention slice (layer.ts:571-630) as ONE launch: prologue for
 * the token at position pos (norm + RoPE of q and k, append k/v at row pos),
 * then decode attention over pos + 1 keys. qn_out receives the attention input
 * (layer.ts buf.qn). Cache rows are bit-identical to flk_qk_prologue's. */
int32_t flk_decode_layer(const float* q_raw, const float* k_raw, const float* v_raw,
                         const float* gq, const float* gk, const float* inv_freq, float eps,
                         int32_t pairing, float* qn_out, float* kcache, float* vcache,
                         float* o, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t max_keys, void* ws, uint64_t ws_bytes);

/* No counterpart in the reference. For callers that cannot allocate (code
 * under graph capture, serving loops, harnesses that forbid hipMalloc):
 * flk_decode_layer with no workspace argument. The split-K partials go to a
 * static scratch array of 8 MiB that the library holds on each device until
 * the process ends; a call needing more (flk_call_workspace_bytes(
 * FLK_CALL_DECODE, ..., pos + 1, ...) > 8 MiB, i.e. more than ~63 heads of
 * width 128) returns FLK_ERR_WORKSPACE before any launch. Nothing in the
 * array must start at zero: each call's split kernel writes every partial
 * its merge reads. All calls on one device share the array, so calls that
 * overlap on one device (several streams or threads) race: order them on
 * one stream. Same results as flk_decode_layer, bit for bit. */
int32_t flk_decode_layer_noalloc(const float* q_raw, const float* k_raw, const float* v_raw,
                                 const float* gq, const float* gk, const float* inv_freq,
                                 float eps, int32_t pairing, float* qn_out, float* kcache,
                                 float* vcache, float* o, uint32_t pos, uint32_t n_heads,
                                 uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_keys);

/* Extension, no reference counterpart (the reference runs one sequence per
 * Layer, layer.ts:203-204): decode for n_seqs independent sequences in one
 * call. q, o: [n_seqs][n_heads][head_dim]. Sequence b's cache rows start at
 * row seq_row_off[b] of kcache/vcache (rows of n_kv_heads*head_dim floats) and
 * it attends n_keys[b] keys (0: its o rows are zeros). seq_row_off and n_keys
 * are DEVICE arrays (8- and 4-byte aligned), so the library cannot check
 * their contents: rows seq_row_off[b] .. seq_row_off[b] + n_keys[b] - 1 must
 * lie inside kcache and vcache. max_n_keys bounds every n_keys[b] (larger
 * values are clamped to it: such a sequence attends its first max_n_keys
 * rows). Up to 2048 sequences run on persistent workgroups that take
 * the batch's (sequence, split) pieces from a counter kept in the workspace
 * (reset by the call itself); results are the same bits on every call. */
int32_t flk_attn_decode_ragged(const float* q, const float* kcache, const float* vcache,
                               const uint64_t* seq_row_off, const uint32_t* n_keys, float* o,
                               uint32_t n_seqs, uint32_t max_n_keys, uint32_t n_heads,
                               uint32_t n_kv_heads, uint32_t head_dim, void* ws,
                               uint64_t ws_bytes);

/* Extension, no reference counterpart: Layer.encode's attention slice
 * (layer.ts:571-630) for n_seqs independent sequences in one call -- the
 * per-token step of flk_decode_layer applied to every sequence of a batch
 * (the reference runs one sequence per Layer, layer.ts:203-204).
 * q_raw, qn_out, o: [n_seqs][n_heads][head_dim]; k_raw, v_raw:
 * [n_seqs][n_kv_heads][head_dim]. n_keys[b] counts sequence b's keys AFTER
 * this step: its new token sits at position pos_b = n_keys[b] - 1, q and k
 * are normed (gains gq, gk) and rotated at pos_b, k (normed, rotated) and v
 * (raw) are written to cache row seq_row_off[b] + pos_b, and the attention
 * covers the rows seq_row_off[b] .. seq_row_off[b] + pos_b. n_keys[b] == 0
 * marks an idle sequence: its qn and o rows are zeros and nothing is written
 * to the caches. n_keys[b] > max_n_keys (the reference's "KV cache full",
 * layer.ts:575, which the library cannot see on the host: the counts live
 * in device memory) is refused on the device: that sequence's qn and o rows
 * are NaN and nothing is written to the caches. Layouts, alignment,
 * workspace (flk_call_workspace_bytes(FLK_CALL_RAGGED, ...)) and the
 * conditions on seq_row_off are those of flk_attn_decode_ragged. Launches:
 * the prologue (one workgroup per sequence; it also resets the batch's item
 * counters), then flk_attn_decode_ragged's attention and merge. qn and the
 * cache rows are bit-identical to flk_decode_layer's for each sequence. */
int32_t flk_decode_layer_ragged(const float* q_raw, const float* k_raw, const float* v_raw,
                                const float* gq, const float* gk, const float* inv_freq,
                                float eps, int32_t pairing, float* qn_out, float* kcache,
                                float* vcache, const uint64_t* seq_row_off,
                                const uint32_t* n_keys, float* o, uint32_t n_seqs,
                                uint32_t max_n_keys, uint32_t n_heads, uint32_t n_kv_heads,
                                uint32_t head_dim, void* ws, uint64_t ws_bytes);

#ifdef __cplusplus
}
#endif

#endif /* FLOCK_ATTN_H */
