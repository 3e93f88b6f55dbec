// Deno binding of libflock_attn.so: the TypeScript counterpart of
// flock_amd/_lib.py. Every entry point declared in include/flock_attn.h,
// flock_q8.h, flock_graph.h and flock_wire.h is bound here, with the argument
// kinds of its C prototype ("pointer" for device or host addresses, "buffer"
// for host arrays the library reads or fills).
//
// kernels/layer.ts imports `hip`, `check` and the helpers below; the attention
// slice of its Layer is layer.ts in this directory.

const P = "pointer", U32 = "u32", I32 = "i32", U64 = "u64", F32 = "f32";

export const hip = Deno.dlopen(Deno.env.get("FLOCK_ATTN_LIB") ?? "libflock_attn.so", {
  // include/flock_attn.h
  flk_last_error: { parameters: [], result: P },
  flk_version: { parameters: [], result: P },
  flk_device_count: { parameters: [P], result: I32 },
  flk_set_stream: { parameters: [P], result: I32 },
  flk_alloc: { parameters: [P, U64], result: I32 },
  flk_free: { parameters: [P], result: I32 },
  flk_h2d: { parameters: [P, "buffer", U64, U64], result: I32 },
  flk_d2h: { parameters: ["buffer", P, U64, U64], result: I32 },
  flk_memset: { parameters: [P, I32, U64], result: I32 },
  // Blocking: the library's current stream and its error text belong to the
  // calling thread, so the wait and its status check stay on this thread.
  flk_sync: { parameters: [], result: I32 },
  flk_workspace_bytes: { parameters: [U32, U32, U32, U32, U32, U32], result: U64 },
  flk_call_workspace_bytes: { parameters: [I32, U32, U32, U32, U32, U32, U32], result: U64 },
  flk_rmsnorm: { parameters: [P, P, P, U32, U32, F32], result: I32 },
  flk_rope: { parameters: [P, P, U32, U32, U32, U32, I32], result: I32 },
  flk_kv_append: { parameters: [P, P, P, P, U32, U32, U32, U32, U32], result: I32 },
  flk_qk_prologue: {
    parameters: [P, P, P, P, P, P, F32, I32, P, P, P, U32, U32, U32, U32, U32, U32],
    result: I32,
  },
  flk_qk_prologue_strided: {
    parameters: [P, P, P, U32, P, P, P, F32, I32, P, P, P, U32, U32, U32, U32, U32, U32],
    result: I32,
  },
  flk_attn_decode: { parameters: [P, P, P, P, U32, U32, U32, U32, P, U64], result: I32 },
  flk_attn_prefill: { parameters: [P, P, P, P, U32, U32, U32, U32, U32, P, U64], result: I32 },
  flk_decode_layer: {
    parameters: [P, P, P, P, P, P, F32, I32, P, P, P, P, U32, U32, U32, U32, U32, P, U64],
    result: I32,
  },
  flk_decode_layer_noalloc: {
    parameters: [P, P, P, P, P, P, F32, I32, P, P, P, P, U32, U32, U32, U32, U32],
    result: I32,
  },
  flk_attn_decode_ragged: {
    parameters: [P, P, P, P, P, P, U32, U32, U32, U32, U32, P, U64],
    result: I32,
  },
  flk_decode_layer_ragged: {
    parameters: [P, P, P, P, P, P, F32, I32, P, P, P, P, P, P, U32, U32, U32, U32, U32, P, U64],
    result: I32,
  },
  // include/flock_q8.h
  flk_q8_matvec: { parameters: [P, P, P, P, U32, U32, U32], result: I32 },
  flk_q8_split: { parameters: ["buffer", U32, U32, "buffer", "buffer"], result: I32 },
  flk_q8_matvec_ex: { parameters: [P, P, P, P, U32, U32, U32, P, F32, P, P], result: I32 },
  flk_q8_gate_up_swiglu: { parameters: [P, P, P, P, U32, U32, U32, P, F32], result: I32 },
  flk_swiglu: { parameters: [P, P, P, U32], result: I32 },
  flk_add: { parameters: [P, P, P, U32], result: I32 },
  flk_argmax_ws_bytes: { parameters: [U32], result: U64 },
  flk_argmax: { parameters: [P, U32, P, P, P, U64], result: I32 },
  flk_lm_head_ws_bytes: { parameters: [U32, U32], result: U64 },
  flk_lm_head: { parameters: [P, P, F32, P, P, U32, U32, P, P, P, P, P, U64], result: I32 },
  // include/flock_graph.h
  flk_decode_layer_dev: {
    parameters: [P, P, P, P, P, P, F32, I32, P, P, P, P, P, U32, U32, U32, U32, P, U64],
    result: I32,
  },
  flk_embed: { parameters: [P, P, P, U32, U32, U32, P], result: I32 },
  flk_advance: { parameters: [P, U32, P, P, U32], result: I32 },
  flk_stream_create: { parameters: ["buffer"], result: I32 },
  flk_stream_destroy: { parameters: [P], result: I32 },
  flk_capture_begin: { parameters: [], result: I32 },
  flk_capture_end: { parameters: ["buffer"], result: I32 },
  flk_graph_launch: { parameters: [P], result: I32 },
  flk_graph_destroy: { parameters: [P], result: I32 },
  // include/flock_wire.h
  flk_f32_to_f16: { parameters: [P, P, U64], result: I32 },
  flk_f16_to_f32: { parameters: [P, P, U64], result: I32 },
  flk_wire_header_pack: { parameters: [U32, U32, U32, U32, "buffer"], result: I32 },
  flk_wire_header_unpack: {
    parameters: ["buffer", U64, "buffer", "buffer", "buffer", "buffer", "buffer"],
    result: I32,
  },
} as const);

/** Status codes (include/flock_attn.h). */
export const FLK_OK = 0, FLK_ERR_ARG = -1, FLK_ERR_CACHE_FULL = -2, FLK_ERR_UNSUPPORTED = -3,
  FLK_ERR_WORKSPACE = -4, FLK_ERR_HIP = -5;
/** RoPE pairing: NEOX pairs (j, j + d/2), NORM pairs (2j, 2j + 1) (lib.ts:517-531). */
export const FLK_ROPE_NEOX = 0, FLK_ROPE_NORM = 1;

export class FlockAttnError extends Error {
  constructor(readonly code: number, message: string) {
    super(message);
  }
}

/** Throw for a non-zero status, with the library's message (the calls
 *  validate on the host before launching, so a throw leaves nothing queued --
 *  the same place layer.ts throws, layer.ts:575, 689-698). */
export function check(rc: number, what: string): void {
  if (rc === FLK_OK) return;
  const p = hip.symbols.flk_last_error();
  const msg = p === null ? "" : new Deno.UnsafePointerView(p).getCString();
  throw new FlockAttnError(rc, `${what}: ${msg}`);
}

export type DevPtr = Deno.PointerValue;

/** Device memory of `bytes` bytes (storageBuffer, lib.ts:548-566). */
export function alloc(bytes: number): DevPtr {
  const out = new BigUint64Array(1);
  check(hip.symbols.flk_alloc(Deno.UnsafePointer.of(out), BigInt(bytes)), "flk_alloc");
  return Deno.UnsafePointer.create(out[0]);
}

export function free(p: DevPtr): void {
  check(hip.symbols.flk_free(p), "flk_free");
}

/** `p + bytes` for a device address (sub-buffer views, e.g. k inside q|k|v). */
export function offset(p: DevPtr, bytes: number): DevPtr {
  return bytes === 0 ? p : Deno.UnsafePointer.offset(p!, bytes);
}

/** Host -> device copy (writeBuffer), synchronous. */
export function upload(dst: DevPtr, src: Float32Array | Uint32Array, dstOffset = 0): void {
  check(hip.symbols.flk_h2d(dst, src, BigInt(src.byteLength), BigInt(dstOffset)), "flk_h2d");
}

/** Device -> host copy of `count` floats (readBack, lib.ts:575-593). */
export function download(src: DevPtr, count: number, srcOffset = 0): Float32Array {
  const out = new Float32Array(count);
  check(hip.symbols.flk_d2h(out, src, BigInt(out.byteLength), BigInt(srcOffset)), "flk_d2h");
  return out;
}

/** Wait for the library's stream (the mapAsync fence of layer.ts:801-816);
 *  a device error surfaces here as a FlockAttnError. Async like mapAsync. */
export async function sync(): Promise<void> {
  check(hip.symbols.flk_sync(), "flk_sync");
}

/** inv_freq[j] = fround(1 / base^(2j/d)), computed on the host as layer.ts:180-186 does. */
export function invFreqOf(headDim: number, base: number): Float32Array {
  const out = new Float32Array(headDim / 2);
  for (let j = 0; j < headDim / 2; j++) out[j] = Math.fround(1 / Math.pow(base, (2 * j) / headDim));
  return out;
}
