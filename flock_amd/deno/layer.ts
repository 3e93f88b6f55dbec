// The attention slice of flock's Layer (kernels/layer.ts) on libflock_attn:
// the TypeScript form of flock_amd/layer.py, with the reference's names,
// position semantics and guard messages.
//
//   create(cfg, gq, gk)       allocates every buffer once (layer.ts:362-448);
//                             kernels never allocate.
//   nKeys                     host state: advanced by encode / encodePrefill,
//                             reset by reset(), writable (layer.ts:203-204).
//   encode(q, k, v)           one decode step at position nKeys -- per-head
//                             q/k RMSNorm, RoPE, K/V append and decode
//                             attention in ONE call (layer.ts:582-630).
//   encodePrefill(n, q, k, v) n positions at nKeys: the fused prologue, then
//                             causal prefill attention (layer.ts:705-750).
//
// q, k, v are the raw projections (the reference's matvec outputs). Omit them
// to use what a producer already wrote into inputBuffers(), the way layer.ts
// omits `hidden` to chain layers. Every guard throws before anything is
// launched, with the reference's message.

import {
  alloc,
  check,
  download,
  FLK_ROPE_NEOX,
  FLK_ROPE_NORM,
  free,
  hip,
  invFreqOf,
  type DevPtr,
  sync,
  upload,
} from "./hip_attn.ts";

/** LayerConfig (layer.ts:87-112), attention fields. */
export interface AttnConfig {
  nHeads: number;
  nKvHeads: number;
  headDim: number;
  eps: number;
  ropeBase: number;
  maxKeys: number;
  maxPrefill: number;
  ropePairing?: "neox" | "norm";
}

/** QWEN3_06B (layer.ts:119-130), attention fields. */
export const QWEN3_06B_ATTN: AttnConfig = {
  nHeads: 16,
  nKvHeads: 8,
  headDim: 128,
  eps: Math.fround(1e-6),
  ropeBase: 1e6,
  maxKeys: 2048,
  maxPrefill: 512,
  ropePairing: "neox",
};

export class Layer {
  nKeys = 0;
  readonly buf: Record<string, DevPtr> = {};
  private wsBytes = 0n;

  private constructor(readonly cfg: AttnConfig) {}

  static create(cfg: AttnConfig, gq: Float32Array, gk: Float32Array): Layer {
    const { nHeads: H, nKvHeads: Hkv, headDim: d, maxKeys } = cfg;
    if (!(maxKeys >= 1) || !Number.isInteger(maxKeys)) {
      throw new Error(`maxKeys must be a positive integer, got ${maxKeys}`);
    }
    if (gq.length !== d || gk.length !== d) {
      throw new Error(`q/k norm gains must have headDim=${d} entries`);
    }
    const L = new Layer(cfg);
    const P = Math.max(1, cfg.maxPrefill), f = 4;
    L.buf.q = alloc(P * H * d * f);
    L.buf.k = alloc(P * Hkv * d * f);
    L.buf.v = alloc(P * Hkv * d * f);
    L.buf.qn = alloc(P * H * d * f);
    L.buf.attn = alloc(P * H * d * f);
    L.buf.kcache = alloc(maxKeys * Hkv * d * f);
    L.buf.vcache = alloc(maxKeys * Hkv * d * f);
    L.buf.invFreq = alloc((d / 2) * f);
    upload(L.buf.invFreq, invFreqOf(d, cfg.ropeBase));
    L.buf.gq = alloc(d * f);
    upload(L.buf.gq, gq);
    L.buf.gk = alloc(d * f);
    upload(L.buf.gk, gk);
    L.wsBytes = BigInt(hip.symbols.flk_workspace_bytes(H, Hkv, d, maxKeys, P, 1));
    L.buf.ws = alloc(Number(L.wsBytes));
    return L;
  }

  /** Reset the KV cache for a new sequence (layer.ts:451-453). */
  reset(): void {
    this.nKeys = 0;
  }

  private pairing(): number {
    return (this.cfg.ropePairing ?? "neox") === "norm" ? FLK_ROPE_NORM : FLK_ROPE_NEOX;
  }

  private writeInputs(n: number, q?: Float32Array, k?: Float32Array, v?: Float32Array) {
    const { nHeads: H, nKvHeads: Hkv, headDim: d } = this.cfg;
    if (!q && !k && !v) return;
    if (!q || !k || !v) throw new Error("pass all of q, k, v or none of them");
    const want = { q: n * H * d, k: n * Hkv * d, v: n * Hkv * d };
    for (const [name, x] of [["q", q], ["k", k], ["v", v]] as const) {
      if (x.length !== want[name]) throw new Error(`${name} is ${x.length}, expected ${want[name]}`);
    }
    upload(this.buf.q, q);
    upload(this.buf.k, k);
    upload(this.buf.v, v);
  }

  /** One decode step at position nKeys (layer.ts:571-654, attention slice). */
  encode(q?: Float32Array, k?: Float32Array, v?: Float32Array): void {
    const { cfg, buf } = this;
    const pos = this.nKeys;
    if (pos >= cfg.maxKeys) throw new Error(`KV cache full at ${cfg.maxKeys} keys`);
    this.writeInputs(1, q, k, v);
    check(
      hip.symbols.flk_decode_layer(
        buf.q, buf.k, buf.v, buf.gq, buf.gk, buf.invFreq, cfg.eps, this.pairing(),
        buf.qn, buf.kcache, buf.vcache, buf.attn,
        pos, cfg.nHeads, cfg.nKvHeads, cfg.headDim, cfg.maxKeys, buf.ws, this.wsBytes,
      ),
      "decode",
    );
    this.nKeys = pos + 1;
  }

  /** A prefill of nTokens positions starting at nKeys (layer.ts:685-767). */
  encodePrefill(nTokens: number, q?: Float32Array, k?: Float32Array, v?: Float32Array): void {
    const { cfg, buf } = this;
    const pos = this.nKeys;
    if (nTokens < 1) throw new Error(`nTokens must be >= 1, got ${nTokens}`);
    if (nTokens > cfg.maxPrefill) {
      throw new Error(`prefill of ${nTokens} exceeds maxPrefill ${cfg.maxPrefill}; chunk it`);
    }
    if (pos + nTokens > cfg.maxKeys) {
      throw new Error(`KV cache would exceed ${cfg.maxKeys} keys (${pos} + ${nTokens})`);
    }
    this.writeInputs(nTokens, q, k, v);
    check(
      hip.symbols.flk_qk_prologue(
        buf.q, buf.k, buf.v, buf.gq, buf.gk, buf.invFreq, cfg.eps, this.pairing(),
        buf.qn, buf.kcache, buf.vcache, nTokens, pos, cfg.nHeads, cfg.nKvHeads, cfg.headDim,
        cfg.maxKeys,
      ),
      "prologue",
    );
    check(
      hip.symbols.flk_attn_prefill(
        buf.qn, buf.kcache, buf.vcache, buf.attn, cfg.nHeads, cfg.nKvHeads, cfg.headDim,
        nTokens, pos, buf.ws, this.wsBytes,
      ),
      "prefill",
    );
    this.nKeys = pos + nTokens;
  }

  /** Raw q/k/v device buffers a producer (the projections) may write directly. */
  inputBuffers(): { q: DevPtr; k: DevPtr; v: DevPtr } {
    return { q: this.buf.q, k: this.buf.k, v: this.buf.v };
  }

  /** The attention output [n][nHeads][headDim] (layer.ts buf.attn). */
  outputBuffer(): DevPtr {
    return this.buf.attn;
  }

  /** The KV cache buffers (layer.ts:787-789). */
  cacheBuffers(): { k: DevPtr; v: DevPtr } {
    return { k: this.buf.kcache, v: this.buf.vcache };
  }

  /** The attention output of the last encode / encodePrefill. */
  async readOutput(nTokens = 1): Promise<Float32Array> {
    await sync();
    return download(this.buf.attn, nTokens * this.cfg.nHeads * this.cfg.headDim);
  }

  destroy(): void {
    for (const p of Object.values(this.buf)) free(p);
  }
}
