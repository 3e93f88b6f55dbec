"""The attention slice of flock's ``Layer`` (kernels/layer.ts), on libflock_attn.

Same names, position semantics and guard rails as the reference class:

* ``Layer.create(cfg, gq, gk)`` allocates every buffer once (layer.ts:362-448):
  q/k/v inputs, qn, the attention output, the KV cache ``[maxKeys][Hkv][d]``,
  inv_freq and the split-K workspace. Kernels never allocate.
* ``nKeys`` is host state: advanced only by ``encode`` / ``encodePrefill``,
  reset by ``reset()``, and writable for benchmarks (layer.ts:203-204, 451-453).
* ``encode(q, k, v)`` is one decode step at position ``nKeys`` (layer.ts:571-654):
  per-head q/k RMSNorm -> RoPE -> K/V append -> decode attention, in one launch.
* ``encodePrefill(n, q, k, v)`` is an n-token prefill at ``nKeys``
  (layer.ts:685-767): the fused prologue, then causal prefill attention.
* Inputs are the raw q/k/v projections (the reference's matvec outputs, which
  are outside this path). Omit them to consume what is already in
  ``inputBuffers()``, the way the reference omits ``hidden`` to chain layers.
* Guard failures raise before anything is launched, with the reference's
  messages: cache full (layer.ts:575, 693-695), prefill larger than maxPrefill
  (690-692), wrong input length (696-698), n < 1 (689), and an ``offset``
  different from ``nKeys`` (the desync check of web/bird.html:563-567).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from ._lib import CacheFullError, FlockError
from . import ops


class DesyncError(FlockError):
    """The caller's position does not match the cache (bird.html:563-567)."""

    def __init__(self, message: str):
        super().__init__(-6, message)


@dataclass(frozen=True)
class LayerConfig:
    """LayerConfig (layer.ts:87-112), attention fields only."""

    nHeads: int = 16
    nKvHeads: int = 8
    headDim: int = 128
    eps: float = 9.999999974752427e-7
    ropeBase: float = 1e6
    maxKeys: int = 2048
    maxPrefill: int = 512
    ropePairing: str = "neox"


# QWEN3_06B (layer.ts:119-130), attention fields.
QWEN3_06B = LayerConfig()


class Layer:
    def __init__(self, cfg: LayerConfig, gq: np.ndarray, gk: np.ndarray):
        if cfg.maxKeys < 1 or int(cfg.maxKeys) != cfg.maxKeys:
            raise ValueError(f"maxKeys must be a positive integer, got {cfg.maxKeys}")
        if cfg.ropePairing not in ("neox", "norm"):
            raise ValueError(f"ropePairing must be 'neox' or 'norm', got {cfg.ropePairing!r}")
        H, Hkv, d = cfg.nHeads, cfg.nKvHeads, cfg.headDim
        gq = np.ascontiguousarray(gq, np.float32).ravel()
        gk = np.ascontiguousarray(gk, np.float32).ravel()
        if gq.size != d or gk.size != d:
            raise ValueError(f"q/k norm gains must have headDim={d} entries")
        self.cfg = cfg
        P = max(1, cfg.maxPrefill)
        f = 4
        self.buf = {
            "q": ops.DeviceBuffer(P * H * d * f),
            "k": ops.DeviceBuffer(P * Hkv * d * f),
            "v": ops.DeviceBuffer(P * Hkv * d * f),
            "qn": ops.DeviceBuffer(P * H * d * f),
            "attn": ops.DeviceBuffer(P * H * d * f),
            "kcache": ops.DeviceBuffer(cfg.maxKeys * Hkv * d * f),
            "vcache": ops.DeviceBuffer(cfg.maxKeys * Hkv * d * f),
            "invFreq": ops.DeviceBuffer.from_array(ops.rope_inv_freq(d, cfg.ropeBase)),
            "g_attn_q_norm": ops.DeviceBuffer.from_array(gq),
            "g_attn_k_norm": ops.DeviceBuffer.from_array(gk),
        }
        self.ws = ops.Workspace(H, Hkv, d, cfg.maxKeys, P, 1)
        self.nKeys = 0

    @classmethod
    def create(cls, cfg: LayerConfig, gq: np.ndarray, gk: np.ndarray) -> "Layer":
        return cls(cfg, gq, gk)

    def reset(self) -> None:
        """Reset the KV cache for a new sequence (layer.ts:451-453)."""
        self.nKeys = 0

    # ------------------------------------------------------------------ inputs
    def _write_inputs(self, n: int, q, k, v) -> None:
        H, Hkv, d = self.cfg.nHeads, self.cfg.nKvHeads, self.cfg.headDim
        given = [x is not None for x in (q, k, v)]
        if any(given) and not all(given):
            raise ValueError("pass all of q, k, v or none of them")
        if not any(given):
            return
        want = {"q": n * H * d, "k": n * Hkv * d, "v": n * Hkv * d}
        arrs = {}
        for name, x in (("q", q), ("k", k), ("v", v)):
            a = np.ascontiguousarray(x, np.float32).ravel()
            if a.size != want[name]:
                raise ValueError(f"{name} is {a.size}, expected {want[name]}")
            arrs[name] = a
        for name, a in arrs.items():
            self.buf[name].upload(a)

    def _check_offset(self, offset) -> None:
        if offset is not None and offset != self.nKeys:
            raise DesyncError(f"desync: offset {offset} but the cache holds {self.nKeys} keys")

    # ------------------------------------------------------------------ encode
    def encode(self, q=None, k=None, v=None, offset: int | None = None) -> None:
        """One decode step at position nKeys (layer.ts:571-654, attention slice)."""
        cfg, b = self.cfg, self.buf
        pos = self.nKeys
        self._check_offset(offset)
        if pos >= cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache full at {cfg.maxKeys} keys")
        self._write_inputs(1, q, k, v)
        ops.decode_layer(b["q"], b["k"], b["v"], b["g_attn_q_norm"], b["g_attn_k_norm"],
                         b["invFreq"], cfg.eps, cfg.ropePairing, b["qn"], b["kcache"],
                         b["vcache"], b["attn"], pos, cfg.nHeads, cfg.nKvHeads, cfg.headDim,
                         cfg.maxKeys, self.ws)
        self.nKeys = pos + 1

    def encodePrefill(self, nTokens: int, q=None, k=None, v=None,
                      offset: int | None = None) -> None:
        """A prefill of nTokens positions starting at nKeys (layer.ts:685-767)."""
        cfg, b = self.cfg, self.buf
        pos = self.nKeys
        self._check_offset(offset)
        if nTokens < 1:
            raise ValueError(f"nTokens must be >= 1, got {nTokens}")
        if nTokens > cfg.maxPrefill:
            raise ValueError(f"prefill of {nTokens} exceeds maxPrefill {cfg.maxPrefill}; chunk it")
        if pos + nTokens > cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache would exceed {cfg.maxKeys} keys ({pos} + {nTokens})")
        self._write_inputs(nTokens, q, k, v)
        ops.qk_prologue(b["q"], b["k"], b["v"], b["g_attn_q_norm"], b["g_attn_k_norm"],
                        b["invFreq"], cfg.eps, cfg.ropePairing, b["qn"], b["kcache"],
                        b["vcache"], nTokens, pos, cfg.nHeads, cfg.nKvHeads, cfg.headDim,
                        cfg.maxKeys)
        ops.attn_prefill(b["qn"], b["kcache"], b["vcache"], b["attn"], cfg.nHeads, cfg.nKvHeads,
                         cfg.headDim, nTokens, pos, self.ws)
        self.nKeys = pos + nTokens

    # ----------------------------------------------------------------- buffers
    def inputBuffers(self) -> dict:
        """Raw q/k/v device buffers a producer kernel may write directly."""
        return {"q": self.buf["q"], "k": self.buf["k"], "v": self.buf["v"]}

    def outputBuffer(self) -> ops.DeviceBuffer:
        """The attention output [n][nHeads][headDim] (layer.ts buf.attn)."""
        return self.buf["attn"]

    def cacheBuffers(self) -> dict:
        """The KV cache buffers (layer.ts:787-789)."""
        return {"k": self.buf["kcache"], "v": self.buf["vcache"]}

    def readOutput(self, nTokens: int = 1) -> np.ndarray:
        """Attention output of the last encode/encodePrefill (synchronous)."""
        c = self.cfg
        return self.buf["attn"].download(nTokens * c.nHeads * c.headDim)

    def readQn(self, nTokens: int = 1) -> np.ndarray:
        """The normed + rotated q that attention consumed."""
        c = self.cfg
        return self.buf["qn"].download(nTokens * c.nHeads * c.headDim)

    def readCache(self, nKeys: int) -> tuple[np.ndarray, np.ndarray]:
        """The first nKeys rows of the K and V caches."""
        c = self.cfg
        n = nKeys * c.nKvHeads * c.headDim
        return self.buf["kcache"].download(n), self.buf["vcache"].download(n)

    def free(self) -> None:
        for b in self.buf.values():
            b.free()
        self.ws.free()
