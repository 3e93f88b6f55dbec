"""A whole Qwen3 decoder layer on libflock_attn (kernels/layer.ts ``Layer``).

``DecoderLayer`` is the full ``Layer`` of the reference: the attention block
(attn_norm -> q/k/v projections -> per-head q/k RMSNorm -> RoPE -> K/V append
-> attention -> o projection + residual) and the feed-forward block (ffn_norm
-> gate/up -> SwiGLU -> down + residual), layer.ts:571-654 (decode) and
685-767 (prefill). The attention-only mirror is ``flock_amd.layer.Layer``.

Weights use the reference's tensor names (``LayerWeights``, layer.ts:114-118):
Q8_0 projections as GGUF 34-byte blocks (``attn_q.weight``, ``attn_k.weight``,
``attn_v.weight``, ``attn_output.weight``, ``ffn_gate.weight``,
``ffn_up.weight``, ``ffn_down.weight``) and f32 gains (``attn_norm.weight``,
``ffn_norm.weight``, ``attn_q_norm.weight``, ``attn_k_norm.weight``).

Launches per decode step (the reference dispatches ~16): the norms, residual
adds and SwiGLU ride inside the projections, q/k/v are one projection over
the row-stacked matrix, gate/up one over the row-interleaved matrix:

  1. qkv = W_qkv rmsnorm(h)                 flk_q8_matvec_ex (norm fused)
  2. attention slice                        flk_decode_layer (2 kernels)
  3. h2 = h + W_o attn                      flk_q8_matvec_ex (residual fused)
  4. act = swiglu(W_gate|up rmsnorm(h2))    flk_q8_gate_up_swiglu (norm fused)
  5. out = h2 + W_down act                  flk_q8_matvec_ex (residual fused)

(hidden > 1024: gate/up stacked, SwiGLU computed as the down projection
loads its input.)

Every op keeps the reference's arithmetic, so the K/V rows this layer writes
are bit-identical to layerForwardRef's and the output differs from it only
through attention's summation order. Prefill runs the same ops over n tokens
(layer_ref.ts:112-128; 8 or more tokens take the weight-reusing tile
projections): one projection over q|k|v into a [n][q|k|v] buffer, the
prologue reading it strided (flk_qk_prologue_strided), prefill attention,
then o, gate/up and down as in decode.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from ._lib import CacheFullError
from . import ops
from .layer import DesyncError

PROJ = ("attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
        "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight")
GAINS = ("attn_norm.weight", "ffn_norm.weight", "attn_q_norm.weight", "attn_k_norm.weight")


@dataclass(frozen=True)
class DecoderConfig:
    """LayerConfig (layer.ts:87-112)."""

    hidden: int = 1024
    ffn: int = 3072
    nHeads: int = 16
    nKvHeads: int = 8
    headDim: int = 128
    eps: float = 9.999999974752427e-7
    ropeBase: float = 1e6
    maxKeys: int = 2048
    maxPrefill: int = 512
    ropePairing: str = "neox"

    def shapes(self) -> dict:
        H, Hkv, d, hid, ffn = self.nHeads, self.nKvHeads, self.headDim, self.hidden, self.ffn
        return {"attn_q.weight": (H * d, hid), "attn_k.weight": (Hkv * d, hid),
                "attn_v.weight": (Hkv * d, hid), "attn_output.weight": (hid, H * d),
                "ffn_gate.weight": (ffn, hid), "ffn_up.weight": (ffn, hid),
                "ffn_down.weight": (hid, ffn)}


QWEN3_06B = DecoderConfig()


class _Rows:
    """Rows [r0, r0 + rows) of a device Q8Matrix, usable as a Q8Matrix."""

    def __init__(self, m: ops.Q8Matrix, r0: int, rows: int):
        self.rows, self.cols = rows, m.cols
        self.qs = m.qs.ptr + r0 * m.cols
        self.scales = m.scales.ptr + r0 * (m.cols // 32) * 2


class DecoderLayer:
    def __init__(self, cfg: DecoderConfig, weights: dict):
        self.cfg = cfg
        H, Hkv, d, hid, ffn = cfg.nHeads, cfg.nKvHeads, cfg.headDim, cfg.hidden, cfg.ffn
        shapes = cfg.shapes()
        split = {}
        for name in PROJ:
            rows, cols = shapes[name]
            packed = np.ascontiguousarray(weights[name], np.uint8).ravel()
            if packed.size != rows * cols // 32 * 34:
                raise ValueError(f"{name}: {packed.size} bytes, expected {rows} x {cols} Q8_0")
            split[name] = ops.q8_split(packed, rows, cols)

        def stack(names):
            qs = np.concatenate([split[n][0] for n in names])
            sc = np.concatenate([split[n][1] for n in names])
            return ops.Q8Matrix(qs, sc, sum(shapes[n][0] for n in names), shapes[names[0]][1])

        # q|k|v stacked row-wise: one launch (same bits per row).
        self.w_qkv = stack(("attn_q.weight", "attn_k.weight", "attn_v.weight"))
        self.w_o = ops.Q8Matrix(*split["attn_output.weight"], hid, H * d)
        self.w_down = ops.Q8Matrix(*split["ffn_down.weight"], hid, ffn)
        self.w_q = _Rows(self.w_qkv, 0, H * d)
        self.w_k = _Rows(self.w_qkv, H * d, Hkv * d)
        self.w_v = _Rows(self.w_qkv, (H + Hkv) * d, Hkv * d)
        # gate and up: rows interleaved (gate_i, up_i), so one projection also
        # applies SwiGLU (flk_q8_gate_up_swiglu, hidden <= 1024); else stacked
        # and SwiGLU rides in the down projection's input.
        self.paired = hid <= 1024
        if self.paired:
            g_qs, g_sc = split["ffn_gate.weight"]
            u_qs, u_sc = split["ffn_up.weight"]
            self.w_gu = ops.Q8Matrix(ops.interleave_rows(g_qs, u_qs, ffn, hid),
                                     ops.interleave_rows(g_sc, u_sc, ffn, hid // 32), 2 * ffn, hid)
        else:
            self.w_gu = stack(("ffn_gate.weight", "ffn_up.weight"))
            self.w_gate = _Rows(self.w_gu, 0, ffn)
            self.w_up = _Rows(self.w_gu, ffn, ffn)
        self.g = {}
        for name in GAINS:
            want = d if "q_norm" in name or "k_norm" in name else hid
            g = np.ascontiguousarray(weights[name], np.float32).ravel()
            if g.size != want:
                raise ValueError(f"{name}: {g.size} entries, expected {want}")
            self.g[name] = ops.DeviceBuffer.from_array(g)

        P = max(1, cfg.maxPrefill)
        f = 4
        B = ops.DeviceBuffer
        self.buf = {
            "h": B(P * hid * f), "h2": B(P * hid * f), "out": B(P * hid * f),
            "qkv": B(P * (H + 2 * Hkv) * d * f),  # per token: q | k | v
            "qn": B(P * H * d * f), "attn": B(P * H * d * f),
            "gu": B(2 * ffn * f), "gate": B(P * ffn * f), "up": B(P * ffn * f),
            "act": B(P * ffn * f),
            "kcache": B(cfg.maxKeys * Hkv * d * f), "vcache": B(cfg.maxKeys * Hkv * d * f),
            "invFreq": B.from_array(ops.rope_inv_freq(d, cfg.ropeBase)),
        }
        self.out_dev = B(hid * f)
        self.ws = ops.Workspace(H, Hkv, d, cfg.maxKeys, P, 1)
        self.nKeys = 0

    @classmethod
    def create(cls, cfg: DecoderConfig, weights: dict) -> "DecoderLayer":
        return cls(cfg, weights)

    def reset(self) -> None:
        """Reset the KV cache for a new sequence (layer.ts:451-453)."""
        self.nKeys = 0

    def _hidden_in(self, n: int, hidden) -> None:
        if hidden is None:
            return
        a = np.ascontiguousarray(hidden, np.float32).ravel()
        if a.size != n * self.cfg.hidden:
            raise ValueError(f"hidden is {a.size}, expected {n * self.cfg.hidden}")
        self.buf["h"].upload(a)

    def _check_offset(self, offset) -> None:
        if offset is not None and offset != self.nKeys:
            raise DesyncError(f"desync: offset {offset} but the cache holds {self.nKeys} keys")

    # ------------------------------------------------------------------ decode
    def encode(self, hidden=None, offset: int | None = None, src=None) -> None:
        """One decode step at position nKeys (layer.ts:571-654). ``hidden``
        omitted: consume the previous step's output (layer.ts:645-648);
        ``src``: read the input from that device buffer instead (the previous
        layer's ``outputBuffer()``, no copy)."""
        cfg, b, g = self.cfg, self.buf, self.g
        H, Hkv, d = cfg.nHeads, cfg.nKvHeads, cfg.headDim
        pos = self.nKeys
        self._check_offset(offset)
        if pos >= cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache full at {cfg.maxKeys} keys")
        self._hidden_in(1, hidden)
        hin = b["h"] if src is None else src
        qkv = b["qkv"].ptr
        ops.q8_matvec_ex(self.w_qkv, hin, b["qkv"], 1, norm_gain=g["attn_norm.weight"],
                         eps=cfg.eps)
        ops.decode_layer(qkv, qkv + H * d * 4, qkv + (H + Hkv) * d * 4, g["attn_q_norm.weight"],
                         g["attn_k_norm.weight"], b["invFreq"], cfg.eps, cfg.ropePairing,
                         b["qn"], b["kcache"], b["vcache"], b["attn"], pos, H, Hkv, d,
                         cfg.maxKeys, self.ws)
        ops.q8_matvec_ex(self.w_o, b["attn"], b["h2"], 1, res=hin)
        self._ffn(1, b["out"])
        self._chain()
        self.nKeys = pos + 1

    def _ffn(self, n: int, out) -> None:
        """out = h2 + W_down swiglu(W_gate nh2, W_up nh2), nh2 = rmsnorm(h2)."""
        cfg, b, g = self.cfg, self.buf, self.g
        if self.paired:
            ops.q8_gate_up_swiglu(self.w_gu, b["h2"], b["act"], n, norm_gain=g["ffn_norm.weight"],
                                  eps=cfg.eps)
            ops.q8_matvec_ex(self.w_down, b["act"], out, n, res=b["h2"])
        elif n == 1:
            ops.q8_matvec_ex(self.w_gu, b["h2"], b["gu"], 1, norm_gain=g["ffn_norm.weight"],
                             eps=cfg.eps)
            ops.q8_matvec_ex(self.w_down, b["gu"], out, 1, up=b["gu"].ptr + cfg.ffn * 4,
                             res=b["h2"])
        else:
            for w, o in ((self.w_gate, b["gate"]), (self.w_up, b["up"])):
                ops.q8_matvec_ex(w, b["h2"], o, n, norm_gain=g["ffn_norm.weight"], eps=cfg.eps)
            ops.q8_matvec_ex(self.w_down, b["gate"], out, n, up=b["up"], res=b["h2"])

    def encode_dev(self, src, n_keys_dev) -> None:
        """One decode step whose position lives in device memory
        (*n_keys_dev = position + 1): the form a captured, replayed step uses.
        Reads its input from ``src`` and writes ``outputBufferDev()``; no host
        bookkeeping (the caller tracks the position and the cache bound)."""
        cfg, b, g = self.cfg, self.buf, self.g
        H, Hkv, d = cfg.nHeads, cfg.nKvHeads, cfg.headDim
        qkv = b["qkv"].ptr
        ops.q8_matvec_ex(self.w_qkv, src, b["qkv"], 1, norm_gain=g["attn_norm.weight"],
                         eps=cfg.eps)
        ops.decode_layer_dev(qkv, qkv + H * d * 4, qkv + (H + Hkv) * d * 4,
                             g["attn_q_norm.weight"], g["attn_k_norm.weight"], b["invFreq"],
                             cfg.eps, cfg.ropePairing, b["qn"], b["kcache"], b["vcache"],
                             b["attn"], n_keys_dev, H, Hkv, d, cfg.maxKeys, self.ws)
        ops.q8_matvec_ex(self.w_o, b["attn"], b["h2"], 1, res=src)
        self._ffn(1, self.out_dev)

    def outputBufferDev(self) -> ops.DeviceBuffer:
        """Where encode_dev writes (fixed, so a captured step can chain layers)."""
        return self.out_dev

    # ----------------------------------------------------------------- prefill
    def encodePrefill(self, nTokens: int, hidden=None, offset: int | None = None,
                      src=None) -> None:
        """nTokens positions starting at nKeys (layer.ts:685-767); ``src``: read
        the input rows from that device buffer (no copy)."""
        cfg, b, g = self.cfg, self.buf, self.g
        H, Hkv, d, hid, ffn = cfg.nHeads, cfg.nKvHeads, cfg.headDim, cfg.hidden, cfg.ffn
        pos = self.nKeys
        self._check_offset(offset)
        if nTokens < 1:
            raise ValueError(f"nTokens must be >= 1, got {nTokens}")
        if nTokens > cfg.maxPrefill:
            raise ValueError(f"prefill of {nTokens} exceeds maxPrefill {cfg.maxPrefill}; chunk it")
        if pos + nTokens > cfg.maxKeys:
            raise CacheFullError(-2, f"KV cache would exceed {cfg.maxKeys} keys ({pos} + {nTokens})")
        self._hidden_in(nTokens, hidden)
        n = nTokens
        hin = b["h"] if src is None else src
        # One projection over q|k|v stacked (layer.ts:722-724 runs three); the
        # prologue reads each token's q, k and v rows out of its q|k|v row.
        ops.q8_matvec_ex(self.w_qkv, hin, b["qkv"], n, norm_gain=g["attn_norm.weight"],
                         eps=cfg.eps)
        qkv, row = b["qkv"].ptr, (H + 2 * Hkv) * d
        ops.qk_prologue(qkv, qkv + H * d * 4, qkv + (H + Hkv) * d * 4, g["attn_q_norm.weight"],
                        g["attn_k_norm.weight"], b["invFreq"], cfg.eps, cfg.ropePairing, b["qn"],
                        b["kcache"], b["vcache"], n, pos, H, Hkv, d, cfg.maxKeys, in_stride=row)
        ops.attn_prefill(b["qn"], b["kcache"], b["vcache"], b["attn"], H, Hkv, d, n, pos, self.ws)
        ops.q8_matvec_ex(self.w_o, b["attn"], b["h2"], n, res=hin)
        self._ffn(n, b["out"])
        self._chain()
        self.nKeys = pos + n

    def _chain(self) -> None:
        # The output becomes the next call's input (layer.ts:645-648 copies
        # out -> h); swapping the two buffers' roles does it without a copy.
        self.buf["h"], self.buf["out"] = self.buf["out"], self.buf["h"]

    # ----------------------------------------------------------------- readout
    def outputBuffer(self) -> ops.DeviceBuffer:
        """The device buffer holding the last call's output (the next layer's input)."""
        return self.buf["h"]

    def readOutput(self, nTokens: int = 1) -> np.ndarray:
        """The layer output of the last encode / encodePrefill (synchronous)."""
        return self.buf["h"].download(nTokens * self.cfg.hidden)

    def readCache(self, nKeys: int) -> tuple[np.ndarray, np.ndarray]:
        c = self.cfg
        n = nKeys * c.nKvHeads * c.headDim
        return self.buf["kcache"].download(n), self.buf["vcache"].download(n)

    def free(self) -> None:
        for m in (self.w_qkv, self.w_gu, self.w_o, self.w_down):
            m.qs.free()
            m.scales.free()
        for x in list(self.buf.values()) + list(self.g.values()) + [self.out_dev]:
            x.free()
        self.ws.free()
