"""CPU oracle for flock's attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker. The product (flock_amd) never imports it.

Two independent formulations live here:

* ``flock_oracle.c`` (wrapped below): the reference's strict-f32 CPU oracle
  restated rounding point for rounding point (kernels/ops_ref.ts,
  kernels/head_ref.ts, kernels/layer_ref.ts, kernels/lib.ts:169-171).
* ``flock_oracle_q8.c``: the Q8_0 projection references (kernels/lib.ts:28-53,
  141-156, 196-278; web/js/wire.mjs:33-53).
* ``closed_form``: textbook float64 formulas (softmax(q k^T / sqrt d) v with
  the GQA map and causal bound, RMSNorm, rotation) used to pin the
  restatement. They share no code with it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libflock_oracle.so")
_lib = None

NEOX, NORM = 0, 1
PAIRING = {"neox": NEOX, "norm": NORM}
# qwen3.attention.layer_norm_rms_epsilon as the f32 the reference uploads
# (kernels/layer.ts:124).
QWEN3_EPS = 9.999999974752427e-7
QWEN3_ROPE_BASE = 1e6

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> str:
    """Compile flock_oracle.c with oracle/Makefile (gcc, strict IEEE)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i, d, i64 = ctypes.c_int, ctypes.c_double, ctypes.c_int64
        sig = {
            "flko_rmsnorm": (None, [_f32p, _f32p, _f32p, i, i, d, i]),
            "flko_rope": (None, [_f32p, i, i, i, i, _f32p, i]),
            "flko_rope_inv_freq": (None, [i, d, _f32p]),
            "flko_attn": (None, [_f32p, _f32p, _f32p, _f32p, i, i, i, i]),
            "flko_attn_prefill": (None, [_f32p, _f32p, _f32p, _f32p, i, i, i, i, i, i, i]),
            "flko_argmax": (i, [_f32p, i]),
            "flko_rel_err": (d, [_f32p, _f32p, i64, d]),
            "flko_abs_err_scaled": (d, [_f32p, _f32p, i64, d]),
            "flko_amax": (d, [_f32p, i64]),
            "flko_layer_attn_decode": (
                None,
                [_f32p] * 6 + [d, i] + [_f32p] * 4 + [i, i, i, i],
            ),
            "flko_layer_attn_prefill": (
                None,
                [_f32p] * 6 + [d, i] + [_f32p] * 4 + [i, i, i, i, i],
            ),
            "flko_set_threads": (i, [i]),
            "flko_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "flko_half_to_f32": (d, [ctypes.c_uint16]),
            "flko_quant_row_q8": (None, [_f32p, i64, _u8p]),
            "flko_split_q8": (None, [_u8p, i, i, _u8p, _u8p]),
            "flko_q8_matvec": (None, [_u8p, _f32p, i, i, i, i, _f32p]),
            "flko_argmax_wgsl": (None, [_f32p, i64, _f32p, ctypes.POINTER(ctypes.c_uint32)]),
            "flko_swiglu": (None, [_f32p, _f32p, _f32p, i64]),
            "flko_f16_to_f32_wire": (d, [ctypes.c_uint16]),
            "flko_add": (None, [_f32p, _f32p, _f32p, i64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def set_threads(n: int) -> int:
    """Threads for the oracle's parallel loops (heads / query-head pairs)."""
    return lib().flko_set_threads(int(n))


def rmsnorm(x, g, n: int, n_vecs: int, eps: float = QWEN3_EPS, wg: int = 128) -> np.ndarray:
    """rmsnormRef, kernels/ops_ref.ts:20-49."""
    x, g = _f32(x), _f32(g)
    assert x.size == n * n_vecs and g.size == n and wg & (wg - 1) == 0
    o = np.empty(n * n_vecs, np.float32)
    lib().flko_rmsnorm(_p(x), _p(g), _p(o), n, n_vecs, float(eps), wg)
    return o


def rope(x, n_tokens: int, n_heads: int, head_dim: int, pos0: int, inv_freq,
         pairing: str = "neox") -> np.ndarray:
    """ropeRef, kernels/ops_ref.ts:65-92 (returns a rotated copy)."""
    out = _f32(x).copy()
    inv = _f32(inv_freq)
    assert out.size == n_tokens * n_heads * head_dim and inv.size == head_dim // 2
    lib().flko_rope(_p(out), n_tokens, n_heads, head_dim, pos0, _p(inv), PAIRING[pairing])
    return out


def rope_inv_freq(head_dim: int, base: float = QWEN3_ROPE_BASE) -> np.ndarray:
    """ropeInvFreq, kernels/ops_ref.ts:95-100."""
    out = np.empty(head_dim // 2, np.float32)
    lib().flko_rope_inv_freq(head_dim, float(base), _p(out))
    return out


def attn(q, k, v, n_heads: int, n_kv_heads: int, head_dim: int, n_keys: int) -> np.ndarray:
    """attnRef, kernels/ops_ref.ts:135-174."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    assert q.size == n_heads * head_dim
    assert k.size >= n_keys * n_kv_heads * head_dim and v.size >= n_keys * n_kv_heads * head_dim
    o = np.empty(n_heads * head_dim, np.float32)
    lib().flko_attn(_p(q), _p(k), _p(v), _p(o), n_heads, n_kv_heads, head_dim, n_keys)
    return o


def attn_prefill(q, k, v, n_heads: int, n_kv_heads: int, head_dim: int, n_queries: int,
                 pos0: int, tile: int = 64, wg: int = 128) -> np.ndarray:
    """attnPrefillRef, kernels/head_ref.ts:99-183."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    n_keys = pos0 + n_queries
    assert q.size == n_queries * n_heads * head_dim
    assert k.size >= n_keys * n_kv_heads * head_dim and v.size >= n_keys * n_kv_heads * head_dim
    o = np.empty(n_queries * n_heads * head_dim, np.float32)
    lib().flko_attn_prefill(_p(q), _p(k), _p(v), _p(o), n_heads, n_kv_heads, head_dim,
                            n_queries, pos0, tile, wg)
    return o


def argmax(x) -> int:
    """argmaxRef, kernels/head_ref.ts:65-74 (lowest index wins ties)."""
    x = _f32(x)
    return int(lib().flko_argmax(_p(x), x.size))


def rel_err(a, b, floor: float = 1e-6) -> float:
    """relErr, kernels/ops_ref.ts:185-191."""
    a, b = _f32(a), _f32(b)
    assert a.size == b.size
    return float(lib().flko_rel_err(_p(a), _p(b), a.size, floor))


def abs_err_scaled(a, b, scale: float) -> float:
    """absErrScaled, kernels/ops_ref.ts:206-210."""
    a, b = _f32(a), _f32(b)
    assert a.size == b.size
    return float(lib().flko_abs_err_scaled(_p(a), _p(b), a.size, float(scale)))


def amax(a) -> float:
    """amax, kernels/ops_ref.ts:213-217."""
    a = _f32(a)
    return float(lib().flko_amax(_p(a), a.size))


def layer_attn_decode(q_raw, k_raw, v_raw, gq, gk, inv_freq, kcache: np.ndarray,
                      vcache: np.ndarray, pos: int, n_heads: int, n_kv_heads: int,
                      head_dim: int, eps: float = QWEN3_EPS, pairing: str = "neox"):
    """Attention slice of layerForwardRef, kernels/layer_ref.ts:46-70.

    Appends row ``pos`` to ``kcache``/``vcache`` (float32, modified in place) and
    returns ``(qn, o)``.
    """
    assert kcache.dtype == np.float32 and kcache.flags.c_contiguous
    assert vcache.dtype == np.float32 and vcache.flags.c_contiguous
    assert kcache.size >= (pos + 1) * n_kv_heads * head_dim
    args = [_f32(a) for a in (q_raw, k_raw, v_raw, gq, gk, inv_freq)]
    qn = np.empty(n_heads * head_dim, np.float32)
    o = np.empty(n_heads * head_dim, np.float32)
    lib().flko_layer_attn_decode(*[_p(a) for a in args], float(eps), PAIRING[pairing],
                                 _p(kcache), _p(vcache), _p(qn), _p(o), pos, n_heads,
                                 n_kv_heads, head_dim)
    return qn, o


def layer_attn_prefill(q_raw, k_raw, v_raw, gq, gk, inv_freq, kcache: np.ndarray,
                       vcache: np.ndarray, n: int, pos0: int, n_heads: int, n_kv_heads: int,
                       head_dim: int, eps: float = QWEN3_EPS, pairing: str = "neox"):
    """Attention slice of layerPrefillRef, kernels/layer_ref.ts:137-165.

    Appends rows ``pos0 .. pos0+n-1`` to the caches in place; returns ``(qn, o)``.
    """
    assert kcache.dtype == np.float32 and kcache.flags.c_contiguous
    assert vcache.dtype == np.float32 and vcache.flags.c_contiguous
    assert kcache.size >= (pos0 + n) * n_kv_heads * head_dim
    args = [_f32(a) for a in (q_raw, k_raw, v_raw, gq, gk, inv_freq)]
    qn = np.empty(n * n_heads * head_dim, np.float32)
    o = np.empty(n * n_heads * head_dim, np.float32)
    lib().flko_layer_attn_prefill(*[_p(a) for a in args], float(eps), PAIRING[pairing],
                                  _p(kcache), _p(vcache), _p(qn), _p(o), n, pos0, n_heads,
                                  n_kv_heads, head_dim)
    return qn, o


# ---------------------------------------------------------------- Q8_0 ------
Q8_BLOCK, Q8_BYTES = 32, 34


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


def _pu8(a: np.ndarray):
    return a.ctypes.data_as(_u8p)


def f32_to_f16(v) -> int:
    """f32to16, web/js/wire.mjs:33-53 (f16 bits of an f32, round to nearest even)."""
    return int(lib().flko_f32_to_f16(float(np.float32(v))))


def f32_to_f16_array(a) -> np.ndarray:
    a = _f32(a).ravel()
    f = lib().flko_f32_to_f16
    return np.array([f(float(v)) for v in a], dtype=np.uint16)


def half_to_f32(h: int) -> float:
    """halfToF32, kernels/lib.ts:28-33 (exponent 31 clamps to +-3.4028235e38)."""
    return float(lib().flko_half_to_f32(int(h) & 0xFFFF))


def quant_matrix_q8(w, rows: int, cols: int) -> np.ndarray:
    """quantMatrixQ8 / quantRowQ8, kernels/lib.ts:38-53, 102-109: 34-byte blocks.

    Rows are concatenations of independent 32-value blocks, so the whole
    matrix goes through quantRowQ8's block loop in one call.
    """
    w = _f32(w).ravel()
    assert w.size == rows * cols and cols % Q8_BLOCK == 0
    out = np.empty(rows * cols // Q8_BLOCK * Q8_BYTES, np.uint8)
    lib().flko_quant_row_q8(_p(w), rows * cols, _pu8(out))
    return out


def split_q8(packed, rows: int, cols: int):
    """splitQ8, kernels/lib.ts:141-156: (qs int8 [rows*cols], scales f16 bits [rows*cols/32])."""
    packed = _u8(packed)
    assert packed.size == rows * cols // Q8_BLOCK * Q8_BYTES
    qs = np.empty(rows * cols, np.uint8)
    sc = np.empty(rows * cols // Q8_BLOCK * 2, np.uint8)
    lib().flko_split_q8(_pu8(packed), rows, cols, _pu8(qs), _pu8(sc))
    return qs.view(np.int8), sc.view(np.uint16)


def q8_matvec(packed, x, rows: int, cols: int, lanes: int = 64, fused: bool = False) -> np.ndarray:
    """cpuMatmulQ8F32, kernels/lib.ts:196-278: W (34-byte Q8_0 blocks) times x.

    ``lanes=0`` is SERIAL (q8_matmul.wgsl), ``lanes=64`` is coop(64)
    (q8_coop.wgsl). ``fused`` swaps the reference's fma32 (two roundings) for
    a one-rounding fmaf. ``x`` may hold several tokens ([n_tokens][cols]).
    """
    packed, x = _u8(packed), _f32(x)
    assert packed.size == rows * cols // Q8_BLOCK * Q8_BYTES and x.size % cols == 0
    assert lanes == 0 or (lanes & (lanes - 1) == 0 and lanes <= 1024)
    nt = x.size // cols
    out = np.empty(nt * rows, np.float32)
    for t in range(nt):
        xt = np.ascontiguousarray(x[t * cols:(t + 1) * cols])
        ot = np.empty(rows, np.float32)
        lib().flko_q8_matvec(_pu8(packed), _p(xt), rows, cols, lanes, int(bool(fused)), _p(ot))
        out[t * rows:(t + 1) * rows] = ot
    return out


def argmax_wgsl(x):
    """argmax.wgsl (kernels/argmax.wgsl:54-56, 92-134): (value, index) of the
    largest element, lowest index among equal values, NaN never chosen,
    (-3.4028235e38, 0xffffffff) when nothing beats that."""
    x = _f32(x).ravel()
    v = np.empty(1, np.float32)
    i = np.empty(1, np.uint32)
    lib().flko_argmax_wgsl(_p(x), x.size, _p(v), i.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return float(v[0]), int(i[0])


def lm_head(x, gain, eps: float, packed, vocab: int, hidden: int):
    """encodeHead, kernels/model.ts:307-346: rmsnorm (rmsnorm.wgsl, one vector)
    -> Q8_0 vocab projection (coop(64)) -> argmax.wgsl.
    Returns (normed, logits, value, index)."""
    normed = rmsnorm(x, gain, hidden, 1, eps)
    logits = q8_matvec(packed, normed, vocab, hidden, 64, fused=True)
    v, i = argmax_wgsl(logits)
    return normed, logits, v, i


def swiglu(gate, up) -> np.ndarray:
    """swigluRef, kernels/ops_ref.ts:103-110."""
    gate, up = _f32(gate).ravel(), _f32(up).ravel()
    assert gate.size == up.size
    o = np.empty(gate.size, np.float32)
    lib().flko_swiglu(_p(gate), _p(up), _p(o), gate.size)
    return o


def add(a, b) -> np.ndarray:
    """addRef, kernels/ops_ref.ts:113-117."""
    a, b = _f32(a).ravel(), _f32(b).ravel()
    assert a.size == b.size
    o = np.empty(a.size, np.float32)
    lib().flko_add(_p(a), _p(b), _p(o), a.size)
    return o


def layer_forward(hidden, w: dict, cfg: dict, kcache: np.ndarray, vcache: np.ndarray, pos: int,
                  fused: bool = False) -> np.ndarray:
    """layerForwardRef (kernels/layer_ref.ts:32-82): one decode step of a whole
    Qwen3 layer, composed of the restated ops. ``w`` maps the reference's
    tensor names to 34-byte Q8_0 bytes (projections) or f32 gains; the cache
    rows ``pos`` are written in place. Returns the layer output."""
    H, Hkv, d = cfg["nHeads"], cfg["nKvHeads"], cfg["headDim"]
    hid, ffn, eps = cfg["hidden"], cfg["ffn"], cfg["eps"]
    mv = lambda name, x, rows, cols: q8_matvec(w[name], x, rows, cols, 64, fused)  # noqa: E731
    nh = rmsnorm(hidden, w["attn_norm.weight"], hid, 1, eps)
    q = mv("attn_q.weight", nh, H * d, hid)
    k = mv("attn_k.weight", nh, Hkv * d, hid)
    v = mv("attn_v.weight", nh, Hkv * d, hid)
    _, attn_o = layer_attn_decode(q, k, v, w["attn_q_norm.weight"], w["attn_k_norm.weight"],
                                  rope_inv_freq(d, cfg.get("ropeBase", QWEN3_ROPE_BASE)), kcache,
                                  vcache, pos, H, Hkv, d, eps, cfg.get("ropePairing", "neox"))
    h = add(hidden, mv("attn_output.weight", attn_o, hid, H * d))
    nh2 = rmsnorm(h, w["ffn_norm.weight"], hid, 1, eps)
    act = swiglu(mv("ffn_gate.weight", nh2, ffn, hid), mv("ffn_up.weight", nh2, ffn, hid))
    return add(h, mv("ffn_down.weight", act, hid, ffn))


def layer_prefill(hidden, n: int, w: dict, cfg: dict, kcache: np.ndarray, vcache: np.ndarray,
                  pos0: int, fused: bool = False) -> np.ndarray:
    """layerPrefillRef (kernels/layer_ref.ts:84-177): n tokens at positions
    pos0 .. pos0+n-1; the batched matvec is the per-token one (layer_ref.ts:
    112-128). Cache rows are written in place; returns [n][hidden]."""
    H, Hkv, d = cfg["nHeads"], cfg["nKvHeads"], cfg["headDim"]
    hid, ffn, eps = cfg["hidden"], cfg["ffn"], cfg["eps"]
    mv = lambda name, x, rows, cols: q8_matvec(w[name], x, rows, cols, 64, fused)  # noqa: E731
    nh = rmsnorm(hidden, w["attn_norm.weight"], hid, n, eps)
    q = mv("attn_q.weight", nh, H * d, hid)
    k = mv("attn_k.weight", nh, Hkv * d, hid)
    v = mv("attn_v.weight", nh, Hkv * d, hid)
    _, attn_o = layer_attn_prefill(q, k, v, w["attn_q_norm.weight"], w["attn_k_norm.weight"],
                                   rope_inv_freq(d, cfg.get("ropeBase", QWEN3_ROPE_BASE)), kcache,
                                   vcache, n, pos0, H, Hkv, d, eps, cfg.get("ropePairing", "neox"))
    h = add(hidden, mv("attn_output.weight", attn_o, hid, H * d))
    nh2 = rmsnorm(h, w["ffn_norm.weight"], hid, n, eps)
    act = swiglu(mv("ffn_gate.weight", nh2, ffn, hid), mv("ffn_up.weight", nh2, ffn, hid))
    return add(h, mv("ffn_down.weight", act, hid, ffn))


# ---------------------------------------------------------------- FLK1 frames
WIRE_MAGIC = 0x314B4C46  # "FLK1" little-endian (web/js/wire.mjs:25)


def f16_to_f32_wire(h: int) -> float:
    """f16to32, web/js/wire.mjs:55-61 (inf and NaN kept)."""
    return float(lib().flko_f16_to_f32_wire(int(h) & 0xFFFF))


def wire_pack(floats, seq: int, hidden: int, offset: int = 0, reset: bool = False,
              replay: bool = False) -> bytes:
    """pack, web/js/wire.mjs:66-78."""
    import struct
    a = _f32(floats).ravel()
    head = struct.pack("<5I", WIRE_MAGIC, seq, hidden, offset, (1 if reset else 0) | (2 if replay else 0))
    return head + f32_to_f16_array(a).astype("<u2").tobytes()


def wire_unpack(buf: bytes):
    """unpack, web/js/wire.mjs:80-94: (data f32, meta dict)."""
    import struct
    if len(buf) < 20 or struct.unpack_from("<I", buf, 0)[0] != WIRE_MAGIC:
        raise ValueError("not a flock frame")
    _, seq, hidden, offset, flags = struct.unpack_from("<5I", buf, 0)
    n = (len(buf) - 20) // 2
    hs = np.frombuffer(buf, "<u2", n, 20)
    data = np.array([f16_to_f32_wire(int(h)) for h in hs], np.float32)
    return data, dict(seq=seq, hidden=hidden, offset=offset, reset=bool(flags & 1),
                      replay=bool(flags & 2))


def embed(packed, ids, vocab: int, hidden: int) -> np.ndarray:
    """embed.wgsl (kernels/embed.wgsl:52-75): row ids[t] of a Q8_0 matrix,
    each element the f32 product q * scale (scale per halfToF32)."""
    qs, sc = split_q8(packed, vocab, hidden)
    ids = np.asarray(ids, np.int64).ravel()
    out = np.empty((ids.size, hidden), np.float32)
    nb = hidden // 32
    for t, r in enumerate(ids):
        s = np.array([half_to_f32(int(h)) for h in sc[r * nb:(r + 1) * nb]], np.float32)
        out[t] = qs[r * hidden:(r + 1) * hidden].astype(np.float32) * np.repeat(s, 32)
    return out.ravel()
