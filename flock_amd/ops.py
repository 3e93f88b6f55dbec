"""Python wrappers over the C ABI: device buffers, workspace, stream, and one
function per entry point of include/flock_attn.h.

Device arrays may be passed as a DeviceBuffer, a raw device pointer (int), or a
contiguous device tensor exposing ``data_ptr()`` (e.g. a torch tensor on the
GPU). Shapes are the reference's flat layouts (see flock_attn.h).
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from ._lib import ROPE_NEOX, ROPE_NORM, FlockError, check, lib

PAIRING = {"neox": ROPE_NEOX, "norm": ROPE_NORM}


def _pairing(p) -> int:
    if isinstance(p, str):
        if p not in PAIRING:
            raise ValueError(f"rope pairing must be 'neox' or 'norm', got {p!r}")
        return PAIRING[p]
    return int(p)


# Device pointers of buffers that were garbage-collected. flk_free waits for
# the device, so a collection must not free on the spot (it could stall a
# timed loop, or land inside a graph capture); the pointers are released at
# the next sync() or release_pending().
_pending_free: list[int] = []


def release_pending(raise_errors: bool = True) -> None:
    """Free the buffers collected since the last sync() (waits for the device).

    A pointer leaves the list only once flk_free has released it: a refused
    free (e.g. during a graph capture) keeps it for a later call."""
    while _pending_free:
        rc = lib().flk_free(_pending_free[-1])
        if rc != 0:
            if raise_errors:
                check(rc, "flk_free")
            return
        _pending_free.pop()


class DeviceBuffer:
    """Device memory from flk_alloc (the reference's storageBuffer).

    free() releases it at once (flk_free waits for the device); a buffer that
    is simply dropped is released at the next sync(), release_pending() or
    allocation."""

    def __init__(self, nbytes: int):
        if nbytes <= 0:
            raise ValueError("DeviceBuffer needs a positive size")
        # An allocation is a natural point to return collected buffers (a
        # loop that only reads results back never calls sync()); a refused
        # free, as under graph capture, leaves them for later.
        release_pending(raise_errors=False)
        p = ctypes.c_void_p()
        check(lib().flk_alloc(ctypes.byref(p), nbytes), "flk_alloc")
        self.ptr = p.value
        self.nbytes = nbytes

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 4))
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset_bytes: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset_bytes + a.nbytes > self.nbytes:
            raise ValueError(f"upload of {a.nbytes} B at {offset_bytes} overruns {self.nbytes} B")
        check(lib().flk_h2d(self.ptr, a.ctypes.data, a.nbytes, offset_bytes), "flk_h2d")

    def download(self, count: int, dtype=np.float32, offset_bytes: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        if offset_bytes + out.nbytes > self.nbytes:
            raise ValueError("download overruns the buffer")
        check(lib().flk_d2h(out.ctypes.data, self.ptr, out.nbytes, offset_bytes), "flk_d2h")
        return out

    def zero(self) -> None:
        check(lib().flk_memset(self.ptr, 0, self.nbytes), "flk_memset")

    def free(self) -> None:
        if getattr(self, "ptr", None):
            check(lib().flk_free(self.ptr), "flk_free")
            self.ptr = None

    def __del__(self):
        p = getattr(self, "ptr", None)
        if p and _pending_free is not None:  # None while the interpreter shuts down
            _pending_free.append(p)
            self.ptr = None


def ptr(x) -> int | None:
    """Device address of a DeviceBuffer, int pointer or device tensor."""
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        if getattr(x, "is_cuda", True) is False:
            raise ValueError("host tensor passed where a device array is required")
        if hasattr(x, "is_contiguous") and not x.is_contiguous():
            raise ValueError("device tensor must be contiguous")
        return int(x.data_ptr())
    raise TypeError(f"cannot take a device pointer of {type(x).__name__}")


def workspace_bytes(n_heads: int, n_kv_heads: int, head_dim: int, max_keys: int,
                    max_queries: int = 0, max_seqs: int = 1) -> int:
    n = lib().flk_workspace_bytes(n_heads, n_kv_heads, head_dim, max_keys, max_queries, max_seqs)
    if n == 0:
        raise FlockError(-1, "invalid shape for flk_workspace_bytes")
    return int(n)


class Workspace(DeviceBuffer):
    """Split-K scratch sized by flk_workspace_bytes (no initialisation needed)."""

    def __init__(self, n_heads: int, n_kv_heads: int, head_dim: int, max_keys: int,
                 max_queries: int = 0, max_seqs: int = 1):
        super().__init__(workspace_bytes(n_heads, n_kv_heads, head_dim, max_keys, max_queries,
                                         max_seqs))


def set_stream(stream) -> None:
    """Launch on ``stream``: a hipStream_t (int), a torch stream, or None."""
    if stream is None:
        h = None
    elif isinstance(stream, int):
        h = stream
    elif isinstance(stream, Stream):
        h = stream.handle
    else:
        h = int(stream.cuda_stream)
    check(lib().flk_set_stream(h), "flk_set_stream")


def sync() -> None:
    """Wait for the library stream, then release dropped buffers."""
    check(lib().flk_sync(), "flk_sync")
    release_pending()


def device_count() -> int:
    n = ctypes.c_int32(0)
    check(lib().flk_device_count(ctypes.byref(n)))
    return n.value


def rope_inv_freq(head_dim: int, base: float) -> np.ndarray:
    """inv_freq[j] = f32(1 / base^(2j/d)) on the host (kernels/layer.ts:180-186)."""
    return np.array([1.0 / math.pow(base, (2.0 * j) / head_dim) for j in range(head_dim // 2)],
                    dtype=np.float32)


def _ws(ws) -> tuple[int, int]:
    if ws is None:
        return None, 0
    if isinstance(ws, DeviceBuffer):
        return ws.ptr, ws.nbytes
    p, n = ws
    return ptr(p), int(n)


def rmsnorm(x, g, o, n: int, n_vecs: int, eps: float) -> None:
    check(lib().flk_rmsnorm(ptr(x), ptr(g), ptr(o), n, n_vecs, eps), "flk_rmsnorm")


def rope(x, inv_freq, n_tokens: int, n_heads: int, head_dim: int, pos0: int,
         pairing="neox") -> None:
    check(lib().flk_rope(ptr(x), ptr(inv_freq), n_tokens, n_heads, head_dim, pos0,
                         _pairing(pairing)), "flk_rope")


def kv_append(kn, v, kcache, vcache, n_tokens: int, pos0: int, n_kv_heads: int, head_dim: int,
              max_keys: int) -> None:
    check(lib().flk_kv_append(ptr(kn), ptr(v), ptr(kcache), ptr(vcache), n_tokens, pos0,
                              n_kv_heads, head_dim, max_keys), "flk_kv_append")


def qk_prologue(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps: float, pairing, qn_out, kcache,
                vcache, n_tokens: int, pos0: int, n_heads: int, n_kv_heads: int, head_dim: int,
                max_keys: int, in_stride: int = 0) -> None:
    """flk_qk_prologue; in_stride > 0: raw rows of consecutive tokens lie that
    many floats apart (flk_qk_prologue_strided, e.g. a q|k|v stacked output)."""
    if in_stride:
        check(lib().flk_qk_prologue_strided(ptr(q_raw), ptr(k_raw), ptr(v_raw), in_stride,
                                            ptr(gq), ptr(gk), ptr(inv_freq), eps,
                                            _pairing(pairing), ptr(qn_out), ptr(kcache),
                                            ptr(vcache), n_tokens, pos0, n_heads, n_kv_heads,
                                            head_dim, max_keys), "flk_qk_prologue_strided")
        return
    check(lib().flk_qk_prologue(ptr(q_raw), ptr(k_raw), ptr(v_raw), ptr(gq), ptr(gk),
                                ptr(inv_freq), eps, _pairing(pairing), ptr(qn_out), ptr(kcache),
                                ptr(vcache), n_tokens, pos0, n_heads, n_kv_heads, head_dim,
                                max_keys), "flk_qk_prologue")


def attn_decode(q, kcache, vcache, o, n_heads: int, n_kv_heads: int, head_dim: int,
                n_keys: int, ws) -> None:
    w, nb = _ws(ws)
    check(lib().flk_attn_decode(ptr(q), ptr(kcache), ptr(vcache), ptr(o), n_heads, n_kv_heads,
                                head_dim, n_keys, w, nb), "flk_attn_decode")


def attn_prefill(q, kcache, vcache, o, n_heads: int, n_kv_heads: int, head_dim: int,
                 n_queries: int, pos0: int, ws) -> None:
    w, nb = _ws(ws)
    check(lib().flk_attn_prefill(ptr(q), ptr(kcache), ptr(vcache), ptr(o), n_heads, n_kv_heads,
                                 head_dim, n_queries, pos0, w, nb), "flk_attn_prefill")


def decode_layer(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps: float, pairing, qn_out, kcache,
                 vcache, o, pos: int, n_heads: int, n_kv_heads: int, head_dim: int,
                 max_keys: int, ws) -> None:
    w, nb = _ws(ws)
    check(lib().flk_decode_layer(ptr(q_raw), ptr(k_raw), ptr(v_raw), ptr(gq), ptr(gk),
                                 ptr(inv_freq), eps, _pairing(pairing), ptr(qn_out), ptr(kcache),
                                 ptr(vcache), ptr(o), pos, n_heads, n_kv_heads, head_dim,
                                 max_keys, w, nb), "flk_decode_layer")


def decode_layer_noalloc(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps: float, pairing, qn_out,
                         kcache, vcache, o, pos: int, n_heads: int, n_kv_heads: int,
                         head_dim: int, max_keys: int) -> None:
    """flk_decode_layer without a workspace: the library's static scratch holds
    the split-K partials (no allocation; calls on one device must not overlap)."""
    check(lib().flk_decode_layer_noalloc(ptr(q_raw), ptr(k_raw), ptr(v_raw), ptr(gq), ptr(gk),
                                         ptr(inv_freq), eps, _pairing(pairing), ptr(qn_out),
                                         ptr(kcache), ptr(vcache), ptr(o), pos, n_heads,
                                         n_kv_heads, head_dim, max_keys),
          "flk_decode_layer_noalloc")


def decode_layer_dev(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps: float, pairing, qn_out, kcache,
                     vcache, o, n_keys_dev, n_heads: int, n_kv_heads: int, head_dim: int,
                     max_keys: int, ws) -> None:
    """flk_decode_layer with the key count (position + 1) in device memory."""
    w, nb = _ws(ws)
    check(lib().flk_decode_layer_dev(ptr(q_raw), ptr(k_raw), ptr(v_raw), ptr(gq), ptr(gk),
                                     ptr(inv_freq), eps, _pairing(pairing), ptr(qn_out),
                                     ptr(kcache), ptr(vcache), ptr(o), ptr(n_keys_dev), n_heads,
                                     n_kv_heads, head_dim, max_keys, w, nb),
          "flk_decode_layer_dev")


def attn_decode_ragged(q, kcache, vcache, seq_row_off, n_keys, o, n_seqs: int, max_n_keys: int,
                       n_heads: int, n_kv_heads: int, head_dim: int, ws) -> None:
    w, nb = _ws(ws)
    check(lib().flk_attn_decode_ragged(ptr(q), ptr(kcache), ptr(vcache), ptr(seq_row_off),
                                       ptr(n_keys), ptr(o), n_seqs, max_n_keys, n_heads,
                                       n_kv_heads, head_dim, w, nb), "flk_attn_decode_ragged")


def decode_layer_ragged(q_raw, k_raw, v_raw, gq, gk, inv_freq, eps: float, pairing, qn_out,
                        kcache, vcache, seq_row_off, n_keys, o, n_seqs: int, max_n_keys: int,
                        n_heads: int, n_kv_heads: int, head_dim: int, ws) -> None:
    """One decode step for every sequence of a ragged batch (flk_decode_layer_ragged):
    sequence b's new token is at position n_keys[b] - 1 of its cache rows."""
    w, nb = _ws(ws)
    check(lib().flk_decode_layer_ragged(ptr(q_raw), ptr(k_raw), ptr(v_raw), ptr(gq), ptr(gk),
                                        ptr(inv_freq), eps, _pairing(pairing), ptr(qn_out),
                                        ptr(kcache), ptr(vcache), ptr(seq_row_off), ptr(n_keys),
                                        ptr(o), n_seqs, max_n_keys, n_heads, n_kv_heads,
                                        head_dim, w, nb), "flk_decode_layer_ragged")


# ------------------------------------------------------------ Q8_0 projections
def q8_split(packed, n_rows: int, n_cols: int):
    """splitQ8 (kernels/lib.ts:141-156) on the host: GGUF Q8_0 bytes -> (qs int8, scales f16 bits)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    if n_cols % 32 or packed.size != n_rows * n_cols // 32 * 34:
        raise ValueError(f"{packed.size} bytes is not {n_rows} x {n_cols} Q8_0")
    qs = np.empty(n_rows * n_cols, np.int8)
    sc = np.empty(n_rows * n_cols // 32, np.uint16)
    check(lib().flk_q8_split(packed.ctypes.data, n_rows, n_cols, qs.ctypes.data, sc.ctypes.data),
          "flk_q8_split")
    return qs, sc


class Q8Matrix:
    """One Q8_0 weight matrix resident on the device (the reference's
    `wq[name]` = {qs, sc, rows, cols}, kernels/layer.ts:430-448)."""

    def __init__(self, qs, scales, n_rows: int, n_cols: int):
        self.rows, self.cols = n_rows, n_cols
        self.qs = DeviceBuffer.from_array(np.ascontiguousarray(qs, np.int8))
        self.scales = DeviceBuffer.from_array(np.ascontiguousarray(scales, np.uint16))

    @classmethod
    def from_packed(cls, packed, n_rows: int, n_cols: int) -> "Q8Matrix":
        qs, sc = q8_split(packed, n_rows, n_cols)
        return cls(qs, sc, n_rows, n_cols)


def q8_matvec(w, x, o, n_tokens: int = 1, qs=None, scales=None, n_rows: int | None = None,
              n_cols: int | None = None) -> None:
    """Layer.matvec (kernels/layer.ts:495-510): o[t] = W x[t] for t < n_tokens.

    ``w`` is a Q8Matrix, or None with ``qs``/``scales``/``n_rows``/``n_cols``
    given as device buffers and sizes.
    """
    if w is not None:
        qs, scales, n_rows, n_cols = w.qs, w.scales, w.rows, w.cols
    check(lib().flk_q8_matvec(ptr(qs), ptr(scales), ptr(x), ptr(o), n_rows, n_cols, n_tokens),
          "flk_q8_matvec")


def q8_matvec_ex(w: "Q8Matrix", x, o, n_tokens: int = 1, norm_gain=None, eps: float = 0.0,
                 up=None, res=None) -> None:
    """flk_q8_matvec_ex: o = [res +] W f(x), f = rmsnorm (norm_gain) or swiglu(., up)."""
    check(lib().flk_q8_matvec_ex(ptr(w.qs), ptr(w.scales), ptr(x), ptr(o), w.rows, w.cols,
                                 n_tokens, ptr(norm_gain), eps, ptr(up), ptr(res)),
          "flk_q8_matvec_ex")


def q8_gate_up_swiglu(w: "Q8Matrix", x, act, n_tokens: int = 1, norm_gain=None,
                      eps: float = 0.0) -> None:
    """act = swiglu(gate, up) of the (gate, up)-interleaved matrix ``w`` times f(x)."""
    check(lib().flk_q8_gate_up_swiglu(ptr(w.qs), ptr(w.scales), ptr(x), ptr(act), w.rows // 2,
                                      w.cols, n_tokens, ptr(norm_gain), eps),
          "flk_q8_gate_up_swiglu")


def interleave_rows(a, b, rows: int, row_len: int) -> np.ndarray:
    """Rows a0, b0, a1, b1, ... of two [rows][row_len] arrays."""
    a = np.asarray(a).reshape(rows, row_len)
    b = np.asarray(b).reshape(rows, row_len)
    return np.stack([a, b], axis=1).reshape(-1)


def swiglu(gate, up, o, n: int) -> None:
    """elementwise.wgsl swiglu: o = silu(gate) * up."""
    check(lib().flk_swiglu(ptr(gate), ptr(up), ptr(o), n), "flk_swiglu")


def add(a, b, o, n: int) -> None:
    """elementwise.wgsl add: o = a + b."""
    check(lib().flk_add(ptr(a), ptr(b), ptr(o), n), "flk_add")


# ---------------------------------------------------------------- the head
def argmax_ws_bytes(n: int) -> int:
    return int(lib().flk_argmax_ws_bytes(n))


def argmax(x, n: int, oval, oidx, ws) -> None:
    """argmax.wgsl pass1 + pass2 (model.ts:337-346): largest value, lowest index."""
    w, nb = _ws(ws)
    check(lib().flk_argmax(ptr(x), n, ptr(oval), ptr(oidx), w, nb), "flk_argmax")


def lm_head_ws_bytes(vocab: int, hidden: int) -> int:
    return int(lib().flk_lm_head_ws_bytes(vocab, hidden))


def lm_head(x, gain, eps: float, w: "Q8Matrix", normed, logits, oval, oidx, ws) -> None:
    """encodeHead (model.ts:307-346): rmsnorm -> tied Q8_0 projection -> argmax.

    ``w`` is the vocab x hidden matrix; ``logits`` may be None.
    """
    wsp, nb = _ws(ws)
    check(lib().flk_lm_head(ptr(x), ptr(gain), eps, ptr(w.qs), ptr(w.scales), w.rows, w.cols,
                            ptr(normed), ptr(logits), ptr(oval), ptr(oidx), wsp, nb),
          "flk_lm_head")



# ------------------------------------------------------------- graphs
def embed(w: "Q8Matrix", ids, n_tokens: int, out) -> None:
    """embed.wgsl: out[t] = dequantized row ids[t] of ``w`` (device ids)."""
    check(lib().flk_embed(ptr(w.qs), ptr(w.scales), ptr(ids), n_tokens, w.rows, w.cols, ptr(out)),
          "flk_embed")


def advance(state, delta: int = 1, value=None, log=None, log_len: int = 0) -> None:
    """state = device {n_keys, cursor}: n_keys += delta; log[cursor++] = *value."""
    check(lib().flk_advance(ptr(state), delta, ptr(value), ptr(log), log_len), "flk_advance")


class Stream:
    """A library-created stream of default priority (capturable)."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().flk_stream_create(ctypes.byref(h)), "flk_stream_create")
        self.handle = h.value

    def free(self) -> None:
        if self.handle:
            lib().flk_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Graph:
    """Calls made inside ``with Graph() as g:`` are captured from the library
    stream (not run); ``g.launch()`` replays them."""

    def __init__(self):
        self.handle = None

    def __enter__(self):
        check(lib().flk_capture_begin(), "flk_capture_begin")
        return self

    def __exit__(self, exc_type, exc, tb):
        h = ctypes.c_void_p()
        rc = lib().flk_capture_end(ctypes.byref(h))
        if exc_type is None:
            check(rc, "flk_capture_end")
        self.handle = h.value
        return False

    def launch(self) -> None:
        check(lib().flk_graph_launch(self.handle), "flk_graph_launch")

    def free(self) -> None:
        if self.handle:
            lib().flk_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
