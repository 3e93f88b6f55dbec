"""Rebuilding a KV cache by replaying journaled activations, on the GPU.

flock journals the f16 activation of every token it feeds (FLK1 frames,
web/js/wire.mjs:24-94) and, when a bird's cache is lost, replays the journal
to it in chunks of FLOCK_REPLAY_CHUNK = 64 positions, the first chunk with
`reset` (server/server.js:1013, 1034-1077). The rebuilt cache is claimed to be
bit-for-bit the cache an uninterrupted run holds (README.md:189-197), resting
on two facts: f16 round-trips exactly, and prefill leaves the KV cache
bit-identical to decoding the same hidden states one at a time
(kernels/test_prefill.ts:119-132). Both are exercised here end to end through
libflock_attn: the activations are packed into FLK1 frames and unpacked on the
device (flk_f32_to_f16 / flk_wire_header_pack / flk_wire_header_unpack /
flk_f16_to_f32), then fed to a DecoderLayer once token by token (the
uninterrupted run) and once as 64-token replay chunks (the rebuild; chunks
after the first land on a non-empty cache).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

from flock_amd import _lib, ops  # noqa: E402
from flock_amd.decoder import DecoderConfig, DecoderLayer  # noqa: E402
from flock_amd.model import Model  # noqa: E402
from test_gpu_decoder import make_weights  # noqa: E402
from test_gpu_model import VOCAB, build  # noqa: E402

REPLAY_CHUNK = 64
FLAG_RESET, FLAG_REPLAY = 1, 2


def journal(acts: np.ndarray, hidden: int) -> list[bytes]:
    """One FLK1 frame per token: the payload converted to f16 on the device,
    the 20-byte header packed by the library."""
    n = acts.size // hidden
    src = ops.DeviceBuffer.from_array(np.ascontiguousarray(acts, np.float32))
    h16 = ops.DeviceBuffer(2 * acts.size)
    ops.check(_lib.lib().flk_f32_to_f16(src.ptr, h16.ptr, acts.size), "flk_f32_to_f16")
    payload = h16.download(acts.size, np.uint16).astype("<u2")
    frames = []
    for t in range(n):
        head = ctypes.create_string_buffer(20)
        ops.check(_lib.lib().flk_wire_header_pack(t, hidden, t, 0, head), "header")
        frames.append(head.raw + payload[t * hidden:(t + 1) * hidden].tobytes())
    return frames


def replay_chunks(frames: list[bytes], hidden: int):
    """The journal as the rebuild sends it: chunks of REPLAY_CHUNK tokens,
    marked replay (the first also reset), unpacked to f32 on the device.
    Yields (offset, n_tokens, activations)."""
    for off in range(0, len(frames), REPLAY_CHUNK):
        chunk = frames[off:off + REPLAY_CHUNK]
        want_flags = FLAG_REPLAY | (FLAG_RESET if off == 0 else 0)
        payload = bytearray()
        for i, journaled in enumerate(chunk):
            head = ctypes.create_string_buffer(20)  # re-sent with the replay flags
            ops.check(_lib.lib().flk_wire_header_pack(off + i, hidden, off + i, want_flags, head),
                      "header")
            f = head.raw + journaled[20:]
            seq, hid, offset, flags, nvals = (ctypes.c_uint32(), ctypes.c_uint32(),
                                              ctypes.c_uint32(), ctypes.c_uint32(),
                                              ctypes.c_uint64())
            ops.check(_lib.lib().flk_wire_header_unpack(
                f, len(f), ctypes.byref(seq), ctypes.byref(hid), ctypes.byref(offset),
                ctypes.byref(flags), ctypes.byref(nvals)), "unpack")
            assert hid.value == hidden and offset.value == off + i and nvals.value == hidden
            assert flags.value == want_flags
            payload += f[20:]
        h16 = ops.DeviceBuffer.from_array(np.frombuffer(bytes(payload), "<u2"))
        out = ops.DeviceBuffer(4 * len(chunk) * hidden)
        ops.check(_lib.lib().flk_f16_to_f32(h16.ptr, out.ptr, len(chunk) * hidden), "f16_to_f32")
        yield off, len(chunk), out.download(len(chunk) * hidden)


@pytest.mark.parametrize("n", [64, 130])
def test_replayed_layer_cache_equals_the_decoded_one(rng, n):
    cfg = DecoderConfig(maxKeys=256, maxPrefill=REPLAY_CHUNK)
    w = make_weights(rng, cfg)
    hid = cfg.hidden
    acts = rng.standard_normal(n * hid).astype(np.float32)
    frames = journal(acts, hid)
    fed = np.concatenate([a for _, _, a in replay_chunks(frames, hid)])
    # What the bird receives is the f16 value of what was sent, exactly.
    assert np.array_equal(fed, oracle.wire_unpack(oracle.wire_pack(acts, 0, hid))[0])

    # The uninterrupted run: one decode step per token.
    A = DecoderLayer.create(cfg, w)
    out_a = []
    for t in range(n):
        A.encode(fed[t * hid:(t + 1) * hid])
        out_a.append(A.readOutput())
    out_a = np.concatenate(out_a)

    # The rebuild: the journal replayed in 64-token chunks.
    B = DecoderLayer.create(cfg, w)
    out_b = []
    for off, m, chunk in replay_chunks(frames, hid):
        B.encodePrefill(m, chunk, offset=off)
        out_b.append(B.readOutput(m))
    out_b = np.concatenate(out_b)

    ka, va = A.readCache(n)
    kb, vb = B.readCache(n)
    assert A.nKeys == B.nKeys == n
    assert np.array_equal(ka, kb) and np.array_equal(va, vb), "rebuilt KV cache differs"
    # The layer's outputs (what the next bird is sent) agree to the bar of
    # test_prefill.ts:110-115; attention sums in a different order on the
    # two paths, so they are not bit-identical.
    err = oracle.abs_err_scaled(out_b, out_a, oracle.amax(out_a))
    print(f"n={n}: layer output abs/scale {err:.2e}; f16 values that differ: "
          f"{int(np.sum(oracle.f32_to_f16_array(out_a) != oracle.f32_to_f16_array(out_b)))}"
          f" of {out_a.size}")
    assert err < 2e-6
    A.free()
    B.free()


def test_replayed_model_gives_the_same_next_token(rng):
    # A whole (small) model: a 130-id prompt fed one id at a time versus the
    # same ids prefilled in chunks of 64. The first layer's cache is fed the
    # same embeddings on both paths and must be bit-identical; deeper layers
    # are fed the previous layer's outputs, which differ in their last bits
    # (attention's summation order), so their caches agree to rounding only.
    # The next greedy token must be the same.
    cfg, layers, embd, gout = build(rng, n_layers=3, maxKeys=256, maxPrefill=REPLAY_CHUNK)
    prompt = rng.integers(0, VOCAB, 130).astype(np.uint32)
    a = Model(cfg, layers, embd, gout, VOCAB, max_generate=4)
    for t in prompt[:-1]:
        a.step([t])
    next_a = a.step([prompt[-1]])
    b = Model(cfg, layers, embd, gout, VOCAB, max_generate=4)
    next_b = b.step(prompt)
    assert a.nKeys == b.nKeys == prompt.size
    assert next_a == next_b
    for i, (la, lb) in enumerate(zip(a.layers, b.layers)):
        ka, va = la.readCache(prompt.size)
        kb, vb = lb.readCache(prompt.size)
        if i == 0:
            assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        else:
            assert oracle.abs_err_scaled(kb, ka, oracle.amax(ka)) < 1e-4
            assert oracle.abs_err_scaled(vb, va, oracle.amax(va)) < 1e-4
    a.free()
    b.free()
