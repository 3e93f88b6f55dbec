"""FLK1 payload conversions on the GPU against the oracle (web/js/wire.mjs)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

from flock_amd import _lib, ops  # noqa: E402


def test_f32_to_f16_every_class(rng):
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),
        (rng.standard_normal(50000) * 1e-8).astype(np.float32),
        (rng.standard_normal(50000) * 4e4).astype(np.float32),
        rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 65504, 65520, 2.0 ** -24, 2.0 ** -25,
                    1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11]),
    ])
    n = vals.size
    src = ops.DeviceBuffer.from_array(vals)
    dst = ops.DeviceBuffer(2 * n)
    ops.check(_lib.lib().flk_f32_to_f16(src.ptr, dst.ptr, n), "flk_f32_to_f16")
    got = dst.download(n, np.uint16)
    want = oracle.f32_to_f16_array(vals)
    assert np.array_equal(got, want)


def test_f16_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    src = ops.DeviceBuffer.from_array(h)
    dst = ops.DeviceBuffer(4 * h.size)
    ops.check(_lib.lib().flk_f16_to_f32(src.ptr, dst.ptr, h.size), "flk_f16_to_f32")
    got = dst.download(h.size)
    want = np.array([oracle.f16_to_f32_wire(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # -0 kept
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)


def test_frame_round_trip_through_the_device(rng):
    # A worker packs its activations on the GPU and the coordinator's unpack
    # reads them; the reverse feeds a replay chunk back in.
    hidden, n = 1024, 64
    acts = (rng.standard_normal(n * hidden) * 0.05).astype(np.float32)
    a = ops.DeviceBuffer.from_array(acts)
    h16 = ops.DeviceBuffer(2 * acts.size)
    ops.check(_lib.lib().flk_f32_to_f16(a.ptr, h16.ptr, acts.size), "pack")
    import ctypes
    head = ctypes.create_string_buffer(20)
    _lib.lib().flk_wire_header_pack(3, hidden, 128, 2, head)
    frame = head.raw + h16.download(acts.size, np.uint16).astype("<u2").tobytes()
    assert frame == oracle.wire_pack(acts, 3, hidden, 128, replay=True)
    data, meta = oracle.wire_unpack(frame)
    back = ops.DeviceBuffer(4 * acts.size)
    ops.check(_lib.lib().flk_f16_to_f32(h16.ptr, back.ptr, acts.size), "unpack")
    assert np.array_equal(back.download(acts.size), data)
