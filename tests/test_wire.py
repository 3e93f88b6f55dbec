"""FLK1 frames (web/js/wire.mjs): the oracle pinned against numpy's IEEE
float16 and hand-built headers; the library's host-side header functions
against the oracle (no GPU needed)."""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest

import oracle
from flock_amd import _lib


def test_f16_to_f32_wire_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float64)
    got = np.array([oracle.f16_to_f32_wire(int(v)) for v in h])
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])  # +-inf kept, unlike halfToF32


def test_pack_layout_and_round_trip():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(1024) * 0.05).astype(np.float32)
    frame = oracle.wire_pack(x, seq=7, hidden=1024, offset=33, reset=True, replay=True)
    assert frame[:20] == struct.pack("<5I", 0x314B4C46, 7, 1024, 33, 3)
    assert frame[:4] == b"FLK1"
    assert len(frame) == 20 + 2 * x.size
    data, meta = oracle.wire_unpack(frame)
    assert meta == dict(seq=7, hidden=1024, offset=33, reset=True, replay=True)
    assert np.array_equal(data, x.astype(np.float16).astype(np.float32))
    with pytest.raises(ValueError, match="not a flock frame"):
        oracle.wire_unpack(b"FLK2" + frame[4:])


def test_library_header_matches_oracle():
    L = _lib.lib()
    out = ctypes.create_string_buffer(20)
    assert L.flk_wire_header_pack(9, 1024, 5, 2, out) == 0
    assert out.raw == oracle.wire_pack(np.zeros(0, np.float32), 9, 1024, 5, replay=True)
    frame = oracle.wire_pack(np.ones(6, np.float32), 11, 6, 64, reset=True)
    vals = [ctypes.c_uint32() for _ in range(4)]
    n = ctypes.c_uint64()
    assert L.flk_wire_header_unpack(frame, len(frame), *[ctypes.byref(v) for v in vals],
                                    ctypes.byref(n)) == 0
    assert [v.value for v in vals] == [11, 6, 64, 1] and n.value == 6
    bad = b"XXXX" + frame[4:]
    assert L.flk_wire_header_unpack(bad, len(bad), None, None, None, None, None) == _lib.FLK_ERR_ARG
    assert b"not a flock frame" in L.flk_last_error()
    assert L.flk_wire_header_unpack(frame, 12, None, None, None, None, None) == _lib.FLK_ERR_ARG
