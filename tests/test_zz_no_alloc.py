"""flk_decode_layer_noalloc against flk_decode_layer, on the GPU, through the C ABI.

The no-allocation variant takes its split-K partials from the library's static
per-device scratch array instead of a caller workspace; it runs the same
kernels with the same plan, so its results must equal flk_decode_layer's bit
for bit. Two calls in a row, the second over fewer keys (the array keeps the
first call's partials, which the second must not pick up).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import randn
from parity import fmt, meets_bar, metrics

pytestmark = pytest.mark.gpu

from flock_amd import ops  # noqa: E402

H, HKV, D = 16, 8, 128
EPS = oracle.QWEN3_EPS


def dev(a):
    return ops.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


def test_noalloc_decode_layer_equals_workspace_call(rng):
    maxk = 32769
    kc0, vc0 = randn(rng, maxk * HKV * D), randn(rng, maxk * HKV * D)
    gq = rng.normal(1, 0.1, D).astype(np.float32)
    gk = rng.normal(1, 0.1, D).astype(np.float32)
    inv = dev(ops.rope_inv_freq(D, 1e6))
    gqd, gkd = dev(gq), dev(gk)
    # Two cache copies: one for each entry point.
    kc_a, vc_a, kc_b, vc_b = dev(kc0), dev(vc0), dev(kc0), dev(vc0)
    ws = ops.Workspace(H, HKV, D, maxk)
    for pos in (32768, 700):  # the second call reads fewer keys (fewer splits)
        print(f"noalloc decode: pos {pos}", flush=True)
        q, k, v = randn(rng, H * D), randn(rng, HKV * D), randn(rng, HKV * D)
        qd, kd, vd = dev(q), dev(k), dev(v)
        qn_a, o_a = ops.DeviceBuffer(H * D * 4), ops.DeviceBuffer(H * D * 4)
        qn_b, o_b = ops.DeviceBuffer(H * D * 4), ops.DeviceBuffer(H * D * 4)
        ops.decode_layer(qd, kd, vd, gqd, gkd, inv, EPS, "neox", qn_a, kc_a, vc_a, o_a, pos, H,
                         HKV, D, maxk, ws)
        ops.decode_layer_noalloc(qd, kd, vd, gqd, gkd, inv, EPS, "neox", qn_b, kc_b, vc_b, o_b,
                                 pos, H, HKV, D, maxk)
        ops.sync()
        want, got = o_a.download(H * D), o_b.download(H * D)
        assert np.array_equal(got, want), np.max(np.abs(got - want))
        assert np.array_equal(qn_b.download(H * D), qn_a.download(H * D))
        row = HKV * D
        for a, b in ((kc_a, kc_b), (vc_a, vc_b)):
            assert np.array_equal(b.download(row, offset_bytes=pos * row * 4),
                                  a.download(row, offset_bytes=pos * row * 4))
        # And both meet the parity bar against the oracle.
        kco, vco = kc0.copy(), vc0.copy()  # rows 0 .. pos - 1 are unchanged on the device
        _, want_o = oracle.layer_attn_decode(q, k, v, gq, gk, ops.rope_inv_freq(D, 1e6), kco,
                                             vco, pos, H, HKV, D)
        m = metrics(got, want_o)
        print(fmt(m))
        assert meets_bar(m), fmt(m)
