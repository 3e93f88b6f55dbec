"""The benchmark configurations at their full sizes, on the GPU, against the oracle.

decode at 32769 keys with the fused prologue (one layer of the 28-layer
config), causal prefill of 2048 tokens, a 64-token chunk onto a 32768-key
cache, and the 64-sequence ragged batch. Inputs are N(0, 1) (gains
N(1, 0.1)) like the benchmark's; each output is held to the parity bar
against the oracle and, where cheap, the float64 closed form.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import closed_form as cf
from conftest import randn
from parity import argmax_rows, fmt, meets_bar, metrics

pytestmark = pytest.mark.gpu

from flock_amd import ops  # noqa: E402

H, HKV, D = 16, 8, 128
EPS = oracle.QWEN3_EPS


def dev(a):
    return ops.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


def gains(rng):
    return rng.normal(1, 0.1, D).astype(np.float32), rng.normal(1, 0.1, D).astype(np.float32)


def test_decode_layer_at_32k(rng):
    # Config 2, one layer: norm + RoPE (theta 1e6) at position 32768, append,
    # attention over 32769 keys.
    pos = 32768
    maxk = pos + 1
    kc0, vc0 = randn(rng, maxk * HKV * D), randn(rng, maxk * HKV * D)
    q, k, v = randn(rng, H * D), randn(rng, HKV * D), randn(rng, HKV * D)
    gq, gk = gains(rng)
    inv = ops.rope_inv_freq(D, 1e6)
    kc, vc = dev(kc0), dev(vc0)
    qn, o = ops.DeviceBuffer(H * D * 4), ops.DeviceBuffer(H * D * 4)
    ws = ops.Workspace(H, HKV, D, maxk)
    ops.decode_layer(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, "neox", qn, kc, vc,
                     o, pos, H, HKV, D, maxk, ws)
    ops.sync()
    got_o, got_qn = o.download(H * D), qn.download(H * D)
    kco, vco = kc0.copy(), vc0.copy()
    want_qn, want_o = oracle.layer_attn_decode(q, k, v, gq, gk, inv, kco, vco, pos, H, HKV, D)
    assert np.array_equal(got_qn, want_qn)
    row = HKV * D
    assert np.array_equal(kc.download(row, offset_bytes=pos * row * 4), kco[pos * row:])
    assert np.array_equal(vc.download(row, offset_bytes=pos * row * 4), vco[pos * row:])
    m = metrics(got_o, want_o, cf.attention(want_qn, kco, vco, H, HKV, D, 1, pos))
    print(fmt(m))
    assert meets_bar(m), fmt(m)
    assert np.array_equal(argmax_rows(got_o, H), argmax_rows(want_o, H))


def _prefill_layer(rng, n, pos0):
    maxk = pos0 + n
    kc0 = np.zeros(maxk * HKV * D, np.float32)
    vc0 = np.zeros_like(kc0)
    kc0[:pos0 * HKV * D] = randn(rng, pos0 * HKV * D)
    vc0[:pos0 * HKV * D] = randn(rng, pos0 * HKV * D)
    q, k, v = randn(rng, n * H * D), randn(rng, n * HKV * D), randn(rng, n * HKV * D)
    gq, gk = gains(rng)
    inv = ops.rope_inv_freq(D, 1e6)
    kc, vc = dev(kc0), dev(vc0)
    qn, o = ops.DeviceBuffer(n * H * D * 4), ops.DeviceBuffer(n * H * D * 4)
    ops.qk_prologue(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, "neox", qn, kc, vc,
                    n, pos0, H, HKV, D, maxk)
    ws = ops.Workspace(H, HKV, D, maxk, n)
    ops.attn_prefill(qn, kc, vc, o, H, HKV, D, n, pos0, ws)
    ops.sync()
    got_o, got_qn = o.download(n * H * D), qn.download(n * H * D)
    got_kc = kc.download(maxk * HKV * D)
    kco, vco = kc0.copy(), vc0.copy()
    want_qn, want_o = oracle.layer_attn_prefill(q, k, v, gq, gk, inv, kco, vco, n, pos0, H, HKV, D)
    assert np.array_equal(got_qn, want_qn)
    assert np.array_equal(got_kc, kco)
    return got_o, want_o, want_qn, kco, vco


def test_prefill_2048_tokens(rng):
    # Config 4: a 2048-token prompt at position 0 (the paired, unsplit schedule).
    n = 2048
    got, want, qn, kc, vc = _prefill_layer(rng, n, 0)
    m = metrics(got, want, cf.attention(qn, kc, vc, H, HKV, D, n, 0))
    print(fmt(m))
    assert meets_bar(m), fmt(m)
    assert oracle.abs_err_scaled(got, want, oracle.amax(want)) < 1e-5  # test_head.ts:312-316


def test_chunk_onto_32k_cache(rng):
    # Config 5, one layer: a 64-token chunk at position 32768 (split keys +
    # merge), compared on every row.
    n, pos0 = 64, 32768
    got, want, qn, kc, vc = _prefill_layer(rng, n, pos0)
    m = metrics(got, want, cf.attention(qn, kc, vc, H, HKV, D, n, pos0))
    print(fmt(m))
    assert meets_bar(m), fmt(m)


def test_ragged_batch_of_64(rng):
    # Config 3: 64 sequences, n_keys ~ U[1025, 16385], one call. Every
    # sequence must match a single-sequence decode of its own rows (a
    # different split plan) to the parity bar, and a sample matches the oracle.
    B = 64
    lens = (rng.integers(1024, 16385, B) + 1).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(lens.astype(np.uint64))[:-1]]).astype(np.uint64)
    rows = int(lens.astype(np.uint64).sum())
    kc, vc = randn(rng, rows * HKV * D), randn(rng, rows * HKV * D)
    q = randn(rng, B * H * D)
    kcb, vcb = dev(kc), dev(vc)
    ws = ops.Workspace(H, HKV, D, int(lens.max()), 0, B)
    o = ops.DeviceBuffer(B * H * D * 4)
    ops.attn_decode_ragged(dev(q), kcb, vcb, ops.DeviceBuffer.from_array(offs),
                           ops.DeviceBuffer.from_array(lens), o, B, int(lens.max()), H, HKV, D, ws)
    ops.sync()
    got = o.download(B * H * D).reshape(B, H * D)
    row = HKV * D
    ws1 = ops.Workspace(H, HKV, D, int(lens.max()))
    o1 = ops.DeviceBuffer(H * D * 4)
    for b in range(B):
        s = int(offs[b]) * row
        n = int(lens[b])
        qb = dev(q[b * H * D:(b + 1) * H * D])
        kb, vb = dev(kc[s:s + n * row]), dev(vc[s:s + n * row])
        ops.attn_decode(qb, kb, vb, o1, H, HKV, D, n, ws1)
        ops.sync()
        single = o1.download(H * D)
        assert np.max(np.abs(single - got[b])) < 1e-5, b
        if b % 16 == 0:
            want = oracle.attn(q[b * H * D:(b + 1) * H * D], kc[s:s + n * row], vc[s:s + n * row],
                               H, HKV, D, n)
            m = metrics(got[b], want, cf.attention(q[b * H * D:(b + 1) * H * D], kc[s:s + n * row],
                                                   vc[s:s + n * row], H, HKV, D, 1, n - 1))
            assert meets_bar(m), (b, fmt(m))
