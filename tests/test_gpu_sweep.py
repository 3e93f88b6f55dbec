"""Seeded sweeps over the supported shape space, against the oracle, on the GPU.

The hand-picked cases of test_gpu_ops.py follow the reference's own test
shapes; these add shapes drawn at random (fixed seed, so every run sees the
same cases and each case's shape is in its test id): kv heads 1, 2, 3, 4, 5, 8
(and 16 in the wide-head cases), GQA groups 1..8, head_dim 64 and 128, key and query counts biased towards
the edges of the 64-key tiles and 4/32-key decode blocks, and positions that
do or do not start on a tile. Every case is held to the same bar as the
reference's tests (meets_bar: max-abs 2e-5 and relErr 1e-4, or no farther
from the float64 result than twice the oracle), the fused decode layer's
normed q and cache rows must match bit for bit, and each output row's argmax
must match wherever the oracle's top-2 margin exceeds four times the case's
largest error (closer rows are ties at f32 resolution).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import closed_form as cf
from conftest import randn
from parity import fmt, meets_bar, metrics

pytestmark = pytest.mark.gpu

from flock_amd import ops  # noqa: E402  (no skip: a missing library must fail)

EPS = oracle.QWEN3_EPS
KV_HEADS = (1, 2, 3, 4, 5, 8)
EDGE_KEYS = (1, 2, 3, 4, 5, 31, 32, 33, 63, 64, 65, 127, 128, 129)


def _edge_or_random(r: np.random.Generator, edges, hi: int) -> int:
    return int(r.choice(edges)) if r.random() < 0.5 else int(r.integers(1, hi + 1))


def _decode_cases(n: int, seed: int = 20261202):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        hkv = int(r.choice(KV_HEADS))
        g = int(r.integers(1, 9))
        d = int(r.choice((64, 128)))
        nk = _edge_or_random(r, EDGE_KEYS + (255, 256, 257, 4095, 4097), 20000)
        out.append((hkv * g, hkv, d, nk))
    return out


def _prefill_cases(n: int, seed: int = 20261203, max_flop: float = 8e8):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        hkv = int(r.choice(KV_HEADS))
        g = int(r.integers(1, 9))
        d = int(r.choice((64, 128)))
        nq = _edge_or_random(r, EDGE_KEYS, 200)
        pos0 = int(r.choice((0, 1, 63, 64, 65))) if r.random() < 0.5 else int(r.integers(0, 3001))
        if 4 * hkv * g * d * (nq * pos0 + nq * (nq + 1) // 2) > max_flop:
            continue
        out.append((hkv * g, hkv, d, nq, pos0))
    return out


def _layer_cases(n: int, seed: int = 20261204):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        hkv = int(r.choice(KV_HEADS))
        g = int(r.integers(1, 9))
        d = int(r.choice((64, 128)))
        pos = _edge_or_random(r, (0,) + EDGE_KEYS, 6000) - (0 if r.random() < 0.5 else 1)
        pos = max(pos, 0)
        maxk = pos + 1 + int(r.integers(0, 100))
        pairing = str(r.choice(("neox", "norm")))
        out.append((hkv * g, hkv, d, pos, maxk, pairing))
    return out


def _argmax_agrees(got, want, rows: int, err: float) -> tuple[bool, int]:
    g = np.asarray(got, np.float32).reshape(rows, -1)
    w = np.asarray(want, np.float32).reshape(rows, -1)
    s = np.sort(w, axis=1)
    clear = (s[:, -1] - s[:, -2]) > 4 * err
    return bool(np.all(np.argmax(g[clear], axis=1) == np.argmax(w[clear], axis=1))), int(np.sum(~clear))


def dev(a) -> "ops.DeviceBuffer":
    return ops.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


def empty(n: int) -> "ops.DeviceBuffer":
    return ops.DeviceBuffer(max(n, 1) * 4)


def get(b, n: int) -> np.ndarray:
    ops.sync()
    return b.download(n)


@pytest.mark.parametrize("H,Hkv,d,nk", _decode_cases(24))
def test_decode_shape_sweep(rng, H, Hkv, d, nk):
    q = randn(rng, H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    ws = ops.Workspace(H, Hkv, d, nk)
    o = empty(H * d)
    ops.attn_decode(dev(q), dev(k), dev(v), o, H, Hkv, d, nk, ws)
    got = get(o, H * d)
    want = oracle.attn(q, k, v, H, Hkv, d, nk)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, 1, nk - 1))
    assert meets_bar(m), fmt(m)
    ok, ties = _argmax_agrees(got, want, H, m["max_abs"])
    assert ok, (fmt(m), ties)


@pytest.mark.parametrize("H,Hkv,d,nq,pos0", _prefill_cases(20))
def test_prefill_shape_sweep(rng, H, Hkv, d, nq, pos0):
    nk = pos0 + nq
    q = randn(rng, nq * H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    ws = ops.Workspace(H, Hkv, d, nk, nq)
    o = empty(nq * H * d)
    ops.attn_prefill(dev(q), dev(k), dev(v), o, H, Hkv, d, nq, pos0, ws)
    got = get(o, nq * H * d)
    want = oracle.attn_prefill(q, k, v, H, Hkv, d, nq, pos0)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, nq, pos0))
    assert meets_bar(m), fmt(m)
    ok, ties = _argmax_agrees(got, want, nq * H, m["max_abs"])
    assert ok, (fmt(m), ties)


@pytest.mark.parametrize("H,Hkv,d,pos,maxk,pairing", _layer_cases(12))
def test_decode_layer_shape_sweep(rng, H, Hkv, d, pos, maxk, pairing):
    kc0, vc0 = randn(rng, maxk * Hkv * d), randn(rng, maxk * Hkv * d)
    q, k, v = randn(rng, H * d), randn(rng, Hkv * d), randn(rng, Hkv * d)
    gq = rng.normal(1, 0.1, d).astype(np.float32)
    gk = rng.normal(1, 0.1, d).astype(np.float32)
    inv = ops.rope_inv_freq(d, 1e6)
    kc, vc = dev(kc0), dev(vc0)
    qn, o = empty(H * d), empty(H * d)
    ws = ops.Workspace(H, Hkv, d, maxk)
    ops.decode_layer(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, pairing, qn, kc,
                     vc, o, pos, H, Hkv, d, maxk, ws)
    got_o, got_qn = get(o, H * d), qn.download(H * d)
    got_kc, got_vc = kc.download(maxk * Hkv * d), vc.download(maxk * Hkv * d)
    kco, vco = kc0.copy(), vc0.copy()
    want_qn, want_o = oracle.layer_attn_decode(q, k, v, gq, gk, inv, kco, vco, pos, H, Hkv, d,
                                               pairing=pairing)
    assert np.array_equal(got_qn, want_qn)
    assert np.array_equal(got_kc, kco) and np.array_equal(got_vc, vco)
    m = metrics(got_o, want_o, cf.attention(want_qn, kco, vco, H, Hkv, d, 1, pos))
    assert meets_bar(m), fmt(m)
    ok, ties = _argmax_agrees(got_o, want_o, H, m["max_abs"])
    assert ok, (fmt(m), ties)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_ragged_batch_sweep(seed):
    r = np.random.default_rng(100 + seed)
    hkv = int(r.choice(KV_HEADS))
    g = int(r.integers(1, 9))
    d = int(r.choice((64, 128)))
    H = hkv * g
    B = int(r.integers(1, 13))
    _ragged_vs_oracle(r, H, hkv, d, B)


def _ragged_vs_oracle(r: np.random.Generator, H: int, hkv: int, d: int, B: int) -> None:
    lens = np.array([_edge_or_random(r, (0,) + EDGE_KEYS, 5000) for _ in range(B)], np.uint32)
    gaps = r.integers(0, 5, B)
    offs = np.concatenate([[0], np.cumsum(lens + gaps)[:-1]]).astype(np.uint64)
    rows = max(int(offs[-1] + lens[-1] + gaps[-1]), 1)
    kc, vc = randn(r, rows * hkv * d), randn(r, rows * hkv * d)
    q = randn(r, B * H * d)
    max_len = max(int(lens.max()), 1)
    ws = ops.Workspace(H, hkv, d, max_len, 0, B)
    o = empty(B * H * d)
    ops.attn_decode_ragged(dev(q), dev(kc), dev(vc), ops.DeviceBuffer.from_array(offs),
                           ops.DeviceBuffer.from_array(lens), o, B, max_len, H, hkv, d, ws)
    got = get(o, B * H * d).reshape(B, H * d)
    row = hkv * d
    for b in range(B):
        if lens[b] == 0:
            assert np.all(got[b] == 0), b
            continue
        s = int(offs[b]) * row
        qb = q[b * H * d:(b + 1) * H * d]
        kb, vb = kc[s:s + int(lens[b]) * row], vc[s:s + int(lens[b]) * row]
        want = oracle.attn(qb, kb, vb, H, hkv, d, int(lens[b]))
        m = metrics(got[b], want, cf.attention(qb, kb, vb, H, hkv, d, 1, int(lens[b]) - 1))
        assert meets_bar(m), (b, int(lens[b]), fmt(m))


# 16 kv heads (two groups of 8 per workgroup: two item counters in a ragged
# batch, two grid columns in decode) and decode key counts up to 40000, which
# the draws above do not reach.
def _wide_decode_cases(n: int, seed: int = 20261205):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        g = int(r.integers(1, 6))
        d = int(r.choice((64, 128)))
        nk = _edge_or_random(r, (4097, 32769), 40000)
        out.append((16 * g, 16, d, nk))
    return out


@pytest.mark.parametrize("H,Hkv,d,nk", _wide_decode_cases(6))
def test_decode_wide_heads_sweep(rng, H, Hkv, d, nk):
    q = randn(rng, H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    ws = ops.Workspace(H, Hkv, d, nk)
    o = empty(H * d)
    ops.attn_decode(dev(q), dev(k), dev(v), o, H, Hkv, d, nk, ws)
    got = get(o, H * d)
    want = oracle.attn(q, k, v, H, Hkv, d, nk)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, 1, nk - 1))
    assert meets_bar(m), fmt(m)
    ok, ties = _argmax_agrees(got, want, H, m["max_abs"])
    assert ok, (fmt(m), ties)


@pytest.mark.parametrize("seed", [1, 2])
def test_ragged_wide_heads_sweep(seed):
    r = np.random.default_rng(200 + seed)
    g = int(r.integers(1, 5))
    d = int(r.choice((64, 128)))
    _ragged_vs_oracle(r, 16 * g, 16, d, int(r.integers(10, 31)))
