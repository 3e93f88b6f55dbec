"""Kernel-level parity on the GPU, through the C ABI, against the CPU oracle.

Mirrors the reference's kernel suites: test_ops.ts (rmsnorm, rope, decode
attention, GQA planted map) and test_head.ts:259-389 (prefill attention, last
query vs decode, causality). Shapes and tolerances follow those files; inputs
are seeded (uniform [-1, 1) like randVec for the reference's own cases, N(0, 1)
for the long-context cases), and each case also reports the distance of both
results from the float64 closed form.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import closed_form as cf
from conftest import rand_unit, randn
from parity import argmax_rows, fmt, meets_bar, metrics, top2_margin

pytestmark = pytest.mark.gpu

from flock_amd import ops  # noqa: E402  (no skip: a missing library must fail)

EPS = oracle.QWEN3_EPS


def dev(a) -> "ops.DeviceBuffer":
    return ops.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


def empty(n: int) -> "ops.DeviceBuffer":
    return ops.DeviceBuffer(max(n, 1) * 4)


def get(b, n: int) -> np.ndarray:
    ops.sync()
    return b.download(n)


# ------------------------------------------------------------------ rmsnorm --
@pytest.mark.parametrize("n,n_vecs", [(1024, 1), (128, 16), (128, 8), (1024, 4), (300, 3)])
def test_rmsnorm_bit_exact(rng, n, n_vecs):
    # test_ops.ts:100-135 (there: rel < 3e-7; here the oracle's rounding is
    # reproduced exactly, so the bar is bit equality).
    x, g = rand_unit(rng, n * n_vecs), rand_unit(rng, n, 0.5)
    o = empty(n * n_vecs)
    ops.rmsnorm(dev(x), dev(g), o, n, n_vecs, EPS)
    got = get(o, n * n_vecs)
    want = oracle.rmsnorm(x, g, n, n_vecs, EPS)
    assert np.array_equal(got, want), f"{np.sum(got != want)} differ, rel {oracle.rel_err(got, want)}"


def test_rmsnorm_deterministic_and_zero(rng):
    # test_ops.ts:137-181: 6 runs bit-identical; zero input gives exactly 0.
    n, nv = 128, 16
    x, g = dev(rand_unit(rng, n * nv)), dev(rand_unit(rng, n, 0.5))
    runs = []
    for _ in range(6):
        o = empty(n * nv)
        ops.rmsnorm(x, g, o, n, nv, EPS)
        runs.append(get(o, n * nv))
    assert all(np.array_equal(r, runs[0]) for r in runs)
    o = empty(n)
    ops.rmsnorm(dev(np.zeros(n, np.float32)), g, o, n, 1, EPS)
    z = get(o, n)
    assert np.all(z == 0)


# --------------------------------------------------------------------- rope --
@pytest.mark.parametrize("pairing", ["neox", "norm"])
@pytest.mark.parametrize("n_tokens,n_heads,pos0", [(1, 16, 0), (1, 16, 137), (1, 8, 137),
                                                   (7, 16, 0), (3, 8, 32768)])
def test_rope_matches_oracle(rng, pairing, n_tokens, n_heads, pos0):
    # test_ops.ts:189-227 (abs/scale < 4e-7); plus positions near 32k.
    d = 128
    inv = ops.rope_inv_freq(d, 1e6)
    assert np.array_equal(inv, oracle.rope_inv_freq(d, 1e6))
    x = rand_unit(rng, n_tokens * n_heads * d)
    xb = dev(x)
    ops.rope(xb, dev(inv), n_tokens, n_heads, d, pos0, pairing)
    got = get(xb, x.size)
    want = oracle.rope(x, n_tokens, n_heads, d, pos0, inv, pairing)
    e = oracle.abs_err_scaled(got, want, oracle.amax(x))
    assert e < 4e-7
    assert np.sum(got != want) == 0, f"{np.sum(got != want)} of {x.size} not bit-identical"


@pytest.mark.parametrize("pairing", ["neox", "norm"])
def test_rope_planted_pair(pairing):
    # test_ops.ts:229-263.
    d = 128
    inv = ops.rope_inv_freq(d, 1e6)
    x = np.zeros(d, np.float32)
    x[0] = 1
    xb = dev(x)
    ops.rope(xb, dev(inv), 1, 1, d, 1, pairing)
    got = get(xb, d)
    partner, other = (1, 64) if pairing == "norm" else (64, 1)
    assert abs(got[0] - np.cos(inv[0])) < 1e-6 and abs(got[partner] - np.sin(inv[0])) < 1e-6
    assert got[other] == 0


# ----------------------------------------------------------------- prologue --
@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("pairing", ["neox", "norm"])
@pytest.mark.parametrize("n,pos0", [(1, 0), (5, 40), (33, 900), (2, 32767)])
def test_prologue_bit_exact(rng, d, pairing, n, pos0):
    # layer.ts:598-622 / 722-741 fused: qn and the appended cache rows equal the
    # oracle's rmsnorm -> rope -> append bit for bit, and equal the unfused
    # flk_rmsnorm + flk_rope + flk_kv_append path.
    H, Hkv = 16, 8
    maxk = pos0 + n + 3
    q, k, v = randn(rng, n * H * d), randn(rng, n * Hkv * d), randn(rng, n * Hkv * d)
    gq = rng.normal(1, 0.1, d).astype(np.float32)
    gk = rng.normal(1, 0.1, d).astype(np.float32)
    inv = ops.rope_inv_freq(d, 1e6)
    kc, vc, qn = empty(maxk * Hkv * d), empty(maxk * Hkv * d), empty(n * H * d)
    ops.qk_prologue(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, pairing, qn, kc, vc,
                    n, pos0, H, Hkv, d, maxk)
    row = Hkv * d
    got_q = get(qn, n * H * d)
    got_k = kc.download(maxk * row)[pos0 * row:(pos0 + n) * row]
    got_v = vc.download(maxk * row)[pos0 * row:(pos0 + n) * row]
    want_q = oracle.rope(oracle.rmsnorm(q, gq, d, n * H, EPS), n, H, d, pos0, inv, pairing)
    want_k = oracle.rope(oracle.rmsnorm(k, gk, d, n * Hkv, EPS), n, Hkv, d, pos0, inv, pairing)
    assert np.array_equal(got_q, want_q), f"q: {np.sum(got_q != want_q)} differ"
    assert np.array_equal(got_k, want_k), f"k: {np.sum(got_k != want_k)} differ"
    assert np.array_equal(got_v, v)
    # Unfused path.
    qb, kb = empty(n * H * d), empty(n * Hkv * d)
    ops.rmsnorm(dev(q), dev(gq), qb, d, n * H, EPS)
    ops.rmsnorm(dev(k), dev(gk), kb, d, n * Hkv, EPS)
    ops.rope(qb, dev(inv), n, H, d, pos0, pairing)
    ops.rope(kb, dev(inv), n, Hkv, d, pos0, pairing)
    kc2, vc2 = empty(maxk * Hkv * d), empty(maxk * Hkv * d)
    ops.kv_append(kb, dev(v), kc2, vc2, n, pos0, Hkv, d, maxk)
    assert np.array_equal(get(qb, n * H * d), got_q)
    assert np.array_equal(kc2.download(maxk * row)[pos0 * row:(pos0 + n) * row], got_k)
    # The same rows read out of one [n][q | k | v] buffer (a stacked
    # projection's output) by the strided entry point.
    wide = (H + 2 * Hkv) * d
    qkv = np.concatenate([q.reshape(n, H * d), k.reshape(n, Hkv * d), v.reshape(n, Hkv * d)],
                         axis=1).ravel()
    qkvb = dev(qkv)
    kc3, vc3, qn3 = empty(maxk * Hkv * d), empty(maxk * Hkv * d), empty(n * H * d)
    ops.qk_prologue(qkvb.ptr, qkvb.ptr + H * d * 4, qkvb.ptr + (H + Hkv) * d * 4, dev(gq), dev(gk),
                    dev(inv), EPS, pairing, qn3, kc3, vc3, n, pos0, H, Hkv, d, maxk,
                    in_stride=wide)
    assert np.array_equal(get(qn3, n * H * d), got_q)
    assert np.array_equal(kc3.download(maxk * row)[pos0 * row:(pos0 + n) * row], got_k)
    assert np.array_equal(vc3.download(maxk * row)[pos0 * row:(pos0 + n) * row], got_v)


# ------------------------------------------------------------------- decode --
def _decode(q, k, v, H, Hkv, d, nk):
    ws = ops.Workspace(H, Hkv, d, nk)
    o = empty(H * d)
    ops.attn_decode(dev(q), dev(k), dev(v), o, H, Hkv, d, nk, ws)
    return get(o, H * d)


@pytest.mark.parametrize("H,Hkv,nk", [(16, 8, 1), (16, 8, 137), (16, 8, 512), (16, 16, 64),
                                      (4, 1, 33)])
def test_decode_reference_cases(rng, H, Hkv, nk):
    # test_ops.ts:316-355: relErr(floor 1e-3) < 1e-4 on randVec inputs.
    d = 128
    q = rand_unit(rng, H * d)
    k, v = rand_unit(rng, nk * Hkv * d), rand_unit(rng, nk * Hkv * d)
    got = _decode(q, k, v, H, Hkv, d, nk)
    want = oracle.attn(q, k, v, H, Hkv, d, nk)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, 1, nk - 1))
    print(fmt(m))
    assert m["rel"] < 1e-4 and m["max_abs"] < 2e-5
    assert np.array_equal(argmax_rows(got, H), argmax_rows(want, H))


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("nk", [1, 2, 63, 64, 65, 513, 2049, 32769])
def test_decode_parity_bar_long_context(rng, d, nk):
    # N(0,1) inputs (the long-context configs' distribution), split-K in play
    # from a few hundred keys on.
    H, Hkv = 16, 8
    q = randn(rng, H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    got = _decode(q, k, v, H, Hkv, d, nk)
    want = oracle.attn(q, k, v, H, Hkv, d, nk)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, 1, nk - 1))
    print(fmt(m))
    assert meets_bar(m), fmt(m)
    assert np.array_equal(argmax_rows(got, H), argmax_rows(want, H)), top2_margin(want, H)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("H,Hkv,nk", [(12, 4, 700), (24, 4, 1500), (16, 2, 2049), (8, 1, 513),
                                      (32, 4, 300), (6, 2, 4097), (10, 2, 777), (14, 2, 1000),
                                      (7, 1, 3000)])
def test_decode_group_sizes(rng, d, H, Hkv, nk):
    # GQA groups 3, 6, 8, 5 and 7, with one kv head per workgroup (KH = 1, 2,
    # 4): the template cases Qwen3's 16 / 8 layout never reaches, with key
    # splits.
    q = randn(rng, H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    got = _decode(q, k, v, H, Hkv, d, nk)
    want = oracle.attn(q, k, v, H, Hkv, d, nk)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, 1, nk - 1))
    print(fmt(m))
    assert meets_bar(m), fmt(m)
    assert np.array_equal(argmax_rows(got, H), argmax_rows(want, H)), top2_margin(want, H)


def test_decode_gqa_planted_kat():
    # test_ops.ts:357-392: heads 0,1 read kv head 0 (all 7), heads 2,3 read kv
    # head 1 (all -3), exactly.
    d = 128
    v = np.concatenate([np.full(d, 7, np.float32), np.full(d, -3, np.float32)])
    got = _decode(np.zeros(4 * d, np.float32), np.zeros(2 * d, np.float32), v, 4, 2, d, 1)
    got = got.reshape(4, d)
    assert np.all(got[:2] == 7) and np.all(got[2:] == -3)


def test_decode_deterministic_across_runs(rng):
    # The race check of test_ops.ts:137-165 applied to split-K decode: the
    # cross-split merge order is fixed, so repeated runs are bit-identical.
    H, Hkv, d, nk = 16, 8, 128, 20000
    q, k, v = dev(randn(rng, H * d)), dev(randn(rng, nk * Hkv * d)), dev(randn(rng, nk * Hkv * d))
    ws = ops.Workspace(H, Hkv, d, nk)
    outs = []
    for _ in range(6):
        o = empty(H * d)
        ops.attn_decode(q, k, v, o, H, Hkv, d, nk, ws)
        outs.append(get(o, H * d))
    assert all(np.array_equal(x, outs[0]) for x in outs)


@pytest.mark.parametrize("H,Hkv", [(16, 8), (12, 4), (8, 1)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("pairing", ["neox", "norm"])
def test_decode_layer_fused_matches_oracle(rng, H, Hkv, d, pairing):
    # Layer.encode's attention slice in one launch (layer.ts:571-630) vs the
    # oracle's layerForwardRef slice (layer_ref.ts:46-70). The in-kernel
    # prologue has a d = 64 branch (partner lane xor 32), the norm pairing,
    # and workgroups holding 8, 4 or 1 kv heads with GQA groups of 2, 3, 8.
    pos = 700
    maxk = 1024
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
    assert np.array_equal(argmax_rows(got_o, H), argmax_rows(want_o, H)), top2_margin(want_o, H)


@pytest.mark.parametrize("n_keys_dev", [0, 1025, 5000])
def test_decode_layer_dev_rejects_a_bad_position_on_the_device(rng, n_keys_dev):
    # flk_decode_layer_dev reads the key count from device memory, where no
    # host guard sees it. Past max_keys (the reference's "KV cache full",
    # layer.ts:575) or 0, the kernel appends nothing, leaves qn as it was and
    # fills o with NaN; the cache is unchanged.
    H, Hkv, d, maxk = 16, 8, 128, 1024
    kc0, vc0 = randn(rng, maxk * Hkv * d), randn(rng, maxk * Hkv * d)
    q, k, v = randn(rng, H * d), randn(rng, Hkv * d), randn(rng, Hkv * d)
    gq = rng.normal(1, 0.1, d).astype(np.float32)
    gk = rng.normal(1, 0.1, d).astype(np.float32)
    inv = ops.rope_inv_freq(d, 1e6)
    kc, vc = dev(kc0), dev(vc0)
    qn0 = np.full(H * d, 5.0, np.float32)
    qn, o = dev(qn0), empty(H * d)
    nk = ops.DeviceBuffer.from_array(np.array([n_keys_dev], np.uint32))
    ws = ops.Workspace(H, Hkv, d, maxk)
    ops.decode_layer_dev(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, "neox", qn, kc,
                         vc, o, nk, H, Hkv, d, maxk, ws)
    ops.sync()
    assert np.isnan(get(o, H * d)).all()
    assert np.array_equal(qn.download(H * d), qn0)
    assert np.array_equal(kc.download(maxk * Hkv * d), kc0)
    assert np.array_equal(vc.download(maxk * Hkv * d), vc0)
    # A valid count right after runs normally (nothing stuck from the bad call).
    nk.upload(np.array([maxk], np.uint32))
    ops.decode_layer_dev(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, "neox", qn, kc,
                         vc, o, nk, H, Hkv, d, maxk, ws)
    got_o = get(o, H * d)
    kco, vco = kc0.copy(), vc0.copy()
    _, want_o = oracle.layer_attn_decode(q, k, v, gq, gk, inv, kco, vco, maxk - 1, H, Hkv, d)
    assert np.array_equal(kc.download(maxk * Hkv * d), kco)
    m = metrics(got_o, want_o)
    assert meets_bar(m), fmt(m)


@pytest.mark.parametrize("pos", [0, 1, 5, 700, 5000])
def test_decode_layer_ignores_the_row_being_appended(rng, pos):
    # The row at pos is written by one workgroup of the same launch; before
    # that it may hold anything (here NaN). Workgroups whose last block runs
    # past the end re-read that row; its contents must never reach the output.
    H, Hkv, d = 16, 8, 128
    maxk = pos + 1
    kc0, vc0 = randn(rng, maxk * Hkv * d), randn(rng, maxk * Hkv * d)
    row = Hkv * d
    kc0[pos * row:] = np.nan
    vc0[pos * row:] = np.nan
    q, k, v = randn(rng, H * d), randn(rng, Hkv * d), randn(rng, Hkv * d)
    gq = rng.normal(1, 0.1, d).astype(np.float32)
    gk = rng.normal(1, 0.1, d).astype(np.float32)
    inv = ops.rope_inv_freq(d, 1e6)
    kc, vc = dev(kc0), dev(vc0)
    qn, o = empty(H * d), empty(H * d)
    ws = ops.Workspace(H, Hkv, d, maxk)
    ops.decode_layer(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, "neox", qn, kc, vc,
                     o, pos, H, Hkv, d, maxk, ws)
    got_o = get(o, H * d)
    kco, vco = kc0.copy(), vc0.copy()
    want_qn, want_o = oracle.layer_attn_decode(q, k, v, gq, gk, inv, kco, vco, pos, H, Hkv, d)
    assert not np.isnan(got_o).any()
    m = metrics(got_o, want_o, cf.attention(want_qn, kco, vco, H, Hkv, d, 1, pos))
    assert meets_bar(m), fmt(m)


# ------------------------------------------------------------------ prefill --
def _prefill(q, k, v, H, Hkv, d, nq, pos0):
    ws = ops.Workspace(H, Hkv, d, pos0 + nq, nq)
    o = empty(nq * H * d)
    ops.attn_prefill(dev(q), dev(k), dev(v), o, H, Hkv, d, nq, pos0, ws)
    return get(o, nq * H * d)


PREFILL_CASES = [
    # test_head.ts:290-304
    (16, 8, 1, 0), (16, 8, 7, 0), (16, 8, 13, 0), (16, 8, 64, 0), (16, 8, 65, 0),
    (16, 8, 129, 0), (16, 8, 5, 40), (16, 8, 20, 300), (16, 16, 9, 0), (4, 1, 11, 0),
    (16, 8, 3, 2100),
]


@pytest.mark.parametrize("H,Hkv,nq,pos0", PREFILL_CASES)
def test_prefill_reference_cases(rng, H, Hkv, nq, pos0):
    # abs/scale < 1e-5 against attnPrefillRef (test_head.ts:306-318), and the
    # north-star bar.
    d = 128
    nk = pos0 + nq
    q = rand_unit(rng, nq * H * d)
    k, v = rand_unit(rng, nk * Hkv * d), rand_unit(rng, nk * Hkv * d)
    got = _prefill(q, k, v, H, Hkv, d, nq, pos0)
    want = oracle.attn_prefill(q, k, v, H, Hkv, d, nq, pos0)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, nq, pos0))
    print(fmt(m))
    assert m["abs_scaled"] < 1e-5
    assert meets_bar(m), fmt(m)
    assert np.array_equal(argmax_rows(got, nq * H), argmax_rows(want, nq * H))


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("H,Hkv,nq,pos0", [(16, 8, 200, 0), (16, 8, 64, 4000), (12, 4, 50, 77),
                                           (16, 2, 33, 10), (8, 8, 130, 3)])
def test_prefill_split_and_shapes(rng, d, H, Hkv, nq, pos0):
    # Long caches exercise the key-split + merge; odd groups exercise the
    # row -> (query, head) map (group 3 leaves rows 126, 127 of a tile unused).
    nk = pos0 + nq
    q = randn(rng, nq * H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    got = _prefill(q, k, v, H, Hkv, d, nq, pos0)
    want = oracle.attn_prefill(q, k, v, H, Hkv, d, nq, pos0)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, nq, pos0))
    print(fmt(m))
    assert meets_bar(m), fmt(m)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("H,Hkv,nq,pos0", [
    (10, 2, 40, 3000), (12, 2, 45, 700), (14, 2, 30, 5000),  # split plans
    (40, 8, 600, 0), (48, 8, 600, 0), (56, 8, 600, 0),        # paired plans
])
def test_prefill_groups_5_6_7(rng, d, H, Hkv, nq, pos0):
    # 64 rows / G is 12, 10 and 9 queries: the last 4, 4 and 1 rows of every
    # q tile have no query; the paired cases have >= 192 balanced pairs.
    nk = pos0 + nq
    q = randn(rng, nq * H * d)
    k, v = randn(rng, nk * Hkv * d), randn(rng, nk * Hkv * d)
    got = _prefill(q, k, v, H, Hkv, d, nq, pos0)
    want = oracle.attn_prefill(q, k, v, H, Hkv, d, nq, pos0)
    m = metrics(got, want, cf.attention(q, k, v, H, Hkv, d, nq, pos0))
    print(fmt(m))
    assert meets_bar(m), fmt(m)


def test_prefill_queries_match_decode(rng):
    # test_head.ts:321-351: prefill query `at` equals the decode reference over
    # keys 0..at -- proves the causal bound is pos0 + qi + 1.
    H, Hkv, d, nq = 16, 8, 128, 9
    q = rand_unit(rng, nq * H * d)
    k, v = rand_unit(rng, nq * Hkv * d), rand_unit(rng, nq * Hkv * d)
    pre = _prefill(q, k, v, H, Hkv, d, nq, 0).reshape(nq, H * d)
    for at in (0, 1, 4, nq - 1):
        want = oracle.attn(q.reshape(nq, -1)[at], k[:(at + 1) * Hkv * d], v[:(at + 1) * Hkv * d],
                           H, Hkv, d, at + 1)
        assert oracle.abs_err_scaled(pre[at], want, oracle.amax(want)) < 2e-5


def test_prefill_causality_bit_identical(rng):
    # test_head.ts:353-389.
    H, Hkv, d, nq = 16, 8, 128, 8
    q = rand_unit(rng, nq * H * d)
    k, v = rand_unit(rng, nq * Hkv * d), rand_unit(rng, nq * Hkv * d)
    base = _prefill(q, k, v, H, Hkv, d, nq, 0).reshape(nq, -1)
    k2, v2 = k.copy(), v.copy()
    idx = np.arange(Hkv * d)
    k2[5 * Hkv * d + idx] = 9 + idx * 0.01
    v2[5 * Hkv * d + idx] = -7 - idx * 0.01
    pert = _prefill(q, k2, v2, H, Hkv, d, nq, 0).reshape(nq, -1)
    assert np.array_equal(base[:5], pert[:5])
    assert np.sum(base[5:] != pert[5:]) > H * d


# Causality on longer calls: several q tiles, and a chunk whose keys are
# split over workgroups and merged (a long cache).
@pytest.mark.parametrize("nq,pos0,at", [(200, 0, 150), (64, 5000, 30), (300, 40, 7),
                                         (8192, 0, 5000)])
def test_prefill_causality_bit_identical_long(rng, nq, pos0, at):
    H, Hkv, d = 16, 8, 128
    nk = pos0 + nq
    q = rand_unit(rng, nq * H * d)
    k, v = rand_unit(rng, nk * Hkv * d), rand_unit(rng, nk * Hkv * d)
    base = _prefill(q, k, v, H, Hkv, d, nq, pos0).reshape(nq, -1)
    k2, v2 = k.copy(), v.copy()
    idx = np.arange(Hkv * d)
    key = pos0 + at
    k2[key * Hkv * d + idx] = 9 + idx * 0.01
    v2[key * Hkv * d + idx] = -7 - idx * 0.01
    pert = _prefill(q, k2, v2, H, Hkv, d, nq, pos0).reshape(nq, -1)
    assert np.array_equal(base[:at], pert[:at])
    assert np.sum(base[at:] != pert[at:]) > H * d


def test_prefill_queries_match_decode_across_tiles(rng):
    # test_head.ts:321-351 over several q tiles: query `at` equals the decode
    # reference over keys 0 .. at.
    H, Hkv, d, nq = 16, 8, 128, 193
    q = rand_unit(rng, nq * H * d)
    k, v = rand_unit(rng, nq * Hkv * d), rand_unit(rng, nq * Hkv * d)
    pre = _prefill(q, k, v, H, Hkv, d, nq, 0).reshape(nq, H * d)
    for at in (0, 63, 64, 127, 128, 191, 192):
        want = oracle.attn(q.reshape(nq, -1)[at], k[:(at + 1) * Hkv * d], v[:(at + 1) * Hkv * d],
                           H, Hkv, d, at + 1)
        assert oracle.abs_err_scaled(pre[at], want, oracle.amax(want)) < 2e-5


def test_prefill_deterministic_across_runs(rng):
    H, Hkv, d, nq, pos0 = 16, 8, 128, 64, 5000
    nk = pos0 + nq
    q, k, v = dev(randn(rng, nq * H * d)), dev(randn(rng, nk * Hkv * d)), dev(randn(rng, nk * Hkv * d))
    ws = ops.Workspace(H, Hkv, d, nk, nq)
    outs = []
    for _ in range(6):
        o = empty(nq * H * d)
        ops.attn_prefill(q, k, v, o, H, Hkv, d, nq, pos0, ws)
        outs.append(get(o, nq * H * d))
    assert all(np.array_equal(x, outs[0]) for x in outs)


# ------------------------------------------------------------------- ragged --
def _ragged_vs_oracle(rng, H, Hkv, d, lens):
    lens = np.asarray(lens, np.uint32)
    B = len(lens)
    offs = np.concatenate([[0], np.cumsum(lens + 3)[:-1]]).astype(np.uint64)  # gaps between seqs
    rows = int(offs[-1] + lens[-1] + 3)
    kc, vc = randn(rng, rows * Hkv * d), randn(rng, rows * Hkv * d)
    q = randn(rng, B * H * d)
    ws = ops.Workspace(H, Hkv, d, int(lens.max()), 0, B)
    o = empty(B * H * d)
    ops.attn_decode_ragged(dev(q), dev(kc), dev(vc), ops.DeviceBuffer.from_array(offs),
                           ops.DeviceBuffer.from_array(lens), o, B, int(lens.max()), H, Hkv, d, ws)
    got = get(o, B * H * d).reshape(B, H * d)
    row = Hkv * d
    for b in range(B):
        if lens[b] == 0:
            assert np.all(got[b] == 0), b
            continue
        s = int(offs[b]) * row
        qb = q[b * H * d:(b + 1) * H * d]
        kb, vb = kc[s:s + int(lens[b]) * row], vc[s:s + int(lens[b]) * row]
        want = oracle.attn(qb, kb, vb, H, Hkv, d, int(lens[b]))
        m = metrics(got[b], want, cf.attention(qb, kb, vb, H, Hkv, d, 1, int(lens[b]) - 1))
        assert meets_bar(m), (b, int(lens[b]), fmt(m))


# Every kv-heads-per-workgroup instance (8, 4, 2, 1), groups on both sides of
# 4 (the batched instance keeps 4 keys per slot in flight up to G = 4, 2
# above), both head sizes. Lengths sit at and around the instance's block of
# keys per iteration: 512 / (d / 4) slots / KH kv heads x keys per slot.
@pytest.mark.parametrize("H,Hkv,d", [(16, 8, 128), (16, 8, 64), (32, 8, 128), (64, 8, 64),
                                     (4, 4, 128), (12, 4, 64), (10, 2, 128), (8, 1, 128),
                                     (5, 1, 64), (15, 5, 128)])
def test_decode_ragged_head_layouts(rng, H, Hkv, d):
    G = H // Hkv
    kh = next(k for k in (8, 4, 2, 1) if Hkv % k == 0)
    kpi = (512 // (d // 4)) // kh * (4 if G <= 4 else 2)
    _ragged_vs_oracle(rng, H, Hkv, d, [1, kpi - 1, kpi, kpi + 1, 2 * kpi + 3, 0, 1500])


def test_decode_ragged_matches_per_sequence_oracle(rng):
    # Extension (no reference counterpart): independent sequences, one launch.
    _ragged_vs_oracle(rng, 16, 8, 128, [1, 5, 64, 65, 300, 1000, 2500, 0, 777])


# Batches of up to 2048 sequences run on the persistent kernel (its tables
# live in LDS); bigger ones on one workgroup per split. Both sides of the
# boundary, with empty and one-key sequences among them.
@pytest.mark.parametrize("n_seqs", [2048, 2100])
def test_decode_ragged_many_sequences(rng, n_seqs):
    lens = rng.integers(0, 41, n_seqs).astype(np.uint32)
    lens[:3] = [0, 1, 40]
    _ragged_vs_oracle(rng, 16, 8, 128, lens)


def test_decode_ragged_graph_replay(rng):
    # A captured ragged call replays its item-counter reset (a kernel, not a
    # memset), so every replay gives the eager call's bits; eager calls in
    # between leave the counters anywhere.
    H, Hkv, d = 16, 8, 128
    lens = np.array([2500, 0, 900, 4097, 1], np.uint32)
    B = len(lens)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    rows = int(lens.sum())
    kc, vc, q = dev(randn(rng, rows * Hkv * d)), dev(randn(rng, rows * Hkv * d)), dev(randn(rng, B * H * d))
    offs_d, lens_d = ops.DeviceBuffer.from_array(offs), ops.DeviceBuffer.from_array(lens)
    maxn = int(lens.max())
    ws = ops.Workspace(H, Hkv, d, maxn, 0, B)
    o = empty(B * H * d)
    call = lambda: ops.attn_decode_ragged(q, kc, vc, offs_d, lens_d, o, B, maxn, H, Hkv, d, ws)
    st = ops.Stream()
    ops.set_stream(st)
    try:
        call()
        ops.sync()
        eager = get(o, B * H * d)
        with ops.Graph() as g:
            call()
        for i in range(3):
            o.zero()  # eager, between replays
            g.launch()
            ops.sync()
            assert np.array_equal(get(o, B * H * d), eager), i
            call()  # an eager call between replays
            ops.sync()
        g.free()
    finally:
        ops.set_stream(None)
        st.free()


def test_decode_ragged_repeats_bit_for_bit(rng):
    # The batch's (sequence, split) items are claimed by whichever workgroup
    # is free; every item still writes its own partial, so repeated calls on
    # one workspace (whose item counters each call resets) agree bit for bit,
    # also after the workspace has served a prefill in between.
    H, Hkv, d = 16, 8, 128
    lens = np.array([3000, 1, 0, 4097, 700, 2048, 33, 1500], np.uint32)
    B = len(lens)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    rows = int(lens.sum())
    kc, vc, q = dev(randn(rng, rows * Hkv * d)), dev(randn(rng, rows * Hkv * d)), dev(randn(rng, B * H * d))
    offs_d, lens_d = ops.DeviceBuffer.from_array(offs), ops.DeviceBuffer.from_array(lens)
    maxn = int(lens.max())
    ws = ops.Workspace(H, Hkv, d, maxn, 64, B)
    o = empty(B * H * d)
    outs = []
    for i in range(5):
        if i == 3:  # the workspace serves a 64-query prefill in between
            pq, po = dev(randn(rng, 64 * H * d)), empty(64 * H * d)
            ops.attn_prefill(pq, kc, vc, po, H, Hkv, d, 64, 2000, ws)
        ops.attn_decode_ragged(q, kc, vc, offs_d, lens_d, o, B, maxn, H, Hkv, d, ws)
        outs.append(get(o, B * H * d))
    assert all(np.array_equal(x, outs[0]) for x in outs[1:])


# Past the bound: flk_attn_decode_ragged clamps n_keys[b] > max_n_keys, so such
# a sequence attends its first max_n_keys rows. Both sides of the persistent
# kernel's 2048-sequence limit.
@pytest.mark.parametrize("n_seqs", [40, 2100])
def test_decode_ragged_clamps_counts_past_the_bound(rng, n_seqs):
    H, Hkv, d = 16, 8, 128
    maxn = 300
    lens = rng.integers(1, maxn + 1, n_seqs).astype(np.uint32)
    over = [1, n_seqs // 2, n_seqs - 1]
    lens[over] = [maxn + 1, maxn + 57, 4 * maxn]
    offs = (np.arange(n_seqs, dtype=np.uint64) * np.uint64(4 * maxn + 2))
    rows = int(offs[-1]) + 4 * maxn + 2
    kc, vc = randn(rng, rows * Hkv * d), randn(rng, rows * Hkv * d)
    q = randn(rng, n_seqs * H * d)
    ws = ops.Workspace(H, Hkv, d, maxn, 0, n_seqs)
    o = empty(n_seqs * H * d)
    ops.attn_decode_ragged(dev(q), dev(kc), dev(vc), ops.DeviceBuffer.from_array(offs),
                           ops.DeviceBuffer.from_array(lens), o, n_seqs, maxn, H, Hkv, d, ws)
    got = get(o, n_seqs * H * d).reshape(n_seqs, H * d)
    row = Hkv * d
    for b in over + [0, 2]:
        n = min(int(lens[b]), maxn)
        s = int(offs[b]) * row
        qb = q[b * H * d:(b + 1) * H * d]
        want = oracle.attn(qb, kc[s:s + n * row], vc[s:s + n * row], H, Hkv, d, n)
        m = metrics(got[b], want, cf.attention(qb, kc[s:s + n * row], vc[s:s + n * row], H, Hkv,
                                               d, 1, n - 1))
        assert meets_bar(m), (b, int(lens[b]), fmt(m))


# ------------------------------------------------------- ragged layer step --
def _ragged_layer_vs_oracle(rng, H, Hkv, d, lens, pairing="neox", max_n_keys=None):
    """flk_decode_layer_ragged against oracle.layer_attn_decode per sequence
    (layer_ref.ts:46-70 at position n_keys[b] - 1 of that sequence's rows):
    qn and every cache row bit-identical, o to the parity bar; idle
    sequences (0 keys) give zero rows and refused ones (past max_n_keys) NaN
    rows, and neither writes to the caches."""
    lens = np.asarray(lens, np.uint32)
    B = len(lens)
    maxn = int(lens.max()) if max_n_keys is None else int(max_n_keys)
    span = np.minimum(lens.astype(np.int64), maxn) + 3  # rows per sequence, gaps between
    offs = np.concatenate([[0], np.cumsum(span)[:-1]]).astype(np.uint64)
    rows = int(offs[-1]) + int(span[-1])
    row = Hkv * d
    kc0, vc0 = randn(rng, rows * row), randn(rng, rows * row)
    q, k, v = randn(rng, B * H * d), randn(rng, B * row), randn(rng, B * row)
    gq, gk = rng.normal(1, 0.1, d).astype(np.float32), rng.normal(1, 0.1, d).astype(np.float32)
    inv = oracle.rope_inv_freq(d, 1e6)
    kc, vc = dev(kc0), dev(vc0)
    qn, o = empty(B * H * d), empty(B * H * d)
    ws = ops.Workspace(H, Hkv, d, maxn, 0, B)
    ops.decode_layer_ragged(dev(q), dev(k), dev(v), dev(gq), dev(gk), dev(inv), EPS, pairing, qn,
                            kc, vc, ops.DeviceBuffer.from_array(offs),
                            ops.DeviceBuffer.from_array(lens), o, B, maxn, H, Hkv, d, ws)
    got_o = get(o, B * H * d).reshape(B, H * d)
    got_qn = qn.download(B * H * d).reshape(B, H * d)
    got_kc, got_vc = kc.download(rows * row), vc.download(rows * row)
    kco, vco = kc0.copy(), vc0.copy()
    for b in range(B):
        n = int(lens[b])
        if n == 0:
            assert np.all(got_o[b] == 0) and np.all(got_qn[b] == 0), b
            continue
        if n > maxn:
            assert np.all(np.isnan(got_o[b])) and np.all(np.isnan(got_qn[b])), b
            continue
        s = int(offs[b]) * row
        kb, vb = kco[s:s + n * row], vco[s:s + n * row]  # views: the oracle appends in place
        hq, hk = slice(b * H * d, (b + 1) * H * d), slice(b * row, (b + 1) * row)
        want_qn, want_o = oracle.layer_attn_decode(q[hq], k[hk], v[hk], gq, gk, inv, kb, vb,
                                                   n - 1, H, Hkv, d, EPS, pairing)
        assert np.array_equal(got_qn[b], want_qn), b
        m = metrics(got_o[b], want_o, cf.attention(want_qn, kb, vb, H, Hkv, d, 1, n - 1))
        assert meets_bar(m), (b, n, fmt(m))
    assert np.array_equal(got_kc, kco)
    assert np.array_equal(got_vc, vco)


@pytest.mark.parametrize("H,Hkv,d", [(16, 8, 128), (16, 8, 64), (12, 4, 64), (10, 2, 128),
                                     (8, 1, 128), (32, 8, 128)])
def test_decode_layer_ragged_head_layouts(rng, H, Hkv, d):
    G = H // Hkv
    kh = next(k for k in (8, 4, 2, 1) if Hkv % k == 0)
    kpi = (512 // (d // 4)) // kh * (4 if G <= 4 else 2)
    _ragged_layer_vs_oracle(rng, H, Hkv, d, [1, kpi - 1, kpi, kpi + 1, 2 * kpi + 3, 0, 1500, 2])


@pytest.mark.parametrize("pairing", ["neox", "norm"])
def test_decode_layer_ragged_positions_past_32k(rng, pairing):
    # RoPE at large positions (the reference's theta 1e6 at 32768+), one
    # sequence on each side of a block edge.
    _ragged_layer_vs_oracle(rng, 16, 8, 128, [32769, 33000, 5], pairing)


def test_decode_layer_ragged_single_sequence(rng):
    # One sequence takes the single-sequence split plan; same results as a batch.
    _ragged_layer_vs_oracle(rng, 16, 8, 128, [4097])


def test_decode_layer_ragged_refuses_counts_past_the_bound(rng):
    # The counts live in device memory, so the host cannot throw "KV cache
    # full" (layer.ts:575): a sequence past max_n_keys gets NaN rows and no
    # append; its neighbours are unaffected.
    _ragged_layer_vs_oracle(rng, 16, 8, 128, [700, 1001, 0, 1000, 5000, 3], max_n_keys=1000)


@pytest.mark.parametrize("n_seqs", [2048, 2100])
def test_decode_layer_ragged_many_sequences(rng, n_seqs):
    # Both sides of the persistent kernel's limit, with idle, one-key and
    # refused sequences among them.
    lens = rng.integers(0, 41, n_seqs).astype(np.uint32)
    lens[:4] = [0, 1, 40, 41]
    _ragged_layer_vs_oracle(rng, 16, 8, 128, lens, max_n_keys=40)


def test_decode_layer_ragged_graph_replay(rng):
    # The prologue launch also resets the batch kernel's item counters; a
    # captured step replays that reset, so every replay gives the eager bits
    # (each replay rewrites the same cache rows with the same values).
    H, Hkv, d = 16, 8, 128
    lens = np.array([2500, 0, 900, 4097, 1], np.uint32)
    B = len(lens)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    rows = int(lens.sum())
    kc, vc = dev(randn(rng, rows * Hkv * d)), dev(randn(rng, rows * Hkv * d))
    q, k, v = dev(randn(rng, B * H * d)), dev(randn(rng, B * Hkv * d)), dev(randn(rng, B * Hkv * d))
    gq, gk = dev(rng.normal(1, 0.1, d)), dev(rng.normal(1, 0.1, d))
    inv = dev(oracle.rope_inv_freq(d, 1e6))
    offs_d, lens_d = ops.DeviceBuffer.from_array(offs), ops.DeviceBuffer.from_array(lens)
    maxn = int(lens.max())
    ws = ops.Workspace(H, Hkv, d, maxn, 0, B)
    qn, o = empty(B * H * d), empty(B * H * d)
    call = lambda: ops.decode_layer_ragged(q, k, v, gq, gk, inv, EPS, "neox", qn, kc, vc, offs_d,
                                           lens_d, o, B, maxn, H, Hkv, d, ws)
    st = ops.Stream()
    ops.set_stream(st)
    try:
        call()
        ops.sync()
        eager = get(o, B * H * d)
        eager_kc = kc.download(rows * Hkv * d)
        with ops.Graph() as g:
            call()
        for i in range(3):
            o.zero()  # eager, between replays
            g.launch()
            ops.sync()
            assert np.array_equal(get(o, B * H * d), eager), i
            assert np.array_equal(kc.download(rows * Hkv * d), eager_kc), i
            call()  # an eager call between replays
            ops.sync()
        g.free()
    finally:
        ops.set_stream(None)
        st.free()


# ------------------------------------------------------------ golden fixtures --
def test_golden_fixtures_on_gpu():
    # tests/golden/golden.npz: seeded inputs with the oracle's outputs and the
    # float64 closed form; the GPU path through the C ABI must meet the bar on
    # each, with the prologue's qn and cache rows bit-identical.
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
    H, Hkv, d = 16, 8, 128
    got = _decode(z["dec_q"], z["dec_k"], z["dec_v"], H, Hkv, d, 33)
    m = metrics(got, z["dec_o"], z["dec_o_f64"])
    assert meets_bar(m), fmt(m)
    got = _prefill(z["pre_q"], z["pre_k"], z["pre_v"], H, Hkv, d, 13, 5)
    m = metrics(got, z["pre_o"], z["pre_o_f64"])
    assert meets_bar(m), fmt(m)
    # Prologue + prefill of 3 tokens at position 12 onto a 16-row cache.
    maxk = 16
    kc = np.zeros(maxk * Hkv * d, np.float32)
    vc = np.zeros_like(kc)
    kc[:12 * Hkv * d], vc[:12 * Hkv * d] = z["pro_kc_prefix"], z["pro_vc_prefix"]
    kcb, vcb, qn, o = dev(kc), dev(vc), empty(3 * H * d), empty(3 * H * d)
    inv = dev(z["inv_freq"])
    ops.qk_prologue(dev(z["pro_q"]), dev(z["pro_k"]), dev(z["pro_v"]), dev(z["pro_gq"]),
                    dev(z["pro_gk"]), inv, EPS, "neox", qn, kcb, vcb, 3, 12, H, Hkv, d, maxk)
    ws = ops.Workspace(H, Hkv, d, maxk, 3)
    ops.attn_prefill(qn, kcb, vcb, o, H, Hkv, d, 3, 12, ws)
    assert np.array_equal(get(qn, 3 * H * d), z["pro_qn"])
    assert np.array_equal(kcb.download(maxk * Hkv * d)[12 * Hkv * d:15 * Hkv * d], z["pro_kn"])
    got_o = get(o, 3 * H * d)
    kfull = kcb.download(maxk * Hkv * d)
    vfull = vcb.download(maxk * Hkv * d)
    m = metrics(got_o, z["pro_o"], cf.attention(z["pro_qn"], kfull, vfull, H, Hkv, d, 3, 12))
    assert meets_bar(m), fmt(m)
