"""flk_q8_matvec on the GPU against the Q8_0 oracle, bit for bit.

The kernel follows q8_coop.wgsl's summation order (coop(64) in
cpuMatmulQ8F32, kernels/lib.ts:196-278) with one-rounding FMAs, so every
output must equal the oracle's (fused=True) exactly. Shapes cover the Qwen3
projections (q 2048x1024, k/v 1024x1024, o 1024x2048, gate/up 3072x1024,
down 1024x3072, LM head 151936x1024), every lanes-per-row layout (1..64 and
2-4 blocks per lane), the wide fallback (> 8192 columns), batched tokens and
the f16 scale edge cases (subnormal, exponent 31). Batches of 8 or more
tokens go through the tile kernel that reuses each weight block across
tokens; it is held to the same exactness.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

from flock_amd import ops  # noqa: E402


def run_gpu(packed, x, rows, cols, n_tokens=1):
    w = ops.Q8Matrix.from_packed(packed, rows, cols)
    xb = ops.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    ob = ops.DeviceBuffer(n_tokens * rows * 4)
    ops.q8_matvec(w, xb, ob, n_tokens)
    ops.sync()
    return ob.download(n_tokens * rows)


def problem(rng, rows, cols, n_tokens=1, wscale=0.05):
    packed = oracle.quant_matrix_q8((rng.standard_normal(rows * cols) * wscale).astype(np.float32),
                                    rows, cols)
    x = rng.standard_normal(n_tokens * cols).astype(np.float32)
    return packed, x


@pytest.mark.parametrize("rows,cols", [
    (2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072),  # Qwen3 projections
    (4096, 1024),                                   # q, k, v stacked
    (64, 32), (33, 64), (17, 96), (9, 160), (5, 288), (130, 512),  # 1..16 lanes per row
    (70, 4096), (40, 6144), (24, 8192),             # 2, 3, 4 blocks per lane
    (13, 8224),                                     # wide path (257 blocks)
    (1, 1024), (3, 1024),                           # fewer rows than a wave covers
])
def test_matches_oracle_exactly(rng, rows, cols):
    packed, x = problem(rng, rows, cols)
    got = run_gpu(packed, x, rows, cols)
    want = oracle.q8_matvec(packed, x, rows, cols, 64, fused=True)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]
    # The reference's own CPU model (two roundings per fma32) agrees too.
    assert np.array_equal(got, oracle.q8_matvec(packed, x, rows, cols, 64, fused=False))


@pytest.mark.parametrize("n_tokens", [2, 3, 7])
def test_batched_tokens(rng, n_tokens):
    rows, cols = 1024, 1024
    packed, x = problem(rng, rows, cols, n_tokens)
    got = run_gpu(packed, x, rows, cols, n_tokens)
    want = oracle.q8_matvec(packed, x, rows, cols, 64, fused=True)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,cols,n_tokens", [
    (96, 1024, 8), (100, 1024, 13),                 # one chunk; ragged row and token tiles
    (1024, 2048, 9), (33, 1536, 8),                 # two leaves per lane (the second partial)
    (70, 3072, 17), (13, 8224, 8), (24, 8192, 10),  # three and more chunks
    (40, 512, 10), (5, 32, 8), (3, 96, 11),         # fewer blocks than lanes
])
def test_token_tiles_match_oracle(rng, rows, cols, n_tokens):
    """Batches of 8 or more tokens take the weight-reusing tile kernel; its
    sums keep the coop(64) order, so it is exact too."""
    packed, x = problem(rng, rows, cols, n_tokens)
    got = run_gpu(packed, x, rows, cols, n_tokens)
    want = oracle.q8_matvec(packed, x, rows, cols, 64, fused=True)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]


@pytest.mark.parametrize("mode,rows,n", [
    ("plain", 4096, 1024), ("norm", 4096, 1024), ("gate_up", 4096, 1024),  # 8 row tiles
    ("norm", 2050, 256), ("gate_up", 2050, 256),  # 2 row tiles, ragged last group and tile
])
def test_row_streaming_matches_small_batches(rng, mode, rows, n):
    """Large batches stream several row tiles through one staged token tile
    (8 at 1024 tokens x 4096 rows, 2 at 256 x 2050); they must equal the same
    tokens projected 8 at a time (one row tile per workgroup), which the tests
    above hold to the oracle -- and the first tokens are held to it here too."""
    cols = 1024
    packed = random_packed(rng, rows, cols)
    w = ops.Q8Matrix.from_packed(packed, rows, cols)
    x = rng.standard_normal(n * cols).astype(np.float32)
    gain = rng.normal(1, 0.1, cols).astype(np.float32)
    xb = ops.DeviceBuffer.from_array(x)
    gb = ops.DeviceBuffer.from_array(gain)
    n_out = rows // 2 if mode == "gate_up" else rows

    def project(xbuf, ntok, out):
        if mode == "plain":
            ops.q8_matvec(w, xbuf, out, ntok)
        elif mode == "norm":
            ops.q8_matvec_ex(w, xbuf, out, ntok, norm_gain=gb, eps=oracle.QWEN3_EPS)
        else:
            ops.q8_gate_up_swiglu(w, xbuf, out, ntok, norm_gain=gb, eps=oracle.QWEN3_EPS)

    big = ops.DeviceBuffer(n * n_out * 4)
    project(xb, n, big)
    small = ops.DeviceBuffer(8 * n_out * 4)
    xs = ops.DeviceBuffer(8 * cols * 4)
    got = big.download(n * n_out).reshape(n, n_out)
    for t0 in range(0, n, 8):
        xs.upload(x[t0 * cols:(t0 + 8) * cols])
        project(xs, 8, small)
        ops.sync()
        assert np.array_equal(got[t0:t0 + 8], small.download(8 * n_out).reshape(8, n_out)), t0
    xin = x[:8 * cols]
    if mode != "plain":
        xin = oracle.rmsnorm(xin, gain, cols, 8, oracle.QWEN3_EPS)
    want = oracle.q8_matvec(packed, xin, rows, cols, 64, fused=True).reshape(8, rows)
    if mode == "gate_up":  # rows 2i, 2i + 1 are a (gate, up) pair
        want = oracle.swiglu(want[:, 0::2].ravel(), want[:, 1::2].ravel()).reshape(8, n_out)
    assert np.array_equal(got[:8], want)


def test_tile_kernels_equal_per_token_kernel_on_random_shapes():
    """Seeded random shapes and fusions: a batch of >= 8 tokens (tile kernels,
    any row tiling) equals the same tokens projected at most 7 at a time (the
    per-token kernel), bit for bit."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        rows = int(rng.integers(1, 2600))
        cols = 32 * int(rng.integers(1, 130))
        n = int(rng.integers(8, 300))
        fuse = ["plain", "norm", "up", "res", "gate_up"][case % 5]
        if fuse == "gate_up":
            rows += rows % 2
            cols = min(cols, 1024)
        packed = random_packed(rng, rows, cols)
        w = ops.Q8Matrix.from_packed(packed, rows, cols)
        x = rng.standard_normal(n * cols).astype(np.float32)
        aux = rng.standard_normal(n * max(rows, cols)).astype(np.float32)
        gain = ops.DeviceBuffer.from_array(rng.normal(1, 0.1, cols).astype(np.float32))
        n_out = rows // 2 if fuse == "gate_up" else rows

        def run(t0, t1):
            k = t1 - t0
            xb = ops.DeviceBuffer.from_array(x[t0 * cols:t1 * cols])
            ob = ops.DeviceBuffer(k * n_out * 4)
            if fuse == "plain":
                ops.q8_matvec(w, xb, ob, k)
            elif fuse == "norm":
                ops.q8_matvec_ex(w, xb, ob, k, norm_gain=gain, eps=oracle.QWEN3_EPS)
            elif fuse == "up":
                ub = ops.DeviceBuffer.from_array(aux[t0 * cols:t1 * cols])
                ops.q8_matvec_ex(w, xb, ob, k, up=ub)
            elif fuse == "res":
                rb = ops.DeviceBuffer.from_array(aux[t0 * rows:t1 * rows])
                ops.q8_matvec_ex(w, xb, ob, k, res=rb)
            else:
                ops.q8_gate_up_swiglu(w, xb, ob, k, norm_gain=gain, eps=oracle.QWEN3_EPS)
            ops.sync()
            return ob.download(k * n_out)

        big = run(0, n)
        small = np.concatenate([run(t, min(t + 7, n)) for t in range(0, n, 7)])
        assert np.array_equal(big, small), (case, rows, cols, n, fuse)


def random_packed(rng, rows, cols):
    """Q8_0 bytes with random int8 quants and f16 scales around 4e-4 (what
    quantRowQ8 gives for N(0, 0.05) weights), built without the quantizer."""
    blocks = np.empty((rows * cols // 32, 34), np.uint8)
    sc = (np.abs(rng.standard_normal(blocks.shape[0])) * 4e-4 + 1e-5).astype(np.float16)
    blocks[:, :2] = sc.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = rng.integers(0, 256, (blocks.shape[0], 32), dtype=np.uint8)
    return blocks.ravel()


def test_lm_head_shape(rng):
    # Qwen3-0.6B's tied LM head: 151936 x 1024 (165 MB of Q8_0).
    rows, cols = 151936, 1024
    packed = random_packed(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    got = run_gpu(packed, x, rows, cols)
    want = oracle.q8_matvec(packed, x, rows, cols, 64, fused=True)
    assert np.array_equal(got, want)
    assert oracle.argmax(got) == oracle.argmax(want)


def test_scale_edge_cases(rng):
    # Subnormal, tiny normal, largest finite and exponent-31 scales (inf and
    # nan patterns read as +-FLT_MAX); x small so products stay finite.
    rows, cols = 8, 64
    scales = [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x3C00]
    q = rng.integers(-128, 128, (rows, cols))
    parts = []
    for r in range(rows):
        for b in range(cols // 32):
            h = scales[r]
            parts.append(bytes([h & 0xFF, h >> 8]) +
                         bytes((q[r, 32 * b:32 * b + 32] & 0xFF).astype(np.uint8)))
    packed = np.frombuffer(b"".join(parts), np.uint8)
    x = (rng.standard_normal(cols) * 1e-3).astype(np.float32)
    got = run_gpu(packed, x, rows, cols)
    want = oracle.q8_matvec(packed, x, rows, cols, 64, fused=True)
    assert np.array_equal(got, want)


def test_integer_problem_is_exact(rng):
    # Integer quants, unit scales, integer x: the exact product, whatever the order.
    rows, cols = 512, 2048
    q = rng.integers(-128, 128, (rows, cols))
    x = rng.integers(-8, 9, cols).astype(np.float32)
    packed = np.frombuffer(b"".join(
        bytes([0x00, 0x3C]) + bytes((q[r, 32 * b:32 * b + 32] & 0xFF).astype(np.uint8))
        for r in range(rows) for b in range(cols // 32)), np.uint8)
    got = run_gpu(packed, x, rows, cols)
    assert np.array_equal(got, (q @ x.astype(np.int64)).astype(np.float32))


# ---------------------------------------------------------------- argmax / head
def gpu_argmax(x):
    n = x.size
    xb = ops.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    ov, oi = ops.DeviceBuffer(4), ops.DeviceBuffer(4)
    ws = ops.DeviceBuffer(ops.argmax_ws_bytes(n))
    ops.argmax(xb, n, ov, oi, ws)
    ops.sync()
    return float(ov.download(1)[0]), int(oi.download(1, np.uint32)[0])


@pytest.mark.parametrize("n", [1, 100, 256, 257, 4096, 151936, 1 << 20])
def test_argmax_matches_oracle(rng, n):
    x = rng.standard_normal(n).astype(np.float32)
    assert gpu_argmax(x) == oracle.argmax_wgsl(x)


def test_argmax_ties_nan_and_sentinel(rng):
    n = 151936
    x = rng.standard_normal(n).astype(np.float32)
    top = float(x.max()) + 1.0
    for i in (90000, 1234, 150000, 70001):  # equal maxima in different workgroups
        x[i] = top
    assert gpu_argmax(x) == (top, 1234) == oracle.argmax_wgsl(x)
    x[5] = np.nan
    x[1233] = np.nan
    assert gpu_argmax(x) == oracle.argmax_wgsl(x) == (top, 1234)
    y = np.full(1000, -np.inf, np.float32)
    y[::7] = np.nan
    assert gpu_argmax(y) == oracle.argmax_wgsl(y) == (-np.finfo(np.float32).max, 0xFFFFFFFF)
    y[400] = -np.finfo(np.float32).max
    assert gpu_argmax(y) == oracle.argmax_wgsl(y)


def run_head(x, gain, packed, vocab, hidden, with_logits=True):
    w = ops.Q8Matrix.from_packed(packed, vocab, hidden)
    xb = ops.DeviceBuffer.from_array(x)
    gb = ops.DeviceBuffer.from_array(gain)
    normed = ops.DeviceBuffer(hidden * 4)
    logits = ops.DeviceBuffer(vocab * 4) if with_logits else None
    ov, oi = ops.DeviceBuffer(4), ops.DeviceBuffer(4)
    ws = ops.DeviceBuffer(ops.lm_head_ws_bytes(vocab, hidden))
    ops.lm_head(xb, gb, oracle.QWEN3_EPS, w, normed, logits, ov, oi, ws)
    ops.sync()
    return (normed.download(hidden), logits.download(vocab) if with_logits else None,
            float(ov.download(1)[0]), int(oi.download(1, np.uint32)[0]))


@pytest.mark.parametrize("vocab,hidden", [(151936, 1024), (1000, 64), (5003, 2048), (300, 8224)])
def test_lm_head_matches_oracle(rng, vocab, hidden):
    packed = random_packed(rng, vocab, hidden)
    x = rng.standard_normal(hidden).astype(np.float32)
    gain = rng.normal(1, 0.1, hidden).astype(np.float32)
    normed, logits, v, i = run_head(x, gain, packed, vocab, hidden)
    w_normed, w_logits, w_v, w_i = oracle.lm_head(x, gain, oracle.QWEN3_EPS, packed, vocab, hidden)
    assert np.array_equal(normed, w_normed)
    assert np.array_equal(logits, w_logits)
    assert (v, i) == (w_v, w_i)
    # Without a logits buffer: the same token.
    assert run_head(x, gain, packed, vocab, hidden, with_logits=False)[2:] == (w_v, w_i)


def test_lm_head_tie_picks_lowest_row(rng):
    vocab, hidden = 151936, 1024
    packed = random_packed(rng, vocab, hidden).reshape(vocab, -1)
    x = rng.standard_normal(hidden).astype(np.float32)
    gain = np.ones(hidden, np.float32)
    _, logits, _, m = oracle.lm_head(x, gain, oracle.QWEN3_EPS, packed.ravel(), vocab, hidden)
    for r in (3, m // 2, vocab - 1):  # identical rows give identical logits
        packed[r] = packed[m]
    want = oracle.lm_head(x, gain, oracle.QWEN3_EPS, packed.ravel(), vocab, hidden)
    assert want[3] == min(3, m)
    got = run_head(x, gain, packed.ravel(), vocab, hidden)
    assert got[2:] == want[2:]
