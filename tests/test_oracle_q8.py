"""Pins the Q8_0 oracle (oracle/flock_oracle_q8.c) before it judges the GPU.

Each check is independent of the restated code: numpy's IEEE float16
conversions, exact integer arithmetic, hand-derived expected values of the
reference's algorithm (kernels/lib.ts:28-53, 141-156, 196-318;
web/js/wire.mjs:33-53), and an f64 error bound.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

F32_MAX = float(np.finfo(np.float32).max)


def block(scale_bits: int, q) -> bytes:
    q = np.asarray(q, np.int64)
    assert q.size == 32
    return bytes([scale_bits & 0xFF, scale_bits >> 8]) + bytes((q & 0xFF).astype(np.uint8))


# ---------------------------------------------------------------- f32 -> f16
def test_f32_to_f16_matches_ieee_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32),
        (rng.standard_normal(2000) * 1e-5).astype(np.float32),        # f16 subnormals
        (rng.standard_normal(2000) * 1e-8).astype(np.float32),        # below / near 2^-24
        (rng.standard_normal(2000) * 3e4).astype(np.float32),         # near the top
        np.array([65504, 65519.99, 65520, 1e6, -1e6, 0.0, -0.0, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, np.inf,
                  -np.inf], np.float32),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16_array(vals)
    assert np.array_equal(got, want)


def test_f32_to_f16_ties_and_nan():
    # 1 + 2^-11 lies halfway between 1 and 1 + 2^-10: even wins (1.0 = 0x3C00);
    # 1 + 3 * 2^-11 lies halfway between 1 + 2^-10 and 1 + 2^-9: 0x3C02.
    assert oracle.f32_to_f16(1 + 2.0 ** -11) == 0x3C00
    assert oracle.f32_to_f16(1 + 3 * 2.0 ** -11) == 0x3C02
    assert oracle.f32_to_f16(float("nan")) & 0x7FFF == 0x7E00
    assert oracle.f32_to_f16(-65520.0) == 0xFC00  # rounds past the largest finite: -inf


# ---------------------------------------------------------------- f16 -> f32
def test_half_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float64)
    exp31 = (h & 0x7C00) == 0x7C00
    want[exp31] = np.where(h[exp31] & 0x8000, -3.4028235e38, 3.4028235e38)
    got = np.array([oracle.half_to_f32(int(v)) for v in h])
    assert np.array_equal(got[~exp31], want[~exp31])
    assert np.array_equal(got[exp31], want[exp31])
    # Rounded to f32 (as cpuMatmulQ8F32 does with fr) the clamp is FLT_MAX.
    assert np.float32(oracle.half_to_f32(0x7C00)) == np.float32(F32_MAX)


# ---------------------------------------------------------------- quantizer
def test_quant_row_invariants():
    rng = np.random.default_rng(1)
    rows, cols = 8, 256
    w = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
    w[:32] = 0.0  # an all-zero block
    packed = oracle.quant_matrix_q8(w, rows, cols).reshape(-1, 34)
    vals = w.reshape(-1, 32).astype(np.float64)
    for b in range(packed.shape[0]):
        h = int(packed[b, 0]) | (int(packed[b, 1]) << 8)
        q = packed[b, 2:].view(np.int8).astype(np.float64)
        amax = np.max(np.abs(vals[b]))
        d = amax / 127
        assert h == oracle.f32_to_f16(np.float32(d))
        if amax == 0:
            assert h == 0 and not q.any()
            continue
        assert np.all(np.abs(vals[b] / d - q) <= 0.5)
        assert np.abs(q[np.argmax(np.abs(vals[b]))]) == 127


def test_quant_ties_round_toward_plus_infinity():
    # amax 127 makes d exactly 1, so v / d are the values themselves. JS
    # Math.round sends x.5 up: 2.5 -> 3, -2.5 -> -2, 0.5 -> 1, -0.5 -> 0.
    v = np.zeros(32, np.float32)
    v[:6] = [127, 2.5, -2.5, 0.5, -0.5, -127]
    q = oracle.quant_matrix_q8(v, 1, 32)[2:].view(np.int8)
    assert list(q[:6]) == [127, 3, -2, 1, 0, -127]


def test_split_is_a_byte_permutation():
    rows, cols = 3, 64
    packed = np.arange(rows * cols // 32 * 34, dtype=np.int64).astype(np.uint8)
    qs, sc = oracle.split_q8(packed, rows, cols)
    blocks = packed.reshape(-1, 34)
    assert np.array_equal(sc, blocks[:, 0].astype(np.uint16) | (blocks[:, 1].astype(np.uint16) << 8))
    assert np.array_equal(qs.view(np.uint8), blocks[:, 2:].ravel())


# ---------------------------------------------------------------- matvec
def int_problem(rng, rows, cols, scale_bits=0x3C00):
    """Integer quants, power-of-two scales, small integer x: every partial sum
    is an integer well inside 2^24, so any summation order is exact."""
    q = rng.integers(-128, 128, (rows, cols))
    x = rng.integers(-8, 9, cols).astype(np.float32)
    scales = np.full((rows, cols // 32), scale_bits, np.int64)
    packed = b"".join(block(int(scales[r, b]), q[r, 32 * b:32 * b + 32])
                      for r in range(rows) for b in range(cols // 32))
    return np.frombuffer(packed, np.uint8), q, x, scales


@pytest.mark.parametrize("lanes", [0, 64])
@pytest.mark.parametrize("rows,cols", [(7, 32), (16, 1024), (4, 3072), (3, 8192)])
def test_matvec_exact_on_integer_problems(lanes, rows, cols):
    rng = np.random.default_rng(rows * cols + lanes)
    packed, q, x, _ = int_problem(rng, rows, cols)
    want = (q @ x.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.q8_matvec(packed, x, rows, cols, lanes), want)


def test_matvec_uses_each_blocks_own_scale():
    # Scales 2^k per block (f16 exponent bits), integer data: still exact.
    rng = np.random.default_rng(7)
    rows, cols = 5, 256
    q = rng.integers(-128, 128, (rows, cols))
    x = rng.integers(-4, 5, cols).astype(np.float32)
    k = rng.integers(-3, 4, (rows, cols // 32))
    packed = np.frombuffer(b"".join(
        block(int((15 + k[r, b]) << 10), q[r, 32 * b:32 * b + 32])
        for r in range(rows) for b in range(cols // 32)), np.uint8)
    w = q.astype(np.float64) * np.repeat(2.0 ** k, 32, axis=1)
    want = (w @ x.astype(np.float64)).astype(np.float32)
    for lanes in (0, 64):
        assert np.array_equal(oracle.q8_matvec(packed, x, rows, cols, lanes), want)


def test_matvec_coop_order_is_the_lane_tree():
    # Hand-derived from q8_coop.wgsl / matmulF32: with 64 lanes, block b goes
    # to lane b % 64 and the 64 partials meet in a pairwise tree. Lane 0 holds
    # 2^24 (block 0), lane 1 holds -2^24 (block 1), lane 32 holds 1 (block 32).
    # Tree: stride 32 rounds 2^24 + 1 back to 2^24 (ties to even), lanes 0 and
    # 1 then cancel: result 0. Serial order (blocks 0, 1, ..., 32) gives 1.
    cols = 33 * 32
    q = np.zeros((1, cols), np.int64)
    x = np.zeros(cols, np.float32)
    q[0, 0], x[0] = 64, 2.0 ** 18
    q[0, 32], x[32] = -64, 2.0 ** 18
    q[0, 32 * 32], x[32 * 32] = 1, 1.0
    packed = np.frombuffer(b"".join(block(0x3C00, q[0, 32 * b:32 * b + 32]) for b in range(33)),
                           np.uint8)
    assert oracle.q8_matvec(packed, x, 1, cols, 64)[0] == 0.0
    assert oracle.q8_matvec(packed, x, 1, cols, 0)[0] == 1.0


def lane_tree(p):
    """The reference's pairwise tree over 64 lane partials (strides 32 .. 1),
    in f32 with the lower lane as the left operand; p is [64, ...]."""
    p = np.array(p, np.float32)
    for s in (32, 16, 8, 4, 2, 1):
        p[:s] = p[:s] + p[s:2 * s]
    return p[0]


def recursive_halving(p64):
    """What the tile kernels do with 64 leaf partials of 32 outputs: lane q
    (of 32) adds leaf q + 32 to leaf q in place (the stride-32 step), then at
    stride s = 16 .. 1 keeps the lower half of its value list when bit s of q
    is clear (else the upper half moved down) and adds the copy its partner
    q ^ s sends. Returns out[q] = the value lane q ends with."""
    v = (p64[:32] + p64[32:]).astype(np.float32)     # [lane][output]
    n = 32
    for s in (16, 8, 4, 2, 1):
        hi = (np.arange(32) & s) != 0
        lo_half, up_half = v[:, :n // 2], v[:, n // 2:n]
        keep = np.where(hi[:, None], up_half, lo_half)
        send = np.where(hi[:, None], lo_half, up_half)
        recv = send[np.arange(32) ^ s]
        v = (keep + recv).astype(np.float32)
        n //= 2
    return v[:, 0]


def test_recursive_halving_is_the_lane_tree():
    # Partials with wildly different magnitudes make every rounding count: a
    # wrong pairing or order would change the bits.
    rng = np.random.default_rng(21)
    for _ in range(20):
        p = (rng.standard_normal((64, 32)) * 2.0 ** rng.integers(-20, 20, (64, 32))).astype(np.float32)
        p[rng.random((64, 32)) < 0.2] = 0
        want = lane_tree(p)
        assert np.array_equal(recursive_halving(p), want)
    # And the serial sum would differ somewhere (the check has teeth).
    serial = np.zeros(32, np.float32)
    for lane in range(64):
        serial = (serial + p[lane]).astype(np.float32)
    assert not np.array_equal(serial, want)


def test_matvec_within_f32_bound_of_f64():
    rng = np.random.default_rng(11)
    rows, cols = 64, 3072
    w = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
    packed = oracle.quant_matrix_q8(w, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    qs, sc = oracle.split_q8(packed, rows, cols)
    deq = qs.astype(np.float64).reshape(rows, cols // 32, 32) * np.array(
        [oracle.half_to_f32(int(h)) for h in sc], np.float64).reshape(rows, cols // 32, 1)
    exact = deq.reshape(rows, cols) @ x.astype(np.float64)
    mag = np.abs(deq.reshape(rows, cols)) @ np.abs(x.astype(np.float64))
    for lanes in (0, 64):
        got = oracle.q8_matvec(packed, x, rows, cols, lanes).astype(np.float64)
        # Every term passes through at most ~cols/32 + 40 roundings of 2^-24.
        assert np.all(np.abs(got - exact) <= (cols / 32 + 40) * 2.0 ** -24 * mag)


def test_fused_and_two_rounding_fma_agree_on_typical_data():
    # The reference's fma32 rounds twice; v_fma_f32 once. With int8 weights the
    # f64 sums are exact in practice, so the two models give the same bits.
    rng = np.random.default_rng(12)
    rows, cols = 256, 1024
    packed = oracle.quant_matrix_q8((rng.standard_normal(rows * cols) * 0.05).astype(np.float32),
                                    rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    a = oracle.q8_matvec(packed, x, rows, cols, 64, fused=False)
    b = oracle.q8_matvec(packed, x, rows, cols, 64, fused=True)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- argmax
def test_argmax_wgsl_matches_numpy_lowest_index():
    rng = np.random.default_rng(13)
    for n in (1, 7, 256, 151936):
        x = rng.standard_normal(n).astype(np.float32)
        v, i = oracle.argmax_wgsl(x)
        assert i == int(np.argmax(x)) and v == x[i]
        assert i == oracle.argmax(x)  # argmaxRef (head_ref.ts:65-74) agrees on finite input
    # Ties: several equal maxima, including -0 / +0 (equal under ==).
    x = np.array([1, 5, 2, 5, 5, 0], np.float32)
    assert oracle.argmax_wgsl(x) == (5.0, 1)
    x = np.array([-1, -0.0, 0.0, -2], np.float32)
    assert oracle.argmax_wgsl(x)[1] == 1


def test_argmax_wgsl_nan_and_sentinel():
    x = np.array([np.nan, 2, np.nan, 3, 3], np.float32)
    assert oracle.argmax_wgsl(x) == (3.0, 3)
    assert oracle.argmax_wgsl(x)[1] == int(np.nanargmax(x))
    # Nothing beats the start value: argmax.wgsl returns its sentinel.
    v, i = oracle.argmax_wgsl(np.array([-np.inf, np.nan], np.float32))
    assert i == 0xFFFFFFFF and v == -F32_MAX
    # -FLT_MAX itself wins (equal to the start value, lower index).
    assert oracle.argmax_wgsl(np.array([-np.inf, -F32_MAX], np.float32))[1] == 1


# ---------------------------------------------------------------- swiglu / add
def test_swiglu_against_f64_and_exact_cases():
    rng = np.random.default_rng(21)
    g = (rng.standard_normal(100000) * 4).astype(np.float32)
    u = rng.standard_normal(100000).astype(np.float32)
    got = oracle.swiglu(g, u).astype(np.float64)
    g64 = g.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u.astype(np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    # Four f32 roundings (exp, 1 + e, the quotient, the product), each within
    # half an ulp of its own value: at most 4 ulp of the result.
    assert np.all(np.abs(got - want) <= 4 * ulp)
    z = oracle.swiglu(np.zeros(4, np.float32), np.ones(4, np.float32))
    assert np.array_equal(z, np.zeros(4, np.float32))
    assert np.array_equal(oracle.swiglu(g[:8], np.zeros(8, np.float32)), np.zeros(8, np.float32))
    # Large positive g: silu(g) == g exactly once exp(-g) underflows below ulp(1).
    assert oracle.swiglu(np.float32([100.0]), np.float32([3.0]))[0] == np.float32(300.0)


def test_add_is_f32_addition():
    rng = np.random.default_rng(22)
    a = rng.standard_normal(5000).astype(np.float32)
    b = rng.standard_normal(5000).astype(np.float32)
    assert np.array_equal(oracle.add(a, b), a + b)


# ---------------------------------------------------------------- whole layer
def tiny_layer(rng, hid=128, ffn=256, H=4, Hkv=2, d=64):
    cfg = dict(nHeads=H, nKvHeads=Hkv, headDim=d, hidden=hid, ffn=ffn, eps=oracle.QWEN3_EPS)
    shapes = {"attn_q.weight": (H * d, hid), "attn_k.weight": (Hkv * d, hid),
              "attn_v.weight": (Hkv * d, hid), "attn_output.weight": (hid, H * d),
              "ffn_gate.weight": (ffn, hid), "ffn_up.weight": (ffn, hid),
              "ffn_down.weight": (hid, ffn)}
    w = {n: oracle.quant_matrix_q8((rng.standard_normal(r * c) * 0.05).astype(np.float32), r, c)
         for n, (r, c) in shapes.items()}
    for n, sz in (("attn_norm.weight", hid), ("ffn_norm.weight", hid),
                  ("attn_q_norm.weight", d), ("attn_k_norm.weight", d)):
        w[n] = rng.normal(1, 0.1, sz).astype(np.float32)
    return cfg, w, shapes


def dequant(packed, rows, cols):
    qs, sc = oracle.split_q8(packed, rows, cols)
    s = np.array([oracle.half_to_f32(int(h)) for h in sc]).reshape(rows, cols // 32, 1)
    return (qs.astype(np.float64).reshape(rows, cols // 32, 32) * s).reshape(rows, cols)


def layer_f64(hidden, n, w, shapes, cfg, kc, vc, pos0):
    """The layer's mathematics in float64 (dequantized weights), for wiring."""
    from oracle import closed_form as cf
    H, Hkv, d, hid, eps = cfg["nHeads"], cfg["nKvHeads"], cfg["headDim"], cfg["hidden"], cfg["eps"]
    W = {k: dequant(w[k], *shapes[k]) for k in shapes}
    x = hidden.reshape(n, hid).astype(np.float64)
    nh = cf.rmsnorm(x.ravel(), w["attn_norm.weight"], hid, n, eps).reshape(n, hid)
    q = nh @ W["attn_q.weight"].T
    k = nh @ W["attn_k.weight"].T
    v = nh @ W["attn_v.weight"].T
    inv = cf.inv_freq(d, 1e6)
    q = cf.rope(cf.rmsnorm(q.ravel(), w["attn_q_norm.weight"], d, n * H, eps), n, H, d, pos0, inv)
    k = cf.rope(cf.rmsnorm(k.ravel(), w["attn_k_norm.weight"], d, n * Hkv, eps), n, Hkv, d, pos0, inv)
    row = Hkv * d
    kc[pos0 * row:(pos0 + n) * row] = k
    vc[pos0 * row:(pos0 + n) * row] = v.ravel()
    a = cf.attention(q, kc, vc, H, Hkv, d, n, pos0).reshape(n, H * d)
    h = x + a @ W["attn_output.weight"].T
    nh2 = cf.rmsnorm(h.ravel(), w["ffn_norm.weight"], hid, n, eps).reshape(n, -1)
    g, u = nh2 @ W["ffn_gate.weight"].T, nh2 @ W["ffn_up.weight"].T
    return (h + (g / (1 + np.exp(-g)) * u) @ W["ffn_down.weight"].T).ravel()


@pytest.mark.parametrize("n,pos0", [(1, 0), (1, 9), (5, 0), (6, 11)])
def test_layer_composition_against_f64(n, pos0):
    rng = np.random.default_rng(31 + n + pos0)
    cfg, w, shapes = tiny_layer(rng)
    hid, row = cfg["hidden"], cfg["nKvHeads"] * cfg["headDim"]
    maxk = pos0 + n
    kc = np.zeros(maxk * row, np.float32)
    vc = np.zeros(maxk * row, np.float32)
    kc[:pos0 * row] = rng.standard_normal(pos0 * row)
    vc[:pos0 * row] = rng.standard_normal(pos0 * row)
    kc64, vc64 = kc.astype(np.float64), vc.astype(np.float64)
    hidden = rng.standard_normal(n * hid).astype(np.float32)
    if n == 1:
        got = oracle.layer_forward(hidden, w, cfg, kc, vc, pos0)
    else:
        got = oracle.layer_prefill(hidden, n, w, cfg, kc, vc, pos0)
    want = layer_f64(hidden, n, w, shapes, cfg, kc64, vc64, pos0)
    assert np.max(np.abs(got - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))
    assert np.max(np.abs(kc - kc64)) < 1e-5 and np.max(np.abs(vc - vc64)) < 1e-6


def test_layer_prefill_rows_equal_decode_steps():
    # layerPrefillRef over n tokens == n layerForwardRef steps (same cache, same
    # outputs), because every op is per token or causal (test_prefill.ts:119-132).
    rng = np.random.default_rng(40)
    cfg, w, _ = tiny_layer(rng)
    n, hid, row = 4, cfg["hidden"], cfg["nKvHeads"] * cfg["headDim"]
    hidden = rng.standard_normal(n * hid).astype(np.float32)
    kc1, vc1 = np.zeros(n * row, np.float32), np.zeros(n * row, np.float32)
    pre = oracle.layer_prefill(hidden, n, w, cfg, kc1, vc1, 0)
    kc2, vc2 = np.zeros(n * row, np.float32), np.zeros(n * row, np.float32)
    steps = np.concatenate([oracle.layer_forward(hidden[i * hid:(i + 1) * hid], w, cfg, kc2, vc2, i)
                            for i in range(n)])
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)
    assert np.max(np.abs(pre - steps)) < 1e-5
