"""The whole decoder layer and its fused projections on the GPU.

* flk_q8_matvec_ex's fusions (rmsnorm in, swiglu in, residual out) and
  flk_swiglu / flk_add equal the oracle's separate ops bit for bit.
* DecoderLayer (flock_amd/decoder.py) against layerForwardRef /
  layerPrefillRef restated (oracle.layer_forward / layer_prefill) on the
  Qwen3-0.6B shapes with random Q8_0 weights: the K/V rows it appends are
  bit-identical; the layer output differs only through attention's summation
  order (held to 1e-4 of its magnitude, and no farther from the float64 layer
  than the oracle is, plus 1e-5).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

from flock_amd import ops  # noqa: E402
from flock_amd.decoder import QWEN3_06B, DecoderConfig, DecoderLayer  # noqa: E402
from test_gpu_q8 import random_packed  # noqa: E402

EPS = oracle.QWEN3_EPS


def dev(a):
    return ops.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


@pytest.mark.parametrize("rows,cols,n", [(4096, 1024, 1), (1024, 3072, 1), (2048, 1024, 3),
                                         (300, 8224, 2),
                                         # token tiles (8 or more tokens)
                                         (2048, 1024, 11), (1024, 3072, 9), (300, 8224, 8)])
def test_matvec_fusions_match_separate_ops(rng, rows, cols, n):
    packed = random_packed(rng, rows, cols)
    w = ops.Q8Matrix.from_packed(packed, rows, cols)
    x = rng.standard_normal(n * cols).astype(np.float32) * 3
    up = rng.standard_normal(n * cols).astype(np.float32)
    res = rng.standard_normal(n * rows).astype(np.float32)
    gain = rng.normal(1, 0.1, cols).astype(np.float32)
    o = ops.DeviceBuffer(n * rows * 4)
    mv = lambda xx: oracle.q8_matvec(packed, xx, rows, cols, 64, fused=True)  # noqa: E731

    ops.q8_matvec_ex(w, dev(x), o, n, norm_gain=dev(gain), eps=EPS)
    ops.sync()
    assert np.array_equal(o.download(n * rows), mv(oracle.rmsnorm(x, gain, cols, n, EPS)))

    ops.q8_matvec_ex(w, dev(x), o, n, up=dev(up), res=dev(res))
    ops.sync()
    assert np.array_equal(o.download(n * rows), oracle.add(res, mv(oracle.swiglu(x, up))))

    ob = dev(res)  # res aliasing o: o <- o + W x
    ops.q8_matvec_ex(w, dev(x), ob, n, res=ob)
    ops.sync()
    assert np.array_equal(ob.download(n * rows), oracle.add(res, mv(x)))


def test_elementwise_ops(rng):
    n = 100003
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    o = ops.DeviceBuffer(n * 4)
    ops.swiglu(dev(g), dev(u), o, n)
    ops.sync()
    assert np.array_equal(o.download(n), oracle.swiglu(g, u))
    ops.add(dev(g), dev(u), o, n)
    ops.sync()
    assert np.array_equal(o.download(n), oracle.add(g, u))


def make_weights(rng, cfg: DecoderConfig):
    w = {n: random_packed(rng, r, c) for n, (r, c) in cfg.shapes().items()}
    for n, sz in (("attn_norm.weight", cfg.hidden), ("ffn_norm.weight", cfg.hidden),
                  ("attn_q_norm.weight", cfg.headDim), ("attn_k_norm.weight", cfg.headDim)):
        w[n] = rng.normal(1, 0.1, sz).astype(np.float32)
    return w


def ocfg(cfg: DecoderConfig) -> dict:
    return dict(nHeads=cfg.nHeads, nKvHeads=cfg.nKvHeads, headDim=cfg.headDim,
                hidden=cfg.hidden, ffn=cfg.ffn, eps=cfg.eps)


def close(got, want):
    scale = max(1.0, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= 1e-4 * scale, (err, scale)


def test_decode_steps_match_layer_forward_ref(rng):
    cfg = DecoderConfig(maxKeys=64, maxPrefill=8)
    w = make_weights(rng, cfg)
    layer = DecoderLayer.create(cfg, w)
    row = cfg.nKvHeads * cfg.headDim
    kc = np.zeros(cfg.maxKeys * row, np.float32)
    vc = np.zeros_like(kc)
    h = rng.standard_normal(cfg.hidden).astype(np.float32)
    want = h
    for step in range(5):
        if step % 2 == 0:  # fresh input, or chain the previous output (layer.ts:645-648)
            h = rng.standard_normal(cfg.hidden).astype(np.float32)
            layer.encode(h)
            want = oracle.layer_forward(h, w, ocfg(cfg), kc, vc, step)
        else:
            layer.encode()
            want = oracle.layer_forward(got, w, ocfg(cfg), kc, vc, step)
        got = layer.readOutput()
        gk, gv = layer.readCache(step + 1)
        assert np.array_equal(gk, kc[:(step + 1) * row]), step
        assert np.array_equal(gv, vc[:(step + 1) * row]), step
        close(got, want)
    layer.free()


@pytest.mark.parametrize("n,pos0", [(5, 0), (8, 3), (21, 6)])
def test_prefill_matches_layer_prefill_ref(rng, n, pos0):
    cfg = DecoderConfig(maxKeys=32, maxPrefill=max(8, n))
    w = make_weights(rng, cfg)
    layer = DecoderLayer.create(cfg, w)
    row = cfg.nKvHeads * cfg.headDim
    kc = np.zeros(cfg.maxKeys * row, np.float32)
    vc = np.zeros_like(kc)
    if pos0:
        h0 = rng.standard_normal(pos0 * cfg.hidden).astype(np.float32)
        layer.encodePrefill(pos0, h0)
        oracle.layer_prefill(h0, pos0, w, ocfg(cfg), kc, vc, 0)
    h = rng.standard_normal(n * cfg.hidden).astype(np.float32)
    layer.encodePrefill(n, h)
    want = oracle.layer_prefill(h, n, w, ocfg(cfg), kc, vc, pos0)
    got = layer.readOutput(n)
    gk, gv = layer.readCache(pos0 + n)
    assert np.array_equal(gk, kc[:(pos0 + n) * row]) and np.array_equal(gv, vc[:(pos0 + n) * row])
    close(got, want)
    # A decode step after the prefill sees the prefill's cache.
    x = rng.standard_normal(cfg.hidden).astype(np.float32)
    layer.encode(x)
    close(layer.readOutput(), oracle.layer_forward(x, w, ocfg(cfg), kc, vc, pos0 + n))
    layer.free()


def test_guards(rng):
    cfg = DecoderConfig(maxKeys=2, maxPrefill=2)
    layer = DecoderLayer.create(cfg, make_weights(rng, cfg))
    x = np.zeros(cfg.hidden, np.float32)
    with pytest.raises(ValueError):
        layer.encodePrefill(3, np.zeros(3 * cfg.hidden, np.float32))
    with pytest.raises(ValueError):
        layer.encode(np.zeros(5, np.float32))
    assert layer.nKeys == 0
    layer.encode(x)
    layer.encode(x)
    with pytest.raises(Exception, match="KV cache full at 2 keys"):
        layer.encode(x)
    layer.free()


@pytest.mark.parametrize("ffn,hid,n", [(3072, 1024, 1), (3072, 1024, 3), (500, 256, 2), (64, 64, 1),
                                       (3072, 1024, 12), (500, 256, 9)])
def test_gate_up_swiglu_matches_separate_ops(rng, ffn, hid, n):
    gate = random_packed(rng, ffn, hid)
    up = random_packed(rng, ffn, hid)
    gq, gs = ops.q8_split(gate, ffn, hid)
    uq, us = ops.q8_split(up, ffn, hid)
    w = ops.Q8Matrix(ops.interleave_rows(gq, uq, ffn, hid),
                     ops.interleave_rows(gs, us, ffn, hid // 32), 2 * ffn, hid)
    x = rng.standard_normal(n * hid).astype(np.float32) * 2
    gain = rng.normal(1, 0.1, hid).astype(np.float32)
    act = ops.DeviceBuffer(n * ffn * 4)
    ops.q8_gate_up_swiglu(w, dev(x), act, n, norm_gain=dev(gain), eps=EPS)
    ops.sync()
    nx = oracle.rmsnorm(x, gain, hid, n, EPS)
    want = oracle.swiglu(oracle.q8_matvec(gate, nx, ffn, hid, 64, fused=True),
                         oracle.q8_matvec(up, nx, ffn, hid, 64, fused=True))
    assert np.array_equal(act.download(n * ffn), want)
    # Without the norm.
    ops.q8_gate_up_swiglu(w, dev(x), act, n)
    ops.sync()
    want = oracle.swiglu(oracle.q8_matvec(gate, x, ffn, hid, 64, fused=True),
                         oracle.q8_matvec(up, x, ffn, hid, 64, fused=True))
    assert np.array_equal(act.download(n * ffn), want)


def test_gate_up_swiglu_rejects_wide_rows():
    from flock_amd import _lib
    rc = _lib.lib().flk_q8_gate_up_swiglu(0x1000, 0x1000, 0x1000, 0x1000, 8, 2048, 1, None, 0.0)
    assert rc == _lib.FLK_ERR_UNSUPPORTED
