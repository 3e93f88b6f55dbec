"""RoPE's cos/sin evaluation (flock_amd/csrc/trig.hpp), run on the CPU.

The kernels must reproduce the oracle's fr(cos(theta)) / fr(sin(theta))
(ops_ref.ts:76, computed there in double and rounded once) bit for bit. The
same __host__ __device__ function is compiled here for the host and compared
with the C library over every angle the 32k-context configs produce (64
frequencies x positions 0..40000), special angles near multiples of pi/2, and
2M random angles up to 4e6 (beyond which the kernels use the device libm).
"""
from __future__ import annotations

import ctypes
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

SHIM = r'''
#include "%s"
extern "C" void sincos_batch(const float* th, long n, float* s, float* c) {
  for (long i = 0; i < n; i++) flk::sincos_f32_exact(th[i], s[i], c[i]);
}
'''


@pytest.fixture(scope="module")
def sincos(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("trig")
    src = d / "shim.hip"
    src.write_text(SHIM % os.path.join(ROOT, "flock_amd", "csrc", "trig.hpp"))
    so = d / "shim.so"
    subprocess.run([HIPCC, "-x", "hip", "--offload-arch=gfx950", "-O2", "-ffp-contract=off",
                    "-fPIC", "-shared", "-o", str(so), str(src)], check=True,
                   capture_output=True)
    lib = ctypes.CDLL(str(so))
    lib.sincos_batch.argtypes = [ctypes.c_void_p, ctypes.c_long, ctypes.c_void_p,
                                 ctypes.c_void_p]

    def run(th):
        th = np.ascontiguousarray(th, np.float32)
        s, c = np.empty_like(th), np.empty_like(th)
        lib.sincos_batch(th.ctypes.data, th.size, s.ctypes.data, c.ctypes.data)
        return s, c
    return run


def _check(sincos, th, use_math=False):
    s, c = sincos(th)
    if use_math:  # the C library itself, one call at a time
        ws = np.array([math.sin(float(t)) for t in th], np.float64).astype(np.float32)
        wc = np.array([math.cos(float(t)) for t in th], np.float64).astype(np.float32)
    else:
        ws = np.sin(th.astype(np.float64)).astype(np.float32)
        wc = np.cos(th.astype(np.float64)).astype(np.float32)
    bad = np.nonzero((s != ws) | (c != wc))[0]
    assert bad.size == 0, [(float(th[i]), s[i], ws[i], c[i], wc[i]) for i in bad[:5]]


def test_rope_angles_of_long_contexts(sincos):
    inv = np.array([1.0 / math.pow(1e6, 2 * j / 128) for j in range(64)], np.float32)
    pos = np.arange(0, 40001, dtype=np.float64)
    th = (pos[:, None] * inv[None, :].astype(np.float64)).astype(np.float32).ravel()
    _check(sincos, th)
    _check(sincos, th[::97], use_math=True)


def test_special_and_random_angles(sincos):
    k = np.arange(1, 200000, dtype=np.float64)
    near = (k * (np.pi / 2)).astype(np.float32)  # the f32 nearest multiples of pi/2
    th = np.concatenate([
        np.float32([0.0, 1e-30, 1e-10, 0.5, 0.78539816, 1.0, 4194303.5]),
        near, np.nextafter(near, np.float32(np.inf)), np.nextafter(near, np.float32(0)),
        np.random.default_rng(0).uniform(0, 4.1e6, 2_000_000).astype(np.float32)])
    _check(sincos, th)
    _check(sincos, th[:20000], use_math=True)


def test_planted_mistake_is_caught(sincos):
    # A restatement that skipped the second reduction constant would differ
    # from libm on large angles: check the comparison is sharp enough to see it.
    th = np.random.default_rng(1).uniform(1e5, 4e6, 200000).astype(np.float32)
    x = th.astype(np.float64)
    k = np.rint(x * (2 / np.pi))
    r = x - k * 1.5707963267948966  # one-constant reduction
    q = k.astype(np.int64) & 3
    bad_s = np.where(q == 0, np.sin(r), np.where(q == 1, np.cos(r),
                     np.where(q == 2, -np.sin(r), -np.cos(r)))).astype(np.float32)
    assert np.sum(bad_s != np.sin(x).astype(np.float32)) > 0
    s, _ = sincos(th)
    assert np.sum(s != np.sin(x).astype(np.float32)) == 0
