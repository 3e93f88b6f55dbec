"""The parity bar itself (tests/parity.py), exercised on the CPU.

Mistakes are planted in the oracle's own output -- a dropped key, the wrong kv
head, a causal bound off by one, a missing 1/sqrt(d) -- and the bar must
reject each, while the oracle's honest result and a re-rounded copy of it pass.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import closed_form as cf
from conftest import randn
from parity import meets_bar, metrics

H, HKV, D = 16, 8, 128


@pytest.fixture(scope="module")
def decode_case():
    rng = np.random.default_rng(11)
    nk = 700
    q, k, v = randn(rng, H * D), randn(rng, nk * HKV * D), randn(rng, nk * HKV * D)
    return q, k, v, nk


def test_bar_accepts_the_oracle_and_a_reordered_sum(decode_case):
    q, k, v, nk = decode_case
    want = oracle.attn(q, k, v, H, HKV, D, nk)
    exact = cf.attention(q, k, v, H, HKV, D, 1, nk - 1)
    assert meets_bar(metrics(want, want, exact))
    # The exact result rounded once to f32 is a legitimate (better) answer.
    assert meets_bar(metrics(exact.astype(np.float32), want, exact))


def test_bar_rejects_a_dropped_key(decode_case):
    q, k, v, nk = decode_case
    want = oracle.attn(q, k, v, H, HKV, D, nk)
    exact = cf.attention(q, k, v, H, HKV, D, 1, nk - 1)
    bad = oracle.attn(q, k, v, H, HKV, D, nk - 1)
    assert not meets_bar(metrics(bad, want, exact))


def test_bar_rejects_a_wrong_kv_head(decode_case):
    q, k, v, nk = decode_case
    want = oracle.attn(q, k, v, H, HKV, D, nk)
    exact = cf.attention(q, k, v, H, HKV, D, 1, nk - 1)
    # Heads read kv head (h + 1) mod Hkv's V rows: swap the kv-head blocks.
    v_rot = np.roll(v.reshape(nk, HKV, D), 1, axis=1).ravel()
    bad = oracle.attn(q, k, v_rot, H, HKV, D, nk)
    assert not meets_bar(metrics(bad, want, exact))


def test_bar_rejects_a_missing_scale(decode_case):
    q, k, v, nk = decode_case
    want = oracle.attn(q, k, v, H, HKV, D, nk)
    exact = cf.attention(q, k, v, H, HKV, D, 1, nk - 1)
    bad = oracle.attn(q * np.float32(np.sqrt(D)), k, v, H, HKV, D, nk)
    assert not meets_bar(metrics(bad, want, exact))


def test_bar_rejects_an_off_by_one_causal_bound():
    rng = np.random.default_rng(12)
    nq, pos0 = 40, 30
    nk = pos0 + nq
    q, k, v = randn(rng, nq * H * D), randn(rng, (nk + 1) * HKV * D), randn(rng, (nk + 1) * HKV * D)
    want = oracle.attn_prefill(q, k, v, H, HKV, D, nq, pos0)
    exact = cf.attention(q, k, v, H, HKV, D, nq, pos0)
    assert meets_bar(metrics(want, want, exact))
    bad = oracle.attn_prefill(q, k, v, H, HKV, D, nq, pos0 + 1)  # one key too many
    assert not meets_bar(metrics(bad, want, exact))
