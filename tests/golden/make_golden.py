"""Write tests/golden/golden.npz: small seeded inputs with the oracle's outputs
and the float64 closed-form outputs beside them.

    python tests/golden/make_golden.py

The reference ships no vectors for this path (its randVec is unseeded,
kernels/lib.ts:595-599), so these fixtures come from the CPU oracle
(oracle/flock_oracle.c) after it has been pinned by tests/test_oracle.py; the
f64 columns let a later reader re-check them against the mathematics. Inputs
are N(0,1) f32 from numpy's PCG64 with fixed seeds.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from oracle import closed_form as cf  # noqa: E402

H, HKV, D = 16, 8, 128


def main() -> None:
    rng = np.random.default_rng(20261201)
    n = lambda k: rng.standard_normal(k, dtype=np.float32)  # noqa: E731
    out = {"inv_freq": oracle.rope_inv_freq(D)}

    # decode: 16/8 heads, 33 keys
    q, k, v = n(H * D), n(33 * HKV * D), n(33 * HKV * D)
    out.update(dec_q=q, dec_k=k, dec_v=v, dec_o=oracle.attn(q, k, v, H, HKV, D, 33),
               dec_o_f64=cf.attention(q, k, v, H, HKV, D, 1, 32))

    # prefill: 13 queries on top of 5 cached keys
    q, k, v = n(13 * H * D), n(18 * HKV * D), n(18 * HKV * D)
    out.update(pre_q=q, pre_k=k, pre_v=v, pre_o=oracle.attn_prefill(q, k, v, H, HKV, D, 13, 5),
               pre_o_f64=cf.attention(q, k, v, H, HKV, D, 13, 5))

    # layer prologue + prefill: 3 tokens at position 12 of a 16-row cache
    q, k, v = n(3 * H * D), n(3 * HKV * D), n(3 * HKV * D)
    gq = rng.normal(1, 0.1, D).astype(np.float32)
    gk = rng.normal(1, 0.1, D).astype(np.float32)
    kc, vc = np.zeros(16 * HKV * D, np.float32), np.zeros(16 * HKV * D, np.float32)
    kc[:12 * HKV * D], vc[:12 * HKV * D] = n(12 * HKV * D), n(12 * HKV * D)
    out.update(pro_q=q, pro_k=k, pro_v=v, pro_gq=gq, pro_gk=gk,
               pro_kc_prefix=kc[:12 * HKV * D].copy(), pro_vc_prefix=vc[:12 * HKV * D].copy())
    qn, o = oracle.layer_attn_prefill(q, k, v, gq, gk, out["inv_freq"], kc, vc, 3, 12, H, HKV, D)
    out.update(pro_qn=qn, pro_o=o, pro_kn=kc[12 * HKV * D:15 * HKV * D].copy())

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
