"""Writes the small golden vectors under tests/golden/ from the CPU oracle.

The reference keeps no stored attention vectors (its tests regenerate inputs from seeds and
compare with reference.rs); these fixtures freeze, for a few small seeded cases generated with
the reference's own xorshift64* RNG (crates/kernels/src/testutil.rs:4-28), the inputs and the
oracle's outputs, so that any later change of the oracle or of the device path is measured
against fixed numbers:

* ``decode_f16.npz``   decode, hq 8 / hkv 2, lk 300, fp16 KV (reference.rs:150-171)
* ``decode_q8.npz``    decode, hq 8 / hkv 2, lk 300, q8_0 KV (cache bytes included)
* ``prefill_q16.npz``  causal prefill, T 40 at pos0 3, hq 8 / hkv 2, attention_q16 (:129-145)
* ``kv_q8.npz``        quantize_kv_q8 of 8 rows, including an all-zero row and exact ties

Run from the repository root: ``python tests/golden/make_fixtures.py``.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

D = 128


def decode(kv: str, seed: int) -> dict:
    hq, hkv, lk = 8, 2, 300
    rng = oracle.Rng(seed)
    q = rng.vec(hq * D, 2.0)
    k = rng.vec(lk * hkv * D, 2.0)
    v = rng.vec(lk * hkv * D, 3.0)
    if kv == "f16":
        kc, vc = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
        ks, vs = oracle.f16_to_f32(kc), oracle.f16_to_f32(vc)
    else:
        kc, vc = oracle.quantize_kv_q8(k), oracle.quantize_kv_q8(v)
        ks, vs = oracle.dequantize_kv_q8(kc), oracle.dequantize_kv_q8(vc)
    o, vmax = oracle.attention(q, ks, vs, 1, hq, hkv, D, lk - 1)
    return dict(hq=hq, hkv=hkv, lk=lk, q=q, k_cache=kc, v_cache=vc, o=o, vmax=vmax)


def prefill() -> dict:
    hq, hkv, tokens, pos0 = 8, 2, 40, 3
    rng = oracle.Rng(22)
    n = (pos0 + tokens) * hkv * D
    q = oracle.round_f16(rng.vec(tokens * hq * D, 2.0))
    kc = oracle.f32_to_f16(rng.vec(n, 2.0))
    vc = oracle.f32_to_f16(rng.vec(n, 3.0))
    o, vmax = oracle.attention(q, oracle.f16_to_f32(kc), oracle.f16_to_f32(vc), tokens, hq, hkv,
                               D, pos0, q16=True)
    return dict(hq=hq, hkv=hkv, tokens=tokens, pos0=pos0, q=q, k_cache=kc, v_cache=vc, o=o,
                vmax=vmax)


def kv_q8() -> dict:
    rng = oracle.Rng(26)
    x = rng.vec(8 * D, 4.0)
    x[D:2 * D] = 0.0                                   # all-zero row
    d = np.float32(oracle.f16_to_f32(oracle.f32_to_f16(np.float32([1.0 / 127]))))[0]
    x[2 * D:2 * D + 32] = (np.arange(32, dtype=np.float32) - 15.5) * d  # exact ties
    x[2 * D + 31] = 1.0                                # amax 1 -> d = f16(1/127)
    return dict(x=x, q8=oracle.quantize_kv_q8(x))


def main() -> None:
    oracle.build()
    np.savez_compressed(os.path.join(HERE, "decode_f16.npz"), **decode("f16", 23))
    np.savez_compressed(os.path.join(HERE, "decode_q8.npz"), **decode("q8", 24))
    np.savez_compressed(os.path.join(HERE, "prefill_q16.npz"), **prefill())
    np.savez_compressed(os.path.join(HERE, "kv_q8.npz"), **kv_q8())
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
