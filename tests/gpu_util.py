"""Helpers shared by the GPU parity tests: caches built like the reference's ``KvPair``
(crates/kernels/src/testutil.rs:86-153) -- the host quantises K/V to the cache type with the
oracle and uploads the bytes, and the oracle later sees exactly the values the GPU reads --
plus the BASELINE.json input generators and the tolerance metrics.
"""
from __future__ import annotations

import numpy as np

import oracle
from brasa_amd import KvType
from brasa_amd.device import DeviceBuffer

HQ, HKV, DIM = 32, 8, 128


def cache_bytes(kv: KvType, values: np.ndarray) -> np.ndarray:
    """f32 values -> the cache's bytes for type kv (host reference conversion)."""
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if kv == KvType.F32:
        return values.view(np.uint8)
    if kv == KvType.F16:
        return oracle.f32_to_f16(values).view(np.uint8)
    return oracle.quantize_kv_q8(values)


def seen_values(kv: KvType, raw: np.ndarray) -> np.ndarray:
    """The f32 values the kernels read from cache bytes ``raw``."""
    if kv == KvType.F32:
        return raw.view(np.float32).copy()
    if kv == KvType.F16:
        return oracle.f16_to_f32(raw.view(np.uint16))
    return oracle.dequantize_kv_q8(raw)


class KvPair:
    """K and V caches of one layer on the device plus the values the GPU sees."""

    def __init__(self, kv: KvType, k: np.ndarray, v: np.ndarray):
        self.kv = kv
        kb, vb = cache_bytes(kv, k), cache_bytes(kv, v)
        self.k = seen_values(kv, kb)
        self.v = seen_values(kv, vb)
        self.kbuf = DeviceBuffer.from_array(kb)
        self.vbuf = DeviceBuffer.from_array(vb)


def f16_normal(rng: np.random.Generator, n: int) -> np.ndarray:
    """Seeded N(0, 1) drawn in f32 and rounded to f16 (returned as f32 values)."""
    return oracle.round_f16(rng.standard_normal(n, dtype=np.float32))


def post_norm_rope(x: np.ndarray, tokens: int, heads: int, pos0: int, cos_t, sin_t) -> np.ndarray:
    """Per-head RMSNorm (weight 1, eps 1e-6) then RoPE-NeoX, as the prefill inputs of the
    benchmark configs are described (post QK-norm, post RoPE theta 1e6)."""
    y = oracle.rms_norm(x, np.ones(DIM, np.float32), DIM, 1e-6)
    return oracle.rope_neox(y, tokens, heads, DIM, pos0, cos_t, sin_t)


def bars(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    """(max-abs, max-rel) of got vs ref. max-rel is |got - ref| / max(|ref|, 0.2): below
    |ref| = 0.2 = 2e-3 / 1e-2 the absolute bar is the binding one."""
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float((d / np.maximum(np.abs(ref), 0.2)).max())
