"""The producer step before attention: rms_norm, rope_neox and the fused qk_norm_rope_store.

Mirrors the reference's crates/kernels/tests/ops.rs:16-45 (rms_norm against the f64 reference,
max_rel <= 1e-5 with floor 1e-3), ops.rs:66-96 (rope_neox, error / (|a| + |b|) <= 1e-6) and
crates/kernels/tests/fused.rs:8-98 (fused == the unfused sequence, bit for bit, for every cache
type), with the same seeds, sizes and RNG. Beyond the reference: the fused output is also checked
against the f64 oracle, and its cache bytes against the oracle's f16 / q8_0 conversion of the
fused kernel's own k and v.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from brasa_amd import AttnShape, Kernels, KvType, RopeTable
from brasa_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu
D = 128


def max_rel(got, expected, floor):
    """testutil.rs:86-91."""
    got = np.asarray(got, np.float32)
    expected = np.asarray(expected, np.float32)
    return float(np.max(np.abs(got - expected) / np.maximum(np.abs(expected), floor)))


def rope_err(x, got, expected, dim):
    """ops.rs:88-96: |g - e| / (|a| + |b|) per RoPE pair."""
    x = x.reshape(-1, dim)
    got, expected = got.reshape(-1, dim), expected.reshape(-1, dim)
    h = dim // 2
    scale = np.maximum(np.abs(x[:, :h]) + np.abs(x[:, h:]), 1e-30)
    e1 = np.abs(got[:, :h] - expected[:, :h]) / scale
    e2 = np.abs(got[:, h:] - expected[:, h:]) / scale
    return float(max(e1.max(), e2.max()))


def test_rms_norm_matches_reference():
    k = Kernels()
    rng = oracle.Rng(11)
    worst = 0.0
    for rows, n in [(1, 2560), (37, 2560), (64 * 32, 128), (3, 100)]:
        x = rng.vec(rows * n, 30.0)
        w = rng.vec(n, 2.0)
        expected = oracle.rms_norm(x, w, n, 1e-6)
        gx, gw = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
        out = DeviceBuffer(4 * rows * n)
        k.rms_norm(gx, gw, out, rows, n, 1e-6)
        synchronize()
        worst = max(worst, max_rel(out.download(np.float32), expected, 1e-3))
        # in place (out == x), as qwen3.rs normalises q / k in place
        k.rms_norm(gx, gw, gx, rows, n, 1e-6)
        synchronize()
        assert np.array_equal(gx.download(np.float32).view(np.uint32),
                              out.download(np.float32).view(np.uint32))
    print(f"rms_norm: max relative error {worst:.2e}")
    assert worst <= 1e-5, worst


def test_rope_neox_matches_reference():
    k = Kernels()
    rng = oracle.Rng(13)
    heads, dim, max_pos = 32, 128, 40960
    table = RopeTable(1e6, dim, max_pos)
    cos, sin = oracle.rope_table(1e6, dim, max_pos)
    worst = 0.0
    for tokens, pos0 in [(1, 0), (7, 3), (16, 40944)]:
        x = rng.vec(tokens * heads * dim, 3.0)
        expected = oracle.rope_neox(x, tokens, heads, dim, pos0, cos, sin)
        gx = DeviceBuffer.from_array(x)
        k.rope_neox(gx, table, tokens, heads, dim, pos0)
        synchronize()
        worst = max(worst, rope_err(x, gx.download(np.float32), expected, dim))
    print(f"rope: max error / (|a| + |b|) {worst:.2e}")
    assert worst <= 1e-6, worst


@pytest.mark.parametrize("kv", [KvType.F32, KvType.F16, KvType.Q8_0], ids=lambda k: k.name_str)
def test_qk_norm_rope_store_equals_sequence(kv):
    k = Kernels()
    hq, hkv, eps = 32, 8, 1e-6
    table = RopeTable(1e6, D, 4096)
    cos, sin = oracle.rope_table(1e6, D, 4096)
    rng = oracle.Rng(31)
    # the reference draws the inputs of all three cache types from one generator in this order
    for drawn_for in [KvType.F32, KvType.F16, KvType.Q8_0]:
        cases = []
        for tokens, pos0 in [(1, 0), (1, 2999), (5, 37), (64, 128)]:
            q0 = rng.vec(tokens * hq * D, 3.0)
            k0 = rng.vec(tokens * hkv * D, 3.0)
            v0 = rng.vec(tokens * hkv * D, 3.0)
            qn, kn = rng.vec(D, 1.5), rng.vec(D, 1.5)
            cases.append((tokens, pos0, q0, k0, v0, qn, kn))
        if drawn_for == kv:
            break
    for tokens, pos0, q0, k0, v0, qn, kn in cases:
        shape = AttnShape(tokens, hq, hkv, D, pos0, kv)
        nkv = tokens * hkv * D
        cbytes = kv.bytes(nkv)
        gqn, gkn = DeviceBuffer.from_array(qn), DeviceBuffer.from_array(kn)

        def run(fused: bool):
            q, kb, v = (DeviceBuffer.from_array(a) for a in (q0, k0, v0))
            kc, vc = DeviceBuffer(cbytes), DeviceBuffer(cbytes)
            kc.fill(0xA5)
            vc.fill(0x5A)
            if fused:
                k.qk_norm_rope_store(kv, (q, kb, v), (gqn, gkn), eps, table, (kc, vc), shape)
            else:
                k.rms_norm(q, gqn, q, tokens * hq, D, eps)
                k.rms_norm(kb, gkn, kb, tokens * hkv, D, eps)
                k.rope_neox(q, table, tokens, hq, D, pos0)
                k.rope_neox(kb, table, tokens, hkv, D, pos0)
                k.store_kv(kv, kb, kc, nkv)
                k.store_kv(kv, v, vc, nkv)
            synchronize()
            return (q.download(np.float32), kb.download(np.float32),
                    kc.download(np.uint8), vc.download(np.uint8))

        a, b = run(False), run(True)
        name = f"KV {kv.name_str} T={tokens} pos0={pos0}"
        assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)), f"{name}: q differs"
        assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32)), f"{name}: k differs"
        assert np.array_equal(a[2], b[2]), f"{name}: K cache differs"
        assert np.array_equal(a[3], b[3]), f"{name}: V cache differs"

        # beyond the reference: against the f64 oracle and the oracle's cache conversion
        qe = oracle.rope_neox(oracle.rms_norm(q0, qn, D, eps), tokens, hq, D, pos0, cos, sin)
        ke = oracle.rope_neox(oracle.rms_norm(k0, kn, D, eps), tokens, hkv, D, pos0, cos, sin)
        for got, exp in ((b[0], qe), (b[1], ke)):
            assert np.max(np.abs(got - exp)) <= 1e-6 * np.max(np.abs(exp)), name
        if kv == KvType.F16:
            assert np.array_equal(b[2].view(np.uint16), oracle.f32_to_f16(b[1])), name
            assert np.array_equal(b[3].view(np.uint16), oracle.f32_to_f16(v0)), name
        elif kv == KvType.Q8_0:
            assert np.array_equal(b[2], oracle.quantize_kv_q8(b[1])), name
            assert np.array_equal(b[3], oracle.quantize_kv_q8(v0)), name
        else:
            assert np.array_equal(b[2].view(np.float32), b[1]), name
            assert np.array_equal(b[3].view(np.float32), v0), name


def test_qk_norm_rope_store_writes_at_pos0_view():
    """The cache pointers are views at row pos0 * hkv of the layer (qwen3.rs:555,592): rows
    before and after the written range keep their bytes."""
    k = Kernels()
    hq, hkv, tokens, pos0, cap = 32, 8, 3, 61, 128
    table = RopeTable(1e6, D, cap)
    rng = oracle.Rng(5)
    q = DeviceBuffer.from_array(rng.vec(tokens * hq * D, 2.0))
    kb = DeviceBuffer.from_array(rng.vec(tokens * hkv * D, 2.0))
    v = DeviceBuffer.from_array(rng.vec(tokens * hkv * D, 2.0))
    qn = DeviceBuffer.from_array(np.ones(D, np.float32))
    kn = DeviceBuffer.from_array(np.ones(D, np.float32))
    row = KvType.Q8_0.bytes(hkv * D)  # bytes per position
    kc, vc = DeviceBuffer(cap * row), DeviceBuffer(cap * row)
    kc.fill(0x33)
    vc.fill(0x44)
    shape = AttnShape(tokens, hq, hkv, D, pos0, KvType.Q8_0)
    k.qk_norm_rope_store(KvType.Q8_0, (q, kb, v), (qn, kn), 1e-6, table,
                         (kc.ptr + pos0 * row, vc.ptr + pos0 * row), shape)
    synchronize()
    kk, vv = kc.download(np.uint8), vc.download(np.uint8)
    lo, hi = pos0 * row, (pos0 + tokens) * row
    assert np.all(kk[:lo] == 0x33) and np.all(kk[hi:] == 0x33)
    assert np.all(vv[:lo] == 0x44) and np.all(vv[hi:] == 0x44)
    assert np.array_equal(kk[lo:hi], oracle.quantize_kv_q8(kb.download(np.float32)))
