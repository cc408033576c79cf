"""GPU: KV-cache writers and the q8_0 dequantiser, bit-exact against the oracle.

Mirrors crates/kernels/tests/attention.rs:223-285 (store_kv_convierte, seed 24;
store_kv_q8_igual_a_la_especificacion, seed 26) and the BASELINE.json requirement that Q8
dequantisation is bit-exact.
"""
import numpy as np
import pytest

import oracle
from brasa_amd import BrasaError, Kernels, KvType
from brasa_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def test_store_kv_f32_f16_edge_cases():
    k = Kernels()
    rng = oracle.Rng(24)
    x = rng.vec(4099, 50.0)
    mid = (oracle.f16_to_f32(np.array([0x3C01], np.uint16))[0] +
           oracle.f16_to_f32(np.array([0x3C02], np.uint16))[0]) / np.float32(2)
    x[:8] = [mid, -mid, 65520.0, 1e-7, 3e-8, 0.0, -0.0, 70000.0]
    src = DeviceBuffer.from_array(x)
    d32 = DeviceBuffer(x.nbytes)
    d16 = DeviceBuffer(x.size * 2)
    _say("store_kv f32/f16 n=4099")
    k.store_kv(KvType.F32, src, d32, x.size)
    k.store_kv(KvType.F16, src, d16, x.size)
    synchronize()
    assert np.array_equal(d32.download(np.uint32), x.view(np.uint32))
    assert np.array_equal(d16.download(np.uint16), oracle.f32_to_f16(x))


@pytest.mark.parametrize("n", [1, 3, 4, 5, 127, 1 << 20])
def test_store_kv_f16_sizes(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * np.exp2(rng.uniform(-26, 17, n))).astype(np.float32)
    src = DeviceBuffer.from_array(x)
    dst = DeviceBuffer(2 * n)
    _say(f"store_kv f16 n={n}")
    Kernels().store_kv(KvType.F16, src, dst, n)
    synchronize()
    assert np.array_equal(dst.download(np.uint16), oracle.f32_to_f16(x))


def test_store_kv_q8_matches_spec():
    k = Kernels()
    rng = oracle.Rng(26)
    x = rng.vec(128 * 64, 20.0)
    x[32:64] = 0.0
    d = oracle.round_f16(np.array([np.float32(1) / np.float32(127)], np.float32))[0]
    for j in range(32):
        x[128 + j] = np.float32(j - 15.5) * d
    x[128 + 31] = 1.0
    x[256:288] = 3000.0
    src = DeviceBuffer.from_array(x)
    dst = DeviceBuffer(KvType.Q8_0.bytes(x.size))
    _say("store_kv q8 (seed 26 KATs)")
    k.store_kv(KvType.Q8_0, src, dst, x.size)
    synchronize()
    assert np.array_equal(dst.download(np.uint8), oracle.quantize_kv_q8(x))


def test_store_kv_q8_wide_range_and_dequant_bit_exact():
    k = Kernels()
    rng = np.random.default_rng(5)
    n = 128 * 8 * 4097
    x = (rng.standard_normal(n) * np.exp2(rng.uniform(-20, 14, n))).astype(np.float32)
    x[:128] = 0.0
    src = DeviceBuffer.from_array(x)
    dst = DeviceBuffer(KvType.Q8_0.bytes(n))
    back = DeviceBuffer(4 * n)
    _say(f"store_kv q8 n={n} + dequantize")
    k.store_kv(KvType.Q8_0, src, dst, n)
    k.dequantize_kv_q8(dst, back, n // 128)
    synchronize()
    want = oracle.quantize_kv_q8(x)
    got = dst.download(np.uint8)
    assert np.array_equal(got, want)
    assert np.array_equal(back.download(np.uint32), oracle.dequantize_kv_q8(want).view(np.uint32))


def test_dequant_arbitrary_bytes_bit_exact():
    # any code/scale bytes, including f16 subnormal, inf and NaN scales
    rng = np.random.default_rng(9)
    raw = rng.integers(0, 256, size=136 * 5000, dtype=np.uint8)
    src = DeviceBuffer.from_array(raw)
    dst = DeviceBuffer(4 * 128 * 5000)
    _say("dequantize arbitrary bytes")
    Kernels().dequantize_kv_q8(src, dst, 5000)
    synchronize()
    got = dst.download(np.uint32)
    want = oracle.dequantize_kv_q8(raw).view(np.uint32)
    nan_g = np.isnan(got.view(np.float32))
    nan_w = np.isnan(want.view(np.float32))
    assert np.array_equal(nan_g, nan_w)
    assert np.array_equal(got[~nan_w], want[~nan_w])


def test_store_kv_q8_rejects_ragged():
    with pytest.raises(BrasaError) as e:
        Kernels().store_kv(KvType.Q8_0, 1, 1, 100)
    assert e.value.code == 1
