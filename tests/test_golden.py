"""Committed golden vectors (tests/golden/*.npz, written by tests/golden/make_fixtures.py).

CPU: the oracle still reproduces every fixture bit for bit. GPU (marker ``gpu``): the C ABI
reproduces them -- the q8_0 cache bytes exactly, attention within the reference's decode bar
(worst <= 1e-5 of max|v|, tests/attention.rs:25-32) and the fp16 prefill bars (max-abs 2e-3,
max-rel 1e-2 against attention_q16).
"""
import os

import numpy as np
import pytest

import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D = 128


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_decode_fixtures():
    for name, kv in (("decode_f16.npz", "f16"), ("decode_q8.npz", "q8")):
        g = load(name)
        hq, hkv, lk = int(g["hq"]), int(g["hkv"]), int(g["lk"])
        if kv == "f16":
            ks, vs = oracle.f16_to_f32(g["k_cache"]), oracle.f16_to_f32(g["v_cache"])
        else:
            ks, vs = oracle.dequantize_kv_q8(g["k_cache"]), oracle.dequantize_kv_q8(g["v_cache"])
        o, vmax = oracle.attention(g["q"], ks, vs, 1, hq, hkv, D, lk - 1)
        assert np.array_equal(o.view(np.uint32), g["o"].view(np.uint32)), name
        assert np.array_equal(vmax, g["vmax"]), name


def test_oracle_reproduces_prefill_fixture():
    g = load("prefill_q16.npz")
    o, _ = oracle.attention(g["q"], oracle.f16_to_f32(g["k_cache"]), oracle.f16_to_f32(g["v_cache"]),
                            int(g["tokens"]), int(g["hq"]), int(g["hkv"]), D, int(g["pos0"]),
                            q16=True)
    assert np.array_equal(o.view(np.uint32), g["o"].view(np.uint32))


def test_oracle_reproduces_q8_fixture():
    g = load("kv_q8.npz")
    assert np.array_equal(oracle.quantize_kv_q8(g["x"]), g["q8"])
    q8 = g["q8"].reshape(8, 136)
    assert np.all(q8[1, :128] == 0) and np.all(q8[1, 128:] == 0)  # zero row: codes and scale 0


@pytest.mark.gpu
def test_device_matches_decode_fixtures():
    from brasa_amd import AttnShape, Kernels, KvType, decode_partials_len
    from brasa_amd.device import DeviceBuffer, synchronize
    k = Kernels()
    for name, kv in (("decode_f16.npz", KvType.F16), ("decode_q8.npz", KvType.Q8_0)):
        g = load(name)
        hq, hkv, lk = int(g["hq"]), int(g["hkv"]), int(g["lk"])
        print(f"golden decode {name}", flush=True)
        q = DeviceBuffer.from_array(g["q"])
        kb, vb = DeviceBuffer.from_array(g["k_cache"]), DeviceBuffer.from_array(g["v_cache"])
        part = DeviceBuffer(4 * decode_partials_len(hq, lk))
        o = DeviceBuffer(4 * hq * D)
        k.decode_attention_lanes(q, kb, vb, part, o, AttnShape(1, hq, hkv, D, lk - 1, kv))
        synchronize()
        assert oracle.worst(o.download(np.float32), g["o"], g["vmax"]) <= 1e-5, name


@pytest.mark.gpu
def test_device_matches_prefill_fixture():
    from brasa_amd import AttnShape, Kernels, KvType
    from brasa_amd.device import DeviceBuffer, synchronize
    g = load("prefill_q16.npz")
    hq, hkv, tokens, pos0 = int(g["hq"]), int(g["hkv"]), int(g["tokens"]), int(g["pos0"])
    cap = (pos0 + tokens + 63) // 64 * 64
    kc = np.zeros(cap * hkv * D, np.uint16)
    vc = np.zeros(cap * hkv * D, np.uint16)
    kc[: g["k_cache"].size] = g["k_cache"]
    vc[: g["v_cache"].size] = g["v_cache"]
    print("golden prefill", flush=True)
    k = Kernels()
    q = DeviceBuffer.from_array(g["q"])
    kb, vb = DeviceBuffer.from_array(kc), DeviceBuffer.from_array(vc)
    o = DeviceBuffer(2 * tokens * hq * D)
    k.flash_attention(q, kb, vb, o, AttnShape(tokens, hq, hkv, D, pos0, KvType.F16))
    synchronize()
    got = oracle.f16_to_f32(o.download(np.uint16))
    want = g["o"].reshape(-1)
    # the fp16 bars: max-abs 2e-3, max-rel 1e-2 (relative to max(|ref|, 0.2), where the
    # absolute bar binds below |ref| = 2e-3 / 1e-2)
    err = np.abs(got.astype(np.float64) - want)
    assert err.max() <= 2e-3
    assert np.max(err / np.maximum(np.abs(want), 0.2)) <= 1e-2


@pytest.mark.gpu
def test_device_matches_q8_fixture():
    from brasa_amd import Kernels, KvType
    from brasa_amd.device import DeviceBuffer, synchronize
    g = load("kv_q8.npz")
    print("golden store_kv q8", flush=True)
    k = Kernels()
    src = DeviceBuffer.from_array(g["x"])
    dst = DeviceBuffer(g["q8"].size)
    k.store_kv(KvType.Q8_0, src, dst, g["x"].size)
    synchronize()
    assert np.array_equal(dst.download(np.uint8), g["q8"])
