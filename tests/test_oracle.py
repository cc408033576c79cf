"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

Each check is chosen so a plausible restatement mistake fails it: the reference's own
known-answer tests (crates/quant/src/qtype.rs:182-260, crates/kernels/tests/attention.rs:
256-285), closed forms (lk = 1, equal keys, GQA head mapping, exact Q8 ties), independent
implementations (numpy's float16 cast, a numpy f64 softmax) and invariants (causal mask).
"""
import math

import numpy as np
import pytest

import oracle


# ---- f16 conversion (qtype.rs:32-78) ---------------------------------------------------------

def test_f16_known_values():
    # qtype.rs:220-233
    f = lambda h: float(oracle.f16_to_f32(np.array([h], np.uint16))[0])
    assert f(0x3C00) == 1.0
    assert f(0xC000) == -2.0
    assert np.float32(f(0x3555)) == np.float32(0.33325195)
    assert np.float32(f(0x0001)) == np.float32(5.9604645e-8)
    assert f(0x7BFF) == 65504.0
    assert math.isinf(f(0x7C00))
    finite = oracle.f16_to_f32(np.arange(0x7C00, dtype=np.uint16))
    assert np.all(np.isfinite(finite)) and np.all(finite >= 0)


def test_f16_roundtrip_and_ties_exhaustive():
    # qtype.rs:236-260: every non-NaN f16 round-trips; midpoints go to even; one f32 ulp either
    # side goes to the nearest.
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    f = oracle.f16_to_f32(h)
    keep = ~np.isnan(f)
    assert np.array_equal(oracle.f32_to_f16(f[keep]), h[keep])
    lo = np.arange(0x7BFF, dtype=np.uint16)
    a, b = oracle.f16_to_f32(lo), oracle.f16_to_f32(lo + 1)
    mid = ((a + b) / np.float32(2)).astype(np.float32)
    even = np.where(lo % 2 == 0, lo, lo + 1).astype(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(mid), even)
    up = (mid.view(np.uint32) + 1).view(np.float32)
    dn = (mid.view(np.uint32) - 1).view(np.float32)
    assert np.array_equal(oracle.f32_to_f16(up), lo + 1)
    assert np.array_equal(oracle.f32_to_f16(dn), lo)
    assert np.array_equal(oracle.f32_to_f16(-mid), even | 0x8000)


def test_f16_special_cases():
    c = lambda x: int(oracle.f32_to_f16(np.array([x], np.float32))[0])
    assert c(65520.0) == 0x7C00
    assert c(1e10) == 0x7C00
    assert c(2.0 ** -25) == 0
    assert c(np.float32(2.0 ** -25) * np.float32(1.0001)) == 1
    assert math.isnan(float(oracle.f16_to_f32(np.array([c(float("nan"))], np.uint16))[0]))


def test_f16_matches_numpy_cast():
    # numpy's float32 -> float16 cast is an independent round-to-nearest-even implementation
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    # bias towards the f16 range, subnormals and the overflow edge
    y = (rng.standard_normal(500_000) * np.exp2(rng.uniform(-26, 17, 500_000))).astype(np.float32)
    for v in (x, y):
        with np.errstate(over="ignore"):
            want = v.astype(np.float16).view(np.uint16)
        assert np.array_equal(oracle.f32_to_f16(v), want)


# ---- KV-Q8 spec (qtype.rs:85-130) --------------------------------------------------------------

def test_q8_roundtrip_bound():
    # qtype.rs:186-218
    x = np.array([((i * 37 % 101) - 50.0) * 0.173 for i in range(128)], dtype=np.float32)
    x[32:64] = 0.0
    q = oracle.quantize_kv_q8(x)
    y = oracle.dequantize_kv_q8(q)
    for b in range(4):
        blk = x[32 * b:32 * b + 32]
        amax = float(np.max(np.abs(blk)))
        err = np.abs(blk - y[32 * b:32 * b + 32])
        assert np.all(err <= amax / 127.0 * 0.5 * (1 + 1e-3) + 1e-12)
        if amax > 0:
            codes = q[32 * b:32 * b + 32].view(np.int8)
            assert np.any(np.abs(codes.astype(np.int32)) == 127)
    assert np.all(y[32:64] == 0.0)


def test_q8_kat_of_store_kv_test():
    # crates/kernels/tests/attention.rs:256-285 with expectations derived in closed form
    rng = oracle.Rng(26)
    x = rng.vec(128 * 64, 20.0)
    x[32:64] = 0.0
    d = np.float32(oracle.round_f16(np.array([np.float32(1.0) / np.float32(127.0)]))[0])
    assert d == np.float32(129 * 2.0 ** -14)  # f16(1/127) = 0.00787353515625
    for j in range(32):
        x[128 + j] = np.float32(j - 15.5) * d
    x[128 + 31] = 1.0
    x[256:288] = 3000.0
    q = oracle.quantize_kv_q8(x).reshape(64, 136)
    # zero block: codes 0, scale 0
    assert np.all(q[0, 32:64] == 0) and q[0, 130] == 0 and q[0, 131] == 0
    # exact ties x / d = n + 0.5 go to even; amax = 1 -> d = f16(1/127); 1 / d -> 127
    codes = q[1, :32].view(np.int8).astype(int)
    for j in range(31):
        n = j - 15.5
        even = math.floor(n) if math.floor(n) % 2 == 0 else math.ceil(n)
        assert codes[j] == even, (j, codes[j], even)
    assert codes[31] == 127
    assert int(q[1, 128]) | (int(q[1, 129]) << 8) == 0x2008  # f16 bits of 129 * 2^-14
    # 3000-valued block: d = f16(3000 / 127) = 23.625, code round(3000 / 23.625) = 127
    assert int(q[2, 128]) | (int(q[2, 129]) << 8) == int(np.float16(23.625).view(np.uint16))
    assert np.all(q[2, :32].view(np.int8) == 127)


def test_q8_matches_numpy_restatement():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(128 * 4096) * np.exp2(rng.uniform(-12, 12, 128 * 4096))).astype(np.float32)
    x[:128] = 0.0
    got = oracle.quantize_kv_q8(x).reshape(-1, 136)
    g = x.reshape(-1, 4, 32)
    amax = np.max(np.abs(g), axis=2)
    dh = (amax / np.float32(127.0)).astype(np.float32).astype(np.float16)
    d = dh.astype(np.float32)[:, :, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        qv = np.where(d == 0, 0, np.clip(np.rint(g / d), -127, 127)).astype(np.int8)
    assert np.array_equal(got[:, :128].view(np.int8), qv.reshape(-1, 128))
    assert np.array_equal(got[:, 128:].copy().view(np.uint16), dh.view(np.uint16))
    # dequantisation is the exact f32 product scale * code
    back = oracle.dequantize_kv_q8(got.reshape(-1)).reshape(-1, 4, 32)
    assert np.array_equal(back, (d * qv.astype(np.float32)).astype(np.float32))


# ---- xorshift64* (testutil.rs:4-28) ------------------------------------------------------------

def test_rng_closed_form():
    M = (1 << 64) - 1
    for seed in (0, 1, 23, 26, 0xDEADBEEF):
        s = seed or 1
        r = oracle.Rng(seed)
        for _ in range(6):
            s ^= s >> 12
            s ^= (s << 25) & M
            s ^= s >> 27
            assert r.next_u64() == (s * 0x2545F4914F6CDD1D) & M
    r1, r2 = oracle.Rng(23), oracle.Rng(23)
    v = r1.vec(1000, 2.0)
    u = np.array([r2.next_u64() for _ in range(1000)], dtype=np.uint64)
    want = ((u >> np.uint64(40)).astype(np.float32) / np.float32(2 ** 23) - np.float32(1)) * np.float32(2)
    assert np.array_equal(v, want.astype(np.float32))
    assert v.min() >= -2.0 and v.max() < 2.0


# ---- attention (reference.rs:129-218) ----------------------------------------------------------

def _np_attention(q, k, v, tokens, hq, hkv, dim, pos0, scale):
    g = hq // hkv
    q = q.reshape(tokens, hq, dim).astype(np.float64)
    k = k.reshape(-1, hkv, dim).astype(np.float64)
    v = v.reshape(-1, hkv, dim).astype(np.float64)
    o = np.zeros((tokens, hq, dim))
    for t in range(tokens):
        n = pos0 + t + 1
        for h in range(hq):
            s = (k[:n, h // g, :] @ q[t, h]) * scale
            w = np.exp(s - s.max())
            w /= w.sum()
            o[t, h] = w @ v[:n, h // g, :]
    return o.astype(np.float32)


@pytest.mark.parametrize("tokens,pos0,hq,hkv", [(3, 5, 8, 2), (1, 40, 4, 4), (9, 0, 32, 8),
                                                (5, 11, 6, 3)])
def test_attention_matches_numpy_f64(tokens, pos0, hq, hkv):
    dim = 128
    rng = np.random.default_rng(tokens * 100 + pos0)
    q = rng.uniform(-2, 2, tokens * hq * dim).astype(np.float32)
    k = rng.uniform(-2, 2, (pos0 + tokens) * hkv * dim).astype(np.float32)
    v = rng.uniform(-3, 3, (pos0 + tokens) * hkv * dim).astype(np.float32)
    o, vmax = oracle.attention(q, k, v, tokens, hq, hkv, dim, pos0)
    want = _np_attention(q, k, v, tokens, hq, hkv, dim, pos0, 1 / math.sqrt(dim))
    np.testing.assert_allclose(o, want, rtol=2e-6, atol=1e-6)
    # vmax = max_j |v[j, kh, d]| over the visible keys
    vv = np.abs(v.reshape(-1, hkv, dim))
    for t in range(tokens):
        for h in range(hq):
            assert np.array_equal(vmax[t, h], vv[:pos0 + t + 1, h // (hq // hkv)].max(axis=0))
    # q16 variant: Q * (1/sqrt(dim) in f32) rounded to f16, scale 1
    o16, _ = oracle.attention(q, k, v, tokens, hq, hkv, dim, pos0, q16=True)
    qs = (q * np.float32(1 / np.sqrt(np.float32(dim)))).astype(np.float32).astype(np.float16)
    want16 = _np_attention(qs.astype(np.float32), k, v, tokens, hq, hkv, dim, pos0, 1.0)
    np.testing.assert_allclose(o16, want16, rtol=2e-6, atol=1e-6)


def test_attention_closed_forms():
    dim, hq, hkv = 128, 8, 2
    rng = np.random.default_rng(3)
    # lk = 1: the single key gets weight exp(0) / 1 = 1, so o = v_0 exactly
    q = rng.standard_normal(hq * dim).astype(np.float32)
    k = rng.standard_normal(hkv * dim).astype(np.float32)
    v = rng.standard_normal(hkv * dim).astype(np.float32)
    o, _ = oracle.attention(q, k, v, 1, hq, hkv, dim, 0)
    for h in range(hq):
        assert np.array_equal(o[0, h], v.reshape(hkv, dim)[h // 4])
    # equal keys: uniform weights, o = mean of v
    lk = 37
    k = np.tile(rng.standard_normal(dim).astype(np.float32), lk * hkv)
    v = rng.standard_normal(lk * hkv * dim).astype(np.float32)
    o, _ = oracle.attention(q, k, v, 1, hq, hkv, dim, lk - 1)
    mean = v.reshape(lk, hkv, dim).astype(np.float64).mean(axis=0)
    for h in range(hq):
        np.testing.assert_allclose(o[0, h], mean[h // 4], rtol=1e-6, atol=1e-7)
    # GQA mapping: head h reads KV head h // (hq / hkv)
    v = np.repeat(np.arange(1, hkv + 1, dtype=np.float32), dim)[None, :].repeat(lk, 0).reshape(-1)
    k = rng.standard_normal(lk * hkv * dim).astype(np.float32)
    o, _ = oracle.attention(q, k, v, 1, hq, hkv, dim, lk - 1)
    for h in range(hq):
        np.testing.assert_allclose(o[0, h], h // 4 + 1, rtol=1e-6)


def test_attention_causal_mask_and_exp_modes():
    dim, hq, hkv, tokens, pos0 = 128, 4, 2, 6, 3
    rng = oracle.Rng(5)
    q = rng.vec(tokens * hq * dim, 2.0)
    k = rng.vec((pos0 + tokens) * hkv * dim, 2.0)
    v = rng.vec((pos0 + tokens) * hkv * dim, 3.0)
    o, vm = oracle.attention(q, k, v, tokens, hq, hkv, dim, pos0)
    o2, vm2 = oracle.attention(q, k, v, tokens, hq, hkv, dim, pos0, recompute_exp=True)
    assert np.array_equal(o, o2) and np.array_equal(vm, vm2)
    # perturbing keys/values past pos0 + t leaves query t unchanged
    t = 2
    k2, v2 = k.copy(), v.copy()
    cut = (pos0 + t + 1) * hkv * dim
    k2[cut:] += 5.0
    v2[cut:] -= 7.0
    o3, _ = oracle.attention(q, k2, v2, tokens, hq, hkv, dim, pos0)
    assert np.array_equal(o3[:t + 1], o[:t + 1])
    assert not np.array_equal(o3[t + 1:], o[t + 1:])
    # row sampling computes exactly the selected rows
    o4, _ = oracle.attention(q, k, v, tokens, hq, hkv, dim, pos0, rows=(2, 4))
    assert np.array_equal(o4[2:4], o[2:4]) and np.all(o4[:2] == 0) and np.all(o4[4:] == 0)


def test_worst_functions():
    # attention.rs:12-32
    got = np.array([1.0, 2.0, -1.0], np.float32)
    exp = np.array([1.5, 2.0, -1.25], np.float32)
    vmax = np.array([2.0, 1.0, 0.5], np.float32)
    assert oracle.worst(got, exp, vmax) == pytest.approx(0.5)
    # f16: the final rounding (2^-11 |expected|) is discounted before dividing by max|v|
    exp = np.array([1.0, 1000.0], np.float32)
    gbits = oracle.f32_to_f16(np.array([1.0 + 2.0 ** -11, 1000.5], np.float32))
    vm = np.array([1.0, 1.0], np.float32)
    got = oracle.f16_to_f32(gbits)
    want = max(max(abs(got[0] - 1.0) - 2.0 ** -11, 0.0), max(abs(got[1] - 1000.0) - 1000.0 * 2.0 ** -11, 0.0))
    assert oracle.worst_f16(gbits, exp, vm) == pytest.approx(want)


# ---- rms_norm / rope (reference.rs:22-58, lib.rs:1388-1404) -------------------------------------

def test_rms_norm_and_rope():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(5 * 128).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    y = oracle.rms_norm(x, w, 128, 1e-6)
    xr = x.reshape(5, 128).astype(np.float64)
    want = xr / np.sqrt((xr ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(y.reshape(5, 128), want, rtol=1e-6)
    c, s = oracle.rope_table(1e6, 128, 64)
    p, i = 37, 5
    a = p * (1e6 ** (-(2 * i) / 128))
    assert c[p * 64 + i] == np.float32(math.cos(a)) and s[p * 64 + i] == np.float32(math.sin(a))
    assert c[0] == 1.0 and s[0] == 0.0
    # rotation of each (i, i + 64) pair preserves its norm
    t = rng.standard_normal(3 * 2 * 128).astype(np.float32)
    r = oracle.rope_neox(t, 3, 2, 128, 10, c, s).reshape(3, 2, 2, 64)
    t4 = t.reshape(3, 2, 2, 64)
    np.testing.assert_allclose(np.hypot(r[:, :, 0], r[:, :, 1]), np.hypot(t4[:, :, 0], t4[:, :, 1]),
                               rtol=1e-6)


def test_rope_neox_rotation_closed_form():
    """reference.rs:45-58 pinned by unit vectors, independently of the table: at position p,
    e_i (i < 64) turns into (cos a, sin a) in slots (i, i + 64) and e_{i+64} into (-sin a, cos a),
    a = p * theta^(-2 i / 128). A swapped sign or slot (rotation the other way) fails here."""
    theta, dim, max_pos = 1e6, 128, 4096
    c, s = oracle.rope_table(theta, dim, max_pos)
    for pos0, tokens in [(1, 3), (1000, 2), (4090, 6)]:
        for i in (0, 1, 17, 63):
            for hi in (False, True):
                x = np.zeros((tokens, 2, dim), np.float32)
                x[:, 1, i + 64 if hi else i] = 1.0  # head 1 of 2; head 0 stays zero
                y = oracle.rope_neox(x, tokens, 2, dim, pos0, c, s).reshape(tokens, 2, dim)
                assert not y[:, 0].any()
                for t in range(tokens):
                    a = (pos0 + t) * theta ** (-(2 * i) / dim)
                    ca, sa = math.cos(a), math.sin(a)
                    want_lo, want_hi = (-sa, ca) if hi else (ca, sa)
                    assert abs(y[t, 1, i] - want_lo) <= 1e-6 and abs(y[t, 1, i + 64] - want_hi) <= 1e-6
                    others = np.delete(y[t, 1], [i, i + 64])
                    assert not others.any()
    # i = 0 at p = 1: one radian, counter-clockwise (sin 1 > 0 lands in the upper half)
    x = np.zeros(dim, np.float32)
    x[0] = 1.0
    y = oracle.rope_neox(x, 1, 1, dim, 1, c, s)
    assert y[64] > 0.84 and abs(y[0] - math.cos(1.0)) <= 1e-7
