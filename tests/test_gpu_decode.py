"""GPU: split-K decode attention against the f64 oracle.

Mirrors crates/kernels/tests/attention.rs:112-177 (decode_case, seed 23, pos0 in
{0, 1, 255, 256, 700, 4095, 16383} x KV {f32, f16, q8_0}), :287-345 (other GQA groups, seed 25)
and crates/kernels/tests/launch.rs:119-168 (seed 78, lk in {1, 37, 300, 1025}); the bar is the
reference's ``worst <= 1e-5 * max|v|`` (attention.rs:25-32, lib.rs:5-18).
"""
import numpy as np
import pytest

import oracle
from brasa_amd import AttnShape, BrasaError, Kernels, KvType, OutDType, decode_partials_len
from brasa_amd._lib import lib
from brasa_amd.device import DeviceBuffer, synchronize
from gpu_util import DIM, HKV, HQ, KvPair

pytestmark = pytest.mark.gpu

KVS = [KvType.F32, KvType.F16, KvType.Q8_0]


def _say(msg):
    print(msg, flush=True)


def run_decode(k, variant, q, cache, hq, hkv, pos0, out=OutDType.F32):
    lk = pos0 + 1
    gq = DeviceBuffer.from_array(q)
    part = DeviceBuffer(4 * decode_partials_len(hq, lk))
    o = DeviceBuffer(hq * DIM * (4 if out == OutDType.F32 else 2))
    shape = AttnShape(1, hq, hkv, DIM, pos0, cache.kv)
    fn = k.decode_attention_lanes if variant == "lanes" else k.decode_attention
    fn(gq, cache.kbuf, cache.vbuf, part, o, shape, out=out)
    synchronize()
    if out == OutDType.F32:
        return o.download(np.float32).reshape(hq, DIM)
    return o.download(np.uint16).reshape(hq, DIM)


@pytest.mark.parametrize("variant", ["lanes", "per_head"])
@pytest.mark.parametrize("kv", KVS)
def test_decode_case(variant, kv):
    k = Kernels()
    rng = oracle.Rng(23)
    w = 0.0
    for pos0 in [0, 1, 255, 256, 700, 4095, 16383]:
        lk = pos0 + 1
        q = rng.vec(HQ * DIM, 2.0)
        cache = KvPair(kv, rng.vec(lk * HKV * DIM, 2.0), rng.vec(lk * HKV * DIM, 3.0))
        _say(f"decode {variant} kv={kv.name_str} pos0={pos0}")
        got = run_decode(k, variant, q, cache, HQ, HKV, pos0)
        want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, pos0)
        w = max(w, oracle.worst(got, want, vmax))
    print(f"decode {variant} KV {kv.name_str}: worst / max|v| = {w:.2e}")
    assert w <= 1e-5, w


@pytest.mark.parametrize("kv", KVS)
def test_decode_other_groups(kv):
    k = Kernels()
    rng = oracle.Rng(25)
    for hq in [8, 16, 64]:
        w = 0.0
        for pos0 in [0, 300, 4095]:
            lk = pos0 + 1
            q = rng.vec(hq * DIM, 2.0)
            cache = KvPair(kv, rng.vec(lk * HKV * DIM, 2.0), rng.vec(lk * HKV * DIM, 3.0))
            _say(f"decode lanes group={hq // HKV} kv={kv.name_str} pos0={pos0}")
            got = run_decode(k, "lanes", q, cache, hq, HKV, pos0)
            want, vmax = oracle.attention(q, cache.k, cache.v, 1, hq, HKV, DIM, pos0)
            w = max(w, oracle.worst(got, want, vmax))
        assert w <= 1e-5, (hq, w)


@pytest.mark.parametrize("kv", KVS)
def test_decode_partial_head_group_row(kv):
    # six KV heads at GQA group 4: at short lengths the plan puts four head groups in a
    # workgroup, so the second grid row holds two real head groups and two past the last one
    # (waves without keys, merge threads past hq)
    k = Kernels()
    rng = oracle.Rng(31)
    hq, hkv = 24, 6
    w = 0.0
    for pos0 in [0, 37, 300, 1024]:
        lk = pos0 + 1
        q = rng.vec(hq * DIM, 2.0)
        cache = KvPair(kv, rng.vec(lk * hkv * DIM, 2.0), rng.vec(lk * hkv * DIM, 3.0))
        _say(f"decode lanes hq={hq} hkv={hkv} kv={kv.name_str} pos0={pos0}")
        got = run_decode(k, "lanes", q, cache, hq, hkv, pos0)
        want, vmax = oracle.attention(q, cache.k, cache.v, 1, hq, hkv, DIM, pos0)
        w = max(w, oracle.worst(got, want, vmax))
    assert w <= 1e-5, w


def test_decode_non_power_of_two_group():
    # group 3 is outside GQA_GROUPS: lanes is rejected (the reference panics), the per-head
    # variant serves it (lib.rs:1056-1103)
    k = Kernels()
    rng = oracle.Rng(27)
    hq, hkv, pos0 = 24, 8, 777
    q = rng.vec(hq * DIM, 2.0)
    cache = KvPair(KvType.F16, rng.vec((pos0 + 1) * hkv * DIM, 2.0),
                   rng.vec((pos0 + 1) * hkv * DIM, 3.0))
    with pytest.raises(BrasaError) as e:
        run_decode(k, "lanes", q, cache, hq, hkv, pos0)
    assert e.value.code == 3
    _say("decode per_head group=3")
    got = run_decode(k, "per_head", q, cache, hq, hkv, pos0)
    want, vmax = oracle.attention(q, cache.k, cache.v, 1, hq, hkv, DIM, pos0)
    assert oracle.worst(got, want, vmax) <= 1e-5


@pytest.mark.parametrize("kv", KVS)
def test_decode_launch_seed78_and_determinism(kv):
    k = Kernels()
    rng = oracle.Rng(78)
    for lk in [1, 37, 300, 1025]:
        n = ((lk + 127) // 128 * 128) * HKV * DIM
        cache = KvPair(kv, rng.vec(n, 2.0), rng.vec(n, 3.0))
        q = rng.vec(HQ * DIM, 2.0)
        _say(f"decode seed78 kv={kv.name_str} lk={lk}")
        a = run_decode(k, "lanes", q, cache, HQ, HKV, lk - 1)
        b = run_decode(k, "lanes", q, cache, HQ, HKV, lk - 1)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # the same bits from scratch holding garbage and through the batched entry point with
        # one sequence (launch.rs:119-168: no launch choice changes the result)
        gq = DeviceBuffer.from_array(q)
        part = DeviceBuffer.from_array(np.full(decode_partials_len(HQ, lk), np.nan, np.float32))
        o = DeviceBuffer(HQ * DIM * 4)
        k.decode_attention_batch(gq, [cache.kbuf], [cache.vbuf], [lk], part, o, HQ, HKV, kv)
        synchronize()
        c = o.download(np.float32).reshape(HQ, DIM)
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        want, vmax = oracle.attention(q, cache.k[: lk * HKV * DIM], cache.v[: lk * HKV * DIM],
                                      1, HQ, HKV, DIM, lk - 1)
        assert oracle.worst(a, want, vmax) <= 1e-5


def test_decode_f16_output_is_rne_of_f32_output():
    k = Kernels()
    rng = oracle.Rng(31)
    pos0 = 5000
    q = rng.vec(HQ * DIM, 2.0)
    cache = KvPair(KvType.F16, rng.vec((pos0 + 1) * HKV * DIM, 2.0),
                   rng.vec((pos0 + 1) * HKV * DIM, 3.0))
    _say("decode f16 output")
    o32 = run_decode(k, "lanes", q, cache, HQ, HKV, pos0)
    o16 = run_decode(k, "lanes", q, cache, HQ, HKV, pos0, out=OutDType.F16)
    assert np.array_equal(o16, oracle.f32_to_f16(o32))


def test_decode_scratch_too_small():
    k = Kernels()
    cache = KvPair(KvType.F16, np.zeros(300 * HKV * DIM, np.float32),
                   np.zeros(300 * HKV * DIM, np.float32))
    q = DeviceBuffer(HQ * DIM * 4)
    o = DeviceBuffer(HQ * DIM * 4)
    part = DeviceBuffer(4 * (decode_partials_len(HQ, 300) - 1))
    with pytest.raises(BrasaError) as e:
        k.decode_attention_lanes(q, cache.kbuf, cache.vbuf, part, o,
                                 AttnShape(1, HQ, HKV, DIM, 299, KvType.F16))
    assert e.value.code == 2


@pytest.mark.parametrize("vscale", [40.0, 3e3, 2.7e6])
def test_decode_q8_large_v_scales(vscale):
    """q8_0 V groups with scales from ~1 up to ~6.4e4 (near the f16 maximum): the part of a scale
    above 2^5 stays in the factor folded into P, which must neither overflow f16 nor lose
    precision; the result holds the 1e-5 bar relative to max|v|."""
    k = Kernels()
    rng = oracle.Rng(58)
    for pos0 in [300, 4095]:
        lk = pos0 + 1
        q = rng.vec(HQ * DIM, 2.0)
        kv_k = rng.vec(lk * HKV * DIM, 2.0)
        kv_v = rng.vec(lk * HKV * DIM, 3.0) * np.float32(vscale)
        cache = KvPair(KvType.Q8_0, kv_k, kv_v)
        assert np.isfinite(cache.v).all()
        _say(f"decode q8 large V scales {vscale} pos0={pos0}")
        got = run_decode(k, "lanes", q, cache, HQ, HKV, pos0)
        want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, pos0)
        w = oracle.worst(got, want, vmax)
        print(f"q8 V scale {vscale} pos0 {pos0}: max |v| {np.abs(cache.v).max():.3g}, worst {w:.2e}")
        assert w <= 1e-5, w


@pytest.mark.parametrize("vscale", [1e-3, 1e-4, 3e-6])
def test_decode_q8_small_scales(vscale):
    """q8_0 caches whose group scales are small or f16-subnormal (|v| ~ vscale): the dequantised
    products must stay at the reference's bar relative to max|v| (attention.rs:25-32), which
    rules out rounding p * scale into an f16 subnormal."""
    k = Kernels()
    rng = oracle.Rng(57)
    for pos0 in [300, 4095]:
        lk = pos0 + 1
        q = rng.vec(HQ * DIM, 2.0)
        kv_k = rng.vec(lk * HKV * DIM, 2.0) * np.float32(vscale)
        kv_v = rng.vec(lk * HKV * DIM, 3.0) * np.float32(vscale)
        cache = KvPair(KvType.Q8_0, kv_k, kv_v)
        _say(f"decode q8 small scales {vscale} pos0={pos0}")
        got = run_decode(k, "lanes", q, cache, HQ, HKV, pos0)
        want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, pos0)
        assert vmax.max() > 0  # scales 1e-4 / 3e-6 groups: f16-subnormal scales, nonzero V
        w = oracle.worst(got, want, vmax)
        print(f"q8 scale {vscale} pos0 {pos0}: worst {w:.2e}")
        assert w <= 1e-5, w


def test_decode_stream_without_counter_slot():
    """With all 64 counter slots of the device taken, a launch on another stream decodes with one
    split per head group (no merge, no counters): still at the reference's bar, and its result
    matches the split launch's to the decode tolerance. brasa_release_workspaces() frees the
    slots again."""
    import ctypes
    from brasa_amd.device import Stream
    k = Kernels()
    rng = oracle.Rng(64)
    pos0 = 4095
    q = rng.vec(HQ * DIM, 2.0)
    cache = KvPair(KvType.F16, rng.vec((pos0 + 1) * HKV * DIM, 2.0),
                   rng.vec((pos0 + 1) * HKV * DIM, 3.0))
    _say("decode on a stream without a counter slot")
    split = run_decode(k, "lanes", q, cache, HQ, HKV, pos0)
    s = ctypes.c_int()
    for i in range(64):  # fill every free slot of device 0 with stand-in stream keys
        assert lib().brasa_test_stream_slot(0, 0x7000 + 16 * i, ctypes.byref(s)) == 0
    try:
        st = Stream()
        assert lib().brasa_test_stream_slot(0, st.handle, ctypes.byref(s)) == 0
        assert s.value == -1
        gq = DeviceBuffer.from_array(q)
        part = DeviceBuffer(4 * decode_partials_len(HQ, pos0 + 1))
        o = DeviceBuffer(HQ * DIM * 4)
        k.decode_attention_lanes(gq, cache.kbuf, cache.vbuf, part, o,
                                 AttnShape(1, HQ, HKV, DIM, pos0, KvType.F16), stream=st)
        st.synchronize()
        got = o.download(np.float32).reshape(HQ, DIM)
    finally:
        synchronize()
        assert lib().brasa_release_workspaces() == 0
    want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, pos0)
    assert oracle.worst(got, want, vmax) <= 1e-5
    assert np.max(np.abs(got - split)) <= 1e-5 * float(vmax.max())


def stepped_scores(rng: np.random.Generator, lk: int, hq: int = HQ, hkv: int = HKV):
    """Q / K / V whose scores jump between levels from one 32-key block to the next.

    Every KV head has a unit direction d; K row j = 68 level(j // 32) d + noise with level in
    {0, 1, 2, 3}, and query head h of that KV head is (1 + h % 4) d, so its scores sit near
    6 (1 + h % 4) level nats. A wave whose next block is one level up sees its max grow by
    ~8.7 log2 units (head factor 1) up to ~35 (factor 4): the lazy rescale of the running sum
    runs after the first block, with a different factor for each query head of a group, and
    the rescaled old part of the sum still weighs ~2^-8.7 for the factor-1 heads, so a wrong
    factor shows far above the 1e-5 bar."""
    g = hq // hkv
    d = rng.standard_normal((hkv, DIM)).astype(np.float32)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    level = rng.integers(0, 4, size=(lk + 31) // 32).astype(np.float32)
    lev = np.repeat(level, 32)[:lk]
    k = 68.0 * lev[:, None, None] * d[None] + 0.05 * rng.standard_normal((lk, hkv, DIM))
    v = rng.standard_normal((lk, hkv, DIM))
    q = np.stack([(1 + h % 4) * d[h // g] for h in range(hq)])
    return (q.astype(np.float32).reshape(-1), k.astype(np.float32).reshape(-1),
            v.astype(np.float32).reshape(-1))


@pytest.mark.parametrize("kv", KVS)
def test_decode_rescale_after_first_block(kv):
    """Scores that jump by 2^8.7 and more between blocks (stepped_scores): every kernel's lazy
    rescale runs inside splits, once per query head with that head's own factor. The q8_0
    group-4 kernel once scaled all four heads' accumulators by the lane's own head factor:
    with these inputs that was 1.3e-4 max|v| off at pos0 700 (and 1.8 max|v| on one head group
    of the seeded ragged batch once its keys were taken in another order)."""
    k = Kernels()
    rng = np.random.default_rng(91)
    for pos0 in [700, 4095, 16383]:
        q, kk, vv = stepped_scores(rng, pos0 + 1)
        cache = KvPair(kv, kk, vv)
        _say(f"decode rescale kv={kv.name_str} pos0={pos0}")
        got = run_decode(k, "lanes", q, cache, HQ, HKV, pos0)
        want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, pos0)
        w = oracle.worst(got, want, vmax)
        print(f"decode rescale KV {kv.name_str} pos0 {pos0}: worst / max|v| = {w:.2e}")
        assert w <= 1e-5, w


@pytest.mark.parametrize("kv", KVS)
@pytest.mark.parametrize("hq,hkv,variant", [(32, 32, "lanes"), (32, 16, "lanes"), (64, 8, "lanes"),
                                            (32, 8, "per_head")])
def test_decode_rescale_other_groups(kv, hq, hkv, variant):
    """stepped_scores at GQA groups 1, 2 and 8 (the generic q8_0 kernel, other head-group
    layouts) and through the per-head decode_attention: the reference's 1e-5 bar."""
    k = Kernels()
    rng = np.random.default_rng(95)
    pos0 = 4095
    q, kk, vv = stepped_scores(rng, pos0 + 1, hq, hkv)
    cache = KvPair(kv, kk, vv)
    _say(f"decode rescale kv={kv.name_str} hq={hq} hkv={hkv} {variant}")
    got = run_decode(k, variant, q, cache, hq, hkv, pos0)
    want, vmax = oracle.attention(q, cache.k, cache.v, 1, hq, hkv, DIM, pos0)
    w = oracle.worst(got, want, vmax)
    print(f"decode rescale KV {kv.name_str} hq {hq} hkv {hkv} {variant}: worst / max|v| = {w:.2e}")
    assert w <= 1e-5, w
