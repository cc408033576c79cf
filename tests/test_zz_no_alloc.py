"""GPU: brasa_decode_attention_lanes_noalloc (split partials in the library's fixed device array)
gives the same bits as brasa_decode_attention_lanes with caller scratch, on two calls in a row,
the second one smaller (the array keeps the first call's contents)."""
import numpy as np
import pytest

import oracle
from brasa_amd import AttnShape, Kernels, KvType, OutDType, decode_partials_len
from brasa_amd.device import DeviceBuffer, synchronize
from gpu_util import DIM, HKV, HQ, KvPair

pytestmark = pytest.mark.gpu


def _both(k, q, cache, pos0, out):
    lk = pos0 + 1
    shape = AttnShape(1, HQ, HKV, DIM, pos0, cache.kv)
    gq = DeviceBuffer.from_array(q)
    nbytes = HQ * DIM * (4 if out == OutDType.F32 else 2)
    o_ref, o_na = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    part = DeviceBuffer(4 * decode_partials_len(HQ, lk))
    k.decode_attention_lanes(gq, cache.kbuf, cache.vbuf, part, o_ref, shape, out=out)
    k.decode_attention_lanes_noalloc(gq, cache.kbuf, cache.vbuf, o_na, shape, out=out)
    synchronize()
    dt = np.float32 if out == OutDType.F32 else np.uint16
    return o_ref.download(dt), o_na.download(dt)


@pytest.mark.parametrize("kv", [KvType.F16, KvType.Q8_0])
def test_noalloc_matches_scratch_entry_point(kv):
    k = Kernels()
    rng = oracle.Rng(91)
    for pos0, out in [(16383, OutDType.F32), (700, OutDType.F16)]:
        lk = pos0 + 1
        print(f"noalloc kv={kv.name_str} pos0={pos0} out={out.name}", flush=True)
        q = rng.vec(HQ * DIM, 2.0)
        cache = KvPair(kv, rng.vec(lk * HKV * DIM, 2.0), rng.vec(lk * HKV * DIM, 3.0))
        ref, got = _both(k, q, cache, pos0, out)
        assert np.array_equal(ref.view(np.uint32 if ref.dtype == np.float32 else np.uint16),
                              got.view(np.uint32 if got.dtype == np.float32 else np.uint16))
        if out == OutDType.F32:
            want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, pos0)
            assert oracle.worst(got.reshape(HQ, DIM), want, vmax) <= 1e-5


@pytest.mark.parametrize("hq,hkv", [(32, 32), (32, 4), (16, 8)])
def test_noalloc_other_groups(hq, hkv):
    """Other GQA groups (1, 8, 2): the no-allocation call gives the scratch call's bits, twice
    in a row with the second call smaller, and holds the reference's bar."""
    k = Kernels()
    rng = oracle.Rng(92)
    for pos0 in [9000, 300]:
        lk = pos0 + 1
        print(f"noalloc hq={hq} hkv={hkv} pos0={pos0}", flush=True)
        q = rng.vec(hq * DIM, 2.0)
        cache = KvPair(KvType.F16, rng.vec(lk * hkv * DIM, 2.0), rng.vec(lk * hkv * DIM, 3.0))
        shape = AttnShape(1, hq, hkv, DIM, pos0, KvType.F16)
        gq = DeviceBuffer.from_array(q)
        o_ref, o_na = DeviceBuffer(hq * DIM * 4), DeviceBuffer(hq * DIM * 4)
        part = DeviceBuffer(4 * decode_partials_len(hq, lk))
        k.decode_attention_lanes(gq, cache.kbuf, cache.vbuf, part, o_ref, shape)
        k.decode_attention_lanes_noalloc(gq, cache.kbuf, cache.vbuf, o_na, shape)
        synchronize()
        ref, got = o_ref.download(np.float32), o_na.download(np.float32)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
        want, vmax = oracle.attention(q, cache.k, cache.v, 1, hq, hkv, DIM, pos0)
        assert oracle.worst(got.reshape(hq, DIM), want, vmax) <= 1e-5
