"""GPU: the attention entry points through KvCache views, as Qwen3::encode_layer uses them
(qwen3.rs:554-556, 592, 603): blocks are written at ``at(li, pos)`` by store_kv, decode and
prefill read ``layer(li)``. Every layer holds different data, so a wrong view offset shows as a
mismatch against the f64 oracle on that layer's values (bar: worst <= 1e-5 * max|v|,
attention.rs:25-32, for decode; F32 prefill likewise).
"""
import numpy as np
import pytest

import oracle
from brasa_amd import AttnShape, KvCache, Kernels, KvType, OutDType, PrefillPrecision, decode_partials_len
from brasa_amd.device import DeviceBuffer, synchronize
from gpu_util import DIM, HKV, HQ, seen_values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv", [KvType.F16, KvType.Q8_0])
def test_cache_views_decode_and_prefill(kv):
    k = Kernels()
    layers, ctx = 3, 200
    cache = KvCache(kv, layers, ctx, HKV)
    rng = oracle.Rng(61)
    kvd = HKV * DIM
    lk = 150
    seen = {}
    for li in range(layers):
        kvals = rng.vec(lk * kvd, 2.0)
        vvals = rng.vec(lk * kvd, 3.0)
        # two blocks per layer, written at their positions like the per-step cache writes
        for p0, p1 in [(0, 100), (100, lk)]:
            ks, vs = (DeviceBuffer.from_array(x[p0 * kvd:p1 * kvd]) for x in (kvals, vvals))
            kd, vd = cache.at(li, p0)
            k.store_kv(kv, ks, kd, (p1 - p0) * kvd)
            k.store_kv(kv, vs, vd, (p1 - p0) * kvd)
        synchronize()
        kb = cache.k.download(np.uint8, kv.bytes(lk * kvd), kv.bytes(li * cache.cap * kvd))
        vb = cache.v.download(np.uint8, kv.bytes(lk * kvd), kv.bytes(li * cache.cap * kvd))
        seen[li] = (seen_values(kv, kb), seen_values(kv, vb))
    for li in range(layers):
        kl, vl = cache.layer(li)
        print(f"kvcache kv={kv.name_str} layer {li}", flush=True)
        q = rng.vec(HQ * DIM, 2.0)
        part = DeviceBuffer(4 * decode_partials_len(HQ, lk))
        o = DeviceBuffer(4 * HQ * DIM)
        k.decode_attention_lanes(DeviceBuffer.from_array(q), kl, vl, part, o,
                                 AttnShape(1, HQ, HKV, DIM, lk - 1, kv), OutDType.F32)
        synchronize()
        want, vmax = oracle.attention(q, *seen[li], 1, HQ, HKV, DIM, lk - 1)
        assert oracle.worst(o.download(np.float32).reshape(HQ, DIM), want, vmax) <= 1e-5, li
        t, pos0 = 20, lk - 20
        qp = rng.vec(t * HQ * DIM, 2.0)
        op = DeviceBuffer(4 * t * HQ * DIM)
        k.flash_attention_with(DeviceBuffer.from_array(qp), kl, vl, op,
                               AttnShape(t, HQ, HKV, DIM, pos0, kv), PrefillPrecision.F32)
        synchronize()
        want, vmax = oracle.attention(qp, *seen[li], t, HQ, HKV, DIM, pos0)
        assert oracle.worst(op.download(np.float32).reshape(t, HQ, DIM), want, vmax) <= 1e-5, li
    cache.free()
