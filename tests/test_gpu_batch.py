"""GPU: ragged batched decode (one launch for many sequences) against the f64 oracle.

The reference decodes one sequence per call (crates/kernels/src/lib.rs:1110-1164); its mixed
workload batches 8 sequences with seeded lengths U[1024, 16384]. Every
sequence of a batch must meet the reference's decode bar (worst <= 1e-5 * max|v|,
tests/attention.rs:25-32) on its own inputs.
"""
import numpy as np
import pytest

import oracle
from brasa_amd import Kernels, KvType, OutDType, decode_batch_partials_len
from brasa_amd.device import DeviceBuffer, synchronize
from gpu_util import DIM, HKV, HQ, KvPair

pytestmark = pytest.mark.gpu


def run_batch(k, kv, lens, seed, out=OutDType.F32, hq=HQ, hkv=HKV):
    rng = oracle.Rng(seed)
    qs, caches = [], []
    for lk in lens:
        qs.append(rng.vec(hq * DIM, 2.0))
        caches.append(KvPair(kv, rng.vec(lk * hkv * DIM, 2.0), rng.vec(lk * hkv * DIM, 3.0)))
    q = DeviceBuffer.from_array(np.concatenate(qs))
    part = DeviceBuffer(4 * decode_batch_partials_len(hq, lens))
    esz = 4 if out == OutDType.F32 else 2
    o = DeviceBuffer(len(lens) * hq * DIM * esz)
    print(f"batch kv={kv.name_str} n={len(lens)} seed={seed}", flush=True)
    k.decode_attention_batch(q, [c.kbuf for c in caches], [c.vbuf for c in caches], lens, part,
                             o, hq, hkv, kv, out)
    synchronize()
    got = o.download(np.float32 if out == OutDType.F32 else np.uint16).reshape(len(lens), -1)
    return qs, caches, got


@pytest.mark.parametrize("kv", [KvType.F16, KvType.Q8_0])
def test_ragged_batch_config(kv):
    lens = [int(x) for x in np.random.default_rng(12345).integers(1024, 16385, size=8)]
    k = Kernels()
    qs, caches, got = run_batch(k, kv, lens, 41)
    w = 0.0
    for i, lk in enumerate(lens):
        want, vmax = oracle.attention(qs[i], caches[i].k, caches[i].v, 1, HQ, HKV, DIM, lk - 1)
        w = max(w, oracle.worst(got[i], want, vmax))
    print(f"ragged batch KV {kv.name_str} lens {lens}: worst / max|v| = {w:.2e}")
    assert w <= 1e-5, w


def test_batch_mixed_short_and_many_sequences():
    """70 sequences (more than one launch's worth), lengths from 1 to 3000, including sequences
    that fit in one split next to sequences that need several; f16 output."""
    lens = [1, 2, 37, 64, 65, 127, 128, 129, 300, 1025, 3000] * 6 + [5, 999, 2048, 17]
    k = Kernels()
    qs, caches, got = run_batch(k, KvType.F16, lens, 43, out=OutDType.F16)
    for i, lk in enumerate(lens):
        want, _ = oracle.attention(qs[i], caches[i].k, caches[i].v, 1, HQ, HKV, DIM, lk - 1)
        got_f = oracle.f16_to_f32(got[i])
        # f16 output: max-abs 2e-3 (the fp16 bar), i.e. the f32 result rounded once to f16
        assert np.max(np.abs(got_f - want.reshape(-1))) <= 2e-3, (i, lk)


@pytest.mark.parametrize("group", [1, 2, 8])
def test_batch_other_groups(group):
    hkv = 4
    hq = hkv * group
    lens = [700, 33, 2500]
    k = Kernels()
    qs, caches, got = run_batch(k, KvType.F16, lens, 47, hq=hq, hkv=hkv)
    for i, lk in enumerate(lens):
        want, vmax = oracle.attention(qs[i], caches[i].k, caches[i].v, 1, hq, hkv, DIM, lk - 1)
        assert oracle.worst(got[i], want, vmax) <= 1e-5


@pytest.mark.parametrize("kv", [KvType.F16, KvType.Q8_0])
def test_ragged_batch_rescale_after_first_block(kv):
    """The ragged batch (four adjacent KV heads per workgroup) on inputs whose scores jump
    between blocks (test_gpu_decode.stepped_scores): rescales inside splits with a different
    factor per query head."""
    from test_gpu_decode import stepped_scores
    lens = [int(x) for x in np.random.default_rng(12345).integers(1024, 16385, size=8)]
    rng = np.random.default_rng(92)
    data = [stepped_scores(rng, lk) for lk in lens]
    caches = [KvPair(kv, kk, vv) for _, kk, vv in data]
    q = DeviceBuffer.from_array(np.concatenate([d[0] for d in data]))
    part = DeviceBuffer(4 * decode_batch_partials_len(HQ, lens))
    o = DeviceBuffer(len(lens) * HQ * DIM * 4)
    k = Kernels()
    print(f"batch rescale kv={kv.name_str}", flush=True)
    k.decode_attention_batch(q, [c.kbuf for c in caches], [c.vbuf for c in caches], lens, part,
                             o, HQ, HKV, kv, OutDType.F32)
    synchronize()
    got = o.download(np.float32).reshape(len(lens), -1)
    w = 0.0
    for i, lk in enumerate(lens):
        want, vmax = oracle.attention(data[i][0], caches[i].k, caches[i].v, 1, HQ, HKV, DIM, lk - 1)
        w = max(w, oracle.worst(got[i], want, vmax))
    print(f"ragged batch rescale KV {kv.name_str}: worst / max|v| = {w:.2e}")
    assert w <= 1e-5, w
