"""GPU: the attention entry points captured into HIP graphs and replayed.

The library's launch state survives replays: the split merges' arrival counters return to zero
in every launch, the prefill workspace is a fixed array, and the q8_0 range flag is cleared by
the launch that reads it. Each case captures one call on a stream, then replays the graph
several times, with new inputs uploaded between replays, other eager calls on the same and on
another stream in between, and back-to-back replays with no synchronisation; after every replay
the graph's output must equal, bit for bit, the eager call on the same inputs (which the other
GPU tests check against the oracle). No graph here records a memset node: the library enqueues
kernels only.
"""
import numpy as np
import pytest

from brasa_amd import (AttnShape, Kernels, KvType, OutDType, PrefillPrecision,
                       decode_batch_partials_len, decode_partials_len)
from brasa_amd._lib import lib
from brasa_amd.device import DeviceBuffer, Graph, Stream, synchronize
from gpu_util import DIM, HKV, HQ, KvPair, cache_bytes, f16_normal

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _release_after():
    """The streams of each test are destroyed after it: hand their counter slots and the fixed
    prefill workspace back first, as the header asks before stream handles can be reused."""
    yield
    synchronize()
    assert lib().brasa_release_workspaces() == 0


def _say(msg):
    print(msg, flush=True)


def _replay_and_compare(name, s, run, set_inputs, og, oe, variants):
    """run(stream, out) enqueues the op writing `out`; set_inputs(i) uploads input variant i."""
    other = Stream()
    set_inputs(variants[0])
    with Graph.capture(s) as g:
        run(s, og)
    for rep, i in enumerate(variants):
        _say(f"graph {name}: replay {rep} inputs {i}")
        s.synchronize()
        set_inputs(i)
        g.launch(s)
        s.synchronize()
        got = og.download(np.uint8).copy()
        run(other, oe)                   # eager on another stream (its own slot)
        other.synchronize()
        run(s, oe)                       # eager, same stream, same slot
        s.synchronize()
        want = oe.download(np.uint8)
        assert np.array_equal(got, want), f"{name}: replay {rep} differs from the eager call"
    # back-to-back replays without a wait, then one check
    for _ in range(4):
        g.launch(s)
    s.synchronize()
    run(s, oe)
    s.synchronize()
    assert np.array_equal(og.download(np.uint8), oe.download(np.uint8)), f"{name}: back-to-back"


@pytest.mark.parametrize("kv,lk", [(KvType.F16, 16384), (KvType.F16, 4096), (KvType.Q8_0, 16384),
                                   (KvType.F32, 3000)])
def test_graph_decode(kv, lk):
    k = Kernels()
    rng = np.random.default_rng(7000 + lk)
    qs = [f16_normal(rng, HQ * DIM) for _ in range(3)]
    raw = [(cache_bytes(kv, f16_normal(rng, lk * HKV * DIM)),
            cache_bytes(kv, f16_normal(rng, lk * HKV * DIM))) for _ in range(2)]
    kbuf = DeviceBuffer(raw[0][0].nbytes)
    vbuf = DeviceBuffer(raw[0][1].nbytes)
    gq = DeviceBuffer(HQ * DIM * 4)
    part = DeviceBuffer(4 * decode_partials_len(HQ, lk))
    og, oe = DeviceBuffer(HQ * DIM * 4), DeviceBuffer(HQ * DIM * 4)
    shape = AttnShape(1, HQ, HKV, DIM, lk - 1, kv)

    def set_inputs(i):
        gq.upload(qs[i % 3])
        kb, vb = raw[i // 3]
        kbuf.upload(kb)
        vbuf.upload(vb)

    def run(stream, out):
        k.decode_attention_lanes(gq, kbuf, vbuf, part, out, shape, stream=stream)

    # (the calls share `part`; they run one at a time, and every call rewrites what it reads)
    _replay_and_compare(f"decode kv={kv.name_str} lk={lk}", Stream(), run, set_inputs, og, oe,
                        [0, 1, 2, 3, 1, 0])


def test_graph_decode_noalloc_and_batch():
    k = Kernels()
    rng = np.random.default_rng(7100)
    lks = [11000, 3000, 16384]
    caches = [KvPair(KvType.F16, f16_normal(rng, n * HKV * DIM), f16_normal(rng, n * HKV * DIM))
              for n in lks]
    qs = [f16_normal(rng, len(lks) * HQ * DIM) for _ in range(2)]
    gq = DeviceBuffer(len(lks) * HQ * DIM * 4)
    part = DeviceBuffer(4 * decode_batch_partials_len(HQ, lks))
    ob = [DeviceBuffer(len(lks) * HQ * DIM * 2) for _ in range(2)]
    on = [DeviceBuffer(HQ * DIM * 4) for _ in range(2)]
    shape = AttnShape(1, HQ, HKV, DIM, lks[2] - 1, KvType.F16)

    def set_inputs(i):
        gq.upload(qs[i])

    def run_batch(stream, out):
        k.decode_attention_batch(gq, [c.kbuf for c in caches], [c.vbuf for c in caches], lks,
                                 part, out, HQ, HKV, KvType.F16, out=OutDType.F16, stream=stream)

    def run_noalloc(stream, out):
        k.decode_attention_lanes_noalloc(gq, caches[2].kbuf, caches[2].vbuf, out, shape,
                                         stream=stream)

    _replay_and_compare("decode batch", Stream(), run_batch, set_inputs, ob[0], ob[1], [0, 1, 0])
    # (the no-allocation decode shares one device array; the helper runs one call at a time)
    _replay_and_compare("decode noalloc", Stream(), run_noalloc, set_inputs, on[0], on[1],
                        [0, 1, 1, 0])


@pytest.mark.parametrize("kv,tokens,pos0", [(KvType.F16, 512, 0), (KvType.F16, 128, 8192),
                                            (KvType.Q8_0, 64, 0), (KvType.Q8_0, 384, 0)])
def test_graph_prefill(kv, tokens, pos0):
    k = Kernels()
    rng = np.random.default_rng(7200 + tokens + pos0)
    cap = (pos0 + tokens + 63) // 64 * 64
    qs = [f16_normal(rng, tokens * HQ * DIM) for _ in range(2)]
    kk = f16_normal(rng, cap * HKV * DIM)
    vv = f16_normal(rng, cap * HKV * DIM)
    raw = [(cache_bytes(kv, kk), cache_bytes(kv, vv))]
    if kv == KvType.Q8_0:
        # a cache whose K scales leave the f16 range: the range flag and the exact recompute
        raw.append((cache_bytes(kv, kk * np.float32(4e4)), cache_bytes(kv, vv)))
        qs[1] = qs[1] * np.float32(1e-4)
    gq = DeviceBuffer(tokens * HQ * DIM * 4)
    kbuf = DeviceBuffer(raw[0][0].nbytes)
    vbuf = DeviceBuffer(raw[0][1].nbytes)
    og, oe = DeviceBuffer(tokens * HQ * DIM * 2), DeviceBuffer(tokens * HQ * DIM * 2)
    shape = AttnShape(tokens, HQ, HKV, DIM, pos0, kv)

    def set_inputs(i):
        gq.upload(qs[i % 2])
        kb, vb = raw[min(i, len(raw) - 1)]
        kbuf.upload(kb)
        vbuf.upload(vb)

    def run(stream, out):
        k.flash_attention_with(gq, kbuf, vbuf, out, shape, PrefillPrecision.F16, stream=stream)

    variants = [0, 1, 0, 1, 0] if kv == KvType.Q8_0 else [0, 1, 0]
    _replay_and_compare(f"prefill kv={kv.name_str} T={tokens} pos0={pos0}", Stream(), run,
                        set_inputs, og, oe, variants)
