"""GPU: the BASELINE.json configurations at their full sizes, on seeded N(0, 1) inputs.

Inputs: numpy PCG64 ``default_rng(seed)``; seed s -> Q, s + 1 -> K, s + 2 -> V; values drawn in
f32 and rounded to f16 (Q is passed as f32 holding those f16 values, as the reference's decode
and prefill take f32 Q). Q8 caches quantise the f32 draws. Prefill inputs are put through
per-head RMSNorm (weight 1, eps 1e-6) and RoPE-NeoX (theta 1e6) first.

Decode is checked in full against the oracle (the reference's 1e-5 * max|v| bar). Prefill at
T = 2048 / 8192 and the 512-token chunk at pos0 = 16384 is checked on one query row of every
32-row tile (a seeded offset in each tile, all 32 heads; the oracle computes exactly those rows)
with the BASELINE.json bar; F16_PF32 at T = 2048 the same way at the reference's 1e-5 bar.
"""
import numpy as np
import pytest

import oracle
from brasa_amd import AttnShape, Kernels, KvType, PrefillPrecision, decode_partials_len
from brasa_amd.device import DeviceBuffer, synchronize
from gpu_util import DIM, HKV, HQ, KvPair, bars, f16_normal, post_norm_rope

# worst_f16 (attention.rs:12-23: error over max|v|, the f16 output rounding discounted) that the
# F16 hot path (P rounded to f16 for the matrix cores; q8_0 values as f16(code * scale)) holds at
# the BASELINE.json prefill configurations, measured 7.1e-5 / 8.0e-5 / 2.7e-6 (f16: T 2048,
# 8192, 512 at 16384) and 4.0e-4 / 5.0e-6 (q8_0: T 2048, 512 at 16384), held with ~1.3-1.5x
# margin (deterministic results). The reference's F16 kernel keeps P in f32 and reads q8_0 values
# exactly and is held to 1e-5 (attention.rs:99-104); F16_PF32 is held to that here.
F16_WORST_BOUND = 1.2e-4
Q8_F16_WORST_BOUND = 6e-4

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("kv,lk", [(KvType.F16, 2048), (KvType.F16, 4096), (KvType.F16, 16384),
                                   (KvType.F16, 32768), (KvType.Q8_0, 16384)])
def test_decode_config(kv, lk):
    seed = 1000 + lk + int(kv)
    q = f16_normal(np.random.default_rng(seed), HQ * DIM)
    if kv == KvType.F16:
        kk = f16_normal(np.random.default_rng(seed + 1), lk * HKV * DIM)
        vv = f16_normal(np.random.default_rng(seed + 2), lk * HKV * DIM)
    else:
        kk = np.random.default_rng(seed + 1).standard_normal(lk * HKV * DIM, dtype=np.float32)
        vv = np.random.default_rng(seed + 2).standard_normal(lk * HKV * DIM, dtype=np.float32)
    cache = KvPair(kv, kk, vv)
    gq = DeviceBuffer.from_array(q)
    part = DeviceBuffer(4 * decode_partials_len(HQ, lk))
    o = DeviceBuffer(HQ * DIM * 4)
    _say(f"decode config kv={kv.name_str} lk={lk}")
    Kernels().decode_attention_lanes(gq, cache.kbuf, cache.vbuf, part, o,
                                     AttnShape(1, HQ, HKV, DIM, lk - 1, kv))
    synchronize()
    got = o.download(np.float32).reshape(1, HQ, DIM)
    want, vmax = oracle.attention(q, cache.k, cache.v, 1, HQ, HKV, DIM, lk - 1)
    w = oracle.worst(got, want, vmax)
    a, r = bars(got, want)
    print(f"decode kv={kv.name_str} lk={lk}: worst {w:.2e} max-abs {a:.2e} max-rel {r:.2e}")
    assert w <= 1e-5 and a <= 2e-3 and r <= 1e-2


def _prefill_inputs(tokens, pos0, seed):
    lk = pos0 + tokens
    cap = (lk + 63) // 64 * 64
    c, s = oracle.rope_table(1e6, DIM, cap)
    q = oracle.round_f16(post_norm_rope(
        np.random.default_rng(seed).standard_normal(tokens * HQ * DIM, dtype=np.float32),
        tokens, HQ, pos0, c, s))
    # the cache holds positions 0..cap: RMSNorm + RoPE at their own positions
    k = oracle.round_f16(post_norm_rope(
        np.random.default_rng(seed + 1).standard_normal(cap * HKV * DIM, dtype=np.float32),
        cap, HKV, 0, c, s))
    v = f16_normal(np.random.default_rng(seed + 2), cap * HKV * DIM)
    return q, k, v


def _tile_rows(tokens, seed):
    """One query row from every 32-row tile (a seeded offset inside each tile), plus the last."""
    rng = np.random.default_rng(seed)
    rows = [t0 + int(rng.integers(0, min(32, tokens - t0))) for t0 in range(0, tokens, 32)]
    return sorted(set(rows + [tokens - 1]))


def _oracle_rows(q, cache, tokens, pos0, rows):
    """The oracle's q16 attention (reference.rs:129-145) for the given query rows, every head:
    row t is the one-token problem at absolute position pos0 + t (it sees keys [0, pos0 + t]),
    so rows are computed independently, on several host threads."""
    from concurrent.futures import ThreadPoolExecutor
    qr = np.asarray(q, np.float32).reshape(tokens, HQ, DIM)

    def one(t):
        o, vm = oracle.attention(qr[t], cache.k, cache.v, 1, HQ, HKV, DIM, pos0 + t, q16=True)
        return o[0], vm[0]

    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(one, rows))
    return np.stack([r[0] for r in res]), np.stack([r[1] for r in res])


@pytest.mark.parametrize("tokens,pos0", [(2048, 0), (8192, 0), (512, 16384)])
def test_prefill_config(tokens, pos0):
    q, kk, vv = _prefill_inputs(tokens, pos0, 2000 + tokens + pos0)
    cache = KvPair(KvType.F16, kk, vv)
    gq = DeviceBuffer.from_array(q)
    o = DeviceBuffer(tokens * HQ * DIM * 2)
    _say(f"prefill config T={tokens} pos0={pos0}")
    Kernels().flash_attention(gq, cache.kbuf, cache.vbuf, o,
                              AttnShape(tokens, HQ, HKV, DIM, pos0, KvType.F16))
    synchronize()
    got = oracle.f16_to_f32(o.download(np.uint16)).reshape(tokens, HQ, DIM)
    assert np.all(np.isfinite(got))
    rows = _tile_rows(tokens, tokens + pos0)
    _say(f"prefill config T={tokens} pos0={pos0}: oracle on {len(rows)} rows (one per tile)")
    want, vmax = _oracle_rows(q, cache, tokens, pos0, rows)
    a, r = bars(got[rows], want)
    w = oracle.worst_f16(o.download(np.uint16).reshape(tokens, HQ, DIM)[rows], want, vmax)
    print(f"prefill T={tokens} pos0={pos0}, {len(rows)} rows x {HQ} heads: max-abs {a:.2e} "
          f"max-rel {r:.2e} worst_f16 {w:.2e}")
    assert a <= 2e-3 and r <= 1e-2
    assert w <= F16_WORST_BOUND, w


def test_prefill_config_f16_pf32_2048():
    """The reference's own F16 numerics (P kept in f32, flash_attention.metal:197) at the
    BASELINE prefill size, every tile, at the reference's bar worst_f16 <= 1e-5
    (attention.rs:12-23, 99-104)."""
    tokens, pos0 = 2048, 0
    q, kk, vv = _prefill_inputs(tokens, pos0, 2000 + tokens + pos0)
    cache = KvPair(KvType.F16, kk, vv)
    gq = DeviceBuffer.from_array(q)
    o = DeviceBuffer(tokens * HQ * DIM * 2)
    _say("prefill config T=2048 F16_PF32")
    Kernels().flash_attention_with(gq, cache.kbuf, cache.vbuf, o,
                                   AttnShape(tokens, HQ, HKV, DIM, pos0, KvType.F16),
                                   PrefillPrecision.F16_PF32)
    synchronize()
    bits = o.download(np.uint16).reshape(tokens, HQ, DIM)
    rows = _tile_rows(tokens, 7)
    want, vmax = _oracle_rows(q, cache, tokens, pos0, rows)
    w = oracle.worst_f16(bits[rows], want, vmax)
    print(f"prefill T=2048 F16_PF32, {len(rows)} rows: worst_f16 {w:.2e}")
    assert w <= 1e-5


def test_prefill_config_q8_chunk():
    tokens, pos0 = 256, 4096
    q, kk, vv = _prefill_inputs(tokens, pos0, 77)
    cache = KvPair(KvType.Q8_0, kk, vv)
    gq = DeviceBuffer.from_array(q)
    o = DeviceBuffer(tokens * HQ * DIM * 2)
    _say("prefill q8 chunk")
    Kernels().flash_attention(gq, cache.kbuf, cache.vbuf, o,
                              AttnShape(tokens, HQ, HKV, DIM, pos0, KvType.Q8_0))
    synchronize()
    got = oracle.f16_to_f32(o.download(np.uint16)).reshape(tokens, HQ, DIM)
    want, _ = oracle.attention(q, cache.k, cache.v, tokens, HQ, HKV, DIM, pos0, q16=True,
                               rows=(tokens - 8, tokens))
    a, r = bars(got[-8:], want[-8:])
    assert a <= 2e-3 and r <= 1e-2


@pytest.mark.parametrize("tokens,pos0", [(2048, 0), (512, 16384)])
def test_prefill_config_q8_every_tile(tokens, pos0):
    """q8_0 KV cache (quantised from the same post-RMSNorm / RoPE draws), F16 precision: one row
    of every query tile against the q16 oracle over the dequantised cache."""
    q, kk, vv = _prefill_inputs(tokens, pos0, 3000 + tokens + pos0)
    cache = KvPair(KvType.Q8_0, kk, vv)
    gq = DeviceBuffer.from_array(q)
    o = DeviceBuffer(tokens * HQ * DIM * 2)
    _say(f"prefill config q8 T={tokens} pos0={pos0}")
    Kernels().flash_attention(gq, cache.kbuf, cache.vbuf, o,
                              AttnShape(tokens, HQ, HKV, DIM, pos0, KvType.Q8_0))
    synchronize()
    got = oracle.f16_to_f32(o.download(np.uint16)).reshape(tokens, HQ, DIM)
    rows = _tile_rows(tokens, 5 + tokens)
    want, vmax = _oracle_rows(q, cache, tokens, pos0, rows)
    a, r = bars(got[rows], want)
    w = oracle.worst_f16(o.download(np.uint16).reshape(tokens, HQ, DIM)[rows], want, vmax)
    print(f"prefill q8 T={tokens} pos0={pos0}, {len(rows)} rows: max-abs {a:.2e} max-rel {r:.2e} "
          f"worst_f16 {w:.2e}")
    assert a <= 2e-3 and r <= 1e-2
    assert w <= Q8_F16_WORST_BOUND, w

