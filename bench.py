"""Benchmark of the attention hot path on one MI355X.

Metric: decode-attention µs/layer and HBM GB/s at 16K context; prefill-attention
TFLOP/s at 2K tokens. One step = decode attention for one token through 36 layers (Qwen3-4B),
each layer reading its own fp16 K/V cache of 16384 positions (36 distinct caches, 2.4 GB, so the
256 MB last-level cache cannot serve repeats), hq 32 / hkv 8 / head_dim 128. ``value`` is the
HBM bandwidth of that step: algorithmic bytes (2 * lk * hkv * 256 + |Q| + |O| per layer) over
the event-timed step. The other BASELINE.json configurations are reported beside it.

Inputs are synthetic N(0, 1) values generated on the device (fill_normal), stored in the cache
type by the library's own store_kv. Everything the timed region touches is resident in HBM
before it starts. The CPU baseline is the oracle's faithful restatement of the reference's
serial f64 attention (crates/kernels/src/reference.rs:150-218) timed on a bounded sample on this
host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from brasa_amd import (AttnShape, Kernels, KvType, OutDType, PrefillPrecision,  # noqa: E402
                       RopeTable,
                       decode_batch_partials_len,
                       decode_partials_len)  # noqa: E402
from brasa_amd.device import (DeviceBuffer, Event, Stream, device_name, fill_normal,  # noqa: E402
                              synchronize)

HQ, HKV, DIM, LAYERS = 32, 8, 128, 36
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = "decode-attn µs/layer + HBM GB/s @16K ctx; prefill-attn TFLOP/s @2K tokens"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def decode_bytes(lk: int, kv: KvType) -> int:
    row = {KvType.F16: 256, KvType.Q8_0: 136, KvType.F32: 512}[kv]
    return 2 * lk * HKV * row + 2 * HQ * DIM * 4  # K + V + f32 Q + f32 O


def prefill_flops(tokens: int, pos0: int) -> float:
    # crates/kernels/benches/kernels.rs:206-208
    return 4.0 * HQ * DIM * (tokens * pos0 + tokens * (tokens + 1) / 2)


class DecodeLayers:
    """LAYERS distinct caches of lk positions, one Q/O, the partials scratch."""

    def __init__(self, k: Kernels, lk: int, kv: KvType, stream: Stream, seed: int = 1):
        self.lk, self.kv, self.k = lk, kv, k
        n = lk * HKV * DIM
        tmp = DeviceBuffer(4 * n)
        self.caches = []
        for layer in range(LAYERS):
            kb = DeviceBuffer(kv.bytes(n))
            vb = DeviceBuffer(kv.bytes(n))
            fill_normal(tmp, n, seed * 1000 + 2 * layer, 1.0, stream)
            k.store_kv(kv, tmp, kb, n, stream)
            fill_normal(tmp, n, seed * 1000 + 2 * layer + 1, 1.0, stream)
            k.store_kv(kv, tmp, vb, n, stream)
            self.caches.append((kb, vb))
        self.q = DeviceBuffer(4 * HQ * DIM)
        fill_normal(self.q, HQ * DIM, seed * 7919, 1.0, stream)
        self.o = DeviceBuffer(4 * HQ * DIM)
        self.part = DeviceBuffer(4 * decode_partials_len(HQ, lk))
        self.shape = AttnShape(1, HQ, HKV, DIM, lk - 1, kv)
        stream.synchronize()
        tmp.free()

    def step(self, stream: Stream) -> None:
        for kb, vb in self.caches:
            self.k.decode_attention_lanes(self.q, kb, vb, self.part, self.o, self.shape,
                                          OutDType.F32, stream)

    def free(self) -> None:
        for kb, vb in self.caches:
            kb.free()
            vb.free()
        self.caches = []


def time_steps(fn, stream: Stream, steps: int, warmup: int) -> float:
    """Seconds per step over `steps` timed steps (events on `stream`)."""
    for _ in range(warmup):
        fn(stream)
    stream.synchronize()
    synchronize()
    e0, e1 = Event(), Event()
    e0.record(stream)
    for _ in range(steps):
        fn(stream)
    e1.record(stream)
    e1.synchronize()
    synchronize()
    return e0.elapsed_ms(e1) / 1e3 / steps


def bench_decode(k, stream, lk, kv, steps, warmup):
    log(f"decode: building {LAYERS} caches kv={kv.name_str} lk={lk}")
    layers = DecodeLayers(k, lk, kv, stream)
    t = time_steps(layers.step, stream, steps, warmup)
    layers.free()
    per_layer = t / LAYERS
    gbs = decode_bytes(lk, kv) / per_layer / 1e9
    log(f"decode kv={kv.name_str} lk={lk}: {per_layer * 1e6:.2f} µs/layer, {gbs:.0f} GB/s")
    return {"us_per_layer": per_layer * 1e6, "us_36_layers": t * 1e6, "GBps": gbs,
            "bytes_per_layer": decode_bytes(lk, kv), "frac_hbm_peak": gbs / HBM_PEAK_GBS}, t


def bench_ragged(k, stream, steps, warmup, seed=12345):
    """8 sequences with seeded KV lengths U[1024, 16384], one query each. The reference has no
    batched decode API, so this is 8 calls in sequence on one stream."""
    lens = np.random.default_rng(seed).integers(1024, 16385, size=8)
    seqs = []
    for i, lk in enumerate(lens):
        n = int(lk) * HKV * DIM
        tmp = DeviceBuffer(4 * n)
        kb, vb = DeviceBuffer(2 * n), DeviceBuffer(2 * n)
        fill_normal(tmp, n, 500 + 2 * i, 1.0, stream)
        k.store_kv(KvType.F16, tmp, kb, n, stream)
        fill_normal(tmp, n, 501 + 2 * i, 1.0, stream)
        k.store_kv(KvType.F16, tmp, vb, n, stream)
        stream.synchronize()
        tmp.free()
        q = DeviceBuffer(4 * HQ * DIM)
        fill_normal(q, HQ * DIM, 900 + i, 1.0, stream)
        seqs.append((kb, vb, q, DeviceBuffer(4 * HQ * DIM),
                     DeviceBuffer(4 * decode_partials_len(HQ, int(lk))),
                     AttnShape(1, HQ, HKV, DIM, int(lk) - 1, KvType.F16)))

    def step(s):
        for kb, vb, q, o, part, shape in seqs:
            k.decode_attention_lanes(q, kb, vb, part, o, shape, OutDType.F32, s)

    t = time_steps(step, stream, steps, warmup)
    total = sum(decode_bytes(int(lk), KvType.F16) for lk in lens)
    log(f"ragged decode x8, sequential calls: {t * 1e6:.1f} µs, {total / t / 1e9:.0f} GB/s")

    # the same 8 sequences in one batched call
    qb = DeviceBuffer(4 * 8 * HQ * DIM)
    for i, (_, _, q, _, _, _) in enumerate(seqs):
        synchronize()
        qb.upload(q.download(np.float32), offset=4 * i * HQ * DIM)
    ob = DeviceBuffer(4 * 8 * HQ * DIM)
    pb = DeviceBuffer(4 * decode_batch_partials_len(HQ, lens))
    ks, vs = [x[0] for x in seqs], [x[1] for x in seqs]
    lks = [int(x) for x in lens]

    def step_b(s):
        k.decode_attention_batch(qb, ks, vs, lks, pb, ob, HQ, HKV, KvType.F16, OutDType.F32, s)

    tb = time_steps(step_b, stream, steps, warmup)
    log(f"ragged decode x8, one batched call: {tb * 1e6:.1f} µs, {total / tb / 1e9:.0f} GB/s")
    return {"lengths": lks, "bytes": total, "us_sequential": t * 1e6,
            "GBps_sequential": total / t / 1e9, "us_batched": tb * 1e6,
            "GBps_batched": total / tb / 1e9}


def sustained_calls(fn, stream: Stream, blocks: int = 15, per_block: int = 10) -> dict:
    """blocks x per_block back-to-back calls, one event pair per block (nothing waits between
    blocks): per-call µs of every block, their median and the last block's. Shows the rate once
    the clock has settled under continuous load."""
    stream.synchronize()
    evs = [Event() for _ in range(blocks + 1)]
    evs[0].record(stream)
    for b in range(blocks):
        for _ in range(per_block):
            fn(stream)
        evs[b + 1].record(stream)
    evs[-1].synchronize()
    per = [evs[b].elapsed_ms(evs[b + 1]) * 1e3 / per_block for b in range(blocks)]
    return {"calls": blocks * per_block, "us_median": float(np.median(per)),
            "us_last_block": per[-1], "us_blocks": [round(x, 2) for x in per]}


def bench_prefill(k, stream, tokens, pos0, kv, steps, warmup, seed=3,
                  precision=PrefillPrecision.F16, sustained=False):
    """Causal prefill of `tokens` queries at positions pos0.. over a cache of ceil64(pos0 +
    tokens) positions. As BASELINE.json config 4 describes the inputs: Q and K are N(0, 1) put
    through per-head RMSNorm (weight 1, eps 1e-6) and RoPE-NeoX (theta 1e6) at their positions
    by the library's own kernels, V is N(0, 1); K and V are stored in the cache type."""
    lk = pos0 + tokens
    cap = (lk + 63) // 64 * 64
    n = cap * HKV * DIM
    table = RopeTable(1e6, DIM, cap)
    ones = DeviceBuffer.from_array(np.ones(DIM, np.float32))
    tmp = DeviceBuffer(4 * n)
    kb, vb = DeviceBuffer(kv.bytes(n)), DeviceBuffer(kv.bytes(n))
    fill_normal(tmp, n, seed, 1.0, stream)
    k.rms_norm(tmp, ones, tmp, cap * HKV, DIM, 1e-6, stream)
    k.rope_neox(tmp, table, cap, HKV, DIM, 0, stream)
    k.store_kv(kv, tmp, kb, n, stream)
    fill_normal(tmp, n, seed + 1, 1.0, stream)
    k.store_kv(kv, tmp, vb, n, stream)
    q = DeviceBuffer(4 * tokens * HQ * DIM)
    fill_normal(q, tokens * HQ * DIM, seed + 2, 1.0, stream)
    k.rms_norm(q, ones, q, tokens * HQ, DIM, 1e-6, stream)
    k.rope_neox(q, table, tokens, HQ, DIM, pos0, stream)
    obytes = 4 if precision == PrefillPrecision.F32 else 2
    o = DeviceBuffer(obytes * tokens * HQ * DIM)
    stream.synchronize()
    tmp.free()
    shape = AttnShape(tokens, HQ, HKV, DIM, pos0, kv)
    t = time_steps(lambda s: k.flash_attention_with(q, kb, vb, o, shape, precision, s), stream,
                   steps, warmup)
    tf = prefill_flops(tokens, pos0) / t / 1e12
    log(f"prefill kv={kv.name_str} {precision.name} T={tokens} pos0={pos0}: {t * 1e6:.1f} µs, "
        f"{tf:.1f} TFLOP/s")
    out = {"us": t * 1e6, "TFLOPs": tf, "flop": prefill_flops(tokens, pos0),
           "frac_mfma_f16_peak": tf / MFMA_F16_PEAK_TFLOPS}
    if sustained:
        sus = sustained_calls(lambda s: k.flash_attention_with(q, kb, vb, o, shape, precision, s),
                              stream)
        sus["TFLOPs_median"] = prefill_flops(tokens, pos0) / (sus["us_median"] * 1e-6) / 1e12
        sus["frac_mfma_f16_peak_median"] = sus["TFLOPs_median"] / MFMA_F16_PEAK_TFLOPS
        log(f"prefill sustained ({sus['calls']} calls): median {sus['us_median']:.1f} µs, "
            f"last block {sus['us_last_block']:.1f} µs")
        out["sustained"] = sus
    for b in (kb, vb, q, o, ones):
        b.free()
    table.free()
    return out, t


def bench_qkv(k, stream, tokens, kv, steps, warmup, seed=21):
    """qk_norm_rope_store for `tokens` tokens at pos0 = 0 (the step before attention): bytes =
    q, k, v read + q, k written (f32) + K and V cache rows written."""
    nq, nk = tokens * HQ * DIM, tokens * HKV * DIM
    bufs = [DeviceBuffer(4 * n) for n in (nq, nk, nk)]
    for i, b in enumerate(bufs):
        fill_normal(b, b.nbytes // 4, seed + i, 1.0, stream)
    qn, kn = DeviceBuffer(4 * DIM), DeviceBuffer(4 * DIM)
    fill_normal(qn, DIM, seed + 5, 1.0, stream)
    fill_normal(kn, DIM, seed + 6, 1.0, stream)
    kc, vc = DeviceBuffer(kv.bytes(nk)), DeviceBuffer(kv.bytes(nk))
    table = RopeTable(1e6, DIM, max(tokens, 64))
    shape = AttnShape(tokens, HQ, HKV, DIM, 0, kv)
    stream.synchronize()
    t = time_steps(lambda s: k.qk_norm_rope_store(kv, bufs, (qn, kn), 1e-6, table, (kc, vc),
                                                  shape, s), stream, steps, warmup)
    nbytes = 4 * (2 * nq + 3 * nk) + 2 * kv.bytes(nk)
    log(f"qk_norm_rope_store kv={kv.name_str} T={tokens}: {t * 1e6:.2f} µs, "
        f"{nbytes / t / 1e9:.0f} GB/s")
    return {"us": t * 1e6, "bytes": nbytes, "GBps": nbytes / t / 1e9}


def cpu_baseline(budget_s: float = 20.0):
    """The reference's CPU attention (serial f64 oracle, exp re-evaluated per output component as
    reference.rs:209 does) on BASELINE.json configs[0]: decode, lk = 2048, fp16 KV. Bounded:
    as many single-layer calls as fit in ~budget_s / 2, then prefill T = 2048 on a sample of
    query rows for the rest."""
    import oracle
    rng = np.random.default_rng(0)
    lk = 2048
    q = oracle.round_f16(rng.standard_normal(HQ * DIM, dtype=np.float32))
    kk = oracle.round_f16(rng.standard_normal(lk * HKV * DIM, dtype=np.float32))
    vv = oracle.round_f16(rng.standard_normal(lk * HKV * DIM, dtype=np.float32))
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle.attention(q, kk, vv, 1, HQ, HKV, DIM, lk - 1, recompute_exp=True)
        calls += 1
        el = time.perf_counter() - t0
        if el > budget_s / 2 or calls >= 200:
            break
    dec_s = el / calls
    # prefill T = 2048 at pos0 = 0: rows spread over the causal range, scaled by their key count
    T = 2048
    qp = oracle.round_f16(rng.standard_normal(T * HQ * DIM, dtype=np.float32))
    rows = [T - 1, T // 2, T // 4, 3 * T // 4, T - 2, T // 2 + 1, 7 * T // 8, T // 8]
    keys, t0 = 0, time.perf_counter()
    for r in rows:
        oracle.attention(qp, kk, vv, T, HQ, HKV, DIM, 0, q16=True, recompute_exp=True,
                         rows=(r, r + 1))
        keys += r + 1
        if time.perf_counter() - t0 > budget_s / 2:
            break
    pre_s = time.perf_counter() - t0
    pre_tflops = 4.0 * HQ * DIM * keys / pre_s / 1e12
    return {
        "value": decode_bytes(lk, KvType.F16) / dec_s / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"decode lk=2048 fp16 KV, {calls} single-layer calls "
                   f"({dec_s * 1e6:.0f} µs/layer); prefill T=2048 on {len(rows)} query rows "
                   f"({pre_tflops * 1e3:.3f} GFLOP/s)"),
        "decode_us_per_layer": dec_s * 1e6,
        "prefill_GFLOPs": pre_tflops * 1e3,
        "host_cpu": _cpu_model(),
        "nproc": os.cpu_count(),
    }


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if present."""
    p = os.path.join(ROOT, "profiles", "decode_f16_16k_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    return None


COPY_BYTES = 256 << 20


def profile_run(k: Kernels, stream: Stream, what: str) -> int:
    """A short run for rocprofv3: three dispatches of a plain copy kernel of COPY_BYTES read and
    COPY_BYTES written (store_kv with f32 cache type is a straight copy, the calibration of the
    FETCH_SIZE / WRITE_SIZE counters), then the workload's kernels."""
    n = COPY_BYTES // 4
    src, dst = DeviceBuffer(COPY_BYTES), DeviceBuffer(COPY_BYTES)
    fill_normal(src, n, 11, 1.0, stream)
    for _ in range(3):
        k.store_kv(KvType.F32, src, dst, n, stream)
    stream.synchronize()
    src.free()
    dst.free()
    decode_cases = {"decode": (16384, KvType.F16), "decode_q8": (16384, KvType.Q8_0),
                    "decode_4k": (4096, KvType.F16), "decode_32k": (32768, KvType.F16)}
    f16, q8, pf32 = KvType.F16, KvType.Q8_0, PrefillPrecision.F16_PF32
    prefill_cases = {"prefill": (2048, 0, f16, PrefillPrecision.F16),
                     "prefill_8k": (8192, 0, f16, PrefillPrecision.F16),
                     "prefill_chunk": (512, 16384, f16, PrefillPrecision.F16),
                     "prefill_pf32": (2048, 0, f16, pf32),
                     "prefill_q8": (2048, 0, q8, PrefillPrecision.F16),
                     "prefill_q8_chunk": (512, 16384, q8, PrefillPrecision.F16)}
    if what in decode_cases:
        lk, kv = decode_cases[what]
        layers = DecodeLayers(k, lk, kv, stream)
        for _ in range(6):  # the first step is the cold one (brasa_amd.trace_summary drops it)
            layers.step(stream)
        stream.synchronize()
        layers.free()
    elif what == "decode_ragged":
        bench_ragged(k, stream, 3, 1)
    else:
        tokens, pos0, kv, prec = prefill_cases[what]
        bench_prefill(k, stream, tokens, pos0, kv, 10, 2, precision=prec)
    log(f"profile run '{what}' done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="only the headline decode + 2K prefill")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile", choices=("decode", "decode_q8", "decode_4k", "decode_32k",
                                          "decode_ragged", "prefill", "prefill_8k",
                                          "prefill_chunk", "prefill_pf32", "prefill_q8",
                                          "prefill_q8_chunk"),
                    help="short fixed run for rocprofv3 (kernel trace / counters), no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the attention path has no "
                                   "multi-GPU code (it would shard by KV head, one GPU per head "
                                   "group, with no communication); run --gpus 1"}))
        return 2
    stream = Stream()
    k = Kernels(stream)
    log(f"device: {device_name()}")
    if args.profile:
        return profile_run(k, stream, args.profile)

    head, t_step = bench_decode(k, stream, 16384, KvType.F16, args.steps, args.warmup)
    pre2k, _ = bench_prefill(k, stream, 2048, 0, KvType.F16, max(args.steps, 20), args.warmup,
                             sustained=True)
    extra_decode, extra_prefill = {}, {}
    if not args.quick:
        for lk in (4096, 32768):
            extra_decode[f"f16_{lk}"], _ = bench_decode(k, stream, lk, KvType.F16,
                                                        max(10, args.steps // 2), 2)
        extra_decode["q8_16384"], _ = bench_decode(k, stream, 16384, KvType.Q8_0,
                                                   max(10, args.steps // 2), 2)
        extra_decode["ragged_8seq"] = bench_ragged(k, stream, max(10, args.steps // 2), 2)
        extra_prefill["qk_norm_rope_store_f16_T1"] = bench_qkv(k, stream, 1, KvType.F16, 50, 5)
        extra_prefill["qk_norm_rope_store_f16_T2048"] = bench_qkv(k, stream, 2048, KvType.F16,
                                                                  20, 3)
        extra_prefill["qk_norm_rope_store_q8_T2048"] = bench_qkv(k, stream, 2048, KvType.Q8_0,
                                                                 20, 3)
        extra_prefill["T8192"], _ = bench_prefill(k, stream, 8192, 0, KvType.F16, 10, 2)
        extra_prefill["T512_pos16384"], _ = bench_prefill(k, stream, 512, 16384, KvType.F16, 10, 2)
        extra_prefill["T2048_f16_pf32"], _ = bench_prefill(
            k, stream, 2048, 0, KvType.F16, 20, 3, precision=PrefillPrecision.F16_PF32)
        extra_prefill["q8_T2048"], _ = bench_prefill(k, stream, 2048, 0, KvType.Q8_0, 10, 2)
        extra_prefill["q8_T512_pos16384"], _ = bench_prefill(k, stream, 512, 16384, KvType.Q8_0,
                                                             10, 2)
    cpu = None if args.no_cpu else cpu_baseline()

    per_layer_s = head["us_per_layer"] / 1e6
    achieved = head["bytes_per_layer"] / per_layer_s / 1e9
    line = {
        "metric": METRIC,
        "value": round(head["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 softmax/accumulation",
        "data": "synthetic N(0,1) generated on device, 36 distinct per-layer caches",
        "config": {"workload": "decode attention, 1 token x 36 layers, fp16 KV cache at 16384 "
                               "positions, hq 32 / hkv 8 / head_dim 128, batch 1",
                   "decode_us_per_layer": round(head["us_per_layer"], 3),
                   "prefill_2k_TFLOPs": round(pre2k["TFLOPs"], 1)},
        "decode_f16_16384": head,
        "prefill_f16_T2048": pre2k,
        "decode_other": extra_decode,
        "prefill_other": extra_prefill,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(),
                     "kernel": "decode_f16_kernel (splits merged in the same launch), per layer"},
        "roofline_prefill": {"bound": "mfma", "achieved": round(pre2k["TFLOPs"], 1),
                             "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(pre2k["TFLOPs"] / MFMA_F16_PEAK_TFLOPS, 4)},
        "cpu_baseline": cpu,
        "device": device_name(),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
