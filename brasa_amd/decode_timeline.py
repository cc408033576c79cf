"""Phase timeline of one decode launch, from the timeline build of the library.

    python -m brasa_amd.decode_timeline --lk 16384 --kv f16

Loads ``libbrasa_attn_trace.so`` (the library with the decode kernels compiled with
``BRASA_DECODE_TRACE``: thread 0 of each workgroup stamps the 100 MHz real-time counter at the
phases of ``DecodeStamp`` in ``csrc/decode.hip``), runs 36 back-to-back layers of
``decode_attention_lanes`` over distinct synthetic caches (the bench workload) several times and
prints, for the last launch, each phase's time after the first workgroup started: over all
workgroups, and for the last arrival of every merge group. The stamps cost one store each; the
per-layer time printed beside them is that of the timeline build.
"""
from __future__ import annotations

import argparse
import ctypes
import os

import numpy as np

HQ, HKV, DIM, LAYERS = 32, 8, 128, 36
STAMPS = 16
SLOTS = 8192
PHASES = ["start", "first block in (wave 0)", "last block in (wave 0)", "wave 0 done",
          "all waves merged in LDS", "partials visible", "arrival counted",
          "partial loads issued (last)", "partials loaded (last)", "splits merged (last)", "o written (last)"]


def _load_trace_lib():
    from . import _lib
    here = os.path.dirname(os.path.abspath(__file__))
    path = os.path.join(here, "libbrasa_attn_trace.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C {_lib.CSRC}`")
    _lib.LIB_PATH = path  # before the first lib() call
    lib = _lib.lib()
    lib.brasa_decode_trace_read.restype = ctypes.c_int
    lib.brasa_decode_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    return lib


def run(lk: int, kv_name: str, reps: int = 5) -> dict:
    lib = _load_trace_lib()
    from .device import DeviceBuffer, Event, Stream, fill_normal, synchronize
    from .kernels import AttnShape, Kernels, KvType, OutDType, decode_partials_len

    kv = KvType.parse(kv_name)
    k = Kernels()
    stream = Stream()
    n = lk * HKV * DIM
    tmp = DeviceBuffer(4 * n)
    caches = []
    for layer in range(LAYERS):
        kb, vb = DeviceBuffer(kv.bytes(n)), DeviceBuffer(kv.bytes(n))
        fill_normal(tmp, n, 1000 + 2 * layer, 1.0, stream)
        k.store_kv(kv, tmp, kb, n, stream)
        fill_normal(tmp, n, 1001 + 2 * layer, 1.0, stream)
        k.store_kv(kv, tmp, vb, n, stream)
        caches.append((kb, vb))
    q = DeviceBuffer(4 * HQ * DIM)
    fill_normal(q, HQ * DIM, 7919, 1.0, stream)
    o = DeviceBuffer(4 * HQ * DIM)
    part = DeviceBuffer(4 * decode_partials_len(HQ, lk))
    shape = AttnShape(1, HQ, HKV, DIM, lk - 1, kv)
    stream.synchronize()
    tmp.free()

    best = float("inf")
    for _ in range(reps):
        e0, e1 = Event(), Event()
        e0.record(stream)
        for kb, vb in caches:
            k.decode_attention_lanes(q, kb, vb, part, o, shape, OutDType.F32, stream)
        e1.record(stream)
        e1.synchronize()
        best = min(best, e0.elapsed_ms(e1) * 1e3 / LAYERS)
    synchronize()
    t = np.zeros(SLOTS * STAMPS, dtype=np.uint64)
    if lib.brasa_decode_trace_read(t.ctypes.data, t.size) != 0:
        raise RuntimeError("brasa_decode_trace_read failed")
    for kb, vb in caches:
        kb.free()
        vb.free()
    t = t.reshape(SLOTS, STAMPS)
    used = t[:, 0] != 0                 # slots the launches wrote (one grid, every launch)
    slot = np.nonzero(used)[0]          # = blockIdx.x (a single-sequence grid has < SLOTS)
    t = t[used]
    t0 = t[:, 0].min()
    rel = np.where(t >= t0, (t.astype(np.float64) - float(t0)) * 0.01, np.nan)  # us
    rows = []
    for i, name in enumerate(PHASES):
        v = rel[:, i]
        v = np.sort(v[np.isfinite(v)])
        if v.size == 0:
            continue
        rows.append((name, v.size, v[0], v[v.size // 10], v[v.size // 2], v[v.size * 9 // 10],
                     v[-1]))
    last = rel[np.isfinite(rel[:, PHASES.index("partials loaded (last)")])]
    # per KV head: the fp16 kernel's grid has the head groups innermost (one head per workgroup
    # at these lengths), so workgroup b reads KV head b % HKV
    per_head = []
    if kv.name_str == "f16":
        col = PHASES.index("all waves merged in LDS")
        for h in range(HKV):
            v = rel[slot % HKV == h, col]
            v = v[np.isfinite(v)]
            if v.size:
                per_head.append((h, v.size, float(np.median(v)), float(v.max())))
    return {"lk": lk, "kv": kv.name_str, "workgroups": int(used.sum()),
            "us_per_layer": best, "phases": rows, "last": last[:, :len(PHASES)],
            "per_head": per_head}


def report(r: dict) -> str:
    out = [f"decode kv={r['kv']} lk={r['lk']}: {r['workgroups']} workgroups, "
           f"{r['us_per_layer']:.2f} us/layer (36 back-to-back layers, timeline build)",
           "",
           "| phase (us after the first workgroup started) | n | min | p10 | median | p90 | max |",
           "|---|---|---|---|---|---|---|"]
    for name, n, *v in r["phases"]:
        out.append(f"| {name} | {n} | " + " | ".join(f"{x:.2f}" for x in v) + " |")
    out += ["", "Last arrival of each merge group (us):", "",
            "| " + " | ".join(PHASES) + " |", "|" + "---|" * len(PHASES)]
    for row in r["last"]:
        out.append("| " + " | ".join("" if not np.isfinite(x) else f"{x:.2f}" for x in row) + " |")
    if r["per_head"]:
        out += ["", "All waves of a workgroup merged in LDS, per KV head (us):", "",
                "| KV head | workgroups | median | max |", "|---|---|---|---|"]
        for h, n, med, mx in r["per_head"]:
            out.append(f"| {h} | {n} | {med:.2f} | {mx:.2f} |")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--lk", type=int, default=16384)
    ap.add_argument("--kv", default="f16", choices=["f16", "q8_0"])
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args()
    print(report(run(a.lk, a.kv, a.reps)), flush=True)


if __name__ == "__main__":
    main()
