"""Phase timeline of the two-group prefill kernel, from the timeline build of the library.

    python -m brasa_amd.prefill_timeline --tokens 2048 --pos0 0

Loads ``libbrasa_attn_trace.so`` (prefill_f16_kernel compiled with ``BRASA_PREFILL_TRACE``:
thread 0 of each workgroup stamps the 100 MHz real-time counter at the phases of
``PrefillStamp`` in ``csrc/prefill.hip``, for each of the one or two query tiles the workgroup
runs), runs ``flash_attention`` (F16) on the bench's inputs (Q and K N(0, 1) through per-head
RMSNorm and RoPE-NeoX, V N(0, 1), fp16 cache) several times and prints, for the last call, each
phase's time after the first workgroup started, over all workgroups and per tile ordinal.
"""
from __future__ import annotations

import argparse
import ctypes
import os

import numpy as np

HQ, HKV, DIM = 32, 8, 128
STAMPS = 16
SLOTS = 8192
PHASES = ["tile start", "prologue done (Q in, first copies issued)", "first K/V tile landed",
          "key loop done", "key groups merged", "o stored"]


def _load_trace_lib():
    from . import _lib
    here = os.path.dirname(os.path.abspath(__file__))
    path = os.path.join(here, "libbrasa_attn_trace.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C {_lib.CSRC}`")
    _lib.LIB_PATH = path  # before the first lib() call
    lib = _lib.lib()
    lib.brasa_prefill_trace_read.restype = ctypes.c_int
    lib.brasa_prefill_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    return lib


def run(tokens: int, pos0: int, reps: int = 5) -> dict:
    lib = _load_trace_lib()
    from .device import DeviceBuffer, Event, Stream, fill_normal, synchronize
    from .kernels import AttnShape, Kernels, KvType, PrefillPrecision, RopeTable

    k = Kernels()
    stream = Stream()
    lk = pos0 + tokens
    cap = (lk + 63) // 64 * 64
    n = cap * HKV * DIM
    table = RopeTable(1e6, DIM, cap)
    ones = DeviceBuffer.from_array(np.ones(DIM, np.float32))
    tmp = DeviceBuffer(4 * n)
    kb, vb = DeviceBuffer(2 * n), DeviceBuffer(2 * n)
    fill_normal(tmp, n, 3, 1.0, stream)
    k.rms_norm(tmp, ones, tmp, cap * HKV, DIM, 1e-6, stream)
    k.rope_neox(tmp, table, cap, HKV, DIM, 0, stream)
    k.store_kv(KvType.F16, tmp, kb, n, stream)
    fill_normal(tmp, n, 4, 1.0, stream)
    k.store_kv(KvType.F16, tmp, vb, n, stream)
    q = DeviceBuffer(4 * tokens * HQ * DIM)
    fill_normal(q, tokens * HQ * DIM, 5, 1.0, stream)
    k.rms_norm(q, ones, q, tokens * HQ, DIM, 1e-6, stream)
    k.rope_neox(q, table, tokens, HQ, DIM, pos0, stream)
    o = DeviceBuffer(2 * tokens * HQ * DIM)
    shape = AttnShape(tokens, HQ, HKV, DIM, pos0, KvType.F16)
    stream.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = Event(), Event()
        e0.record(stream)
        k.flash_attention_with(q, kb, vb, o, shape, PrefillPrecision.F16, stream)
        e1.record(stream)
        e1.synchronize()
        best = min(best, e0.elapsed_ms(e1) * 1e3)
    synchronize()
    t = np.zeros(SLOTS * STAMPS, dtype=np.uint64)
    if lib.brasa_prefill_trace_read(t.ctypes.data, t.size) != 0:
        raise RuntimeError("brasa_prefill_trace_read failed")
    for b in (tmp, kb, vb, q, o, ones):
        b.free()
    table.free()
    t = t.reshape(SLOTS, STAMPS)
    used = t[:, 0] != 0
    if not used.any():
        raise RuntimeError("no workgroup stamped: this launch did not use prefill_f16_kernel "
                           "(the two-group kernel; longer prompts take the four-wave kernels)")
    t = t[used]
    t0 = t[:, 0].min()
    rel = np.where(t >= t0, (t.astype(np.float64) - float(t0)) * 0.01, np.nan)  # us
    rows = []
    for ti in (0, 1):
        for i, name in enumerate(PHASES):
            v = rel[:, 1 + 6 * ti + i]
            v = np.sort(v[np.isfinite(v)])
            if v.size:
                rows.append((f"tile {ti}: {name}", v.size, v[0], v[v.size // 10], v[v.size // 2],
                             v[v.size * 9 // 10], v[-1]))
    # per-workgroup durations of each tile's phases (medians and maxima)
    dur = {}
    for ti in (0, 1):
        base = 1 + 6 * ti
        for i in range(1, 6):
            d = rel[:, base + i] - rel[:, base + i - 1]
            d = d[np.isfinite(d)]
            if d.size:
                dur[f"tile {ti}: {PHASES[i - 1]} -> {PHASES[i]}"] = (np.median(d), d.max())
    return {"tokens": tokens, "pos0": pos0, "workgroups": int(used.sum()), "us": best,
            "phases": rows, "durations": dur, "end": np.nanmax(rel)}


def report(r: dict) -> str:
    out = [f"prefill F16 T={r['tokens']} pos0={r['pos0']}: {r['workgroups']} workgroups, "
           f"{r['us']:.1f} us per call (timeline build; last stamp at {r['end']:.1f} us)", "",
           "| phase (us after the first workgroup started) | n | min | p10 | median | p90 | max |",
           "|---|---|---|---|---|---|---|"]
    for name, n, *v in r["phases"]:
        out.append(f"| {name} | {n} | " + " | ".join(f"{x:.2f}" for x in v) + " |")
    out += ["", "| per-workgroup step | median us | max us |", "|---|---|---|"]
    for name, (med, mx) in r["durations"].items():
        out.append(f"| {name} | {med:.2f} | {mx:.2f} |")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--tokens", type=int, default=2048)
    ap.add_argument("--pos0", type=int, default=0)
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args()
    print(report(run(a.tokens, a.pos0, a.reps)), flush=True)


if __name__ == "__main__":
    main()
