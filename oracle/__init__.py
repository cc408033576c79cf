"""CPU oracle for the Brasa attention hot path -- TEST INFRASTRUCTURE ONLY.

numpy front-end over ``liboracle.so`` (built from ``brasa_oracle.c`` by ``oracle/Makefile``).
It restates the reference's f64 attention (``crates/kernels/src/reference.rs:129-218``), its f16
conversions and KV-Q8 spec (``crates/quant/src/qtype.rs:32-130``), its xorshift64* test RNG
(``crates/kernels/src/testutil.rs:4-28``) and its tolerance functions
(``crates/kernels/tests/attention.rs:12-32``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, and only as the checker / the timed CPU baseline. The product (``brasa_amd``) never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")

F32P = ctypes.POINTER(ctypes.c_float)
U16P = ctypes.POINTER(ctypes.c_uint16)
U8P = ctypes.POINTER(ctypes.c_uint8)
SZ = ctypes.c_size_t


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_SO):
        build()
    lib = ctypes.CDLL(_SO)
    lib.or_f16_to_f32.restype = ctypes.c_float
    lib.or_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.or_f32_to_f16.restype = ctypes.c_uint16
    lib.or_f32_to_f16.argtypes = [ctypes.c_float]
    lib.or_f32_to_f16_n.argtypes = [F32P, U16P, SZ]
    lib.or_f16_to_f32_n.argtypes = [U16P, F32P, SZ]
    lib.or_quantize_kv_q8.argtypes = [F32P, SZ, U8P]
    lib.or_dequantize_kv_q8.argtypes = [U8P, SZ, F32P]
    lib.or_rng_vec.argtypes = [ctypes.c_void_p, F32P, SZ, ctypes.c_float]
    lib.or_rng_init.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    lib.or_rng_next_u64.restype = ctypes.c_uint64
    lib.or_rng_next_u64.argtypes = [ctypes.c_void_p]
    lib.or_attention_rows.argtypes = [F32P, F32P, F32P, SZ, SZ, SZ, SZ, SZ, SZ, SZ, F32P, F32P,
                                      ctypes.c_int, ctypes.c_int]
    lib.or_worst.restype = ctypes.c_float
    lib.or_worst.argtypes = [F32P, F32P, F32P, SZ]
    lib.or_worst_f16.restype = ctypes.c_float
    lib.or_worst_f16.argtypes = [U16P, F32P, F32P, SZ]
    lib.or_rms_norm.argtypes = [F32P, F32P, SZ, SZ, ctypes.c_float, F32P]
    lib.or_rope_neox.argtypes = [F32P, SZ, SZ, SZ, SZ, F32P, F32P]
    lib.or_rope_table.argtypes = [ctypes.c_double, SZ, SZ, F32P, F32P]
    return lib


_lib = _load()


def _p(a: np.ndarray, ty):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ty)


def f32_to_f16(x) -> np.ndarray:
    """qtype.rs:52-78, elementwise; returns the f16 bit patterns as uint16."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib.or_f32_to_f16_n(_p(x, F32P), _p(out, U16P), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    """qtype.rs:32-50, elementwise, from uint16 bit patterns."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    _lib.or_f16_to_f32_n(_p(h, U16P), _p(out, F32P), h.size)
    return out


def round_f16(x) -> np.ndarray:
    """reference.rs:66-69."""
    return f16_to_f32(f32_to_f16(x))


KV_Q8_DIM = 128
KV_Q8_ROW = 136


def quantize_kv_q8(x) -> np.ndarray:
    """qtype.rs:85-111: f32 rows of 128 -> uint8 rows of 136."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % KV_Q8_DIM == 0
    out = np.empty(x.size // KV_Q8_DIM * KV_Q8_ROW, dtype=np.uint8)
    _lib.or_quantize_kv_q8(_p(x, F32P), x.size, _p(out, U8P))
    return out


def dequantize_kv_q8(data) -> np.ndarray:
    """qtype.rs:113-130."""
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    assert data.size % KV_Q8_ROW == 0
    rows = data.size // KV_Q8_ROW
    out = np.empty(rows * KV_Q8_DIM, dtype=np.float32)
    _lib.or_dequantize_kv_q8(_p(data, U8P), rows, _p(out, F32P))
    return out


class Rng:
    """testutil.rs:4-28: xorshift64* with uniform values in [-1, 1)."""

    def __init__(self, seed: int):
        self._state = ctypes.c_uint64(0)
        _lib.or_rng_init(ctypes.byref(self._state), seed)

    def next_u64(self) -> int:
        return int(_lib.or_rng_next_u64(ctypes.byref(self._state)))

    def vec(self, n: int, scale: float) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        _lib.or_rng_vec(ctypes.byref(self._state), _p(out, F32P), n, scale)
        return out


def attention(q, k, v, tokens, hq, hkv, dim, pos0, *, q16=False, recompute_exp=False,
              rows=None):
    """reference.rs:150-171 (q16=False) or reference.rs:129-145 (q16=True).

    q: [tokens, hq, dim]; k, v: [>= pos0 + tokens, hkv, dim] f32. Returns (o, vmax), each
    [tokens, hq, dim] f32. ``rows=(t0, t1)`` computes only those query tokens (others stay 0).
    """
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    assert q.size == tokens * hq * dim
    assert k.size >= (pos0 + tokens) * hkv * dim and v.size >= (pos0 + tokens) * hkv * dim
    o = np.zeros(tokens * hq * dim, dtype=np.float32)
    vmax = np.zeros(tokens * hq * dim, dtype=np.float32)
    t0, t1 = rows if rows is not None else (0, tokens)
    _lib.or_attention_rows(_p(q, F32P), _p(k, F32P), _p(v, F32P), tokens, hq, hkv, dim, pos0,
                           t0, t1, _p(o, F32P), _p(vmax, F32P), int(recompute_exp), int(q16))
    return o.reshape(tokens, hq, dim), vmax.reshape(tokens, hq, dim)


def worst(got, expected, vmax) -> float:
    """attention.rs:25-32: max |got - expected| / max|v|."""
    g = np.ascontiguousarray(got, dtype=np.float32).reshape(-1)
    e = np.ascontiguousarray(expected, dtype=np.float32).reshape(-1)
    m = np.ascontiguousarray(vmax, dtype=np.float32).reshape(-1)
    assert g.size == e.size == m.size
    return float(_lib.or_worst(_p(g, F32P), _p(e, F32P), _p(m, F32P), g.size))


def worst_f16(got_bits, expected, vmax) -> float:
    """attention.rs:12-23: as worst() for f16 output, discounting the final rounding."""
    g = np.ascontiguousarray(got_bits, dtype=np.uint16).reshape(-1)
    e = np.ascontiguousarray(expected, dtype=np.float32).reshape(-1)
    m = np.ascontiguousarray(vmax, dtype=np.float32).reshape(-1)
    assert g.size == e.size == m.size
    return float(_lib.or_worst_f16(_p(g, U16P), _p(e, F32P), _p(m, F32P), g.size))


def rms_norm(x, w, n, eps) -> np.ndarray:
    """reference.rs:22-30."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    out = np.empty_like(x)
    _lib.or_rms_norm(_p(x, F32P), _p(w, F32P), x.size // n, n, eps, _p(out, F32P))
    return out


def rope_neox(x, tokens, heads, dim, pos0, cos_t, sin_t) -> np.ndarray:
    """reference.rs:45-58 (returns a rotated copy)."""
    y = np.array(x, dtype=np.float32).reshape(-1).copy()
    c = np.ascontiguousarray(cos_t, dtype=np.float32)
    s = np.ascontiguousarray(sin_t, dtype=np.float32)
    _lib.or_rope_neox(_p(y, F32P), tokens, heads, dim, pos0, _p(c, F32P), _p(s, F32P))
    return y


def rope_table(theta, dim, max_pos):
    """lib.rs:1388-1404: cos/sin [max_pos, dim/2] computed in f64, stored f32."""
    c = np.empty(max_pos * (dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    _lib.or_rope_table(theta, dim, max_pos, _p(c, F32P), _p(s, F32P))
    return c, s
