"""Host-side mirror of the reference's attention interface (``brasa_kernels``).

Names, argument meaning and error behaviour follow ``crates/kernels/src/lib.rs``: ``KvType``
(:92-143), ``PrefillPrecision`` (:1311-1318), ``AttnShape`` (:1354-1364), ``gqa_supported``
(:1323-1327), ``decode_partials_len`` (:1334-1337), ``DECODE_CHUNK``/``KV_ALIGN`` and the
``Kernels`` methods ``store_kv`` (:1029-1050), ``decode_attention`` (:1056-1103),
``decode_attention_lanes`` (:1110-1164), ``flash_attention`` / ``flash_attention_with``
(:1169-1248). Where the reference panics on a violated ``assert!``, these raise
``BrasaError`` carrying the C ABI status; every call goes through ``libbrasa_attn.so``.

Buffers are ``DeviceBuffer`` objects or raw device addresses (ints); a view at a byte offset
(the reference's ``Arg::Buf(buffer, offset)``) is ``(buffer, offset)``.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

from ._lib import AttnShapeC, RopeTableC, check, lib
from .device import DeviceBuffer, Stream

DECODE_CHUNK = 128
KV_ALIGN = 64
GQA_GROUPS = (1, 2, 4, 8)
KV_Q8_DIM = 128
KV_Q8_ROW = 136


class KvType(enum.IntEnum):
    """lib.rs:92-143 (values are the reference's ``KvType as usize``)."""

    F32 = 0
    F16 = 1
    Q8_0 = 2

    def block_bytes(self) -> int:
        return {KvType.F32: 128, KvType.F16: 64, KvType.Q8_0: 34}[self]

    def bytes(self, n: int) -> int:
        if self is KvType.Q8_0:
            if n % KV_Q8_DIM:
                from ._lib import RopeTableC, BrasaError
                raise BrasaError(1, f"KV Q8: rows of {KV_Q8_DIM} values")
            return n // KV_Q8_DIM * KV_Q8_ROW
        return n * self.block_bytes() // 32

    @property
    def name_str(self) -> str:
        return {KvType.F32: "f32", KvType.F16: "f16", KvType.Q8_0: "q8_0"}[self]

    @staticmethod
    def parse(s: str) -> "KvType | None":
        return {"f32": KvType.F32, "f16": KvType.F16, "q8_0": KvType.Q8_0,
                "q8": KvType.Q8_0}.get(s)


class PrefillPrecision(enum.IntEnum):
    """lib.rs:1311-1318."""

    F16 = 0
    F32 = 1
    #: F16 inputs/output with P kept at f32 accuracy (the reference F16 kernel's numerics)
    F16_PF32 = 2


class OutDType(enum.IntEnum):
    F32 = 0
    F16 = 1


@dataclass(frozen=True)
class AttnShape:
    """lib.rs:1354-1364."""

    tokens: int
    hq: int
    hkv: int
    dim: int
    pos0: int
    kv: KvType

    def c(self) -> AttnShapeC:
        return AttnShapeC(self.tokens, self.hq, self.hkv, self.dim, self.pos0, int(self.kv))


def decode_batch_partials_len(hq: int, lks) -> int:
    """Scratch floats of a batched decode: the sum of decode_partials_len over the sequences."""
    return sum(decode_partials_len(hq, int(x)) for x in lks)


def gqa_supported(hq: int, hkv: int) -> bool:
    return bool(lib().brasa_gqa_supported(hq, hkv))


def decode_partials_len(hq: int, lk: int) -> int:
    return int(lib().brasa_decode_partials_len(hq, lk))


def _ptr(x) -> int:
    if x is None:
        return 0
    if isinstance(x, tuple):
        buf, off = x
        return _ptr(buf) + int(off)
    if hasattr(x, "ptr"):  # DeviceBuffer or anything exposing a device address
        return int(x.ptr)
    return int(x)


def _stream(s) -> int | None:
    if s is None:
        return None
    return s.handle if isinstance(s, Stream) else int(s)


def rope_table(theta: float, dim: int, max_pos: int):
    """``rope_table`` (lib.rs:1388-1404) computed by the library on the host: (cos, sin) as f32
    numpy arrays of shape [max_pos, dim // 2]."""
    import numpy as np
    half = dim // 2
    cos = np.empty(max_pos * half, dtype=np.float32)
    sin = np.empty(max_pos * half, dtype=np.float32)
    check(lib().brasa_rope_table(float(theta), dim, max_pos, cos.ctypes.data, sin.ctypes.data))
    return cos.reshape(max_pos, half), sin.reshape(max_pos, half)


class RopeTable:
    """``RopeTable::new`` (lib.rs:1376-1386): the f64-computed table uploaded to the device."""

    def __init__(self, theta: float, dim: int, max_pos: int):
        cos, sin = rope_table(theta, dim, max_pos)
        self.cos = DeviceBuffer(max(cos.nbytes, 4))
        self.sin = DeviceBuffer(max(sin.nbytes, 4))
        self.cos.upload(cos)
        self.sin.upload(sin)
        self.dim, self.max_pos = dim, max_pos

    def c(self) -> RopeTableC:
        return RopeTableC(self.cos.ptr, self.sin.ptr, self.dim, self.max_pos)

    def free(self) -> None:
        self.cos.free()
        self.sin.free()


class Kernels:
    """Attention methods of ``brasa_kernels::Kernels`` on gfx950.

    The reference encodes onto a caller-owned ``Command``; here every method enqueues on
    ``stream`` (``None`` = default stream) and returns without waiting, which is the same
    in-order contract.
    """

    def __init__(self, stream: Stream | None = None):
        lib()  # load (and fail loudly) now, as Kernels::new compiles its pipelines up front
        self.stream = stream

    def store_kv(self, kv: KvType, src, dst, n: int, stream=None) -> None:
        check(lib().brasa_store_kv(int(kv), _ptr(src), _ptr(dst), n,
                                   _stream(stream or self.stream)))

    def dequantize_kv_q8(self, src, dst, rows: int, stream=None) -> None:
        check(lib().brasa_dequantize_kv_q8(_ptr(src), _ptr(dst), rows,
                                           _stream(stream or self.stream)))

    def decode_attention_lanes(self, q, k, v, partials: DeviceBuffer, o, shape: AttnShape,
                               out: OutDType = OutDType.F32, stream=None,
                               partials_len: int | None = None) -> None:
        plen = partials.nbytes // 4 if partials_len is None else partials_len
        check(lib().brasa_decode_attention_lanes(_ptr(q), _ptr(k), _ptr(v), _ptr(partials),
                                                 plen, _ptr(o), int(out), shape.c(),
                                                 _stream(stream or self.stream)))

    def decode_attention_lanes_noalloc(self, q, k, v, o, shape: AttnShape,
                                       out: OutDType = OutDType.F32, stream=None) -> None:
        """decode_attention_lanes with the split partials in the library's fixed device array
        (no caller scratch, no allocation; calls overlapping on one GPU race)."""
        check(lib().brasa_decode_attention_lanes_noalloc(_ptr(q), _ptr(k), _ptr(v), _ptr(o),
                                                         int(out), shape.c(),
                                                         _stream(stream or self.stream)))

    def decode_attention(self, q, k, v, partials: DeviceBuffer, o, shape: AttnShape,
                         out: OutDType = OutDType.F32, stream=None,
                         partials_len: int | None = None) -> None:
        plen = partials.nbytes // 4 if partials_len is None else partials_len
        check(lib().brasa_decode_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(partials), plen,
                                           _ptr(o), int(out), shape.c(),
                                           _stream(stream or self.stream)))

    def decode_attention_batch(self, q, ks, vs, lks, partials: DeviceBuffer, o, hq: int,
                               hkv: int, kv: KvType, out: OutDType = OutDType.F32, stream=None,
                               partials_len: int | None = None) -> None:
        """Ragged batched decode: sequence i has query q[i], caches ks[i] / vs[i] and lks[i]
        keys; one launch for all of them (the reference decodes one sequence per call)."""
        import ctypes
        n = len(lks)
        assert len(ks) == n and len(vs) == n
        karr = (ctypes.c_void_p * max(n, 1))(*[_ptr(x) for x in ks])
        varr = (ctypes.c_void_p * max(n, 1))(*[_ptr(x) for x in vs])
        larr = (ctypes.c_size_t * max(n, 1))(*[int(x) for x in lks])
        plen = partials.nbytes // 4 if partials_len is None else partials_len
        check(lib().brasa_decode_attention_batch(
            _ptr(q), ctypes.cast(karr, ctypes.c_void_p), ctypes.cast(varr, ctypes.c_void_p),
            ctypes.cast(larr, ctypes.c_void_p), n, _ptr(partials), plen, _ptr(o), int(out), hq,
            hkv, 128, int(kv), _stream(stream or self.stream)))

    def rms_norm(self, x, w, out, rows: int, n: int, eps: float, stream=None) -> None:
        check(lib().brasa_rms_norm(_ptr(x), _ptr(w), _ptr(out), rows, n, eps,
                                   _stream(stream or self.stream)))

    def rope_neox(self, x, table: RopeTable, tokens: int, heads: int, dim: int, pos0: int,
                  stream=None) -> None:
        check(lib().brasa_rope_neox(_ptr(x), table.c(), tokens, heads, dim, pos0,
                                    _stream(stream or self.stream)))

    def qk_norm_rope_store(self, kv: KvType, qkv, norms, eps: float, table: RopeTable, dst,
                           shape: AttnShape, stream=None) -> None:
        """``qk_norm_rope_store`` (lib.rs:976-1025): ``qkv = (q, k, v)``, ``norms = (qn, kn)``,
        ``dst = (k_cache_at_pos0, v_cache_at_pos0)``."""
        q, k, v = qkv
        qn, kn = norms
        kd, vd = dst
        check(lib().brasa_qk_norm_rope_store(int(kv), _ptr(q), _ptr(k), _ptr(v), _ptr(qn),
                                             _ptr(kn), eps, table.c(), _ptr(kd), _ptr(vd),
                                             shape.c(), _stream(stream or self.stream)))

    def flash_attention(self, q, k, v, o, shape: AttnShape, stream=None) -> None:
        self.flash_attention_with(q, k, v, o, shape, PrefillPrecision.F16, stream)

    def flash_attention_with(self, q, k, v, o, shape: AttnShape,
                             precision: PrefillPrecision, stream=None) -> None:
        check(lib().brasa_flash_attention_with(_ptr(q), _ptr(k), _ptr(v), _ptr(o), shape.c(),
                                               int(precision), _stream(stream or self.stream)))

    @staticmethod
    def flash_attention_workspace_len(shape: AttnShape, precision: PrefillPrecision) -> int:
        """Bytes of caller workspace ``flash_attention_ws`` needs (no reference counterpart)."""
        return int(lib().brasa_flash_attention_workspace_len(shape.c(), int(precision)))

    def flash_attention_ws(self, q, k, v, o, shape: AttnShape, precision: PrefillPrecision,
                           workspace, workspace_len: int | None = None, stream=None) -> None:
        """``flash_attention_with`` on a caller-owned workspace (no reference counterpart)."""
        wlen = (workspace.nbytes if workspace is not None and hasattr(workspace, "nbytes") else 0) \
            if workspace_len is None else workspace_len
        check(lib().brasa_flash_attention_ws(_ptr(q), _ptr(k), _ptr(v), _ptr(o), shape.c(),
                                             int(precision), _ptr(workspace), wlen,
                                             _stream(stream or self.stream)))
