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

from ._lib import AttnShapeC, check, lib
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
                from ._lib import BrasaError
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

    def decode_attention(self, q, k, v, partials: DeviceBuffer, o, shape: AttnShape,
                         out: OutDType = OutDType.F32, stream=None,
                         partials_len: int | None = None) -> None:
        plen = partials.nbytes // 4 if partials_len is None else partials_len
        check(lib().brasa_decode_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(partials), plen,
                                           _ptr(o), int(out), shape.c(),
                                           _stream(stream or self.stream)))

    def flash_attention(self, q, k, v, o, shape: AttnShape, stream=None) -> None:
        self.flash_attention_with(q, k, v, o, shape, PrefillPrecision.F16, stream)

    def flash_attention_with(self, q, k, v, o, shape: AttnShape,
                             precision: PrefillPrecision, stream=None) -> None:
        check(lib().brasa_flash_attention_with(_ptr(q), _ptr(k), _ptr(v), _ptr(o), shape.c(),
                                               int(precision), _stream(stream or self.stream)))
