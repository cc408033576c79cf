"""The model's KV cache as the attention entry points see it.

Mirrors ``KvCache`` (crates/models/src/qwen3.rs:211-273) and the sizes the model and the memory
planner derive from it: the per-layer capacity ``ctx.next_multiple_of(KV_ALIGN)``
(qwen3.rs:384-386), one K and one V buffer of ``layers * cap * hkv * dim`` elements in the cache
type (qwen3.rs:386; q8_0 as 136-byte rows), the view of position ``pos`` of layer ``li`` at element
``(li * cap + pos) * hkv * dim`` (qwen3.rs:554-556), converted to bytes for q8_0 as
``off / 128 * 136`` (``KvCache::args``, qwen3.rs:246-257), and the planner's
``kv_bytes`` (crates/memory/src/planner.rs:77-81) without its Metal page rounding
(``buffer_bytes``: the reference rounds each buffer up to 16 KiB pages; hipMalloc's granularity is
not part of this contract).

The formulas are the C ABI's (``brasa_kv_capacity``, ``brasa_kv_cache_len``, ``brasa_kv_offset``,
``brasa_kv_bytes``), so a Rust caller and this mirror agree by construction.
"""
from __future__ import annotations

from ._lib import lib
from .device import DeviceBuffer
from .kernels import KvType


def kv_capacity(ctx: int) -> int:
    """Positions per layer: ctx rounded up to KV_ALIGN (qwen3.rs:384-386)."""
    return int(lib().brasa_kv_capacity(ctx))


def kv_cache_len(layers: int, ctx: int, hkv: int, dim: int = 128) -> int:
    """Elements of the K (or V) buffer (qwen3.rs:386)."""
    return int(lib().brasa_kv_cache_len(layers, ctx, hkv, dim))


def kv_offset(layer: int, ctx: int, hkv: int, pos: int, dim: int = 128) -> int:
    """Element offset of position ``pos`` of ``layer`` (qwen3.rs:554-556)."""
    return int(lib().brasa_kv_offset(layer, ctx, hkv, dim, pos))


def kv_cache_bytes(kv: KvType, layers: int, ctx: int, hkv: int, dim: int = 128) -> int:
    """Bytes of K plus V (planner.rs:77-81: ``2 * elems.div_ceil(32) * kv_block_bytes``)."""
    return 2 * kv.bytes(kv_cache_len(layers, ctx, hkv, dim))


class KvCache:
    """K and V caches of ``layers`` layers, ``ctx`` positions, ``hkv`` heads of ``dim`` values.

    ``layer(li)`` is the (K, V) view pair the attention entry points take (the layer base);
    ``at(li, pos)`` the pair ``qk_norm_rope_store`` / ``store_kv`` write a block at. Views are
    ``(buffer, byte_offset)`` tuples, as every ``Kernels`` method accepts.
    """

    def __init__(self, kv: KvType, layers: int, ctx: int, hkv: int, dim: int = 128):
        self.kv, self.layers, self.ctx, self.hkv, self.dim = kv, layers, ctx, hkv, dim
        self.cap = kv_capacity(ctx)
        self.len = kv_cache_len(layers, ctx, hkv, dim)
        nbytes = kv.bytes(self.len)
        self.k = DeviceBuffer(nbytes)
        self.v = DeviceBuffer(nbytes)
        # zero-filled: prefill reads whole 64-position blocks, so positions not yet written must
        # hold finite values (lib.rs:1182-1183); zero bytes are 0.0 in every cache type
        self.k.fill(0)
        self.v.fill(0)

    def args(self, off: int):
        """``KvCache::args`` (qwen3.rs:246-257): K and V views from element ``off`` (a multiple
        of 128 for q8_0, where it becomes the byte offset of that row)."""
        b = self.kv.bytes(off)
        return (self.k, b), (self.v, b)

    def layer(self, li: int):
        if not 0 <= li < self.layers:
            raise IndexError(f"layer {li} of {self.layers}")
        return self.args(kv_offset(li, self.ctx, self.hkv, 0, self.dim))

    def at(self, li: int, pos: int):
        if not 0 <= li < self.layers or not 0 <= pos < self.cap:
            raise IndexError(f"layer {li} position {pos} of {self.layers} x {self.cap}")
        return self.args(kv_offset(li, self.ctx, self.hkv, pos, self.dim))

    def bytes(self) -> int:
        return 2 * self.kv.bytes(self.len)

    def free(self) -> None:
        self.k.free()
        self.v.free()
