"""brasa_amd: the Brasa attention hot path (split-K decode + causal flash prefill over f16 / q8_0
KV caches) as hand-written gfx950 HIP kernels behind a C ABI (``include/brasa_attn.h``).

The compute lives in ``libbrasa_attn.so`` (built from ``csrc/`` by hipcc); this package is the
host-side mirror of the reference's ``brasa_kernels`` attention interface plus the device
plumbing the harnesses need.
"""
from ._lib import BrasaError, LIB_PATH, build
from .kernels import (DECODE_CHUNK, GQA_GROUPS, KV_ALIGN, AttnShape, Kernels, KvType, OutDType,
                      PrefillPrecision, RopeTable, decode_batch_partials_len, decode_partials_len, gqa_supported,
                      rope_table)
from .kvcache import KvCache, kv_cache_bytes, kv_cache_len, kv_capacity, kv_offset

__all__ = [
    "AttnShape", "BrasaError", "DECODE_CHUNK", "GQA_GROUPS", "KV_ALIGN", "Kernels", "KvType",
    "LIB_PATH", "OutDType", "PrefillPrecision", "RopeTable", "build", "decode_batch_partials_len", "decode_partials_len",
    "gqa_supported", "rope_table", "KvCache", "kv_cache_bytes", "kv_cache_len", "kv_capacity",
    "kv_offset",
]
