"""ctypes binding of ``libbrasa_attn.so`` (the hipcc-built C ABI in ``include/brasa_attn.h``).

Loading fails loudly when the library has not been built: there is no CPU fallback anywhere in
this package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("BRASA_ATTN_LIB") or os.path.join(_HERE, "libbrasa_attn.so")
CSRC = os.path.join(_HERE, "csrc")

SZ = ctypes.c_size_t
VP = ctypes.c_void_p
INT = ctypes.c_int


class AttnShapeC(ctypes.Structure):
    """``brasa_attn_shape`` (mirrors the reference's ``AttnShape``, lib.rs:1354-1364)."""

    _fields_ = [("tokens", SZ), ("hq", SZ), ("hkv", SZ), ("dim", SZ), ("pos0", SZ),
                ("kv", INT)]


class RopeTableC(ctypes.Structure):
    """``brasa_rope_table_view`` (the device side of the reference's ``RopeTable``, lib.rs:1369-1374)."""

    _fields_ = [("cos", VP), ("sin", VP), ("dim", SZ), ("max_pos", SZ)]


# name -> (restype, argtypes) for every symbol the two public headers declare
SYMBOLS = {
    "brasa_decode_partials_len": (SZ, [SZ, SZ]),
    "brasa_gqa_supported": (INT, [SZ, SZ]),
    "brasa_kv_bytes": (SZ, [INT, SZ]),
    "brasa_kv_capacity": (SZ, [SZ]),
    "brasa_kv_cache_len": (SZ, [SZ, SZ, SZ, SZ]),
    "brasa_kv_offset": (SZ, [SZ, SZ, SZ, SZ, SZ]),
    "brasa_store_kv": (INT, [INT, VP, VP, SZ, VP]),
    "brasa_dequantize_kv_q8": (INT, [VP, VP, SZ, VP]),
    "brasa_decode_attention_lanes": (INT, [VP, VP, VP, VP, SZ, VP, INT, AttnShapeC, VP]),
    "brasa_decode_attention": (INT, [VP, VP, VP, VP, SZ, VP, INT, AttnShapeC, VP]),
    "brasa_decode_attention_lanes_noalloc": (INT, [VP, VP, VP, VP, INT, AttnShapeC, VP]),
    "brasa_decode_batch_partials_len": (SZ, [SZ, VP, SZ]),
    "brasa_decode_attention_batch": (INT, [VP, VP, VP, VP, SZ, VP, SZ, VP, INT, SZ, SZ, SZ, INT,
                                           VP]),
    "brasa_flash_attention_with": (INT, [VP, VP, VP, VP, AttnShapeC, INT, VP]),
    "brasa_flash_attention": (INT, [VP, VP, VP, VP, AttnShapeC, VP]),
    "brasa_flash_attention_workspace_len": (SZ, [AttnShapeC, INT]),
    "brasa_flash_attention_ws": (INT, [VP, VP, VP, VP, AttnShapeC, INT, VP, SZ, VP]),
    "brasa_rope_table": (INT, [ctypes.c_double, SZ, SZ, VP, VP]),
    "brasa_rms_norm": (INT, [VP, VP, VP, SZ, SZ, ctypes.c_float, VP]),
    "brasa_rope_neox": (INT, [VP, RopeTableC, SZ, SZ, SZ, SZ, VP]),
    "brasa_qk_norm_rope_store": (INT, [INT, VP, VP, VP, VP, VP, ctypes.c_float, RopeTableC, VP,
                                       VP, AttnShapeC, VP]),
    "brasa_test_flash_attention_layout": (INT, [VP, VP, VP, VP, AttnShapeC, INT, INT, INT, INT,
                                                VP]),
    "brasa_test_stream_slot": (INT, [INT, VP, ctypes.POINTER(INT)]),
    "brasa_test_decode_plan": (INT, [VP, INT, INT, INT, INT, ctypes.POINTER(INT),
                                     ctypes.POINTER(INT), VP]),
    "brasa_test_split_blocks": (INT, [INT, INT, INT, ctypes.POINTER(INT), ctypes.POINTER(INT),
                                      ctypes.POINTER(INT)]),
    "brasa_release_workspaces": (INT, []),
    "brasa_last_error": (ctypes.c_char_p, []),
    "brasa_version": (ctypes.c_char_p, []),
    "brasa_rt_device_count": (INT, [ctypes.POINTER(INT)]),
    "brasa_rt_set_device": (INT, [INT]),
    "brasa_rt_device_name": (INT, [ctypes.c_char_p, SZ]),
    "brasa_rt_malloc": (INT, [ctypes.POINTER(VP), SZ]),
    "brasa_rt_free": (INT, [VP]),
    "brasa_rt_memcpy_htod": (INT, [VP, VP, SZ]),
    "brasa_rt_memcpy_dtoh": (INT, [VP, VP, SZ]),
    "brasa_rt_memcpy_dtod": (INT, [VP, VP, SZ, VP]),
    "brasa_rt_fill_u8": (INT, [VP, ctypes.c_uint8, SZ, VP]),
    "brasa_rt_device_synchronize": (INT, []),
    "brasa_rt_stream_create": (INT, [ctypes.POINTER(VP)]),
    "brasa_rt_stream_destroy": (INT, [VP]),
    "brasa_rt_stream_synchronize": (INT, [VP]),
    "brasa_rt_event_create": (INT, [ctypes.POINTER(VP)]),
    "brasa_rt_event_destroy": (INT, [VP]),
    "brasa_rt_event_record": (INT, [VP, VP]),
    "brasa_rt_event_elapsed_ms": (INT, [ctypes.POINTER(ctypes.c_float), VP, VP]),
    "brasa_rt_event_synchronize": (INT, [VP]),
    "brasa_rt_stream_begin_capture": (INT, [VP]),
    "brasa_rt_stream_end_capture": (INT, [VP, ctypes.POINTER(VP)]),
    "brasa_rt_graph_launch": (INT, [VP, VP]),
    "brasa_rt_graph_destroy": (INT, [VP]),
    "brasa_rt_mem_info": (INT, [ctypes.POINTER(SZ), ctypes.POINTER(SZ)]),
    "brasa_rt_fill_normal_f32": (INT, [VP, SZ, ctypes.c_uint64, ctypes.c_float, VP]),
}


def build(jobs: int = 8) -> None:
    """Compile libbrasa_attn.so for gfx950 with hipcc (always rebuilds)."""
    subprocess.run(["make", "-s", "-C", CSRC, "-B", f"-j{jobs}"], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {CSRC}` or "
                "`python -c 'import __graft_entry__ as g; g.build()'` (no CPU fallback exists)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SYMBOLS.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


class BrasaError(RuntimeError):
    """A nonzero status from the C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def check(status: int) -> None:
    if status != 0:
        raise BrasaError(status, lib().brasa_last_error().decode())
