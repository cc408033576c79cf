"""CPU: the C ABI library loads, exports every symbol the public headers declare, and rejects
bad calls with the reference's assert conditions before touching the device (no GPU needed).
"""
import ctypes
import os
import re

import pytest

import brasa_amd
from brasa_amd import AttnShape, BrasaError, Kernels, KvType, decode_partials_len, gqa_supported
from brasa_amd._lib import SYMBOLS, lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


TRACE_BLOCK = re.compile(r"#ifdef BRASA_TIMELINE_BUILD(.*?)#endif", flags=re.S)


def _declared(trace=False):
    """Names the public headers declare: those of the default library, or with trace=True only
    those of the timeline build (declared under #ifdef BRASA_TIMELINE_BUILD)."""
    names = set()
    for h in ("brasa_attn.h", "brasa_hip_rt.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        if trace:
            text = "\n".join(TRACE_BLOCK.findall(text))
        else:
            text = TRACE_BLOCK.sub("", text)
        names |= set(re.findall(r"\b(brasa_\w+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported_and_bound():
    declared = _declared()
    assert len(declared) >= 30
    l = ctypes.CDLL(brasa_amd.LIB_PATH)
    for name in declared:
        assert hasattr(l, name), name
    assert declared == set(SYMBOLS), declared ^ set(SYMBOLS)


def test_timeline_build_exports_the_trace_reader():
    path = os.path.join(ROOT, "brasa_amd", "libbrasa_attn_trace.so")
    if not os.path.exists(path):
        pytest.skip("timeline build not compiled")
    l = ctypes.CDLL(path)
    trace = _declared(trace=True)
    assert trace == {"brasa_decode_trace_read", "brasa_prefill_trace_read"}
    for name in trace | _declared():
        assert hasattr(l, name), name
    for name in trace:
        assert not hasattr(ctypes.CDLL(brasa_amd.LIB_PATH), name), name


def test_built_for_gfx950_only():
    data = open(brasa_amd.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    for other in (b"amdgcn-amd-amdhsa--gfx942", b"amdgcn-amd-amdhsa--gfx90a"):
        assert other not in data


def test_constants_mirror_reference():
    # lib.rs:1323-1351
    assert decode_partials_len(32, 16384) == 32 * 128 * 130
    assert decode_partials_len(32, 1) == 32 * 130
    assert decode_partials_len(32, 129) == 32 * 2 * 130
    assert all(gqa_supported(8 * g, 8) for g in (1, 2, 4, 8))
    assert not gqa_supported(24, 8) and not gqa_supported(32, 0) and not gqa_supported(30, 8)
    assert KvType.F16.bytes(128) == 256 and KvType.F32.bytes(128) == 512
    assert KvType.Q8_0.bytes(256) == 272
    assert lib().brasa_kv_bytes(2, 256) == 272
    assert lib().brasa_kv_bytes(2, 100) == 0
    assert KvType.parse("q8") == KvType.Q8_0 and KvType.parse("bf16") is None


def _err(fn):
    with pytest.raises(BrasaError) as e:
        fn()
    return e.value.code


def test_decode_asserts_without_device():
    k = Kernels()
    # the checks run before any pointer is dereferenced, so fake addresses are fine
    fake = 0x1000

    class P:  # partials stand-in with a byte size
        def __init__(self, nbytes):
            self.nbytes, self.ptr = nbytes, fake

    big = P(4 * decode_partials_len(32, 1 << 20))
    sh = lambda **kw: AttnShape(**{**dict(tokens=1, hq=32, hkv=8, dim=128, pos0=99,
                                          kv=KvType.F16), **kw})
    assert _err(lambda: k.decode_attention_lanes(fake, fake, fake, big, fake, sh(tokens=2))) == 1
    assert _err(lambda: k.decode_attention_lanes(fake, fake, fake, big, fake, sh(dim=64))) == 1
    assert _err(lambda: k.decode_attention_lanes(fake, fake, fake, big, fake, sh(hq=30))) == 1
    assert _err(lambda: k.decode_attention_lanes(fake, fake, fake, big, fake, sh(hq=24))) == 3
    assert _err(lambda: k.decode_attention_lanes(fake, fake, fake, P(4 * (32 * 130 - 1)), fake,
                                                 sh(pos0=0))) == 2
    assert _err(lambda: k.decode_attention_lanes(0, fake, fake, big, fake, sh())) == 5
    assert "scratch" in _scratch_msg(k, fake, P)


def _scratch_msg(k, fake, P):
    try:
        k.decode_attention(fake, fake, fake, P(4), fake,
                           AttnShape(1, 32, 8, 128, 500, KvType.F16))
    except BrasaError as e:
        return str(e)
    return ""


def test_prefill_and_store_asserts_without_device():
    k = Kernels()
    fake = 0x1000
    sh = AttnShape(16, 32, 8, 64, 0, KvType.F16)
    assert _err(lambda: k.flash_attention(fake, fake, fake, fake, sh)) == 1
    assert _err(lambda: k.flash_attention(fake, fake, fake, fake,
                                          AttnShape(16, 30, 8, 128, 0, KvType.F16))) == 1
    assert _err(lambda: k.flash_attention_with(fake, fake, fake, fake,
                                               AttnShape(16, 32, 8, 128, 0, KvType.F16), 7)) == 5
    # lib.rs:1227-1231: a group outside {1, 2, 4, 8} has only the f32 kernel
    for prec in (0, 2):
        assert _err(lambda: k.flash_attention_with(fake, fake, fake, fake,
                                                   AttnShape(16, 24, 8, 128, 0, KvType.F16),
                                                   prec)) == 3
    assert _err(lambda: k.store_kv(KvType.Q8_0, fake, fake, 100)) == 1
    assert _err(lambda: k.store_kv(9, fake, fake, 128)) == 5
    # zero-size calls are no-ops
    k.store_kv(KvType.F16, fake, fake, 0)
    k.flash_attention(fake, fake, fake, fake, AttnShape(0, 32, 8, 128, 5, KvType.F16))


class _FakeTable:
    """A RoPE table view with fake device addresses (the calls below fail before any launch)."""

    def __init__(self, dim, max_pos):
        self.dim, self.max_pos = dim, max_pos

    def c(self):
        from brasa_amd._lib import RopeTableC
        return RopeTableC(0x2000, 0x3000, self.dim, self.max_pos)


def test_qkv_asserts_without_device():
    k = Kernels()
    fake = 0x1000
    t = _FakeTable(128, 4096)
    ok = AttnShape(5, 32, 8, 128, 37, KvType.F16)
    qkv, norms, dst = (fake, fake, fake), (fake, fake), (fake, fake)
    # lib.rs:996-1001: head_dim 128, table dimension, position inside the table
    assert _err(lambda: k.qk_norm_rope_store(KvType.F16, qkv, norms, 1e-6, t, dst,
                                             AttnShape(5, 32, 8, 64, 37, KvType.F16))) == 1
    assert _err(lambda: k.qk_norm_rope_store(KvType.F16, qkv, norms, 1e-6, _FakeTable(64, 4096),
                                             dst, ok)) == 1
    assert _err(lambda: k.qk_norm_rope_store(KvType.F16, qkv, norms, 1e-6, _FakeTable(128, 41),
                                             dst, ok)) == 1
    assert _err(lambda: k.qk_norm_rope_store(7, qkv, norms, 1e-6, t, dst, ok)) == 5
    assert _err(lambda: k.qk_norm_rope_store(KvType.F16, (fake, 0, fake), norms, 1e-6, t, dst,
                                             ok)) == 5
    # lib.rs:579-583
    assert _err(lambda: k.rope_neox(fake, t, 16, 32, 128, 4081)) == 1
    assert _err(lambda: k.rope_neox(fake, t, 16, 32, 64, 0)) == 1
    assert _err(lambda: k.rms_norm(fake, fake, fake, 4, 0, 1e-6)) == 1
    # zero-size calls are no-ops
    k.qk_norm_rope_store(KvType.F16, qkv, norms, 1e-6, t, dst,
                         AttnShape(0, 32, 8, 128, 37, KvType.F16))
    k.rms_norm(fake, fake, fake, 0, 128, 1e-6)


def test_rope_table_host_matches_oracle():
    """brasa_rope_table runs on the host: same f32 bits as the oracle's f64 table
    (lib.rs:1388-1404), including large positions."""
    import numpy as np
    import oracle
    cos, sin = brasa_amd.rope_table(1e6, 128, 40960)
    oc, os_ = oracle.rope_table(1e6, 128, 40960)
    assert np.array_equal(cos.ravel().view(np.uint32), np.asarray(oc).view(np.uint32))
    assert np.array_equal(sin.ravel().view(np.uint32), np.asarray(os_).view(np.uint32))
    # position 0 is the identity; p * inv_freq for i = 0 is p radians
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    assert cos[1000, 0] == np.float32(np.cos(1000.0))


def test_decode_noalloc_asserts_without_device():
    k = Kernels()
    fake = 0x1000
    assert _err(lambda: k.decode_attention_lanes_noalloc(
        fake, fake, fake, fake, AttnShape(2, 32, 8, 128, 5, KvType.F16))) == 1
    assert _err(lambda: k.decode_attention_lanes_noalloc(
        fake, fake, fake, fake, AttnShape(1, 24, 8, 128, 5, KvType.F16))) == 3
    assert _err(lambda: k.decode_attention_lanes_noalloc(
        fake, fake, 0, fake, AttnShape(1, 32, 8, 128, 5, KvType.F16))) == 5


def test_decode_batch_asserts_without_device():
    k = Kernels()
    fake = 0x1000

    class Part:
        ptr, nbytes = 0x1000, 4 << 20

    lens = [100, 3000]
    need = brasa_amd.decode_batch_partials_len(32, lens)
    assert lib().brasa_decode_batch_partials_len(
        32, (ctypes.c_size_t * 2)(*lens), 2) == need
    # a sequence without keys, a bad group, a small scratch, head_dim != 128 is fixed at 128
    assert _err(lambda: k.decode_attention_batch(fake, [fake, fake], [fake, fake], [0, 5], Part,
                                                 fake, 32, 8, KvType.F16)) == 1
    assert _err(lambda: k.decode_attention_batch(fake, [fake], [fake], [5], Part, fake, 24, 8,
                                                 KvType.F16)) == 3
    assert _err(lambda: k.decode_attention_batch(fake, [fake, fake], [fake, fake], lens, Part,
                                                 fake, 32, 8, KvType.F16,
                                                 partials_len=need - 1)) == 2
    assert _err(lambda: k.decode_attention_batch(fake, [fake, 0], [fake, fake], lens, Part,
                                                 fake, 32, 8, KvType.F16)) == 5
    # an empty batch is a no-op
    k.decode_attention_batch(fake, [], [], [], Part, fake, 32, 8, KvType.F16)


def test_prefill_layout_entry_validates():
    """The per-call layout of brasa_test_flash_attention_layout is checked before anything is
    enqueued (no GPU needed: the errors come first)."""
    from brasa_amd import AttnShape, KvType, PrefillPrecision
    from brasa_amd._lib import BrasaError, check
    shape = AttnShape(64, 32, 8, 128, 0, KvType.F16).c()
    for bad in [(3, 1, 1), (1, 1, 0), (1, 1, 9)]:
        with pytest.raises(BrasaError):
            check(lib().brasa_test_flash_attention_layout(1, 1, 1, 1, shape,
                                                          int(PrefillPrecision.F16), *bad, None))


def test_stream_slots():
    """Counter slots are per stream: a stream keeps its slot, distinct streams get distinct
    slots, the 65th stream on a device gets none (-1), hipStreamPerThread gets one per host
    thread, and brasa_release_workspaces() starts the assignment over. (Stream handles are
    only keys here; no GPU is touched.)"""
    import threading
    from brasa_amd._lib import check

    def slot(dev, handle):
        s = ctypes.c_int(-2)
        check(lib().brasa_test_stream_slot(dev, handle, ctypes.byref(s)))
        return s.value

    dev = 63  # a device index no other test uses
    check(lib().brasa_release_workspaces())
    first = [slot(dev, 0x5000 + 16 * i) for i in range(64)]
    assert sorted(first) == list(range(64))
    assert [slot(dev, 0x5000 + 16 * i) for i in range(64)] == first  # stable
    assert slot(dev, 0x9000) == -1                                   # all 64 taken
    assert slot(dev - 1, 0x9000) == 0                                # per device
    check(lib().brasa_release_workspaces())
    assert slot(dev, 0x9000) == 0
    per_thread = 2  # hipStreamPerThread: one stream per live host thread
    got = []
    bar = threading.Barrier(3)

    def look():
        got.append(slot(dev, per_thread))
        bar.wait()  # every thread alive until all have looked up (thread ids can be reused)

    ts = [threading.Thread(target=look) for _ in range(3)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert sorted(got) == [1, 2, 3]
    check(lib().brasa_release_workspaces())
    with pytest.raises(Exception):
        check(lib().brasa_test_stream_slot(64, None, ctypes.byref(ctypes.c_int())))


def test_prefill_workspace_len():
    """Workspace sizes of brasa_flash_attention_ws: none for a full launch, the key split's
    partials for a short chunk after a long prefix, the f16 staging (512 B per row of K and V
    read) plus its key split for q8_0."""
    from brasa_amd import AttnShape, Kernels, PrefillPrecision
    wl = Kernels.flash_attention_workspace_len
    F16 = PrefillPrecision.F16
    assert wl(AttnShape(2048, 32, 8, 128, 0, KvType.F16), F16) == 0
    assert wl(AttnShape(2048, 32, 8, 128, 0, KvType.F16), PrefillPrecision.F32) == 0
    # 512 tokens after 16384: 128 workgroups, two key parts of 68 KB per query tile
    assert wl(AttnShape(512, 32, 8, 128, 16384, KvType.F16), F16) == 128 * 2 * 4 * 17 * 64 * 16
    staging = 2048 * 8 * 128 * 2 * 2
    assert wl(AttnShape(2048, 32, 8, 128, 0, KvType.Q8_0), F16) == staging
    assert wl(AttnShape(2048, 32, 8, 128, 0, KvType.Q8_0), PrefillPrecision.F16_PF32) == 0
    assert wl(AttnShape(512, 32, 8, 128, 16384, KvType.Q8_0), F16) == \
        16896 * 8 * 128 * 2 * 2 + 128 * 2 * 4 * 17 * 64 * 16
    assert wl(AttnShape(0, 32, 8, 128, 0, KvType.F16), F16) == 0
    assert wl(AttnShape(16, 32, 8, 64, 0, KvType.F16), F16) == 0  # invalid shape


def _plan(lens, hq=32, hkv=8, kv=KvType.F16):
    from brasa_amd._lib import check
    arr = (ctypes.c_int * len(lens))(*lens)
    splits = (ctypes.c_int * len(lens))()
    chunk, hpw = ctypes.c_int(), ctypes.c_int()
    check(lib().brasa_test_decode_plan(arr, len(lens), hq, hkv, int(kv), ctypes.byref(chunk),
                                       ctypes.byref(hpw), splits))
    return chunk.value, hpw.value, list(splits)


def _blocks(lk, splits, split):
    from brasa_amd._lib import check
    f, st, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(lib().brasa_test_split_blocks(lk, splits, split, ctypes.byref(f), ctypes.byref(st),
                                        ctypes.byref(n)))
    return [f.value + st.value * i for i in range(n.value)]


@pytest.mark.parametrize("lens,hq,hkv,kv", [
    ([1], 32, 8, KvType.F16), ([37], 32, 8, KvType.Q8_0), ([128], 32, 8, KvType.F16),
    ([129], 32, 8, KvType.F16), ([2048], 32, 8, KvType.F16), ([4096], 32, 8, KvType.Q8_0),
    ([5889], 32, 8, KvType.F16), ([16384], 32, 8, KvType.F16), ([16384], 32, 8, KvType.Q8_0),
    ([32768], 32, 8, KvType.F16), ([131072], 32, 8, KvType.F16), ([16384], 32, 32, KvType.F16),
    ([4095], 64, 8, KvType.F32),
    ([11764, 4516, 13138, 5889, 4160, 13272, 10896, 11411], 32, 8, KvType.F16),
    ([11764, 4516, 13138, 5889, 4160, 13272, 10896, 11411], 32, 8, KvType.Q8_0),
    ([1, 2, 37, 64, 65, 127, 128, 129, 300, 1025, 3000] * 5 + [5, 999, 2048, 17], 32, 8,
     KvType.F16)])
def test_decode_splits_partition_the_keys(lens, hq, hkv, kv):
    """The decode plan and the kernels' split_blocks, called through the library: for every
    sequence, the splits' 32-key blocks (interleaved: block s + S i of split s) cover each of its
    blocks exactly once, every split has at least one block and at most chunk / 32, the split
    count stays within the reference-sized scratch (ceil(lk / 128) splits), chunks are multiples
    of 32 keys and at least 128, and only the sequence's last block reaches past lk."""
    chunk, hpw, splits = _plan(lens, hq, hkv, kv)
    assert chunk % 32 == 0 and chunk >= 128 and hpw in (1, 2, 4)
    for lk, s in zip(lens, splits):
        assert s == -(-lk // chunk) and s <= -(-lk // 128)
        seen = []
        for sp in range(s):
            b = _blocks(lk, s, sp)
            assert 1 <= len(b) <= chunk // 32, (lk, s, sp, len(b))
            assert all(k % 32 == 0 and k < lk for k in b)
            seen += b
        assert sorted(seen) == list(range(0, lk, 32)), lk
