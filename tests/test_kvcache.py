"""CPU: the KV cache layout formulas (brasa_kv_capacity / _cache_len / _offset and the q8_0 byte
conversion) against the reference's: qwen3.rs:384-386 (capacity), :386 (buffer length),
:554-556 (layer and block views), KvCache::args :246-257 (q8_0 offsets to bytes), and the memory
planner's kv_bytes (planner.rs:77-81) with its own known answer for Qwen3-4B at 16K f32
(planner.rs:223-229: 2 * 36 * 16384 * 8 * 128 * 4 bytes, 4.5 GiB).
"""
import pytest

from brasa_amd import (KV_ALIGN, BrasaError, KvType, kv_cache_bytes, kv_cache_len, kv_capacity,
                       kv_offset)

LAYERS, HKV, DIM = 36, 8, 128


def test_planner_known_answer():
    # planner.rs:223-229
    assert kv_cache_bytes(KvType.F32, LAYERS, 16384, HKV) == 2 * 36 * 16384 * 8 * 128 * 4
    assert kv_cache_bytes(KvType.F32, LAYERS, 16384, HKV) / 2**30 == 4.5


@pytest.mark.parametrize("kv,block", [(KvType.F32, 128), (KvType.F16, 64), (KvType.Q8_0, 34)])
@pytest.mark.parametrize("ctx", [1, 63, 64, 65, 1000, 4096, 16384, 40000])
def test_kv_bytes_is_planner_formula(kv, block, ctx):
    # planner.rs:77-81: cap = ctx.next_multiple_of(KV_ALIGN);
    # 2 * elems.div_ceil(32) * kv_block_bytes (f32 128, f16 64, q8_0 34 per 32 values)
    cap = -(-ctx // KV_ALIGN) * KV_ALIGN
    elems = LAYERS * cap * HKV * DIM
    assert kv_capacity(ctx) == cap
    assert kv_cache_len(LAYERS, ctx, HKV, DIM) == elems
    assert kv_cache_bytes(kv, LAYERS, ctx, HKV, DIM) == 2 * (-(-elems // 32)) * block


def test_capacity_rounds_up_to_kv_align():
    assert [kv_capacity(c) for c in (0, 1, 64, 65, 128, 129)] == [0, 64, 64, 128, 128, 192]


@pytest.mark.parametrize("ctx", [100, 4096, 16385])
def test_views_follow_encode_layer(ctx):
    # qwen3.rs:554-556: kv_off = (li * cap + pos0) * kvd, layer_off = li * cap * kvd
    cap, kvd = kv_capacity(ctx), HKV * DIM
    for li in (0, 1, 17, 35):
        assert kv_offset(li, ctx, HKV, 0, DIM) == li * cap * kvd
        for pos0 in (0, 1, 77, cap - 1):
            off = kv_offset(li, ctx, HKV, pos0, DIM)
            assert off == (li * cap + pos0) * kvd
            # KvCache::args (qwen3.rs:246-257): q8_0 views are the byte of row off / 128
            assert KvType.Q8_0.bytes(off) == off // 128 * 136
            assert KvType.F16.bytes(off) == 2 * off and KvType.F32.bytes(off) == 4 * off
    # the last position of the last layer ends exactly at the buffer end
    end = kv_offset(LAYERS - 1, ctx, HKV, cap - 1, DIM) + kvd
    assert end == kv_cache_len(LAYERS, ctx, HKV, DIM)


def test_q8_offsets_must_be_whole_rows():
    # KvType::bytes asserts n % KV_Q8_DIM == 0 for q8_0 (lib.rs:112-121)
    with pytest.raises(BrasaError):
        KvType.Q8_0.bytes(64)
