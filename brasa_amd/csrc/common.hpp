// Shared device helpers for the gfx950 attention kernels: KV-row access per cache type, f16
// conversion, wave64 cross-lane reductions and the error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstdlib>

#include "../../include/brasa_attn.h"

namespace brasa {

constexpr int kDim = 128;        // head_dim (the reference asserts 128 on every attention path)
constexpr int kQ8Row = 136;      // 128 int8 + 4 f16 scales
constexpr float kLog2e = 1.4426950408889634f;

// ---- host-side error plumbing -------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---- per-stream slots of the library's device-side launch state (slots.hip) ----------------
constexpr int kMaxDevices = 64;
constexpr int kStreamSlots = 64;
// The current device and the slot of `stream` on it (0 .. kStreamSlots - 1, the same slot for
// every call on that stream until release_stream_slots()); slot -1 when every slot of the
// device is taken.
int stream_slot(hipStream_t stream, int* dev, int* slot);
void release_stream_slots();

// Decode launch plan (decode.hip): keys per split, splits of the longest sequence, and head
// groups per workgroup.
struct DecodePlan {
    int chunk;
    int splits;
    int hpw;
};
DecodePlan decode_plan(const int* lk, int n, int ngroups, int G, int kv);

// The 32-key blocks of split `split` of a sequence of lk keys cut into `splits` splits: blocks
// split, split + splits, split + 2 splits, ... of the sequence, interleaved with the other splits'
// so that at any time the grid reads one region of the cache. `first` is the first block's key,
// `stride` the keys from one of the split's blocks to the next, `count` its blocks (at least one
// whenever blocks >= splits; only the sequence's last block can be partial).
struct SplitBlocks {
    int first;
    int stride;
    int count;
};
__host__ __device__ inline SplitBlocks split_blocks(int lk, int splits, int split) {
    const int nblocks = (lk + 31) / 32;
    return SplitBlocks{32 * split, 32 * splits, (nblocks - split + splits - 1) / splits};
}

// ---- f16 helpers --------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__ushort_as_half(h));
}
// v_cvt_f16_f32: round to nearest even, overflow to inf, f16 subnormals kept.
__device__ __forceinline__ uint16_t f2h(float f) {
    return __half_as_ushort(__float2half_rn(f));
}
// Materialises x as an f32 register value. The backend otherwise folds f16(a * b) into one
// v_fma_mixlo_f16 (a single rounding of the exact product), whereas the reference rounds the
// product to f32 first and then to f16. The empty asm emits no instruction.
__device__ __forceinline__ float as_f32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// ---- q8_0 quantisation of one 32-group (quantize_kv_q8, crates/quant/src/qtype.rs:85-111) ----
// d = f16(amax / 127) with an IEEE f32 divide rounded to nearest even in f16.
__device__ __forceinline__ uint16_t q8_scale_bits(float amax) { return f2h(amax / 127.0f); }
// q = d == 0 ? 0 : clamp(round_ties_even(x / d), -127, 127), as the int8 byte.
__device__ __forceinline__ uint32_t q8_code(float x, float d) {
    float qv = 0.0f;
    if (d != 0.0f) qv = fminf(fmaxf(rintf(x / d), -127.0f), 127.0f);
    return (uint32_t)(uint8_t)(int8_t)qv;
}

// 4 int8 codes (one dword) -> 4 exact f16 values: f16 bits 0x6400 | (code + 128) encode
// 1024 + code + 128, minus 1152 (exact in f16 for these integers)
__device__ __forceinline__ void codes4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t x = w ^ 0x80808080u;
    const uint32_t l = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);  // [64, b1, 64, b0]
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);  // [64, b3, 64, b2]
    typedef _Float16 half2 __attribute__((ext_vector_type(2)));
    const half2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, l) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, h) + bias);
}

// As codes4_to_f16 with the values scaled by 2^e, -14 <= e <= 5: the magic's exponent byte
// ebyte = 4 (e + 25) (in every byte) encodes 2^e (1024 + code + 128), and bias = -1152 * 2^e
// (a normal f16 in that range) leaves code * 2^e, exact (7 significant bits, >= 2^-14 steps).
__device__ __forceinline__ void codes4_to_f16_exp(uint32_t w, uint32_t ebyte, uint32_t bias,
                                                  uint32_t& lo, uint32_t& hi) {
    const uint32_t x = w ^ 0x80808080u;
    const uint32_t l = __builtin_amdgcn_perm(ebyte, x, 0x04010400u);  // [e, b1, e, b0]
    const uint32_t h = __builtin_amdgcn_perm(ebyte, x, 0x04030402u);  // [e, b3, e, b2]
    typedef _Float16 half2 __attribute__((ext_vector_type(2)));
    const half2 b = __builtin_bit_cast(half2, bias);
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, l) + b);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, h) + b);
}

// ---- DPP / cross-lane helpers (wave64) ----------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Sum over the 16 lanes of a DPP row with a butterfly of xor masks 15, 7, 3, 1 (row_mirror,
// row_half_mirror, quad_perm [3,2,1,0], quad_perm [1,0,3,2]). Partners add the same two values,
// so every lane of the row ends with identical bits.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp<0x140>(x);
    x += dpp<0x141>(x);
    x += dpp<0x1B>(x);
    x += dpp<0xB1>(x);
    return x;
}

// ---- KV row access ------------------------------------------------------------------------
// Cache element types, one per KvType value.
template <int KV> struct KvTraits;
template <> struct KvTraits<BRASA_KV_F32> { static constexpr int row_bytes = 512; };
template <> struct KvTraits<BRASA_KV_F16> { static constexpr int row_bytes = 256; };
template <> struct KvTraits<BRASA_KV_Q8_0> { static constexpr int row_bytes = kQ8Row; };

// Eight consecutive values [d0, d0 + 8) of a cache row, in their storage form. For q8_0 the
// values are the raw int8 codes and `scale` is the f16 scale of their 32-group (exact product:
// value = scale * code, as dequantize_kv_q8).
template <int KV> struct Kv8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Streaming loads: K/V rows are read once per kernel, so they should not displace reused data.
template <typename T>
__device__ __forceinline__ T ld_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const T*>(p));
}

template <> struct Kv8<BRASA_KV_F16> {
    u32x4 raw;
    __device__ __forceinline__ void load(const uint8_t* row, int d0) {
        raw = ld_stream<u32x4>(row + 2 * d0);
    }
    __device__ __forceinline__ void to_float(float (&x)[8]) const {
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = h2f(static_cast<uint16_t>(w[i] & 0xffffu));
            x[2 * i + 1] = h2f(static_cast<uint16_t>(w[i] >> 16));
        }
    }
    __device__ __forceinline__ float scale() const { return 1.0f; }
};

template <> struct Kv8<BRASA_KV_F32> {
    f32x4 a, b;
    __device__ __forceinline__ void load(const uint8_t* row, int d0) {
        a = ld_stream<f32x4>(row + 4 * d0);
        b = ld_stream<f32x4>(row + 4 * d0 + 16);
    }
    __device__ __forceinline__ void to_float(float (&x)[8]) const {
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
    __device__ __forceinline__ float scale() const { return 1.0f; }
};

template <> struct Kv8<BRASA_KV_Q8_0> {
    u32x2 raw;
    uint16_t sc;
    __device__ __forceinline__ void load(const uint8_t* row, int d0) {
        // rows are 136 bytes: 8-byte aligned, so the 8 codes are one dwordx2
        raw = ld_stream<u32x2>(row + d0);
        sc = *reinterpret_cast<const uint16_t*>(row + 128 + 2 * (d0 >> 5));
    }
    __device__ __forceinline__ void to_float(float (&x)[8]) const {
        const uint32_t w[2] = {raw.x, raw.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int b = 0; b < 4; ++b)
                x[4 * i + b] = static_cast<float>(static_cast<int8_t>((w[i] >> (8 * b)) & 0xffu));
        }
    }
    __device__ __forceinline__ float scale() const { return h2f(sc); }
};

// 16-byte HBM -> LDS copy per lane (global_load_lds_dwordx4): lane i writes lds + 16 i.
// M0 (the LDS base) is saved and restored around it. An LDS-DMA load needs a wait state after
// an SALU write of M0, which the compiler cannot insert inside the asm (the s_nop). The SGPR
// base of the _s variants comes from sgpr_offset (an SALU write). Issued as
// inline asm so that the compiler's vector-memory counter bookkeeping never relies on it (its
// own waits can only become more conservative); the wait before the LDS reads of such a tile
// is wait_vmcnt below.
__device__ __forceinline__ void lds_dma16(const uint8_t* src, uint16_t* lds_wave_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)lds_wave_base);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 2\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(m0)
        : "memory");
}
// As lds_dma16 with the nontemporal hint, for data read exactly once (K/V rows).
__device__ __forceinline__ void lds_dma16_nt(const uint8_t* src, uint16_t* lds_wave_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)lds_wave_base);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 2\n\t"
        "global_load_lds_dwordx4 %1, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(m0)
        : "memory");
}
// Uniform 64-bit addresses as the SGPR pairs the _s copy helpers read. The compiler may hold
// a uniform value in VGPRs and move it to SGPRs with v_readfirstlane (a VALU write of the SGPRs)
// just before the copy. On gfx950 a vector memory instruction that read the SGPRs 5 wait states
// after that write copied from a wrong base now and then (q8_0 decode at 16K keys: whole KV
// heads wrong or NaN in most calls); with 18 wait states no call in 24 was.
// sgpr_base: once per kernel for a cache base; the asm that holds the SGPRs pads 18 wait states
// after their write.
__device__ __forceinline__ const uint8_t* sgpr_base(const uint8_t* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" : "+s"(lo), "+s"(hi));
    return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}
// sgpr_offset: a block's address, base (from sgpr_base) + a uniform byte offset, summed by SALU
// instructions in the asm, so the copies read SGPRs no VALU instruction wrote (a VALU write of
// the offset's SGPRs read by those SALU instructions needs no wait states).
__device__ __forceinline__ const uint8_t* sgpr_offset(const uint8_t* sbase, uint64_t off) {
    const uint64_t b = reinterpret_cast<uint64_t>(sbase);
    const uint32_t olo = __builtin_amdgcn_readfirstlane((uint32_t)off);
    const uint32_t ohi = __builtin_amdgcn_readfirstlane((uint32_t)(off >> 32));
    uint32_t lo, hi;
    asm volatile("s_add_u32 %0, %2, %4\n\ts_addc_u32 %1, %3, %5"
                 : "=&s"(lo), "=&s"(hi)
                 : "s"((uint32_t)b), "s"((uint32_t)(b >> 32)), "s"(olo), "s"(ohi)
                 : "scc");
    return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}
// As lds_dma16 with a uniform 64-bit base in SGPRs (from sgpr_offset) and a per-lane 32-bit
// byte offset.
__device__ __forceinline__ void lds_dma16_s(const uint8_t* sbase, uint32_t voff,
                                            uint32_t lds_wave_base /* uniform LDS address */) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 2\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sbase), "s"(lds_wave_base)
        : "memory");
}
// 4-byte variant of lds_dma16_s (lane i writes lds + 4 i).
__device__ __forceinline__ void lds_dma4_s(const uint8_t* sbase, uint32_t voff,
                                           uint32_t lds_wave_base /* uniform LDS address */) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 2\n\t"
        "global_load_lds_dword %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sbase), "s"(lds_wave_base)
        : "memory");
}
// Device-coherent stores and loads (written through / read past the XCD's L2): a partial
// stored by a workgroup on one XCD is then visible to the merging workgroup on any other.
__device__ __forceinline__ void st_dev16(float* p, f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_dev8(float* p, f32x2 v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ f32x4 ld_dev16(const float* p) {
    f32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(r) : "v"(p) : "memory");
    return r;
}
__device__ __forceinline__ f32x2 ld_dev8(const float* p) {
    f32x2 r;
    asm volatile("global_load_dwordx2 %0, %1, off sc1" : "=v"(r) : "v"(p) : "memory");
    return r;
}

// LDS address of a __shared__ location, as a 32-bit value.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited), then a compiler memory barrier.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
}

}  // namespace brasa
