// KV-cache writers and the q8_0 dequantiser for gfx950.
//
// store_kv (crates/kernels/src/lib.rs:1029-1050; kv.metal:6-40) converts an f32 scratch into
// the cache type: f32 copy, f16 round-to-nearest-even (v_cvt_f16_f32), q8_0 per 32-group
// d = f16(amax / 127), q = d == 0 ? 0 : clamp(rint(x / d), -127, 127) with IEEE f32 divides
// (hipcc's default correctly rounded division) and v_rndne_f32 (ties to even), bit-exact with
// quantize_kv_q8 (crates/quant/src/qtype.rs:85-111).
//
// The writers are HBM-bound streams: f16 moves 4 values (16 B in, 8 B out) per thread; q8_0
// gives each 32-group to 8 consecutive lanes (4 values each), so a wave quantises 2 full rows
// with 128-bit loads and reduces amax with 3 xor shuffles.
#include "common.hpp"

namespace brasa {
namespace {

constexpr int kTpb = 256;

__global__ void store_f32_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                 size_t n) {
    const size_t i = (size_t)blockIdx.x * kTpb + threadIdx.x;
    const size_t base = 4 * i;
    if (base + 4 <= n) {
        reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(src)[i];
    } else {
        for (size_t e = base; e < n; ++e) dst[e] = src[e];
    }
}

__global__ void store_f16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                 size_t n) {
    const size_t i = (size_t)blockIdx.x * kTpb + threadIdx.x;
    const size_t base = 4 * i;
    if (base + 4 <= n) {
        const float4 x = reinterpret_cast<const float4*>(src)[i];
        uint2 w;
        w.x = (uint32_t)f2h(x.x) | ((uint32_t)f2h(x.y) << 16);
        w.y = (uint32_t)f2h(x.z) | ((uint32_t)f2h(x.w) << 16);
        reinterpret_cast<uint2*>(dst)[i] = w;
    } else {
        for (size_t e = base; e < n; ++e) dst[e] = f2h(src[e]);
    }
}

// 8 lanes per 32-group; groups = n / 32 (n a multiple of 128).
__global__ void store_q8_kernel(const float* __restrict__ src, uint8_t* __restrict__ dst,
                                size_t groups) {
    const size_t t = (size_t)blockIdx.x * kTpb + threadIdx.x;
    const size_t grp = t >> 3;
    const int sub = threadIdx.x & 7;
    // every lane of a wave takes part in the shuffles; lanes past the end use group 0's data
    const size_t g = grp < groups ? grp : 0;
    const float4 x = reinterpret_cast<const float4*>(src + g * 32)[sub];
    float amax = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    if (grp >= groups) return;
    const uint16_t dh = q8_scale_bits(amax);
    const float d = h2f(dh);
    const float xs[4] = {x.x, x.y, x.z, x.w};
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) packed |= q8_code(xs[e], d) << (8 * e);
    uint8_t* row = dst + (grp >> 2) * kQ8Row;
    const int b = (int)(grp & 3);
    *reinterpret_cast<uint32_t*>(row + 32 * b + 4 * sub) = packed;
    if (sub == 0) *reinterpret_cast<uint16_t*>(row + 128 + 2 * b) = dh;
}

// dequantize_kv_q8 (qtype.rs:113-130): 16 threads per row, 8 values each.
__global__ void dequant_q8_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                  size_t rows) {
    const size_t t = (size_t)blockIdx.x * kTpb + threadIdx.x;
    const size_t row = t >> 4;
    if (row >= rows) return;
    const int d0 = (int)(t & 15) * 8;
    Kv8<BRASA_KV_Q8_0> x;
    x.load(src + row * kQ8Row, d0);
    float f[8];
    x.to_float(f);
    const float sc = x.scale();
    float4* out = reinterpret_cast<float4*>(dst + row * kDim + d0);
    out[0] = make_float4(sc * f[0], sc * f[1], sc * f[2], sc * f[3]);
    out[1] = make_float4(sc * f[4], sc * f[5], sc * f[6], sc * f[7]);
}

__global__ void fill_u8_kernel(uint8_t* dst, uint8_t value, size_t bytes) {
    const size_t i = (size_t)blockIdx.x * kTpb + threadIdx.x;
    if (i < bytes) dst[i] = value;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ULL;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
    return x ^ (x >> 31);
}

__global__ void fill_normal_kernel(float* out, size_t n, uint64_t seed, float scale) {
    const size_t i = (size_t)blockIdx.x * kTpb + threadIdx.x;
    if (i >= n) return;
    const uint64_t h = splitmix64(seed * 0xd1342543de82ef95ULL + i);
    const float u1 = ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);  // (0, 1)
    const float u2 = (float)(uint32_t)(h & 0xffffffu) * (1.0f / 16777216.0f);
    out[i] = scale * sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

unsigned blocks_for(size_t threads) { return (unsigned)((threads + kTpb - 1) / kTpb); }

}  // namespace

int store_kv_launch(int kv, const float* src, void* dst, size_t n, hipStream_t stream) {
    if (n == 0) return BRASA_OK;
    switch (kv) {
        case BRASA_KV_F32:
            hipLaunchKernelGGL(store_f32_kernel, dim3(blocks_for((n + 3) / 4)), dim3(kTpb), 0,
                               stream, src, static_cast<float*>(dst), n);
            return check_launch("store_kv_f32");
        case BRASA_KV_F16:
            hipLaunchKernelGGL(store_f16_kernel, dim3(blocks_for((n + 3) / 4)), dim3(kTpb), 0,
                               stream, src, static_cast<uint16_t*>(dst), n);
            return check_launch("store_kv_f16");
        case BRASA_KV_Q8_0:
            hipLaunchKernelGGL(store_q8_kernel, dim3(blocks_for(n / 32 * 8)), dim3(kTpb), 0,
                               stream, src, static_cast<uint8_t*>(dst), n / 32);
            return check_launch("store_kv_q8");
    }
    return set_error(BRASA_ERR_ARG, "store_kv: invalid kv type %d", kv);
}

int dequant_q8_launch(const void* src, float* dst, size_t rows, hipStream_t stream) {
    if (rows == 0) return BRASA_OK;
    hipLaunchKernelGGL(dequant_q8_kernel, dim3(blocks_for(rows * 16)), dim3(kTpb), 0, stream,
                       static_cast<const uint8_t*>(src), dst, rows);
    return check_launch("dequantize_kv_q8");
}

int fill_u8_launch(void* dst, uint8_t value, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return BRASA_OK;
    hipLaunchKernelGGL(fill_u8_kernel, dim3(blocks_for(bytes)), dim3(kTpb), 0, stream,
                       static_cast<uint8_t*>(dst), value, bytes);
    return check_launch("fill_u8");
}

int fill_normal_launch(float* out, size_t n, uint64_t seed, float scale, hipStream_t stream) {
    if (n == 0) return BRASA_OK;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(blocks_for(n)), dim3(kTpb), 0, stream, out, n,
                       seed, scale);
    return check_launch("fill_normal");
}

}  // namespace brasa
