// Producer side of the attention path on gfx950: per-head QK-RMSNorm, RoPE-NeoX and the KV-cache
// write, fused in one launch, plus the unfused RMSNorm and RoPE it must agree with bit for bit.
//
// Behaviour follows Kernels::qk_norm_rope_store (crates/kernels/src/lib.rs:976-1025;
// qkv.metal:37-94): for every token t and head, q and k rows are normalised
// (x * (1 / sqrt(sum x^2 / 128 + eps))) * w, rotated by RoPE-NeoX at position pos0 + t with the
// f64-computed cos/sin table, written back in place, and k (rotated) and v (as given) are stored
// into the cache from pos0 on in the cache type (store_kv rounding: f16 RNE or q8_0).
//
// Design: lane l of a wave64 holds elements l and l + 64 of a 128-element row (exactly a RoPE
// pair); each wave takes four consecutive rows and issues every load of the four (row, norm
// weights, cos/sin) before the first reduction, so a wave keeps 4 rows of reads in flight (in-place
// writes of one row could otherwise alias the next row's loads and serialise them). The sum of
// squares has one fixed order shared with the unfused rms_norm kernel (lane partials in index
// order, then a butterfly inside 16-lane rows by DPP and across rows by v_permlane16/32_swap), so
// fused and unfused results are identical bits, as the reference's fused test demands
// (crates/kernels/tests/fused.rs:8-98). The q8_0 groups of 32 are half-waves: the group amax is
// the same exchanges without the last one. HBM-bound: T * (hq + 2 hkv) * 512 B read, q/k
// rewritten, cache rows written.
#include <cmath>
#include <vector>

#include "common.hpp"

namespace brasa {
namespace {

constexpr int kRowsPerWg = 4;    // rms_norm: one row per wave
constexpr int kWavesPerWg = 4;   // qk_norm_rope_store
constexpr int kRowsPerWave = 4;

// Sum over the wave of the per-lane partials in one fixed order: the 16-lane DPP butterfly, then
// lanes l ^ 16 and l ^ 32. Partners always add the same two values, so every lane ends with
// identical bits.
__device__ __forceinline__ float wave_sum(float p) {
    p = row16_sum(p);
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_int(p), __float_as_int(p), false, false);
    p = __int_as_float(a[0]) + __int_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_int(p), __float_as_int(p), false, false);
    return __int_as_float(b[0]) + __int_as_float(b[1]);
}
// max over the 32 lanes of each half-wave
__device__ __forceinline__ float half_wave_max(float x) {
    x = fmaxf(x, dpp<0x140>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x1B>(x));
    x = fmaxf(x, dpp<0xB1>(x));
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
    return fmaxf(__int_as_float(a[0]), __int_as_float(a[1]));
}
// 1 / sqrt(ss / n + eps) with IEEE divides and square root (the reference's precise::sqrt).
__device__ __forceinline__ float rms_scale(float ss, int n, float eps) {
    return 1.0f / sqrtf(ss / (float)n + eps);
}

// rms_norm (lib.rs:531-547; norm.metal:8-48): one wave per row of n elements.
__global__ void __launch_bounds__(64 * kRowsPerWg)
rms_norm_kernel(const float* x, const float* __restrict__ w, float* out, int rows,
                int n, float eps) {
    const int row = blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * n;  // out may alias x (in-place use)
    float p = 0.0f;
    for (int i = lane; i < n; i += 64) p += xr[i] * xr[i];
    const float scale = rms_scale(wave_sum(p), n, eps);
    float* orow = out + (size_t)row * n;
    for (int i = lane; i < n; i += 64) orow[i] = (xr[i] * scale) * w[i];
}

// rope_neox (lib.rs:569-596; rope.metal:8-27): one thread per pair (i, i + dim / 2).
__global__ void rope_neox_kernel(float* x, const float* __restrict__ cos_t,
                                 const float* __restrict__ sin_t, int tokens, int heads, int dim,
                                 int pos0) {
    const int half = dim / 2;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)tokens * heads * half) return;
    const int i = (int)(idx % half);
    const size_t th = idx / half;  // t * heads + h
    const int t = (int)(th / heads);
    float* v = x + th * dim;
    const size_t p = (size_t)(pos0 + t) * half + i;
    const float c = cos_t[p], s = sin_t[p];
    const float a = v[i], b = v[i + half];
    v[i] = a * c - b * s;
    v[i + half] = b * c + a * s;
}

// Writes this lane's two elements (l and l + 64) of cache row `row`. q8_0 rows go through
// `stage` (this wave's 136-byte LDS row): the codes and scales are written there byte by byte and
// the row leaves as 34 dword stores (one instruction) instead of two byte stores per lane.
template <int KV>
__device__ __forceinline__ void store_row(uint8_t* cache, size_t row, int lane, float y0,
                                          float y1, uint8_t* stage) {
    if constexpr (KV == BRASA_KV_F32) {
        float* r = reinterpret_cast<float*>(cache) + row * kDim;
        r[lane] = y0;
        r[lane + 64] = y1;
    } else if constexpr (KV == BRASA_KV_F16) {
        uint16_t* r = reinterpret_cast<uint16_t*>(cache) + row * kDim;
        r[lane] = f2h(y0);
        r[lane + 64] = f2h(y1);
    } else {
        // groups: elements 32 g .. 32 g + 31; y0 is in group lane / 32, y1 in 2 + lane / 32
        const uint16_t d0 = q8_scale_bits(half_wave_max(fabsf(y0)));
        const uint16_t d1 = q8_scale_bits(half_wave_max(fabsf(y1)));
        stage[lane] = (uint8_t)q8_code(y0, h2f(d0));
        stage[lane + 64] = (uint8_t)q8_code(y1, h2f(d1));
        if ((lane & 31) == 0) {
            uint16_t* sc = reinterpret_cast<uint16_t*>(stage + 128);
            sc[lane >> 5] = d0;
            sc[2 + (lane >> 5)] = d1;
        }
        // (one wave: its LDS writes are done before its reads; the next row's writes come after)
        if (lane < kQ8Row / 4)
            reinterpret_cast<uint32_t*>(cache + row * kQ8Row)[lane] =
                reinterpret_cast<const uint32_t*>(stage)[lane];
    }
}

struct QkvArgs {
    float* q;
    float* k;
    const float* v;
    const float* qn;
    const float* kn;
    const float* cos_t;
    const float* sin_t;
    uint8_t* kc;
    uint8_t* vc;
    int hq, hkv, pos0, rows;
    float eps;
};

// Row gr of T * (hq + 2 hkv): within a token, first the hq query heads, then the hkv key heads,
// then the hkv value heads (the reference's order, qkv.metal:59-61). Wave w takes rows
// 4 w .. 4 w + 3.
template <int KV>
__global__ void __launch_bounds__(64 * kWavesPerWg) qk_norm_rope_store_kernel(QkvArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t s_stage[kWavesPerWg][KV == BRASA_KV_Q8_0 ? kQ8Row : 4];
    const int gr0 = (blockIdx.x * kWavesPerWg + (threadIdx.x >> 6)) * kRowsPerWave;
    const int lane = threadIdx.x & 63;
    uint8_t* stage = s_stage[threadIdx.x >> 6];
    if (gr0 >= a.rows) return;
    const int per_tok = a.hq + 2 * a.hkv;
    float x0[kRowsPerWave], x1[kRowsPerWave], w0[kRowsPerWave], w1[kRowsPerWave];
    float c[kRowsPerWave], sn[kRowsPerWave];
    float* dst[kRowsPerWave];
    size_t crow[kRowsPerWave];
    int kind[kRowsPerWave];  // 0 q, 1 k, 2 v, 3 past the last row
    // every load of the four rows first
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
        const int gr = gr0 + j;
        kind[j] = 3;
        if (gr >= a.rows) continue;
        const int t = gr / per_tok, r = gr % per_tok;
        if (r >= a.hq + a.hkv) {
            kind[j] = 2;
            crow[j] = (size_t)t * a.hkv + (r - a.hq - a.hkv);
            const float* vr = a.v + crow[j] * kDim;
            x0[j] = vr[lane];
            x1[j] = vr[lane + 64];
            continue;
        }
        const bool is_q = r < a.hq;
        kind[j] = is_q ? 0 : 1;
        crow[j] = is_q ? (size_t)t * a.hq + r : (size_t)t * a.hkv + (r - a.hq);
        dst[j] = (is_q ? a.q : a.k) + crow[j] * kDim;
        x0[j] = dst[j][lane];
        x1[j] = dst[j][lane + 64];
        const float* w = is_q ? a.qn : a.kn;
        w0[j] = w[lane];
        w1[j] = w[lane + 64];
        const size_t tp = (size_t)(a.pos0 + t) * (kDim / 2) + lane;
        c[j] = a.cos_t[tp];
        sn[j] = a.sin_t[tp];
    }
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
        if (kind[j] == 3) break;
        if (kind[j] == 2) {
            store_row<KV>(a.vc, crow[j], lane, x0[j], x1[j], stage);
            continue;
        }
        float p = 0.0f;
        p += x0[j] * x0[j];
        p += x1[j] * x1[j];
        const float scale = rms_scale(wave_sum(p), kDim, a.eps);
        const float a0 = (x0[j] * scale) * w0[j];
        const float b0 = (x1[j] * scale) * w1[j];
        const float y0 = a0 * c[j] - b0 * sn[j];
        const float y1 = b0 * c[j] + a0 * sn[j];
        dst[j][lane] = y0;
        dst[j][lane + 64] = y1;
        if (kind[j] == 1) store_row<KV>(a.kc, crow[j], lane, y0, y1, stage);
    }
}

unsigned row_blocks(size_t rows) { return (unsigned)((rows + kRowsPerWg - 1) / kRowsPerWg); }

}  // namespace

int rms_norm_launch(const float* x, const float* w, float* out, size_t rows, size_t n, float eps,
                    hipStream_t stream) {
    if (rows == 0) return BRASA_OK;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(row_blocks(rows)), dim3(64 * kRowsPerWg), 0, stream,
                       x, w, out, (int)rows, (int)n, eps);
    return check_launch("rms_norm");
}

int rope_neox_launch(float* x, const float* cos_t, const float* sin_t, size_t tokens,
                     size_t heads, size_t dim, size_t pos0, hipStream_t stream) {
    const size_t pairs = tokens * heads * (dim / 2);
    if (pairs == 0) return BRASA_OK;
    hipLaunchKernelGGL(rope_neox_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0,
                       stream, x, cos_t, sin_t, (int)tokens, (int)heads, (int)dim, (int)pos0);
    return check_launch("rope_neox");
}

int qk_norm_rope_store_launch(int kv, float* q, float* k, const float* v, const float* qn,
                              const float* kn, float eps, const float* cos_t, const float* sin_t,
                              void* kdst, void* vdst, size_t tokens, size_t hq, size_t hkv,
                              size_t pos0, hipStream_t stream) {
    QkvArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.qn = qn;
    a.kn = kn;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.kc = static_cast<uint8_t*>(kdst);
    a.vc = static_cast<uint8_t*>(vdst);
    a.hq = (int)hq;
    a.hkv = (int)hkv;
    a.pos0 = (int)pos0;
    a.rows = (int)(tokens * (hq + 2 * hkv));
    a.eps = eps;
    if (a.rows == 0) return BRASA_OK;
    const int per_wg = kWavesPerWg * kRowsPerWave;
    const dim3 grid((unsigned)((a.rows + per_wg - 1) / per_wg)), block(64 * kWavesPerWg);
    switch (kv) {
        case BRASA_KV_F32:
            hipLaunchKernelGGL(qk_norm_rope_store_kernel<BRASA_KV_F32>, grid, block, 0, stream, a);
            break;
        case BRASA_KV_F16:
            hipLaunchKernelGGL(qk_norm_rope_store_kernel<BRASA_KV_F16>, grid, block, 0, stream, a);
            break;
        case BRASA_KV_Q8_0:
            hipLaunchKernelGGL(qk_norm_rope_store_kernel<BRASA_KV_Q8_0>, grid, block, 0, stream, a);
            break;
        default:
            return set_error(BRASA_ERR_ARG, "qk_norm_rope_store: invalid kv type %d", kv);
    }
    return check_launch("qk_norm_rope_store");
}

// rope_table (lib.rs:1388-1404): cos/sin(p * theta^(-2 i / dim)) in f64, stored as f32.
void rope_table_host(double theta, size_t dim, size_t max_pos, float* cos_out, float* sin_out) {
    const size_t half = dim / 2;
    std::vector<double> inv(half);
    for (size_t i = 0; i < half; ++i) inv[i] = 1.0 / std::pow(theta, (double)(2 * i) / (double)dim);
    for (size_t p = 0; p < max_pos; ++p) {
        for (size_t i = 0; i < half; ++i) {
            const double ang = (double)p * inv[i];
            cos_out[p * half + i] = (float)std::cos(ang);
            sin_out[p * half + i] = (float)std::sin(ang);
        }
    }
}

}  // namespace brasa
