// Split-K decode attention for gfx950 (one query token per sequence).
//
// Behaviour follows Kernels::decode_attention_lanes / decode_attention of the reference
// (crates/kernels/src/lib.rs:1056-1164; decode_attention.metal:15-199): keys [0, lk) of one
// layer cache are cut into splits; each split produces per query head the online-softmax
// partial (m, l, acc[128]) and a second pass merges the splits as
// o = sum_s w_s acc_s / sum_s w_s l_s with w_s = exp(m_s - max m).
//
// Design for MI355X (HBM-bound: every K/V byte is read once per GQA group):
//   * workgroup = 4 wave64 = (split, KV head); the G query heads of the group are all served
//     from one read of each K/V row, the rows never leave registers;
//   * lane layout: lane = 16 * r + c holds dims [8c, 8c + 8) of key row (4i + r) of a 32-key
//     block, so a 16-lane DPP row reads one 256 B f16 row with one 128-bit load per lane and
//     the wave reads 4 rows per load instruction (fully coalesced);
//   * QK: 8 FMAs per lane per head, then a 16-lane DPP butterfly (bit-identical in all lanes);
//   * online softmax in fp32 with exp2 (v_exp_f32); per-row partial sums l/acc are only merged
//     across rows (xor 16/32 shuffles) once per wave, then across the 4 waves through LDS;
//   * q8_0: the 8 int8 codes of a lane share one f16 scale (8 | 32), so the scale is applied
//     once to the lane's partial dot (as decode_attention.metal:148-162 does per block) and
//     folded into p for P.V; dequantised values are exact (scale * code in f32);
//   * when one split covers all keys the first kernel normalises and writes o directly.
#include "common.hpp"

namespace brasa {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlock = 32;  // keys per wave iteration: 8 quads of 4 rows

struct DecodeArgs {
    const float* q;       // [hq, 128]
    const uint8_t* k;     // layer cache base
    const uint8_t* v;
    float* part_acc;      // [hq, splits, 128]
    float* part_ml;       // [hq, splits, 2]
    void* o;              // [hq, 128] (used when splits == 1)
    int o_f16;
    int hq, hkv, group;   // group = hq / hkv
    int lk, chunk, splits;
    float scale;
};

template <int KV, int G>
__global__ void __launch_bounds__(kThreads)
decode_split_kernel(DecodeArgs a) {
    constexpr int RB = KvTraits<KV>::row_bytes;
    __shared__ float s_acc[kWaves][G][kDim];
    __shared__ float s_m[kWaves][G];
    __shared__ float s_l[kWaves][G];

    const int split = blockIdx.x;
    const int h0 = blockIdx.y * G;         // first query head of this workgroup
    const int kh = h0 / a.group;           // its KV head
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane >> 4;               // key row within a quad
    const int d0 = (lane & 15) * 8;        // first of the lane's 8 dims

    // Q * scale in f32 (decode_attention.metal:124)
    float qv[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float4* qp = reinterpret_cast<const float4*>(a.q + (size_t)(h0 + h) * kDim + d0);
        float4 x0 = qp[0], x1 = qp[1];
        qv[h][0] = x0.x * a.scale; qv[h][1] = x0.y * a.scale;
        qv[h][2] = x0.z * a.scale; qv[h][3] = x0.w * a.scale;
        qv[h][4] = x1.x * a.scale; qv[h][5] = x1.y * a.scale;
        qv[h][6] = x1.z * a.scale; qv[h][7] = x1.w * a.scale;
    }

    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
    }

    const int s0 = split * a.chunk;
    const int s1 = min(a.lk, s0 + a.chunk);
    const size_t kstride = (size_t)a.hkv * RB;  // bytes between consecutive positions
    const uint8_t* kbase = a.k + (size_t)kh * RB;
    const uint8_t* vbase = a.v + (size_t)kh * RB;

    for (int jb = s0 + wave * kBlock; jb < s1; jb += kWaves * kBlock) {
        Kv8<KV> kr[8], vr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int j = min(jb + 4 * i + r, s1 - 1);
            kr[i].load(kbase + (size_t)j * kstride, d0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int j = min(jb + 4 * i + r, s1 - 1);
            vr[i].load(vbase + (size_t)j * kstride, d0);
        }
        // scores
        float s[8][G];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float kf[8];
            kr[i].to_float(kf);
            const float ksc = kr[i].scale();
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float t = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) t = fmaf(qv[h][e], kf[e], t);
                t = row16_sum(t);
                if (KV == BRASA_KV_Q8_0) t *= ksc;
                s[i][h] = (jb + 4 * i + r < s1) ? t : -INFINITY;
            }
        }
        // online softmax update (block max over the wave's 32 keys)
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float bm = s[0][h];
#pragma unroll
            for (int i = 1; i < 8; ++i) bm = fmaxf(bm, s[i][h]);
            bm = fmaxf(bm, shfl_xor(bm, 16));
            bm = fmaxf(bm, shfl_xor(bm, 32));
            const float mn = fmaxf(m[h], bm);  // finite: row 0 of quad 0 is always a key
            const float alpha = __builtin_amdgcn_exp2f((m[h] - mn) * kLog2e);
            m[h] = mn;
            l[h] *= alpha;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] *= alpha;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p = __builtin_amdgcn_exp2f((s[i][h] - mn) * kLog2e);
                s[i][h] = p;
                l[h] += p;
            }
        }
        // P.V
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float vf[8];
            vr[i].to_float(vf);
            const float vsc = vr[i].scale();
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float p = (KV == BRASA_KV_Q8_0) ? s[i][h] * vsc : s[i][h];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
            }
        }
    }

    // merge the 4 key rows of the wave (lanes r = 0..3 hold disjoint keys)
#pragma unroll
    for (int h = 0; h < G; ++h) {
        l[h] += shfl_xor(l[h], 16);
        l[h] += shfl_xor(l[h], 32);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            acc[h][e] += shfl_xor(acc[h][e], 16);
            acc[h][e] += shfl_xor(acc[h][e], 32);
        }
    }
    if (r == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float4* dst = reinterpret_cast<float4*>(&s_acc[wave][h][d0]);
            dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                s_m[wave][h] = m[h];
                s_l[wave][h] = l[h];
            }
        }
    }
    __syncthreads();

    // merge the 4 waves (decode_attention.metal:46-65); waves without keys have m = -inf
    for (int idx = threadIdx.x; idx < G * kDim; idx += kThreads) {
        const int h = idx / kDim, d = idx % kDim;
        float M = s_m[0][h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][h]);
        float A = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = __builtin_amdgcn_exp2f((s_m[w][h] - M) * kLog2e);
            A = fmaf(s_acc[w][h][d], wt, A);
            L = fmaf(s_l[w][h], wt, L);
        }
        const int hh = h0 + h;
        if (a.splits == 1) {
            const float out = A / L;
            if (a.o_f16)
                reinterpret_cast<uint16_t*>(a.o)[hh * kDim + d] = f2h(out);
            else
                reinterpret_cast<float*>(a.o)[hh * kDim + d] = out;
        } else {
            a.part_acc[((size_t)hh * a.splits + split) * kDim + d] = A;
            if (d == 0) {
                a.part_ml[((size_t)hh * a.splits + split) * 2] = M;
                a.part_ml[((size_t)hh * a.splits + split) * 2 + 1] = L;
            }
        }
    }
}

// attn_decode_reduce (decode_attention.metal:68-84): one workgroup per query head, one thread
// per dim.
__global__ void __launch_bounds__(kDim)
decode_reduce_kernel(const float* __restrict__ part_acc, const float* __restrict__ part_ml,
                     void* o, int o_f16, int splits) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float* ml = part_ml + (size_t)h * splits * 2;
    const float* pa = part_acc + (size_t)h * splits * kDim + d;
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s) M = fmaxf(M, ml[2 * s]);
    float L = 0.0f, A = 0.0f;
    for (int s = 0; s < splits; ++s) {
        const float w = __builtin_amdgcn_exp2f((ml[2 * s] - M) * kLog2e);
        L = fmaf(ml[2 * s + 1], w, L);
        A = fmaf(pa[(size_t)s * kDim], w, A);
    }
    const float out = A / L;
    if (o_f16)
        reinterpret_cast<uint16_t*>(o)[h * kDim + d] = f2h(out);
    else
        reinterpret_cast<float*>(o)[h * kDim + d] = out;
}

template <int KV, int G>
int launch_split(const DecodeArgs& a, int groups_y, hipStream_t stream) {
    hipLaunchKernelGGL((decode_split_kernel<KV, G>), dim3(a.splits, groups_y), dim3(kThreads), 0,
                       stream, a);
    return check_launch("decode_split_kernel");
}

template <int KV>
int launch_split_g(const DecodeArgs& a, int G, int groups_y, hipStream_t stream) {
    switch (G) {
        case 1: return launch_split<KV, 1>(a, groups_y, stream);
        case 2: return launch_split<KV, 2>(a, groups_y, stream);
        case 4: return launch_split<KV, 4>(a, groups_y, stream);
        case 8: return launch_split<KV, 8>(a, groups_y, stream);
    }
    return set_error(BRASA_ERR_UNSUPPORTED, "decode: GQA group %d not compiled", G);
}

}  // namespace

// Split plan: keys per split are a multiple of 128 (so splits <= ceil(lk / 128) and the
// reference's partials size always suffices) chosen so that about 1024 workgroups cover the
// 256 CUs. BRASA_DECODE_CHUNK overrides the chunk (a multiple of 128). The plan depends only
// on (lk, workgroups per split), so results are reproducible bit for bit.
void decode_plan(int lk, int wg_per_split, int* chunk_out, int* splits_out) {
    static int env_chunk = [] {
        const char* e = getenv("BRASA_DECODE_CHUNK");
        int c = e ? atoi(e) : 0;
        return (c > 0 && c % 128 == 0) ? c : 0;
    }();
    int chunk;
    if (env_chunk) {
        chunk = env_chunk;
    } else {
        const int max_splits = (lk + 127) / 128;
        int target = (1024 + wg_per_split - 1) / wg_per_split;
        if (target > max_splits) target = max_splits;
        if (target < 1) target = 1;
        chunk = ((lk + target - 1) / target + 127) / 128 * 128;
    }
    *chunk_out = chunk;
    *splits_out = (lk + chunk - 1) / chunk;
}

int decode_launch(const float* q, const void* k, const void* v, float* partials, void* o,
                  int o_f16, int hq, int hkv, int lk, int kv, bool per_head,
                  hipStream_t stream) {
    const int group = hq / hkv;
    const int G = per_head ? 1 : group;
    const int groups_y = per_head ? hq : hkv;
    DecodeArgs a;
    a.q = q;
    a.k = static_cast<const uint8_t*>(k);
    a.v = static_cast<const uint8_t*>(v);
    decode_plan(lk, groups_y, &a.chunk, &a.splits);
    a.part_acc = partials;
    a.part_ml = partials + (size_t)hq * a.splits * kDim;
    a.o = o;
    a.o_f16 = o_f16;
    a.hq = hq;
    a.hkv = hkv;
    a.group = group;
    a.lk = lk;
    a.scale = 1.0f / sqrtf(static_cast<float>(kDim));
    int st;
    switch (kv) {
        case BRASA_KV_F32: st = launch_split_g<BRASA_KV_F32>(a, G, groups_y, stream); break;
        case BRASA_KV_F16: st = launch_split_g<BRASA_KV_F16>(a, G, groups_y, stream); break;
        case BRASA_KV_Q8_0: st = launch_split_g<BRASA_KV_Q8_0>(a, G, groups_y, stream); break;
        default: return set_error(BRASA_ERR_ARG, "decode: invalid kv type %d", kv);
    }
    if (st != BRASA_OK || a.splits == 1) return st;
    hipLaunchKernelGGL(decode_reduce_kernel, dim3(hq), dim3(kDim), 0, stream, a.part_acc,
                       a.part_ml, o, o_f16, a.splits);
    return check_launch("decode_reduce_kernel");
}

}  // namespace brasa
