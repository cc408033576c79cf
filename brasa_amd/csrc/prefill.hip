// Causal flash-attention prefill on gfx950 MFMA.
//
// Behaviour follows Kernels::flash_attention_with (crates/kernels/src/lib.rs:1185-1248;
// flash_attention.metal:152-323): query t of the chunk sits at absolute position pos0 + t and
// attends to keys [0, pos0 + t]; softmax and accumulation in f32. PrefillPrecision::F16 rounds
// Q * scale (computed in f32) to f16 and writes f16 output (flash_attention.metal:213,320);
// ::F32 keeps Q and output in f32.
//
// Design for MI355X (dense contraction on the matrix cores):
//   * workgroup = 4 wave64 sharing one KV head: the HW (<= 4) query heads of a GQA group times
//     32 * 4 / HW query tokens; every wave owns 32 queries of one head, so the 4 waves of a
//     G = 4 group read each K/V tile from LDS once per head instead of from HBM;
//   * S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_32x32x16_f16: the S^T accumulator layout
//     (lane = query column, 16 keys per lane) is exactly the B-operand layout P^T needs, so P
//     never goes through LDS; K is read from LDS row-major, V is stored transposed in LDS
//     (d-major) so each A operand is two ds_read_b64;
//   * 64-key K/V tiles, global loads for tile i+1 issued before the MFMAs of tile i;
//   * causal skipping per wave (32-key sub-blocks past its last query are not computed) and
//     masking only on sub-blocks that cross the diagonal; heaviest query tiles dispatch first
//     (flash_attention.metal:202-205) and the head-group index varies fastest so the 8 KV heads
//     spread over the 8 XCDs (each XCD's L2 keeps its head's K/V);
//   * values that f16 cannot hold exactly (f32 and q8_0 caches, f32 Q, f32 P) are split as
//     x = hi + lo with hi = f16(x), lo = f16(x - hi) and contracted with extra MFMAs
//     (hi*hi + hi*lo + lo*hi), which keeps ~22 significant bits;
//   * fp16 caches in the F16 / F16_PF32 precisions run one of three specialised kernels, picked
//     by workgroup count: prefill_f16_kernel (8 waves, two key groups whose MFMA and softmax
//     phases alternate; up to two workgroups per CU), prefill_f16_kernel4 (4 waves, two per CU)
//     and prefill_f16_kernel4s (4 waves on 32-key stages, three per CU).
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace brasa {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

constexpr int kThreads = 256;
constexpr int kTile = 64;       // keys per LDS tile
constexpr int kKStr = 136;      // K row stride in halves (128 + 8 pad)
constexpr int kVStr = 72;       // V^T row stride in halves (64 + 8 pad)

struct PrefillArgs {
    const float* q;
    const uint8_t* k;
    const uint8_t* v;
    void* o;
    int tokens, hq, hkv, group, pos0;
    int ntiles;                 // query tiles
    int pair;                   // prefill_f16_kernel: workgroup y runs tiles ntiles - 1 - y and y
    float scale;
    // prefill_f16_kernel key split: each query tile's keys are cut into kparts parts, one
    // workgroup each; the parts' partials (part) are merged by the last to arrive (ctr)
    int kparts;
    float* part;
    unsigned* ctr;
    // q8_0 caches in F16 precision, whose values go through f16(code * scale): a launch that
    // meets a scale outside the range where that product is a normal f16 (see q8_f16_unsafe)
    // stores `tag` at `taint`; the launch after it that holds gate = taint (the gated two-group
    // f16 kernel, or prefill_exact_kernel) recomputes the call exactly only when *gate == tag
    unsigned* taint;
    const unsigned* gate;
    unsigned tag;
    // q8_0 rows staged as f16: the cache itself, read by the exact path of a gated f16 launch
    const uint8_t* k8;
    const uint8_t* v8;
};

// True for the f16 scale bits of a q8_0 group whose f16(code * scale) products can leave the
// normal f16 range: |scale| >= 516 (127 * 516 > 65504 rounds to inf), f16-subnormal scales (the
// products of small codes are subnormal, with fewer significant bits), and inf / NaN. Scales of
// 0 (an all-zero group) are exact.
__device__ __forceinline__ bool q8_f16_unsafe(uint32_t sc) {
    const uint32_t m = sc & 0x7fffu;
    return m >= 0x6008u || (m != 0 && m < 0x0400u);
}


// Two values d, d + 1 (d even) of cache row `row` as f32 (q8_0: code * scale, exact).
template <int KV>
__device__ __forceinline__ f32x2 row_pair(const uint8_t* cache, size_t row, int d) {
    if constexpr (KV == BRASA_KV_F32) {
        return *reinterpret_cast<const f32x2*>(cache + row * 512 + 4 * d);
    } else if constexpr (KV == BRASA_KV_F16) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(cache + row * 256 + 2 * d);
        return f32x2{h2f((uint16_t)(w & 0xffffu)), h2f((uint16_t)(w >> 16))};
    } else {
        const uint8_t* r = cache + row * kQ8Row;
        const uint16_t c = *reinterpret_cast<const uint16_t*>(r + d);
        const float sc = h2f(*reinterpret_cast<const uint16_t*>(r + 128 + 2 * (d >> 5)));
        return f32x2{(float)(int8_t)(c & 0xffu) * sc, (float)(int8_t)(c >> 8) * sc};
    }
}

// Exact F16 prefill in plain f32 arithmetic, the reference F16 kernel's numerics
// (flash_attention.metal:152-323: Q * scale rounded to f16, K / V as exact f32 values, scores,
// softmax, P and O in f32, o rounded to f16): query row rw = token * hq + head of the cache
// (k, v), computed by one wave, lane l holding dims 2 l, 2 l + 1, one key per step (the score
// is a wave sum). Slow, and free of any f16 range limit on the cache values.
template <int KV>
__device__ __forceinline__ void exact_row(const PrefillArgs& a, const uint8_t* k, const uint8_t* v,
                                          int rw, int lane) {
    const int t = rw / a.hq, h = rw - t * a.hq, kh = h / a.group, d = 2 * lane;
    const f32x2 qv = *reinterpret_cast<const f32x2*>(a.q + (size_t)rw * kDim + d);
    const float q0 = h2f(f2h(as_f32(qv.x * a.scale))), q1 = h2f(f2h(as_f32(qv.y * a.scale)));
    float m = -INFINITY, l = 0.0f, o0 = 0.0f, o1 = 0.0f;
    const int kend = a.pos0 + t + 1;
    for (int j = 0; j < kend; ++j) {
        const size_t row = (size_t)j * a.hkv + kh;
        const f32x2 kk = row_pair<KV>(k, row, d);
        const f32x2 vv = row_pair<KV>(v, row, d);
        float sc = row16_sum(fmaf(q0, kk.x, q1 * kk.y));
        sc += __shfl_xor(sc, 16, 64);
        sc += __shfl_xor(sc, 32, 64);
        const float x = sc * kLog2e;
        const float mn = fmaxf(m, x);
        const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
        const float p = __builtin_amdgcn_exp2f(x - mn);
        l = fmaf(l, alpha, p);
        o0 = fmaf(o0, alpha, p * vv.x);
        o1 = fmaf(o1, alpha, p * vv.y);
        m = mn;
    }
    const float inv = 1.0f / l;
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.o) + (size_t)rw * kDim + d) =
        (uint32_t)f2h(o0 * inv) | ((uint32_t)f2h(o1 * inv) << 16);
}

// The range gate of a q8_0 F16 call (every thread of the workgroup calls it): true when the
// launch before this one flagged a scale (*gate == tag). A workgroup that finds it set counts
// itself in the word 8 past the flag; the last of the grid stores 0 there, so the flag is
// cleared once every workgroup has read it, and a graph replayed with the same tag starts each
// replay unflagged.
__device__ __forceinline__ bool gate_open(const PrefillArgs& a) {
    __shared__ int s_go;
    if (threadIdx.x == 0) {
        const bool go = __hip_atomic_load(a.gate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.tag;
        if (go) {
            const unsigned n = gridDim.x * gridDim.y;
            const unsigned t = __builtin_amdgcn_atomic_inc32(a.taint + 8, n - 1, __ATOMIC_RELAXED,
                                                             "agent");
            if (t == n - 1) __hip_atomic_store(a.taint, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_go = go;
    }
    __syncthreads();
    return s_go;
}


#ifdef BRASA_PREFILL_TRACE
// Timeline build (libbrasa_attn_trace.so only): thread 0 of each prefill_f16_kernel workgroup
// (wave 0: group 0, first head) writes the 100 MHz real-time counter at the phases of
// PrefillStamp into slot (blockIdx.x + gridDim.x * blockIdx.y) % kPfTraceWgs.
constexpr int kPfTraceWgs = 8192;
constexpr int kPfTraceStamps = 16;
__device__ unsigned long long g_prefill_trace[kPfTraceWgs * kPfTraceStamps];
#define PREFILL_STAMP(k)                                                                        \
    do {                                                                                        \
        if (threadIdx.x == 0)                                                                   \
            g_prefill_trace[((blockIdx.x + gridDim.x * blockIdx.y) % kPfTraceWgs) *           \
                                kPfTraceStamps + (k)] = __builtin_amdgcn_s_memrealtime();      \
    } while (0)
#else
#define PREFILL_STAMP(k) \
    do {                 \
    } while (0)
#endif
// Phases of each query tile a workgroup runs (ti = 0 for its first tile, 1 for the second),
// stamped at 1 + 6 ti + phase; stamp 0 is the workgroup's start.
enum PrefillStamp {
    kPfTileStart = 0,   // the tile's code entered
    kPfPrologue,        // Q loaded, converted and exchanged; the first copies issued
    kPfFirstTile,       // the first K/V tile landed (wave 0's first wait and barrier)
    kPfLoopEnd,         // every key tile contracted
    kPfMerged,          // the two key groups merged
    kPfStored,          // o written (the timeline build waits for the stores)
};

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, not for its
// outstanding global loads (which __syncthreads' fence also waits for).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// x is materialised as one f32 value for both halves (see as_f32): a product folded into a
// single-rounding conversion for hi alone would leave hi + lo one f16 ulp off at f16 ties.
__device__ __forceinline__ void split_f16(float x, uint16_t& hi, uint16_t& lo) {
    x = as_f32(x);
    hi = f2h(x);
    lo = f2h(x - h2f(hi));
}

__device__ __forceinline__ half8 lds_b128(const uint16_t* p) {
    return __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ half8 lds_2xb64(const uint16_t* p0, const uint16_t* p1) {
    uint2 a = *reinterpret_cast<const uint2*>(p0);
    uint2 b = *reinterpret_cast<const uint2*>(p1);
    uint4 c = make_uint4(a.x, a.y, b.x, b.y);
    return __builtin_bit_cast(half8, c);
}
__device__ __forceinline__ half8 pack8(const uint16_t (&x)[8]) {
    uint4 c;
    c.x = x[0] | ((uint32_t)x[1] << 16);
    c.y = x[2] | ((uint32_t)x[3] << 16);
    c.z = x[4] | ((uint32_t)x[5] << 16);
    c.w = x[6] | ((uint32_t)x[7] << 16);
    return __builtin_bit_cast(half8, c);
}

// value combined with that of lane l ^ 32 (v_permlane32_swap: VALU, no LDS round trip)
__device__ __forceinline__ float max_xor32(float x) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return fmaxf(__int_as_float(sw[0]), __int_as_float(sw[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float(sw[0]) + __int_as_float(sw[1]);
}

__device__ __forceinline__ f32x16 mfma(half8 a, half8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Q of one query column for the f16 kernels: 16 raw 16-byte loads per lane (k-step t holds
// floats 16 t + 8 u .. + 8 of the row), all issued before anything else: the scheduling barrier
// keeps the conversion (and its waits) below the first K/V copies the caller issues next, so Q
// and those copies travel together instead of Q arriving in serial round trips first. The
// compiler's own waits for these loads stay exact: they also cover any copy issued after them.
__device__ __forceinline__ void q_load(const float* qrow, int u, u32x4 (&raw)[16]) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            raw[2 * t + h] = *reinterpret_cast<const u32x4*>(qrow + 16 * t + 8 * u + 4 * h);
    __builtin_amdgcn_sched_barrier(0);
}
// f16(Q * scale) with the product in f32 (flash_attention.metal:213); zero for a padding column
__device__ __forceinline__ void q_convert(const u32x4 (&raw)[16], float scale, bool valid,
                                          half8 (&qh)[8]) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const f32x4 x0 = __builtin_bit_cast(f32x4, raw[2 * t]);
        const f32x4 x1 = __builtin_bit_cast(f32x4, raw[2 * t + 1]);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        uint16_t hi[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sx = as_f32(xs[j] * scale);  // f32 product, then f16
            hi[j] = f2h(valid ? sx : 0.0f);
        }
        qh[t] = pack8(hi);
    }
}

// Output of one f16-kernel wave: its 32 x 128 tile (accumulator layout, times inv) rounded to f16
// and written row-major into 8 KB of LDS at ot (16-byte chunk c of row r at chunk c ^ (r & 15),
// conflict-free both ways), then stored 4 whole 256-byte rows per instruction (instead of 16
// bytes of each of 32 rows). Rows tw0 + r at or past tokens are not stored.
__device__ __forceinline__ void store_o_rows(const f32x16 (&acc)[4], float inv, uint8_t* ot,
                                             int lane, void* o, int tw0, int tokens, int hq, int h) {
    const int col = lane & 31, u = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint2 w;
            w.x = (uint32_t)f2h(as_f32(acc[dt][4 * g] * inv)) |
                  ((uint32_t)f2h(as_f32(acc[dt][4 * g + 1] * inv)) << 16);
            w.y = (uint32_t)f2h(as_f32(acc[dt][4 * g + 2] * inv)) |
                  ((uint32_t)f2h(as_f32(acc[dt][4 * g + 3] * inv)) << 16);
            *reinterpret_cast<uint2*>(ot + col * 256 + 16 * ((4 * dt + g) ^ (col & 15)) + 8 * u) = w;
        }
    }
    asm volatile("" ::: "memory");  // a wave's LDS accesses execute in order
    const int rq = lane >> 4, cq = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = 4 * i + rq;
        const uint4 v = *reinterpret_cast<const uint4*>(ot + row * 256 + 16 * (cq ^ (row & 15)));
        if (tw0 + row < tokens)
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(o) + ((size_t)(tw0 + row) * hq + h) * kDim + 8 * cq) = v;
    }
}

// Half of a Q row for the two-group kernel: group g loads and converts the k-steps 4 g .. 4 g + 3
// (head dims 64 g .. 64 g + 63) of its column, the other group the rest, and the halves meet in
// LDS: each row is read from HBM once per workgroup instead of once per group.
__device__ __forceinline__ void q_load_half(const float* qrow, int u, int g, u32x4 (&raw)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            raw[2 * j + h] = *reinterpret_cast<const u32x4*>(qrow + 16 * (4 * g + j) + 8 * u + 4 * h);
    __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void q_convert_half(const u32x4 (&raw)[8], float scale, bool valid,
                                               half8 (&qh)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x4 x0 = __builtin_bit_cast(f32x4, raw[2 * j]);
        const f32x4 x1 = __builtin_bit_cast(f32x4, raw[2 * j + 1]);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        uint16_t hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float sx = as_f32(xs[i] * scale);  // f32 product, then f16
            hi[i] = f2h(valid ? sx : 0.0f);
        }
        qh[j] = pack8(hi);
    }
}

// KV = cache type; HW = query heads per workgroup (1, 2, 4); QS = split Q (F32 precision);
// PS = split P; OF32 = f32 output.
template <int KV, int HW, bool QS, bool PS, bool OF32>
__global__ void __launch_bounds__(kThreads, 2)
prefill_kernel(PrefillArgs a) {
    if (a.gate && *a.gate != a.tag) return;  // the fast launch before this one was exact
    constexpr bool KS = (KV != BRASA_KV_F16);  // cache values need hi/lo
    constexpr int NK = KS ? 2 : 1;
    constexpr int TPW = 32 * 4 / HW;            // query tokens per workgroup
    constexpr int RB = KvTraits<KV>::row_bytes;

    __shared__ __attribute__((aligned(16))) uint16_t s_k[NK][kTile * kKStr];
    __shared__ __attribute__((aligned(16))) uint16_t s_vt[NK][kDim * kVStr];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 31;       // query column of the MFMA tiles
    const int u = lane >> 5;         // lane half

    const int hg = blockIdx.x;                            // head group (fastest: spreads XCDs)
    const int tile = a.ntiles - 1 - (int)blockIdx.y;      // heaviest query tiles first
    const int h = hg * HW + (wave % HW);
    const int kh = (hg * HW) / a.group;
    const int t0 = tile * TPW;
    const int tw0 = t0 + 32 * (wave / HW);                // first query token of this wave
    const int lk = a.pos0 + a.tokens;
    const int kend_wg = a.pos0 + min(t0 + TPW, a.tokens);  // keys [0, kend_wg) are read
    const int kend_w = a.pos0 + min(tw0 + 32, a.tokens);   // this wave needs [0, kend_w)

    // ---- Q^T B-operands: k-step t holds d = 16t + 8u + j ------------------------------
    const int tq = tw0 + col;
    const bool qvalid = tq < a.tokens;
    half8 qh[8], ql[QS ? 8 : 1];
    {
        const float* qrow = a.q + ((size_t)(qvalid ? tq : 0) * a.hq + h) * kDim;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float4* p = reinterpret_cast<const float4*>(qrow + 16 * t + 8 * u);
            float4 x0 = p[0], x1 = p[1];
            float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            uint16_t hi[8], lo[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float sx = qvalid ? as_f32(xs[j] * a.scale) : 0.0f;
                if (QS) split_f16(sx, hi[j], lo[j]);
                else hi[j] = f2h(sx);
            }
            qh[t] = pack8(hi);
            if (QS) ql[t] = pack8(lo);
        }
    }

    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m2 = -INFINITY;  // running max of s * log2(e)
    float lsum = 0.0f;     // this lane's share of the softmax denominator
    const int qabs = a.pos0 + tq;

    // ---- global -> register staging of one 64-key tile ----------------------------------
    // item i of thread (wave, lane): key = lane, 8-dim chunk = wave + 4 i (i = 0..3)
    const size_t kstride = (size_t)a.hkv * RB;
    const uint8_t* kbase = a.k + (size_t)kh * RB;
    const uint8_t* vbase = a.v + (size_t)kh * RB;
    Kv8<KV> rk[4], rv[4];
    auto load_tile = [&](int kb) {
        const size_t row = (size_t)(kb + lane) * kstride;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rk[i].load(kbase + row, 8 * (wave + 4 * i));
            rv[i].load(vbase + row, 8 * (wave + 4 * i));
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c8 = 8 * (wave + 4 * i);
            float kf[8], vf[8];
            rk[i].to_float(kf);
            rv[i].to_float(vf);
            const float ks = rk[i].scale(), vs = rv[i].scale();
            uint16_t khi[8], klo[8], vhi[8], vlo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (KS) {
                    split_f16(KV == BRASA_KV_Q8_0 ? as_f32(kf[e] * ks) : kf[e], khi[e], klo[e]);
                    split_f16(KV == BRASA_KV_Q8_0 ? as_f32(vf[e] * vs) : vf[e], vhi[e], vlo[e]);
                } else {
                    khi[e] = f2h(kf[e]);
                    vhi[e] = f2h(vf[e]);
                }
            }
            *reinterpret_cast<half8*>(&s_k[0][lane * kKStr + c8]) = pack8(khi);
            if (KS) *reinterpret_cast<half8*>(&s_k[NK - 1][lane * kKStr + c8]) = pack8(klo);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s_vt[0][(c8 + e) * kVStr + lane] = vhi[e];
                if (KS) s_vt[NK - 1][(c8 + e) * kVStr + lane] = vlo[e];
            }
        }
    };

    load_tile(0);
    for (int kb = 0; kb < kend_wg; kb += kTile) {
        __syncthreads();  // previous tile fully consumed
        store_tile();
        __syncthreads();
        if (kb + kTile < kend_wg) load_tile(kb + kTile);

        if (kb >= kend_w) continue;  // this wave's queries are all before the tile
        const int nsub = (kb + 32 < kend_w) ? 2 : 1;

        // S^T for the two 32-key sub-blocks
        f32x16 s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s[b][i] = 0.0f;
            if (b < nsub) {
                const uint16_t* krow = &s_k[0][(32 * b + col) * kKStr + 8 * u];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const half8 ka = lds_b128(krow + 16 * t);
                    s[b] = mfma(ka, qh[t], s[b]);
                    if (QS) s[b] = mfma(ka, ql[t], s[b]);
                    if (KS) {
                        const half8 kl = lds_b128(&s_k[NK - 1][(32 * b + col) * kKStr + 8 * u + 16 * t]);
                        s[b] = mfma(kl, qh[t], s[b]);
                    }
                }
            }
        }
        // scale to log2 domain, causal mask, tile max
        float tmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int kb2 = kb + 32 * b;
            const bool need_mask = (kb2 + 31 > a.pos0 + tw0) || (kb2 + 31 >= lk);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kb2 + 8 * (i / 4) + 4 * u + (i % 4);
                float x = s[b][i] * kLog2e;
                if (b >= nsub || (need_mask && (key > qabs || key >= lk))) x = -INFINITY;
                s[b][i] = x;
                tmax = fmaxf(tmax, x);
            }
        }
        tmax = max_xor32(tmax);
        const float mn = fmaxf(m2, tmax);  // finite: key 0 is visible to every query
        const float alpha = __builtin_amdgcn_exp2f(m2 - mn);
        m2 = mn;
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;

        // P^T B-operands and O^T += V^T P^T
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nsub) break;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint16_t ph[8], pl[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(s[b][8 * st + j] - mn);
                    lsum += p;
                    if (PS) split_f16(p, ph[j], pl[j]);
                    else ph[j] = f2h(p);
                }
                const half8 pb = pack8(ph);
                half8 plb;
                if (PS) plb = pack8(pl);
                const int key0 = 32 * b + 16 * st + 4 * u;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const int d = 32 * dt + col;
                    const half8 va = lds_2xb64(&s_vt[0][d * kVStr + key0], &s_vt[0][d * kVStr + key0 + 8]);
                    acc[dt] = mfma(va, pb, acc[dt]);
                    if (PS) acc[dt] = mfma(va, plb, acc[dt]);
                    if (KS) {
                        const half8 vl = lds_2xb64(&s_vt[NK - 1][d * kVStr + key0],
                                                   &s_vt[NK - 1][d * kVStr + key0 + 8]);
                        acc[dt] = mfma(vl, pb, acc[dt]);
                    }
                }
            }
        }
    }

    // ---- normalise and write O[t, h, d] --------------------------------------------------
    const float L = sum_xor32(lsum);
    if (!qvalid) return;
    const float inv = 1.0f / L;
    const size_t obase = ((size_t)tq * a.hq + h) * kDim;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * dt + 8 * g + 4 * u;
            const float y0 = as_f32(acc[dt][4 * g] * inv), y1 = as_f32(acc[dt][4 * g + 1] * inv);
            const float y2 = as_f32(acc[dt][4 * g + 2] * inv), y3 = as_f32(acc[dt][4 * g + 3] * inv);
            if (OF32) {
                *reinterpret_cast<float4*>(static_cast<float*>(a.o) + obase + d) =
                    make_float4(y0, y1, y2, y3);
            } else {
                uint2 w;
                w.x = (uint32_t)f2h(y0) | ((uint32_t)f2h(y1) << 16);
                w.y = (uint32_t)f2h(y2) | ((uint32_t)f2h(y3) << 16);
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.o) + obase + d) = w;
            }
        }
    }
}


// ---- f16 cache, F16 / F16_PF32 precision: the hot path -------------------------------------
//
// Same work decomposition and MFMA formulation as prefill_kernel, with the K/V staging moved off
// the vector ALUs: each 64-key stage is copied HBM -> LDS by global_load_lds_dwordx4 (raw f16
// rows, 16-byte chunks XOR-swizzled so the operand reads are bank-conflict free), K A-operands
// are ds_read_b128 of those rows and V^T A-operands are ds_read_tr16_b64 of the same row-major
// tile. Two stages alternate so stage i + 1 streams in while stage i is contracted. The O
// accumulator is only rescaled when a column's running max grows by more than 2^8 (P then stays
// below 256, well inside f16), and masking runs only on tiles that cross the diagonal.
constexpr int kStageHalves = kTile * kDim;  // one 64 x 128 f16 tile

// physical 16-byte chunk of logical chunk c in row r
__device__ __forceinline__ int kswz(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int vswz(int r, int c) { return c ^ (4 * (r & 3)); }

constexpr int kMaxKeyParts = 8;
constexpr size_t kKeyPartFloats = 4 * 17 * 64 * 4;  // one part of one query tile

// Key split of prefill_f16_kernel: after its two key groups have merged, each group-0 wave of
// part `part` holds (acc, m, lsum) of its 32 queries over that part's keys. It stores them to
// a.part (layout [query tile][part][wave][17 x 16-byte chunks][lane]: acc in 16 chunks, then
// (m, lsum)) with device-coherent stores, waits until they are visible and counts its arrival
// on the wave's counter (atomic inc wrapping at kparts - 1, so the last arrival returns it to
// zero). The last wave to arrive loads every part's state and merges them in part order (max
// first, then 2^(m_p - max)-weighted sums), so the result does not depend on the arrival
// order; it returns true and its acc / lsum then hold the merged state. Other waves return false.
__device__ __forceinline__ bool merge_key_parts(const PrefillArgs& a, int tile, int part, int qw,
                                             int lane, f32x16 (&acc)[4], float& m_used,
                                             float& lsum) {
    constexpr int kChunks = 17;
    const size_t qt = (size_t)blockIdx.x * a.ntiles + tile;  // query tile (head group, tile)
    const size_t wave_floats = (size_t)kChunks * 64 * 4;
    auto state = [&](int p) {
        return a.part + ((qt * a.kparts + p) * 4 + qw) * wave_floats + 4 * lane;
    };
    float* mine = state(part);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            st_dev16(mine + (4 * dt + c) * 256,
                     f32x4{acc[dt][4 * c], acc[dt][4 * c + 1], acc[dt][4 * c + 2], acc[dt][4 * c + 3]});
    st_dev16(mine + 16 * 256, f32x4{m_used, lsum, 0.0f, 0.0f});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's stores are visible
    unsigned t = 0;
    if (lane == 0)
        t = __builtin_amdgcn_atomic_inc32(a.ctr + (qt * 4 + qw) * 16, (unsigned)(a.kparts - 1),
                                          __ATOMIC_RELAXED, "agent");
    // (every lane's stores were waited for before lane 0's increment: a wave's instructions
    // issue in order)
    if (__builtin_amdgcn_readlane(t, 0) != (unsigned)(a.kparts - 1)) return false;

    // ld_dev16 is a bare load: its registers are written when the data returns, so every batch
    // of loads below is followed by s_waitcnt vmcnt(0) and an asm that names the loaded
    // registers, which keeps any use of them (or reuse of those registers) after the wait.
    // maximum over the parts, then the weighted sums in part order
    // every slot gets a real load (parts past kparts and the own part read the own state,
    // unused): selecting between a load's result and another value before the wait would copy
    // the register before the data lands
    f32x4 ld[kMaxKeyParts];
#pragma unroll
    for (int p = 0; p < kMaxKeyParts; ++p)
        ld[p] = ld_dev16(state(p < a.kparts && p != part ? p : part) + 16 * 256);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int p = 0; p < kMaxKeyParts; ++p) asm volatile("" : "+v"(ld[p]));
    f32x4 ml[kMaxKeyParts];
#pragma unroll
    for (int p = 0; p < kMaxKeyParts; ++p)
        ml[p] = p == part ? f32x4{m_used, lsum, 0.0f, 0.0f}
                : p < a.kparts ? ld[p]
                               : f32x4{-INFINITY, 0.0f, 0.0f, 0.0f};
    float M = -INFINITY;
#pragma unroll
    for (int p = 0; p < kMaxKeyParts; ++p)
        if (p < a.kparts) M = fmaxf(M, ml[p][0]);
    float wp[kMaxKeyParts];
    float L = 0.0f;
#pragma unroll
    for (int p = 0; p < kMaxKeyParts; ++p) {
        wp[p] = (p >= a.kparts || ml[p][0] == -INFINITY) ? 0.0f
                                                        : __builtin_amdgcn_exp2f((ml[p][0] - M) * kLog2e);
        if (p < a.kparts) L += wp[p] * ml[p][1];
    }
    f32x16 sum[4] = {};
#pragma unroll
    for (int p = 0; p < kMaxKeyParts; ++p) {
        if (p >= a.kparts) break;
        if (p == part) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) sum[dt] += wp[p] * acc[dt];
            continue;
        }
        f32x4 v[16];  // part p's accumulator, one round trip
        const float* st = state(p);
#pragma unroll
        for (int c = 0; c < 16; ++c) v[c] = ld_dev16(st + c * 256);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int c = 0; c < 16; ++c) asm volatile("" : "+v"(v[c]));
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int j = 0; j < 4; ++j) sum[dt][4 * c + j] += wp[p] * v[4 * dt + c][j];
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = sum[dt];
    lsum = L;
    m_used = M;
    return true;
}

// One query tile of prefill_f16_kernel (the workgroup's whole work for it, merge and store
// included); s_kv = [K / V][group][buffer]: each group streams its own 64-key tiles; K and V
// have their own double buffers because K of tile i is free after tile i's QK^T, V only after
// its PV.
// qraw: this wave's raw half Q row. With q_ready it already holds the tile's Q, loaded by the
// previous tile's call (next_tile) while that tile merged and stored; next_tile >= 0 loads the
// next tile's Q into it the same way.
template <int HW, bool PS>
__device__ __forceinline__ void f16_pp_tile(const PrefillArgs& a, const int tile, const int part,
                                            const int ti, uint16_t (&s_kv)[2][2][2][kStageHalves],
                                            u32x4 (&qraw)[8], const bool q_ready,
                                            const int next_tile) {
    PREFILL_STAMP(1 + 6 * ti + kPfTileStart);
    constexpr int TPW = 32 * 4 / HW;
    constexpr int kTileBytes = kStageHalves * 2;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave >> 2;  // group g contracts the workgroup's tiles g, g + 2, g + 4, ...
    const int qw = wave & 3;    // head and 32-query block, as in prefill_kernel
    const int col = lane & 31;
    const int u = lane >> 5;

    const int hg = blockIdx.x;
    const int h = hg * HW + (qw % HW);
    const int kh = (hg * HW) / a.group;
    const int t0 = tile * TPW;
    const int tw0 = t0 + 32 * (qw / HW);
    const int lk = a.pos0 + a.tokens;
    const int kend_wg = a.pos0 + min(t0 + TPW, a.tokens);
    const int ntile_all = (kend_wg + kTile - 1) / kTile;  // 64-key tiles the query tile needs
    // this workgroup's part of them: tiles [tb, tb + ntile)
    const int tb = (int)((long long)ntile_all * part / a.kparts);
    const int ntile = (int)((long long)ntile_all * (part + 1) / a.kparts) - tb;
    const int ng = (ntile - grp + 1) / 2;               // tiles of this wave's group

    const int tq = tw0 + col;
    const bool qvalid = tq < a.tokens;
    half8 qh[8];
    if (q_ready) {
        // the loads were issued before the previous tile's output stores: this waits for them
        // only (the stores may still be in flight), before this tile's copies are issued
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(qraw[j]));
    } else {
        q_load_half(a.q + ((size_t)(qvalid ? tq : 0) * a.hq + h) * kDim, u, grp, qraw);
    }

    // lane-constant byte offsets: K operand rows (per k-step t), V^T tr16 sources (per dt),
    // DMA sources (per row quad r)
    // K operand of k-step t: row col, logical chunk 2 t + u = physical chunk (2 t ^ c14) + x0
    const uint32_t kcol = col * 256 + 16 * (u ^ (col & 1));
    const int c14 = col & 14;
    // (recomputed at each use from an opaque copy of c14: 2 VALU per MFMA instead of 8 live
    // registers the compiler would otherwise hoist and spill)
    auto koff = [&](int t, int c) { return kcol + 16 * ((2 * t) ^ c); };
    uint32_t voff[4];
    {
        const int sl = lane & 15, j = sl >> 2;
        const int low = 2 * ((lane >> 4) & 1) + ((sl & 3) >> 1);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            voff[dt] = (4 * u + j) * 256 + 16 * (4 * (dt ^ j) + low) + 8 * (sl & 1);
    }
    const uint32_t rstride = (uint32_t)a.hkv * 256;
    // DMA sources of row quad r (rows 16 qw + 4 r + lane / 16, chunk lane % 16 swizzled)
    const int lrow = lane >> 4, lchunk = lane & 15;
    auto kdo = [&](int r, int lr, int lc) {
        const int row = 16 * qw + 4 * r + lr;
        return (uint32_t)(row * rstride + 16 * kswz(row, lc));
    };
    auto vdo = [&](int r, int lr, int lc) {
        const int row = 16 * qw + 4 * r + lr;
        return (uint32_t)(row * rstride + 16 * vswz(row, lc));
    };
    const uint8_t* kbase = sgpr_base(a.k + (size_t)kh * 256);
    const uint8_t* vbase = sgpr_base(a.v + (size_t)kh * 256);
    // the 4 waves of a group copy 16 rows each of the group's tiles
    const uint32_t lds_k = lds_addr(&s_kv[0][grp][0][0]) + qw * 16 * 256;
    const uint32_t lds_v = lds_addr(&s_kv[1][grp][0][0]) + qw * 16 * 256;
    // tile i of this group = workgroup tile 2 i + grp, keys [kb(i), kb(i) + 64)
    auto kb_of = [&](int i) { return (tb + 2 * i + grp) * kTile; };
    // lane-constant copy sources, computed once (8 registers; the copies are issued in the
    // softmax phase, whose VALU slots are the less loaded ones)
    uint32_t kso[4], vso[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        kso[r] = kdo(r, lrow, lchunk);
        vso[r] = vdo(r, lrow, lchunk);
    }
    auto dma_k = [&](int i) {
        const uint8_t* g = sgpr_offset(kbase, (size_t)kb_of(i) * rstride);
#pragma unroll
        for (int r = 0; r < 4; ++r) lds_dma16_s(g, kso[r], lds_k + (i & 1) * kTileBytes + r * 1024);
    };
    auto dma_v = [&](int i) {
        const uint8_t* g = sgpr_offset(vbase, (size_t)kb_of(i) * rstride);
#pragma unroll
        for (int r = 0; r < 4; ++r) lds_dma16_s(g, vso[r], lds_v + (i & 1) * kTileBytes + r * 1024);
    };

    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_used = -INFINITY;  // shift of the column's exponentials (raw score units)
    float lsum = 0.0f;
    const int qabs = a.pos0 + tq;
    const float kGrow = 8.0f / kLog2e;  // rescale when the max grows by 2^8 in exp2 terms
    f32x16 s[2];                        // S^T of the current tile (32-key sub-blocks)
    half8 pb[4], plb[PS ? 4 : 1];       // P^T of the current tile, per 16-key k-step

    // MFMA phase i: O += V(i - 1) P(i - 1)^T, then S(i) = K(i) Q^T (each part if it exists;
    // P(i - 1) is dead before S(i) is written, which keeps the two out of registers together).
    // Both 32-key sub-blocks are always contracted: keys past the diagonal are masked to
    // -inf (P = 0), which keeps the tile code straight-line.
    auto mphase = [&](int i) {
        if (i > 0) {
            // O^T += V^T P^T over the 4 16-key k-steps; each k-step's 8 transposed V reads are
            // issued two k-steps ahead of its MFMAs (LDS latency under 8 waves is several MFMAs)
            const uint8_t* vt = reinterpret_cast<const uint8_t*>(&s_kv[1][grp][(i - 1) & 1][0]);
            half8 va[4][4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const int rows = 16 * ks * 256;
                    const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + voff[dt] + rows));
                    const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + voff[dt] + rows + 8 * 256));
                    va[ks][dt] = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    acc[dt] = mfma(va[ks][dt], pb[ks], acc[dt]);
                    if (PS) acc[dt] = mfma(va[ks][dt], plb[ks], acc[dt]);
                }
            // reads of k-steps 0 and 1 first, then one MFMA per 2 reads, then the rest
            __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, PS ? 2 : 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, PS ? 16 : 8, 0);
        }
        if (i < ng) {
            const f32x16 zero = {};
            const uint8_t* kt = reinterpret_cast<const uint8_t*>(&s_kv[0][grp][i & 1][0]);
            int c = c14;
            asm volatile("" : "+v"(c));
            half8 ka[2][8];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    ka[b][t] = lds_b128(reinterpret_cast<const uint16_t*>(kt + koff(t, c) + b * 32 * 256));
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                s[b] = mfma(ka[b][0], qh[0], zero);
#pragma unroll
                for (int t = 1; t < 8; ++t) s[b] = mfma(ka[b][t], qh[t], s[b]);
            }
            // sub-block 0's 8 K reads first, then one MFMA per read of sub-block 1, then the rest
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 1);
        }
    };
    // softmax phase i: mask, running max (lazy rescale of O), P(i) = exp(S(i) - m) in f16
    auto vphase = [&](int i) {
        const int kb = kb_of(i);
        // keys past this wave's last query or past lk: only tiles that reach that far
        if (kb + 63 > a.pos0 + tw0 || kb + 63 >= lk) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb + 32 * b + 8 * (r / 4) + 4 * u + (r % 4);
                    s[b][r] = (key > qabs || key >= lk) ? -INFINITY : s[b][r];
                }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[b][r]);
        tmax = max_xor32(tmax);
        const bool grow = tmax > m_used + kGrow;  // false while the column has no key
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_used - tmax) * kLog2e) : 1.0f;
            if (grow) m_used = tmax;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
        }
        // a column without a key so far (group 1's first tile for the first queries) has
        // m = -inf and every s = -inf: P = 2^(-inf - 0) = 0
        const float mb = m_used == -INFINITY ? 0.0f : m_used * kLog2e;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int b = ks >> 1, st = ks & 1;
            uint16_t ph[8], pl[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[b][8 * st + j], kLog2e, -mb));
                lsum += p;
                if (PS) split_f16(p, ph[j], pl[j]);
                else ph[j] = f2h(p);
            }
            pb[ks] = pack8(ph);
            if (PS) plb[ks] = pack8(pl);
        }
    };
    // copies issued after MFMA phase j: K(j + 2), then V(j + 1). Before MFMA phase i, K(i) and
    // V(i - 1) (issued after phase i - 2) must have landed; only the copies issued after phase
    // i - 1 (K(i + 1), V(i)) may still be in flight.
    auto copies_after = [&](int j) {
        if (j + 2 < ng) dma_k(j + 2);
        if (j + 1 < ng) dma_v(j + 1);
    };
    auto wait_for = [&](int i) {
        const int pend = 4 * (i + 1 < ng) + 4 * (i < ng);
        if (pend == 8) wait_vmcnt<8>();
        else if (pend == 4) wait_vmcnt<4>();
        else wait_vmcnt<0>();
    };

    // prologue: K(0), K(1), V(0) right behind the Q loads, then the Q conversion; the two
    // halves of each Q operand meet in group g's V buffer 1, idle until V(1) is copied after
    // MFMA phase 0 (every wave has read its Q by then: the barriers before that copy wait for
    // outstanding LDS reads)
    if (0 < ng) dma_k(0);
    if (1 < ng) dma_k(1);
    if (0 < ng) dma_v(0);
    {
        half8 qpart[4];
        q_convert_half(qraw, a.scale, qvalid, qpart);
        uint8_t* qx = reinterpret_cast<uint8_t*>(&s_kv[1][grp][1][0]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<uint4*>(qx + ((qw * 4 + j) * 64 + lane) * 16) = __builtin_bit_cast(uint4, qpart[j]);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 8; ++t)
            qh[t] = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(
                reinterpret_cast<const uint8_t*>(&s_kv[1][t >> 2][1][0]) + ((qw * 4 + (t & 3)) * 64 + lane) * 16));
    }
    PREFILL_STAMP(1 + 6 * ti + kPfPrologue);
    // Both groups run the same loop (MFMA phase k, barrier, softmax phase k, barrier); group 1
    // passes one extra barrier before it and group 0 one after it, so the barrier counts match
    // while group 1 runs one phase behind: each group's MFMA phase overlaps the other group's
    // softmax phase.
    const int niter = (ntile + 1) / 2 + 1;  // group 0's tiles + the final PV-only phase
    if (grp == 1) __syncthreads();
    for (int k = 0; k < niter; ++k) {
        const bool on = k <= ng;
        if (on) wait_for(k);
        __syncthreads();
        if (k == 0) PREFILL_STAMP(1 + 6 * ti + kPfFirstTile);
        if (on) mphase(k);
        __syncthreads();
        // after the barrier every wave of the group has read K(k) and V(k - 1): their buffers
        // take K(k + 2) and V(k + 1)
        if (on) copies_after(k);
        if (k < ng) vphase(k);
    }
    if (grp == 0) __syncthreads();
    wait_vmcnt<0>();
    PREFILL_STAMP(1 + 6 * ti + kPfLoopEnd);

    // ---- merge the two groups' key halves: group 1 hands (m, l, O) to group 0 through LDS ---
    __syncthreads();  // all tiles contracted, every copy waited for
    // The next tile's Q is loaded once this tile's LDS exchange is done (issued earlier, the
    // eight waves' loads delay the exchange behind them on the CU's vector-memory issue), in
    // flight during this tile's output stores. The barriers below order LDS accesses only.
    auto prefetch_q = [&]() {
        if (next_tile >= 0) {
            const int ntq = next_tile * TPW + 32 * (qw / HW) + col;
            q_load_half(a.q + ((size_t)(ntq < a.tokens ? ntq : 0) * a.hq + h) * kDim, u, grp, qraw);
        }
    };
    float* xch = reinterpret_cast<float*>(&s_kv[0][0][0][0]) + (size_t)(qw * 64 + lane) * 67;
    if (grp == 1) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) xch[16 * dt + i] = acc[dt][i];
        xch[64] = m_used;
        xch[65] = lsum;
    }
    lds_barrier();
    // the last barrier of the tile: after it the exchange area (the LDS of the next tile's
    // copies) has been read
    if (grp == 1) {
        lds_barrier();
        prefetch_q();
        return;
    }
    {
        const float mb2 = xch[64], lb = xch[65];
        const float M = fmaxf(m_used, mb2);
        // a group that saw no key of this column has m = -inf and weight 0
        const float wa = (m_used == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((m_used - M) * kLog2e);
        const float wb = (mb2 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((mb2 - M) * kLog2e);
        lsum = lsum * wa + lb * wb;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[dt][i] = acc[dt][i] * wa + xch[16 * dt + i] * wb;
        m_used = M;  // acc and lsum are now relative to M (the key split stores it with them)
    }
    lds_barrier();
    PREFILL_STAMP(1 + 6 * ti + kPfMerged);
    prefetch_q();

    if (a.kparts > 1 && !merge_key_parts(a, tile, part, qw, lane, acc, m_used, lsum)) return;
    const float L = sum_xor32(lsum);
    const float inv = 1.0f / L;  // padding columns: never stored
    // this wave's 8 KB of group 0's K buffers: group 0 copies into them only after this
    // epilogue; group 1, possibly in its next tile already, uses its own buffers
    store_o_rows(acc, inv, reinterpret_cast<uint8_t*>(&s_kv[0][0][0][0]) + qw * 32 * 256, lane, a.o,
                 tw0, a.tokens, a.hq, h);
#ifdef BRASA_PREFILL_TRACE
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    PREFILL_STAMP(1 + 6 * ti + kPfStored);
#endif
}

// Work order: head groups fastest (they spread over the XCDs), query tiles heaviest first. With
// a.pair the workgroup for y also takes the light tile y after the heavy tile ntiles - 1 - y, so
// each CU receives a pair of equal total work in one round (without it, a CU that finishes a
// light tile early takes the next one).
// GATED (q8_0 rows staged as f16 in F16 precision): the workgroup first reads the range gate
// of the call (gate_open); when the staging flagged a scale, it computes its query tiles with the
// exact path from the q8_0 cache (a.k8, a.v8) instead (the tile's key part 0 does, the other
// parts return), so such calls need no separate exact launch.
template <int HW, bool PS, bool GATED = false>
__global__ void __launch_bounds__(2 * kThreads, 1)
prefill_f16_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t s_kv[2][2][2][kStageHalves];
    if constexpr (GATED) {
        if (gate_open(a)) {
            constexpr int TPW = 32 * 4 / HW;
            const int y = blockIdx.y;
            int tiles[2] = {-1, -1};
            if (a.kparts > 1) {
                if (y % a.kparts == 0) tiles[0] = a.ntiles - 1 - y / a.kparts;
            } else {
                tiles[0] = a.ntiles - 1 - y;
                if (a.pair && y < tiles[0]) tiles[1] = y;
            }
            const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
            for (int ti = 0; ti < 2; ++ti) {
                if (tiles[ti] < 0) continue;
                const int t0 = tiles[ti] * TPW, nt = min(TPW, a.tokens - t0);
                // rows (token t0 + i, head blockIdx.x * HW + j), one per wave at a time
                for (int r = wave; r < nt * HW; r += 2 * kThreads / 64)
                    exact_row<BRASA_KV_Q8_0>(a, a.k8, a.v8,
                                             (t0 + r / HW) * a.hq + blockIdx.x * HW + r % HW, lane);
            }
            return;
        }
    }
    PREFILL_STAMP(0);
    u32x4 qraw[8];
    if (a.kparts > 1) {  // workgroup y: key part y % kparts of query tile ntiles - 1 - y / kparts
        f16_pp_tile<HW, PS>(a, a.ntiles - 1 - (int)blockIdx.y / a.kparts,
                            (int)blockIdx.y % a.kparts, 0, s_kv, qraw, false, -1);
        return;
    }
    const int y = blockIdx.y;
    const int heavy = a.ntiles - 1 - y;
    const bool second = a.pair && y < heavy;
    f16_pp_tile<HW, PS>(a, heavy, 0, 0, s_kv, qraw, false, second ? y : -1);
    if (second) f16_pp_tile<HW, PS>(a, y, 0, 1, s_kv, qraw, true, -1);
}

// Four-wave variant (one group, no key split), two workgroups per CU: with many query tiles per
// CU (long prompts) the second workgroup on each CU gives the overlap that the two key groups of
// prefill_f16_kernel give for short ones, without their merge and per-phase barriers.
template <int HW, bool PS>
__global__ void __launch_bounds__(kThreads, 2)
prefill_f16_kernel4(PrefillArgs a) {
    constexpr int TPW = 32 * 4 / HW;
    constexpr int kTileBytes = kStageHalves * 2;
    __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kStageHalves];
    __shared__ __attribute__((aligned(16))) uint16_t s_vv[2][kStageHalves];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31;
    const int u = lane >> 5;

    // Work order: head groups fastest (they spread over the XCDs); query tiles heaviest first
    // for the first half of the grid and lightest first for the second, so the two workgroups
    // that share a CU (first and second wave of dispatch) carry about the same total work.
    const int hg = blockIdx.x;
    const int half = (a.ntiles + 1) / 2;
    const int y = (int)blockIdx.y;
    const int tile = y < half ? a.ntiles - 1 - y : y - half;
    const int h = hg * HW + (wave % HW);
    const int kh = (hg * HW) / a.group;
    const int t0 = tile * TPW;
    const int tw0 = t0 + 32 * (wave / HW);
    const int lk = a.pos0 + a.tokens;
    const int kend_wg = a.pos0 + min(t0 + TPW, a.tokens);
    const int kend_w = a.pos0 + min(tw0 + 32, a.tokens);

    const int tq = tw0 + col;
    const bool qvalid = tq < a.tokens;
    half8 qh[8];
    u32x4 qraw[16];
    q_load(a.q + ((size_t)(qvalid ? tq : 0) * a.hq + h) * kDim, u, qraw);

    // lane-constant byte offsets: K operand rows (per k-step t), V^T tr16 sources (per dt),
    // DMA sources (per row quad r)
    uint32_t koff[8], voff[4], kdo[4], vdo[4];
#pragma unroll
    for (int t = 0; t < 8; ++t) koff[t] = col * 256 + 16 * kswz(col, 2 * t + u);
    {
        const int sl = lane & 15, j = sl >> 2;
        const int low = 2 * ((lane >> 4) & 1) + ((sl & 3) >> 1);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            voff[dt] = (4 * u + j) * 256 + 16 * (4 * (dt ^ j) + low) + 8 * (sl & 1);
    }
    const uint32_t rstride = (uint32_t)a.hkv * 256;
    {
        const int lrow = lane >> 4, lchunk = lane & 15;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * wave + 4 * r + lrow;
            kdo[r] = row * rstride + 16 * kswz(row, lchunk);
            vdo[r] = row * rstride + 16 * vswz(row, lchunk);
        }
    }
    const uint8_t* kbase = sgpr_base(a.k + (size_t)kh * 256);
    const uint8_t* vbase = sgpr_base(a.v + (size_t)kh * 256);
    const uint32_t lds_k = lds_addr(&s_k[0][0]) + wave * 16 * 256;
    const uint32_t lds_v = lds_addr(&s_vv[0][0]) + wave * 16 * 256;
    auto dma = [&](int kb, int buf) {
        const uint8_t* kg = sgpr_offset(kbase, (size_t)kb * rstride);
        const uint8_t* vg = sgpr_offset(vbase, (size_t)kb * rstride);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            lds_dma16_s(kg, kdo[r], lds_k + buf * kTileBytes + r * 1024);
            lds_dma16_s(vg, vdo[r], lds_v + buf * kTileBytes + r * 1024);
        }
    };

    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_used = -INFINITY;  // shift of the column's exponentials (raw score units)
    float lsum = 0.0f;
    const int qabs = a.pos0 + tq;
    const float kGrow = 8.0f / kLog2e;  // rescale when the max grows by 2^8 in exp2 terms

    auto stage = [&](int kb, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const uint8_t* kt = reinterpret_cast<const uint8_t*>(&s_k[buf][0]);
        const uint8_t* vt = reinterpret_cast<const uint8_t*>(&s_vv[buf][0]);
        const int nsub = (kb + 32 < kend_w) ? 2 : 1;
        const f32x16 zero = {};
        f32x16 s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b < nsub) {
                s[b] = mfma(lds_b128(reinterpret_cast<const uint16_t*>(kt + koff[0] + b * 32 * 256)), qh[0], zero);
#pragma unroll
                for (int t = 1; t < 8; ++t)
                    s[b] = mfma(lds_b128(reinterpret_cast<const uint16_t*>(kt + koff[t] + b * 32 * 256)), qh[t], s[b]);
            }
        }
        // causal mask (only on sub-blocks that reach past the wave's first query)
        float tmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b < nsub) {
                const int kb2 = kb + 32 * b;
                if ((kb2 + 31 > a.pos0 + tw0) || (kb2 + 31 >= lk)) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = kb2 + 8 * (i / 4) + 4 * u + (i % 4);
                        s[b][i] = (key > qabs || key >= lk) ? -INFINITY : s[b][i];
                    }
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[b][i]);
            }
        }
        tmax = max_xor32(tmax);
        const bool grow = tmax > m_used + kGrow;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_used - tmax) * kLog2e) : 1.0f;
            if (grow) m_used = tmax;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
        }
        const float mb = m_used * kLog2e;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nsub) break;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint16_t ph[8], pl[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[b][8 * st + j], kLog2e, -mb));
                    lsum += p;
                    if (PS) split_f16(p, ph[j], pl[j]);
                    else ph[j] = f2h(p);
                }
                const half8 pb = pack8(ph);
                half8 plb;
                if (PS) plb = pack8(pl);
                const int rows = (32 * b + 16 * st) * 256;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_v4s*)(vt + voff[dt] + rows));
                    const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_v4s*)(vt + voff[dt] + rows + 8 * 256));
                    const half8 va = __builtin_bit_cast(
                        half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc[dt] = mfma(va, pb, acc[dt]);
                    if (PS) acc[dt] = mfma(va, plb, acc[dt]);
                }
            }
        }
    };

    // stages alternate between the two LDS buffers; stage i + 1 streams in during stage i.
    // Stage 0's copies go out right behind the Q loads, then the Q conversion.
    dma(0, 0);
    q_convert(qraw, a.scale, qvalid, qh);
    for (int kb = 0; kb < kend_wg; kb += 2 * kTile) {
#pragma unroll
        for (int half_i = 0; half_i < 2; ++half_i) {
            const int kbi = kb + half_i * kTile;
            if (kbi >= kend_wg) break;
            __syncthreads();  // every wave is done with the buffer the next copy overwrites
            if (kbi + kTile < kend_wg) {
                dma(kbi + kTile, half_i ^ 1);
                wait_vmcnt<8>();
            } else {
                wait_vmcnt<0>();
            }
            __syncthreads();
            if (kbi < kend_w) {
                if (half_i == 0) stage(kbi, std::integral_constant<int, 0>{});
                else stage(kbi, std::integral_constant<int, 1>{});
            }
        }
    }

    const float L = sum_xor32(lsum);
    const float inv = 1.0f / L;  // padding columns: never stored
    __syncthreads();  // every wave is done with the K stages: wave w stages its output in 8 KB of them
    store_o_rows(acc, inv, reinterpret_cast<uint8_t*>(&s_k[0][0]) + wave * 32 * 256, lane, a.o, tw0,
                 a.tokens, a.hq, h);
}

// ---- q8_0 cache, F16 precision ------------------------------------------------------------
// prefill_f16_kernel4's work order and tile code, fed from a q8_0 cache: each wave loads its 16
// rows of a 64-key stage (codes and the group scales) into registers one stage ahead, converts
// every value to f16(code * scale) (the exact dequantised value rounded once, like Q * scale in
// this precision; codes4_to_f16 gives the codes exactly, one packed f16 multiply the rounding)
// and writes the f16 rows in the swizzled layouts the f16 kernels read, so the contraction runs
// at one MFMA per product instead of the generic kernel's hi / lo splits.
struct Q8Rows {
    u32x4 kc[2], vc[2];   // 16 codes of rows r0, r0 + 8 (lane's 16-byte chunk)
    uint32_t ks[2], vs[2];  // the f16 scale of the chunk's 32-group, per row (low half)
};

template <int HW>
__global__ void __launch_bounds__(kThreads, 2)
prefill_q8_kernel4(PrefillArgs a) {
    constexpr int TPW = 32 * 4 / HW;
    constexpr int RB = kQ8Row;
    __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kStageHalves];
    __shared__ __attribute__((aligned(16))) uint16_t s_vv[2][kStageHalves];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31;
    const int u = lane >> 5;

    const int hg = blockIdx.x;
    const int half = (a.ntiles + 1) / 2;
    const int y = (int)blockIdx.y / a.kparts;  // query tile order; key part y % kparts
    const int part = (int)blockIdx.y % a.kparts;
    const int tile = y < half ? a.ntiles - 1 - y : y - half;
    const int h = hg * HW + (wave % HW);
    const int kh = (hg * HW) / a.group;
    const int t0 = tile * TPW;
    const int tw0 = t0 + 32 * (wave / HW);
    const int lk = a.pos0 + a.tokens;
    const int kend_wg = a.pos0 + min(t0 + TPW, a.tokens);
    const int kend_w = a.pos0 + min(tw0 + 32, a.tokens);

    const int tq = tw0 + col;
    const bool qvalid = tq < a.tokens;
    half8 qh[8];
    u32x4 qraw[16];
    q_load(a.q + ((size_t)(qvalid ? tq : 0) * a.hq + h) * kDim, u, qraw);

    uint32_t koff[8], voff[4];
#pragma unroll
    for (int t = 0; t < 8; ++t) koff[t] = col * 256 + 16 * kswz(col, 2 * t + u);
    {
        const int sl = lane & 15, j = sl >> 2;
        const int low = 2 * ((lane >> 4) & 1) + ((sl & 3) >> 1);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            voff[dt] = (4 * u + j) * 256 + 16 * (4 * (dt ^ j) + low) + 8 * (sl & 1);
    }
    // this lane's rows of the stage (16 wave + lane / 8 + 8 i) and 16-byte code chunk lane % 8
    const size_t rstride = (size_t)a.hkv * RB;
    const int rr = lane >> 3, ch = lane & 7;
    const uint8_t* kbase = a.k + (size_t)kh * RB;
    const uint8_t* vbase = a.v + (size_t)kh * RB;
    auto load_rows = [&](int kb, Q8Rows& q) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // rows past the cache's last valid position are never read: the tile's keys are
            // below kend_wg <= cap, and rows past lk are finite (masked later)
            const size_t row = (size_t)(kb + 16 * wave + rr + 8 * i) * rstride;
            q.kc[i] = *reinterpret_cast<const u32x4*>(kbase + row + 16 * ch);
            q.vc[i] = *reinterpret_cast<const u32x4*>(vbase + row + 16 * ch);
            q.ks[i] = *reinterpret_cast<const uint16_t*>(kbase + row + 128 + 2 * (ch >> 1));
            q.vs[i] = *reinterpret_cast<const uint16_t*>(vbase + row + 128 + 2 * (ch >> 1));
        }
    };
    typedef _Float16 half2 __attribute__((ext_vector_type(2)));
    // 16 codes -> 16 f16 values code * scale (exact f16 codes, one rounding in the multiply)
    auto deq = [&](u32x4 c, uint32_t sc, uint32_t (&w)[8]) {
        const half2 s2 = __builtin_bit_cast(half2, sc | (sc << 16));
        const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t lo, hi;
            codes4_to_f16(cw[e], lo, hi);
            w[2 * e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, lo) * s2);
            w[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, hi) * s2);
        }
    };
    bool unsafe = false;  // a scale outside q8_f16_unsafe's range was met
    auto store_rows = [&](const Q8Rows& q, int buf) {
        uint8_t* kt = reinterpret_cast<uint8_t*>(&s_k[buf][0]);
        uint8_t* vt = reinterpret_cast<uint8_t*>(&s_vv[buf][0]);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = 16 * wave + rr + 8 * i;
            unsafe = unsafe || q8_f16_unsafe(q.ks[i]) || q8_f16_unsafe(q.vs[i]);
            uint32_t w[8];
            deq(q.kc[i], q.ks[i], w);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                *reinterpret_cast<u32x4*>(kt + row * 256 + 16 * kswz(row, 2 * ch + j)) =
                    u32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
            deq(q.vc[i], q.vs[i], w);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                *reinterpret_cast<u32x4*>(vt + row * 256 + 16 * vswz(row, 2 * ch + j)) =
                    u32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
        }
    };

    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_used = -INFINITY;
    float lsum = 0.0f;
    const int qabs = a.pos0 + tq;
    const float kGrow = 8.0f / kLog2e;

    auto stage = [&](int kb, int buf) {
        const uint8_t* kt = reinterpret_cast<const uint8_t*>(&s_k[buf][0]);
        const uint8_t* vt = reinterpret_cast<const uint8_t*>(&s_vv[buf][0]);
        const int nsub = (kb + 32 < kend_w) ? 2 : 1;
        const f32x16 zero = {};
        f32x16 s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b < nsub) {
                s[b] = mfma(lds_b128(reinterpret_cast<const uint16_t*>(kt + koff[0] + b * 32 * 256)), qh[0], zero);
#pragma unroll
                for (int t = 1; t < 8; ++t)
                    s[b] = mfma(lds_b128(reinterpret_cast<const uint16_t*>(kt + koff[t] + b * 32 * 256)), qh[t], s[b]);
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b < nsub) {
                const int kb2 = kb + 32 * b;
                if ((kb2 + 31 > a.pos0 + tw0) || (kb2 + 31 >= lk)) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = kb2 + 8 * (i / 4) + 4 * u + (i % 4);
                        s[b][i] = (key > qabs || key >= lk) ? -INFINITY : s[b][i];
                    }
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[b][i]);
            }
        }
        tmax = max_xor32(tmax);
        const bool grow = tmax > m_used + kGrow;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_used - tmax) * kLog2e) : 1.0f;
            if (grow) m_used = tmax;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
        }
        const float mb = m_used * kLog2e;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nsub) break;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint16_t ph[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[b][8 * st + j], kLog2e, -mb));
                    lsum += p;
                    ph[j] = f2h(p);
                }
                const half8 pb = pack8(ph);
                const int rows = (32 * b + 16 * st) * 256;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + voff[dt] + rows));
                    const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + voff[dt] + rows + 8 * 256));
                    const half8 va = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc[dt] = mfma(va, pb, acc[dt]);
                }
            }
        }
    };

    // stage i is converted into buffer i % 2 right after stage i - 1 was contracted (the barrier
    // before stage i - 1 saw every wave done with stage i - 2, the buffer's previous content);
    // its raw rows were loaded one stage earlier
    // this workgroup's key stages: [sb, sb + nst) of the tile's (all of them without a key split)
    const int nst_all = (kend_wg + kTile - 1) / kTile;
    const int sb = (int)((long long)nst_all * part / a.kparts);
    const int nst = (int)((long long)nst_all * (part + 1) / a.kparts) - sb;
    Q8Rows raw;
    load_rows(sb * kTile, raw);
    q_convert(qraw, a.scale, qvalid, qh);
    store_rows(raw, 0);
    if (1 < nst) load_rows((sb + 1) * kTile, raw);
    for (int i = 0; i < nst; ++i) {
        __syncthreads();  // stage i written by every wave; stage i - 1's buffer free
        const int kb = (sb + i) * kTile;
        if (kb < kend_w) stage(kb, i & 1);
        if (i + 1 < nst) {
            store_rows(raw, (i + 1) & 1);
            if (i + 2 < nst) load_rows((sb + i + 2) * kTile, raw);
        }
    }

    __syncthreads();  // every wave is done with the K stages: wave w stages its output in 8 KB of them
    if (a.taint && __builtin_amdgcn_ballot_w64(unsafe) != 0 && lane == 0) *a.taint = a.tag;
    if (a.kparts > 1 && !merge_key_parts(a, tile, part, wave, lane, acc, m_used, lsum)) return;
    const float L = sum_xor32(lsum);
    const float inv = 1.0f / L;
    store_o_rows(acc, inv, reinterpret_cast<uint8_t*>(&s_k[0][0]) + wave * 32 * 256, lane, a.o, tw0,
                 a.tokens, a.hq, h);
}

// Three workgroups per CU: prefill_f16_kernel4's tile code on 32-key stages in a three-stage
// ring (48 KB of LDS per workgroup), with the per-lane operand offsets recomputed at each use so
// a wave fits 168 registers and each SIMD holds three waves. The kernel is latency-bound (matrix
// cores ~27 % busy, LDS ~15 %): a third wave per SIMD and two stages in flight hide more of the
// dependent chains and of the copies' latency. Query tiles heaviest first; the dispatcher hands
// the light ones to CUs as they free up.
constexpr int kTileS = 32;                    // keys per stage
constexpr int kStageHalvesS = kTileS * kDim;  // one 32 x 128 f16 tile
template <int HW, bool PS>
__global__ void __launch_bounds__(kThreads, 3)
prefill_f16_kernel4s(PrefillArgs a) {
    constexpr int TPW = 32 * 4 / HW;
    constexpr int kTileBytes = kStageHalvesS * 2;
    // three-stage ring: the copies of stage i + 2 are issued when stage i starts (48 KB)
    __shared__ __attribute__((aligned(16))) uint16_t s_k[3][kStageHalvesS];
    __shared__ __attribute__((aligned(16))) uint16_t s_vv[3][kStageHalvesS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31;
    const int u = lane >> 5;

    const int hg = blockIdx.x;
    const int tile = a.ntiles - 1 - (int)blockIdx.y;
    const int h = hg * HW + (wave % HW);
    const int kh = (hg * HW) / a.group;
    const int t0 = tile * TPW;
    const int tw0 = t0 + 32 * (wave / HW);
    const int lk = a.pos0 + a.tokens;
    const int kend_wg = a.pos0 + min(t0 + TPW, a.tokens);
    const int kend_w = a.pos0 + min(tw0 + 32, a.tokens);

    const int tq = tw0 + col;
    const bool qvalid = tq < a.tokens;
    half8 qh[8];
    u32x4 qraw[16];
    q_load(a.q + ((size_t)(qvalid ? tq : 0) * a.hq + h) * kDim, u, qraw);

    // lane-constant byte offsets: K operand rows (recomputed per k-step from an opaque copy of
    // the row, as in prefill_f16_kernel), V^T tr16 sources (per dt), DMA sources (per row pair)
    const uint32_t kcol = col * 256 + 16 * (u ^ (col & 1));
    const int c14 = col & 14;
    auto koff = [&](int t, int c) { return kcol + 16 * ((2 * t) ^ c); };
    uint32_t voff[4];
    {
        const int sl = lane & 15, j = sl >> 2;
        const int low = 2 * ((lane >> 4) & 1) + ((sl & 3) >> 1);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            voff[dt] = (4 * u + j) * 256 + 16 * (4 * (dt ^ j) + low) + 8 * (sl & 1);
    }
    const uint32_t rstride = (uint32_t)a.hkv * 256;
    const uint8_t* kbase = sgpr_base(a.k + (size_t)kh * 256);
    const uint8_t* vbase = sgpr_base(a.v + (size_t)kh * 256);
    // each wave copies 8 rows of a 32-key stage: rows 8 wave + 4 r + lane / 16
    const uint32_t lds_k = lds_addr(&s_k[0][0]) + wave * 8 * 256;
    const uint32_t lds_v = lds_addr(&s_vv[0][0]) + wave * 8 * 256;
    // lane-constant copy sources, computed once (4 registers instead of a 32-bit multiply per copy)
    uint32_t kso[2], vso[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int row = 8 * wave + 4 * r + (lane >> 4), lc = lane & 15;
        kso[r] = (uint32_t)(row * rstride + 16 * kswz(row, lc));
        vso[r] = (uint32_t)(row * rstride + 16 * vswz(row, lc));
    }
    auto dma = [&](int kb, int buf) {
        const uint8_t* kg = sgpr_offset(kbase, (size_t)kb * rstride);
        const uint8_t* vg = sgpr_offset(vbase, (size_t)kb * rstride);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            lds_dma16_s(kg, kso[r], lds_k + buf * kTileBytes + r * 1024);
            lds_dma16_s(vg, vso[r], lds_v + buf * kTileBytes + r * 1024);
        }
    };

    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_used = -INFINITY;  // shift of the column's exponentials (raw score units)
    float lsum = 0.0f;
    const int qabs = a.pos0 + tq;
    const float kGrow = 8.0f / kLog2e;  // rescale when the max grows by 2^8 in exp2 terms

    auto stage = [&](int kb, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const uint8_t* kt = reinterpret_cast<const uint8_t*>(&s_k[buf][0]);
        const uint8_t* vt = reinterpret_cast<const uint8_t*>(&s_vv[buf][0]);
        const f32x16 zero = {};
        int c = c14;
        asm volatile("" : "+v"(c));
        f32x16 s = mfma(lds_b128(reinterpret_cast<const uint16_t*>(kt + koff(0, c))), qh[0], zero);
#pragma unroll
        for (int t = 1; t < 8; ++t)
            s = mfma(lds_b128(reinterpret_cast<const uint16_t*>(kt + koff(t, c))), qh[t], s);
        // causal mask (only on stages that reach past the wave's first query)
        if ((kb + 31 > a.pos0 + tw0) || (kb + 31 >= lk)) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kb + 8 * (i / 4) + 4 * u + (i % 4);
                s[i] = (key > qabs || key >= lk) ? -INFINITY : s[i];
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
        tmax = max_xor32(tmax);
        const bool grow = tmax > m_used + kGrow;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_used - tmax) * kLog2e) : 1.0f;
            if (grow) m_used = tmax;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
        }
        // a column without a key so far has m = -inf and every s = -inf: P = 0
        const float mb = m_used == -INFINITY ? 0.0f : m_used * kLog2e;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            uint16_t ph[8], pl[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[8 * st + j], kLog2e, -mb));
                lsum += p;
                if (PS) split_f16(p, ph[j], pl[j]);
                else ph[j] = f2h(p);
            }
            const half8 pb = pack8(ph);
            half8 plb;
            if (PS) plb = pack8(pl);
            const int rows = 16 * st * 256;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + voff[dt] + rows));
                const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + voff[dt] + rows + 8 * 256));
                const half8 va = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[dt] = mfma(va, pb, acc[dt]);
                if (PS) acc[dt] = mfma(va, plb, acc[dt]);
            }
        }
    };

    // stage i sits in ring slot i % 3; the copies of stage i + 2 go out when stage i starts, so
    // two stages stream in while one is contracted. Stages 0 and 1 go out right behind the Q
    // loads, then the Q conversion.
    dma(0, 0);
    if (kTileS < kend_wg) dma(kTileS, 1);
    q_convert(qraw, a.scale, qvalid, qh);
    for (int kb = 0; kb < kend_wg; kb += 3 * kTileS) {
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int kbi = kb + r * kTileS;
            if (kbi >= kend_wg) break;
            __syncthreads();  // every wave is done with the slot the next copy overwrites
            if (kbi + 2 * kTileS < kend_wg) {
                dma(kbi + 2 * kTileS, (r + 2) % 3);
                wait_vmcnt<8>();
            } else if (kbi + kTileS < kend_wg) {
                wait_vmcnt<4>();
            } else {
                wait_vmcnt<0>();
            }
            __syncthreads();
            if (kbi < kend_w) {
                if (r == 0) stage(kbi, std::integral_constant<int, 0>{});
                else if (r == 1) stage(kbi, std::integral_constant<int, 1>{});
                else stage(kbi, std::integral_constant<int, 2>{});
            }
        }
    }

    const float L = sum_xor32(lsum);
    const float inv = 1.0f / L;  // padding columns: never stored
    __syncthreads();  // every wave is done with the stages: waves 0-2 stage their output in the
                      // three 8 KB K stages, wave 3 in V stage 0
    store_o_rows(acc, inv, reinterpret_cast<uint8_t*>(wave < 3 ? &s_k[wave][0] : &s_vv[0][0]), lane,
                 a.o, tw0, a.tokens, a.hq, h);
}

// Kernel choice by workgroup count (one per query tile and head group), measured on one box at
// hq 32 / hkv 8: up to two per CU the two-group kernel, which splits each tile's keys over two
// wave groups (T = 2048: 512 workgroups, 58 vs 63 µs for the others; T = 512 at pos0 16384: 128
// workgroups, 269 vs 358 µs); from three per CU the 32-key-stage kernel with three workgroups per
// CU (T = 4096: 156 vs 187 µs; T = 8192: 580 vs 631 µs); in between the four-wave kernel
// (T = 2560: 76 vs 82 µs). The two-group kernel pairs heavy and light query tiles when the pairs
// still fill every CU (T = 2048: 57.0 vs 58.6 µs; at T = 1536 the 192 pairs leave CUs idle,
// 44 vs 39 µs). The test entry point brasa_test_flash_attention_layout() forces a kernel, turns
// pairing off or sets the key split for one call (PfCtx::variant / pair / parts), so tests cover
// every kernel at small sizes; the reference-signature entry points keep the choice by size.


// Arrival counters of the key-split merge: one per (query tile, wave), 64 bytes apart; a slot
// of kPfSlotWords per stream (stream_slot), zero at load, returned to zero by every launch (the
// last arrival wraps them). Next to them, one word per stream for the q8_0 range flag.
constexpr int kPfSlotWords = 16384;
__device__ unsigned g_pf_arrivals[kStreamSlots * kPfSlotWords];
__device__ unsigned g_pf_taint[kStreamSlots * 16];
unsigned* g_pf_ctr_base[kMaxDevices];
unsigned* g_pf_taint_base[kMaxDevices];
std::once_flag g_pf_ctr_once[kMaxDevices];
// Launch tags of the q8_0 range flag: one per call, never 0.
std::atomic<unsigned> g_pf_tag{0};

// The workspace of the reference-signature entry points (brasa_flash_attention[_with]), which
// take none: a fixed device array, so those calls allocate nothing. One stream per device owns
// it (the first to need it, until brasa_release_workspaces()); calls on other streams, and calls
// whose plan needs more, use the plans that fit (no key split, no q8_0 staging: slower, same
// results up to the split's last-bit effects). Sized for a q8_0 chunk of 512 tokens after 16384
// cached positions with its key split (69 MB of staging, 17 MB of partials).
constexpr size_t kStaticWsBytes = (size_t)96 << 20;
__device__ __align__(256) uint8_t g_pf_static_ws[kStaticWsBytes];
uint8_t* g_pf_static_base[kMaxDevices];
std::once_flag g_pf_static_once[kMaxDevices];
std::atomic<int> g_pf_static_owner[kMaxDevices];  // 0: free, slot + 1: owner

// One call's resources: its workspace (carved front to back), the stream's counters and flag.
// measure: nothing is launched; `need` sums what a workspace big enough for every feature of the
// plan would hold (brasa_flash_attention_workspace_len).
struct PfCtx {
    hipStream_t stream = nullptr;
    uint8_t* ws = nullptr;
    size_t ws_len = 0;
    size_t used = 0;
    bool measure = false;
    size_t need = 0;
    unsigned* ctr = nullptr;
    unsigned* taint = nullptr;
    unsigned tag = 0;
    // layout of this call: variant 0 chooses the f16 kernel by size, 1 / 2 / 4 force one (the
    // two-group kernel, four waves, four waves on 32-key stages); pair 0 keeps the two-group
    // kernel from pairing query tiles; parts: key parts of a forced two-group launch
    int variant = 0;
    int pair = 1;
    int parts = 1;

    void* take(size_t bytes) {
        bytes = (bytes + 255) / 256 * 256;
        if (measure) {
            need += bytes;
            return reinterpret_cast<void*>(static_cast<uintptr_t>(256));  // never dereferenced
        }
        if (!ws || used + bytes > ws_len) return nullptr;
        void* p = ws + used;
        used += bytes;
        return p;
    }
};

// Key parts per query tile: 1 (no split) unless the launch fills at most half of the
// workgroup slots (`slots`: CUs x workgroups per CU of the kernel) and the tiles' keys are long
// (a short chunk after a long cached prefix, e.g. 512 tokens at pos0 16384: 128 workgroups),
// then enough parts to fill the slots with parts of at least 16 64-key tiles each.
int key_parts(long long wgs, int keys, int slots) {
    int parts = 1;
    while (parts < kMaxKeyParts && wgs * parts * 2 <= slots && keys / (64 * parts * 2) >= 16) parts *= 2;
    return parts;
}

// parts within the limits of the workspace layout and the counter slot, else 1
int clamp_parts(int parts, long long wgs) {
    return (parts < 1 || parts > kMaxKeyParts || wgs * 4 * 16 > kPfSlotWords) ? 1 : parts;
}

// Launches `kernel` over (hq / HW) x (rows * parts) workgroups with a key split of `parts`
// (the stream's arrival counters, the parts' partials in the call's workspace). Returns 1 when
// the workspace or the counters are missing: the caller then launches unsplit.
template <typename K>
int launch_split(PfCtx& c, K kernel, const char* name, PrefillArgs b, int hw, long long wgs,
                 int parts, int threads) {
    void* ws = c.take((size_t)wgs * parts * kKeyPartFloats * sizeof(float));
    if (!ws || !c.ctr) return 1;
    if (c.measure) return BRASA_OK;
    b.pair = 0;
    b.kparts = parts;
    b.part = static_cast<float*>(ws);
    b.ctr = c.ctr;
    hipLaunchKernelGGL(kernel, dim3(b.hq / hw, b.ntiles * parts), dim3(threads), 0, c.stream, b);
    return check_launch(name);
}

// q8_0 rows -> f16 rows [rows, 128], each value f16(code * scale) by the same packed f16 multiply
// as prefill_q8_kernel4 (bit-identical values). One thread per 16-code chunk (two 8-byte code
// loads and the chunk's scale; 136-byte rows are 8-byte aligned); grid y: K, V. A scale for
// which those values can leave the normal f16 range stores `tag` at `taint`.
__global__ void __launch_bounds__(256)
dequant_q8_f16_kernel(const uint8_t* k, const uint8_t* v, uint16_t* kd, uint16_t* vd,
                      long long rows, unsigned* taint, unsigned tag) {
    const long long chunk = (long long)blockIdx.x * 256 + threadIdx.x;
    if (chunk >= rows * 8) return;
    const uint8_t* src = (blockIdx.y ? v : k) + (chunk >> 3) * kQ8Row;
    uint16_t* dst = (blockIdx.y ? vd : kd) + (chunk >> 3) * kDim;
    const int c = (int)(chunk & 7);
    const u32x2 c0 = *reinterpret_cast<const u32x2*>(src + 16 * c);
    const u32x2 c1 = *reinterpret_cast<const u32x2*>(src + 16 * c + 8);
    const uint32_t sc = *reinterpret_cast<const uint16_t*>(src + 128 + 2 * (c >> 1));
    if (q8_f16_unsafe(sc)) *taint = tag;
    typedef _Float16 half2 __attribute__((ext_vector_type(2)));
    const half2 s2 = __builtin_bit_cast(half2, sc | (sc << 16));
    const uint32_t cw[4] = {c0.x, c0.y, c1.x, c1.y};
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t lo, hi;
        codes4_to_f16(cw[e], lo, hi);
        w[2 * e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, lo) * s2);
        w[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, hi) * s2);
    }
    u32x4* out = reinterpret_cast<u32x4*>(dst + 16 * c);
    out[0] = u32x4{w[0], w[1], w[2], w[3]};
    out[1] = u32x4{w[4], w[5], w[6], w[7]};
}

// The recompute of q8_0 calls whose f16(code * scale) values leave the normal f16 range, for the
// launches whose fast kernel has no gate of its own (prefill_q8_kernel4, the four-wave f16
// kernels): it runs only when *gate == tag, i.e. after the fast launch flagged such a scale;
// otherwise every wave exits at once.
template <int KV>
__global__ void __launch_bounds__(256)
prefill_exact_kernel(PrefillArgs a) {
    if (a.gate && !gate_open(a)) return;
    const int lane = threadIdx.x & 63;
    // query token * hq + query head, grid-stride (a small grid: the common launch only reads
    // the gate)
    for (int rw = blockIdx.x * 4 + (threadIdx.x >> 6); rw < a.tokens * a.hq; rw += gridDim.x * 4)
        exact_row<KV>(a, a.k, a.v, rw, lane);
}

template <int KV>
int launch_exact(PfCtx& c, const PrefillArgs& a) {
    if (c.measure) return BRASA_OK;
    const long long rows = (long long)a.tokens * a.hq;
    hipLaunchKernelGGL(prefill_exact_kernel<KV>, dim3((unsigned)std::min<long long>((rows + 3) / 4, 64)),
                       dim3(256), 0, c.stream, a);
    return check_launch("prefill_exact_kernel");
}

template <int KV, int HW, bool QS, bool PS, bool OF32>
int launch(PfCtx& c, const PrefillArgs& a) {
    if (c.measure) return BRASA_OK;
    hipLaunchKernelGGL((prefill_kernel<KV, HW, QS, PS, OF32>), dim3(a.hq / HW, a.ntiles),
                       dim3(kThreads), 0, c.stream, a);
    return check_launch("prefill_kernel");
}

// GATED: a q8_0 F16 launch on staged f16 rows (a.gate set); *gated is set when the kernel
// launched reads the gate itself (the two-group kernel), so the caller needs no exact launch.
template <int HW, bool PS, bool GATED = false>
int launch_f16(PfCtx& c, const PrefillArgs& a, bool* gated = nullptr) {
    const long long wgs = (long long)(a.hq / HW) * a.ntiles;
    const int variant = c.variant;
    const int pick = variant ? variant : wgs <= 2 * 256 ? 1 : wgs < 3 * 256 ? 2 : 4;
    if (pick == 1) {
        if (gated) *gated = GATED;
        PrefillArgs b = a;
        b.pair = c.pair && wgs >= 2 * 256;
        // one workgroup per CU
        const int parts = clamp_parts(variant ? c.parts : key_parts(wgs, a.pos0 + a.tokens, 256),
                                      wgs);
        if (parts > 1) {
            const int st = launch_split(c, prefill_f16_kernel<HW, PS, GATED>, "prefill_f16_kernel",
                                        b, HW, wgs, parts, 2 * kThreads);
            if (st != 1) return st;
        }
        if (c.measure) return BRASA_OK;
        const int rows = b.pair ? (a.ntiles + 1) / 2 : a.ntiles;
        hipLaunchKernelGGL((prefill_f16_kernel<HW, PS, GATED>), dim3(a.hq / HW, rows),
                           dim3(2 * kThreads), 0, c.stream, b);
        return check_launch("prefill_f16_kernel");
    }
    if (c.measure) return BRASA_OK;
    if (pick == 4) {
        hipLaunchKernelGGL((prefill_f16_kernel4s<HW, PS>), dim3(a.hq / HW, a.ntiles), dim3(kThreads),
                           0, c.stream, a);
        return check_launch("prefill_f16_kernel4s");
    }
    hipLaunchKernelGGL((prefill_f16_kernel4<HW, PS>), dim3(a.hq / HW, a.ntiles), dim3(kThreads), 0,
                       c.stream, a);
    return check_launch("prefill_f16_kernel4");
}

// q8_0 cache, F16 precision, small launches: prefill_q8_kernel4 (f16(code * scale) in registers)
template <int HW>
int launch_q8_kernel4(PfCtx& c, const PrefillArgs& a) {
    // two workgroups per CU
    const long long wgs = (long long)(a.hq / HW) * a.ntiles;
    const int parts = clamp_parts(key_parts(wgs, a.pos0 + a.tokens, 512), wgs);
    if (parts > 1) {
        const int st = launch_split(c, prefill_q8_kernel4<HW>, "prefill_q8_kernel4", a, HW, wgs,
                                    parts, kThreads);
        if (st != 1) return st;
    }
    if (c.measure) return BRASA_OK;
    hipLaunchKernelGGL((prefill_q8_kernel4<HW>), dim3(a.hq / HW, a.ntiles), dim3(kThreads), 0,
                       c.stream, a);
    return check_launch("prefill_q8_kernel4");
}

// q8_0 cache, F16 precision, large launches: the rows the kernels read (ceil64(pos0 + tokens)
// positions) are dequantised into the call's workspace and the f16 kernels run on them: the
// values are those prefill_q8_kernel4 computes in registers, f16(code * scale), and the f16
// kernels' tile schedule is the faster one. Without room for the staging: prefill_q8_kernel4.
template <int HW>
int launch_q8_via_f16(PfCtx& c, const PrefillArgs& a, bool* gated) {
    const long long rows = (long long)((a.pos0 + a.tokens + 63) / 64 * 64) * a.hkv;
    const size_t bytes = (size_t)rows * kDim * 2;
    void* ws = c.take(2 * bytes);
    if (!ws) return launch_q8_kernel4<HW>(c, a);
    uint16_t* kd = static_cast<uint16_t*>(ws);
    uint16_t* vd = kd + rows * kDim;
    if (!c.measure) {
        hipLaunchKernelGGL(dequant_q8_f16_kernel, dim3((unsigned)((rows * 8 + 255) / 256), 2),
                           dim3(256), 0, c.stream, a.k, a.v, kd, vd, rows, a.taint, a.tag);
        const int st = check_launch("dequant_q8_f16_kernel");
        if (st != BRASA_OK) return st;
    }
    PrefillArgs b = a;
    b.k = reinterpret_cast<const uint8_t*>(kd);
    b.v = reinterpret_cast<const uint8_t*>(vd);
    b.k8 = a.k;
    b.v8 = a.v;
    b.gate = a.taint;  // flagged by the staging launch above; read (and cleared) by the f16 launch
    return launch_f16<HW, false, true>(c, b, gated);
}

template <int KV, int HW>
int launch_prec(PfCtx& c, PrefillArgs& a, int precision) {
    if constexpr (KV == BRASA_KV_F16) {
        if (precision == BRASA_PREFILL_F16) return launch_f16<HW, false>(c, a);
        if (precision == BRASA_PREFILL_F16_PF32) return launch_f16<HW, true>(c, a);
    }
    if constexpr (KV == BRASA_KV_Q8_0) {
        if (precision == BRASA_PREFILL_F16 && c.taint) {
            // the f16 kernels on dequantised rows when the work is large enough to hide the
            // dequantisation launch (measured: T = 384 at pos0 0 is the crossover; 128 tokens
            // after 16384 cached positions already gain 81 -> 71 us), else the q8_0 kernel.
            // Both flag scales whose f16(code * scale) can leave the normal f16 range; the next
            // launch then recomputes the call exactly (the reference's F16 numerics in f32):
            // the gated two-group f16 kernel itself, or else prefill_exact_kernel, which
            // otherwise exits at once.
            a.taint = c.taint;
            a.tag = c.tag;
            bool gated = false;
            const int st = (long long)a.tokens * (a.pos0 + a.tokens) < 384LL * 384
                               ? launch_q8_kernel4<HW>(c, a)
                               : launch_q8_via_f16<HW>(c, a, &gated);
            if (st != BRASA_OK || gated) return st;
            PrefillArgs g = a;
            g.taint = c.taint;  // cleared by the exact kernel (count at c.taint + 8)
            g.gate = c.taint;
            return launch_exact<KV>(c, g);
        }
        // (no range flag for this stream: the exact kernel directly)
        if (precision == BRASA_PREFILL_F16) return launch_exact<KV>(c, a);
    }
    switch (precision) {
        case BRASA_PREFILL_F32: return launch<KV, HW, true, true, true>(c, a);
        case BRASA_PREFILL_F16_PF32: return launch<KV, HW, false, true, false>(c, a);
        default: return launch<KV, HW, false, false, false>(c, a);
    }
}

template <int KV>
int launch_kv(PfCtx& c, PrefillArgs& a, int precision) {
    const int HW = (a.group % 4 == 0) ? 4 : (a.group % 2 == 0) ? 2 : 1;
    const int tpw = 32 * 4 / HW;
    a.ntiles = (a.tokens + tpw - 1) / tpw;
    switch (HW) {
        case 4: return launch_prec<KV, 4>(c, a, precision);
        case 2: return launch_prec<KV, 2>(c, a, precision);
        default: return launch_prec<KV, 1>(c, a, precision);
    }
}

PrefillArgs make_args(const float* q, const void* k, const void* v, void* o, int tokens, int hq,
                      int hkv, int pos0) {
    PrefillArgs a;
    a.q = q;
    a.k = static_cast<const uint8_t*>(k);
    a.v = static_cast<const uint8_t*>(v);
    a.o = o;
    a.tokens = tokens;
    a.hq = hq;
    a.hkv = hkv;
    a.group = hq / hkv;
    a.pos0 = pos0;
    a.ntiles = 0;
    a.pair = 0;
    a.kparts = 1;
    a.part = nullptr;
    a.ctr = nullptr;
    a.taint = nullptr;
    a.gate = nullptr;
    a.tag = 0;
    a.k8 = nullptr;
    a.v8 = nullptr;
    a.scale = 1.0f / sqrtf(static_cast<float>(kDim));
    return a;
}

int run(PfCtx& c, PrefillArgs& a, int kv, int precision) {
    switch (kv) {
        case BRASA_KV_F32: return launch_kv<BRASA_KV_F32>(c, a, precision);
        case BRASA_KV_F16: return launch_kv<BRASA_KV_F16>(c, a, precision);
        case BRASA_KV_Q8_0: return launch_kv<BRASA_KV_Q8_0>(c, a, precision);
    }
    return set_error(BRASA_ERR_ARG, "flash_attention: invalid kv type %d", kv);
}

}  // namespace

void prefill_release_workspaces() {
    for (auto& o : g_pf_static_owner) o.store(0, std::memory_order_relaxed);
}


size_t prefill_workspace_len(int tokens, int hq, int hkv, int pos0, int kv, int precision) {
    PrefillArgs a = make_args(nullptr, nullptr, nullptr, nullptr, tokens, hq, hkv, pos0);
    PfCtx c;
    c.measure = true;
    c.ctr = c.taint = reinterpret_cast<unsigned*>(static_cast<uintptr_t>(256));  // never used
    run(c, a, kv, precision);
    return c.need;
}

// caller_ws: the caller's workspace of ws_len bytes, at least prefill_workspace_len(); otherwise
// the reference-signature call (the fixed workspace when this stream owns it).
int prefill_launch(const float* q, const void* k, const void* v, void* o, int tokens, int hq,
                   int hkv, int pos0, int kv, int precision, bool caller_ws, void* ws,
                   size_t ws_len, hipStream_t stream, const int* layout) {
    int dev = 0, slot = -1;
    int st = stream_slot(stream, &dev, &slot);
    if (st != BRASA_OK) return st;
    std::call_once(g_pf_ctr_once[dev], [dev] {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_pf_arrivals)) == hipSuccess)
            g_pf_ctr_base[dev] = static_cast<unsigned*>(p);
        p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_pf_taint)) == hipSuccess)
            g_pf_taint_base[dev] = static_cast<unsigned*>(p);
    });
    if (!g_pf_ctr_base[dev] || !g_pf_taint_base[dev])
        return set_error(BRASA_ERR_LAUNCH, "flash_attention: arrival counters not found");
    PfCtx c;
    c.stream = stream;
    if (layout) {
        c.variant = layout[0];
        c.pair = layout[1];
        c.parts = layout[2];
    }
    if (slot >= 0) {
        c.ctr = g_pf_ctr_base[dev] + (size_t)slot * kPfSlotWords;
        c.taint = g_pf_taint_base[dev] + (size_t)slot * 16;
        unsigned t = 0;
        while (t == 0) t = g_pf_tag.fetch_add(1, std::memory_order_relaxed) + 1;
        c.tag = t;
    }
    if (caller_ws) {
        c.ws = static_cast<uint8_t*>(ws);
        c.ws_len = ws ? ws_len : 0;
    } else if (slot >= 0) {
        int expect = 0;
        if (g_pf_static_owner[dev].compare_exchange_strong(expect, slot + 1) || expect == slot + 1) {
            std::call_once(g_pf_static_once[dev], [dev] {
                void* p = nullptr;
                if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_pf_static_ws)) == hipSuccess)
                    g_pf_static_base[dev] = static_cast<uint8_t*>(p);
            });
            c.ws = g_pf_static_base[dev];
            c.ws_len = c.ws ? kStaticWsBytes : 0;
        }
    }
    PrefillArgs a = make_args(q, k, v, o, tokens, hq, hkv, pos0);
    return run(c, a, kv, precision);
}

}  // namespace brasa

#ifdef BRASA_PREFILL_TRACE
// Copies min(n, 8192 * 16) stamps of the timeline build to host memory `dst`.
extern "C" int brasa_prefill_trace_read(unsigned long long* dst, size_t n) {
    using namespace brasa;
    const size_t cnt = std::min(n, (size_t)kPfTraceWgs * kPfTraceStamps);
    const hipError_t e = hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_prefill_trace), cnt * sizeof(*dst));
    return e == hipSuccess ? 0 : BRASA_ERR_LAUNCH;
}
#endif
