// Split-K decode attention for gfx950 (one query token per sequence), one kernel per call.
//
// Behaviour follows Kernels::decode_attention_lanes / decode_attention of the reference
// (crates/kernels/src/lib.rs:1056-1164; decode_attention.metal:15-199): keys [0, lk) of one
// layer cache are cut into splits; each split produces per query head the online-softmax
// partial (m, l, acc[128]) and a second pass merges the splits as
// o = sum_s w_s acc_s / sum_s w_s l_s with w_s = exp(m_s - max m).
//
// Design for MI355X (HBM-bound: every K/V byte is read once per GQA group):
//   * workgroup = 4 wave64 = (split, KV head); a wave streams 32-key blocks of its split with the
//     next block's K/V loads in flight while the current one is computed;
//   * S^T = K Q^T on v_mfma_f32_16x16x32_f16. K rows go from HBM straight into the A operand
//     (lane = key row, 8 contiguous dims: 16-byte loads, no conversion for f16 caches). The
//     B operand holds the G query heads as columns, Q*scale split as hi + lo f16 (two MFMAs),
//     so the scores keep f32 accuracy (the reference computes them in f32);
//   * the S^T accumulator layout (lane = head column, 4 keys per lane) is used as the P^T
//     B operand as it stands; P is split hi + lo as well. O^T += V^T P^T on the same MFMA, with
//     V staged row-major in a wave-private LDS tile and read transposed by ds_read_tr16_b64;
//   * online softmax in fp32 (exp2 domain) with two xor-shuffles per block for the row max;
//   * the 4 waves merge through LDS into one partial per (head, split); a second small kernel
//     merges the splits (an in-kernel "last workgroup merges" protocol was measured slower:
//     its agent-scope release fence writes back the L2 of every workgroup's XCD);
//   * q8_0: codes are exact in f16; K scales multiply the per-32-dim-group MFMA partials (one
//     MFMA k-step is one group), V scales are folded into P per group; f32 caches are split
//     hi + lo like Q.
#include <cstring>

#include "common.hpp"

namespace brasa {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// Waves per workgroup: f16 caches use 8 (2 per SIMD, so one computes while the other's loads
// are in flight); the register-staged q8_0 / f32 paths use 4 (LDS).
template <int KV, int G> constexpr int waves_for() { return (KV == BRASA_KV_F16 && G <= 4) ? 8 : 4; }
constexpr int kBlock = 32;        // keys per wave iteration
constexpr int kVStr = 144;        // V tile row stride in halves (256 B + 32 B pad)
constexpr int kMaxSplits = 256;   // splits per sequence (the plan lengthens splits beyond that)

// Sequences per launch: their descriptors travel in the kernel arguments (no device-side
// metadata, so a call allocates and copies nothing).
constexpr int kMaxSeqs = 64;

struct SeqDesc {
    const uint8_t* k;     // layer cache base of this sequence
    const uint8_t* v;
    size_t part_off;      // floats: this sequence's partials (acc [hq][splits][128], then ml)
    int lk;               // keys
    int splits;
    int split0;           // first grid column of this sequence
    int pad;
};

struct DecodeArgs {
    const float* q;       // [nseq, hq, 128]
    float* part;          // caller scratch
    void* o;              // [nseq, hq, 128]
    int o_f16;
    int hq, hkv, group;   // group = hq / hkv
    int chunk;            // keys per split (the same for every sequence)
    int nseq;
    float scale;
    SeqDesc seq[kMaxSeqs];
};

// Grid column -> sequence (uniform per workgroup; nseq is small).
__device__ __forceinline__ int seq_of(const DecodeArgs& a, int col) {
    int si = 0;
    while (si + 1 < a.nseq && col >= a.seq[si + 1].split0) ++si;
    return si;
}

__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half8 as_half8(u32x4 x) { return __builtin_bit_cast(half8, x); }
__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) { return a | ((uint32_t)b << 16); }

// x = hi + lo with hi = f16(x), lo = f16(x - hi): ~22 significant bits through f16 MFMAs.
__device__ __forceinline__ void split8(const float (&x)[8], half8& hi, half8& lo) {
    u32x4 h, l;
    uint16_t hh[8], ll[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // x must be one f32 value for both halves: the backend would otherwise fold a product
        // x = a * b into a single-rounding f16 conversion for hi only, and when the f32 product
        // lies exactly on an f16 tie, hi + lo then misses x by one f16 ulp.
        const float xv = as_f32(x[j]);
        hh[j] = f2h(xv);
        ll[j] = f2h(xv - h2f(hh[j]));
    }
    h.x = pack2(hh[0], hh[1]); h.y = pack2(hh[2], hh[3]); h.z = pack2(hh[4], hh[5]); h.w = pack2(hh[6], hh[7]);
    l.x = pack2(ll[0], ll[1]); l.y = pack2(ll[2], ll[3]); l.z = pack2(ll[4], ll[5]); l.w = pack2(ll[6], ll[7]);
    hi = as_half8(h);
    lo = as_half8(l);
}

// 8 int8 codes -> 8 f16 values (exact: |code| <= 127).
__device__ __forceinline__ half8 codes_to_half8(u32x2 c) {
    u32x4 r;
    uint32_t w[2] = {c.x, c.y};
    uint16_t h[8];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            h[4 * i + b] = __half_as_ushort(__int2half_rn((int)(int8_t)((w[i] >> (8 * b)) & 0xffu)));
    r.x = pack2(h[0], h[1]); r.y = pack2(h[2], h[3]); r.z = pack2(h[4], h[5]); r.w = pack2(h[6], h[7]);
    return as_half8(r);
}

// One cache chunk of 8 consecutive dims as MFMA operand data: hi (and lo for f32 caches).
template <int KV> struct Chunk;
template <> struct Chunk<BRASA_KV_F16> {
    static constexpr bool kSplit = false;
    u32x4 raw;
    __device__ __forceinline__ void load(const uint8_t* row, int d) { raw = ld_stream<u32x4>(row + 2 * d); }
    __device__ __forceinline__ void get(half8& hi, half8&) const { hi = as_half8(raw); }
};
template <> struct Chunk<BRASA_KV_Q8_0> {
    static constexpr bool kSplit = false;
    u32x2 raw;
    __device__ __forceinline__ void load(const uint8_t* row, int d) { raw = ld_stream<u32x2>(row + d); }
    __device__ __forceinline__ void get(half8& hi, half8&) const { hi = codes_to_half8(raw); }
};
template <> struct Chunk<BRASA_KV_F32> {
    static constexpr bool kSplit = true;
    f32x4 a, b;
    __device__ __forceinline__ void load(const uint8_t* row, int d) {
        a = ld_stream<f32x4>(row + 4 * d);
        b = ld_stream<f32x4>(row + 4 * d + 16);
    }
    __device__ __forceinline__ void get(half8& hi, half8& lo) const {
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        split8(x, hi, lo);
    }
};

// Per-block register state of one wave: K fragments (2 key tiles x 4 dim steps), V chunks
// (8 rows of 4 per lane), and for q8_0 the f16 scales of the rows each lane needs.
template <int KV> struct Block {
    Chunk<KV> k[2][4];
    Chunk<KV> v[8];
    u32x2 ksc[2][4];   // q8_0: scales of S rows 16 kt + 4 u + i
    u32x2 vsc[8];      // q8_0: scales of P slot keys kappa(u, j)
    uint16_t vrs[8];   // q8_0: scale of V chunk i (row 4 i + u, group c16 / 4)
};

// A q8_0 scale s is applied as 2^e * (s * 2^-e), e = min(exponent(s), 9) (-14 for f16
// subnormals): 2^e goes into the f16 V codes (code * 2^e is exact in f16 for |code| <= 127) and
// the mantissa part into P, so P * mantissa keeps its hi/lo split clear of f16 subnormals.
__device__ __forceinline__ int q8_exp(uint16_t sc) {
    const int e = (int)((sc >> 10) & 31u);
    return e == 0 ? -14 : min(e - 15, 9);
}

template <int KV, int G>
__global__ void __launch_bounds__((64 * waves_for<KV, G>()), 1)
decode_kernel(DecodeArgs a) {
    constexpr int RB = KvTraits<KV>::row_bytes;
    constexpr bool KS = Chunk<KV>::kSplit;
    constexpr bool Q8 = (KV == BRASA_KV_Q8_0);
    constexpr int NV = KS ? 2 : 1;
    constexpr int kWaves = waves_for<KV, G>();
    constexpr int kThreads = 64 * kWaves;
    // f16 caches: V rows go HBM -> LDS directly (global_load_lds_dwordx4), double-buffered,
    // 16-byte chunks XOR-swizzled by 2 * (row & 3) so the transposed reads are conflict-free.
    // Other caches: V goes through registers (conversion), one padded tile (+ lo tile for f32).
    constexpr bool DMA = (KV == BRASA_KV_F16);
    constexpr int kVTile = DMA ? kBlock * kDim : NV * kBlock * kVStr;

    __shared__ __attribute__((aligned(16))) uint16_t s_v[kWaves][kVTile];
    // second V buffer of the DMA path, a distinct object so the compiler can tell its loads
    // from the first buffer's when it places waits
    __shared__ __attribute__((aligned(16))) uint16_t s_v2[kWaves][DMA ? kBlock * kDim : 8];
    __shared__ float s_acc[kWaves][G][kDim];
    __shared__ float s_m[kWaves][G];
    __shared__ float s_l[kWaves][G];

    const int si = seq_of(a, blockIdx.x);
    const SeqDesc& sd = a.seq[si];
    const int split = blockIdx.x - sd.split0;
    const float* qseq = a.q + (size_t)si * a.hq * kDim;
    const int h0 = blockIdx.y * G;         // first query head of this workgroup
    const int kh = h0 / a.group;           // its KV head
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;             // MFMA row/column index
    const int u = lane >> 4;               // MFMA k-group (8 of the 32 k-slots)
    const bool colq = c16 < G;             // this lane's column is a query head

    // ---- Q^T B-operands: column c = head h0 + c, k-step t holds dims 32 t + 8 u + j ----------
    half8 qhi[4], qlo[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        // unconditional 128-bit loads (a valid head for every lane), masked afterwards
        const f32x4* qp = reinterpret_cast<const f32x4*>(
            qseq + (size_t)(h0 + (colq ? c16 : 0)) * kDim + 32 * t + 8 * u);
        const f32x4 q0 = qp[0], q1 = qp[1];
        const float sc = colq ? a.scale : 0.0f;
        const float x[8] = {q0.x * sc, q0.y * sc, q0.z * sc, q0.w * sc,
                            q1.x * sc, q1.y * sc, q1.z * sc, q1.w * sc};  // f32, as reference
        split8(x, qhi[t], qlo[t]);
    }

    const int s0 = split * a.chunk;
    const int s1 = min(sd.lk, s0 + a.chunk);
    const size_t kstride = (size_t)a.hkv * RB;
    const uint8_t* kbase = sd.k + (size_t)kh * RB;
    const uint8_t* vbase = sd.v + (size_t)kh * RB;
    uint16_t* vt = &s_v[wave][0];
    uint16_t* vt2 = &s_v2[wave][0];

    auto load = [&](Block<KV>& b, int jb, int buf) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const uint8_t* row = kbase + (size_t)min(jb + 16 * kt + c16, s1 - 1) * kstride;
#pragma unroll
            for (int t = 0; t < 4; ++t) b.k[kt][t].load(row, 32 * t + 8 * u);
        }
        if constexpr (DMA) {
            // instruction i fills LDS rows 4 i .. 4 i + 3 of buffer `buf`; lane (u, p) writes
            // physical chunk p of row 4 i + u with logical chunk p ^ 2u
#pragma unroll
            for (int i = 0; i < 8; ++i)
                lds_dma16(vbase + (size_t)min(jb + 4 * i + u, s1 - 1) * kstride + 16 * (c16 ^ (2 * u)),
                          (buf ? vt2 : vt) + 512 * i);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                b.v[i].load(vbase + (size_t)min(jb + 4 * i + u, s1 - 1) * kstride, 8 * c16);
        }
        if constexpr (Q8) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                b.vrs[i] = *reinterpret_cast<const uint16_t*>(
                    vbase + (size_t)min(jb + 4 * i + u, s1 - 1) * kstride + 128 + 2 * (c16 >> 2));
        }
        if constexpr (Q8) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    b.ksc[kt][i] = *reinterpret_cast<const u32x2*>(
                        kbase + (size_t)min(jb + 16 * kt + 4 * u + i, s1 - 1) * kstride + 128);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = (j < 4) ? 4 * u + j : 16 + 4 * u + (j - 4);
                b.vsc[j] = *reinterpret_cast<const u32x2*>(
                    vbase + (size_t)min(jb + key, s1 - 1) * kstride + 128);
            }
        }
    };

    float m2[1] = {-INFINITY};  // running max of the column's scores, log2 domain
    float lsum = 0.0f;          // this lane's share of the column's softmax denominator
    f32x4 acc[8];               // O^T rows 16 dt + 4 u + i, column c16
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const Block<KV>& b, int jb, int buf) {
        // V rows -> wave-private LDS tile (row-major, 8 dims per lane and row)
#pragma unroll
        for (int i = 0; i < (DMA ? 0 : 8); ++i) {
            half8 hi, lo;
            b.v[i].get(hi, lo);
            if constexpr (Q8) {
                const _Float16 p2 = (_Float16)__builtin_amdgcn_ldexpf(1.0f, q8_exp(b.vrs[i]));
#pragma unroll
                for (int e = 0; e < 8; ++e) hi[e] = hi[e] * p2;  // exact: code * 2^e
            }
            *reinterpret_cast<half8*>(&vt[(4 * i + u) * kVStr + 8 * c16]) = hi;
            if constexpr (KS) *reinterpret_cast<half8*>(&vt[kBlock * kVStr + (4 * i + u) * kVStr + 8 * c16]) = lo;
        }
        // S^T tiles: rows = keys jb + 16 kt + 4 u + i, column = head
        float x[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            if constexpr (Q8) {
                float sk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    half8 kh8, unused;
                    b.k[kt][t].get(kh8, unused);
                    f32x4 p = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    p = mfma16(kh8, qhi[t], p);
                    p = mfma16(kh8, qlo[t], p);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t w = (t < 2) ? b.ksc[kt][i].x : b.ksc[kt][i].y;
                        const float sc = h2f((uint16_t)((t & 1) ? (w >> 16) : (w & 0xffffu)));
                        sk[i] = fmaf(p[i], sc, sk[i]);  // sum over groups of (q . codes) * scale
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) x[kt][i] = sk[i];
            } else {
                f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    half8 khi, klo;
                    b.k[kt][t].get(khi, klo);
                    s = mfma16(khi, qhi[t], s);
                    s = mfma16(khi, qlo[t], s);
                    if constexpr (KS) s = mfma16(klo, qhi[t], s);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) x[kt][i] = s[i];
            }
        }
        // online softmax (exp2 domain), keys past the split masked
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = jb + 16 * kt + 4 * u + i < s1;
                x[kt][i] = ok ? x[kt][i] * kLog2e : -INFINITY;
                bm = fmaxf(bm, x[kt][i]);
            }
        bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const float mn = fmaxf(m2[0], bm);  // finite: key jb is always valid
        const float alpha = __builtin_amdgcn_exp2f(m2[0] - mn);
        m2[0] = mn;
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(x[j >> 2][j & 3] - mn);
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ps += p[j];
        lsum = fmaf(lsum, alpha, ps);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;

        // O^T += V^T P^T; P^T slot j of lane (c, u) is key kappa(u, j) = j < 4 ? 4u + j : 16 + 4u + j - 4
        half8 phi[Q8 ? 4 : 1], plo[Q8 ? 4 : 1];
        if constexpr (Q8) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float pg[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t w = (g < 2) ? b.vsc[j].x : b.vsc[j].y;
                    const uint16_t sc = (uint16_t)((g & 1) ? (w >> 16) : (w & 0xffffu));
                    pg[j] = p[j] * __builtin_amdgcn_ldexpf(h2f(sc), -q8_exp(sc));
                }
                split8(pg, phi[g], plo[g]);
            }
        } else {
            split8(p, phi[0], plo[0]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const int trc = (c16 & 3), trj = (c16 >> 2);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const int col = 16 * dt + 4 * trc;
            const int g = Q8 ? (dt >> 1) : 0;
#pragma unroll
            for (int part = 0; part < NV; ++part) {
                const uint16_t *p1, *p2;
                if constexpr (DMA) {
                    // this tile's 8 DMA loads were followed by the next block's 8 K loads and
                    // 8 DMA loads; vector-memory counts retire in order
                    if (dt == 0) wait_vmcnt<16>();
                    // swizzled rows of 128 halves: physical chunk = logical ^ 2 (row & 3)
                    const uint16_t* base = buf ? vt2 : vt;
                    const int off = ((((2 * dt + (trc >> 1)) ^ (2 * trj))) << 3) + 4 * (trc & 1);
                    p1 = base + (4 * u + trj) * kDim + off;
                    p2 = base + (16 + 4 * u + trj) * kDim + off;
                } else {
                    const uint16_t* base = vt + part * kBlock * kVStr;
                    p1 = base + (4 * u + trj) * kVStr + col;
                    p2 = base + (16 + 4 * u + trj) * kVStr + col;
                }
                const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p1);
                const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p2);
                const half8 va = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[dt] = mfma16(va, phi[g], acc[dt]);
                if (part == 0) acc[dt] = mfma16(va, plo[g], acc[dt]);
            }
        }
    };

    // ---- stream this wave's blocks: jb = s0 + 32 (wave + 4 n), next block's loads in flight --
    const int stride = kWaves * kBlock;
    int jb = s0 + wave * kBlock;
    if (jb < s1) {
        Block<KV> A, B;
        load(A, jb, 0);
        // the prefetch is unconditional (rows clamp to s1 - 1): a branch around it would make
        // the compiler wait for every outstanding load before the current block's V writes
        while (true) {
            load(B, jb + stride, 1);
            compute(A, jb, 0);
            jb += stride;
            if (jb >= s1) break;
            load(A, jb + stride, 0);
            compute(B, jb, 1);
            jb += stride;
            if (jb >= s1) break;
        }
        // The last prefetch's HBM -> LDS copies are still in flight. They must land before the
        // wave ends: the workgroup's LDS is handed to the next workgroup on this CU when it
        // exits, and a late copy would overwrite that workgroup's data.
        if constexpr (DMA) wait_vmcnt<0>();
    }

    // ---- merge the wave's 4 k-groups (disjoint keys) and the 4 waves -----------------------
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    if (colq) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            *reinterpret_cast<f32x4*>(&s_acc[wave][c16][16 * dt + 4 * u]) = acc[dt];
        if (u == 0) {
            s_m[wave][c16] = m2[0];
            s_l[wave][c16] = lsum;
        }
    }
    __syncthreads();

    const int splits = sd.splits;
    const bool multi = splits > 1;
    float* acc_out = a.part + sd.part_off;
    float* ml_out = acc_out + (size_t)a.hq * splits * kDim;
    const size_t obase = (size_t)si * a.hq * kDim;
    for (int idx = threadIdx.x; idx < G * kDim; idx += kThreads) {
        const int h = idx / kDim, d = idx % kDim;
        float M = s_m[0][h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][h]);
        float A = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = __builtin_amdgcn_exp2f(s_m[w][h] - M);  // 0 for waves without keys
            A = fmaf(s_acc[w][h][d], wt, A);
            L = fmaf(s_l[w][h], wt, L);
        }
        const int hh = h0 + h;
        if (!multi) {
            const float out = A / L;
            if (a.o_f16) reinterpret_cast<uint16_t*>(a.o)[obase + hh * kDim + d] = f2h(out);
            else reinterpret_cast<float*>(a.o)[obase + hh * kDim + d] = out;
        } else {
            acc_out[((size_t)hh * splits + split) * kDim + d] = A;
            if (d == 0) {
                ml_out[((size_t)hh * splits + split) * 2] = M;
                ml_out[((size_t)hh * splits + split) * 2 + 1] = L;
            }
        }
    }
}

// Second pass (attn_decode_reduce, decode_attention.metal:68-84): one wave per (head, 32-dim
// slice). Lane = (split subset sub = lane / 8, float4 column oi = lane % 8): every lane issues
// all its loads at once ((m, l) and the acc float4 of splits sub, sub + 8, ...), so the pass
// costs one memory round trip; max, denominator and the split sum are xor-shuffle reductions.
constexpr int kRedSlice = 32;                          // dims per wave
constexpr int kRedPer = 8;                             // splits per lane held in registers

struct ReduceArgs {
    const float* part;
    void* o;
    int o_f16, hq, nseq;
    int splits[kMaxSeqs];
    size_t part_off[kMaxSeqs];
};

__global__ void __launch_bounds__(64) decode_reduce_kernel(ReduceArgs ra) {
    const int si = blockIdx.z;
    const int splits = ra.splits[si];
    if (splits == 1) return;  // the split kernel wrote this sequence's output
    const float* part = ra.part + ra.part_off[si];
    const int hq = ra.hq, o_f16 = ra.o_f16;
    void* o = o_f16 ? (void*)(static_cast<uint16_t*>(ra.o) + (size_t)si * hq * kDim)
                    : (void*)(static_cast<float*>(ra.o) + (size_t)si * hq * kDim);
    const int h = blockIdx.x, d0 = blockIdx.y * kRedSlice;
    const int lane = threadIdx.x, oi = lane & 7, sub = lane >> 3;
    const f32x4* acc = reinterpret_cast<const f32x4*>(part + (size_t)h * splits * kDim + d0) + oi;
    const f32x2* ml = reinterpret_cast<const f32x2*>(part + (size_t)hq * splits * kDim) + (size_t)h * splits;
    float M = -INFINITY;
    for (int s0 = sub; s0 < splits; s0 += 8 * kRedPer) {  // max pass over (m, l) (tiny)
#pragma unroll
        for (int r = 0; r < kRedPer; ++r) {
            const int s = s0 + 8 * r;
            if (s < splits) M = fmaxf(M, ml[s].x);
        }
    }
#pragma unroll
    for (int x = 8; x <= 32; x <<= 1) M = fmaxf(M, __shfl_xor(M, x, 64));
    f32x4 A = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float L = 0.0f;
    for (int s0 = sub; s0 < splits; s0 += 8 * kRedPer) {
        f32x2 mlv[kRedPer];
        f32x4 av[kRedPer];
#pragma unroll
        for (int r = 0; r < kRedPer; ++r) {
            const int s = min(s0 + 8 * r, splits - 1);
            mlv[r] = ml[s];
            av[r] = acc[(size_t)s * (kDim / 4)];
        }
#pragma unroll
        for (int r = 0; r < kRedPer; ++r) {
            if (s0 + 8 * r < splits) {
                const float w = __builtin_amdgcn_exp2f(mlv[r].x - M);
                A += av[r] * w;
                L = fmaf(mlv[r].y, w, L);
            }
        }
    }
#pragma unroll
    for (int x = 8; x <= 32; x <<= 1) {
        L += __shfl_xor(L, x, 64);
        A.x += __shfl_xor(A.x, x, 64);
        A.y += __shfl_xor(A.y, x, 64);
        A.z += __shfl_xor(A.z, x, 64);
        A.w += __shfl_xor(A.w, x, 64);
    }
    if (sub == 0) {
        const float y[4] = {A.x / L, A.y / L, A.z / L, A.w / L};
        const int off = h * kDim + d0 + 4 * oi;
        if (o_f16) {
            uint2 w;
            w.x = pack2(f2h(y[0]), f2h(y[1]));
            w.y = pack2(f2h(y[2]), f2h(y[3]));
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(o) + off) = w;
        } else {
            *reinterpret_cast<f32x4*>(static_cast<float*>(o) + off) = f32x4{y[0], y[1], y[2], y[3]};
        }
    }
}

template <int KV, int G>
int launch(const DecodeArgs& a, int groups_y, hipStream_t stream) {
    const int cols = a.seq[a.nseq - 1].split0 + a.seq[a.nseq - 1].splits;
    hipLaunchKernelGGL((decode_kernel<KV, G>), dim3(cols, groups_y), dim3((64 * waves_for<KV, G>())), 0, stream, a);
    return check_launch("decode_kernel");
}

template <int KV>
int launch_g(const DecodeArgs& a, int G, int groups_y, hipStream_t stream) {
    switch (G) {
        case 1: return launch<KV, 1>(a, groups_y, stream);
        case 2: return launch<KV, 2>(a, groups_y, stream);
        case 4: return launch<KV, 4>(a, groups_y, stream);
        case 8: return launch<KV, 8>(a, groups_y, stream);
    }
    return set_error(BRASA_ERR_UNSUPPORTED, "decode: GQA group %d not compiled", G);
}


}  // namespace

// Split plan for a batch of sequences: one split length `chunk` (a multiple of `unit` = 32 keys x
// waves per workgroup, >= 128) for all of them, chosen so that about BRASA_DECODE_WGS (default
// 256, one per CU) workgroups cover the GPU. A sequence of lk keys gets ceil(lk / chunk) <=
// ceil(lk / 128) splits, so its partials fit the reference's decode_partials_len(hq, lk) floats.
// The plan depends only on the lengths and the workgroups per split, so results are
// reproducible bit for bit.
int decode_chunk(const int* lk, int n, int wg_per_split, int unit) {
    static const int target_wgs = [] {
        const char* e = getenv("BRASA_DECODE_WGS");
        const int v = e ? atoi(e) : 0;
        return v > 0 ? v : 256;
    }();
    long long total = 0;
    for (int i = 0; i < n; ++i) total += lk[i];
    long long target = (target_wgs + wg_per_split - 1) / wg_per_split;
    if (target < 1) target = 1;
    long long chunk = (total + target - 1) / target;
    chunk = (chunk + unit - 1) / unit * unit;
    // at most kMaxSplits splits per sequence
    for (int i = 0; i < n; ++i) {
        const long long need = ((long long)lk[i] + kMaxSplits - 1) / kMaxSplits;
        if (chunk < need) chunk = (need + unit - 1) / unit * unit;
    }
    return (int)chunk;
}

// Floats of scratch a batch uses (<= the sum of decode_partials_len over its sequences).
size_t decode_batch_scratch(const int* lk, int n, int chunk, int hq) {
    size_t f = 0;
    for (int i = 0; i < n; ++i) f += (size_t)hq * ((lk[i] + chunk - 1) / chunk) * (kDim + 2);
    return f;
}

int decode_batch_launch(const float* q, const void* const* k, const void* const* v,
                        const int* lk, int n, float* partials, void* o, int o_f16, int hq,
                        int hkv, int kv, bool per_head, hipStream_t stream) {
    const int group = hq / hkv;
    const int G = per_head ? 1 : group;
    const int groups_y = per_head ? hq : hkv;
    const int waves = (kv == BRASA_KV_F16 && G <= 4) ? 8 : 4;  // waves_for<kv, G>
    const int chunk = decode_chunk(lk, n, groups_y, 32 * waves);
    const size_t oelem = o_f16 ? 2 : 4;
    size_t part_off = 0;
    for (int b0 = 0; b0 < n; b0 += kMaxSeqs) {
        const int nb = min(kMaxSeqs, n - b0);
        DecodeArgs a;
        memset(&a, 0, sizeof(a));
        a.q = q + (size_t)b0 * hq * kDim;
        a.part = partials;
        a.o = static_cast<uint8_t*>(o) + (size_t)b0 * hq * kDim * oelem;
        a.o_f16 = o_f16;
        a.hq = hq;
        a.hkv = hkv;
        a.group = group;
        a.chunk = chunk;
        a.nseq = nb;
        a.scale = 1.0f / sqrtf(static_cast<float>(kDim));
        ReduceArgs ra;
        memset(&ra, 0, sizeof(ra));
        ra.part = partials;
        ra.o = a.o;
        ra.o_f16 = o_f16;
        ra.hq = hq;
        ra.nseq = nb;
        int col = 0;
        bool any_multi = false;
        for (int i = 0; i < nb; ++i) {
            SeqDesc& d = a.seq[i];
            d.k = static_cast<const uint8_t*>(k[b0 + i]);
            d.v = static_cast<const uint8_t*>(v[b0 + i]);
            d.lk = lk[b0 + i];
            d.splits = (d.lk + chunk - 1) / chunk;
            d.split0 = col;
            d.part_off = part_off;
            col += d.splits;
            part_off += (size_t)hq * d.splits * (kDim + 2);
            ra.splits[i] = d.splits;
            ra.part_off[i] = d.part_off;
            any_multi |= d.splits > 1;
        }
        int st;
        switch (kv) {
            case BRASA_KV_F32: st = launch_g<BRASA_KV_F32>(a, G, groups_y, stream); break;
            case BRASA_KV_F16: st = launch_g<BRASA_KV_F16>(a, G, groups_y, stream); break;
            case BRASA_KV_Q8_0: st = launch_g<BRASA_KV_Q8_0>(a, G, groups_y, stream); break;
            default: return set_error(BRASA_ERR_ARG, "decode: invalid kv type %d", kv);
        }
        if (st != BRASA_OK) return st;
        if (!any_multi) continue;
        hipLaunchKernelGGL(decode_reduce_kernel, dim3(hq, kDim / kRedSlice, nb), dim3(64), 0,
                           stream, ra);
        st = check_launch("decode_reduce_kernel");
        if (st != BRASA_OK) return st;
    }
    return BRASA_OK;
}

int decode_launch(const float* q, const void* k, const void* v, float* partials, void* o,
                  int o_f16, int hq, int hkv, int lk, int kv, bool per_head,
                  hipStream_t stream) {
    return decode_batch_launch(q, &k, &v, &lk, 1, partials, o, o_f16, hq, hkv, kv, per_head,
                               stream);
}

}  // namespace brasa
