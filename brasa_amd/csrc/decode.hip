// Split-K decode attention for gfx950 (one query token per sequence), one kernel per call.
//
// Behaviour follows Kernels::decode_attention_lanes / decode_attention of the reference
// (crates/kernels/src/lib.rs:1056-1164; decode_attention.metal:15-199): keys [0, lk) of one
// layer cache are cut into splits; each split produces per query head the online-softmax
// partial (m, l, acc[128]) and the splits are merged as o = sum_s w_s acc_s / sum_s w_s l_s with
// w_s = exp(m_s - max m) (attn_decode_reduce, decode_attention.metal:68-84).
//
// Design for MI355X (HBM-bound: every K/V byte is read once per GQA group):
//   * workgroup = one head group (a KV head and its G query heads) x one split, W wave64 each
//     streaming the split's 32-key blocks w, w + W, ... with the next block's K/V loads in
//     flight. Workgroup b serves head group b % ngroups: with 8 KV heads the 8 XCDs each read
//     one head (workgroups are dealt to the XCDs round robin), and a sequence needs only
//     ~256 / ngroups splits, so the partials of a head group are few (32 at 16K keys);
//   * S^T = K Q^T on v_mfma_f32_16x16x32_f16. K rows go from HBM straight into the A operand;
//     the B operand holds the G query heads as columns, Q*scale split as hi + lo f16 so the
//     scores keep f32 accuracy (the reference computes them in f32). The S^T accumulator
//     layout is the P^T B operand as it stands; O^T += V^T P^T reads V transposed from LDS;
//   * online softmax in fp32 (exp2 domain);
//   * the split merge runs in the same kernel: the W waves merge through LDS, the workgroup
//     stores its partial with device-coherent stores and counts itself in an arrival counter
//     of its head group; the last workgroup to arrive merges all the splits and writes o. One
//     kernel per call: a second dependent launch for the merge costs ~3 us per layer here;
//   * q8_0: codes are exact in f16; K scales multiply the per-32-dim-group MFMA partials (one
//     MFMA k-step is one group), V scales are folded into P per group; f32 caches are split
//     hi + lo like Q.
// A single-sequence call's result is a function of (q, k, v, lk) only: the split length and the
// wave count per workgroup depend on lk alone (no tuning knob changes them) and every merge runs
// in a fixed order. A batched launch shares one split length, taken from the batch's total keys,
// so a sequence's splits, and with them the last bits of its result, can differ from the
// single-sequence call (both within the decode tolerance).
#include <atomic>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace brasa {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

constexpr int kBlock = 32;        // keys per wave iteration
constexpr int kMinChunk = 128;    // keys per split >= DECODE_CHUNK keeps the scratch bound
constexpr int kVStr = 144;        // V tile row stride in halves (256 B + 32 B pad)
constexpr int kTargetWgs = 256;   // workgroups per sequence the plan aims at (one per CU)

// Waves per workgroup (fixed per cache type, so results never depend on the launch).
constexpr int kWavesF16 = 8;
constexpr int kWavesQ8 = 8;
constexpr int kWavesF32 = 4;
// Query heads of one merge group (a workgroup's HPW head groups) the final merge's thread layout
// covers with 8 waves (kWavesF16 / kWavesQ8).
constexpr int kMaxMergeHeads = 16;
// Merge size bounds of the plan, in (query heads x splits) of a merge group; the last workgroup
// loads 520 bytes per (query head, split). Up to kMergeWorkSmall (66 KB) for any layout; up to
// kMergeWorkLong (~200 KB) when splits are long (>= kLongChunk keys), where streaming several KV
// heads per workgroup gains more than the larger merge costs.
constexpr int kMergeWorkSmall = 128;
constexpr int kMergeWorkLong = 384;
constexpr int kLongChunk = 512;

// Sequences per launch: their descriptors travel in the kernel arguments (no device-side
// metadata, so a call allocates and copies nothing).
constexpr int kMaxSeqs = 64;

// Arrival counters of the in-kernel split merge: one per (sequence, grid row) of a launch,
// kCtrStride apart (64 bytes: returning atomics on one line serialize, and with the counters of
// all rows packed in one line the last arrivals of a 16K-key decode waited ~2 us on each
// other), kSlotCounters words per slot. They start at zero when the library is loaded and every
// launch returns the counters it uses to zero (the last arrival wraps them), so nothing clears
// them. Each stream has a slot of its own (stream_slot): launches on one stream run in order,
// so no two launches in flight share counters.
constexpr int kCtrStride = 16;
constexpr int kSlotCounters = 16384;
__device__ unsigned g_arrivals[kStreamSlots * kSlotCounters];

// Split partials of brasa_decode_attention_lanes_noalloc: one fixed array per device, used in
// place of the caller's scratch (BRASA_DECODE_NOALLOC_FLOATS floats; a call needs
// hq * splits * 130 of them). Every call on a device shares it.
static __device__ __align__(256) float scratch[BRASA_DECODE_NOALLOC_FLOATS];

#ifdef BRASA_DECODE_TRACE
// Timeline build (libbrasa_attn_trace.so only): thread 0 of each workgroup writes the 100 MHz
// real-time counter at the phases of DecodeStamp into slot blockIdx.x % kTraceWgs. The stamps
// of waves other than wave 0 are not recorded; phases 4 and later wait for every wave.
constexpr int kTraceWgs = 8192;
constexpr int kTraceStamps = 16;
__device__ unsigned long long g_decode_trace[kTraceWgs * kTraceStamps];
#define DECODE_STAMP(k)                                                                       \
    do {                                                                                      \
        if (threadIdx.x == 0)                                                                 \
            g_decode_trace[(blockIdx.x % kTraceWgs) * kTraceStamps + (k)] =                  \
                __builtin_amdgcn_s_memrealtime();                                             \
    } while (0)
#else
#define DECODE_STAMP(k) \
    do {                \
    } while (0)
#endif
// Phases stamped by the timeline build.
enum DecodeStamp {
    kStampStart = 0,      // workgroup started
    kStampFirstBlock,     // wave 0: its first block's loads have landed
    kStampLastBlock,      // wave 0: its last block's loads have landed
    kStampWaveDone,       // wave 0: its blocks are computed
    kStampLdsMerged,      // every wave's state is in LDS
    kStampStored,         // the workgroup's partials are device-visible
    kStampArrived,        // the arrival counter returned
    kStampIssued,         // last arrival: the loads of every split's partial are issued
    kStampLoaded,         // last arrival: every split's partial has been loaded
    kStampMerged,         // last arrival: the splits are merged
    kStampOut,            // last arrival: o is written
};

struct SeqDesc {
    const uint8_t* k;     // layer cache base of this sequence
    const uint8_t* v;
    size_t part_off;      // floats: this sequence's partials (acc [hq][splits][128], then ml)
    int lk;               // keys
    int chunk;            // keys per split (a function of lk alone)
    int splits;
    int split0;           // first grid column of this sequence
};

template <int NS>
struct DecodeArgs {
    const float* q;       // [nseq, hq, 128]
    float* part;          // caller scratch
    void* o;              // [nseq, hq, 128]
    unsigned* ctr;        // this launch's arrival counters [nseq][ngroups]
    int o_f16;
    int hq, hkv, group;   // group = hq / hkv
    int ngroups;          // head groups: hkv (one per KV head) or hq (one query head each)
    int nseq;
    float scale;
    SeqDesc seq[NS];      // NS = 1 for single-sequence calls (smaller kernel arguments)
};

// Grid column -> sequence (uniform per workgroup; nseq is small).
template <int NS>
__device__ __forceinline__ int seq_of(const DecodeArgs<NS>& a, int col) {
    if constexpr (NS == 1) {
        return 0;
    } else {
        int si = 0;
        while (si + 1 < a.nseq && col >= a.seq[si + 1].split0) ++si;
        return si;
    }
}

// Grid position (row of head groups, split column) of this workgroup for the q8_0 kernel.
// Workgroup b runs on XCD b % 8 (round-robin dispatch), each XCD with its own L2. A q8_0 row
// of one KV head is 136 bytes, so adjacent heads share 128-byte lines; with rows varying
// fastest, the heads of one split sat on eight different XCDs and every shared line was
// fetched from HBM twice. Here the workgroups b, b + 8, ... (one XCD) take the rows of a
// column one after another, so the heads of a split share their lines in one L2 (16K keys:
// 21.5 -> 19.4 us). Any bijection is correct; this one needs the column count to be a
// multiple of 8 and falls back to rows-fastest otherwise.
__device__ __forceinline__ void xcd_grid_pos(int rows, int& row, int& col) {
    const int b = blockIdx.x;
    const int cols = gridDim.x / rows;
    if (cols % 8 == 0) {
        const int j = b >> 3;
        row = j % rows;
        col = (j / rows) * 8 + (b & 7);
    } else {
        row = b % rows;
        col = b / rows;
    }
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
        // callers pass products through as_f32: the backend would otherwise fold x = a * b
        // into a single-rounding f16 conversion for hi only, and when the f32 product lies
        // exactly on an f16 tie, hi + lo then misses x by one f16 ulp
        const float xv = x[j];
        hh[j] = f2h(xv);
        ll[j] = f2h(xv - h2f(hh[j]));
    }
    h.x = pack2(hh[0], hh[1]); h.y = pack2(hh[2], hh[3]); h.z = pack2(hh[4], hh[5]); h.w = pack2(hh[6], hh[7]);
    l.x = pack2(ll[0], ll[1]); l.y = pack2(ll[2], ll[3]); l.z = pack2(ll[4], ll[5]); l.w = pack2(ll[6], ll[7]);
    hi = as_half8(h);
    lo = as_half8(l);
}

// The half of split8 that one MFMA column takes: hi = f16(x), or lo = f16(x - hi) when `lo_part`
// (bit for bit what split8 gives). Pairs go through one v_cvt_pk_f16_f32 each and the residual
// x - hi is one exact fma with the f16 operand (it has at most 13 significant bits), so a lane
// converts only what its column uses.
// The hi or the lo part of the products x[j] * f[j] (f16 each), as split8_sel of the rounded
// products but with lo taken from the exact product: lo = f16(fma(x, f, -hi)). One select on the
// packed hi halves (zero in hi columns, where the fma then just rounds the product again).
__device__ __forceinline__ half8 split8_prod_sel(const float (&x)[8], const float (&f)[8],
                                                 bool lo_part) {
    typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
    typedef float ff2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const ff2 t = {as_f32(x[2 * i] * f[2 * i]), as_f32(x[2 * i + 1] * f[2 * i + 1])};
        const hf2 h = __builtin_convertvector(t, hf2);
        const hf2 hs = __builtin_bit_cast(hf2, lo_part ? __builtin_bit_cast(uint32_t, h) : 0u);
        const ff2 r = {fmaf(x[2 * i], f[2 * i], -(float)hs.x),
                       fmaf(x[2 * i + 1], f[2 * i + 1], -(float)hs.y)};
        w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, hf2));
    }
    return as_half8(u32x4{w[0], w[1], w[2], w[3]});
}
__device__ __forceinline__ half8 split8_sel(const float (&x)[8], bool lo_part) {
    typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
    typedef float ff2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const ff2 v = {x[2 * i], x[2 * i + 1]};
        const hf2 h = __builtin_convertvector(v, hf2);
        const ff2 r = {fmaf((float)h.x, -1.0f, v.x), fmaf((float)h.y, -1.0f, v.y)};
        const hf2 l = __builtin_convertvector(r, hf2);
        w[i] = lo_part ? __builtin_bit_cast(uint32_t, l) : __builtin_bit_cast(uint32_t, h);
    }
    return as_half8(u32x4{w[0], w[1], w[2], w[3]});
}

// f32 caches: 8 consecutive dims of a row as MFMA operand data, split into hi and lo halves.
struct F32Chunk {
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

// Per-block register state of one wave: K fragments (2 key tiles x 4 dim steps) and V chunks
// (8 rows of 4 per lane).
struct F32Block {
    F32Chunk k[2][4];
    F32Chunk v[8];
};

// A q8_0 scale s is applied as 2^e * (s * 2^-e), e = min(exponent(s), 5) (-14 for f16
// subnormals): 2^e goes into the f16 V codes (code * 2^e, exact, made by the conversion itself,
// codes4_to_f16_exp) and the rest m = s * 2^-e into P. m < 2 up to s < 64 and m < 2^11 above;
// with P <= 2^kLazyRescaleQ8 = 16 the product stays below 2^15 (f16 range), and its hi/lo split
// stays clear of f16 subnormals for m >= 2^-10.
__device__ __forceinline__ int q8_exp(uint16_t sc) {
    const int e = (int)((sc >> 10) & 31u);
    return e == 0 ? -14 : min(e - 15, 5);
}
// Row r's 16-byte V-code chunk c sits at chunk c ^ q8_vswz(r) of the row in LDS: the conversion's
// 16-byte reads (lane 2 r + h reads chunk 4 h + j of row r) then hit distinct bank groups.
__device__ __forceinline__ int q8_vswz(int r) { return (r ^ (r >> 2)) & 3; }

// max over the 4 rows of the wave (lanes l, l ^ 16, l ^ 32, l ^ 48)
__device__ __forceinline__ float max_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
    x = fmaxf(__int_as_float(a[0]), __int_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return fmaxf(__int_as_float(b[0]), __int_as_float(b[1]));
}
__device__ __forceinline__ float sum_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
    x = __int_as_float(a[0]) + __int_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float(b[0]) + __int_as_float(b[1]);
}

// ---- the end of a split: merge the W waves, then the splits --------------------------------
// (M, A, L) <- merge of (M, A, L) and (m, a, l): M = max, weights 2^(m - M) (0 for an empty side)
__device__ __forceinline__ void merge_split(float& M, f32x4& A, float& L, float m, f32x4 a,
                                            float l) {
    const float Mn = fmaxf(M, m);
    const float w0 = (M == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
    const float w1 = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - Mn);
    A = A * w0 + a * w1;
    L = L * w0 + l * w1;
    M = Mn;
}

template <int NS>
__device__ __forceinline__ void store_out(const DecodeArgs<NS>& a, int si, int h, int d, f32x4 y) {
    const size_t ob = ((size_t)si * a.hq + h) * kDim + d;
    if (a.o_f16) {
        u32x2 w;
        w.x = pack2(f2h(y.x), f2h(y.y));
        w.y = pack2(f2h(y.z), f2h(y.w));
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.o) + ob) = w;
    } else {
        *reinterpret_cast<f32x4*>(static_cast<float*>(a.o) + ob) = y;
    }
}

// LDS floats finish_split needs: the W waves' states, then the final merge's split groups and
// its (m, l) slots.
template <int G, int W>
constexpr int finish_floats() {
    return W * G * (kDim + 2) > 64 * W * 8 ? W * G * (kDim + 2) : 64 * W * 8;
}

// Every thread of the workgroup calls this once its wave's blocks are done. The workgroup serves
// HPW adjacent head groups (grid row `row`: head groups row * HPW ...), i.e. the HPW * G query
// heads q0 = row * HPW * G ...; wave w works for head group w % HPW. Wave state: acc[dt] holds
// O^T rows 16 dt + 4 u + r of column c16 (query head q0 + (w % HPW) G + c16 for c16 < G), already
// summed over the hi / lo columns; mref the column's reference point (log2 domain, -inf for a
// wave without keys) and lsum its softmax denominator (summed over the wave's rows). `lds` holds
// finish_floats<G, W>() floats that no wave still reads.
//  1. The W / HPW waves of each head group merge through LDS (in wave order, or by quarters of
//     the waves folded with permlane swaps when the thread layout allows). A sequence with one
//     split writes o here.
//  2. Otherwise the workgroup stores its partials (acc [hq][splits][128], then (m, l)
//     [hq][splits][2], the reference's scratch layout), waits until the stores are
//     device-visible and increments the arrival counter of its (sequence, row) (atomic inc
//     wrapping at splits - 1, so the last arrival leaves it at zero).
//  3. The last arrival merges every split: thread (sg, cc, q) takes splits sg, sg + NSG, ... of
//     query head q0 + cc, dims 4 q .. 4 q + 3, kPer per round trip; each round is folded as max
//     first, then sum_r 2^(m_r - max) (acc_r, l_r) in split order (a short dependency chain),
//     rounds and then the NSG split groups (by permlane swaps when they sit in lane bits 4-5,
//     else through LDS) are folded the same way, and o = A / L is written. The (m, l) pairs of a
//     round are loaded once per group of lanes that share them and passed on through LDS. The
//     order is fixed, so the result does not depend on which workgroup is last.
// Steps 1-3 below for kernels that have written their wave states to `lds` themselves:
// m_acc [W][G][128] (wave, head of the wave's head group, dim), then m_ml [W][G][2] (mref, lsum).
template <int G, int W, int HPW, int NS>
__device__ __forceinline__ void finish_split_lds(const DecodeArgs<NS>& a, const SeqDesc& sd, int si,
                                                 int row, int split, float* lds) {
    constexpr int KS = W / HPW;   // waves per head group
    constexpr int HG = HPW * G;   // query heads of the workgroup
    float* m_acc = lds;                   // [W][G][128]
    float* m_ml = lds + W * G * kDim;     // [W][G][2]
    __syncthreads();
    DECODE_STAMP(kStampLdsMerged);
    const int splits = sd.splits;
    const int q0 = row * HG;
    float* part_acc = a.part + sd.part_off;
    float* part_ml = part_acc + (size_t)a.hq * splits * kDim;
    // With 4 x 32 x HG = 64 W threads and KS a multiple of 4, every thread takes a quarter of
    // the waves of one (query head, dims) item, and the quarters (lanes l, l ^ 16, l ^ 32,
    // l ^ 48) are folded by permlane swaps; the lanes with quarter 0 store.
    constexpr bool kLaneQuarters = HG * 32 * 4 == 64 * W && KS % 4 == 0;
    if constexpr (kLaneQuarters) {
        constexpr int KQ = KS / 4;
        const int item = (threadIdx.x & 15) | ((threadIdx.x >> 6) << 4);
        const int kq = (threadIdx.x >> 4) & 3;
        const int hm = item / (G * 32), c = (item >> 5) % G, d = 4 * (item & 31);
        const int h = q0 + hm * G + c;
        float Mq = -INFINITY;
#pragma unroll
        for (int k = 0; k < KQ; ++k) Mq = fmaxf(Mq, m_ml[(((kq * KQ + k) * HPW + hm) * G + c) * 2]);
        f32x4 A = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
            const int wv = ((kq * KQ + k) * HPW + hm) * G + c;
            const float mw = m_ml[wv * 2];
            const float e = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - Mq);
            A += e * *reinterpret_cast<const f32x4*>(m_acc + wv * kDim + d);
            L += e * m_ml[wv * 2 + 1];
        }
        // the quarters: max first, then the weighted sums (the same bits in all four lanes)
        const float M = max_rows(Mq);
        const float w = Mq == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(Mq - M);
        A = f32x4{sum_rows(A.x * w), sum_rows(A.y * w), sum_rows(A.z * w), sum_rows(A.w * w)};
        L = sum_rows(L * w);
        if (kq == 0 && h < a.hq) {
            if (splits == 1) {
                store_out(a, si, h, d, A / L);
            } else {
                st_dev16(part_acc + ((size_t)h * splits + split) * kDim + d, A);
                if (d == 0) st_dev8(part_ml + ((size_t)h * splits + split) * 2, f32x2{M, L});
            }
        }
    }
    for (int idx = threadIdx.x; !kLaneQuarters && idx < HG * 32; idx += 64 * W) {
        const int hm = idx / (G * 32), c = (idx >> 5) % G, d = 4 * (idx & 31);
        const int h = q0 + hm * G + c;
        if (h >= a.hq) continue;  // a partial last row of head groups
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < KS; ++k) M = fmaxf(M, m_ml[((k * HPW + hm) * G + c) * 2]);
        f32x4 A = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const int wv = (k * HPW + hm) * G + c;
            const float mw = m_ml[wv * 2];
            const float e = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            A += e * *reinterpret_cast<const f32x4*>(m_acc + wv * kDim + d);
            L += e * m_ml[wv * 2 + 1];
        }
        if (splits == 1) {
            store_out(a, si, h, d, A / L);
        } else {
            st_dev16(part_acc + ((size_t)h * splits + split) * kDim + d, A);
            if (d == 0) st_dev8(part_ml + ((size_t)h * splits + split) * 2, f32x2{M, L});
        }
    }
    if (splits == 1) return;
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are visible
    DECODE_STAMP(kStampStored);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int rows = (a.ngroups + HPW - 1) / HPW;
        unsigned* ctr = a.ctr + (size_t)(si * rows + row) * kCtrStride;
        const unsigned t = __builtin_amdgcn_atomic_inc32(ctr, (unsigned)(splits - 1),
                                                         __ATOMIC_RELAXED, "agent");
        s_last = t == (unsigned)(splits - 1);
    }
    __syncthreads();
    DECODE_STAMP(kStampArrived);
    if (!s_last) return;

    constexpr int NSG = 64 * W / (HG * 32);  // split groups
    static_assert(NSG >= 1 && NSG * HG * 32 == 64 * W, "final-merge thread layout");
    // With 4 split groups they sit in lane bits 4 and 5 (lanes l, l ^ 16, l ^ 32, l ^ 48 of a
    // wave hold one (query head, dims) item), so the groups are folded by permlane swaps inside
    // the wave, with no LDS round trip or barrier; otherwise in LDS after the loop.
    constexpr bool kLaneGroups = NSG == 4;
    const int item = kLaneGroups ? ((threadIdx.x & 15) | ((threadIdx.x >> 6) << 4)) : threadIdx.x;
    const int q = item & 31, cc = (item >> 5) % HG;
    const int sg = kLaneGroups ? (threadIdx.x >> 4) & 3 : threadIdx.x / (32 * HG);
    const int h = min(q0 + cc, a.hq - 1);  // (duplicate work past hq is not stored)
    const float* pa = part_acc + (size_t)h * splits * kDim + 4 * q;
    const float* pm = part_ml + (size_t)h * splits * 2;
    float M = -INFINITY, L = 0.0f;
    f32x4 A = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int kPer = 8;  // splits per thread per round trip
    for (int s0 = sg; s0 < splits; s0 += kPer * NSG) {
        f32x4 av[kPer];
        f32x2 mv[kPer];
        {
            // The GL lanes of a split group (one query head and split group: 16 lanes with the
            // groups in lane bits 4-5, else 32) need the same kPer (m, l) pairs: lane j of the
            // group loads pair j % kPer, and the pairs go to the others through the wave's own
            // LDS slots (one load instead of kPer with GL equal addresses each; the loads'
            // address processing is the merge's bottleneck)
            constexpr int GL = kLaneGroups ? 16 : 32;
            f32x2 mine;
#pragma unroll
            for (int r = 0; r < kPer; ++r)
                av[r] = ld_dev16(pa + (size_t)min(s0 + NSG * r, splits - 1) * kDim);
            mine = ld_dev8(pm + (size_t)min(s0 + NSG * ((threadIdx.x & (GL - 1)) % kPer), splits - 1) * 2);
            DECODE_STAMP(kStampIssued);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            DECODE_STAMP(kStampLoaded);
#pragma unroll
            for (int r = 0; r < kPer; ++r) asm volatile("" : "+v"(av[r]));
            asm volatile("" : "+v"(mine));
            // 64 W (m, l) slots past the split-group fold's area (the wave merge's reads of
            // this LDS are done; a wave can reach the fold while another still reads its slots)
            f32x2* slots = reinterpret_cast<f32x2*>(lds + 6 * 64 * W);
            slots[threadIdx.x] = mine;
            const f32x2* grp = slots + (threadIdx.x & ~(GL - 1));  // this lane's group
#pragma unroll
            for (int r = 0; r < kPer; ++r) mv[r] = grp[r];
        }
        // this round's splits: max first, then the weighted sums in split order
        float Mr = -INFINITY;
#pragma unroll
        for (int r = 0; r < kPer; ++r)
            if (s0 + NSG * r < splits) Mr = fmaxf(Mr, mv[r].x);
        f32x4 Ar = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float Lr = 0.0f;
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const bool ok = s0 + NSG * r < splits && mv[r].x != -INFINITY;
            const float w = ok ? __builtin_amdgcn_exp2f(mv[r].x - Mr) : 0.0f;
            Ar += w * av[r];
            Lr += w * mv[r].y;
        }
        merge_split(M, A, L, Mr, Ar, Lr);
    }
    if constexpr (kLaneGroups) {
        // max first, then the weighted sums: every lane of the four adds the same values in
        // the same pairs (l with l ^ 16, then with l ^ 32), so all four hold the same bits
        const float Mx = max_rows(M);
        const float w = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mx);
        A = f32x4{sum_rows(A.x * w), sum_rows(A.y * w), sum_rows(A.z * w), sum_rows(A.w * w)};
        L = sum_rows(L * w);
        if (sg != 0) return;
    } else if constexpr (NSG > 1) {
        f32x4* r_a = reinterpret_cast<f32x4*>(lds);  // [NSG][HG][32], then m and l
        float* r_m = lds + 4 * 64 * W;
        float* r_l = r_m + 64 * W;
        r_a[threadIdx.x] = A;
        r_m[threadIdx.x] = M;
        r_l[threadIdx.x] = L;
        __syncthreads();
        if (sg != 0) return;
        float Mx = M;
#pragma unroll
        for (int k = 1; k < NSG; ++k) Mx = fmaxf(Mx, r_m[threadIdx.x + k * HG * 32]);
        A = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        L = 0.0f;
#pragma unroll
        for (int k = 0; k < NSG; ++k) {
            const int t = threadIdx.x + k * HG * 32;
            const float mk = r_m[t];
            const float w = mk == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mk - Mx);
            A += w * r_a[t];
            L += w * r_l[t];
        }
    }
    DECODE_STAMP(kStampMerged);
    if (q0 + cc < a.hq) store_out(a, si, q0 + cc, 4 * q, A / L);
#ifdef BRASA_DECODE_TRACE
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    DECODE_STAMP(kStampOut);
#endif
}

template <int G, int W, int HPW, int NS>
__device__ __forceinline__ void finish_split(const DecodeArgs<NS>& a, const SeqDesc& sd, int si,
                                             int row, int split, float* lds,
                                             const f32x4 (&acc)[8], float mref, float lsum) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;
    const int u = lane >> 4;
    float* m_acc = lds;                   // [W][G][128]
    float* m_ml = lds + W * G * kDim;     // [W][G][2]
    if (c16 < G) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            *reinterpret_cast<f32x4*>(m_acc + (wave * G + c16) * kDim + 16 * dt + 4 * u) = acc[dt];
        if (u == 0) *reinterpret_cast<f32x2*>(m_ml + (wave * G + c16) * 2) = f32x2{mref, lsum};
    }
    finish_split_lds<G, W, HPW>(a, sd, si, row, split, lds);
}

// ---- f32 caches (the reference's exact variant): register-staged K and V -------------------
// Workgroup = one head group x one split, W waves walking the split's blocks w, w + W, ... K and
// V rows are loaded into registers (the next block's loads in flight while the current block is
// computed) and split into f16 hi + lo halves; V goes through a wave-private padded LDS tile (hi
// and lo) to be read transposed.
template <int G, int NS, int W>
__global__ void __launch_bounds__(64 * W)
decode_f32_kernel(DecodeArgs<NS> a) {
    constexpr int RB = KvTraits<BRASA_KV_F32>::row_bytes;
    constexpr int kVTile = 2 * kBlock * kVStr;

    __shared__ __attribute__((aligned(16))) uint16_t s_v[W][kVTile];
    __shared__ __attribute__((aligned(16))) float s_fin[finish_floats<G, W>()];

    const int hg = blockIdx.x % a.ngroups;  // this workgroup's head group
    const int col = blockIdx.x / a.ngroups;
    const int si = seq_of(a, col);
    const SeqDesc& sd = a.seq[si];
    const int split = col - sd.split0;
    const float* qseq = a.q + (size_t)si * a.hq * kDim;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int h0 = hg * G;                 // its first query head
    const int kh = h0 / a.group;           // its KV head
    const int c16 = lane & 15;             // MFMA row/column index
    const int u = lane >> 4;               // MFMA k-group (8 of the 32 k-slots)
    // The 16 MFMA columns: c < G is head h0 + c with the hi halves of the split operands,
    // G <= c < 2 G the same head with the lo halves, the rest zero. Columns c and c ^ G add up
    // to the f32-accurate product, so one MFMA does the work of the hi and lo passes.
    const bool colq = c16 < G;             // this lane's column is a query head (hi half)
    const bool col_lo = c16 >= G && c16 < 2 * G;
    const int hcol = h0 + (c16 & (G - 1));

    // ---- Q^T B-operand: k-step t holds dims 32 t + 8 u + j -----------------------------------
    half8 qb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        // unconditional 128-bit loads (a valid head for every lane), masked afterwards
        const f32x4* qp = reinterpret_cast<const f32x4*>(qseq + (size_t)hcol * kDim + 32 * t + 8 * u);
        const f32x4 q0 = qp[0], q1 = qp[1];
        const float sc = (colq || col_lo) ? a.scale : 0.0f;
        const float x[8] = {as_f32(q0.x * sc), as_f32(q0.y * sc), as_f32(q0.z * sc),
                            as_f32(q0.w * sc), as_f32(q1.x * sc), as_f32(q1.y * sc),
                            as_f32(q1.z * sc), as_f32(q1.w * sc)};  // f32, as reference
        half8 hi, lo;
        split8(x, hi, lo);
        qb[t] = col_lo ? lo : hi;
    }

    // the split's 32-key blocks interleaved with the other splits' (split_blocks)
    const SplitBlocks sb = split_blocks(sd.lk, sd.splits, split);
    const int s0 = sb.first;
    const int s1 = sd.lk;
    const int nblk = sb.count;
    const int nb = nblk > wave ? (nblk - wave + W - 1) / W : 0;  // this wave's blocks
    const size_t kstride = (size_t)a.hkv * RB;
    const uint8_t* kbase = sd.k + (size_t)kh * RB;
    const uint8_t* vbase = sd.v + (size_t)kh * RB;
    uint16_t* vt = &s_v[wave][0];

    auto load = [&](F32Block& b, int jb) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const uint8_t* row = kbase + (size_t)min(jb + 16 * kt + c16, s1 - 1) * kstride;
#pragma unroll
            for (int t = 0; t < 4; ++t) b.k[kt][t].load(row, 32 * t + 8 * u);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            b.v[i].load(vbase + (size_t)min(jb + 4 * i + u, s1 - 1) * kstride, 8 * c16);
    };

    float m2[1] = {-INFINITY};  // running max of the column's scores, log2 domain
    float lsum = 0.0f;          // this lane's share of the column's softmax denominator
    f32x4 acc[8];               // O^T rows 16 dt + 4 u + i, column c16
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const F32Block& b, int jb) {
        // V rows -> wave-private LDS tiles (row-major, 8 dims per lane and row; hi then lo)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            half8 hi, lo;
            b.v[i].get(hi, lo);
            *reinterpret_cast<half8*>(&vt[(4 * i + u) * kVStr + 8 * c16]) = hi;
            *reinterpret_cast<half8*>(&vt[kBlock * kVStr + (4 * i + u) * kVStr + 8 * c16]) = lo;
        }
        // S^T tiles: rows = keys jb + 16 kt + 4 u + i, column = head
        float x[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                half8 khi, klo;
                b.k[kt][t].get(khi, klo);
                s = mfma16(khi, qb[t], s);
                s = mfma16(klo, qb[t], s);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) x[kt][i] = s[i];
        }
        // hi + lo columns: lanes c and c ^ G get the same sum (a + b == b + a), so both go
        // through the softmax below with identical bits
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[kt][i] += __shfl_xor(x[kt][i], G, 64);
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
        // P^T B-operand: hi halves in columns < G, lo halves in [G, 2 G)
        const half8 pb = split8_sel(p, col_lo);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const int trc = (c16 & 3), trj = (c16 >> 2);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const int col = 16 * dt + 4 * trc;
#pragma unroll
            for (int part = 0; part < 2; ++part) {  // V hi tile, then V lo tile
                const uint16_t* base = vt + part * kBlock * kVStr;
                const uint16_t* p1 = base + (4 * u + trj) * kVStr + col;
                const uint16_t* p2 = base + (16 + 4 * u + trj) * kVStr + col;
                const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p1);
                const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p2);
                const half8 va = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[dt] = mfma16(va, pb, acc[dt]);
            }
        }
    };

    // ---- stream this wave's 32-key blocks, the next block's loads in flight -----------------
    if (nb > 0) {
        auto blk = [&](int i) { return s0 + sb.stride * (wave + W * i); };
        F32Block A, B;
        load(A, blk(0));
        // the prefetch is unconditional (rows clamp to s1 - 1): a branch around it would make
        // the compiler wait for every outstanding load before the current block's V writes
        int i = 0;
        while (true) {
            load(B, blk(i + 1));
            compute(A, blk(i));
            if (++i >= nb) break;
            load(A, blk(i + 1));
            compute(B, blk(i));
            if (++i >= nb) break;
        }
    }

    // ---- this wave's partial for its G heads: combine the 4 k-groups' denominators ---------
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    // O^T column c (hi halves of P) plus column c + G (lo halves)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[dt][i] += __shfl_xor(acc[dt][i], G, 64);
    finish_split<G, W, 1>(a, sd, si, hg, split, s_fin, acc, m2[0], lsum);
}

// ---- f16 caches: every load explicit --------------------------------------------------------
// Workgroup = HPW adjacent head groups x one split of sd.chunk keys, W wave64; wave w works for
// head group w % HPW and walks the 32-key blocks ks, ks + KS, ... of the split (ks = w / HPW,
// KS = W / HPW), so at any time the workgroup reads HPW adjacent KV heads' rows. A wave keeps up to kRing blocks in flight: K rows go
// from HBM into registers (the MFMA A operand), V rows HBM -> LDS (global_load_lds_dwordx4, read
// transposed by ds_read_tr16_b64), Q into registers. Every vector-memory instruction of the
// block loop is inline asm, issued in a fixed order, so each wait is an exact count: block i is
// ready when the blocks issued after it (at most kRing - 1, 16 instructions each) are the only
// ones pending. The wait names the registers it guards as operands, so no use of them can be
// scheduled above it. Block i + kRing is issued into block i's ring slot once block i has been
// computed.
// Softmax: columns c < G hold the hi halves of the split Q / P operands, the partner columns
// (col_is_lo) the lo halves; one DPP exchange adds them (the same bits in both lanes). Only the
// sequence's last block masks keys past its end. The running max is lazy: the
// reference point moves only when a block's max exceeds it by more than 2^8, so most blocks skip
// the rescale of O.
constexpr int kRing = 2;                    // blocks in flight per wave (16 instructions each)
constexpr int kMaxLdsWaves = 8;
constexpr int kTileHalves = kBlock * kDim;  // one 32 x 128 f16 tile = 8 KB
constexpr float kLazyRescale = 8.0f;        // log2 of the largest P value before a rescale
constexpr float kLazyRescaleQ8 = 4.0f;      // the same for the q8_0 kernel (P * m in f16 range)

__device__ __forceinline__ u32x4 ld16_asm(const uint8_t* p) {
    u32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
// s_waitcnt vmcnt(N) that also "redefines" the 8 K registers of a ring slot, so the compiler
// cannot move a read of them above the wait.
template <int N>
__device__ __forceinline__ void wait_k(u32x4 (&k)[8]) {
    asm volatile("s_waitcnt vmcnt(%8)"
                 : "+v"(k[0]), "+v"(k[1]), "+v"(k[2]), "+v"(k[3]), "+v"(k[4]), "+v"(k[5]),
                   "+v"(k[6]), "+v"(k[7])
                 : "n"(N)
                 : "memory");
}
// Columns of the S^T / P^T MFMA operands of the f16 and q8_0 kernels for G query heads: head c
// (c < G) in column c with the hi half of its Q / P split, and its lo half in the partner column:
// 7 - c for G <= 4, so one row_half_mirror DPP exchanges the two halves, c + 8 for G = 8
// (row_ror:8). The other columns are zero.
template <int G>
__device__ __forceinline__ bool col_is_lo(int c16) {
    if constexpr (G == 8) return c16 >= 8;
    else return c16 >= 8 - G && c16 < 8;
}
template <int G>
__device__ __forceinline__ int col_head(int c16) {  // query head of a hi or lo column
    if constexpr (G == 8) return c16 & 7;
    else return c16 < G ? c16 : (col_is_lo<G>(c16) ? 7 - c16 : 0);
}
// the value of the partner column's lane (same row, same 4-key group)
template <int G>
__device__ __forceinline__ float partner(float x) {
    if constexpr (G == 8) return dpp<0x128>(x);  // row_ror:8
    else return dpp<0x141>(x);                   // row_half_mirror
}

template <int G, int NS, int HPW, int W>
__global__ void __launch_bounds__(64 * W)
decode_f16_kernel(DecodeArgs<NS> a) {
    DECODE_STAMP(kStampStart);
    constexpr int RB = 256;
    constexpr int KS = W / HPW;
    static_assert(W <= kMaxLdsWaves, "waves per workgroup");
    __shared__ __attribute__((aligned(16))) uint16_t s_v[W][kRing][kTileHalves];
    constexpr int kFin = finish_floats<G, W>();
    constexpr bool kSepFin = W * kRing * kTileHalves * 2 + kFin * 4 <= 160 * 1024;
    __shared__ __attribute__((aligned(16))) float s_fin[kSepFin ? kFin : 1];

    // grid: (split column, row of HPW head groups), rows innermost
    const int rows = (a.ngroups + HPW - 1) / HPW;
    const int row = blockIdx.x % rows;
    const int col = blockIdx.x / rows;
    const int si = seq_of(a, col);
    const SeqDesc& sd = a.seq[si];
    const int split = col - sd.split0;
    const float* qseq = a.q + (size_t)si * a.hq * kDim;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hl = wave % HPW, ks = wave / HPW;
    const int hg = row * HPW + hl;                 // this wave's head group
    const bool hg_ok = hg < a.ngroups;
    const int h0 = min(hg, a.ngroups - 1) * G;     // its first query head
    const int kh = h0 / a.group;                   // its KV head
    const int c16 = lane & 15;
    const int u = lane >> 4;
    const bool colq = c16 < G;
    const bool col_lo = col_is_lo<G>(c16);

    // The split's keys: the 32-key blocks split, split + splits, split + 2 splits, ... of the
    // sequence (the splits' blocks interleaved, so at any time the grid reads one region of the
    // cache: a read of one head's rows per workgroup takes 13.2 us at 16K keys this way against
    // 14.1 us with contiguous splits). Every split has at least one block (blocks >= splits since chunk >= 32),
    // at most chunk / 32, and only the sequence's last block is partial.
    const SplitBlocks sb = split_blocks(sd.lk, sd.splits, split);
    const int s1 = sd.lk;
    const int nblk = sb.count;
    const int bstride = sb.stride;  // keys from one of the split's blocks to the next
    const int s0 = sb.first;
    // this wave's blocks: ks, ks + KS, ...
    const int nb = (hg_ok && nblk > ks) ? (nblk - ks + KS - 1) / KS : 0;
    const size_t kstride = (size_t)a.hkv * RB;
    const uint8_t* kbase = sd.k + (size_t)kh * RB;
    const uint8_t* vbase = sd.v + (size_t)kh * RB;

    // Q rows of this lane's column (dims 32 t + 8 u .. + 8 for t < 4), loaded first
    u32x4 qr[8];
    {
        const uint8_t* qrow = reinterpret_cast<const uint8_t*>(qseq + (size_t)(h0 + col_head<G>(c16)) * kDim);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            qr[2 * t] = ld16_asm(qrow + 4 * (32 * t + 8 * u));
            qr[2 * t + 1] = ld16_asm(qrow + 4 * (32 * t + 8 * u + 4));
        }
    }
    u32x4 kr[kRing][8];
    // block i of this wave -> ring slot S: 8 K loads (tile row 16 kt + c16, dims 32 t + 8 u in
    // register kt * 4 + t), then 8 V copies (instruction r: rows 4 r .. 4 r + 3; chunk c of row
    // q stored at chunk c ^ 2 (q & 3))
    auto issue = [&](auto slot_c, int i) {
        constexpr int S = decltype(slot_c)::value;
        const int jb = s0 + bstride * (ks + KS * i);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const uint8_t* row = kbase + (size_t)min(jb + 16 * kt + c16, s1 - 1) * kstride + 16 * u;
#pragma unroll
            for (int t = 0; t < 4; ++t) kr[S][4 * kt + t] = ld16_asm(row + 64 * t);
        }
        uint16_t* vt = &s_v[wave][S][0];
#pragma unroll
        for (int r = 0; r < 8; ++r)
            lds_dma16_nt(vbase + (size_t)min(jb + 4 * r + u, s1 - 1) * kstride + 16 * (c16 ^ (2 * u)),
                         vt + 512 * r);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if (nb > 0) issue(I0{}, 0);
    if (nb > 1) issue(I1{}, 1);
    // Q was issued first: it has landed when at most the blocks' instructions are pending
    switch (min(nb, kRing)) {
        case 2: wait_k<32>(qr); break;
        case 1: wait_k<16>(qr); break;
        default: wait_k<0>(qr); break;
    }

    // ---- Q^T B-operand: k-step t holds dims 32 t + 8 u + j; column c < G: head h0 + c, hi half;
    // its partner column (col_is_lo): the same head, lo half; other columns zero ------------------
    half8 qb[4];
    {
        const float sc = (colq || col_lo) ? a.scale * kLog2e : 0.0f;  // scores in the log2 domain
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const f32x4 q0 = __builtin_bit_cast(f32x4, qr[2 * t]);
            const f32x4 q1 = __builtin_bit_cast(f32x4, qr[2 * t + 1]);
            const float x[8] = {as_f32(q0.x * sc), as_f32(q0.y * sc), as_f32(q0.z * sc),
                                as_f32(q0.w * sc), as_f32(q1.x * sc), as_f32(q1.y * sc),
                                as_f32(q1.z * sc), as_f32(q1.w * sc)};  // f32: q * (scale log2 e)
            half8 hi, lo;
            split8(x, hi, lo);
            qb[t] = col_lo ? lo : hi;
        }
    }

    float mref = -INFINITY;  // reference point of this column's exponentials, log2 domain
    float lsum = 0.0f;       // this lane's share of the column's softmax denominator
    f32x4 acc[8];            // O^T rows 16 dt + 4 u + i, column c16
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int trc = (c16 & 3), trj = (c16 >> 2);

    // One step computes block i from ring slot S and refills the slot with block i + kRing.
    auto step = [&](auto slot_c, int i) {
        constexpr int S = decltype(slot_c)::value;
        // block i's 16 instructions were followed by those of the block after it in the ring
        if (i + 1 < nb) wait_k<16>(kr[S]);
        else wait_k<0>(kr[S]);
        if (i == 0) DECODE_STAMP(kStampFirstBlock);
        if (i + 1 == nb) DECODE_STAMP(kStampLastBlock);
        const int jb = s0 + bstride * (ks + KS * i);
        // the V^T operands, read from LDS now (the block has landed) so the reads return while
        // S^T and the softmax are computed (after the rescale branch they waited for them)
        const uint16_t* vt = &s_v[wave][S][0];
        half8 va[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const int off = ((((2 * dt + (trc >> 1)) ^ (2 * trj))) << 3) + 4 * (trc & 1);
            const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + (4 * u + trj) * kDim + off));
            const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vt + (16 + 4 * u + trj) * kDim + off));
            va[dt] = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        }
        // S^T tiles: rows = keys jb + 16 kt + 4 u + r, column = head (hi / lo half)
        float x[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x4 sacc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) sacc = mfma16(as_half8(kr[S][4 * kt + t]), qb[t], sacc);
#pragma unroll
            for (int r = 0; r < 4; ++r) x[kt][r] = sacc[r];
        }
        // hi + lo: a lane and its partner add the same two values, so both hold the same bits
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) x[kt][r] = x[kt][r] + partner<G>(x[kt][r]);
        if (jb + kBlock > s1) {  // the sequence's last block: keys past its end get -inf
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (jb + 16 * kt + 4 * u + r >= s1) x[kt][r] = -INFINITY;
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) bm = fmaxf(bm, x[kt][r]);
        bm = max_rows(bm);  // finite: key jb is valid
        // lazy reference point: rescale O only when some column's max grew by more than 2^8
        if (__builtin_amdgcn_ballot_w64(bm > mref + kLazyRescale) != 0) {
            const float mn = fmaxf(mref, bm);
            const float alpha = __builtin_amdgcn_exp2f(mref - mn);
            mref = mn;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
        }
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(x[j >> 2][j & 3] - mref);
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ps += p[j];
        lsum += ps;
        const half8 pb = split8_sel(p, col_lo);
        // O^T += V^T P^T; P^T slot j of lane (c, u) is key j < 4 ? 4u + j : 16 + 4u + j - 4
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt] = mfma16(va[dt], pb, acc[dt]);
        if (i + kRing < nb) {
            // the slot's LDS reads have returned (their values fed the MFMAs above) before the
            // next block's copies into it are issued
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            asm volatile("" ::: "memory");
            issue(slot_c, i + kRing);
        }
    };
    for (int i0 = 0; i0 < nb; i0 += kRing) {
        step(I0{}, i0);
        if (i0 + 1 >= nb) break;
        step(I1{}, i0 + 1);
    }

    // ---- the split's end ---------------------------------------------------------------------
    lsum = sum_rows(lsum);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[dt][r] += partner<G>(acc[dt][r]);
            // every lane adds here (one v_add_f32_dpp), before the hi lanes' LDS stores: left
            // to itself, the compiler moved the adds into their masked region and the exchanges
            // became separate moves with zeroed destinations
            asm volatile("" : "+v"(acc[dt][r]));
        }
    // the merge area has its own LDS when it fits beside the ring; otherwise it reuses the V
    // slots once every wave is done with them (all copies waited for)
    float* fin;
    if constexpr (kSepFin) {
        fin = s_fin;
    } else {
        __syncthreads();
        fin = reinterpret_cast<float*>(&s_v[0][0][0]);
    }
    DECODE_STAMP(kStampWaveDone);
    finish_split<G, W, HPW>(a, sd, si, row, split, fin, acc, mref, lsum);
}

// ---- q8_0 caches: the f16 kernel's structure with codes and scales staged in LDS -----------
// Same workgroup layout, plan, explicit waits and split merge as decode_f16_kernel; two LDS slots
// per wave, but a wave issues block i + 1 only once block i has landed. A slot holds one 32-key
// block of K and V in their storage form: codes (32 x 128 bytes each) and the 4 f16 scales per
// row (32 x 8 bytes each), copied by 16-byte (codes) and 4-byte (scales) global_load_lds; 10
// copy instructions per block.
//  * S^T = K Q^T: K codes are read in the MFMA A layout (16-byte chunk c of row r stored at
//    c ^ ((r >> 1) & 7): conflict-free 8-byte reads), converted exactly to f16, and each 32-dim
//    group (one MFMA k-step) gets its own accumulator, scaled by that row's group scale in f32:
//    s = sum_g scale_g * (q . codes_g), the exact dequantised dot product up to f32 rounding.
//  * O^T += V^T P^T: after the block's S, each lane converts 64 V codes (V rows stored with
//    chunk c of row r at c ^ q8_vswz(r)) to f16 times 2^e (exact: |code| <= 127, -14 <= e <= 5,
//    the 2^e built into the conversion's magic number) and writes them as the f16 V tile over
//    the block's code area (the ds_read_tr16_b64 layout of the f16 kernel); the rest of the
//    scale, scale * 2^-e, is folded into P per 32-dim group, so every product stays exact up to
//    the f32 accumulation.
constexpr int kQ8Codes = kBlock * 128;        // bytes of one tile's codes
constexpr int kQ8Fac = 2 * kQ8Codes + 2 * kBlock * 8;   // K codes, V codes, K scales, V scales,
constexpr int kQ8Slot = kQ8Fac + kBlock * 4 * 4;         // then V mantissa factors [key][group]

// The copies carry no nontemporal hint (the fp16 kernel's V copies do): a 136-byte row of one KV head
// shares 128-byte lines with its scale copy and with the adjacent heads (read by the other
// workgroups of the split on the same XCD, xcd_grid_pos), and cached normally those lines are
// fetched fewer times (measured: 16K keys 16.2 -> 15.2 us per layer, 32K 25.6 -> 23.2, 4K
// 9.7 -> 9.5; for the fp16 kernel's V copies the hint is the faster choice, for its K loads
// plain loads: 17.47 -> 17.33 us at 16K).
template <int G, int NS, int HPW, int W>
__global__ void __launch_bounds__(64 * W)
decode_q8_kernel(DecodeArgs<NS> a) {
    DECODE_STAMP(kStampStart);
    constexpr int RB = kQ8Row;
    constexpr int KS = W / HPW;
    static_assert(W <= kMaxLdsWaves, "waves per workgroup");
    static_assert(finish_floats<G, W>() * 4 <= W * kRing * kQ8Slot, "merge area in the ring");
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[W][kRing][kQ8Slot];

    const int rows = (a.ngroups + HPW - 1) / HPW;
    int row, col;
    xcd_grid_pos(rows, row, col);
    const int si = seq_of(a, col);
    const SeqDesc& sd = a.seq[si];
    const int split = col - sd.split0;
    const float* qseq = a.q + (size_t)si * a.hq * kDim;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR math
    const int hl = wave % HPW, ks = wave / HPW;
    const int hg = row * HPW + hl;
    const bool hg_ok = hg < a.ngroups;
    const int h0 = min(hg, a.ngroups - 1) * G;
    const int kh = h0 / a.group;
    const int c16 = lane & 15;
    const int u = lane >> 4;
    const bool colq = c16 < G;
    const bool col_lo = col_is_lo<G>(c16);

    // the split's 32-key blocks interleaved with the other splits', as in decode_f16_kernel
    const SplitBlocks sb = split_blocks(sd.lk, sd.splits, split);
    const int s1 = sd.lk;
    const int nblk = sb.count;
    const int bstride = sb.stride;
    const int s0 = sb.first;
    const int nb = (hg_ok && nblk > ks) ? (nblk - ks + KS - 1) / KS : 0;
    const size_t kstride = (size_t)a.hkv * RB;
    const uint8_t* kbase = sgpr_base(sd.k + (size_t)kh * RB);
    const uint8_t* vbase = sgpr_base(sd.v + (size_t)kh * RB);

    u32x4 qr[8];
    {
        const uint8_t* qrow = reinterpret_cast<const uint8_t*>(qseq + (size_t)(h0 + col_head<G>(c16)) * kDim);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            qr[2 * t] = ld16_asm(qrow + 4 * (32 * t + 8 * u));
            qr[2 * t + 1] = ld16_asm(qrow + 4 * (32 * t + 8 * u + 4));
        }
    }
    // block i -> slot S: K codes (4 instructions, 8 rows each, swizzled), V codes (4, plain),
    // K scales, V scales (one 4-byte instruction each: lane l -> row l / 2, dword l % 2)
    // Byte offsets of this lane's copies from the block's first row: K code rows 8 r + lane / 8
    // (16-byte chunk lane % 8, swizzled), V code rows likewise (plain), scale row lane / 2. The
    // block's base address is uniform (SGPRs), so a full block issues its copies with no address
    // arithmetic; a block cut by the split's end clamps its rows to the last one.
    const int lr = lane >> 3, lc = lane & 7, sr = lane >> 1;
    uint32_t off_k[4], off_v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int rr = 8 * r + lr;
        off_k[r] = (uint32_t)(rr * kstride) + 16 * (lc ^ ((rr >> 1) & 7));
        off_v[r] = (uint32_t)(rr * kstride) + 16 * (lc ^ q8_vswz(rr));
    }
    const uint32_t off_s = (uint32_t)(sr * kstride) + 128 + 4 * (lane & 1);
    // block starting at key jb (s0 <= jb < s1) -> slot S
    auto issue_at = [&](auto slot_c, int jb) {
        constexpr int S = decltype(slot_c)::value;
        const uint32_t sl = lds_addr(&s_slot[wave][S][0]);
        const uint8_t* kb = sgpr_offset(kbase, (size_t)jb * kstride);
        const uint8_t* vb = sgpr_offset(vbase, (size_t)jb * kstride);
        if (jb + kBlock <= s1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) lds_dma16_s(kb, off_k[r], sl + 1024 * r);
#pragma unroll
            for (int r = 0; r < 4; ++r) lds_dma16_s(vb, off_v[r], sl + kQ8Codes + 1024 * r);
            lds_dma4_s(kb, off_s, sl + 2 * kQ8Codes);
            lds_dma4_s(vb, off_s, sl + 2 * kQ8Codes + 256);
        } else {
            const int last = s1 - 1 - jb;  // rows past it read the last row again
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rr = 8 * r + lr;
                const uint32_t row = (uint32_t)(min(rr, last) * kstride);
                lds_dma16_s(kb, row + 16 * (lc ^ ((rr >> 1) & 7)), sl + 1024 * r);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rr = 8 * r + lr;
                const uint32_t row = (uint32_t)(min(rr, last) * kstride);
                lds_dma16_s(vb, row + 16 * (lc ^ q8_vswz(rr)), sl + kQ8Codes + 1024 * r);
            }
            const uint32_t srow = (uint32_t)(min(sr, last) * kstride) + 128 + 4 * (lane & 1);
            lds_dma4_s(kb, srow, sl + 2 * kQ8Codes);
            lds_dma4_s(vb, srow, sl + 2 * kQ8Codes + 256);
        }
    };
    auto issue = [&](auto slot_c, int i) { issue_at(slot_c, s0 + bstride * (ks + KS * i)); };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // The prologue always issues one block (a wave without blocks copies the split's first one,
    // never read), so one wait with a fixed count follows the Q loads in straight-line code.
    // (A wait chosen by a branch let the compiler copy the Q registers in one arm before the
    // wait, reading them while the loads were in flight.) Block i + 1 is issued once block i
    // has landed (in step i): with one block per wave in flight at the start, the first blocks
    // land earlier and block i's math overlaps block i + 1's copies (18.6 -> 18.3 us per layer
    // at 16K keys).
    issue_at(I0{}, nb > 0 ? s0 + bstride * ks : s0);
    wait_k<10>(qr);

    half8 qb[4];
    {
        const float sc = (colq || col_lo) ? a.scale : 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const f32x4 q0 = __builtin_bit_cast(f32x4, qr[2 * t]);
            const f32x4 q1 = __builtin_bit_cast(f32x4, qr[2 * t + 1]);
            const float x[8] = {as_f32(q0.x * sc), as_f32(q0.y * sc), as_f32(q0.z * sc),
                                as_f32(q0.w * sc), as_f32(q1.x * sc), as_f32(q1.y * sc),
                                as_f32(q1.z * sc), as_f32(q1.w * sc)};  // f32, as reference
            half8 hi, lo;
            split8(x, hi, lo);
            qb[t] = col_lo ? lo : hi;
        }
    }

    float mref = -INFINITY;
    float lsum = 0.0f;
    f32x4 acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int trc = (c16 & 3), trj = (c16 >> 2);
    // V conversion: lane l owns row l / 2, dims 64 (l % 2) .. + 64 (groups 2 (l % 2), + 1)
    const int vr = lane >> 1, vh = lane & 1;

    auto step = [&](auto slot_c, int i) {
        constexpr int S = decltype(slot_c)::value;
        wait_vmcnt<0>();  // block i: the only copies in flight
        if (i + 1 < nb) {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the other slot's reads returned
            asm volatile("" ::: "memory");
            issue(std::integral_constant<int, 1 - S>{}, i + 1);
        }
        if (i == 0) DECODE_STAMP(kStampFirstBlock);
        if (i + 1 == nb) DECODE_STAMP(kStampLastBlock);
        const int jb = s0 + bstride * (ks + KS * i);
        uint8_t* sl = &s_slot[wave][S][0];
        const uint8_t* ksc = sl + 2 * kQ8Codes;
        const uint8_t* vsc = sl + 2 * kQ8Codes + 256;
        // K codes (the MFMA A layout) and the rows' K scales into registers first: the V tile
        // below is written over the block's code area
        u32x2 kc[2][4], ksw[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const int r = 16 * kt + c16;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int L = 2 * t + (u >> 1);
                kc[kt][t] = *reinterpret_cast<const u32x2*>(sl + r * 128 + 16 * (L ^ ((r >> 1) & 7)) + 8 * (u & 1));
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)  // scales of S row 16 kt + 4 u + rr
                ksw[kt][rr] = *reinterpret_cast<const u32x2*>(ksc + (16 * kt + 4 * u + rr) * 8);
        }
        // V codes -> f16 * 2^e tile over the block's code area (the f16 kernel's tr16 layout);
        // the same lane also writes the mantissa factors scale * 2^-e of its row's two groups
        // to the slot's factor table, read back below to fold them into P. Done before S^T: the
        // V^T operand and factor reads then return while S^T and the softmax are computed.
        float* fac = reinterpret_cast<float*>(sl + kQ8Fac);  // [key][group]
        {
            u32x4 vc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                vc[j] = *reinterpret_cast<const u32x4*>(sl + kQ8Codes + vr * 128 +
                                                        16 * ((4 * vh + j) ^ q8_vswz(vr)));
            const uint32_t vs = *reinterpret_cast<const uint32_t*>(vsc + vr * 8 + 4 * vh);
            const uint16_t sc2[2] = {(uint16_t)(vs & 0xffffu), (uint16_t)(vs >> 16)};
            int ex[2];
            float fm[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                ex[q] = q8_exp(sc2[q]);
                fm[q] = __builtin_amdgcn_ldexpf(h2f(sc2[q]), -ex[q]);
            }
            // every LDS read of the code area (K codes and scales above included) has returned
            __builtin_amdgcn_s_waitcnt(0xc07f);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int t = 0; t < 4; ++t) asm volatile("" : "+v"(kc[kt][t]), "+v"(ksw[kt][t]));
            asm volatile("" ::: "memory");
            *reinterpret_cast<f32x2*>(fac + vr * 4 + 2 * vh) = f32x2{fm[0], fm[1]};
            uint16_t* vt = reinterpret_cast<uint16_t*>(sl);
            // per group: the conversion magic's exponent byte and bias for 2^e (codes4_to_f16_exp)
            uint32_t eb[2], bias[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                eb[q] = (uint32_t)(4 * (ex[q] + 25)) * 0x01010101u;
                const uint32_t b16 = (uint32_t)__builtin_bit_cast(
                    uint16_t, (_Float16)__builtin_amdgcn_ldexpf(-1152.0f, ex[q]));
                bias[q] = b16 | (b16 << 16);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t w[4] = {vc[j].x, vc[j].y, vc[j].z, vc[j].w};
                uint32_t hv[8];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    codes4_to_f16_exp(w[e], eb[j >> 1], bias[j >> 1], hv[2 * e], hv[2 * e + 1]);
                // 16 codes = dims 64 vh + 16 j .. + 16: logical chunks 8 vh + 2 j, + 1 of row vr
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int lc2 = 8 * vh + 2 * j + q;
                    *reinterpret_cast<u32x4*>(vt + vr * kDim + 8 * (lc2 ^ (2 * (vr & 3)))) =
                        u32x4{hv[4 * q], hv[4 * q + 1], hv[4 * q + 2], hv[4 * q + 3]};
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // tile and factors written before they are read
            asm volatile("" ::: "memory");
        }
        // the V^T operands and the factors of this lane's keys, read now, used after the softmax
        const uint16_t* vtr = reinterpret_cast<const uint16_t*>(sl);
        half8 va[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const int off = ((((2 * dt + (trc >> 1)) ^ (2 * trj))) << 3) + 4 * (trc & 1);
            const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vtr + (4 * u + trj) * kDim + off));
            const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vtr + (16 + 4 * u + trj) * kDim + off));
            va[dt] = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        }
        f32x4 fk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int key = (j < 4) ? 4 * u + j : 16 + 4 * u + (j - 4);
            fk[j] = *reinterpret_cast<const f32x4*>(fac + key * 4);
        }
        // S^T: per 32-dim group t one MFMA (codes as f16), scaled by the row's group scale
        float x[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x4 part[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t h0l, h0h, h1l, h1h;
                codes4_to_f16(kc[kt][t].x, h0l, h0h);
                codes4_to_f16(kc[kt][t].y, h1l, h1h);
                const u32x4 h = u32x4{h0l, h0h, h1l, h1h};
                part[t] = mfma16(as_half8(h), qb[t], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const u32x2 sw = ksw[kt][rr];
                float v = part[0][rr] * h2f((uint16_t)(sw.x & 0xffffu));
                v = fmaf(part[1][rr], h2f((uint16_t)(sw.x >> 16)), v);
                v = fmaf(part[2][rr], h2f((uint16_t)(sw.y & 0xffffu)), v);
                v = fmaf(part[3][rr], h2f((uint16_t)(sw.y >> 16)), v);
                x[kt][rr] = v;
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) x[kt][r] = (x[kt][r] + partner<G>(x[kt][r])) * kLog2e;
        if (jb + kBlock > s1) {  // the sequence's last block: keys past its end get -inf
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (jb + 16 * kt + 4 * u + r >= s1) x[kt][r] = -INFINITY;
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) bm = fmaxf(bm, x[kt][r]);
        bm = max_rows(bm);
        if (__builtin_amdgcn_ballot_w64(bm > mref + kLazyRescaleQ8) != 0) {
            const float mn = fmaxf(mref, bm);
            const float alpha = __builtin_amdgcn_exp2f(mref - mn);
            mref = mn;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
        }
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(x[j >> 2][j & 3] - mref);
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ps += p[j];
        lsum += ps;
        // P^T per 32-dim group g: p times the mantissa factor of the key's V scale, hi / lo split
        half8 pb[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float fg[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) fg[j] = fk[j][g];
            pb[g] = split8_prod_sel(p, fg, col_lo);
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt] = mfma16(va[dt], pb[dt >> 1], acc[dt]);
    };
    for (int i0 = 0; i0 < nb; i0 += kRing) {
        step(I0{}, i0);
        if (i0 + 1 >= nb) break;
        step(I1{}, i0 + 1);
    }
    wait_vmcnt<0>();  // copies of a wave without blocks land before the LDS is reused below

    // ---- the split's end ---------------------------------------------------------------------
    lsum = sum_rows(lsum);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[dt][r] += partner<G>(acc[dt][r]);
            // every lane adds here (one v_add_f32_dpp), before the hi lanes' LDS stores: left
            // to itself, the compiler moved the adds into their masked region and the exchanges
            // became separate moves with zeroed destinations
            asm volatile("" : "+v"(acc[dt][r]));
        }
    DECODE_STAMP(kStampWaveDone);
    __syncthreads();  // every wave is done with its slots (all copies waited for)
    finish_split<G, W, HPW>(a, sd, si, row, split, reinterpret_cast<float*>(&s_slot[0][0][0]),
                            acc, mref, lsum);
}


// ---- q8_0 caches, GQA group 4: the LDS copies above, cheaper block math -------------------
// decode_q8h_kernel: decode_q8_kernel's workgroup, grid, copies (K and V codes and scales into
// the wave's LDS ring slots, block i + 1 issued once block i has landed) and split merge, with
// block math that needs no V tile rewrite, no factor table and no hi / lo split of P.
// Lane l = (u = l / 16, c = l % 16), c = 4 gq + jh.
//  * S^T = K Q^T on v_mfma_f32_16x16x32_f16, one k-step per 32-dim group t: the A operand is
//    key c of the 16-key tile, dims 32 t + 8 u .. + 7 (codes exact in f16, read from LDS as in
//    decode_q8_kernel); the B operand's 16 columns are the 4 query heads 4 times over (column c:
//    head jh), Q * scale as f16 hi + lo in two chained MFMAs, so every lane ends with the
//    scores of keys 4 u + r (r = 0..3) for its head jh. Each group's partial is scaled by the
//    row's group scale in f32.
//  * O += P V on v_mfma_f32_4x4x1_16b_f32 (16 blocks of 4 x 4, f32): block (u, gq) multiplies
//    A = p(key, head jh) * vscale(key, group gq) (f32, one rounding) by B = the code of dim
//    32 gq + 8 jh + e of the same key (exact f32, one sign-extending byte select), keys 4 u + r;
//    P stays f32. Lane (u, c) reads its 8 codes of the key at byte 8 c of the row in LDS (lanes
//    with u odd take the keys of a step in the order r ^ 1, so the four rows a read instruction
//    touches fall in both halves of the banks). Accumulator e (0..7) holds, in lane (u, c),
//    O[head 0..3][dim 32 gq + 8 jh + e] over the keys 4 u + r; the four u are summed at the
//    wave's end.
constexpr int kQ8hSlot = 2 * kQ8Codes + 2 * kBlock * 8;  // K codes, V codes, K scales, V scales

template <int NS, int HPW, int W>
__global__ void __launch_bounds__(64 * W)
decode_q8h_kernel(DecodeArgs<NS> a) {
    DECODE_STAMP(kStampStart);
    constexpr int G = 4;
    constexpr int RB = kQ8Row;
    constexpr int KS = W / HPW;
    static_assert(W <= kMaxLdsWaves, "waves per workgroup");
    static_assert(finish_floats<G, W>() * 4 <= W * kRing * kQ8hSlot, "merge area in the ring");
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[W][kRing][kQ8hSlot];

    const int rows = (a.ngroups + HPW - 1) / HPW;
    int row, col;
    xcd_grid_pos(rows, row, col);
    const int si = seq_of(a, col);
    const SeqDesc& sd = a.seq[si];
    const int split = col - sd.split0;
    const float* qseq = a.q + (size_t)si * a.hq * kDim;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR math
    const int hl = wave % HPW, ks = wave / HPW;
    const int hg = row * HPW + hl;
    const bool hg_ok = hg < a.ngroups;
    const int h0 = min(hg, a.ngroups - 1) * G;
    const int kh = h0 / a.group;
    const int c = lane & 15;
    const int u = lane >> 4;
    const int gq = c >> 2, jh = c & 3;
    const int uo = u & 1;

    // the split's 32-key blocks interleaved with the other splits', as in decode_f16_kernel
    const SplitBlocks sb = split_blocks(sd.lk, sd.splits, split);
    const int s1 = sd.lk;
    const int nblk = sb.count;
    const int bstride = sb.stride;
    const int s0 = sb.first;
    const int nb = (hg_ok && nblk > ks) ? (nblk - ks + KS - 1) / KS : 0;
    const size_t kstride = (size_t)a.hkv * RB;
    const uint8_t* kbase = sgpr_base(sd.k + (size_t)kh * RB);
    const uint8_t* vbase = sgpr_base(sd.v + (size_t)kh * RB);

    u32x4 qr[8];
    {
        // column c: head h0 + jh; k-step t: dims 32 t + 8 u .. + 7
        const uint8_t* qrow = reinterpret_cast<const uint8_t*>(qseq + (size_t)(h0 + jh) * kDim);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            qr[2 * t] = ld16_asm(qrow + 4 * (32 * t + 8 * u));
            qr[2 * t + 1] = ld16_asm(qrow + 4 * (32 * t + 8 * u + 4));
        }
    }
    // block i -> slot S, as decode_q8_kernel: K codes (4 instructions, 8 rows each, swizzled), V
    // codes (4, swizzled), K scales, V scales (one 4-byte instruction each)
    const int lr = lane >> 3, lc = lane & 7, sr = lane >> 1;
    uint32_t off_k[4], off_v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int rr = 8 * r + lr;
        off_k[r] = (uint32_t)(rr * kstride) + 16 * (lc ^ ((rr >> 1) & 7));
        off_v[r] = (uint32_t)(rr * kstride) + 16 * (lc ^ q8_vswz(rr));
    }
    const uint32_t off_s = (uint32_t)(sr * kstride) + 128 + 4 * (lane & 1);
    auto issue_at = [&](auto slot_c, int jb) {
        constexpr int S = decltype(slot_c)::value;
        const uint32_t sl = lds_addr(&s_slot[wave][S][0]);
        const uint8_t* kb = sgpr_offset(kbase, (size_t)jb * kstride);
        const uint8_t* vb = sgpr_offset(vbase, (size_t)jb * kstride);
        if (jb + kBlock <= s1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) lds_dma16_s(kb, off_k[r], sl + 1024 * r);
#pragma unroll
            for (int r = 0; r < 4; ++r) lds_dma16_s(vb, off_v[r], sl + kQ8Codes + 1024 * r);
            lds_dma4_s(kb, off_s, sl + 2 * kQ8Codes);
            lds_dma4_s(vb, off_s, sl + 2 * kQ8Codes + 256);
        } else {
            const int last = s1 - 1 - jb;  // rows past it read the last row again
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rr = 8 * r + lr;
                const uint32_t rowo = (uint32_t)(min(rr, last) * kstride);
                lds_dma16_s(kb, rowo + 16 * (lc ^ ((rr >> 1) & 7)), sl + 1024 * r);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rr = 8 * r + lr;
                const uint32_t rowo = (uint32_t)(min(rr, last) * kstride);
                lds_dma16_s(vb, rowo + 16 * (lc ^ q8_vswz(rr)), sl + kQ8Codes + 1024 * r);
            }
            const uint32_t srow = (uint32_t)(min(sr, last) * kstride) + 128 + 4 * (lane & 1);
            lds_dma4_s(kb, srow, sl + 2 * kQ8Codes);
            lds_dma4_s(vb, srow, sl + 2 * kQ8Codes + 256);
        }
    };
    auto issue = [&](auto slot_c, int i) { issue_at(slot_c, s0 + bstride * (ks + KS * i)); };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // one block in flight at the start (a wave without blocks copies the split's first one,
    // never read), then one wait with a fixed count for the Q loads, as decode_q8_kernel
    issue_at(I0{}, nb > 0 ? s0 + bstride * ks : s0);
    wait_k<10>(qr);

    half8 qh[4], ql[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const f32x4 q0 = __builtin_bit_cast(f32x4, qr[2 * t]);
        const f32x4 q1 = __builtin_bit_cast(f32x4, qr[2 * t + 1]);
        const float sc = a.scale * kLog2e;  // scores come out in the log2 domain
        const float x[8] = {as_f32(q0.x * sc), as_f32(q0.y * sc), as_f32(q0.z * sc),
                            as_f32(q0.w * sc), as_f32(q1.x * sc), as_f32(q1.y * sc),
                            as_f32(q1.z * sc), as_f32(q1.w * sc)};  // f32: q * (scale log2 e)
        split8(x, qh[t], ql[t]);
    }

    float mref = -INFINITY;
    float lsum = 0.0f;
    f32x4 acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto step = [&](auto slot_c, int i) {
        constexpr int S = decltype(slot_c)::value;
        wait_vmcnt<0>();  // block i: the only copies in flight
        if (i + 1 < nb) {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the other slot's reads returned
            asm volatile("" ::: "memory");
            issue(std::integral_constant<int, 1 - S>{}, i + 1);
        }
        if (i == 0) DECODE_STAMP(kStampFirstBlock);
        if (i + 1 == nb) DECODE_STAMP(kStampLastBlock);
        const int jb = s0 + bstride * (ks + KS * i);
        const uint8_t* sl = &s_slot[wave][S][0];
        const uint8_t* vco = sl + kQ8Codes;
        const uint8_t* ksc = sl + 2 * kQ8Codes;
        const uint8_t* vsc = sl + 2 * kQ8Codes + 256;
        // this lane's V codes and V scales (keys 16 kt + 4 u + (r ^ uo)), read first: they return
        // while S and the softmax are computed
        u32x2 vw[2][4];
        uint16_t vs[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int R = 16 * kt + 4 * u + (r ^ uo);
                vw[kt][r] = *reinterpret_cast<const u32x2*>(vco + R * 128 + 16 * ((c >> 1) ^ q8_vswz(R)) + 8 * (c & 1));
                vs[kt][r] = *reinterpret_cast<const uint16_t*>(vsc + R * 8 + 2 * gq);
            }
        // S^T: per 32-dim group t two chained MFMAs (Q hi, Q lo), scaled by the row's group scale
        float x[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const int r16 = 16 * kt + c;
            f32x4 part[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int L = 2 * t + (u >> 1);
                const u32x2 kc = *reinterpret_cast<const u32x2*>(sl + r16 * 128 + 16 * (L ^ ((r16 >> 1) & 7)) + 8 * (u & 1));
                uint32_t l0, g0, l1, g1;
                codes4_to_f16(kc.x, l0, g0);
                codes4_to_f16(kc.y, l1, g1);
                const half8 kf = as_half8(u32x4{l0, g0, l1, g1});
                part[t] = mfma16(kf, ql[t], mfma16(kf, qh[t], f32x4{0.0f, 0.0f, 0.0f, 0.0f}));
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {  // scales of S row 16 kt + 4 u + r
                const u32x2 sw = *reinterpret_cast<const u32x2*>(ksc + (16 * kt + 4 * u + r) * 8);
                float v = fmaf(part[0][r], h2f((uint16_t)(sw.x & 0xffffu)), 0.0f);  // one mixed FMA
                v = fmaf(part[1][r], h2f((uint16_t)(sw.x >> 16)), v);
                v = fmaf(part[2][r], h2f((uint16_t)(sw.y & 0xffffu)), v);
                v = fmaf(part[3][r], h2f((uint16_t)(sw.y >> 16)), v);
                x[kt][r] = v;
            }
        }
        if (jb + kBlock > s1) {  // the sequence's last block: keys past its end get -inf
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (jb + 16 * kt + 4 * u + r >= s1) x[kt][r] = -INFINITY;
        }
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) bm = fmaxf(bm, x[kt][r]);
        bm = max_rows(bm);
        if (__builtin_amdgcn_ballot_w64(bm > mref + kLazyRescale) != 0) {
            const float mn = fmaxf(mref, bm);
            const float alpha = __builtin_amdgcn_exp2f(mref - mn);  // of head jh
            mref = mn;
            lsum *= alpha;
            // component h of every accumulator belongs to head h (the MFMA block's row), not
            // to the lane's head jh: each gets the factor of lane jh = h of its quad
            const f32x4 ah = f32x4{dpp<0x00>(alpha), dpp<0x55>(alpha), dpp<0xaa>(alpha),
                                   dpp<0xff>(alpha)};
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] *= ah;
        }
        float p[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[kt][r] = __builtin_amdgcn_exp2f(x[kt][r] - mref);
                lsum += p[kt][r];
            }
        // O += P V: the key of step r is 4 u + (r ^ uo), its p picked from the lane's own four
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pk = uo ? p[kt][r ^ 1] : p[kt][r];
                const float av = fmaf(pk, h2f(vs[kt][r]), 0.0f);  // one mixed FMA
                const u32x2 w = vw[kt][r];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[e] = __builtin_amdgcn_mfma_f32_4x4x1f32(
                        av, (float)(int8_t)(w.x >> (8 * e)), acc[e], 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[4 + e] = __builtin_amdgcn_mfma_f32_4x4x1f32(
                        av, (float)(int8_t)(w.y >> (8 * e)), acc[4 + e], 0, 0, 0);
            }
    };
    for (int i0 = 0; i0 < nb; i0 += kRing) {
        step(I0{}, i0);
        if (i0 + 1 >= nb) break;
        step(I1{}, i0 + 1);
    }
    wait_vmcnt<0>();  // copies of a wave without blocks land before the LDS is reused below

    // ---- the split's end: sum the key quarters u, lane (u, c) keeps head u ------------------
    lsum = sum_rows(lsum);
    float o8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        // lanes 0-31 keep heads 0 / 1, lanes 32-63 heads 2 / 3 (each summed over u and u ^ 2) ...
        const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e][0]),
                                                          __float_as_uint(acc[e][2]), false, false);
        const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e][1]),
                                                          __float_as_uint(acc[e][3]), false, false);
        const float r0 = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);
        const float r1 = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);
        // ... then lanes with u even keep r0, odd r1 (summed over u and u ^ 1): head u
        const auto s01 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r0), __float_as_uint(r1),
                                                          false, false);
        o8[e] = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);
    }
    DECODE_STAMP(kStampWaveDone);
    __syncthreads();  // every wave is done with its slots (all copies waited for)
    float* lds = reinterpret_cast<float*>(&s_slot[0][0][0]);
    {
        float* dst = lds + (wave * G + u) * kDim + 32 * gq + 8 * jh;  // m_acc [W][G][128]
        *reinterpret_cast<f32x4*>(dst) = f32x4{o8[0], o8[1], o8[2], o8[3]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o8[4], o8[5], o8[6], o8[7]};
        if (lane < G)  // m_ml [W][G][2]
            *reinterpret_cast<f32x2*>(lds + W * G * kDim + (wave * G + jh) * 2) = f32x2{mref, lsum};
    }
    finish_split_lds<G, W, HPW>(a, sd, si, row, split, lds);
}


template <int KV> struct KernelFor;
template <> struct KernelFor<BRASA_KV_F16> { static constexpr int W = kWavesF16; };
template <> struct KernelFor<BRASA_KV_Q8_0> { static constexpr int W = kWavesQ8; };
template <> struct KernelFor<BRASA_KV_F32> { static constexpr int W = kWavesF32; };

template <int KV, int G, int NS, int HPW>
int launch_hpw(const DecodeArgs<NS>& a, int cols, hipStream_t stream) {
    constexpr int W = KernelFor<KV>::W;
    const int rows = (a.ngroups + HPW - 1) / HPW;
    const dim3 grid(cols * rows), block(64 * W);
    if constexpr (KV == BRASA_KV_F16) {
        hipLaunchKernelGGL((decode_f16_kernel<G, NS, HPW, W>), grid, block, 0, stream, a);
        return check_launch("decode_f16_kernel");
    } else {
        if constexpr (G == 4) {
            hipLaunchKernelGGL((decode_q8h_kernel<NS, HPW, W>), grid, block, 0, stream, a);
            return check_launch("decode_q8h_kernel");
        } else {
            hipLaunchKernelGGL((decode_q8_kernel<G, NS, HPW, W>), grid, block, 0, stream, a);
            return check_launch("decode_q8_kernel");
        }
    }
}

template <int KV, int G, int NS>
int launch(const DecodeArgs<NS>& a, int hpw, int cols, hipStream_t stream) {
    if constexpr (KV == BRASA_KV_F32) {
        constexpr int W = KernelFor<KV>::W;
        hipLaunchKernelGGL((decode_f32_kernel<G, NS, W>), dim3(cols * a.ngroups), dim3(64 * W), 0,
                           stream, a);
        return check_launch("decode_f32_kernel");
    } else {
        if (hpw == 1) return launch_hpw<KV, G, NS, 1>(a, cols, stream);
        if constexpr (2 * G <= kMaxMergeHeads)
            if (hpw == 2) return launch_hpw<KV, G, NS, 2>(a, cols, stream);
        if constexpr (4 * G <= kMaxMergeHeads)
            if (hpw == 4) return launch_hpw<KV, G, NS, 4>(a, cols, stream);
        return set_error(BRASA_ERR_UNSUPPORTED, "decode: %d head groups per workgroup not compiled", hpw);
    }
}

template <int KV, int NS>
int launch_g(const DecodeArgs<NS>& a, int G, int hpw, int cols, hipStream_t stream) {
    switch (G) {
        case 1: return launch<KV, 1, NS>(a, hpw, cols, stream);
        case 2: return launch<KV, 2, NS>(a, hpw, cols, stream);
        case 4: return launch<KV, 4, NS>(a, hpw, cols, stream);
        case 8: return launch<KV, 8, NS>(a, hpw, cols, stream);
    }
    return set_error(BRASA_ERR_UNSUPPORTED, "decode: GQA group %d not compiled", G);
}

template <int NS>
int launch_kv(const DecodeArgs<NS>& a, int kv, int G, int hpw, int cols, hipStream_t stream) {
    switch (kv) {
        case BRASA_KV_F32: return launch_g<BRASA_KV_F32>(a, G, hpw, cols, stream);
        case BRASA_KV_F16: return launch_g<BRASA_KV_F16>(a, G, hpw, cols, stream);
        case BRASA_KV_Q8_0: return launch_g<BRASA_KV_Q8_0>(a, G, hpw, cols, stream);
    }
    return set_error(BRASA_ERR_ARG, "decode: invalid kv type %d", kv);
}

// The first sequence of `a` as single-sequence arguments.
DecodeArgs<1> one_seq(const DecodeArgs<kMaxSeqs>& a) {
    DecodeArgs<1> b;
    b.q = a.q;
    b.part = a.part;
    b.o = a.o;
    b.ctr = a.ctr;
    b.o_f16 = a.o_f16;
    b.hq = a.hq;
    b.hkv = a.hkv;
    b.group = a.group;
    b.ngroups = a.ngroups;
    b.nseq = 1;
    b.scale = a.scale;
    b.seq[0] = a.seq[0];
    return b;
}

// This stream's arrival counters (its slot of g_arrivals; the device address looked up once per
// device), or nullptr when every slot of the device is taken.
unsigned* g_ctr_base[kMaxDevices];
std::once_flag g_ctr_once[kMaxDevices];

int arrival_counters(hipStream_t stream, unsigned** out) {
    int dev = 0, slot = -1;
    const int st = stream_slot(stream, &dev, &slot);
    if (st != BRASA_OK) return st;
    std::call_once(g_ctr_once[dev], [dev] {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_arrivals)) == hipSuccess)
            g_ctr_base[dev] = static_cast<unsigned*>(p);
    });
    if (!g_ctr_base[dev]) return set_error(BRASA_ERR_LAUNCH, "decode: arrival counters not found");
    *out = slot < 0 ? nullptr : g_ctr_base[dev] + (size_t)slot * kSlotCounters;
    return BRASA_OK;
}

}  // namespace

// Split length for `keys` keys spread over about kTargetWgs / ngroups splits: a multiple of 32
// keys and at least 128 keys, so a sequence of lk keys has at most ceil(lk / 128) splits and its
// partials fit the reference's decode_partials_len(hq, lk).
static long long split_chunk(long long keys, int ngroups) {
    const int target = ngroups >= kTargetWgs ? 1 : kTargetWgs / ngroups;
    long long chunk = (keys + target - 1) / target;
    chunk = (chunk + kBlock - 1) / kBlock * kBlock;
    return chunk < kMinChunk ? kMinChunk : chunk;
}

// Launch plan: head groups per workgroup (HPW) and one split length for every sequence of the
// launch. Workgroups that read several adjacent KV heads load the HBM channels evenly (with one
// KV head per workgroup, the heads whose rows sit on the slower channels arrive ~2 us late at
// 16K keys), but each merge group then has HPW * G query heads; the plan takes the largest HPW
// whose merge (query heads x splits of the longest sequence) stays within the bounds above,
// with the split length set for ~kTargetWgs workgroups. f32 caches use one head group per workgroup.
// A function of the lengths and head counts only, so a call's result never depends on anything
// else.
DecodePlan decode_plan(const int* lk, int n, int ngroups, int G, int kv) {
    long long total = 0, lk_max = 0;
    for (int i = 0; i < n; ++i) {
        total += lk[i];
        lk_max = std::max<long long>(lk_max, lk[i]);
    }
    for (int hpw = 4; hpw >= 1; hpw >>= 1) {
        if (hpw > 1 && (kv == BRASA_KV_F32 || hpw * G > kMaxMergeHeads || hpw > ngroups)) continue;
        const int rows = (ngroups + hpw - 1) / hpw;
        const long long chunk = split_chunk(total, rows);
        const long long splits = (lk_max + chunk - 1) / chunk;
        const long long work = splits * hpw * G;
        if (hpw == 1 || work <= kMergeWorkSmall || (chunk >= kLongChunk && work <= kMergeWorkLong))
            return DecodePlan{(int)chunk, (int)splits, hpw};
    }
    return DecodePlan{kMinChunk, 1, 1};  // not reached
}

int decode_batch_launch(const float* q, const void* const* k, const void* const* v,
                        const int* lk, int n, float* partials, void* o, int o_f16, int hq,
                        int hkv, int kv, bool per_head, hipStream_t stream) {
    const int group = hq / hkv;
    const int G = per_head ? 1 : group;
    const int ngroups = per_head ? hq : hkv;
    const size_t oelem = o_f16 ? 2 : 4;
    // sequences per launch: the descriptor array and the counter slot bound it
    const int per_launch = std::min(kMaxSeqs, std::max(1, kSlotCounters / (kCtrStride * ngroups)));
    if (ngroups * kCtrStride > kSlotCounters)
        return set_error(BRASA_ERR_SHAPE, "decode: %d head groups exceed %d", ngroups,
                         kSlotCounters / kCtrStride);
    size_t part_off = 0;
    for (int b0 = 0; b0 < n; b0 += per_launch) {
        const int nb = std::min(per_launch, n - b0);
        DecodeArgs<kMaxSeqs> a;
        memset(&a, 0, sizeof(a));
        a.q = q + (size_t)b0 * hq * kDim;
        a.part = partials;
        a.o = static_cast<uint8_t*>(o) + (size_t)b0 * hq * kDim * oelem;
        a.o_f16 = o_f16;
        a.hq = hq;
        a.hkv = hkv;
        a.group = group;
        a.ngroups = ngroups;
        a.nseq = nb;
        a.scale = 1.0f / sqrtf(static_cast<float>(kDim));
        int st = arrival_counters(stream, &a.ctr);
        if (st != BRASA_OK) return st;
        // one split length for the launch (a sequence's splits never exceed ceil(lk / 128));
        // with no counter slot free (more streams than slots), one split per sequence, which
        // needs no merge
        DecodePlan plan = decode_plan(lk + b0, nb, ngroups, G, kv);
        if (!a.ctr) {
            int lmax = 1;
            for (int i = 0; i < nb; ++i) lmax = std::max(lmax, lk[b0 + i]);
            plan = DecodePlan{(lmax + kBlock - 1) / kBlock * kBlock, 1, plan.hpw};
        }
        const long long chunk = plan.chunk;
        int col = 0;
        for (int i = 0; i < nb; ++i) {
            SeqDesc& d = a.seq[i];
            const DecodePlan p{(int)chunk, (int)((lk[b0 + i] + chunk - 1) / chunk), plan.hpw};
            d.k = static_cast<const uint8_t*>(k[b0 + i]);
            d.v = static_cast<const uint8_t*>(v[b0 + i]);
            d.lk = lk[b0 + i];
            d.chunk = p.chunk;
            d.splits = p.splits;
            d.split0 = col;
            d.part_off = part_off;
            col += d.splits;
            // every plan keeps a sequence's partials inside its share of the scratch
            // (brasa_decode_partials_len of its length)
            if (d.splits > (int)((lk[b0 + i] + kMinChunk - 1) / kMinChunk))
                return set_error(BRASA_ERR_SCRATCH, "decode: %d splits exceed the scratch of %d keys",
                                 d.splits, lk[b0 + i]);
            part_off += (size_t)hq * d.splits * (kDim + 2);
        }
        st = nb == 1 ? launch_kv(one_seq(a), kv, G, plan.hpw, col, stream)
                     : launch_kv(a, kv, G, plan.hpw, col, stream);
        if (st != BRASA_OK) return st;
    }
    return BRASA_OK;
}

// Device address of `scratch`, looked up once per device with that device current.
float* g_scratch_ptr[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

int decode_noalloc_launch(const float* q, const void* k, const void* v, void* o, int o_f16,
                          int hq, int hkv, int lk, int kv, hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(BRASA_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return set_error(BRASA_ERR_LAUNCH, "device %d out of range", dev);
    std::call_once(g_scratch_once[dev], [dev] {
        void* p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (g_scratch_err[dev] == hipSuccess) g_scratch_ptr[dev] = static_cast<float*>(p);
    });
    if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
        return set_error(BRASA_ERR_LAUNCH, "decode_noalloc: hipGetSymbolAddress(scratch): %s",
                         hipGetErrorString(g_scratch_err[dev]));
    const int G = hq / hkv;
    const DecodePlan plan = decode_plan(&lk, 1, hkv, G, kv);
    const size_t need = (size_t)hq * plan.splits * (kDim + 2);
    if (need > (size_t)BRASA_DECODE_NOALLOC_FLOATS)
        return set_error(BRASA_ERR_SCRATCH,
                         "decode_noalloc: needs %zu scratch floats, the fixed array holds %d "
                         "(hq %d, %d keys)", need, BRASA_DECODE_NOALLOC_FLOATS, hq, lk);
    return decode_batch_launch(q, &k, &v, &lk, 1, g_scratch_ptr[dev], o, o_f16, hq, hkv, kv, false,
                               stream);
}

int decode_launch(const float* q, const void* k, const void* v, float* partials, void* o,
                  int o_f16, int hq, int hkv, int lk, int kv, bool per_head,
                  hipStream_t stream) {
    return decode_batch_launch(q, &k, &v, &lk, 1, partials, o, o_f16, hq, hkv, kv, per_head,
                               stream);
}

}  // namespace brasa

#ifdef BRASA_DECODE_TRACE
// Copies min(n, kTraceWgs * 16) stamps of the timeline build to host memory `dst`.
extern "C" int brasa_decode_trace_read(unsigned long long* dst, size_t n) {
    using namespace brasa;
    const size_t cnt = std::min(n, (size_t)kTraceWgs * kTraceStamps);
    const hipError_t e = hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_trace), cnt * sizeof(*dst));
    return e == hipSuccess ? 0 : BRASA_ERR_LAUNCH;
}
#endif

extern "C" int brasa_test_decode_plan(const int* lk, int n, int hq, int hkv, int kv, int* chunk,
                                      int* hpw, int* splits) {
    if (!lk || n <= 0 || n > 64 || hkv <= 0 || hq % hkv != 0 || !chunk || !hpw || !splits)
        return brasa::set_error(BRASA_ERR_ARG, "test_decode_plan: bad arguments");
    const brasa::DecodePlan p = brasa::decode_plan(lk, n, hkv, hq / hkv, kv);
    *chunk = p.chunk;
    *hpw = p.hpw;
    for (int i = 0; i < n; ++i) splits[i] = (lk[i] + p.chunk - 1) / p.chunk;
    return BRASA_OK;
}

extern "C" int brasa_test_split_blocks(int lk, int splits, int split, int* first, int* stride,
                                       int* count) {
    if (lk <= 0 || splits <= 0 || split < 0 || split >= splits || !first || !stride || !count)
        return brasa::set_error(BRASA_ERR_ARG, "test_split_blocks: bad arguments");
    const brasa::SplitBlocks b = brasa::split_blocks(lk, splits, split);
    *first = b.first;
    *stride = b.stride;
    *count = b.count;
    return BRASA_OK;
}
