// Read-only probes of the decode access pattern (measurement tool, not part of the library).
//
// The fp16 decode at 16384 keys reads 2 x 16384 x 8 x 256 bytes (67.1 MB) per layer. These
// kernels read exactly those bytes and do no math, so their time is what the memory system
// gives each access pattern; 36 layer caches are rotated (2.4 GB, past the 256 MB MALL), 36
// back-to-back launches are timed with HIP events, the median of 7 runs is printed per layer.
//   * one / two / four KV heads per workgroup: 256 workgroups of 8 wave64, every wave reads two
//     32-key blocks of K (16-byte loads into registers) and V (16-byte copies into LDS), the
//     decode kernel's instructions, for 1, 2 or 4 adjacent KV heads per workgroup;
//   * contiguous: the same instructions over whole 2 KB key rows (64 keys x 8 heads per workgroup);
//   * stream: a grid-stride read of both caches, 16 bytes per lane, the plain streaming ceiling;
//   * q8_0 (136-byte rows, 35.7 MB per layer at 16384 keys): 256 workgroups of 8 waves, each
//     reading the row slices of 1, 2, 4 or 8 adjacent KV heads (HPW x 136 contiguous bytes per
//     position) of its key range, 8 bytes per lane, every load of a wave issued before it waits;
//     with and without the nontemporal hint.
// Build: make -C brasa_amd/csrc read_probe; run: _build/read_probe (one GPU).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#include "common.hpp"

using namespace brasa;

namespace {

constexpr int kKeys = 16384, kHeads = 8, kRow = 256, kLayers = 36;
constexpr size_t kCache = (size_t)kKeys * kHeads * kRow;

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
    u32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(r) : "v"(p) : "memory");
    return r;
}

// HPW heads per workgroup (1, 2, 4), or 8 for whole contiguous key rows; W waves per workgroup
// and 2048 / W workgroups (every wave reads 64 keys of one head). With W = 16 the two blocks of a
// wave share one LDS slot (160 KB would not hold 16 x 2 x 8 KB): a timing probe only.
template <int HPW, int W = 8, bool XMIX = false, int KIL = 0, bool VREG = false>
__global__ void __launch_bounds__(64 * W) pattern_kernel(const uint8_t* K, const uint8_t* V, unsigned* out) {
    constexpr int kBlocks = W == 8 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t s_v[W][kBlocks][4096];
    const int b = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c16 = lane & 15, u = lane >> 4;
    u32x4 kx[2][8], vx[2][8];
    for (int blk = 0; blk < 2; ++blk) {
        const uint8_t *kr[2], *vr[8];
        if constexpr (HPW == 8) {
            // 4 whole key rows (8 KB) per wave and block: keys 64 b + 4 (2 w + blk) ..
            const size_t base = ((size_t)64 * b + 4 * (2 * w + blk)) * kHeads * kRow;
            for (int kt = 0; kt < 2; ++kt) kr[kt] = K + base + (size_t)(16 * kt + c16) * kRow + 16 * u;
            for (int r = 0; r < 8; ++r) vr[r] = V + base + (size_t)(4 * r + u) * kRow + 16 * c16;
        } else {
            constexpr int rows = 8 / HPW, chunk = kKeys / (2048 / W / rows), per_head = W / HPW;
            // XMIX: workgroups b, b + 8, ... (one XCD) take every row of a split in turn, so each
            // XCD reads whole key rows of its splits; otherwise rows vary fastest (XCD = row)
            const int j = b >> 3;
            const int row = XMIX ? j % rows : b % rows;
            const int split = XMIX ? (j / rows) * 8 + (b & 7) : b / rows;
            const int head = row * HPW + w % HPW;
            // KIL: a split's 32-key blocks interleaved with the other splits' (block i of split s
            // is global block s + splits * i), so the workgroups read one region at a time
            constexpr int splits = 2048 / W / rows;
            const int bi = w / HPW + per_head * blk;
            // KIL = units of KIL blocks
            const int key0 = KIL ? 32 * (KIL * (split + splits * (bi / KIL)) + bi % KIL) : chunk * split + 32 * bi;
            for (int kt = 0; kt < 2; ++kt)
                kr[kt] = K + ((size_t)(key0 + 16 * kt + c16) * kHeads + head) * kRow + 16 * u;
            for (int r = 0; r < 8; ++r)
                vr[r] = V + ((size_t)(key0 + 4 * r + u) * kHeads + head) * kRow + 16 * c16;
        }
        for (int kt = 0; kt < 2; ++kt)
            for (int t = 0; t < 4; ++t) kx[blk][4 * kt + t] = load16(kr[kt] + 64 * t);
        if constexpr (VREG) {
            // VREG: the V rows into registers too (plain 16-byte loads), no LDS copy
            for (int r = 0; r < 8; ++r) vx[blk][r] = load16(vr[r]);
        } else {
            for (int r = 0; r < 8; ++r) lds_dma16_nt(vr[r], &s_v[w][blk % kBlocks][0] + 512 * r);
        }
    }
    // every load has landed before a loaded register is read
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(kx[0][0]), "+v"(kx[0][1]), "+v"(kx[0][2]), "+v"(kx[0][3]), "+v"(kx[0][4]),
                   "+v"(kx[0][5]), "+v"(kx[0][6]), "+v"(kx[0][7]), "+v"(kx[1][0]), "+v"(kx[1][1]),
                   "+v"(kx[1][2]), "+v"(kx[1][3]), "+v"(kx[1][4]), "+v"(kx[1][5]), "+v"(kx[1][6]),
                   "+v"(kx[1][7])
                 :
                 : "memory");
    if constexpr (VREG)  // names the V registers too: no use of them above the wait
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+v"(vx[0][0]), "+v"(vx[0][1]), "+v"(vx[0][2]), "+v"(vx[0][3]), "+v"(vx[0][4]),
                       "+v"(vx[0][5]), "+v"(vx[0][6]), "+v"(vx[0][7]), "+v"(vx[1][0]), "+v"(vx[1][1]),
                       "+v"(vx[1][2]), "+v"(vx[1][3]), "+v"(vx[1][4]), "+v"(vx[1][5]), "+v"(vx[1][6]),
                       "+v"(vx[1][7])
                     :
                     : "memory");
    __syncthreads();
    unsigned x = s_v[w][0][lane] ^ s_v[w][kBlocks - 1][lane];
    for (int j = 0; j < 8; ++j) x ^= kx[0][j].x ^ kx[1][j].y;
    if constexpr (VREG)
        for (int j = 0; j < 8; ++j) x ^= vx[0][j].z ^ vx[1][j].w;
    if (lane == 0) out[b * W + w] = x;
}

__global__ void __launch_bounds__(256) stream_kernel(const uint8_t* K, const uint8_t* V, unsigned* out, int nwg) {
    unsigned acc = 0;
    const size_t n16 = kCache / 16, stride = (size_t)nwg * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) {
        u32x4 x = load16(K + 16 * i), y = load16(V + 16 * i);
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(x), "+v"(y) : : "memory");
        acc ^= x.x ^ y.z;
    }
    if (acc == 0x9e3779b9u) out[0] = acc;  // keeps the loads
}

// ---- q8_0 ------------------------------------------------------------------------------------
constexpr size_t kQ8Cache = (size_t)kKeys * kHeads * kQ8Row;

template <int HPW, bool NT, int W = 8, bool KIL = false, bool XCD = false>
__global__ void __launch_bounds__(64 * W) q8_pattern_kernel(const uint8_t* K, const uint8_t* V, unsigned* out) {
    constexpr int rows = 8 / HPW, splits = 2048 / W / rows, keys = kKeys / splits;
    constexpr int seg = HPW * kQ8Row;           // bytes per position
    constexpr int per_wave = keys * seg / W;    // bytes per wave and cache
    constexpr int n = per_wave / 512;           // 8-byte loads per lane and cache
    static_assert(per_wave % 512 == 0, "whole wave loads");
    const int b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // XCD: the decode kernel's grid order (xcd_grid_pos: workgroups b, b + 8, ... on one XCD take
    // the rows of a split in turn, so the heads of a split share their lines in one L2)
    const int j = b >> 3;
    const int row = XCD ? j % rows : b % rows;
    const int split = XCD ? (j / rows) * 8 + (b & 7) : b / rows;
    const int key0 = split * keys;
    u32x2 xk[n], xv[n];
#pragma unroll
    for (int i = 0; i < n; ++i) {
        const int byte = w * per_wave + i * 512 + lane * 8;
        const int k = byte / seg;  // key within the split; KIL: 32-key blocks interleaved over the splits
        const int key = KIL ? 32 * (split + splits * (k / 32)) + k % 32 : key0 + k;
        const size_t a = ((size_t)key * kHeads + row * HPW) * kQ8Row + byte % seg;
        if constexpr (NT) {
            xk[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(K + a));
            xv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(V + a));
        } else {
            xk[i] = *reinterpret_cast<const u32x2*>(K + a);
            xv[i] = *reinterpret_cast<const u32x2*>(V + a);
        }
    }
    u32x2 acc = {0, 0};
#pragma unroll
    for (int i = 0; i < n; ++i) acc ^= xk[i] ^ xv[i];
    if (acc.x == 0x9e3779b9u) out[b] = acc.y;  // keeps the loads
}

// The q8_0 decode kernel's own copies: per wave two 32-key blocks of one KV head, each 4 + 4
// LDS-DMA copies of 16-byte code chunks and 2 of 4-byte scale pairs into the wave's LDS slots;
// the decode kernel's grid order and interleaved blocks. BOTH: the two blocks issued at once;
// otherwise block 1 only after block 0 has landed (the kernel's issue order), no math between.
template <bool BOTH>
__global__ void __launch_bounds__(512) q8_lds_kernel(const uint8_t* K, const uint8_t* V, unsigned* out) {
    __shared__ __attribute__((aligned(16))) uint8_t s_q8[8][2][8704];
    const int b = blockIdx.x, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR copy bases
    const int j = b >> 3, row = j % 8, split = (j / 8) * 8 + (b & 7);
    constexpr uint32_t kstride = kHeads * kQ8Row;
    const uint8_t* kb0 = sgpr_base(K + row * kQ8Row);
    const uint8_t* vb0 = sgpr_base(V + row * kQ8Row);
    const int lr = lane >> 3, lc = lane & 7, sr = lane >> 1;
    uint32_t off[4];
    for (int r = 0; r < 4; ++r) off[r] = (uint32_t)((8 * r + lr) * kstride) + 16 * lc;
    const uint32_t off_s = (uint32_t)(sr * kstride) + 128 + 4 * (lane & 1);
    for (int blk = 0; blk < 2; ++blk) {
        const int jb = 32 * (split + 32 * (w + 8 * blk));
        const uint8_t* kb = sgpr_offset(kb0, (uint64_t)jb * kstride);
        const uint8_t* vb = sgpr_offset(vb0, (uint64_t)jb * kstride);
        const uint32_t sl = lds_addr(&s_q8[w][blk][0]);
        for (int r = 0; r < 4; ++r) lds_dma16_s(kb, off[r], sl + 1024 * r);
        for (int r = 0; r < 4; ++r) lds_dma16_s(vb, off[r], sl + 4096 + 1024 * r);
        lds_dma4_s(kb, off_s, sl + 8192);
        lds_dma4_s(vb, off_s, sl + 8448);
        if (!BOTH && blk == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const unsigned x = s_q8[w][0][4 * lane] ^ s_q8[w][1][4 * lane + 1];
    if (x == 0x9e3779b9u) out[b] = x;
}

template <class F>
float time_layers(F launch) {
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    std::vector<float> t;
    for (int rep = 0; rep < 7; ++rep) {
        (void)hipEventRecord(e0);
        for (int l = 0; l < kLayers; ++l) launch(l);
        (void)hipEventRecord(e1);
        (void)hipEventSynchronize(e1);
        float ms = 0;
        (void)hipEventElapsedTime(&ms, e0, e1);
        t.push_back(ms * 1000.0f / kLayers);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
}

}  // namespace

int main() {
    std::vector<uint8_t*> ks(kLayers), vs(kLayers);
    for (int l = 0; l < kLayers; ++l) {
        if (hipMalloc(&ks[l], kCache) != hipSuccess || hipMalloc(&vs[l], kCache) != hipSuccess) {
            fprintf(stderr, "hipMalloc failed\n");
            return 1;
        }
        (void)hipMemset(ks[l], 1, kCache);
        (void)hipMemset(vs[l], 2, kCache);
    }
    unsigned* out = nullptr;
    if (hipMalloc(&out, 256 * 8 * sizeof(unsigned)) != hipSuccess) return 1;
    (void)hipDeviceSynchronize();
    const double mb = 2.0 * kCache / 1e6;
    auto line = [&](const char* name, float us) {
        printf("| %s | %.2f | %.2f |\n", name, us, mb / us);  // MB per us = TB/s
    };
    printf("| pattern (%.1f MB per layer) | us per layer | TB/s |\n|---|---|---|\n", mb);
    for (int pass = 0; pass < 2; ++pass) {
        line("1 KV head per workgroup (the decode plan at 16K)",
             time_layers([&](int l) { pattern_kernel<1><<<256, 512>>>(ks[l], vs[l], out); }));
        line("1 KV head per workgroup, 32-key blocks interleaved over the splits",
             time_layers([&](int l) { pattern_kernel<1, 8, false, 1><<<256, 512>>>(ks[l], vs[l], out); }));
        line("1 KV head per workgroup, interleaved 32-key blocks, V into registers (no LDS copy)",
             time_layers([&](int l) { pattern_kernel<1, 8, false, 1, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line("1 KV head per workgroup, 64-key units interleaved over the splits",
             time_layers([&](int l) { pattern_kernel<1, 8, false, 2><<<256, 512>>>(ks[l], vs[l], out); }));
        line("1 KV head per workgroup, 128-key units interleaved over the splits",
             time_layers([&](int l) { pattern_kernel<1, 8, false, 4><<<256, 512>>>(ks[l], vs[l], out); }));
        line("2 KV heads per workgroup, 32-key blocks interleaved over the splits",
             time_layers([&](int l) { pattern_kernel<2, 8, false, 1><<<256, 512>>>(ks[l], vs[l], out); }));
        line("1 KV head per workgroup, the heads of a split on one XCD",
             time_layers([&](int l) { pattern_kernel<1, 8, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line("2 KV heads per workgroup, the heads of a split on one XCD",
             time_layers([&](int l) { pattern_kernel<2, 8, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line("2 KV heads per workgroup",
             time_layers([&](int l) { pattern_kernel<2><<<256, 512>>>(ks[l], vs[l], out); }));
        line("4 KV heads per workgroup",
             time_layers([&](int l) { pattern_kernel<4><<<256, 512>>>(ks[l], vs[l], out); }));
        line("whole 2 KB key rows",
             time_layers([&](int l) { pattern_kernel<8><<<256, 512>>>(ks[l], vs[l], out); }));
        line("1 KV head per workgroup, 128 workgroups of 16 waves",
             time_layers([&](int l) { pattern_kernel<1, 16><<<128, 1024>>>(ks[l], vs[l], out); }));
        line("2 KV heads per workgroup, 128 workgroups of 16 waves",
             time_layers([&](int l) { pattern_kernel<2, 16><<<128, 1024>>>(ks[l], vs[l], out); }));
        for (int nwg : {512, 1024, 4096}) {
            char name[64];
            snprintf(name, sizeof name, "stream, %d workgroups of 256", nwg);
            line(name, time_layers([&](int l) { stream_kernel<<<nwg, 256>>>(ks[l], vs[l], out, nwg); }));
        }
    }
    // q8_0 caches (the f16 buffers are larger than a q8_0 layer: reused)
    const double mb8 = 2.0 * kQ8Cache / 1e6;
    auto line8 = [&](const char* name, float us) { printf("| %s | %.2f | %.2f |\n", name, us, mb8 / us); };
    printf("\n| q8_0 pattern (%.1f MB per layer) | us per layer | TB/s |\n|---|---|---|\n", mb8);
    for (int pass = 0; pass < 2; ++pass) {
        line8("1 KV head per workgroup (the decode plan at 16K), nontemporal",
              time_layers([&](int l) { q8_pattern_kernel<1, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, plain",
              time_layers([&](int l) { q8_pattern_kernel<1, false><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, plain, 32-key blocks interleaved over the splits",
              time_layers([&](int l) { q8_pattern_kernel<1, false, 8, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, plain, the decode kernel's XCD order",
              time_layers([&](int l) { q8_pattern_kernel<1, false, 8, false, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, plain, XCD order, 32-key blocks interleaved over the splits",
              time_layers([&](int l) { q8_pattern_kernel<1, false, 8, true, true><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, the q8_0 kernel's LDS copies, both blocks at once",
              time_layers([&](int l) { q8_lds_kernel<true><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, the q8_0 kernel's LDS copies, block 1 after block 0 landed",
              time_layers([&](int l) { q8_lds_kernel<false><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("2 KV heads per workgroup, plain",
              time_layers([&](int l) { q8_pattern_kernel<2, false><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("4 KV heads per workgroup, plain",
              time_layers([&](int l) { q8_pattern_kernel<4, false><<<256, 512>>>(ks[l], vs[l], out); }));
        line8("1 KV head per workgroup, 128 workgroups of 16 waves, plain",
              time_layers([&](int l) { q8_pattern_kernel<1, false, 16><<<128, 1024>>>(ks[l], vs[l], out); }));
        line8("2 KV heads per workgroup, 128 workgroups of 16 waves, plain",
              time_layers([&](int l) { q8_pattern_kernel<2, false, 16><<<128, 1024>>>(ks[l], vs[l], out); }));
        line8("whole 1088-byte key rows, plain",
              time_layers([&](int l) { q8_pattern_kernel<8, false><<<256, 512>>>(ks[l], vs[l], out); }));
    }
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        fprintf(stderr, "%s\n", hipGetErrorString(e));
        return 1;
    }
    return 0;
}
