// C ABI of libbrasa_attn.so: argument validation mirroring the reference's asserts, the error
// plumbing, and the device plumbing of brasa_hip_rt.h. Kernels live in kv.hip, decode.hip and
// prefill.hip.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/brasa_hip_rt.h"
#include "common.hpp"

namespace brasa {

int store_kv_launch(int kv, const float* src, void* dst, size_t n, hipStream_t stream);
int dequant_q8_launch(const void* src, float* dst, size_t rows, hipStream_t stream);
int fill_u8_launch(void* dst, uint8_t value, size_t bytes, hipStream_t stream);
int fill_normal_launch(float* out, size_t n, uint64_t seed, float scale, hipStream_t stream);
int decode_launch(const float* q, const void* k, const void* v, float* partials, void* o,
                  int o_f16, int hq, int hkv, int lk, int kv, bool per_head, hipStream_t stream);
int decode_noalloc_launch(const float* q, const void* k, const void* v, void* o, int o_f16,
                          int hq, int hkv, int lk, int kv, hipStream_t stream);
int rms_norm_launch(const float* x, const float* w, float* out, size_t rows, size_t n, float eps,
                    hipStream_t stream);
int rope_neox_launch(float* x, const float* cos_t, const float* sin_t, size_t tokens,
                     size_t heads, size_t dim, size_t pos0, hipStream_t stream);
int qk_norm_rope_store_launch(int kv, float* q, float* k, const float* v, const float* qn,
                              const float* kn, float eps, const float* cos_t, const float* sin_t,
                              void* kdst, void* vdst, size_t tokens, size_t hq, size_t hkv,
                              size_t pos0, hipStream_t stream);
void rope_table_host(double theta, size_t dim, size_t max_pos, float* cos_out, float* sin_out);
int decode_batch_launch(const float* q, const void* const* k, const void* const* v,
                        const int* lk, int n, float* partials, void* o, int o_f16, int hq,
                        int hkv, int kv, bool per_head, hipStream_t stream);
int prefill_launch(const float* q, const void* k, const void* v, void* o, int tokens, int hq,
                   int hkv, int pos0, int kv, int precision, bool caller_ws, void* ws,
                   size_t ws_len, hipStream_t stream, const int* layout = nullptr);
size_t prefill_workspace_len(int tokens, int hq, int hkv, int pos0, int kv, int precision);
void prefill_release_workspaces();

namespace {
thread_local char g_err[512] = "";
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(BRASA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return BRASA_OK;
}

static int hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) return set_error(BRASA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return BRASA_OK;
}

static inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

static bool valid_kv(int kv) {
    return kv == BRASA_KV_F32 || kv == BRASA_KV_F16 || kv == BRASA_KV_Q8_0;
}

// Largest sizes the kernels index with 32-bit integers.
static constexpr size_t kMaxPositions = (size_t)1 << 30;
static constexpr size_t kMaxHeads = 1024;

}  // namespace brasa

using namespace brasa;

extern "C" {

size_t brasa_decode_partials_len(size_t hq, size_t lk) {
    return hq * ((lk + BRASA_DECODE_CHUNK - 1) / BRASA_DECODE_CHUNK) * 130;
}

size_t brasa_kv_capacity(size_t ctx) {
    return (ctx + BRASA_KV_ALIGN - 1) / BRASA_KV_ALIGN * BRASA_KV_ALIGN;
}

size_t brasa_kv_cache_len(size_t layers, size_t ctx, size_t hkv, size_t dim) {
    return layers * brasa_kv_capacity(ctx) * hkv * dim;
}

size_t brasa_kv_offset(size_t layer, size_t ctx, size_t hkv, size_t dim, size_t pos) {
    return (layer * brasa_kv_capacity(ctx) + pos) * hkv * dim;
}

int brasa_gqa_supported(size_t hq, size_t hkv) {
    if (hkv == 0 || hq % hkv != 0) return 0;
    const size_t g = hq / hkv;
    return g == 1 || g == 2 || g == 4 || g == 8;
}

size_t brasa_kv_bytes(int kv, size_t n) {
    switch (kv) {
        case BRASA_KV_F32: return n * 4;
        case BRASA_KV_F16: return n * 2;
        case BRASA_KV_Q8_0:
            if (n % kDim != 0) {
                set_error(BRASA_ERR_SHAPE, "KV Q8: rows of %d values (n = %zu)", kDim, n);
                return 0;
            }
            return n / kDim * kQ8Row;
    }
    set_error(BRASA_ERR_ARG, "invalid kv type %d", kv);
    return 0;
}

int brasa_store_kv(int kv, const float* src, void* dst, size_t n, void* stream) {
    g_err[0] = 0;
    if (!valid_kv(kv)) return set_error(BRASA_ERR_ARG, "store_kv: invalid kv type %d", kv);
    if (n == 0) return BRASA_OK;
    if (!src || !dst) return set_error(BRASA_ERR_ARG, "store_kv: null pointer");
    if (kv == BRASA_KV_Q8_0 && n % kDim != 0)  // lib.rs:1039
        return set_error(BRASA_ERR_SHAPE, "KV Q8: rows of %d values (n = %zu)", kDim, n);
    return store_kv_launch(kv, src, dst, n, as_stream(stream));
}

int brasa_dequantize_kv_q8(const void* src, float* dst, size_t rows, void* stream) {
    g_err[0] = 0;
    if (rows == 0) return BRASA_OK;
    if (!src || !dst) return set_error(BRASA_ERR_ARG, "dequantize_kv_q8: null pointer");
    return dequant_q8_launch(src, dst, rows, as_stream(stream));
}

// Shape checks of the decode entry points (lib.rs:1074-1080 / 1128-1135). partials == nullptr
// with noalloc: the library's fixed scratch array is used instead of the caller's.
static int decode_common(const float* q, const void* k, const void* v, float* partials,
                         size_t partials_len, void* o, int o_dtype, brasa_attn_shape s,
                         void* stream, bool per_head, bool noalloc = false) {
    g_err[0] = 0;
    if (!valid_kv(s.kv)) return set_error(BRASA_ERR_ARG, "decode: invalid kv type %d", s.kv);
    if (o_dtype != BRASA_OUT_F32 && o_dtype != BRASA_OUT_F16)
        return set_error(BRASA_ERR_ARG, "decode: invalid output dtype %d", o_dtype);
    // lib.rs:1074-1080 / 1128-1135
    if (s.tokens != 1) return set_error(BRASA_ERR_SHAPE, "decode_attention is for one token");
    if (s.dim != (size_t)kDim)
        return set_error(BRASA_ERR_SHAPE, "decode_attention requires head_dim 128");
    if (s.hkv == 0 || s.hq % s.hkv != 0)
        return set_error(BRASA_ERR_SHAPE, "hq must be a multiple of hkv");
    if (s.hq > kMaxHeads || s.pos0 + 1 > kMaxPositions)
        return set_error(BRASA_ERR_SHAPE, "decode: shape too large");
    const size_t lk = s.pos0 + 1;
    if (!noalloc && partials_len < brasa_decode_partials_len(s.hq, lk))
        return set_error(BRASA_ERR_SCRATCH, "decode scratch too small (%zu < %zu floats)",
                         partials_len, brasa_decode_partials_len(s.hq, lk));
    if (!per_head && !brasa_gqa_supported(s.hq, s.hkv))
        return set_error(BRASA_ERR_UNSUPPORTED,
                         "decode_attention_lanes: GQA group %zu not compiled", s.hq / s.hkv);
    if (!q || !k || !v || (!partials && !noalloc) || !o)
        return set_error(BRASA_ERR_ARG, "decode: null pointer");
    if (noalloc)
        return decode_noalloc_launch(q, k, v, o, o_dtype == BRASA_OUT_F16, (int)s.hq, (int)s.hkv,
                                     (int)lk, s.kv, as_stream(stream));
    return decode_launch(q, k, v, partials, o, o_dtype == BRASA_OUT_F16, (int)s.hq, (int)s.hkv,
                         (int)lk, s.kv, per_head, as_stream(stream));
}

int brasa_decode_attention_lanes(const float* q, const void* k, const void* v, float* partials,
                                 size_t partials_len, void* o, int o_dtype,
                                 brasa_attn_shape shape, void* stream) {
    return decode_common(q, k, v, partials, partials_len, o, o_dtype, shape, stream, false);
}

int brasa_decode_attention_lanes_noalloc(const float* q, const void* k, const void* v, void* o,
                                         int o_dtype, brasa_attn_shape shape, void* stream) {
    return decode_common(q, k, v, nullptr, 0, o, o_dtype, shape, stream, false, true);
}

int brasa_decode_attention(const float* q, const void* k, const void* v, float* partials,
                           size_t partials_len, void* o, int o_dtype, brasa_attn_shape shape,
                           void* stream) {
    return decode_common(q, k, v, partials, partials_len, o, o_dtype, shape, stream, true);
}

size_t brasa_decode_batch_partials_len(size_t hq, const size_t* lk, size_t n) {
    size_t f = 0;
    for (size_t i = 0; i < n; ++i) f += brasa_decode_partials_len(hq, lk[i]);
    return f;
}

int brasa_decode_attention_batch(const float* q, const void* const* k, const void* const* v,
                                 const size_t* lk, size_t n, float* partials,
                                 size_t partials_len, void* o, int o_dtype, size_t hq,
                                 size_t hkv, size_t dim, int kv, void* stream) {
    g_err[0] = 0;
    if (!valid_kv(kv)) return set_error(BRASA_ERR_ARG, "decode batch: invalid kv type %d", kv);
    if (o_dtype != BRASA_OUT_F32 && o_dtype != BRASA_OUT_F16)
        return set_error(BRASA_ERR_ARG, "decode batch: invalid output dtype %d", o_dtype);
    if (dim != (size_t)kDim)
        return set_error(BRASA_ERR_SHAPE, "decode_attention requires head_dim 128");
    if (hkv == 0 || hq % hkv != 0) return set_error(BRASA_ERR_SHAPE, "hq must be a multiple of hkv");
    if (!brasa_gqa_supported(hq, hkv))
        return set_error(BRASA_ERR_UNSUPPORTED, "decode batch: GQA group %zu not compiled", hq / hkv);
    if (hq > kMaxHeads || n > ((size_t)1 << 20))
        return set_error(BRASA_ERR_SHAPE, "decode batch: shape too large");
    if (n == 0) return BRASA_OK;
    if (!lk || !k || !v) return set_error(BRASA_ERR_ARG, "decode batch: null array");
    std::vector<int> lki(n);
    for (size_t i = 0; i < n; ++i) {
        if (lk[i] == 0) return set_error(BRASA_ERR_SHAPE, "decode batch: sequence %zu has no keys", i);
        if (lk[i] > kMaxPositions) return set_error(BRASA_ERR_SHAPE, "decode batch: shape too large");
        if (!k[i] || !v[i]) return set_error(BRASA_ERR_ARG, "decode batch: null cache pointer %zu", i);
        lki[i] = (int)lk[i];
    }
    const size_t need = brasa_decode_batch_partials_len(hq, lk, n);
    if (partials_len < need)
        return set_error(BRASA_ERR_SCRATCH, "decode scratch too small (%zu < %zu floats)",
                         partials_len, need);
    if (!q || !partials || !o) return set_error(BRASA_ERR_ARG, "decode batch: null pointer");
    return decode_batch_launch(q, k, v, lki.data(), (int)n, partials, o, o_dtype == BRASA_OUT_F16,
                               (int)hq, (int)hkv, kv, false, as_stream(stream));
}

// Shape checks of the prefill entry points (lib.rs:1203-1204, 1227-1231).
static int prefill_check(brasa_attn_shape s, int precision) {
    if (!valid_kv(s.kv)) return set_error(BRASA_ERR_ARG, "flash_attention: invalid kv %d", s.kv);
    if (precision != BRASA_PREFILL_F16 && precision != BRASA_PREFILL_F32 &&
        precision != BRASA_PREFILL_F16_PF32)
        return set_error(BRASA_ERR_ARG, "flash_attention: invalid precision %d", precision);
    // lib.rs:1203-1204
    if (s.dim != (size_t)kDim)
        return set_error(BRASA_ERR_SHAPE, "flash_attention requires head_dim 128");
    if (s.hkv == 0 || s.hq % s.hkv != 0)
        return set_error(BRASA_ERR_SHAPE, "hq must be a multiple of hkv");
    if (s.hq > kMaxHeads || s.pos0 + s.tokens + BRASA_KV_ALIGN > kMaxPositions)
        return set_error(BRASA_ERR_SHAPE, "flash_attention: shape too large");
    // lib.rs:1227-1231: outside the compiled GQA groups only the f32 kernel exists
    if (!brasa_gqa_supported(s.hq, s.hkv) && precision != BRASA_PREFILL_F32)
        return set_error(BRASA_ERR_UNSUPPORTED,
                         "flash_attention: without a compiled GQA group (%zu) attention is f32 only",
                         s.hq / s.hkv);
    return BRASA_OK;
}

int brasa_flash_attention_with(const float* q, const void* k, const void* v, void* o,
                               brasa_attn_shape s, int precision, void* stream) {
    g_err[0] = 0;
    const int st = prefill_check(s, precision);
    if (st != BRASA_OK) return st;
    if (s.tokens == 0) return BRASA_OK;
    if (!q || !k || !v || !o) return set_error(BRASA_ERR_ARG, "flash_attention: null pointer");
    return prefill_launch(q, k, v, o, (int)s.tokens, (int)s.hq, (int)s.hkv, (int)s.pos0, s.kv,
                          precision, false, nullptr, 0, as_stream(stream));
}

size_t brasa_flash_attention_workspace_len(brasa_attn_shape s, int precision) {
    g_err[0] = 0;
    if (prefill_check(s, precision) != BRASA_OK || s.tokens == 0) return 0;
    return prefill_workspace_len((int)s.tokens, (int)s.hq, (int)s.hkv, (int)s.pos0, s.kv,
                                 precision);
}

int brasa_flash_attention_ws(const float* q, const void* k, const void* v, void* o,
                             brasa_attn_shape s, int precision, void* workspace,
                             size_t workspace_len, void* stream) {
    g_err[0] = 0;
    const int st = prefill_check(s, precision);
    if (st != BRASA_OK) return st;
    if (s.tokens == 0) return BRASA_OK;
    if (!q || !k || !v || !o) return set_error(BRASA_ERR_ARG, "flash_attention: null pointer");
    const size_t need = prefill_workspace_len((int)s.tokens, (int)s.hq, (int)s.hkv, (int)s.pos0,
                                              s.kv, precision);
    if (workspace_len < need || (need > 0 && !workspace))
        return set_error(BRASA_ERR_SCRATCH, "flash_attention workspace too small (%zu < %zu bytes)",
                         workspace_len, need);
    return prefill_launch(q, k, v, o, (int)s.tokens, (int)s.hq, (int)s.hkv, (int)s.pos0, s.kv,
                          precision, true, workspace, workspace_len, as_stream(stream));
}

int brasa_flash_attention(const float* q, const void* k, const void* v, void* o,
                          brasa_attn_shape shape, void* stream) {
    return brasa_flash_attention_with(q, k, v, o, shape, BRASA_PREFILL_F16, stream);
}

int brasa_rope_table(double theta, size_t dim, size_t max_pos, float* cos_out, float* sin_out) {
    g_err[0] = 0;
    if (dim == 0 || dim % 2 != 0) return set_error(BRASA_ERR_SHAPE, "rope_table: dim must be even");
    if (max_pos > 0 && (!cos_out || !sin_out))
        return set_error(BRASA_ERR_ARG, "rope_table: null pointer");
    rope_table_host(theta, dim, max_pos, cos_out, sin_out);
    return BRASA_OK;
}

int brasa_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t n, float eps,
                   void* stream) {
    g_err[0] = 0;
    if (rows == 0) return BRASA_OK;
    if (n == 0 || n > ((size_t)1 << 24) || rows > ((size_t)1 << 30))
        return set_error(BRASA_ERR_SHAPE, "rms_norm: bad row length %zu", n);
    if (!x || !w || !out) return set_error(BRASA_ERR_ARG, "rms_norm: null pointer");
    return rms_norm_launch(x, w, out, rows, n, eps, as_stream(stream));
}

int brasa_rope_neox(float* x, brasa_rope_table_view table, size_t tokens, size_t heads,
                    size_t dim, size_t pos0, void* stream) {
    g_err[0] = 0;
    // lib.rs:579-583
    if (dim != table.dim) return set_error(BRASA_ERR_SHAPE, "RoPE table dimension");
    if (pos0 + tokens > table.max_pos) return set_error(BRASA_ERR_SHAPE, "position outside the RoPE table");
    if (dim == 0 || dim % 2 != 0 || heads > kMaxHeads)
        return set_error(BRASA_ERR_SHAPE, "rope_neox: bad shape");
    if (tokens == 0 || heads == 0) return BRASA_OK;
    if (!x || !table.cos || !table.sin) return set_error(BRASA_ERR_ARG, "rope_neox: null pointer");
    return rope_neox_launch(x, table.cos, table.sin, tokens, heads, dim, pos0, as_stream(stream));
}

int brasa_qk_norm_rope_store(int kv, float* q, float* k, const float* v, const float* q_norm,
                             const float* k_norm, float eps, brasa_rope_table_view table,
                             void* k_dst, void* v_dst, brasa_attn_shape s, void* stream) {
    g_err[0] = 0;
    if (!valid_kv(kv)) return set_error(BRASA_ERR_ARG, "qk_norm_rope_store: invalid kv type %d", kv);
    // lib.rs:996-1001
    if (s.dim != (size_t)kDim)
        return set_error(BRASA_ERR_SHAPE, "qk_norm_rope_store requires head_dim 128");
    if (s.dim != table.dim) return set_error(BRASA_ERR_SHAPE, "RoPE table dimension");
    if (s.pos0 + s.tokens > table.max_pos)
        return set_error(BRASA_ERR_SHAPE, "position outside the RoPE table");
    if (s.hq > kMaxHeads || s.hkv > kMaxHeads || s.tokens * (s.hq + 2 * s.hkv) > ((size_t)1 << 30))
        return set_error(BRASA_ERR_SHAPE, "qk_norm_rope_store: shape too large");
    if (s.tokens == 0) return BRASA_OK;
    if (!q || !k || !v || !q_norm || !k_norm || !table.cos || !table.sin || !k_dst || !v_dst)
        return set_error(BRASA_ERR_ARG, "qk_norm_rope_store: null pointer");
    return qk_norm_rope_store_launch(kv, q, k, v, q_norm, k_norm, eps, table.cos, table.sin,
                                     k_dst, v_dst, s.tokens, s.hq, s.hkv, s.pos0,
                                     as_stream(stream));
}

int brasa_release_workspaces(void) {
    g_err[0] = 0;
    prefill_release_workspaces();
    release_stream_slots();
    return BRASA_OK;
}

int brasa_test_flash_attention_layout(const float* q, const void* k, const void* v, void* o,
                                      brasa_attn_shape s, int precision, int variant, int pair,
                                      int parts, void* stream) {
    g_err[0] = 0;
    if (variant != 0 && variant != 1 && variant != 2 && variant != 4)
        return set_error(BRASA_ERR_ARG, "prefill layout: variant %d (0, 1, 2 or 4)", variant);
    if (parts < 1 || parts > 8)
        return set_error(BRASA_ERR_ARG, "prefill layout: %d key parts (1 .. 8)", parts);
    const int st = prefill_check(s, precision);
    if (st != BRASA_OK) return st;
    if (s.tokens == 0) return BRASA_OK;
    if (!q || !k || !v || !o) return set_error(BRASA_ERR_ARG, "flash_attention: null pointer");
    const int layout[3] = {variant, pair ? 1 : 0, parts};
    return prefill_launch(q, k, v, o, (int)s.tokens, (int)s.hq, (int)s.hkv, (int)s.pos0, s.kv,
                          precision, false, nullptr, 0, as_stream(stream), layout);
}

const char* brasa_last_error(void) { return g_err; }

const char* brasa_version(void) { return "brasa_attn 0.1.0 (gfx950)"; }

// ---- device plumbing (brasa_hip_rt.h) -----------------------------------------------------

int brasa_rt_device_count(int* count) { return hip_ok(hipGetDeviceCount(count), "hipGetDeviceCount"); }
int brasa_rt_set_device(int device) { return hip_ok(hipSetDevice(device), "hipSetDevice"); }
int brasa_rt_device_name(char* buf, size_t len) {
    hipDeviceProp_t p;
    int dev = 0;
    int st = hip_ok(hipGetDevice(&dev), "hipGetDevice");
    if (st) return st;
    st = hip_ok(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
    if (st) return st;
    snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return BRASA_OK;
}
int brasa_rt_malloc(void** ptr, size_t bytes) { return hip_ok(hipMalloc(ptr, bytes), "hipMalloc"); }
int brasa_rt_free(void* ptr) { return hip_ok(hipFree(ptr), "hipFree"); }
int brasa_rt_memcpy_htod(void* dst, const void* src, size_t bytes) {
    return hip_ok(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}
int brasa_rt_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    return hip_ok(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}
int brasa_rt_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)),
                  "hipMemcpyAsync D2D");
}
int brasa_rt_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream) {
    return fill_u8_launch(dst, value, bytes, as_stream(stream));
}
int brasa_rt_device_synchronize(void) {
    return hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}
int brasa_rt_stream_create(void** stream) {
    hipStream_t s = nullptr;
    int st = hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return st;
}
int brasa_rt_stream_destroy(void* stream) {
    return hip_ok(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
}
int brasa_rt_stream_synchronize(void* stream) {
    return hip_ok(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}
int brasa_rt_event_create(void** event) {
    hipEvent_t e = nullptr;
    int st = hip_ok(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return st;
}
int brasa_rt_event_destroy(void* event) {
    return hip_ok(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}
int brasa_rt_event_record(void* event, void* stream) {
    return hip_ok(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)),
                  "hipEventRecord");
}
int brasa_rt_event_elapsed_ms(float* ms, void* start, void* stop) {
    return hip_ok(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                      static_cast<hipEvent_t>(stop)),
                  "hipEventElapsedTime");
}
int brasa_rt_event_synchronize(void* event) {
    return hip_ok(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
}
int brasa_rt_stream_begin_capture(void* stream) {
    return hip_ok(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
                  "hipStreamBeginCapture");
}
int brasa_rt_stream_end_capture(void* stream, void** graph_exec) {
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    int st = hip_ok(hipStreamEndCapture(as_stream(stream), &g), "hipStreamEndCapture");
    if (st) return st;
    hipGraphExec_t e = nullptr;
    st = hip_ok(hipGraphInstantiate(&e, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    const int st2 = hip_ok(hipGraphDestroy(g), "hipGraphDestroy");
    if (st) return st;
    *graph_exec = e;
    return st2;
}
int brasa_rt_graph_launch(void* graph_exec, void* stream) {
    return hip_ok(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)),
                  "hipGraphLaunch");
}
int brasa_rt_graph_destroy(void* graph_exec) {
    return hip_ok(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)),
                  "hipGraphExecDestroy");
}
int brasa_rt_mem_info(size_t* free_bytes, size_t* total_bytes) {
    return hip_ok(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
}
int brasa_rt_fill_normal_f32(float* out, size_t n, uint64_t seed, float scale, void* stream) {
    return fill_normal_launch(out, n, seed, scale, as_stream(stream));
}

}  // extern "C"
