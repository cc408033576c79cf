/*
 * brasa_attn -- MI355X (gfx950) attention hot path of the Brasa engine behind a C ABI.
 *
 * Each operation below replaces one method of the reference's `brasa_kernels::Kernels`
 * (crates/kernels/src/lib.rs) for attention; a Rust shim turns a nonzero status back into the
 * reference's `assert!` panic (shape/scratch/unsupported-group errors) or `MetalError`
 * (device failures). Conventions shared by every entry point:
 *
 *   - Pointers are device pointers (hipMalloc'ed or views into such allocations). A view at a
 *     byte offset, which the reference expresses as `Arg::Buf(buffer, offset)`
 *     (crates/metal/src/runtime.rs:255-295), is passed as the already-offset pointer.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream). Work is enqueued,
 *     never waited for; ordering is the stream's, as the reference's one in-order command queue.
 *   - No call allocates device memory. Decode scratch (`partials`) is caller-owned, sized by
 *     brasa_decode_partials_len(). The library's own device state is fixed at load: arrival
 *     counters of the in-kernel split merges (decode, and prefill's key split; each launch
 *     returns the ones it uses to zero), one slot of them per stream (the first 64 streams used
 *     on a device each get one, in the order they are first used; a launch on a stream without
 *     a slot uses a plan that needs no counters: one split per sequence in decode, no key split
 *     in prefill), the no-allocation decode array and the fixed prefill workspace (see
 *     brasa_flash_attention_with, brasa_release_workspaces). Every entry point can be captured
 *     into a HIP graph (it enqueues kernels only: no allocation, no memset node, no host wait),
 *     and a replay computes what an eager call on the replay's inputs computes, bit for bit
 *     (the counters return to zero in every launch, the q8_0 range flag of prefill is cleared
 *     by the launch that reads it). A graph captured from a stream keeps that stream's slot:
 *     do not replay it while other work on the same stream, or another replay of a graph
 *     captured there, is in flight.
 *   - Return value: BRASA_OK (0) or a BRASA_ERR_* code; brasa_last_error() then describes it
 *     (thread-local string, valid until the next call on the same thread).
 *
 * KV cache layout (crates/kernels/src/metal/kv_access.metal:1-9; crates/models/src/qwen3.rs:211):
 * one layer is [cap, hkv, 128] rows; row index = position * hkv + kv_head. Row bytes: f32 512,
 * f16 256, q8_0 136 (128 int8 followed by 4 little-endian f16 scales, one per 32 values;
 * crates/quant/src/qtype.rs:80-83).
 */
#ifndef BRASA_ATTN_H
#define BRASA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define BRASA_OK 0
#define BRASA_ERR_SHAPE 1       /* a shape assert of the reference would panic */
#define BRASA_ERR_SCRATCH 2     /* partials scratch smaller than brasa_decode_partials_len */
#define BRASA_ERR_UNSUPPORTED 3 /* GQA group / precision combination not compiled */
#define BRASA_ERR_LAUNCH 4      /* HIP reported an error enqueueing the kernel */
#define BRASA_ERR_ARG 5         /* null pointer or invalid enum value */

/* KvType (crates/kernels/src/lib.rs:92-143); values equal the reference's `KvType as usize`. */
#define BRASA_KV_F32 0
#define BRASA_KV_F16 1
#define BRASA_KV_Q8_0 2

/* PrefillPrecision (crates/kernels/src/lib.rs:1311-1318). */
#define BRASA_PREFILL_F16 0 /* Q*scale rounded to f16, output f16 (hot path) */
#define BRASA_PREFILL_F32 1 /* exact variant: Q and output f32 */
/* F16 inputs and output with P carried to f32 accuracy through the P.V contraction, which is
 * what the reference's F16 kernel computes (flash_attention.metal:197 keeps P in f32). Plain
 * BRASA_PREFILL_F16 rounds P to f16 for the matrix cores (within the 2e-3 / 1e-2 bar). */
#define BRASA_PREFILL_F16_PF32 2

/* Output element type of the decode entry points. The reference writes f32 (its `ws.attn`);
 * f16 (RNE) is offered for callers whose next GEMM reads f16. */
#define BRASA_OUT_F32 0
#define BRASA_OUT_F16 1

/* AttnShape (crates/kernels/src/lib.rs:1354-1364). */
typedef struct brasa_attn_shape {
    size_t tokens;
    size_t hq;
    size_t hkv;
    size_t dim;  /* must be 128 for every attention entry point, as in the reference */
    size_t pos0; /* absolute position of the first query token */
    int kv;      /* BRASA_KV_* */
} brasa_attn_shape;

/* Keys per split-K tramo of the reference (DECODE_CHUNK, lib.rs:1331). */
#define BRASA_DECODE_CHUNK 128
/* Positions the KV cache must be readable past pos0 + tokens for prefill (KV_ALIGN,
 * lib.rs:1350-1351). */
#define BRASA_KV_ALIGN 64

/* decode_partials_len (lib.rs:1334-1337): floats of decode scratch for hq heads and lk keys,
 * hq * ceil(lk / 128) * 130. The kernels here use at most that many. */
size_t brasa_decode_partials_len(size_t hq, size_t lk);

/* gqa_supported (lib.rs:1323-1327): hq / hkv in {1, 2, 4, 8}. */
int brasa_gqa_supported(size_t hq, size_t hkv);

/* KvType::bytes (lib.rs:109-121): bytes of n cache elements (n a multiple of 128 for q8_0);
 * returns 0 and sets the error for an invalid type or a ragged q8_0 count. */
size_t brasa_kv_bytes(int kv, size_t n);

/* KV cache layout of the model (crates/models/src/qwen3.rs:384-386,554-556; the memory
 * planner's kv_bytes, crates/memory/src/planner.rs:77-81). One layer holds
 * cap = brasa_kv_capacity(ctx) positions of hkv x dim values; each of K and V is one buffer of
 * brasa_kv_cache_len(layers, ctx, hkv, dim) elements (brasa_kv_bytes of that many bytes). */
/* ctx rounded up to a multiple of BRASA_KV_ALIGN (ctx.next_multiple_of(KV_ALIGN)). */
size_t brasa_kv_capacity(size_t ctx);
/* layers * cap * hkv * dim: elements of the K (or V) cache buffer. */
size_t brasa_kv_cache_len(size_t layers, size_t ctx, size_t hkv, size_t dim);
/* (layer * cap + pos) * hkv * dim: element offset of position `pos` of `layer` (pos = 0 gives the
 * layer base the attention entry points read; pos = pos0 the rows qk_norm_rope_store writes).
 * The byte offset of the view is brasa_kv_bytes(kv, offset). */
size_t brasa_kv_offset(size_t layer, size_t ctx, size_t hkv, size_t dim, size_t pos);

/*
 * Kernels::store_kv (lib.rs:1029-1050; device code kv.metal:6-40): converts n f32 values at
 * `src` into the cache type at `dst`. f32: copy; f16: round to nearest even; q8_0: n must be a
 * multiple of 128 and each 32-group is quantised bit-exactly as quantize_kv_q8
 * (crates/quant/src/qtype.rs:85-111).
 */
int brasa_store_kv(int kv, const float* src, void* dst, size_t n, void* stream);

/*
 * Dequantises `rows` q8_0 rows (136 bytes each) at `src` into rows*128 f32 values at `dst`,
 * bit-exactly as dequantize_kv_q8 (crates/quant/src/qtype.rs:113-130) and as the in-kernel
 * accessors read them (kv_access.metal:15-27). The reference has no separate kernel for this:
 * it is exported so the "Q8 dequantisation is bit-exact" contract can be checked on the device.
 */
int brasa_dequantize_kv_q8(const void* src, float* dst, size_t rows, void* stream);

/*
 * Kernels::decode_attention_lanes (lib.rs:1110-1164; device code decode_attention.metal:
 * 108-199 + 68-84): attention of one query token at position shape.pos0 over keys
 * [0, pos0 + 1) of the layer cache k/v, all query heads of a GQA group served from one read of
 * each K/V row. q: [hq, 128] f32 (scaled by 1/sqrt(128) inside, in f32); o: [hq, 128] in
 * `o_dtype`. partials: caller scratch of partials_len floats, at least
 * brasa_decode_partials_len(hq, pos0 + 1). Requires tokens == 1, dim == 128 and
 * hq / hkv in {1, 2, 4, 8} (BRASA_ERR_UNSUPPORTED otherwise, where the reference panics).
 * The result bits depend only on q, the cache rows and lk: the launch layout is a function of
 * lk and the head counts (no tuning knob), and the split merge runs in a fixed order, as the
 * reference requires of every launch width (crates/kernels/tests/launch.rs:119-168). The
 * exception is a stream without a counter slot (more than 64 streams in use on the device),
 * which decodes with one split per sequence: the same result to the decode tolerance, slower.
 * The split merge counts arrivals in the stream's slot, so launches in flight on different
 * streams never share counters.
 */
int brasa_decode_attention_lanes(const float* q, const void* k, const void* v, float* partials,
                                 size_t partials_len, void* o, int o_dtype,
                                 brasa_attn_shape shape, void* stream);

/*
 * No counterpart in the reference. brasa_decode_attention_lanes without the caller's scratch,
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the split partials live in a fixed array inside the
 * library, BRASA_DECODE_NOALLOC_FLOATS floats (4 MiB) per device, held until the process ends.
 * A call needs hq * splits * 130 floats, where the launch plan keeps splits <= 256 * h / hkv
 * for h head groups per workgroup (h <= 4, h * hq / hkv <= 16; with 8 KV heads: 32 splits,
 * 133,120 floats for hq 32, at any length), so no valid shape needs more than 16 * 256 * 130
 * floats; a call needing more would fail with BRASA_ERR_SCRATCH. The call allocates nothing.
 * Every call on one device shares the array: calls that overlap on one GPU (different streams
 * without ordering, or graph replays concurrent with other decode calls) race and give wrong
 * results. Its split merge counts arrivals in the calling stream's counter slot, like
 * brasa_decode_attention_lanes; a graph captured from a stream keeps that slot (see the
 * conventions above). Same results, bit for bit, as brasa_decode_attention_lanes on the same
 * arguments.
 */
#define BRASA_DECODE_NOALLOC_FLOATS (1 << 20)
int brasa_decode_attention_lanes_noalloc(const float* q, const void* k, const void* v, void* o,
                                         int o_dtype, brasa_attn_shape shape, void* stream);

/*
 * Kernels::decode_attention (lib.rs:1056-1103; decode_attention.metal:15-84): same contract as
 * brasa_decode_attention_lanes, one query head per workgroup, for any hq multiple of hkv (the
 * reference's fallback for groups outside {1, 2, 4, 8}).
 */
int brasa_decode_attention(const float* q, const void* k, const void* v, float* partials,
                           size_t partials_len, void* o, int o_dtype, brasa_attn_shape shape,
                           void* stream);

/*
 * Ragged batched decode (no counterpart in the reference, which decodes one sequence per call,
 * lib.rs:1110-1164; a caller batching sequences, e.g. a serving scheduler over session.rs:240-245,
 * would otherwise issue one call per sequence). One launch of the split kernel (the split merge
 * runs inside it) covers up to 64 sequences (more: one launch per 64): sequence i has one query q[i] (q: [n, hq, 128] f32), its own layer
 * caches k[i] / v[i] (HOST arrays of device pointers, same layout as decode_attention_lanes) and
 * lk[i] >= 1 keys (HOST array). o: [n, hq, 128] in o_dtype. Each sequence's result agrees with
 * brasa_decode_attention_lanes on it alone to the decode tolerance, not bit for bit: a launch
 * cuts every sequence into splits of one length chosen from the batch's total keys, so the split
 * boundaries (and the f32 rounding of the merge) differ from the single-sequence call's. A
 * single-sequence call's result depends only on its inputs and lk. Scratch: partials_len >=
 * brasa_decode_batch_partials_len(hq, lk, n) floats. Requires dim == 128 and a GQA group in
 * {1, 2, 4, 8}.
 */
size_t brasa_decode_batch_partials_len(size_t hq, const size_t* lk, size_t n);
int brasa_decode_attention_batch(const float* q, const void* const* k, const void* const* v,
                                 const size_t* lk, size_t n, float* partials,
                                 size_t partials_len, void* o, int o_dtype, size_t hq,
                                 size_t hkv, size_t dim, int kv, void* stream);

/*
 * Kernels::flash_attention_with (lib.rs:1185-1248; flash_attention.metal:152-323): causal GQA
 * prefill. q: [tokens, hq, 128] f32; query t (absolute position pos0 + t) attends to keys
 * [0, pos0 + t]. k/v: layer cache readable up to ceil64(pos0 + tokens) positions (values past
 * pos0 + tokens are masked; they must be finite). o: [tokens, hq, 128], f16 bits for
 * BRASA_PREFILL_F16 / BRASA_PREFILL_F16_PF32 (Q*scale rounded to f16 as the reference does,
 * fp32 softmax and accumulation) or f32 for BRASA_PREFILL_F32. Requires dim == 128 and
 * hq % hkv == 0; when hq / hkv is not in {1, 2, 4, 8} only BRASA_PREFILL_F32 is accepted
 * (BRASA_ERR_UNSUPPORTED otherwise), as the reference asserts (lib.rs:1227-1231). A launch
 * that would fill at most half of the GPU with long key ranges per query tile (a short chunk
 * after a long cached prefix, e.g. 512 tokens at pos0 16384) splits each tile's keys over up to
 * 8 workgroups; their partials go to a workspace (68 KB per part and query tile). With a q8_0
 * cache and BRASA_PREFILL_F16, the rows read (ceil64(pos0 + tokens) positions) are first
 * dequantised to f16 (each value f16(code * scale)) into the workspace (512 B per row of K and
 * V), and the f16 kernels run on it; small calls convert the same values in registers. When a
 * group scale lets f16(code * scale) leave the normal f16 range (|scale| >= 516, f16-subnormal,
 * inf or NaN scales) the call is recomputed exactly (the reference's F16 numerics: Q rounded
 * to f16, K / V exact, P f32) by the launch after the conversion, which reads a flag the
 * conversion sets (on some plans a separate short launch on every q8_0 F16 call).
 * Like the reference's, this call allocates nothing: its workspace is a fixed 96 MiB device
 * array of the library, owned by the first stream that needs it (until
 * brasa_release_workspaces); calls on other streams, or whose plan needs more, run without the
 * key split or the staging (slower, the same results up to the split's rounding).
 * brasa_flash_attention_ws takes a caller workspace instead. The key split counts its parts in
 * the stream's counter slot (see brasa_decode_attention_lanes). The result does not depend on
 * the order in which the parts finish.
 */
int brasa_flash_attention_with(const float* q, const void* k, const void* v, void* o,
                               brasa_attn_shape shape, int precision, void* stream);

/* Kernels::flash_attention (lib.rs:1169-1180): brasa_flash_attention_with(.., F16). */
int brasa_flash_attention(const float* q, const void* k, const void* v, void* o,
                          brasa_attn_shape shape, void* stream);

/*
 * No counterpart in the reference (its flash_attention encodes onto buffers the caller owns and
 * needs no scratch; lib.rs:1169-1248). Bytes of workspace brasa_flash_attention_ws needs for
 * this shape and precision: the key split's partials and the q8_0 staging the call's plan uses
 * (0 when it uses neither, or for an invalid shape).
 */
size_t brasa_flash_attention_workspace_len(brasa_attn_shape shape, int precision);

/*
 * brasa_flash_attention_with on a caller-owned device workspace of workspace_len bytes (at least
 * brasa_flash_attention_workspace_len; BRASA_ERR_SCRATCH otherwise), for callers on any stream
 * that want the full plan. Allocates nothing. The same kernels and plan as the fixed-workspace
 * call, so the results are bit-identical to it. Calls in flight at the same time need distinct
 * workspaces.
 */
int brasa_flash_attention_ws(const float* q, const void* k, const void* v, void* o,
                             brasa_attn_shape shape, int precision, void* workspace,
                             size_t workspace_len, void* stream);

/*
 * RopeTable (lib.rs:1365-1386): device arrays cos/sin [max_pos, dim / 2] (f32) built from
 * brasa_rope_table, plus their shape.
 */
typedef struct brasa_rope_table_view {
    const float* cos;
    const float* sin;
    size_t dim;
    size_t max_pos;
} brasa_rope_table_view;

/*
 * rope_table (lib.rs:1388-1404), on the host: cos/sin(p * theta^(-2 i / dim)) for p < max_pos,
 * i < dim / 2, computed in f64 and stored as f32 into HOST arrays of max_pos * dim / 2 floats
 * (upload them once at load time, as RopeTable::new does).
 */
int brasa_rope_table(double theta, size_t dim, size_t max_pos, float* cos_out, float* sin_out);

/*
 * Kernels::rms_norm (lib.rs:529-547; norm.metal:8-48): out[r, :] = x[r, :] * (1 / sqrt(mean x^2
 * + eps)) * w for rows of n values (f32); out may equal x. Same bits as the normalisation inside
 * brasa_qk_norm_rope_store for n == 128.
 */
int brasa_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t n, float eps,
                   void* stream);

/*
 * Kernels::rope_neox (lib.rs:567-596; rope.metal:8-27): RoPE-NeoX in place on x [tokens, heads,
 * dim] (f32) at positions pos0 .. pos0 + tokens. Requires dim == table.dim and
 * pos0 + tokens <= table.max_pos.
 */
int brasa_rope_neox(float* x, brasa_rope_table_view table, size_t tokens, size_t heads,
                    size_t dim, size_t pos0, void* stream);

/*
 * Kernels::qk_norm_rope_store (lib.rs:972-1025; qkv.metal:37-94), one launch: per token, q
 * [tokens, hq, 128] and k [tokens, hkv, 128] (f32, updated in place) are RMS-normalised with
 * q_norm / k_norm [128] and eps and rotated by RoPE-NeoX at pos0 + t; then k and v
 * [tokens, hkv, 128] are stored into the caches k_dst / v_dst (pointing at row pos0 * hkv of
 * the layer) in cache type `kv`, with store_kv's rounding. Bit-identical to brasa_rms_norm,
 * brasa_rope_neox and brasa_store_kv in sequence. Requires dim == 128 == table.dim and
 * pos0 + tokens <= table.max_pos (shape.kv is ignored; `kv` rules, as in the reference).
 */
int brasa_qk_norm_rope_store(int kv, float* q, float* k, const float* v, const float* q_norm,
                             const float* k_norm, float eps, brasa_rope_table_view table,
                             void* k_dst, void* v_dst, brasa_attn_shape shape, void* stream);

/*
 * No counterpart in the reference. Returns the library's per-stream state to its initial
 * condition: the stream -> counter slot assignments (decode and prefill split merges) and the
 * ownership of the fixed prefill workspace. Call it only while no call of this library is in
 * flight or being enqueued (e.g. before destroying streams whose handles may be reused), so that
 * a new stream never inherits a slot whose counters a running launch still uses. Frees nothing:
 * the library holds no allocations.
 */
int brasa_release_workspaces(void);

/*
 * Test entry point (no counterpart in the reference; a production caller never needs it):
 * brasa_flash_attention_with with the prefill layout of this one call forced. The kernel for
 * BRASA_KV_F16 (and for q8_0 rows staged as f16) is otherwise chosen by workgroup count; tests
 * cover each of the three kernels at small sizes with variant 1 (two key groups per workgroup),
 * 2 (four waves) or 4 (four waves, 32-key stages); 0 keeps the choice by size. pair = 0 stops
 * the two-group kernel from pairing heavy and light query tiles (the results are identical
 * either way). parts (1 .. 8) is the number of workgroups each query tile's keys are split over
 * when variant 1 is forced (with variant 0 the split is chosen by size). Nothing outlives the
 * call: there is no process-wide layout state.
 */
int brasa_test_flash_attention_layout(const float* q, const void* k, const void* v, void* o,
                                      brasa_attn_shape shape, int precision, int variant,
                                      int pair, int parts, void* stream);

/*
 * Test hook (no counterpart in the reference). The counter slot of `stream` on `device` that the
 * split merges use (assigning one on first use, as a launch would), or -1 when the device's 64
 * slots are taken. Needs no GPU.
 */
int brasa_test_stream_slot(int device, void* stream, int* slot);

/*
 * Test hooks (no counterpart in the reference). brasa_test_decode_plan: the decode launch plan
 * for n <= 64 sequences of lengths lk (as one batched launch on a stream with a counter slot
 * plans it): keys per split, head groups per workgroup, and each sequence's split count.
 * brasa_test_split_blocks: the 32-key blocks split `split` of a sequence of lk keys in `splits`
 * splits computes (the kernels' own function): the first block's key, the keys between its
 * blocks and their count. Need no GPU.
 */
int brasa_test_decode_plan(const int* lk, int n, int hq, int hkv, int kv, int* chunk, int* hpw,
                           int* splits);
int brasa_test_split_blocks(int lk, int splits, int split, int* first, int* stride, int* count);

#ifdef BRASA_TIMELINE_BUILD
/*
 * Timeline build only (libbrasa_attn_trace.so; no counterpart in the reference): copy up to n
 * of the decode / prefill_f16_kernel phase stamps (16 per workgroup slot, 100 MHz real-time
 * counter, slot = linear workgroup index mod 8192) to host memory. Read by
 * brasa_amd/decode_timeline.py and brasa_amd/prefill_timeline.py.
 */
int brasa_decode_trace_read(unsigned long long* dst, size_t n);
int brasa_prefill_trace_read(unsigned long long* dst, size_t n);
#endif

/* Description of the last error on this thread ("" if none). */
const char* brasa_last_error(void);

/* Library version string. */
const char* brasa_version(void);

#ifdef __cplusplus
}
#endif
#endif
