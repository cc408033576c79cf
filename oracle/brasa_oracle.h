/*
 * CPU oracle for the Brasa attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's CPU attention and KV-cache arithmetic, used
 * as the checker for the HIP kernels in brasa_amd/. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product path never calls into it.
 *
 * Every function names the reference file:line (under Lautaro005/brasa) it restates. What pins
 * each function (known-answer tests, closed forms, independent implementations) is listed in the
 * header of oracle/brasa_oracle.c and exercised by tests/test_oracle.py.
 */
#ifndef BRASA_ORACLE_H
#define BRASA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* crates/quant/src/qtype.rs:32-50 */
float or_f16_to_f32(uint16_t h);
/* crates/quant/src/qtype.rs:52-78 */
uint16_t or_f32_to_f16(float f);
/* bulk helpers over the two scalar conversions */
void or_f32_to_f16_n(const float* x, uint16_t* out, size_t n);
void or_f16_to_f32_n(const uint16_t* x, float* out, size_t n);
/* crates/kernels/src/reference.rs:66-69: f16 round trip */
float or_round_f16(float v);

/* crates/quant/src/qtype.rs:80-83 */
#define OR_KV_Q8_DIM 128
#define OR_KV_Q8_ROW 136
/* crates/quant/src/qtype.rs:85-111. n must be a multiple of 128; out holds n/128*136 bytes. */
void or_quantize_kv_q8(const float* x, size_t n, uint8_t* out);
/* crates/quant/src/qtype.rs:113-130. rows*136 bytes -> rows*128 floats. */
void or_dequantize_kv_q8(const uint8_t* data, size_t rows, float* out);

/* crates/kernels/src/testutil.rs:4-28: xorshift64* generator. */
typedef struct { uint64_t s; } or_rng;
void or_rng_init(or_rng* r, uint64_t seed);
uint64_t or_rng_next_u64(or_rng* r);
float or_rng_uniform(or_rng* r);
void or_rng_vec(or_rng* r, float* out, size_t n, float scale);

/*
 * crates/kernels/src/reference.rs:150-218 (`attention`, scale 1/sqrt(dim) in f64) and
 * reference.rs:129-145 (`attention_q16`: Q*scale in f32 rounded to f16, then scale 1).
 * q: [tokens, hq, dim]; k, v: [pos0 + tokens, hkv, dim] (f32 values as the GPU sees them);
 * o, vmax: [tokens, hq, dim]. vmax may be NULL.
 * recompute_exp != 0 re-evaluates exp(s_j - m) for every output component d, exactly as
 * reference.rs:209 does (the timed CPU baseline); 0 evaluates it once per key and reuses the
 * same double, which gives bit-identical outputs (the fast checker).
 */
void or_attention(const float* q, const float* k, const float* v, size_t tokens, size_t hq,
                  size_t hkv, size_t dim, size_t pos0, float* o, float* vmax,
                  int recompute_exp);
void or_attention_q16(const float* q, const float* k, const float* v, size_t tokens,
                      size_t hq, size_t hkv, size_t dim, size_t pos0, float* o, float* vmax,
                      int recompute_exp);
/*
 * Same as or_attention but only for query token t in [t0, t1) (rows of o/vmax for those tokens
 * are written at their natural offsets). Used to time a bounded sample of a large prefill.
 */
void or_attention_rows(const float* q, const float* k, const float* v, size_t tokens,
                       size_t hq, size_t hkv, size_t dim, size_t pos0, size_t t0, size_t t1,
                       float* o, float* vmax, int recompute_exp, int q16);

/* crates/kernels/tests/attention.rs:25-32: max |got - exp| / max|v|. */
float or_worst(const float* got, const float* expected, const float* vmax, size_t n);
/* crates/kernels/tests/attention.rs:12-23: as or_worst for f16 output, discounting the final
 * rounding (2^-11 * |expected|). */
float or_worst_f16(const uint16_t* got, const float* expected, const float* vmax, size_t n);

/* crates/kernels/src/reference.rs:22-30 (rms_norm, f64 sum of squares). */
void or_rms_norm(const float* x, const float* w, size_t rows, size_t n, float eps, float* out);
/* crates/kernels/src/reference.rs:45-58 (rope_neox in place on [T, heads, dim]). */
void or_rope_neox(float* x, size_t tokens, size_t heads, size_t dim, size_t pos0,
                  const float* cos_t, const float* sin_t);
/* crates/kernels/src/lib.rs:1388-1404 (rope_table: cos/sin in f64 stored as f32). */
void or_rope_table(double theta, size_t dim, size_t max_pos, float* cos_t, float* sin_t);

#ifdef __cplusplus
}
#endif
#endif
