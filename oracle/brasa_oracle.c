/*
 * CPU oracle for the Brasa attention hot path -- TEST INFRASTRUCTURE ONLY (see brasa_oracle.h).
 *
 * Restated from the reference (Lautaro005/brasa), function by function; each cites its source.
 * Built with -ffp-contract=off and without fast-math so every f32 operation rounds exactly as the
 * reference's Rust code does (IEEE binary32 / binary64, round-to-nearest-even).
 *
 * What pins each function (tests/test_oracle.py runs every check):
 *   or_f16_to_f32 / or_f32_to_f16 : the reference's own KATs (qtype.rs:220-260): every non-NaN
 *       f16 round-trips, every midpoint between consecutive f16 goes to even and one f32 ulp
 *       either side goes to the nearest, 65520 -> inf, 2^-25 -> 0, 2^-25*1.0001 -> 1; plus the
 *       exhaustive cross-check against numpy's independent float16 cast (also RNE).
 *   or_quantize_kv_q8 / or_dequantize_kv_q8 : the KATs of qtype.rs:186-218 (round-trip bound,
 *       |q| = 127 present, zero block) and of crates/kernels/tests/attention.rs:256-285 (zero
 *       block, exact ties x/d = n + 0.5 go to even, amax = 1 gives d = f16(1/127), a 3000-valued
 *       block), plus a numpy restatement of the spec on random rows (independent code path).
 *   or_rng_* : closed forms of xorshift64* (first outputs for a seed computed with Python ints).
 *   or_attention / or_attention_q16 : independent f64 numpy softmax(QK^T)V on small cases, lk = 1
 *       gives o = v_0 exactly, all-equal keys give the mean of v, the causal mask (perturbing
 *       keys past pos0 + t leaves row t unchanged), and recompute_exp 0/1 bit-identical.
 *   or_worst / or_worst_f16 : closed-form hand cases.
 *   or_rms_norm / or_rope_neox / or_rope_table : numpy f64 restatements and rotation invariants
 *       (norm preservation of each rotated pair).
 */
#include "brasa_oracle.h"

#include <math.h>
#include <string.h>

typedef union { float f; uint32_t u; } f32bits;

static uint32_t f2u(float f) { f32bits b; b.f = f; return b.u; }
static float u2f(uint32_t u) { f32bits b; b.u = u; return b.f; }

/* crates/quant/src/qtype.rs:32-50 -- exact widening of an IEEE binary16. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: shift the mantissa until its leading one reaches bit 10 */
        uint32_t s = 0;
        while ((m & 0x400u) == 0) { m <<= 1; ++s; }
        return u2f(sign | ((113u - s) << 23) | ((m & 0x3ffu) << 13));
    }
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* crates/quant/src/qtype.rs:52-78 -- binary32 -> binary16, round to nearest even, overflow to
 * inf, NaN stays NaN (quiet bit set). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); /* >= 65536 */
    uint32_t h, rem, half;
    if (a >= 0x38800000u) { /* normal in f16 (>= 2^-14) */
        h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
        rem = a & 0x1fffu;
        half = 0x1000u;
    } else if (a < 0x33000000u) { /* < 2^-25 */
        return sign;
    } else { /* subnormal in f16 */
        uint32_t shift = 126u - (a >> 23);
        uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        h = mant >> shift;
        rem = mant & ((1u << shift) - 1u);
        half = 1u << (shift - 1u);
    }
    /* a carry out of the mantissa correctly bumps the exponent (or reaches inf) */
    uint32_t up = (rem > half || (rem == half && (h & 1u))) ? 1u : 0u;
    return (uint16_t)(sign | (h + up));
}

void or_f32_to_f16_n(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f32_to_f16(x[i]);
}

void or_f16_to_f32_n(const uint16_t* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f16_to_f32(x[i]);
}

/* crates/kernels/src/reference.rs:66-69 */
float or_round_f16(float v) { return or_f16_to_f32(or_f32_to_f16(v)); }

/* crates/quant/src/qtype.rs:85-111 -- the KV-Q8 spec: per 32-group, dh = f16(amax / 127),
 * d = f32(dh), q = d == 0 ? 0 : clamp(round_ties_even(x / d), -127, 127); the row is the 128
 * int8 values followed by the 4 little-endian f16 scales. */
void or_quantize_kv_q8(const float* x, size_t n, uint8_t* out) {
    for (size_t r = 0; r < n / OR_KV_Q8_DIM; ++r) {
        const float* row = x + r * OR_KV_Q8_DIM;
        uint8_t* o = out + r * OR_KV_Q8_ROW;
        for (int b = 0; b < 4; ++b) {
            const float* blk = row + 32 * b;
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) {
                float a = fabsf(blk[j]);
                amax = a > amax ? a : amax; /* f32::max: NaN-free inputs */
            }
            uint16_t dh = or_f32_to_f16(amax / 127.0f);
            float d = or_f16_to_f32(dh);
            for (int j = 0; j < 32; ++j) {
                float q = 0.0f;
                if (d != 0.0f) {
                    q = rintf(blk[j] / d); /* default rounding mode: ties to even */
                    if (q < -127.0f) q = -127.0f;
                    if (q > 127.0f) q = 127.0f;
                }
                o[32 * b + j] = (uint8_t)(int8_t)q;
            }
            o[OR_KV_Q8_DIM + 2 * b] = (uint8_t)(dh & 0xffu);
            o[OR_KV_Q8_DIM + 2 * b + 1] = (uint8_t)(dh >> 8);
        }
    }
}

/* crates/quant/src/qtype.rs:113-130 -- v = f32(scale[i / 32]) * (int8)q[i], exact in f32. */
void or_dequantize_kv_q8(const uint8_t* data, size_t rows, float* out) {
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t* row = data + r * OR_KV_Q8_ROW;
        for (int i = 0; i < OR_KV_Q8_DIM; ++i) {
            int b = i / 32;
            uint16_t dh = (uint16_t)(row[OR_KV_Q8_DIM + 2 * b] |
                                     ((uint16_t)row[OR_KV_Q8_DIM + 2 * b + 1] << 8));
            out[r * OR_KV_Q8_DIM + i] = or_f16_to_f32(dh) * (float)(int8_t)row[i];
        }
    }
}

/* crates/kernels/src/testutil.rs:4-28 -- xorshift64*, seed 0 replaced by 1. */
void or_rng_init(or_rng* r, uint64_t seed) { r->s = seed ? seed : 1; }

uint64_t or_rng_next_u64(or_rng* r) {
    r->s ^= r->s >> 12;
    r->s ^= r->s << 25;
    r->s ^= r->s >> 27;
    return r->s * 0x2545f4914f6cdd1dULL;
}

/* uniform in [-1, 1): top 24 bits / 2^23 - 1, all exact in f32 */
float or_rng_uniform(or_rng* r) {
    return (float)(or_rng_next_u64(r) >> 40) / (float)(1u << 23) - 1.0f;
}

void or_rng_vec(or_rng* r, float* out, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) out[i] = or_rng_uniform(r) * scale;
}

/* crates/kernels/src/reference.rs:173-218 (attention_scaled), restricted to query tokens
 * [t0, t1). Scores and softmax in f64; `scale` multiplies each f64 dot product. */
static void attention_scaled_rows(const float* q, const float* k, const float* v,
                                  size_t hq, size_t hkv, size_t dim, size_t pos0, double scale,
                                  size_t t0, size_t t1, float* o, float* vmax,
                                  int recompute_exp, double* s /* >= pos0 + t1 */) {
    size_t group = hq / hkv;
    for (size_t t = t0; t < t1; ++t) {
        size_t last = pos0 + t;
        for (size_t h = 0; h < hq; ++h) {
            size_t kh = h / group;
            const float* qv = q + (t * hq + h) * dim;
            for (size_t j = 0; j <= last; ++j) {
                const float* kr = k + (j * hkv + kh) * dim;
                double acc = 0.0;
                for (size_t d = 0; d < dim; ++d) acc += (double)qv[d] * (double)kr[d];
                s[j] = acc * scale;
            }
            double m = -INFINITY;
            for (size_t j = 0; j <= last; ++j) m = s[j] > m ? s[j] : m;
            double z = 0.0;
            for (size_t j = 0; j <= last; ++j) z += exp(s[j] - m);
            if (!recompute_exp) {
                /* exp(s_j - m) is a pure function of s_j and m: evaluating it once per key and
                 * reusing the double gives the same bits as re-evaluating it per d. */
                for (size_t j = 0; j <= last; ++j) s[j] = exp(s[j] - m);
            }
            for (size_t d = 0; d < dim; ++d) {
                double acc = 0.0;
                float mx = 0.0f;
                for (size_t j = 0; j <= last; ++j) {
                    float vj = v[(j * hkv + kh) * dim + d];
                    double e = recompute_exp ? exp(s[j] - m) : s[j];
                    acc += e / z * (double)vj;
                    float a = fabsf(vj);
                    mx = a > mx ? a : mx;
                }
                o[(t * hq + h) * dim + d] = (float)acc;
                if (vmax) vmax[(t * hq + h) * dim + d] = mx;
            }
        }
    }
}

#include <stdlib.h>

void or_attention_rows(const float* q, const float* k, const float* v, size_t tokens,
                       size_t hq, size_t hkv, size_t dim, size_t pos0, size_t t0, size_t t1,
                       float* o, float* vmax, int recompute_exp, int q16) {
    if (t1 > tokens) t1 = tokens;
    if (t0 >= t1) return;
    double* s = (double*)malloc(sizeof(double) * (pos0 + t1));
    if (!s) return;
    if (q16) {
        /* reference.rs:129-145: Q * (1/sqrt(dim) in f32), rounded to f16, then scale 1 */
        float scale = 1.0f / sqrtf((float)dim);
        size_t n = tokens * hq * dim;
        float* qs = (float*)malloc(sizeof(float) * n);
        if (!qs) { free(s); return; }
        for (size_t i = 0; i < n; ++i) qs[i] = or_round_f16(q[i] * scale);
        attention_scaled_rows(qs, k, v, hq, hkv, dim, pos0, 1.0, t0, t1, o, vmax,
                              recompute_exp, s);
        free(qs);
    } else {
        /* reference.rs:150-171: scale = 1 / sqrt(dim) in f64 */
        attention_scaled_rows(q, k, v, hq, hkv, dim, pos0, 1.0 / sqrt((double)dim), t0, t1, o,
                              vmax, recompute_exp, s);
    }
    free(s);
}

void or_attention(const float* q, const float* k, const float* v, size_t tokens, size_t hq,
                  size_t hkv, size_t dim, size_t pos0, float* o, float* vmax,
                  int recompute_exp) {
    or_attention_rows(q, k, v, tokens, hq, hkv, dim, pos0, 0, tokens, o, vmax, recompute_exp,
                      0);
}

void or_attention_q16(const float* q, const float* k, const float* v, size_t tokens,
                      size_t hq, size_t hkv, size_t dim, size_t pos0, float* o, float* vmax,
                      int recompute_exp) {
    or_attention_rows(q, k, v, tokens, hq, hkv, dim, pos0, 0, tokens, o, vmax, recompute_exp,
                      1);
}

/* crates/kernels/tests/attention.rs:25-32 */
float or_worst(const float* got, const float* expected, const float* vmax, size_t n) {
    float w = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float m = vmax[i] > 1e-30f ? vmax[i] : 1e-30f;
        float e = fabsf(got[i] - expected[i]) / m;
        w = e > w ? e : w;
    }
    return w;
}

/* crates/kernels/tests/attention.rs:12-23 */
float or_worst_f16(const uint16_t* got, const float* expected, const float* vmax, size_t n) {
    const float ulp_half = 0x1p-11f;
    float w = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float d = fabsf(or_f16_to_f32(got[i]) - expected[i]) - fabsf(expected[i]) * ulp_half;
        if (d < 0.0f) d = 0.0f;
        float m = vmax[i] > 1e-30f ? vmax[i] : 1e-30f;
        float e = d / m;
        w = e > w ? e : w;
    }
    return w;
}

/* crates/kernels/src/reference.rs:22-30 */
void or_rms_norm(const float* x, const float* w, size_t rows, size_t n, float eps, float* out) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * n;
        double ss = 0.0;
        for (size_t i = 0; i < n; ++i) ss += (double)xr[i] * (double)xr[i];
        double scale = 1.0 / sqrt(ss / (double)n + (double)eps);
        for (size_t i = 0; i < n; ++i)
            out[r * n + i] = (float)((double)xr[i] * scale * (double)w[i]);
    }
}

/* crates/kernels/src/reference.rs:45-58 */
void or_rope_neox(float* x, size_t tokens, size_t heads, size_t dim, size_t pos0,
                  const float* cos_t, const float* sin_t) {
    size_t half = dim / 2;
    for (size_t t = 0; t < tokens; ++t) {
        size_t p = pos0 + t;
        for (size_t hh = 0; hh < heads; ++hh) {
            float* vv = x + (t * heads + hh) * dim;
            for (size_t i = 0; i < half; ++i) {
                double c = cos_t[p * half + i], s = sin_t[p * half + i];
                double a = vv[i], b = vv[i + half];
                vv[i] = (float)(a * c - b * s);
                vv[i + half] = (float)(b * c + a * s);
            }
        }
    }
}

/* crates/kernels/src/lib.rs:1388-1404 */
void or_rope_table(double theta, size_t dim, size_t max_pos, float* cos_t, float* sin_t) {
    size_t half = dim / 2;
    for (size_t p = 0; p < max_pos; ++p) {
        for (size_t i = 0; i < half; ++i) {
            double inv = 1.0 / pow(theta, (double)(2 * i) / (double)dim);
            double a = (double)p * inv;
            cos_t[p * half + i] = (float)cos(a);
            sin_t[p * half + i] = (float)sin(a);
        }
    }
}
