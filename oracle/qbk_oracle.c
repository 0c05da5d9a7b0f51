/*
 * qbk_oracle.c -- CPU restatement of quantibbler-kernels' hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -ffp-contract=off
 * -fno-fast-math -fopenmp).
 *
 * Pinning (see tests/test_oracle_*.py):
 *   pack/unpack/validate   pack_bits.json, closed-form byte positions
 *   packed products        packed_matvec.json, packed_matmul.json (f64 bit
 *                          identity), dtype_parity.json (f32/bf16 exact),
 *                          brute-force dense products
 *   fast face              backward error <= 1e-12 sum|v| vs the sequential face
 *   bf16 RNE               half's tie KAT from_acc(1 + 2^-12) == 1.0
 *   qpk1 parse             the reference's 48-byte v1 / 50-byte v2 hex KATs
 *   factor composite       the engine's hand-derived 4x4x r8 layer and bias KATs
 *   attention (exact)      attention_tiled.json, dense softmax closed form
 *   attention (sage, f64)  attention_sage.json quantized-reference.out
 *   attention (sage, f32)  attention_sage.json within the device gate (1e-4)
 *   block-scaled sage      no reference implementation exists (the scheme
 *                          is north_star's); pinned by what the mathematics
 *                          fixes: Q's scale over exactly each 64-token
 *                          window with RNE codes, identical keys giving the
 *                          mean of V, a one-hot softmax giving that V row,
 *                          fp16 P with an f32 row sum on two keys; plus
 *                          exact-attention quality and the quantizer
 *                          invariants
 *   decoder block, trunk   the reference's parity-tiny HF goldens (logits of
 *                          a 2-layer model, 1e-2 budget), planted composition
 *                          mistakes that must fail them, RoPE / RMSNorm
 *                          closed forms, a dense f64 block step
 */
#include "qbk_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define SETERR(...)                                      \
    do {                                                 \
        if (err && errlen) snprintf(err, errlen, __VA_ARGS__); \
    } while (0)

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

/* ======================================================================= */
/* bit layout                                                              */
/* ======================================================================= */

/* core.rs:129-162 pack_bits: byte j holds elements 8j..8j+7, element 8j+k at
 * bit k (LSB-first), +1 -> 1, -1 -> 0, pad bits zero. */
int orc_pack_bits(const int8_t *factor, size_t factor_len, size_t n_rows, size_t n_cols,
                  uint8_t *out, char *err, size_t errlen) {
    if (n_rows * n_cols != factor_len) {
        SETERR("factor length %zu does not match %zux%zu", factor_len, n_rows, n_cols);
        return 1;
    }
    size_t n_words = div_ceil(n_cols, 8);
    for (size_t i = 0; i < n_rows; i++) {
        for (size_t j = 0; j < n_words; j++) {
            uint8_t byte = 0;
            for (size_t k = 0; k < 8; k++) {
                size_t idx = j * 8 + k;
                if (idx >= n_cols) break;
                int8_t v = factor[i * n_cols + idx];
                if (v == 1) {
                    byte |= (uint8_t)(1u << k);
                } else if (v != -1) {
                    SETERR("pack_bits expects values in {-1, +1}; got %d at row %zu, column %zu",
                           (int)v, i, idx);
                    return 1;
                }
            }
            out[i * n_words + j] = byte;
        }
    }
    return 0;
}

/* core.rs:166-189 unpack_bits: pad bits ignored, n_bits == 0 -> empty rows. */
int orc_unpack_bits(const uint8_t *packed, size_t packed_len, size_t n_rows, size_t n_bits,
                    int8_t *out, char *err, size_t errlen) {
    size_t n_words = div_ceil(n_bits, 8);
    if (n_rows * n_words != packed_len) {
        SETERR("packed length %zu does not match %zu rows x %zu bitplanes", packed_len, n_rows,
               n_words);
        return 1;
    }
    for (size_t i = 0; i < n_rows; i++)
        for (size_t k = 0; k < n_bits; k++)
            out[i * n_bits + k] = ((packed[i * n_words + (k >> 3)] >> (k & 7)) & 1) ? 1 : -1;
    return 0;
}

/* core.rs:223-240 validate_packed */
int orc_validate_packed(size_t packed_len, size_t n_rows, size_t n_bits, size_t *n_words,
                        char *err, size_t errlen) {
    if (n_bits == 0 && packed_len != 0 && n_rows != 0) {
        SETERR("n_bits=0 with non-empty packed rows");
        return 1;
    }
    size_t w = div_ceil(n_bits, 8);
    if (n_rows * w != packed_len) {
        SETERR("packed length %zu does not match %zu rows x %zu bitplanes", packed_len, n_rows, w);
        return 1;
    }
    if (n_words) *n_words = w;
    return 0;
}

/* core.rs sign_estimate: v >= 0 (including -0.0) -> +1, else -1. */
void orc_sign_estimate(const double *x, size_t n, int8_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = (x[i] >= 0.0) ? 1 : -1;
}

/* ======================================================================= */
/* bf16 / f16 helpers                                                      */
/* ======================================================================= */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* half 2.7.1 bf16::from_f32: NaN keeps a quiet payload; otherwise round to
 * nearest, ties to even (dtype.rs:77-92 relies on it). */
uint16_t orc_f32_to_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    const uint32_t round_bit = 0x8000u;
    if ((u & round_bit) != 0 && (u & (3u * round_bit - 1u)) != 0) return (uint16_t)((u >> 16) + 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return u2f(((uint32_t)b) << 16); }

/* IEEE binary16 round-to-nearest-even from f32 (subnormals kept). */
static uint16_t f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (ax < 0x33000001u) {                                    /* < half of min subnormal */
        return (uint16_t)sign;
    }
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    if (e < -14) { /* subnormal half: value = mant * 2^(e-23); unit 2^-24 */
        int shift = -14 - e + 13;  /* bits dropped from the 24-bit mantissa */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = mant >> 13;
    uint32_t rem = mant & 0x1fffu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | (q & 0x3ffu);
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* 2^-24 */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* ======================================================================= */
/* sequential packed products (core.rs:202-317)                            */
/* ======================================================================= */

static int bit_at(const uint8_t *row, size_t k) { return (row[k >> 3] >> (k & 7)) & 1; }

int orc_packed_matvec(int dtype, const uint8_t *packed, size_t packed_len, size_t n_rows,
                      size_t n_bits, const void *vec, size_t vec_len, void *out, char *err,
                      size_t errlen) {
    size_t w;
    if (orc_validate_packed(packed_len, n_rows, n_bits, &w, err, errlen)) return 1;
    if (vec_len != n_bits) {
        SETERR("vec must have length %zu, got %zu", n_bits, vec_len);
        return 1;
    }
    for (size_t i = 0; i < n_rows; i++) {
        const uint8_t *row = packed + i * w;
        if (dtype == 0) {
            const double *v = (const double *)vec;
            double acc = 0.0;
            for (size_t k = 0; k < n_bits; k++) acc = acc + (bit_at(row, k) ? 1.0 : -1.0) * v[k];
            ((double *)out)[i] = acc;
        } else if (dtype == 1) {
            const float *v = (const float *)vec;
            float acc = 0.0f;
            for (size_t k = 0; k < n_bits; k++) acc = acc + (bit_at(row, k) ? 1.0f : -1.0f) * v[k];
            ((float *)out)[i] = acc;
        } else {
            const uint16_t *v = (const uint16_t *)vec;
            float acc = 0.0f;
            for (size_t k = 0; k < n_bits; k++)
                acc = acc + (bit_at(row, k) ? 1.0f : -1.0f) * orc_bf16_to_f32(v[k]);
            ((uint16_t *)out)[i] = orc_f32_to_bf16(acc);
        }
    }
    return 0;
}

/* core.rs:288-317: output width k = mat_len / max(n_bits, 1); element t of
 * output column j reads mat[t*n_cols + j].  The reference indexes without a
 * bounds check (a Rust panic); here an out-of-range read is an error. */
int orc_packed_matmul(int dtype, const uint8_t *packed, size_t packed_len, size_t n_rows,
                      size_t n_bits, const void *mat, size_t mat_len, size_t n_cols, void *out,
                      char *err, size_t errlen) {
    size_t w;
    if (orc_validate_packed(packed_len, n_rows, n_bits, &w, err, errlen)) return 1;
    if (n_bits != 0 && mat_len % n_bits != 0) {
        SETERR("mat length %zu is not a multiple of n_bits %zu", mat_len, n_bits);
        return 1;
    }
    size_t kc = mat_len / (n_bits ? n_bits : 1);
    if (n_bits > 0 && kc > 0 && n_rows > 0 && (n_bits - 1) * n_cols + (kc - 1) >= mat_len) {
        SETERR("mat index out of range: n_cols %zu with %zu columns over %zu rows", n_cols, kc,
               n_bits);
        return 1;
    }
    for (size_t i = 0; i < n_rows; i++) {
        const uint8_t *row = packed + i * w;
        for (size_t j = 0; j < kc; j++) {
            if (dtype == 0) {
                const double *m = (const double *)mat;
                double acc = 0.0;
                for (size_t t = 0; t < n_bits; t++)
                    acc = acc + (bit_at(row, t) ? 1.0 : -1.0) * m[t * n_cols + j];
                ((double *)out)[i * kc + j] = acc;
            } else if (dtype == 1) {
                const float *m = (const float *)mat;
                float acc = 0.0f;
                for (size_t t = 0; t < n_bits; t++)
                    acc = acc + (bit_at(row, t) ? 1.0f : -1.0f) * m[t * n_cols + j];
                ((float *)out)[i * kc + j] = acc;
            } else {
                const uint16_t *m = (const uint16_t *)mat;
                float acc = 0.0f;
                for (size_t t = 0; t < n_bits; t++)
                    acc = acc + (bit_at(row, t) ? 1.0f : -1.0f) * orc_bf16_to_f32(m[t * n_cols + j]);
                ((uint16_t *)out)[i * kc + j] = orc_f32_to_bf16(acc);
            }
        }
    }
    return 0;
}

/* ======================================================================= */
/* fast face (fast.rs:28-158)                                              */
/* ======================================================================= */

static double g_lut[256][8];
static int g_lut_ready = 0;

static void lut_init(void) {
    if (g_lut_ready) return;
    for (int b = 0; b < 256; b++)
        for (int k = 0; k < 8; k++) g_lut[b][k] = ((b >> k) & 1) ? 1.0 : -1.0;
    g_lut_ready = 1;
}

/* fast.rs:51-81 row_dot: four lane-sequential partials over 4-element groups
 * held in one f64x4 register (wide::f64x4 there, a GCC vector here: AVX2
 * with -march=x86-64-v3), lane-wise multiply then add (no contraction), the
 * fixed reduce (a0+a2)+(a1+a3), then the scalar tail in element order. */
typedef double orc_f64x4 __attribute__((vector_size(32)));

static double row_dot(const uint8_t *row, const double *vec, size_t n_bits) {
    orc_f64x4 acc = {0.0, 0.0, 0.0, 0.0};
    size_t n4 = n_bits / 4;
    for (size_t t = 0; t < n4; t++) {
        size_t base = t * 4;
        orc_f64x4 sg, v;
        memcpy(&sg, g_lut[row[base >> 3]] + (base & 7), sizeof sg);
        memcpy(&v, vec + base, sizeof v);
        orc_f64x4 p = sg * v;
        acc = acc + p;
    }
    double v4 = (acc[0] + acc[2]) + (acc[1] + acc[3]);
    double tail = 0.0;
    for (size_t k = n4 * 4; k < n_bits; k++) tail = tail + (bit_at(row, k) ? 1.0 : -1.0) * vec[k];
    return v4 + tail;
}

#define ROWS_PER_TASK 64 /* fast.rs:44 */

int orc_fast_packed_matvec_f64(const uint8_t *packed, size_t packed_len, size_t n_rows,
                               size_t n_bits, const double *vec, size_t vec_len, double *out,
                               int threads, char *err, size_t errlen) {
    size_t w;
    if (orc_validate_packed(packed_len, n_rows, n_bits, &w, err, errlen)) return 1;
    if (vec_len != n_bits) {
        SETERR("vec must have length %zu, got %zu", n_bits, vec_len);
        return 1;
    }
    if (n_rows == 0 || n_bits == 0) {
        for (size_t i = 0; i < n_rows; i++) out[i] = 0.0;
        return 0;
    }
    lut_init();
    long nblk = (long)div_ceil(n_rows, ROWS_PER_TASK);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
    for (long b = 0; b < nblk; b++) {
        size_t lo = (size_t)b * ROWS_PER_TASK, hi = lo + ROWS_PER_TASK;
        if (hi > n_rows) hi = n_rows;
        for (size_t i = lo; i < hi; i++) out[i] = row_dot(packed + i * w, vec, n_bits);
    }
    return 0;
}

int orc_fast_packed_matmul_f64(const uint8_t *packed, size_t packed_len, size_t n_rows,
                               size_t n_bits, const double *mat, size_t mat_len, size_t n_cols,
                               double *out, int threads, char *err, size_t errlen) {
    size_t w;
    if (orc_validate_packed(packed_len, n_rows, n_bits, &w, err, errlen)) return 1;
    if (n_bits != 0 && mat_len % n_bits != 0) {
        SETERR("mat length %zu is not a multiple of n_bits %zu", mat_len, n_bits);
        return 1;
    }
    size_t kc = mat_len / (n_bits ? n_bits : 1);
    if (n_rows == 0 || kc == 0) {
        for (size_t i = 0; i < n_rows * kc; i++) out[i] = 0.0;
        return 0;
    }
    if (n_bits > 0 && (n_bits - 1) * n_cols + (kc - 1) >= mat_len) {
        SETERR("mat index out of range: n_cols %zu with %zu columns over %zu rows", n_cols, kc,
               n_bits);
        return 1;
    }
    long nblk = (long)div_ceil(n_rows, ROWS_PER_TASK);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
    for (long b = 0; b < nblk; b++) {
        size_t lo = (size_t)b * ROWS_PER_TASK, hi = lo + ROWS_PER_TASK;
        if (hi > n_rows) hi = n_rows;
        for (size_t i = lo; i < hi; i++) {
            double *acc = out + i * kc;
            for (size_t j = 0; j < kc; j++) acc[j] = 0.0;
            const uint8_t *row = packed + i * w;
            for (size_t t = 0; t < n_bits; t++) {
                double s = bit_at(row, t) ? 1.0 : -1.0;
                const double *m = mat + t * n_cols;
                for (size_t j = 0; j < kc; j++) acc[j] = acc[j] + s * m[j];
            }
        }
    }
    return 0;
}

/* ======================================================================= */
/* qpk1 (crates/quantibbler-qpk1/src/lib.rs:152-320)                       */
/* ======================================================================= */

static uint32_t rd32(const uint8_t *b) {
    return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
}

size_t orc_qpk1_expected_size(size_t dout, size_t din, size_t r, int itemsize, int with_bias) {
    size_t floats = with_bias ? 2 * dout + din : dout + din;
    return 24 + floats * (size_t)itemsize + div_ceil(dout * r, 8) + div_ceil(din * r, 8);
}

/* lib.rs:195-213 f16_to_f64: exact widening. */
static double f16_to_f64(uint16_t bits) {
    double sign = ((bits >> 15) & 1) ? -1.0 : 1.0;
    int e = (bits >> 10) & 0x1f;
    double frac = (double)(bits & 0x3ff);
    if (e == 0) return sign * frac * ldexp(1.0, -24);
    if (e == 0x1f) return frac == 0.0 ? sign * INFINITY : NAN;
    return sign * (1.0 + frac / 1024.0) * ldexp(1.0, e - 15);
}

static void decode_floats(const uint8_t *p, size_t n, int tag, double *dst) {
    for (size_t i = 0; i < n; i++) {
        if (tag == 1) {
            uint16_t h = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
            dst[i] = f16_to_f64(h);
        } else {
            dst[i] = (double)u2f(rd32(p + 4 * i));
        }
    }
}

int orc_qpk1_parse(const uint8_t *bytes, size_t len, orc_qpk1_header *hdr, double *s1,
                   double *s2, double *bias, char *err, size_t errlen) {
    if (len < 24) {
        SETERR("stream is %zu bytes; shorter than the 24-byte header", len);
        return 1;
    }
    if (memcmp(bytes, "QPK1", 4) != 0) {
        SETERR("bad magic [%u, %u, %u, %u]; expected [81, 80, 75, 49]", bytes[0], bytes[1],
               bytes[2], bytes[3]);
        return 1;
    }
    uint32_t version = rd32(bytes + 4);
    if (version != 1 && version != 2) {
        SETERR("unsupported representation version %u; this reader implements version 1 "
               "(pre-bias legacy) and version 2 (current, with bias)", version);
        return 1;
    }
    uint32_t tag = rd32(bytes + 8);
    if (tag != 1 && tag != 2) {
        SETERR("unknown dtype tag %u; expected 1 (float16) or 2 (float32)", tag);
        return 1;
    }
    size_t dout = rd32(bytes + 12), din = rd32(bytes + 16), r = rd32(bytes + 20);
    if (dout == 0 || din == 0 || r == 0) {
        SETERR("dout, din and r must all be >= 1, got (%zu, %zu, %zu)", dout, din, r);
        return 1;
    }
    int item = tag == 1 ? 2 : 4;
    int has_bias = version >= 2;
    size_t expected = orc_qpk1_expected_size(dout, din, r, item, has_bias);
    if (len < expected) {
        SETERR("truncated stream: %zu bytes; header declares %zu", len, expected);
        return 1;
    }
    if (len > expected) {
        SETERR("trailing garbage: %zu bytes; one layer at this header is %zu", len, expected);
        return 1;
    }
    hdr->version = version;
    hdr->dtype_tag = tag;
    hdr->dout = dout;
    hdr->din = din;
    hdr->r = r;
    size_t off = 24;
    hdr->s1_off = off;
    off += dout * item;
    hdr->s2_off = off;
    off += din * item;
    hdr->bias_off = has_bias ? off : 0;
    if (has_bias) off += dout * item;
    hdr->ub_off = off;
    off += div_ceil(dout * r, 8);
    hdr->vb_off = off;
    if (s1) decode_floats(bytes + hdr->s1_off, dout, tag, s1);
    if (s2) decode_floats(bytes + hdr->s2_off, din, tag, s2);
    if (bias && has_bias) decode_floats(bytes + hdr->bias_off, dout, tag, bias);
    return 0;
}

/* ======================================================================= */
/* engine layout repack + factor composite (engine/mod.rs:258-481)        */
/* ======================================================================= */

void orc_container_to_rows(const uint8_t *packed, size_t n_rows, size_t r, uint8_t *out) {
    size_t rw = div_ceil(r, 8);
    if (r % 8 == 0) {
        memcpy(out, packed, n_rows * rw);
        return;
    }
    memset(out, 0, n_rows * rw);
    for (size_t i = 0; i < n_rows; i++)
        for (size_t j = 0; j < r; j++) {
            size_t b = i * r + j;
            if ((packed[b >> 3] >> (b & 7)) & 1) out[i * rw + (j >> 3)] |= (uint8_t)(1u << (j & 7));
        }
}

void orc_container_to_rows_transposed(const uint8_t *packed, size_t din, size_t r, uint8_t *out) {
    size_t rw = div_ceil(din, 8);
    memset(out, 0, r * rw);
    for (size_t j = 0; j < din; j++)
        for (size_t k = 0; k < r; k++) {
            size_t b = j * r + k;
            if ((packed[b >> 3] >> (b & 7)) & 1) out[k * rw + (j >> 3)] |= (uint8_t)(1u << (j & 7));
        }
}

/* engine/mod.rs:393-481 PackedLayer::apply (Fp32: f64 matvecs through the
 * scalar core or the fast face) and apply_bf16 (bf16 operand, f32 acc). */
int orc_factor_apply(int serving, size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                     const uint8_t *vb_t_rows, const float *s1, const float *s2,
                     const float *bias, const float *x, float *y, int fast, int threads) {
    char err[256];
    if (serving == 0) {
        double *z = (double *)malloc(sizeof(double) * (din ? din : 1));
        double *t = (double *)malloc(sizeof(double) * (r ? r : 1));
        double *u = (double *)malloc(sizeof(double) * (dout ? dout : 1));
        for (size_t j = 0; j < din; j++) z[j] = (double)(s2[j] * x[j]);
        int rc;
        if (fast) {
            rc = orc_fast_packed_matvec_f64(vb_t_rows, r * div_ceil(din, 8), r, din, z, din, t,
                                            threads, err, sizeof err);
            if (!rc)
                rc = orc_fast_packed_matvec_f64(ub_rows, dout * div_ceil(r, 8), dout, r, t, r, u,
                                                threads, err, sizeof err);
        } else {
            rc = orc_packed_matvec(0, vb_t_rows, r * div_ceil(din, 8), r, din, z, din, t, err,
                                   sizeof err);
            if (!rc)
                rc = orc_packed_matvec(0, ub_rows, dout * div_ceil(r, 8), dout, r, t, r, u, err,
                                       sizeof err);
        }
        if (!rc)
            for (size_t i = 0; i < dout; i++) y[i] = ((float)u[i]) * s1[i] + (bias ? bias[i] : 0.0f);
        free(z);
        free(t);
        free(u);
        return rc;
    }
    uint16_t *z = (uint16_t *)malloc(2 * (din ? din : 1));
    uint16_t *t = (uint16_t *)malloc(2 * (r ? r : 1));
    uint16_t *u = (uint16_t *)malloc(2 * (dout ? dout : 1));
    for (size_t j = 0; j < din; j++) z[j] = orc_f32_to_bf16(s2[j] * x[j]);
    int rc = orc_packed_matvec(2, vb_t_rows, r * div_ceil(din, 8), r, din, z, din, t, err,
                               sizeof err);
    if (!rc)
        rc = orc_packed_matvec(2, ub_rows, dout * div_ceil(r, 8), dout, r, t, r, u, err, sizeof err);
    if (!rc)
        for (size_t i = 0; i < dout; i++)
            y[i] = orc_bf16_to_f32(u[i]) * s1[i] + (bias ? bias[i] : 0.0f);
    free(z);
    free(t);
    free(u);
    return rc;
}

void orc_factor_apply_bf16_batch(size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                                 const uint8_t *vb_t_rows, const float *s1, const float *s2,
                                 const float *bias, const uint16_t *x, size_t batch, float *y,
                                 uint16_t *t_out, int threads) {
    size_t wd = div_ceil(din, 8), wr = div_ceil(r, 8);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
    for (long bb = 0; bb < (long)batch; bb++) {
        uint16_t *z = (uint16_t *)malloc(2 * (din ? din : 1));
        uint16_t *t = (uint16_t *)malloc(2 * (r ? r : 1));
        const uint16_t *xb = x + (size_t)bb * din;
        for (size_t j = 0; j < din; j++) z[j] = orc_f32_to_bf16(s2[j] * orc_bf16_to_f32(xb[j]));
        for (size_t k = 0; k < r; k++) {
            const uint8_t *row = vb_t_rows + k * wd;
            float acc = 0.0f;
            for (size_t j = 0; j < din; j++)
                acc = acc + (bit_at(row, j) ? 1.0f : -1.0f) * orc_bf16_to_f32(z[j]);
            t[k] = orc_f32_to_bf16(acc);
        }
        if (t_out) memcpy(t_out + (size_t)bb * r, t, 2 * r);
        for (size_t i = 0; i < dout; i++) {
            const uint8_t *row = ub_rows + i * wr;
            float acc = 0.0f;
            for (size_t k = 0; k < r; k++)
                acc = acc + (bit_at(row, k) ? 1.0f : -1.0f) * orc_bf16_to_f32(t[k]);
            float u = orc_bf16_to_f32(orc_f32_to_bf16(acc));
            y[(size_t)bb * dout + i] = u * s1[i] + (bias ? bias[i] : 0.0f);
        }
        free(z);
        free(t);
    }
}

/* ======================================================================= */
/* attention                                                               */
/* ======================================================================= */

/* attention_tiled.py:76-180, exact FlashAttention-1 Algorithm 1 in f64. */
int orc_attention_tiled_f64(const orc_attn_shape *sh, const double *q, const double *k,
                            const double *v, int causal, size_t block, double *out,
                            double *lse) {
    size_t B = sh->batch, H = sh->n_heads, Hk = sh->n_kv_heads, S = sh->seq, d = sh->head_dim,
           dv = sh->val_dim;
    if (!block || !Hk || H % Hk) return 1;
    size_t group = H / Hk;
    double scale = 1.0 / sqrt((double)d);
    double *sc = (double *)malloc(sizeof(double) * block);
    for (size_t b = 0; b < B; b++)
        for (size_t h = 0; h < H; h++) {
            size_t kv = h / group;
            const double *kb = k + (b * Hk + kv) * S * d;
            const double *vb = v + (b * Hk + kv) * S * dv;
            for (size_t i = 0; i < S; i++) {
                const double *qi = q + ((b * H + h) * S + i) * d;
                double *oi = out + ((b * H + h) * S + i) * dv;
                size_t i1 = (i / block + 1) * block;
                if (i1 > S) i1 = S;
                size_t j_stop = causal ? i1 : S;
                double m = -INFINITY, ell = 0.0;
                for (size_t c = 0; c < dv; c++) oi[c] = 0.0;
                for (size_t j0 = 0; j0 < j_stop; j0 += block) {
                    size_t j1 = j0 + block < S ? j0 + block : S;
                    double mb = -INFINITY;
                    for (size_t j = j0; j < j1; j++) {
                        double acc = 0.0;
                        for (size_t c = 0; c < d; c++) acc += qi[c] * kb[j * d + c];
                        double s = acc * scale;
                        if (causal && j > i) s = -INFINITY;
                        sc[j - j0] = s;
                        if (s > mb) mb = s;
                    }
                    double m_new = m > mb ? m : mb;
                    int empty = isinf(m_new) && m_new < 0;
                    double alpha = empty ? 0.0 : exp(m - m_new);
                    double sum = 0.0;
                    for (size_t j = j0; j < j1; j++) {
                        double w = empty ? 0.0 : exp(sc[j - j0] - m_new);
                        sc[j - j0] = w;
                        sum += w;
                    }
                    ell = alpha * ell + sum;
                    for (size_t c = 0; c < dv; c++) {
                        double pv = 0.0;
                        for (size_t j = j0; j < j1; j++) pv += sc[j - j0] * vb[j * dv + c];
                        oi[c] = alpha * oi[c] + pv;
                    }
                    m = m_new;
                }
                for (size_t c = 0; c < dv; c++) oi[c] = oi[c] / ell;
                if (lse) lse[(b * H + h) * S + i] = m + log(ell);
            }
        }
    free(sc);
    return 0;
}

static double clampd(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }

/* attention_sage.py:136-350 in f64 NumPy semantics: per-token Q (1/sqrt(d)
 * folded), per-K-block mean gamma, per-token K, P at the static 1/127 scale
 * after the running-max rescale, per-channel V within the tile, and the
 * unsmoothed score path (the block's shift added back). */
int orc_attention_sage_np_f64(const orc_attn_shape *sh, const double *q, const double *k,
                              const double *v, int causal, size_t block, double *out) {
    size_t B = sh->batch, H = sh->n_heads, Hk = sh->n_kv_heads, S = sh->seq, d = sh->head_dim,
           dv = sh->val_dim;
    if (!block || !Hk || H % Hk) return 1;
    size_t group = H / Hk;
    double inv = 1.0 / sqrt((double)d);
    /* psi_Q over the whole tensor (attention_sage.py:256) */
    size_t nq = B * H * S;
    double *qhat = (double *)malloc(sizeof(double) * nq * d);
    double *qsc = (double *)malloc(sizeof(double) * nq);
    for (size_t r = 0; r < nq; r++) {
        double peak = 0.0;
        for (size_t c = 0; c < d; c++) {
            double x = fabs(q[r * d + c] * inv);
            if (x > peak) peak = x;
        }
        double delta = peak > 0.0 ? peak / 127.0 : 1.0;
        qsc[r] = delta;
        for (size_t c = 0; c < d; c++) qhat[r * d + c] = clampd(rint((q[r * d + c] * inv) / delta), -127, 127);
    }
    double *kmean = (double *)malloc(sizeof(double) * d);
    double *khat = (double *)malloc(sizeof(double) * block * d);
    double *ksc = (double *)malloc(sizeof(double) * block);
    double *vhat = (double *)malloc(sizeof(double) * block * dv);
    double *vsc = (double *)malloc(sizeof(double) * dv);
    double *sc = (double *)malloc(sizeof(double) * block);
    for (size_t b = 0; b < B; b++)
        for (size_t h = 0; h < H; h++) {
            size_t kv = h / group;
            const double *kb = k + (b * Hk + kv) * S * d;
            const double *vb = v + (b * Hk + kv) * S * dv;
            for (size_t i0 = 0; i0 < S; i0 += block) {
                size_t i1 = i0 + block < S ? i0 + block : S;
                size_t j_stop = causal ? i1 : S;
                for (size_t i = i0; i < i1; i++) {
                    size_t row = (b * H + h) * S + i;
                    const double *qh = qhat + row * d;
                    double qs = qsc[row];
                    double *oi = out + row * dv;
                    double m = -INFINITY, ell = 0.0;
                    for (size_t c = 0; c < dv; c++) oi[c] = 0.0;
                    for (size_t j0 = 0; j0 < j_stop; j0 += block) {
                        size_t j1 = j0 + block < S ? j0 + block : S, kj = j1 - j0;
                        for (size_t c = 0; c < d; c++) {
                            double acc = 0.0;
                            for (size_t j = j0; j < j1; j++) acc += kb[j * d + c];
                            kmean[c] = acc / (double)kj;
                        }
                        for (size_t j = j0; j < j1; j++) {
                            double peak = 0.0;
                            for (size_t c = 0; c < d; c++) {
                                double g = fabs(kb[j * d + c] - kmean[c]);
                                if (g > peak) peak = g;
                            }
                            double delta = peak > 0.0 ? peak / 127.0 : 1.0;
                            ksc[j - j0] = delta;
                            for (size_t c = 0; c < d; c++)
                                khat[(j - j0) * d + c] = clampd(rint((kb[j * d + c] - kmean[c]) / delta), -127, 127);
                        }
                        double mb = -INFINITY;
                        for (size_t j = j0; j < j1; j++) {
                            double dot = 0.0, shift = 0.0;
                            for (size_t c = 0; c < d; c++) dot += qh[c] * khat[(j - j0) * d + c];
                            for (size_t c = 0; c < d; c++) shift += (qh[c] * qs) * kmean[c];
                            double s = dot * qs * ksc[j - j0] + shift;
                            if (causal && j > i) s = -INFINITY;
                            sc[j - j0] = s;
                            if (s > mb) mb = s;
                        }
                        double m_new = m > mb ? m : mb;
                        int empty = isinf(m_new) && m_new < 0;
                        double alpha = empty ? 0.0 : exp(m - m_new);
                        double sum = 0.0;
                        for (size_t j = j0; j < j1; j++) {
                            double p = empty ? 0.0 : exp(sc[j - j0] - m_new);
                            sum += p;
                            sc[j - j0] = clampd(rint(p / (1.0 / 127.0)), 0, 127); /* p_hat */
                        }
                        ell = alpha * ell + sum;
                        for (size_t c = 0; c < dv; c++) {
                            double peak = 0.0;
                            for (size_t j = j0; j < j1; j++) {
                                double a = fabs(vb[j * dv + c]);
                                if (a > peak) peak = a;
                            }
                            vsc[c] = peak > 0.0 ? peak / 127.0 : 1.0;
                            for (size_t j = j0; j < j1; j++)
                                vhat[(j - j0) * dv + c] = clampd(rint(vb[j * dv + c] / vsc[c]), -127, 127);
                        }
                        for (size_t c = 0; c < dv; c++) {
                            double pv = 0.0;
                            for (size_t j = j0; j < j1; j++) pv += sc[j - j0] * vhat[(j - j0) * dv + c];
                            double contrib = pv * (1.0 / 127.0) * vsc[c];
                            oi[c] = alpha * oi[c] + (empty ? 0.0 : contrib);
                        }
                        m = m_new;
                    }
                    for (size_t c = 0; c < dv; c++) oi[c] = oi[c] / ell;
                }
            }
        }
    free(qhat); free(qsc); free(kmean); free(khat); free(ksc); free(vhat); free(vsc); free(sc);
    return 0;
}

/* exp(x) for the f32 reference scheme, written from the mathematics:
 * Cody & Waite (1980) reduction x = n*ln2 + r with ln2 split in two parts
 * (the high part has 12 trailing zero bits, so n*ln2_hi is exact for
 * |n| < 2^12), |r| <= ln2/2, then e^r by the degree-7 Taylor polynomial
 * (truncation 0.3466^8/8! < 6e-9), and the result scaled by 2^n through the
 * exponent field in two steps (so 2^n never overflows on its own).
 * The device kernel carries the same operation sequence, so the two agree
 * bit for bit. */
float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return INFINITY;
    if (x < -103.97208f) return 0.0f;
    const float log2e = 1.44269504088896341f;
    const float ln2_hi = 0.693145751953125f;      /* 0x3f317200 */
    const float ln2_lo = 1.428606765330187045e-06f; /* ln2 - ln2_hi */
    float n = rintf(x * log2e);
    float r = x - n * ln2_hi;
    r = r - n * ln2_lo;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    int ni = (int)n;
    int n1 = ni / 2, n2 = ni - n1;
    float s1 = u2f((uint32_t)(n1 + 127) << 23);
    float s2 = u2f((uint32_t)(n2 + 127) << 23);
    return (p * s1) * s2;
}

static int8_t q8(float x) { /* clamp(rint_half_even(x), -127, 127) */
    float r = rintf(x);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    return (int8_t)r;
}

#define MASKED (-3.0e38f)

/* gpu_attention.rs:89-396 sage_int8_tile_kernel, one row at a time, in the
 * kernel's f32 operation order (sentinel -3e38, `live` flag, alpha = 0 on an
 * empty row, O/l at the end).  exp is orc_expf. */
int orc_attention_sage_dev_f32(const orc_attn_shape *sh, const float *q, const float *k,
                               const float *v, int causal, size_t block, float *out,
                               int8_t *qhat_out, float *qdelta_out, int threads) {
    size_t B = sh->batch, H = sh->n_heads, Hk = sh->n_kv_heads, S = sh->seq, d = sh->head_dim,
           dv = sh->val_dim;
    if (!block || !Hk || H % Hk) return 1;
    size_t group = H / Hk;
    float inv_sqrt_d = 1.0f / sqrtf((float)d);
    long rows = (long)(B * H * S);
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        int8_t *qhat = (int8_t *)malloc(d);
        float *kmean = (float *)malloc(sizeof(float) * d);
        float *sc = (float *)malloc(sizeof(float) * block);
        int8_t *ph = (int8_t *)malloc(block);
        float *vd = (float *)malloc(sizeof(float) * dv);
#pragma omp for schedule(dynamic, 16)
        for (long row = 0; row < rows; row++) {
            size_t b = (size_t)row / (H * S), r2 = (size_t)row % (H * S), h = r2 / S, i = r2 % S;
            size_t kvh = h / group;
            size_t i1 = (i / block + 1) * block;
            if (i1 > S) i1 = S;
            size_t j_stop = causal ? i1 : S;
            const float *qi = q + (size_t)row * d;
            float qpeak = 0.0f;
            for (size_t c = 0; c < d; c++) {
                float x = qi[c] * inv_sqrt_d;
                float ax = x < 0.0f ? 0.0f - x : x;
                if (ax > qpeak) qpeak = ax;
            }
            float qdelta = 1.0f;
            if (qpeak > 0.0f) qdelta = qpeak / 127.0f;
            for (size_t c = 0; c < d; c++) qhat[c] = q8((qi[c] * inv_sqrt_d) / qdelta);
            if (qhat_out) memcpy(qhat_out + (size_t)row * d, qhat, d);
            if (qdelta_out) qdelta_out[row] = qdelta;
            float m = MASKED, ell = 0.0f;
            float *oi = out + (size_t)row * dv;
            for (size_t c = 0; c < dv; c++) oi[c] = 0.0f;
            const float *kb = k + (b * Hk + kvh) * S * d;
            const float *vb = v + (b * Hk + kvh) * S * dv;
            for (size_t j0 = 0; j0 < j_stop; j0 += block) {
                size_t j1 = j0 + block;
                if (j1 > S) j1 = S;
                size_t kj = j1 - j0;
                for (size_t c = 0; c < d; c++) {
                    float ssum = 0.0f;
                    for (size_t jj = j0; jj < j1; jj++) ssum += kb[jj * d + c];
                    kmean[c] = ssum / (float)kj;
                }
                for (size_t jj = j0; jj < j1; jj++) {
                    const float *kt = kb + jj * d;
                    float kpeak = 0.0f;
                    for (size_t c = 0; c < d; c++) {
                        float g = kt[c] - kmean[c];
                        float ag = g < 0.0f ? 0.0f - g : g;
                        if (ag > kpeak) kpeak = ag;
                    }
                    float kdelta = 1.0f;
                    if (kpeak > 0.0f) kdelta = kpeak / 127.0f;
                    int32_t acc_i = 0;
                    float shift = 0.0f;
                    for (size_t c = 0; c < d; c++) {
                        float km = kmean[c];
                        int qc = qhat[c];
                        float g = kt[c] - km;
                        int kc = q8(g / kdelta);
                        acc_i += qc * kc;
                        shift += ((float)qc * qdelta) * km;
                    }
                    float s = (float)acc_i * qdelta * kdelta + shift;
                    if (causal && jj > i) s = MASKED;
                    sc[jj - j0] = s;
                }
                float rowmax = MASKED;
                for (size_t kk = 0; kk < kj; kk++)
                    if (sc[kk] > rowmax) rowmax = sc[kk];
                float m_new = m;
                if (rowmax > m_new) m_new = rowmax;
                int live = !(m_new < MASKED * 0.5f);
                float alpha = live ? orc_expf(m - m_new) : 0.0f;
                for (size_t c = 0; c < dv; c++) {
                    float vpeak = 0.0f;
                    for (size_t jj = j0; jj < j1; jj++) {
                        float x = vb[jj * dv + c];
                        float ax = x < 0.0f ? 0.0f - x : x;
                        if (ax > vpeak) vpeak = ax;
                    }
                    vd[c] = vpeak > 0.0f ? vpeak / 127.0f : 1.0f;
                }
                float esum = 0.0f;
                for (size_t kk = 0; kk < kj; kk++) {
                    float p = live ? orc_expf(sc[kk] - m_new) : 0.0f;
                    esum += p;
                    float pr = rintf(p * 127.0f);
                    if (pr > 127.0f) pr = 127.0f;
                    if (pr < 0.0f) pr = 0.0f;
                    ph[kk] = (int8_t)pr;
                }
                ell = alpha * ell + esum;
                for (size_t c = 0; c < dv; c++) {
                    int32_t pv = 0;
                    for (size_t kk = 0; kk < kj; kk++) pv += (int32_t)ph[kk] * q8(vb[(j0 + kk) * dv + c] / vd[c]);
                    float prev = live ? oi[c] : 0.0f;
                    oi[c] = alpha * prev + (float)pv * (1.0f / 127.0f) * vd[c];
                }
                m = m_new;
            }
            for (size_t c = 0; c < dv; c++) oi[c] = oi[c] / ell;
        }
        free(qhat); free(kmean); free(sc); free(ph); free(vd);
    }
    return 0;
}

/* ======================================================================= */
/* block-scaled Sage variant (the north_star scheme; no reference symbol)  */
/* ======================================================================= */

#define QBLK 64
#define LOG2E_F 1.44269504088896341f

static int8_t q8clamp(float x) {
    float r = rintf(x);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    return (int8_t)r;
}

int orc_attention_sage_blk(const orc_attn_shape *sh, const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, int causal, float *out, int8_t *qhat_out,
                           float *qscale_out, int8_t *khat_out, float *kscale_out,
                           float *kmean_out, int threads) {
    size_t B = sh->batch, H = sh->n_heads, Hk = sh->n_kv_heads, S = sh->seq, d = sh->head_dim,
           dv = sh->val_dim;
    if (!Hk || H % Hk || !S || !d || !dv) return 1;
    size_t group = H / Hk, nblk = div_ceil(S, QBLK);
    float inv_sqrt_d = 1.0f / sqrtf((float)d);
    int8_t *khat = (int8_t *)malloc(B * Hk * S * d);
    float *ksc = (float *)malloc(sizeof(float) * B * Hk * nblk);
    float *kmean = (float *)malloc(sizeof(float) * B * Hk * d);
    int8_t *qhat = (int8_t *)malloc(B * H * S * d);
    float *qsc = (float *)malloc(sizeof(float) * B * H * nblk);
    float *vh = (float *)malloc(sizeof(float) * B * Hk * S * dv);
    /* K: whole-sequence channel mean (64-token chunk partials in token
     * order, then the chunks in order), smoothing, per-block INT8. */
#pragma omp parallel for num_threads(threads > 0 ? threads : 1)
    for (long bk = 0; bk < (long)(B * Hk); bk++) {
        const uint16_t *kb = k + (size_t)bk * S * d;
        float *mean = kmean + (size_t)bk * d;
        for (size_t c = 0; c < d; c++) {
            float tot = 0.0f;
            for (size_t blk = 0; blk < nblk; blk++) {
                float part = 0.0f;
                size_t t1 = (blk + 1) * QBLK < S ? (blk + 1) * QBLK : S;
                for (size_t t = blk * QBLK; t < t1; t++) part += orc_bf16_to_f32(kb[t * d + c]);
                tot += part;
            }
            mean[c] = tot / (float)S;
        }
        for (size_t blk = 0; blk < nblk; blk++) {
            size_t t0 = blk * QBLK, t1 = t0 + QBLK < S ? t0 + QBLK : S;
            float peak = 0.0f;
            for (size_t t = t0; t < t1; t++)
                for (size_t c = 0; c < d; c++) {
                    float g = fabsf(orc_bf16_to_f32(kb[t * d + c]) - mean[c]);
                    if (g > peak) peak = g;
                }
            float invs = peak > 0.0f ? 127.0f / peak : 0.0f;
            ksc[(size_t)bk * nblk + blk] = peak > 0.0f ? peak / 127.0f : 1.0f;
            for (size_t t = t0; t < t1; t++)
                for (size_t c = 0; c < d; c++)
                    khat[((size_t)bk * S + t) * d + c] =
                        q8clamp((orc_bf16_to_f32(kb[t * d + c]) - mean[c]) * invs);
        }
        const uint16_t *vb = v + (size_t)bk * S * dv;
        for (size_t t = 0; t < S * dv; t++)
            vh[(size_t)bk * S * dv + t] = f16_to_f32(f32_to_f16(orc_bf16_to_f32(vb[t])));
    }
    /* Q: 1/sqrt(d) folded in, per-block INT8. */
#pragma omp parallel for num_threads(threads > 0 ? threads : 1)
    for (long bh = 0; bh < (long)(B * H); bh++) {
        const uint16_t *qb = q + (size_t)bh * S * d;
        for (size_t blk = 0; blk < nblk; blk++) {
            size_t t0 = blk * QBLK, t1 = t0 + QBLK < S ? t0 + QBLK : S;
            float peak = 0.0f;
            for (size_t t = t0; t < t1; t++)
                for (size_t c = 0; c < d; c++) {
                    float x = fabsf(orc_bf16_to_f32(qb[t * d + c]) * inv_sqrt_d);
                    if (x > peak) peak = x;
                }
            float invs = peak > 0.0f ? 127.0f / peak : 0.0f;
            qsc[(size_t)bh * nblk + blk] = peak > 0.0f ? peak / 127.0f : 1.0f;
            for (size_t t = t0; t < t1; t++)
                for (size_t c = 0; c < d; c++)
                    qhat[((size_t)bh * S + t) * d + c] =
                        q8clamp((orc_bf16_to_f32(qb[t * d + c]) * inv_sqrt_d) * invs);
        }
    }
    long rows = (long)(B * H * S);
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float *sc = (float *)malloc(sizeof(float) * QBLK);
#pragma omp for schedule(dynamic, 16)
        for (long row = 0; row < rows; row++) {
            size_t bh = (size_t)row / S, i = (size_t)row % S, b = bh / H, h = bh % H;
            size_t bk = b * Hk + h / group;
            const int8_t *qi = qhat + (size_t)row * d;
            float qs = qsc[bh * nblk + i / QBLK];
            float *oi = out + (size_t)row * dv;
            for (size_t c = 0; c < dv; c++) oi[c] = 0.0f;
            float m = -INFINITY, ell = 0.0f;
            size_t kb_end = causal ? i / QBLK + 1 : nblk;
            for (size_t kb = 0; kb < kb_end; kb++) {
                size_t j0 = kb * QBLK, j1 = j0 + QBLK < S ? j0 + QBLK : S;
                float cs = (qs * ksc[bk * nblk + kb]) * LOG2E_F;
                float mb = -INFINITY;
                for (size_t j = j0; j < j1; j++) {
                    const int8_t *kj = khat + (bk * S + j) * d;
                    int32_t dot = 0;
                    for (size_t c = 0; c < d; c++) dot += (int32_t)qi[c] * (int32_t)kj[c];
                    float s = (float)dot * cs;
                    if (causal && j > i) s = -INFINITY;
                    sc[j - j0] = s;
                    if (s > mb) mb = s;
                }
                float m_new = m > mb ? m : mb;
                float alpha = exp2f(m - m_new);
                float sum = 0.0f;
                for (size_t j = j0; j < j1; j++) {
                    float p = exp2f(sc[j - j0] - m_new);
                    sum += p;
                    sc[j - j0] = f16_to_f32(f32_to_f16(p));
                }
                ell = alpha * ell + sum;
                for (size_t c = 0; c < dv; c++) {
                    float pv = 0.0f;
                    for (size_t j = j0; j < j1; j++) pv += sc[j - j0] * vh[(bk * S + j) * dv + c];
                    oi[c] = alpha * oi[c] + pv;
                }
                m = m_new;
            }
            for (size_t c = 0; c < dv; c++) oi[c] = oi[c] / ell;
        }
        free(sc);
    }
    if (qhat_out) memcpy(qhat_out, qhat, B * H * S * d);
    if (qscale_out) memcpy(qscale_out, qsc, sizeof(float) * B * H * nblk);
    if (khat_out) memcpy(khat_out, khat, B * Hk * S * d);
    if (kscale_out) memcpy(kscale_out, ksc, sizeof(float) * B * Hk * nblk);
    if (kmean_out) memcpy(kmean_out, kmean, sizeof(float) * B * Hk * d);
    free(khat); free(ksc); free(kmean); free(qhat); free(qsc); free(vh);
    return 0;
}

/* engine/mod.rs:781-800 Engine::logits (and the per-position prefill loop,
 * :1131-1147): one f32 accumulator per vocabulary row, t in order, each term
 * a separate multiply and add (built with -ffp-contract=off).  OpenMP over
 * rows only: each row's sum is sequential. */
void orc_head_logits(const float *head, size_t vocab, size_t d, const float *hidden, size_t batch,
                     float *logits, int threads) {
    if (threads > 0) omp_set_num_threads(threads);
    for (size_t b = 0; b < batch; b++) {
        const float *h = hidden + b * d;
#pragma omp parallel for schedule(static)
        for (size_t v = 0; v < vocab; v++) {
            const float *row = head + v * d;
            float acc = 0.0f;
            for (size_t t = 0; t < d; t++) acc += h[t] * row[t];
            logits[b * vocab + v] = acc;
        }
    }
}

/* ======================================================================= */
/* transformer trunk pieces (engine/mod.rs:878-945 and helpers)            */
/* ======================================================================= */

/* engine/mod.rs:1152-1160 rms_norm_into: f32 end to end; the sum of squares
 * is one sequential f32 fold, then / len, inv = 1 / sqrt(ss + eps as f32),
 * out = (v * inv) * w. */
void orc_rms_norm_f32(const float *x, const float *w, size_t n, double eps, float *out) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n;
    float inv = 1.0f / sqrtf(ss + (float)eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* engine/mod.rs:1169-1187 rope_rotate: rotate_half pairs (i, i + hd/2) of
 * every head_dim slice of v (n values) by pos * theta^(-2i/hd); the angle's
 * pow/sin/cos in f64, the rotation in f32. */
void orc_rope_rotate(float *v, size_t n, size_t hd, size_t pos, double theta) {
    size_t half = hd / 2;
    for (size_t base = 0; base + hd <= n; base += hd)
        for (size_t i = 0; i < half; i++) {
            double inv_freq = pow(theta, -(2.0 * (double)i) / (double)hd);
            double ang = (double)pos * inv_freq;
            float s = (float)sin(ang), c = (float)cos(ang);
            float a = v[base + i], b = v[base + half + i];
            v[base + i] = a * c - b * s;
            v[base + half + i] = b * c + a * s;
        }
}

/* engine/mod.rs:1073-1116 gqa_attention_scalar: one query position over a
 * row-major cache (k, v: [pos + 1][n_kv * hd]); per head, scores are the
 * sequential f32 dot times 1/sqrt(hd), softmax by max-subtracted exp with a
 * sequential denominator, output the sum of w * v over positions whose weight
 * is not zero.  scratch: pos + 1 floats. */
void orc_gqa_attention_scalar(const float *qh, const float *kc, const float *vc, size_t n_heads,
                              size_t n_kv, size_t hd, size_t pos, float *out, float *scratch) {
    size_t groups = n_heads / n_kv, kv_dim = n_kv * hd;
    float scale = 1.0f / sqrtf((float)hd);
    for (size_t i = 0; i < n_heads * hd; i++) out[i] = 0.0f;
    for (size_t h = 0; h < n_heads; h++) {
        size_t kvh = h / groups;
        const float *q = qh + h * hd;
        float maxs = -INFINITY;
        for (size_t p = 0; p <= pos; p++) {
            const float *k = kc + p * kv_dim + kvh * hd;
            float dot = 0.0f;
            for (size_t t = 0; t < hd; t++) dot += q[t] * k[t];
            scratch[p] = dot * scale;
            maxs = fmaxf(maxs, scratch[p]);
        }
        float denom = 0.0f;
        for (size_t p = 0; p <= pos; p++) {
            scratch[p] = expf(scratch[p] - maxs);
            denom += scratch[p];
        }
        float *oh = out + h * hd;
        for (size_t p = 0; p <= pos; p++) {
            float w = scratch[p] / denom;
            if (w == 0.0f) continue;
            const float *v = vc + p * kv_dim + kvh * hd;
            for (size_t t = 0; t < hd; t++) oh[t] += w * v[t];
        }
    }
}
