/*
 * qbk_oracle.h -- CPU restatement of quantibbler-kernels' hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code: it is the checker the parity tests, smoke() and the
 * cpu_baseline leg of bench.py compare the HIP library against.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Reference root: donicrosby/quantibbler.
 */
#ifndef QBK_ORACLE_H
#define QBK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Every fallible function returns 0 on success, 1 on a validation error, and
 * writes the reference's error text into err[0..errlen). */

/* ---- bit layout: crates/quantibbler-kernels/src/core.rs:129-240 ---------- */
int orc_pack_bits(const int8_t *factor, size_t factor_len, size_t n_rows, size_t n_cols,
                  uint8_t *out, char *err, size_t errlen);
int orc_unpack_bits(const uint8_t *packed, size_t packed_len, size_t n_rows, size_t n_bits,
                    int8_t *out, char *err, size_t errlen);
int orc_validate_packed(size_t packed_len, size_t n_rows, size_t n_bits, size_t *n_words,
                        char *err, size_t errlen);
void orc_sign_estimate(const double *x, size_t n, int8_t *out);

/* ---- bf16 (half 2.7.1 bf16::from_f32 RNE, dtype.rs:77-92) ----------------- */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t b);

/* ---- sequential products: core.rs:202-317 (dtype 0=f64 1=f32 2=bf16) ----- */
int orc_packed_matvec(int dtype, const uint8_t *packed, size_t packed_len, size_t n_rows,
                      size_t n_bits, const void *vec, size_t vec_len, void *out,
                      char *err, size_t errlen);
int orc_packed_matmul(int dtype, const uint8_t *packed, size_t packed_len, size_t n_rows,
                      size_t n_bits, const void *mat, size_t mat_len, size_t n_cols,
                      void *out, char *err, size_t errlen);

/* ---- SIMD+rayon CPU face restated (fast.rs:28-158), OpenMP over 64-row blocks */
int orc_fast_packed_matvec_f64(const uint8_t *packed, size_t packed_len, size_t n_rows,
                               size_t n_bits, const double *vec, size_t vec_len, double *out,
                               int threads, char *err, size_t errlen);
int orc_fast_packed_matmul_f64(const uint8_t *packed, size_t packed_len, size_t n_rows,
                               size_t n_bits, const double *mat, size_t mat_len, size_t n_cols,
                               double *out, int threads, char *err, size_t errlen);

/* ---- qpk1 container (crates/quantibbler-qpk1/src/lib.rs:152-320) ---------- */
typedef struct {
    uint32_t version, dtype_tag;
    size_t dout, din, r;
    size_t s1_off, s2_off, bias_off, ub_off, vb_off; /* byte offsets in the stream */
} orc_qpk1_header;
int orc_qpk1_parse(const uint8_t *bytes, size_t len, orc_qpk1_header *hdr, double *s1,
                   double *s2, double *bias, char *err, size_t errlen);
size_t orc_qpk1_expected_size(size_t dout, size_t din, size_t r, int itemsize, int with_bias);

/* ---- engine layout repack: crates/quantibbler-server/src/engine/mod.rs:258-289 */
void orc_container_to_rows(const uint8_t *packed, size_t n_rows, size_t r, uint8_t *out);
void orc_container_to_rows_transposed(const uint8_t *packed, size_t din, size_t r,
                                      uint8_t *out);

/* ---- factor linear composite: engine/mod.rs:393-481 ------------------------ */
/* ub_rows: dout x ceil(r/8); vb_t_rows: r x ceil(din/8).  x is f32[din].      */
/* serving 0 = Fp32 (f64 matvecs, y = f32(u)*s1 + b); 1 = Bf16 (apply_bf16).   */
int orc_factor_apply(int serving, size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                     const uint8_t *vb_t_rows, const float *s1, const float *s2,
                     const float *bias, const float *x, float *y, int fast, int threads);
/* Batched bf16 composite, one column per token (the device GEMM's contract):
 * z = bf16(s2*x); t = bf16(Vb^T z); u = bf16(Ub t); y = f32(u)*s1 + b.
 * x is token-major bf16 [batch][din]; y is f32 [batch][dout]; t_out (optional)
 * receives the bf16 intermediate [batch][r].                                  */
void orc_factor_apply_bf16_batch(size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                                 const uint8_t *vb_t_rows, const float *s1, const float *s2,
                                 const float *bias, const uint16_t *x, size_t batch, float *y,
                                 uint16_t *t_out, int threads);

/* ---- attention --------------------------------------------------------------- */
typedef struct {
    size_t batch, n_heads, n_kv_heads, seq, head_dim, val_dim;
} orc_attn_shape;

/* exact tiled attention, f64: src/quantibbler/kernels/attention_tiled.py:76-180 */
int orc_attention_tiled_f64(const orc_attn_shape *s, const double *q, const double *k,
                            const double *v, int causal, size_t block, double *out,
                            double *lse);
/* [SA] s4 quantized reference, NumPy (f64) semantics:
 * src/quantibbler/kernels/attention_sage.py:206-350                          */
int orc_attention_sage_np_f64(const orc_attn_shape *s, const double *q, const double *k,
                              const double *v, int causal, size_t block, double *out);
/* The same scheme in the device face's f32 operation order:
 * crates/quantibbler-kernels/src/gpu_attention.rs:89-396.  Uses orc_expf.
 * Optional stage outputs (NULL to skip): qhat [rows*d] i8, qdelta [rows] f32. */
int orc_attention_sage_dev_f32(const orc_attn_shape *s, const float *q, const float *k,
                               const float *v, int causal, size_t block, float *out,
                               int8_t *qhat, float *qdelta, int threads);
/* exp for the f32 reference scheme: Cody-Waite ln2 reduction + degree-7 Taylor. */
float orc_expf(float x);

/* Block-scaled variant (no reference symbol; the north_star scheme):
 * whole-sequence K channel mean, INT8 Q/K with one scale per 64-token block
 * per head, fp16 P and V, f32 statistics, base-2 online softmax.
 * q,k,v are bf16 bit patterns; out is f32 (before the device's bf16 store).
 * Stage outputs (NULL to skip): khat [B*Hkv*S*d] i8, kscale [B*Hkv*nblk],
 * qhat [B*H*S*d] i8, qscale [B*H*nblk], kmean [B*Hkv*d].                     */
int orc_attention_sage_blk(const orc_attn_shape *s, const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, int causal, float *out, int8_t *qhat,
                           float *qscale, int8_t *khat, float *kscale, float *kmean,
                           int threads);

/* engine/mod.rs:781-800 Engine::logits: sequential f32 sum per row. */
void orc_head_logits(const float *head, size_t vocab, size_t d, const float *hidden, size_t batch,
                     float *logits, int threads);

/* transformer trunk pieces (engine/mod.rs:1073-1187) */
void orc_rms_norm_f32(const float *x, const float *w, size_t n, double eps, float *out);
void orc_rope_rotate(float *v, size_t n, size_t hd, size_t pos, double theta);
void orc_gqa_attention_scalar(const float *qh, const float *kc, const float *vc, size_t n_heads,
                              size_t n_kv, size_t hd, size_t pos, float *out, float *scratch);

#ifdef __cplusplus
}
#endif

#endif
