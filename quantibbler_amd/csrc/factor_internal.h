// factor_internal.h -- the device-resident factor layer shared by the layer
// upload / prefill GEMM (factor.hip) and the decode GEMV (decode.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "qbk_internal.h"

namespace qbk {

// One layer of a layer set in a prefill-GEMM launch (a device table built
// when the set is made): the stage's signs and scales, its dims, its first
// 128-row tile in the launch, and where its rows (stage 1: in the
// concatenated partials / t) or its activation columns (stage 2: in t) and
// its y block (stage 2: y0 rows of N tokens before it) sit.
struct G32SetLayer {
    const uint32_t *sg;
    const float *s2, *s1, *bias;
    size_t M_p, M_valid, K_p;
    uint32_t tile0;
    size_t col0, y0;
};

// One stage of one layer in a decode launch: an entry of a device-side
// table, so that one launch covers any number of layers of any shapes.
// Offsets count slices (128 k) and elements, so they do not depend on the
// batch; the byte offsets follow from the launch's column count.
struct Q4Layer {
    const uint32_t *bits;        // this stage's signs in the fp4 decode layout
    const float *s_in;           // stage 1: s2
    const float *s_out, *bias;   // stage 2: s1, bias
    const uint16_t *s_out_h, *bias_h;  // stage 2: the same as fp16 when every value is one, else null
    uint32_t rows_p, rows_valid; // this stage's output rows: padded (to 128), valid
    uint32_t ns, k_valid;        // this stage's 128-k slices, valid K
    uint32_t slice0;             // slices of this stage held by the layers before this one
    uint32_t tb_ns, tb_slice0;   // stage 1: stage 2's slices of this layer / before it
    uint32_t wg0;                // first workgroup of this layer in its stage's launch
    uint64_t act0, out0;         // element offsets of this layer's x (stage 1) / y (stage 2)
};

}  // namespace qbk

struct qbk_factor {
    int device, num_cus;
    size_t dout, din, r;
    size_t din_p, r_p, dout_p;  // padded for the MFMA tiles (64 / 128 / 128)
    uint8_t *ub_rows, *vbt_rows;      // reference per-row bitplanes, formed from the decode layout on the
                                      // first f64-face call (null until then)
    uint32_t *vt_g32, *u_g32;         // prefill layout: [r_p/128][din_p/64][64][4], [dout_p/128][r_p/64][64][4]
    size_t din_q, r_q;                // K of the fp4 decode layout: multiples of 128
    uint32_t *vt_q4, *u_q4;           // [r_p/64][din_q/128][64][4], [dout_p/64][r_q/128][64][4]
    float *s1, *s2, *bias;            // dout, din, dout (zeros when absent)
    bool scales_f16;                  // every s1, s2 and bias value is an fp16 value (a v2 qpk1 stream's)
    uint16_t *s1h, *s2h, *biash;      // then the same as fp16, the copies the decode GEMV streams (else null)
    bool bias_zero;                   // bias absent or all +0.0 (the decode skips its load)
    qbk::Q4Layer *q4_tab;             // device Q4Layer[2] of this layer alone: stage 1, stage 2
    std::vector<void *> allocs;
};

namespace qbk {

// decode.hip: the largest batch the factor linear (and the decoder block's
// batched decode step) routes to the fp4 GEMV -- beyond it, the prefill
// GEMM -- and the largest the GEMV serves at all.  Past 8 tokens each
// workgroup takes one 8-token column group.
constexpr size_t Q4_MAXB = 32;
constexpr size_t Q4_MAXB_KERNEL = 32;

// The two table entries of one layer decoded alone (offsets 0).
void q4_layer_entries(const qbk_factor *L, Q4Layer out[2]);

// Workspace bytes of a single-layer decode at `batch` (<= Q4_MAXB_KERNEL).
size_t q4_workspace(const qbk_factor *L, size_t batch);

// Single-layer decode: x [batch][din] (bf16, or f32 when xf32) ->
// y [batch][dout] (bf16 when ybf16, else f32), three launches on s.
int q4_run(const qbk_factor *L, size_t batch, const void *x, bool xf32, void *y, bool ybf16,
           void *ws, hipStream_t s);

// decode.hip: a layer set's three launches with f32 or bf16 x and y, and its
// workspace bytes.
int q4_set_run(const qbk_factor_set *S, const void *x, bool xf32, void *y, bool ybf16, void *ws, hipStream_t s);
size_t q4_set_workspace(const qbk_factor_set *S);
// The set at a batch of n <= Q4_MAXB_KERNEL tokens: x [layer][n][din],
// y [layer][n][dout].
size_t q4_set_workspace_batch(const qbk_factor_set *S, size_t n);
int q4_set_run_batch(const qbk_factor_set *S, size_t n, const void *x, bool xf32, void *y, bool ybf16, void *ws,
                     hipStream_t s);

// A batch-1 decode whose stage-1 operand a caller's kernel writes itself
// (q4_operand.h's runs, flat over the concatenated x: run t covers k = 16t
// .. 16t + 15 at global slice t / 8, two columns): where the operand and its
// scales go in the workspace ws (and, for a set, the layers' s2
// concatenated).  False when some din is not a multiple of 128 (no flat
// layout).  Then the two GEMV launches; resid (f32 y only) is added to y.
// A set's layers on the prefill GEMM for a batch of N tokens (x
// [N][din], the layers' shared input; y [layer][N][dout]) when
// q4_set_gemm_fits: three launches for the set.
bool q4_set_gemm_fits(const qbk_factor_set *S, size_t N);
size_t q4_set_gemm_workspace(const qbk_factor_set *S, size_t N);
int q4_set_gemm_run(const qbk_factor_set *S, size_t N, const void *x, bool xf32, void *y, bool ybf16, void *ws,
                    hipStream_t s);

bool q4_flat_operand(const qbk_factor *L, void *ws, uint8_t **op, uint8_t **sc);
bool q4_set_flat_operand(const qbk_factor_set *S, void *ws, uint8_t **op, uint8_t **sc, const float **s2cat);
int q4_run_staged(const qbk_factor *L, void *y, bool ybf16, const float *resid, void *ws, hipStream_t s);
int q4_set_run_staged(const qbk_factor_set *S, void *y, bool ybf16, void *ws, hipStream_t s);
// The same at a batch of n <= Q4_MAXB_KERNEL tokens: the operand holds 2n
// columns, token b's hi and lo in columns 2b, 2b + 1 (q4_run_slot's b).
bool q4_flat_operand_batch(const qbk_factor *L, size_t n, void *ws, uint8_t **op, uint8_t **sc);
bool q4_set_flat_operand_batch(const qbk_factor_set *S, size_t n, void *ws, uint8_t **op, uint8_t **sc,
                               const float **s2cat);
int q4_run_staged_batch(const qbk_factor *L, size_t n, void *y, bool ybf16, const float *resid, void *ws,
                        hipStream_t s);
int q4_set_run_batch_staged(const qbk_factor_set *S, size_t n, void *y, bool ybf16, void *ws, hipStream_t s);

// prefill.hip: a layer set on the prefill GEMM for a decode step's batch of
// N <= 64 tokens (layers sharing x, din % 8 == 0): the per-layer device
// tables (stage 1, stage 2), the workspace, and the three launches; y is
// [layer][N][dout].
void g32_set_tables(const qbk_factor *const *L, size_t n, G32SetLayer *t1, G32SetLayer *t2);
bool g32_set_fits(const qbk_factor *const *L, size_t n, size_t N);
size_t g32_set_workspace(const qbk_factor *const *L, size_t n, size_t N);
int g32_set_run(const qbk_factor *const *L, size_t n, const G32SetLayer *tab1, const G32SetLayer *tab2, size_t N,
                const void *x, bool xf32, void *y, bool ybf16, void *ws, hipStream_t s);

// gemm.hip: the prefill GEMM on the fp4 x fp8 MFMA, both stages in one
// launch over the decode's sign layout, no workspace: x [N][din] (bf16, or
// f32 when xf32) -> y [N][dout] (bf16 when ybf16, else f32), for layers of
// rank up to 2048.
// t_out (null, or [N][r_p] bf16): t as well, zero past r.  resid (null, or
// f32 [N][dout], with f32 y only): y = resid added to the layer's output.
// s2 (null, or [din]): in place of the layer's s2 (ones for an x that
// already holds z = bf16(s2 x)).
bool q4g_fits(const qbk_factor *L, size_t N);
int q4g_run(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16, uint16_t *t_out,
            hipStream_t s, const float *resid = nullptr, const float *s2 = nullptr);
// The factor linear past the decode GEMV's batches: the fused GEMM where it
// applies (its workspace: t bf16 [N][r_p], left there), else the two-stage
// GEMM below; gemm_workspace gives the bytes ws must hold.
bool q4g_use(const qbk_factor *L, size_t N);
size_t gemm_workspace(const qbk_factor *L, size_t N);
int gemm_run(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16, void *ws,
             hipStream_t s);

// prefill.hip: the sign layout of the prefill GEMM (rows_p a multiple of
// 128, bits_p of 64), its workspace, and the two-stage GEMM for N tokens:
// x [N][din] (bf16, or f32 when xf32) -> y [N][dout].
void g32_repack(const uint8_t *rows, size_t n_rows, size_t n_bits, size_t rows_p, size_t bits_p,
                uint32_t *out);
size_t g32_workspace(const qbk_factor *L, size_t N);
int g32_run(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16, void *ws,
            hipStream_t s);

// apply's fp32 serving on the device (factor.hip): the reference's row
// bitplanes formed once, then one token's f64 product (scratch: din + r + dout
// doubles).
int factor_rows_ready(const qbk_factor *L, hipStream_t s);
int factor_apply_f64_dev(qbk_ctx *ctx, const qbk_factor *L, const float *x, float *y, double *scratch,
                         hipStream_t s);

}  // namespace qbk
