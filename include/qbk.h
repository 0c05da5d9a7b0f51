/*
 * qbk.h -- C ABI of libqbk, the MI355X (gfx950) implementation of the two
 * quantibbler-kernels hot paths:
 *
 *   1. the binary latent-factor linear  y = s1 . (Ub (Vb^T (s2 . x))) + b
 *      over 1-bit sign matrices (decode GEMV and prefill GEMM), and
 *   2. SageAttention (INT8 Q.K^T, online softmax, tiled P.V).
 *
 * Every entry point names the reference interface it replaces
 * (donicrosby/quantibbler, file:line).  Plain pointers and sizes only.
 *
 * Conventions
 *   - Return value: QBK_OK (0) or a QBK_ERR_* code.  On error nothing is
 *     written to the outputs and qbk_last_error() returns the message; for
 *     validation errors that text is the reference's KernelError text
 *     (core.rs, gpu.rs, gpu_attention.rs) verbatim.
 *   - "host" entry points take host buffers and block until the result is in
 *     the output buffer (GpuContext semantics: copy in, launch, copy out).
 *   - "_dev" entry points take device pointers, enqueue on `stream` (a
 *     hipStream_t, NULL = the null stream) and return without waiting.
 *   - bf16 values cross as uint16_t bit patterns (lib.rs:245-261).
 *   - A qbk_ctx may be shared by threads; calls are independent (each host
 *     call uses its own stream and buffers; device calls use the caller's).
 */
#ifndef QBK_H
#define QBK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    QBK_OK = 0,
    QBK_ERR_VALIDATION = 1, /* core::KernelError from input validation      */
    QBK_ERR_DEVICE = 2,     /* a HIP call failed (per-call device error)     */
    QBK_ERR_INIT = 3        /* no usable device (gpu.rs GPU_INIT_HINT)       */
};

/* Dense operand dtype tag: dtype.rs:93-130 Dtype {F64, F32, Bf16}. */
enum { QBK_F64 = 0, QBK_F32 = 1, QBK_BF16 = 2 };

typedef struct qbk_ctx qbk_ctx;
typedef struct qbk_factor qbk_factor;

/* ---- meta ---------------------------------------------------------------- */

/* lib.rs:94-97 backend_version() */
const char *qbk_backend_version(void);
/* Message of the calling thread's last failed call (core.rs:31 KernelError). */
const char *qbk_last_error(void);
/* dtype.rs:110-119 Dtype::from_name: "float64" | "float32" | "bfloat16";
 * an unknown name is refused, naming the value. */
int qbk_dtype_from_name(const char *name, int *dtype_out);

/* ---- host-side bit layout (core.rs) --------------------------------------- */

/* core.rs:129-162 pack_bits: +-1 factor (n_rows x n_cols, row-major) ->
 * n_rows x ceil(n_cols/8) bytes, LSB-first, +1 -> 1, pad bits 0. */
int qbk_pack_bits(const int8_t *factor, size_t factor_len, size_t n_rows, size_t n_cols,
                  uint8_t *out);
/* core.rs:166-189 unpack_bits: pad bits ignored. */
int qbk_unpack_bits(const uint8_t *packed, size_t packed_len, size_t n_rows, size_t n_bits,
                    int8_t *out);
/* core.rs:223-240 validate_packed; *n_words = ceil(n_bits/8). */
int qbk_validate_packed(size_t packed_len, size_t n_rows, size_t n_bits, size_t *n_words);
/* core.rs sign_estimate: x >= 0 (incl. -0.0) -> +1, else -1. */
void qbk_sign_estimate(const double *x, size_t n, int8_t *out);

/* core.rs:318-424 joint_itq (the compressor's alternating Procrustes; host
 * code, as the reference's): u_hat (dout x rank), v_hat (din x rank) f64
 * row-major -> u_t, v_t +-1 int8 of the same shapes, the iteration count and
 * whether ||R_new - R||_F <= tol stopped it (tol == 0 runs max_iter).  The
 * reference's defaults are max_iter 50, tol 1e-12, seed 0. */
int qbk_joint_itq(const double *u_hat, size_t u_len, const double *v_hat, size_t v_len, size_t dout,
                  size_t din, size_t rank, size_t max_iter, double tol, uint64_t seed, int8_t *u_t,
                  int8_t *v_t, size_t *n_iter, int *converged);

/* ---- device context (gpu.rs:76-189 GpuContext) --------------------------- */

/* gpu.rs:85-101 GpuContext::init_at(device_index); failure -> QBK_ERR_INIT
 * with the GPU_INIT_HINT-style message. */
int qbk_ctx_create(int device_index, qbk_ctx **out);
void qbk_ctx_destroy(qbk_ctx *ctx);
/* gpu.rs:187-189 gpu_available() */
int qbk_gpu_available(void);

/* ---- packed products ------------------------------------------------------ */

/* gpu.rs:116-185 GpuContext::packed_matvec generalised to the three dtypes of
 * dispatch.rs:81-92 packed_matvec_dyn.  out[i] = sum_k s(i,k) vec[k] in the
 * dtype's accumulator (f64, f32, f32 for bf16), summed in element order, so
 * results are bit-identical to core::packed_matvec.  At f64 (the reference's
 * device face) a shape past the u32 index ceiling, n_rows * ceil(n_bits/8) or
 * n_rows above 4294967295, is refused with gpu.rs:127-137's text before any
 * device use. */
int qbk_packed_matvec(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t packed_len,
                      size_t n_rows, size_t n_bits, const void *vec, size_t vec_len, void *out);
/* dispatch.rs:95-109 packed_matmul_dyn / core.rs:288-317: output n_rows x k,
 * k = mat_len / max(n_bits,1), element (i,j) = sum_t s(i,t) mat[t*n_cols + j]
 * in element order.  An n_cols that would index past mat_len is a
 * validation error (the reference would panic). */
int qbk_packed_matmul(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t packed_len,
                      size_t n_rows, size_t n_bits, const void *mat, size_t mat_len,
                      size_t n_cols, void *out);
/* Device-pointer forms of the two above (same arithmetic); k_cols = output
 * width.  packed is n_rows x ceil(n_bits/8) bytes. */
int qbk_packed_matvec_dev(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t n_rows,
                          size_t n_bits, const void *vec, void *out, void *stream);
int qbk_packed_matmul_dev(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t n_rows,
                          size_t n_bits, const void *mat, size_t k_cols, size_t n_cols, void *out,
                          void *stream);

/* ---- binary factor linear (engine/mod.rs:313-481 PackedLayer) ------------ */

/* Upload one qpk1 layer stream (quantibbler-qpk1 lib.rs:229-320 parse; v1 or
 * v2, f16 or f32 scales) and repack it once into the device layout
 * (engine/mod.rs:342-381 PackedLayer::from_layer).  Parse errors carry the
 * reference's text. */
int qbk_factor_from_qpk1(qbk_ctx *ctx, const uint8_t *stream, size_t len, qbk_factor **out);
/* Same, from the engine's per-row bitplanes (engine/mod.rs:313-340 fields):
 * ub_rows = dout x ceil(r/8), vb_t_rows = r x ceil(din/8); bias may be NULL
 * (a legacy v1 layer: the zero map). */
int qbk_factor_from_rows(qbk_ctx *ctx, size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                         const uint8_t *vb_t_rows, const float *s1, const float *s2,
                         const float *bias, qbk_factor **out);
void qbk_factor_destroy(qbk_factor *layer);
int qbk_factor_dims(const qbk_factor *layer, size_t *dout, size_t *din, size_t *r);
/* Bytes of device workspace qbk_factor_linear_dev needs at this batch. */
size_t qbk_factor_workspace_size(const qbk_factor *layer, size_t batch);
/* Device factor linear over `batch` tokens (the bf16 serving composite,
 * engine/mod.rs:449-460 apply_bf16, batched):
 *   z = bf16(s2*x); t = bf16(Vb^T z); u = bf16(Ub t); y = f32(u)*s1 + b
 * x: bf16 [batch][din] (token-major); y: [batch][dout] as f32 (y_dtype
 * QBK_F32) or bf16 (QBK_BF16, one more RNE).  batch == 1 runs the decode
 * GEMV, larger batches the MFMA GEMM.  Accumulation is f32. */
int qbk_factor_linear_dev(qbk_ctx *ctx, const qbk_factor *layer, const uint16_t *x, size_t batch,
                          void *y, int y_dtype, void *workspace, size_t workspace_size,
                          void *stream);
/* No counterpart in the reference: qbk_factor_linear_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * or harnesses that forbid hipMalloc).  It allocates nothing: the workspace
 * is a file-scope device array of QBK_NOALLOC_SCRATCH_BYTES (32 MiB) that
 * each GPU the library runs on holds until the process ends.  A call whose
 * workspace (qbk_factor_workspace_size) exceeds that is refused with a
 * validation error.  Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU race, so order them (one stream).  Same
 * arithmetic and results as qbk_factor_linear_dev. */
#define QBK_NOALLOC_SCRATCH_BYTES (32u << 20)
int qbk_factor_linear_noalloc_dev(qbk_ctx *ctx, const qbk_factor *layer, const uint16_t *x,
                                  size_t batch, void *y, int y_dtype, void *stream);
/* Host form of PackedLayer::apply / apply_bf16 (engine/mod.rs:393-460) on
 * the device: x f32 [batch][din] -> y f32 [batch][dout].  serving QBK_BF16 is
 * apply_bf16's composite; serving QBK_F32 is apply's (f64 matvecs). */
int qbk_factor_apply(qbk_ctx *ctx, const qbk_factor *layer, int serving, const float *x,
                     size_t batch, float *y);

/* A set of layers (any shapes) decoded together at batch 1, three launches
 * for the whole set: independent projections such as q/k/v/o/gate/up/down
 * of one or many decoder layers.  The set keeps a device descriptor table;
 * the layers must outlive it.  No counterpart in the reference (its engine
 * applies one layer per call). */
typedef struct qbk_factor_set qbk_factor_set;
int qbk_factor_set_create(qbk_ctx *ctx, const qbk_factor *const *layers, size_t n_layers,
                          qbk_factor_set **out);
void qbk_factor_set_destroy(qbk_factor_set *set);
size_t qbk_factor_set_workspace_size(const qbk_factor_set *set);
/* y_i = layer_i(x_i) at batch 1 for every layer i of the set (device
 * pointers): x bf16 is the concatenation of the x_i (layer i's din values
 * start after the din of layers 0..i-1), y bf16 likewise of the y_i. */
int qbk_factor_set_decode_dev(qbk_ctx *ctx, const qbk_factor_set *set, const uint16_t *x,
                              uint16_t *y, void *workspace, size_t workspace_size, void *stream);
/* One of the three launches of qbk_factor_set_decode_dev (for callers that
 * interleave work or time phases): phase 1 turns every x into stage 1's fp8
 * operand in the workspace; phase 2 runs stage 1 and writes
 * t = bf16(Vb^T bf16(s2*x)) as stage 2's fp8 operand; phase 3 runs stage 2
 * and writes y.  No counterpart in the reference (its apply is one call). */
int qbk_factor_set_stage_dev(qbk_ctx *ctx, const qbk_factor_set *set, int stage,
                             const uint16_t *x, uint16_t *y, void *workspace,
                             size_t workspace_size, void *stream);
/* The set at a batch of n tokens (1 .. 32; engine/mod.rs:1377-1476 decodes a
 * batch of sequences through every projection): x bf16 [layer][n][din_i]
 * (layer i's n rows start after layers 0..i-1's), y bf16 [layer][n][dout_i]
 * likewise.  The signs are read once for the batch: 16 operand columns (8
 * tokens) per fp4 MFMA, the column groups against the same sign registers.
 * Row b of y_i is bit-identical to the layer applied to row b alone.  Beyond
 * batch 8 the column groups hold 280-510 VGPRs a wave (one or two waves a
 * SIMD), so past batch ~12 the prefill GEMM of each layer is faster. */
size_t qbk_factor_set_workspace_size_batch(const qbk_factor_set *set, size_t n);
int qbk_factor_set_decode_batch_dev(qbk_ctx *ctx, const qbk_factor_set *set, size_t n, const uint16_t *x,
                                    uint16_t *y, void *workspace, size_t workspace_size, void *stream);
/* A set whose layers read the same input (q/k/v, gate/up: engine/mod.rs:
 * 901-906, :928-929) at a batch of n tokens (1 .. 64) on the prefill GEMM,
 * one launch per stage for the whole set: x bf16 [n][din] (every layer's
 * din equal and a multiple of 8), y bf16 [layer][n][dout_i].  Sums in MFMA
 * order (bit-identical to the reference on integer-exact inputs, within the
 * stage bounds otherwise); the decoder block's batched step runs its q/k/v
 * and gate/up this way beyond batch 8.  No counterpart in the reference (it
 * applies each layer to one token at a time). */
size_t qbk_factor_set_shared_workspace_size(const qbk_factor_set *set, size_t n);
int qbk_factor_set_shared_dev(qbk_ctx *ctx, const qbk_factor_set *set, size_t n, const uint16_t *x, uint16_t *y,
                              void *workspace, size_t workspace_size, void *stream);


/* ---- decoder block (engine/mod.rs:878-945) --------------------------------- */

/* One decoder block of Engine::transformer at one position, bf16 serving,
 * the sage decode attention (engine/mod.rs:984-1030) on a kept state:
 *   x = bf16(rmsnorm(bf16(h)) w_in); q, k, v = apply_bf16(x); with q/k
 *   norms, q and k per-head norm_apply (engine/mod.rs:854-876, :907-910);
 *   RoPE (engine/mod.rs:1169-1187) at pos; k, v appended to the block's
 *   cache; a = attention over pos + 1 rows; h1 = o(a) + h;
 *   x2 = bf16(rmsnorm(bf16(h1)) w_post); h' = down(g u / (1 + exp(-g))) + h1
 * with g, u = gate(x2), up(x2).  layers: q, k, v, o, gate, up, down (the
 * block borrows them; they must outlive it).  input_norm / post_norm hold
 * d_model floats each (their lengths are checked); q_norm and k_norm are
 * both NULL (no per-head norms, Llama-style) or both head_dim floats
 * (qk_norm_len).  The block owns its KV cache of `capacity` rows and the
 * attention state.  Its norms' sums run as trees and its exp is the
 * device's, so the block agrees with the reference to a tolerance, not bit
 * for bit.  Calls on one block must be ordered. */
typedef struct qbk_block qbk_block;
int qbk_block_create(qbk_ctx *ctx, const qbk_factor *const *layers, const float *input_norm,
                     size_t input_norm_len, const float *post_norm, size_t post_norm_len,
                     const float *q_norm, const float *k_norm, size_t qk_norm_len, size_t n_heads,
                     size_t n_kv_heads, size_t head_dim, double rope_theta, double rms_norm_eps,
                     size_t capacity, size_t block_size, qbk_block **out);
void qbk_block_destroy(qbk_block *block);
/* h: f32 [d_model] on the device, replaced by the block's output; pos = the
 * number of positions already in the block's cache (0 for a new sequence,
 * after qbk_block_reset).  A pos beyond the positions the block holds is a
 * validation error; a smaller pos rewinds (the cache rows from pos on are
 * overwritten and the attention state is rebuilt). */
int qbk_block_decode_dev(qbk_ctx *ctx, qbk_block *block, float *h, size_t pos, void *stream);
int qbk_block_reset(qbk_block *block);
/* Prefill: n tokens of a new sequence at positions 0 .. n - 1 in one pass
 * (engine/mod.rs:811-822 forward_prefill runs them one at a time; each
 * token's row here is the same block arithmetic): h f32 [n][d_model] rows on
 * the device, replaced by the block's outputs.  The projections run at batch
 * n (the bf16-MFMA GEMM beyond batch 8), the attention is the causal
 * block-scaled SageAttention over the n tokens (head_dim 128), and k, v fill
 * cache rows 0 .. n - 1, so that decoding continues at position n (its
 * attention state rebuilds from the cache on the first step).  The caller
 * supplies `workspace` of at least qbk_block_prefill_workspace_size(block, n)
 * bytes; nothing is allocated. */
size_t qbk_block_prefill_workspace_size(const qbk_block *block, size_t n_tokens);
int qbk_block_prefill_dev(qbk_ctx *ctx, qbk_block *block, float *h, size_t n_tokens, void *workspace,
                          size_t workspace_size, void *stream);
/* The block's KV cache (device, f32 [n_seqs][capacity][n_kv_heads * head_dim]
 * each; sequence 0 first).  After writing rows 0 .. rows[i] - 1 of sequence i
 * through these pointers, qbk_block_set_filled declares them: decoding then
 * continues at position rows[i], and the attention state rebuilds its codes
 * from the cache on that step (as after a prefill). */
int qbk_block_cache(const qbk_block *block, float **k_cache, float **v_cache);
/* Sequences 0 .. n - 1 hold rows[i] cache rows written by the caller; their
 * attention state covers none of them yet.  No counterpart in the reference
 * (its KvCache is filled only by its own steps, engine/mod.rs:1224-1268). */
int qbk_block_set_filled(qbk_block *block, const size_t *rows, size_t n);
/* engine/mod.rs:953-968 Engine::gqa_attention's face, chosen once when the
 * engine loads (QUANTIBBLER_ATTN): QBK_ATTN_SAGE (the default) runs the
 * reference-scheme sage decode attention (the gpu:sage face, :984-1030) on a
 * kept state; QBK_ATTN_EXACT the exact f32 attention over cache rows
 * 0 .. pos (the gpu:tiled face, :1041-1067, which the scalar default face
 * computes too, :1073-1116), read in place in the row-major cache, and the o
 * projection from its f32 output.  The exact face serves qbk_block_decode_dev
 * and qbk_block_prefill_dev (sequence 0; its prefill runs forward_prefill's
 * per-token loop, :811-822); the batched and device-position steps refuse
 * it.  Switching keeps the cache: the sage state rebuilds the rows the exact
 * face wrote on its next step. */
enum { QBK_ATTN_SAGE = 0, QBK_ATTN_EXACT = 1 };
int qbk_block_set_attention_face(qbk_block *block, int face);
/* engine/mod.rs ServingDtype, chosen when the engine loads: QBK_BF16 (the
 * default: apply_bf16 on the decode GEMV / prefill GEMM, bf16-rounded norms)
 * or QBK_F32 -- apply's f64 products (z = f64(s2 x), Vb^T z and Ub t in
 * element order, y = f32(u) s1 + b; :393-436), norm_apply and per_head_norm
 * in f32 without bf16 roundings (:837-876), on either attention face.  The
 * first QBK_F32 call forms the layers' row bitplanes and the block's f64
 * scratch (the only allocations).  fp32 serving serves qbk_block_decode_dev
 * and qbk_block_prefill_dev (sequence 0, the prefill token by token); the
 * batched and device-position steps refuse it. */
int qbk_block_set_serving(qbk_ctx *ctx, qbk_block *block, int serving);

/* Batched serving (engine/mod.rs:1377-1476 steps a batch of sequences through
 * the trunk; each sequence keeps its own cache): a block holding n_seqs
 * (1 .. 64) independent sequences, each with a KV cache of `capacity` rows
 * and its own attention state.  qbk_block_create is this with n_seqs = 1,
 * and qbk_block_decode_dev / qbk_block_prefill_dev act on sequence 0. */
int qbk_block_create_seqs(qbk_ctx *ctx, const qbk_factor *const *layers, const float *input_norm,
                          size_t input_norm_len, const float *post_norm, size_t post_norm_len,
                          const float *q_norm, const float *k_norm, size_t qk_norm_len, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, double rope_theta, double rms_norm_eps,
                          size_t capacity, size_t block_size, size_t n_seqs, qbk_block **out);
/* qbk_block_prefill_dev for sequence `seq`. */
int qbk_block_prefill_seq_dev(qbk_ctx *ctx, qbk_block *block, size_t seq, float *h, size_t n_tokens,
                              void *workspace, size_t workspace_size, void *stream);
/* One decode position of each of sequences 0 .. n - 1 (n <= n_seqs):
 * h f32 [n][d_model] on the device (row i is sequence i's token), replaced
 * by the block's outputs; pos (host, n entries) as qbk_block_decode_dev's
 * pos per sequence.  The projections run at batch n (the fp4 decode GEMV up
 * to batch 8, the bf16-MFMA GEMM beyond) and the attention steps every
 * sequence's kept state in one set of launches.  `workspace` of at least
 * qbk_block_decode_batch_workspace_size(block, n) bytes; nothing is
 * allocated. */
size_t qbk_block_decode_batch_workspace_size(const qbk_block *block, size_t n);
int qbk_block_decode_batch_dev(qbk_ctx *ctx, qbk_block *block, float *h, const size_t *pos, size_t n,
                               void *workspace, size_t workspace_size, void *stream);

/* Decode steps whose positions live in device memory, so that a step
 * captured once in a HIP graph serves every later position (the reference
 * steps its engine from the host, engine/mod.rs:1377-1476; these take the
 * host out of the loop).  pos: device uint32, one per sequence (n entries
 * for the batched form), read when the step runs: the position the step
 * writes (as qbk_block_decode_dev's pos).  The attention steps a kept state
 * that must hold every complete key block before that position -- as after
 * an eager step at pos - 1 -- and keeps the same arithmetic, so each step is
 * bit-identical to the eager step at that position; a state that does not
 * cover the cached rows (right after a prefill or qbk_block_set_filled) is a
 * validation error.  A position at or past the capacity skips the cache and
 * attention (the attention output is then 0 and the step's output has no
 * meaning).  Needs the grouped decode attention (head_dim a multiple of
 * 16, up to 16 query heads a kv head, key blocks of up to 64 tokens; a
 * validation error otherwise).  These steps do not update the block's host
 * record of cached positions: qbk_block_set_positions sets it (sequence i
 * holding pos[i] positions, its attention state stepped through them) before
 * the next eager step. */
int qbk_block_decode_pos_dev(qbk_ctx *ctx, qbk_block *block, float *h, const uint32_t *pos, void *stream);
int qbk_block_decode_batch_pos_dev(qbk_ctx *ctx, qbk_block *block, float *h, const uint32_t *pos, size_t n,
                                   void *workspace, size_t workspace_size, void *stream);
int qbk_block_set_positions(qbk_block *block, const size_t *pos, size_t n);

/* ---- trunk pieces around the blocks (engine/mod.rs:763-800, 943) ---------- */

/* Engine::embed (engine/mod.rs:768-778): out[i] = table[tokens[i]], f32
 * rows of d_model, table on the device (vocab x d_model).  The host form
 * takes host token ids and refuses an id outside the vocabulary with the
 * reference's text; it returns once the rows are written.  The device form
 * takes device ids and cannot refuse: an out-of-range id gets a NaN row. */
int qbk_embed(qbk_ctx *ctx, const float *table, size_t vocab, size_t d_model, const int32_t *tokens,
              size_t n, float *out, void *stream);
int qbk_embed_dev(qbk_ctx *ctx, const float *table, size_t vocab, size_t d_model, const int32_t *tokens,
                  size_t n, float *out, void *stream);
/* The final norm (engine/mod.rs:943, norm_apply at bf16 serving, :837-852):
 * per row, bf16 operand, f32 mean square, out = bf16(b * inv * w) held as f32
 * (device pointers, rows x d). */
int qbk_rms_norm_dev(qbk_ctx *ctx, const float *x, size_t rows, size_t d, const float *w, double eps,
                     float *out, void *stream);
/* The same at fp32 serving (norm_apply's Fp32 arm, rms_norm_into as is):
 * no bf16 roundings of the operand and the output. */
int qbk_rms_norm_f32_dev(qbk_ctx *ctx, const float *x, size_t rows, size_t d, const float *w, double eps,
                         float *out, void *stream);
/* sampler.rs:4-15 greedy: per row of `vocab` logits, the first index of the
 * largest value (NaN never wins; 0 when nothing beats -inf). */
int qbk_argmax_dev(qbk_ctx *ctx, const float *logits, size_t rows, size_t vocab, int32_t *out,
                   void *stream);
/* pos[i] += 1 for i < n (device uint32): a greedy loop's positions after a
 * device-position step (no reference counterpart: the reference's loop
 * counts positions on the host). */
int qbk_positions_advance_dev(qbk_ctx *ctx, uint32_t *pos, size_t n, void *stream);

/* ---- attention (gpu_attention.rs) ----------------------------------------- */

/* gpu_attention.rs:402-411 AttentionShape */
typedef struct {
    size_t batch, n_heads, n_kv_heads, seq_q, seq_kv, head_dim, val_dim;
} qbk_attn_shape;

/* gpu_attention.rs:451-570 GpuContext::attention (over cubek-attention's
 * launch_ref in the reference): exact f32 attention, q (B,H,Sq,d) unscaled
 * (1/sqrt(d) applied here), k (B,Hkv,Skv,d), v (B,Hkv,Skv,dv) -> out
 * (B,H,Sq,dv); query head h reads kv head h / (H/Hkv); causal masks key j
 * of query i when j + Sq > i + Skv (so Sq = 1 sees every key), and a row
 * with every key masked is NaN.  Same validation messages and u32 index
 * ceiling as the reference face.  The quality reference of the quantised
 * schemes, and the engine's tiled decode face (engine/mod.rs:1041-1067). */
int qbk_attention(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, size_t q_len, const float *k,
                  size_t k_len, const float *v, size_t v_len, int causal, float *out);
int qbk_attention_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, const float *k,
                      const float *v, int causal, float *out, void *stream);

/* gpu_attention.rs:589-756 GpuContext::attention_sage: the [SA] s4 reference
 * scheme (per-token INT8 Q with 1/sqrt(d) folded, per-K-block mean, per-token
 * INT8 K, P at the static 1/127 scale, per-channel INT8 V per tile), f32
 * q (B,H,S,d), k (B,Hkv,S,d), v (B,Hkv,S,dv) -> out (B,H,S,dv), same
 * validation and messages.  Both INT8 products are exact integer dot
 * products on v_dot4_i32_i8 (the scheme is per-row, VALU-bound). */
int qbk_attention_sage(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, size_t q_len,
                       const float *k, size_t k_len, const float *v, size_t v_len, int causal,
                       size_t block_size, float *out);
/* Device-pointer form of qbk_attention_sage. */
int qbk_attention_sage_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q,
                           const float *k, const float *v, int causal, size_t block_size,
                           float *out, void *stream);

/* engine/mod.rs:984-1030 gqa_attention_sage (with KvCache::keys_head_major /
 * vals_head_major, engine/mod.rs:1236-1268): one decode step of the reference
 * scheme above over a KV cache.  The reference pads the step's query into
 * row 0 of a (pos + 1)-row problem, calls attention_sage with causal = false
 * on the head-major gathered cache and reads row 0; this computes that row
 * alone (bit-identical) in O(seq), reading the cache in place.  shape:
 * batch 1, seq_q 1, seq_kv = pos + 1; q (n_heads, d) f32, k (seq_kv,
 * n_kv_heads, d) and v (seq_kv, n_kv_heads, dv) f32 row-major as cached,
 * out (n_heads, dv) f32. */
int qbk_attention_sage_decode(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, size_t q_len,
                              const float *k, size_t k_len, const float *v, size_t v_len,
                              size_t block_size, float *out, size_t out_len);
/* Device-pointer form; workspace >= qbk_sage_decode_workspace_size(). */
size_t qbk_sage_decode_workspace_size(const qbk_attn_shape *shape, size_t block_size);
int qbk_attention_sage_decode_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, const float *k,
                                  const float *v, size_t block_size, float *out, void *workspace,
                                  size_t workspace_size, void *stream);
/* The same step (engine/mod.rs:984-1030, bit-identical output) for a decode
 * loop that keeps a state across steps: the state is a workspace laid out
 * for a cache of `capacity` tokens (state_size >=
 * qbk_sage_decode_workspace_size() of the shape with seq_kv = capacity).
 * cached_tokens is the previous step's seq_kv on this state (0 for a new
 * state, or after the cache's first cached_tokens rows changed): the codes
 * of the key blocks complete within those rows are kept and only the later
 * blocks -- at most one block plus the new tokens -- are quantised again,
 * which takes the per-step cost of the pre-pass off the cache length.
 * seq_kv <= capacity, cached_tokens <= seq_kv; the shape's heads and dims,
 * block_size and capacity stay those of the state's first call.  Calls that
 * share a state must be ordered (one stream). */
int qbk_attention_sage_decode_step_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q,
                                       const float *k, const float *v, size_t block_size, float *out,
                                       void *state, size_t state_size, size_t capacity, size_t cached_tokens,
                                       void *stream);

/* Block-scaled SageAttention prefill (no reference symbol: the scheme the
 * north_star names).  bf16 q (B,H,S,d), k (B,Hkv,S,d), v (B,Hkv,S,dv),
 * d == 128, dv == 128, seq_q == seq_kv:
 *   K smoothed by its whole-sequence channel mean; Q (1/sqrt(d) folded) and K
 *   INT8 with one scale per 64-token block per head; Q.K^T on INT8 MFMA;
 *   base-2 online softmax in f32; P and V in fp16 on fp16 MFMA.
 * out is bf16 (B,H,S,dv).  workspace >= qbk_sage_blk_workspace_size(). */
size_t qbk_sage_blk_workspace_size(const qbk_attn_shape *shape);
int qbk_attention_sage_blk_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q,
                               const uint16_t *k, const uint16_t *v, int causal, uint16_t *out,
                               void *workspace, size_t workspace_size, void *stream);
/* The quantisation pre-pass alone, exporting its stages (for parity checks):
 * qhat i8 (B,H,S,d), qscale f32 (B,H,ceil(S/64)), khat i8 (B,Hkv,S,d),
 * kscale f32 (B,Hkv,ceil(S/64)), kmean f32 (B,Hkv,d), vh fp16 (B,Hkv,S,dv). */
int qbk_sage_blk_quantize_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q,
                              const uint16_t *k, const uint16_t *v, int8_t *qhat, float *qscale,
                              int8_t *khat, float *kscale, float *kmean, uint16_t *vh,
                              void *stream);

/* ---- language-model head (engine/mod.rs:781-800) -------------------------- */

/* Engine::logits: logits[v] = sum_t hidden[t] * head[v][t], one f32 sum per
 * vocabulary row in t order (each term a separate multiply and add), so the
 * logits are bit-identical to the reference's.  The head is uploaded once
 * from f32 rows (vocab, d_model) and held transposed -- as bf16 when every
 * element is a bf16 value (bf16 serving, engine/mod.rs:695-706), else f32. */
typedef struct qbk_head qbk_head;
int qbk_head_create(qbk_ctx *ctx, const float *head, size_t head_len, size_t vocab, size_t d_model,
                    qbk_head **out);
/* The same from a device buffer of f32 rows (vocab, d_model). */
int qbk_head_create_dev(qbk_ctx *ctx, const float *head, size_t vocab, size_t d_model, qbk_head **out);
void qbk_head_destroy(qbk_head *head);
int qbk_head_info(const qbk_head *head, size_t *vocab, size_t *d_model, int *bf16);
/* hidden: rows of d_model f32 (one per position); logits: rows of vocab f32. */
int qbk_head_logits(qbk_ctx *ctx, const qbk_head *head, const float *hidden, size_t hidden_len, float *logits,
                    size_t logits_len);
/* Device-pointer form, `batch` rows, stream-ordered; allocates nothing. */
int qbk_head_logits_dev(qbk_ctx *ctx, const qbk_head *head, const float *hidden, size_t batch, float *logits,
                        void *stream);

#ifdef __cplusplus
}
#endif
#endif /* QBK_H */
