// qbk_internal.h -- shared internals of libqbk (gfx950 / CDNA4).
//
// Error plumbing (thread-local last error, reference message texts), the
// device context, and small device helpers (bf16 RNE, wave reductions).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/qbk.h"

namespace qbk {

// ---- errors --------------------------------------------------------------

void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));

// HIP call that maps a failure to QBK_ERR_DEVICE with the call's text.
#define QBK_HIP(call)                                                                  \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess)                                                          \
            return ::qbk::fail(QBK_ERR_DEVICE, ::qbk::fmt("%s failed: %s", #call,      \
                                                          hipGetErrorString(e_)));     \
    } while (0)

// ---- context -------------------------------------------------------------

}  // namespace qbk

struct qbk_ctx {
    int device;
    int num_cus;
    hipDeviceProp_t props;
};

namespace qbk {

// Makes ctx->device current for the calling thread.
int bind(qbk_ctx *ctx);

// Scoped device buffer for the host-pointer entry points.
struct DevBuf {
    void *p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t n) {
        if (n == 0) n = 16;
        hipError_t e = hipMalloc(&p, n);
        if (e != hipSuccess) {
            p = nullptr;
            return fail(QBK_ERR_DEVICE, fmt("hipMalloc(%zu) failed: %s", n, hipGetErrorString(e)));
        }
        return QBK_OK;
    }
};

// Scoped non-default stream for a blocking host call.
struct CallStream {
    hipStream_t s = nullptr;
    ~CallStream() {
        if (s) (void)hipStreamDestroy(s);
    }
    int create() {
        hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        if (e != hipSuccess) {
            s = nullptr;
            return fail(QBK_ERR_DEVICE, fmt("hipStreamCreate failed: %s", hipGetErrorString(e)));
        }
        return QBK_OK;
    }
};

// validate_packed (core.rs:223-240) with the reference's messages.
int validate_packed(size_t packed_len, size_t n_rows, size_t n_bits, size_t *n_words);

static inline size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }
static inline size_t round_up(size_t a, size_t b) { return div_ceil(a, b) * b; }

// Decode steps of up to QBK_DEC_MAXSEQ sequences in one set of launches
// (sage.hip), for shapes where sage_decode_batchable holds: sequence i has
// seq_kv[i] cache rows, the state's codes of its first cached[i] of them
// kept from its last step; its query, caches, output and state sit i times
// q_stride, kv_stride, o_stride (floats) and st_stride (bytes) past
// sequence 0's.  `one` gives the heads and dims (its seq_kv is ignored).
#define QBK_DEC_MAXSEQ 64
bool sage_decode_batchable(const qbk_attn_shape *one, size_t block, size_t cap, const float *k, const float *v,
                           size_t kv_stride);
struct DecOpSink;
struct DecRope;
int sage_decode_batch(const qbk_attn_shape *one, const float *q, size_t q_stride, const float *k, const float *v,
                      size_t kv_stride, size_t block, float *out, size_t o_stride, void *state, size_t st_stride,
                      size_t cap, const size_t *seq_kv, const size_t *cached, size_t n, hipStream_t st,
                      const uint32_t *pos_dev = nullptr, const DecOpSink *sink = nullptr,
                      const DecRope *rope = nullptr);
// pos_dev (device, n entries): each sequence's position instead of seq_kv
// and cached -- the step attends over pos + 1 cache rows and keeps the
// codes of the pos / block complete key blocks before it (a state stepped
// through pos - 1); the grids cover the capacity and the kernels read the
// positions, so a captured graph of the step serves every position.  A
// position at or past the capacity skips that sequence.  sink (n == 1):
// the combine writes the o projection's batch-1 operand as well.  rope
// (n == 1): the step's q/k norm, RoPE and cache append run in the pre-pass
// (the caches then take the new row from rope->qkv, not from the caller).

// Exact f32 attention of one query position (q [H][hd]) over rows
// 0 .. rows - 1 of a decoder block's row-major cache ([rows][Hk hd] keys and
// values) -> out [H][hd] (attention.hip; the engine's tiled decode face).
// qbk_attention_sage_blk_dev with the output either head-major [B][H][S][hd]
// (out_rows false, the C ABI's layout) or token-major [B][S][H][hd] (the
// rows of the o projection that reads it).
int sage_blk_run(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                 int causal, uint16_t *out, bool out_rows, void *workspace, size_t workspace_size, void *stream);

int attention_exact_cache(const float *q, const float *kc, const float *vc, size_t H, size_t Hk, size_t hd,
                          size_t rows, float *out, hipStream_t st);

// A decode step (qbk_attention_sage_decode_step_dev's contract) whose
// combine also writes its output [n_heads][val_dim] as the batch-1 stage-1
// fp8 operand of the factor layer it feeds (q4_operand.h's flat runs; val_dim
// a multiple of 128): that layer's s2, operand and scale bytes.
struct DecOpSink {
    const float *s2;
    uint8_t *op, *sc;
};
int sage_decode_step_sink(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, const float *k,
                          const float *v, size_t block_size, float *out, void *state, size_t state_size,
                          size_t capacity, size_t cached_tokens, const DecOpSink *sink, void *stream,
                          const DecRope *rope = nullptr);

// The decode step's q/k norm and RoPE folded into the attention's pre-pass
// (one sequence): the new token's k and v rows written into the cache and
// its query rotated where the pre-pass forms the query's codes.
struct DecRope {
    const float *qkv;      // the step's projections: q (H heads), k (Hk), v (Hk), hd floats a head; null: no fold
    const float2 *rope;    // (cos, sin) [capacity][hd / 2]
    const float *wq, *wk;  // per-head norm weights, or null
    float eps;
    int H;
};

// ---- device helpers -------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}

// half 2.7.1 bf16::from_f32 (round to nearest even; NaN stays quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

// One head of a decode step's q/k norm (a per-head RMSNorm over bf16
// operands when w is given, engine/mod.rs:909-912) and RoPE at the row cs of
// (cos, sin) pairs (engine/mod.rs:878-945): a wave per head.  Each lane sums
// the squares of its channels j = lane, lane + 64, ... in order, then an
// xor-shuffle tree; out(j, value) receives rotated channel j.  The decode
// kernels that rotate a head all call this, so their values agree bit for
// bit.
// F32 (fp32 serving, engine/mod.rs:854-876): the norm without the bf16
// roundings of its input and output.
template <class OUT, bool F32 = false>
__device__ __forceinline__ void rope_head(const float *src, const float *w, float eps, const float2 *cs, int hd,
                                          int lane, OUT out) {
    const int half = hd / 2;
    auto rd = [](float v) { return F32 ? v : bf16_to_f32(f32_to_bf16(v)); };
    float inv = 1.0f;
    if (w) {
        float ss = 0.0f;
        for (int j = lane; j < hd; j += 64) {
            const float b = rd(src[j]);
            ss += b * b;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        inv = 1.0f / sqrtf(ss / (float)hd + eps);
    }
    for (int j = lane; j < half; j += 64) {
        float a = src[j], b = src[j + half];
        if (w) {
            a = rd(rd(a) * inv * w[j]);
            b = rd(rd(b) * inv * w[j + half]);
        }
        const float2 c = cs[j];
        out(j, a * c.x - b * c.y);
        out(j + half, b * c.x + a * c.y);
    }
}

// The same rounding for a pair, packed (a in the low half), in one
// v_cvt_pk_bf16_f32: gfx950's converter rounds to nearest even and quiets a
// NaN as (u >> 16) | 0x40, bit for bit what f32_to_bf16 does (checked on
// the device over 8.4M values: random bit patterns, every exponent's ties
// and near-ties, denormals, overflow to infinity and NaN payloads).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

}  // namespace qbk
