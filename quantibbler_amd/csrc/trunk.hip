// trunk.hip -- the per-token pieces of the transformer trunk around the
// decoder blocks: the embedding lookup (engine/mod.rs:768-778 Engine::embed),
// the final RMSNorm (engine/mod.rs:943, norm_apply at :837-852) and greedy
// argmax (sampler.rs:4-15).  Rows are independent, so each op is one
// workgroup per row over rows laid out contiguously.
#include <math.h>

#include "qbk_internal.h"

#pragma clang fp contract(off)

namespace qbk {

#define TRUNK_THREADS 256

// out[r] = table[tokens[r]] (f32 rows of d).  An id outside the vocabulary
// writes a row of NaN: a device-side id cannot raise the reference's error
// synchronously, so it poisons the row instead (the host form validates).
__global__ void __launch_bounds__(TRUNK_THREADS) trunk_embed(const float *table, size_t vocab, size_t d,
                                                            const int32_t *tokens, float *out) {
    const size_t row = blockIdx.x;
    const int32_t t = tokens[row];
    const bool ok = t >= 0 && (size_t)t < vocab;
    const float *src = table + (ok ? (size_t)t : 0) * d;
    float *dst = out + row * d;
    for (size_t i = threadIdx.x; i < d; i += TRUNK_THREADS) dst[i] = ok ? src[i] : __builtin_nanf("");
}

// norm_apply at bf16 serving (engine/mod.rs:837-852 over rms_norm_into,
// :1152-1160): the row rounded to bf16, its mean square in f32 (a tree over
// the workgroup here; the reference's is one sequential fold), inv =
// 1 / sqrt(ms + eps), out = bf16(b * inv * w) held as f32.
// F32: norm_apply at fp32 serving (no bf16 roundings of the operand and
// the output).
template <bool F32>
__global__ void __launch_bounds__(TRUNK_THREADS) trunk_rms_norm(const float *x, size_t d, const float *w,
                                                               float eps, float *out) {
    __shared__ float red[TRUNK_THREADS / 64];
    const float *xr = x + (size_t)blockIdx.x * d;
    float *orow = out + (size_t)blockIdx.x * d;
    float ss = 0.0f;
    for (size_t i = threadIdx.x; i < d; i += TRUNK_THREADS) {
        const float b = F32 ? xr[i] : bf16_to_f32(f32_to_bf16(xr[i]));
        ss += b * b;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < TRUNK_THREADS / 64; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    for (size_t i = threadIdx.x; i < d; i += TRUNK_THREADS) {
        const float b = F32 ? xr[i] : bf16_to_f32(f32_to_bf16(xr[i]));
        orow[i] = F32 ? b * inv * w[i] : bf16_to_f32(f32_to_bf16(b * inv * w[i]));
    }
}

// sampler.rs:4-15 greedy: the first index holding the largest value, a NaN
// never winning, 0 when nothing beats -inf.  A value v at index i beats the
// running (bv, bi) when v > bv, or v == bv and i < bi (so a tree keeps the
// first of equal maxima); NaN compares as -inf.
__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// A row per workgroup of ARGMAX_THREADS: a scalar head up to a 16-byte
// boundary, the body in 16-byte loads four a thread in flight (a vocabulary
// row is ~0.5 MB: one load at a time per thread left the kernel latency
// bound at 156 us), a scalar tail.  amax_merge is a total order, so the
// merge order does not change the winner.
#define ARGMAX_THREADS 1024
typedef float tr_f32x4_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(ARGMAX_THREADS) trunk_argmax(const float *logits, size_t vocab, int32_t *out) {
    __shared__ float sv[ARGMAX_THREADS / 64];
    __shared__ uint32_t si[ARGMAX_THREADS / 64];
    const float *row = logits + (size_t)blockIdx.x * vocab;
    const uint32_t tid = threadIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0;
    auto take = [&](float v, size_t i) { amax_merge(bv, bi, v != v ? -INFINITY : v, (uint32_t)i); };
    size_t head = (4 - (((uintptr_t)row >> 2) & 3)) & 3;
    head = head < vocab ? head : vocab;
    if (tid < head) take(row[tid], tid);
    const size_t nb = (vocab - head) / 4;
    const tr_f32x4_t *b4 = (const tr_f32x4_t *)(row + head);
    size_t j = tid;
    for (; j + 3 * ARGMAX_THREADS < nb; j += 4 * ARGMAX_THREADS) {
        tr_f32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = b4[j + u * ARGMAX_THREADS];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int e = 0; e < 4; e++) take(v[u][e], head + 4 * (j + u * ARGMAX_THREADS) + e);
    }
    for (; j < nb; j += ARGMAX_THREADS) {
        const tr_f32x4_t v = b4[j];
#pragma unroll
        for (int e = 0; e < 4; e++) take(v[e], head + 4 * j + e);
    }
    for (size_t i = head + 4 * nb + tid; i < vocab; i += ARGMAX_THREADS) take(row[i], i);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v = __shfl_xor(bv, o, 64);
        const uint32_t i = (uint32_t)__shfl_xor((int)bi, o, 64);
        amax_merge(bv, bi, v, i);
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < ARGMAX_THREADS / 64; w++) amax_merge(bv, bi, sv[w], si[w]);
        out[blockIdx.x] = (int32_t)bi;
    }
}

// pos[i] += 1 for the n sequences of a greedy loop's step (device-position
// decode steps read them).
__global__ void trunk_advance(uint32_t *pos, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) pos[i] = pos[i] + 1;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_embed(qbk_ctx *ctx, const float *table, size_t vocab, size_t d_model, const int32_t *tokens_host,
              size_t n, float *out, void *stream) {
    int rc;
    if (!table || !tokens_host || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    for (size_t i = 0; i < n; i++)
        if (tokens_host[i] < 0 || (size_t)tokens_host[i] >= vocab)
            return fail(QBK_ERR_VALIDATION, fmt("token id %d is outside the vocabulary (size %zu)",
                                                tokens_host[i], vocab));
    if (n == 0 || d_model == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipStream_t s = (hipStream_t)stream;
    DevBuf ids;
    if ((rc = ids.alloc(n * 4))) return rc;
    QBK_HIP(hipMemcpy(ids.p, tokens_host, n * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(trunk_embed, dim3((unsigned)n), dim3(TRUNK_THREADS), 0, s, table, vocab, d_model,
                       (const int32_t *)ids.p, out);
    QBK_HIP(hipGetLastError());
    QBK_HIP(hipStreamSynchronize(s));  // the ids buffer is freed on return
    return QBK_OK;
}

int qbk_embed_dev(qbk_ctx *ctx, const float *table, size_t vocab, size_t d_model, const int32_t *tokens,
                  size_t n, float *out, void *stream) {
    int rc;
    if (!table || !tokens || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if (n == 0 || d_model == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipLaunchKernelGGL(trunk_embed, dim3((unsigned)n), dim3(TRUNK_THREADS), 0, (hipStream_t)stream, table, vocab,
                       d_model, tokens, out);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int qbk_rms_norm_dev(qbk_ctx *ctx, const float *x, size_t rows, size_t d, const float *w, double eps, float *out,
                     void *stream) {
    int rc;
    if (!x || !w || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if (rows == 0 || d == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipLaunchKernelGGL(trunk_rms_norm<false>, dim3((unsigned)rows), dim3(TRUNK_THREADS), 0, (hipStream_t)stream, x, d,
                       w, (float)eps, out);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int qbk_rms_norm_f32_dev(qbk_ctx *ctx, const float *x, size_t rows, size_t d, const float *w, double eps,
                         float *out, void *stream) {
    int rc;
    if (!x || !w || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if (rows == 0 || d == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipLaunchKernelGGL(trunk_rms_norm<true>, dim3((unsigned)rows), dim3(TRUNK_THREADS), 0, (hipStream_t)stream, x, d,
                       w, (float)eps, out);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int qbk_positions_advance_dev(qbk_ctx *ctx, uint32_t *pos, size_t n, void *stream) {
    int rc;
    if (!pos) return fail(QBK_ERR_VALIDATION, "null argument");
    if (n == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipLaunchKernelGGL(trunk_advance, dim3((unsigned)div_ceil(n, 256)), dim3(256), 0, (hipStream_t)stream, pos, n);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int qbk_argmax_dev(qbk_ctx *ctx, const float *logits, size_t rows, size_t vocab, int32_t *out, void *stream) {
    int rc;
    if (!logits || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if (vocab == 0 || vocab > 0xFFFFFFFFu) return fail(QBK_ERR_VALIDATION, "argmax needs 1 <= vocab < 2^32");
    if (rows == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipLaunchKernelGGL(trunk_argmax, dim3((unsigned)rows), dim3(ARGMAX_THREADS), 0, (hipStream_t)stream, logits,
                       vocab, out);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // extern "C"
