// attention.hip -- the exact attention face (gpu_attention.rs:451-570
// GpuContext::attention): f32 softmax(Q K^T / sqrt(d)) V with GQA and
// causal masking, the quality reference the reference serves over
// cubek-attention and the engine's tiled decode face
// (engine/mod.rs:1041-1067 gqa_attention_tiled).
//
// Contract kept from the reference: Q is taken unscaled and 1/sqrt(head_dim)
// applied here; query head h reads kv head h / (n_heads / n_kv_heads) (the
// reference materialises that repeat on the host, here it is an index);
// causal masks key j for query i when j + seq_q > i + seq_kv (bottom-right
// aligned, so seq_q = 1 attends to every key); a row with every key masked
// is 0/0 = NaN, as the NumPy reference's is.  Same validation, messages and
// u32 index ceiling as the reference's face.
//
// One workgroup per (batch, head, query row): the row's query in LDS, keys
// in chunks of ATT_CHUNK -- a thread per key for the scores (dot products in
// 16-channel partial sums), the chunk's max and sum by workgroup reductions,
// an online softmax across chunks in f32, and a thread per output channel
// summing p_j v[j][c] over the chunk's keys in 32-key partial sums (blocked
// sums keep f32 rounding growing with the square root of the length).  Not a hot path: it is
// what the quantised schemes are measured against.
#include <math.h>

#include "qbk_internal.h"

#pragma clang fp contract(off)

namespace qbk {

#define ATT_THREADS 256
#define ATT_CHUNK 1024
#define ATT_MAXD 1024

struct AttArgs {
    const float *q, *k, *v;
    float *out;
    size_t H, Hk, Sq, Skv, d, dv;
    int causal;
    float scale;
    // element strides of k and v: between consecutive keys of a kv head and
    // between kv heads (head-major (B, Hkv, Skv, d): d and Skv d; a decoder
    // block's row-major cache (rows, Hkv d): Hkv d and d)
    size_t k_tok, k_head, v_tok, v_head;
};

__device__ __forceinline__ float att_block_max(float v, float *red) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < ATT_THREADS / 64; w++) r = fmaxf(r, red[w]);
    return r;
}

__device__ __forceinline__ float att_block_sum(float v, float *red) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < ATT_THREADS / 64; w++) r += red[w];
    return r;
}

__global__ void __launch_bounds__(ATT_THREADS) att_exact(AttArgs a) {
    __shared__ float qs[ATT_MAXD];
    __shared__ float ps[ATT_CHUNK];
    __shared__ float red[ATT_THREADS / 64];
    const size_t row = blockIdx.x;  // (b * H + h) * Sq + i
    const size_t i = row % a.Sq, bh = row / a.Sq, b = bh / a.H, h = bh % a.H;
    const size_t bk = b * a.Hk + h / (a.H / a.Hk);
    const float *qr = a.q + row * a.d;
    const float *kb = a.k + bk * a.k_head;
    const float *vb = a.v + bk * a.v_head;
    const int tid = threadIdx.x;
    for (size_t c = tid; c < a.d; c += ATT_THREADS) qs[c] = qr[c];
    // keys visible to query i: j < i + 1 + (Skv - Sq), i.e. j + Sq <= i + Skv
    size_t kend = a.Skv;
    if (a.causal) kend = i + a.Skv >= a.Sq ? (i + a.Skv - a.Sq + 1 < a.Skv ? i + a.Skv - a.Sq + 1 : a.Skv) : 0;
    float m = -INFINITY, l = 0.0f;
    float acc[ATT_MAXD / ATT_THREADS];
#pragma unroll
    for (int u = 0; u < ATT_MAXD / ATT_THREADS; u++) acc[u] = 0.0f;
    __syncthreads();
    for (size_t j0 = 0; j0 < kend; j0 += ATT_CHUNK) {
        const size_t j1 = j0 + ATT_CHUNK < kend ? j0 + ATT_CHUNK : kend;
        float cmax = -INFINITY;
        for (size_t j = j0 + tid; j < j1; j += ATT_THREADS) {
            const float *kr = kb + j * a.k_tok;
            float s = 0.0f;
            for (size_t c0 = 0; c0 < a.d; c0 += 16) {  // blocked: 16-term partials
                float sp = 0.0f;
                const size_t c1 = c0 + 16 < a.d ? c0 + 16 : a.d;
                for (size_t c = c0; c < c1; c++) sp += qs[c] * kr[c];
                s += sp;
            }
            s = s * a.scale;
            ps[j - j0] = s;
            cmax = fmaxf(cmax, s);
        }
        cmax = att_block_max(cmax, red);
        const float mn = fmaxf(m, cmax);
        const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
        float part = 0.0f;
        for (size_t j = j0 + tid; j < j1; j += ATT_THREADS) {
            const float p = expf(ps[j - j0] - mn);
            ps[j - j0] = p;
            part += p;
        }
        part = att_block_sum(part, red);  // its barriers also publish ps
        l = l * alpha + part;
#pragma unroll
        for (int u = 0; u < ATT_MAXD / ATT_THREADS; u++) {
            const size_t c = tid + (size_t)u * ATT_THREADS;
            if (c >= a.dv) break;
            float sacc = 0.0f;
            for (size_t jb = j0; jb < j1; jb += 32) {  // blocked: 32-term partials
                float sp = 0.0f;
                const size_t je = jb + 32 < j1 ? jb + 32 : j1;
                for (size_t j = jb; j < je; j++) sp += ps[j - j0] * vb[j * a.v_tok + c];
                sacc += sp;
            }
            acc[u] = acc[u] * alpha + sacc;
        }
        m = mn;
        __syncthreads();  // ps is rewritten by the next chunk
    }
#pragma unroll
    for (int u = 0; u < ATT_MAXD / ATT_THREADS; u++) {
        const size_t c = tid + (size_t)u * ATT_THREADS;
        if (c >= a.dv) break;
        a.out[row * a.dv + c] = acc[u] / l;
    }
}

// gpu_attention.rs:466-509: validation in the reference's order and words,
// then the u32 index ceiling of its device face.
static int validate_exact(const qbk_attn_shape *s, const size_t *lens) {
    if (!s) return fail(QBK_ERR_VALIDATION, "null shape");
    if (s->batch == 0 || s->n_heads == 0 || s->n_kv_heads == 0)
        return fail(QBK_ERR_VALIDATION, "attention requires non-empty batch and head dimensions");
    if (s->n_heads % s->n_kv_heads != 0)
        return fail(QBK_ERR_VALIDATION, fmt("n_kv_heads must divide n_heads: n_heads=%zu, n_kv_heads=%zu",
                                            s->n_heads, s->n_kv_heads));
    if (s->seq_q == 0 || s->seq_kv == 0 || s->head_dim == 0 || s->val_dim == 0)
        return fail(QBK_ERR_VALIDATION, "attention requires non-empty sequence and head dimensions");
    const size_t eq = s->batch * s->n_heads * s->seq_q * s->head_dim;
    const size_t ek = s->batch * s->n_kv_heads * s->seq_kv * s->head_dim;
    const size_t ev = s->batch * s->n_kv_heads * s->seq_kv * s->val_dim;
    const std::string dbg = fmt("AttentionShape { batch: %zu, n_heads: %zu, n_kv_heads: %zu, seq_q: %zu, seq_kv: "
                                "%zu, head_dim: %zu, val_dim: %zu }",
                                s->batch, s->n_heads, s->n_kv_heads, s->seq_q, s->seq_kv, s->head_dim, s->val_dim);
    if (lens) {
        if (lens[0] != eq)
            return fail(QBK_ERR_VALIDATION, fmt("query must hold %zu values for %s, got %zu", eq, dbg.c_str(), lens[0]));
        if (lens[1] != ek)
            return fail(QBK_ERR_VALIDATION, fmt("key must hold %zu values for %s, got %zu", ek, dbg.c_str(), lens[1]));
        if (lens[2] != ev)
            return fail(QBK_ERR_VALIDATION, fmt("value must hold %zu values for %s, got %zu", ev, dbg.c_str(), lens[2]));
    }
    size_t largest = eq > ek ? eq : ek;
    largest = largest > ev ? largest : ev;
    if ((uint64_t)largest > 0xFFFFFFFFull)
        return fail(QBK_ERR_VALIDATION, "attention inputs exceed the device u32 index ceiling (4294967295); use "
                                        "the CPU reference face");
    if (s->head_dim > ATT_MAXD || s->val_dim > ATT_MAXD)
        return fail(QBK_ERR_VALIDATION, fmt("attention on this device supports head_dim and val_dim up to %d, "
                                            "got head_dim=%zu, val_dim=%zu",
                                            ATT_MAXD, s->head_dim, s->val_dim));
    return QBK_OK;
}

static int launch_exact(const qbk_attn_shape *s, const float *q, const float *k, const float *v, int causal,
                        float *out, hipStream_t st) {
    AttArgs a{q, k, v, out, s->n_heads, s->n_kv_heads, s->seq_q, s->seq_kv, s->head_dim, s->val_dim, causal ? 1 : 0,
              1.0f / sqrtf((float)s->head_dim), s->head_dim, s->seq_kv * s->head_dim, s->val_dim,
              s->seq_kv * s->val_dim};
    const size_t rows = s->batch * s->n_heads * s->seq_q;
    if (rows > 0x7FFFFFFFull) return fail(QBK_ERR_VALIDATION, "attention: too many query rows for one launch");
    hipLaunchKernelGGL(att_exact, dim3((unsigned)rows), dim3(ATT_THREADS), 0, st, a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

// One query position of every head over rows 0 .. rows - 1 of a decoder
// block's row-major cache (f32 [rows][Hk hd] keys and values): the engine's
// tiled decode face (engine/mod.rs:1041-1067: seq_q = 1, so every cached key
// is visible), reading the cache in place rather than gathered head-major.
int attention_exact_cache(const float *q, const float *kc, const float *vc, size_t H, size_t Hk, size_t hd,
                          size_t rows, float *out, hipStream_t st) {
    if (rows == 0 || H == 0 || Hk == 0 || H % Hk != 0 || hd == 0 || hd > ATT_MAXD)
        return fail(QBK_ERR_VALIDATION, "exact cache attention: bad shape");
    AttArgs a{q, kc, vc, out, H, Hk, 1, rows, hd, hd, 0, 1.0f / sqrtf((float)hd), Hk * hd, hd, Hk * hd, hd};
    hipLaunchKernelGGL(att_exact, dim3((unsigned)H), dim3(ATT_THREADS), 0, st, a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_attention(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, size_t q_len, const float *k,
                  size_t k_len, const float *v, size_t v_len, int causal, float *out) {
    int rc;
    const size_t lens[3] = {q_len, k_len, v_len};
    if ((rc = validate_exact(shape, lens))) return rc;
    if (!q || !k || !v || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if ((rc = bind(ctx))) return rc;
    const size_t no = shape->batch * shape->n_heads * shape->seq_q * shape->val_dim;
    DevBuf dq, dk, dv, dout;
    CallStream cs;
    if ((rc = dq.alloc(q_len * 4)) || (rc = dk.alloc(k_len * 4)) || (rc = dv.alloc(v_len * 4)) ||
        (rc = dout.alloc(no * 4)) || (rc = cs.create()))
        return rc;
    QBK_HIP(hipMemcpyAsync(dq.p, q, q_len * 4, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dk.p, k, k_len * 4, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dv.p, v, v_len * 4, hipMemcpyHostToDevice, cs.s));
    if ((rc = launch_exact(shape, (const float *)dq.p, (const float *)dk.p, (const float *)dv.p, causal,
                           (float *)dout.p, cs.s)))
        return rc;
    QBK_HIP(hipMemcpyAsync(out, dout.p, no * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_attention_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, const float *k, const float *v,
                      int causal, float *out, void *stream) {
    int rc;
    if ((rc = validate_exact(shape, nullptr))) return rc;
    if (!q || !k || !v || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if ((rc = bind(ctx))) return rc;
    return launch_exact(shape, q, k, v, causal, out, (hipStream_t)stream);
}

}  // extern "C"
