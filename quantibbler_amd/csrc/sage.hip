// sage.hip -- SageAttention on gfx950.
//
// Two schemes behind the reference's contract (gpu_attention.rs:402-756):
//
// 1. qbk_attention_sage: the [SA] s4 reference scheme of
//    gpu_attention.rs:67-397 / attention_sage.py:206-350 -- per-token INT8 Q
//    (1/sqrt(d) folded), per-K-block mean smoothing with the shift added back,
//    per-token INT8 K, P at the static 1/127 scale after the running-max
//    rescale, per-channel INT8 V within the tile, f32 statistics.  The
//    per-key-block work the reference repeats for every query row (block
//    mean, K and V codes) is computed once per (kv head, block) by a pre-pass
//    with the same f32 operation order; each query row then follows the
//    reference kernel's f32 sequence exactly (sequential sums, sentinel
//    -3e38, `live` flag, O/l), with both INT8 products as v_dot4_i32_i8.  The
//    f32 results are bit-identical to the oracle's restatement of that
//    kernel, exp included (qbk_expf below, the same operation sequence).
//
// 2. qbk_attention_sage_blk_dev: the block-scaled scheme -- K smoothed by
//    its whole-sequence channel mean (a per-row constant shift, which softmax
//    ignores, so nothing is added back), INT8 Q and K with one scale per
//    64-token block per head, S^T = K^.Q^T on INT8 MFMA (16x16x64), base-2
//    online softmax in f32 (log2 e folded into the block scale), P and V in
//    fp16, O^T += V^T.P^T on fp16 MFMA (16x16x32) with P kept in registers.
#include <math.h>
#include <string.h>

#include <string>

#include "qbk_internal.h"

namespace qbk {

// ======================================================================
// shared helpers
// ======================================================================

#pragma clang fp contract(off)

// exp(x): Cody & Waite (1980) reduction x = n ln2 + r with ln2 split in two
// (the high part has 12 trailing zero bits, so n*ln2_hi is exact), e^r by
// the degree-7 Taylor polynomial on |r| <= ln2/2, scaled by 2^n in two
// exponent-field steps.  Written without fused multiply-add so host and
// device agree bit for bit.
__device__ __forceinline__ float qbk_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return __builtin_huge_valf();
    if (x < -103.97208f) return 0.0f;
    const float log2e = 1.44269504088896341f;
    const float ln2_hi = 0.693145751953125f;
    const float ln2_lo = 1.428606765330187045e-06f;
    float n = __builtin_rintf(x * log2e);
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
    float s1 = __uint_as_float((uint32_t)(n1 + 127) << 23);
    float s2 = __uint_as_float((uint32_t)(n2 + 127) << 23);
    return (p * s1) * s2;
}

// clamp(rint_half_even(x), -127, 127) as an int
__device__ __forceinline__ int q8(float x) {
    float r = __builtin_rintf(x);
    r = r > 127.0f ? 127.0f : r;
    r = r < -127.0f ? -127.0f : r;
    return (int)r;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

#define MASKED (-3.0e38f)

// ======================================================================
// 1. reference scheme
// ======================================================================

#define REF_ROWS 64  // query rows per workgroup (one wave, one row per lane)
#define REF_CH 64    // key tokens per LDS chunk
#define REF_MAXD 256

struct RefArgs {
    const float *q, *k, *v;
    float *out;
    size_t B, H, Hk, S, d, dv, block;
    int causal;
    float inv_sqrt_d;
    size_t nkb, d4, blk4;
    // pre-pass products
    float *kmean;     // [B*Hk*nkb][d]
    float *kdelta;    // [B*Hk*S]
    uint32_t *khat;   // [B*Hk*S][d4]
    float *vd;        // [B*Hk*nkb][dv]
    uint32_t *vhat;   // [B*Hk*nkb][dv][blk4]
    // per-row state when it does not fit in LDS ([slot][row], rows = B*H*S)
    float *gsc;       // [block][rows]
    uint32_t *gph;    // [blk4][rows]
    int *gpv;         // [dv][rows]
    float *gout;      // [dv][rows]
    int sc_lds, out_lds;
};

// Pre-pass: one workgroup per (kv head, key block).  gpu_attention.rs:192-204
// (block mean, sequential over the block's tokens), :211-226 (per-token peak
// and delta), :232-251 (codes), :290-309 (per-channel V scale), :352-370.
__global__ void __launch_bounds__(256) sage_ref_prep(RefArgs a) {
    __shared__ float km[REF_MAXD];
    const size_t kb = blockIdx.x, bk = blockIdx.y;
    const size_t j0 = kb * a.block;
    const size_t j1 = j0 + a.block < a.S ? j0 + a.block : a.S;
    const size_t kj = j1 - j0;
    const float *K = a.k + bk * a.S * a.d;
    const float *V = a.v + bk * a.S * a.dv;
    for (size_t c = threadIdx.x; c < a.d; c += blockDim.x) {
        float ssum = 0.0f;
        for (size_t jj = j0; jj < j1; jj++) ssum += K[jj * a.d + c];
        float m = ssum / (float)kj;
        km[c] = m;
        a.kmean[(bk * a.nkb + kb) * a.d + c] = m;
    }
    __syncthreads();
    for (size_t jj = j0 + threadIdx.x; jj < j1; jj += blockDim.x) {
        const float *kt = K + jj * a.d;
        float kpeak = 0.0f;
        for (size_t c = 0; c < a.d; c++) {
            float g = kt[c] - km[c];
            float ag = g < 0.0f ? 0.0f - g : g;
            if (ag > kpeak) kpeak = ag;
        }
        float kdelta = 1.0f;
        if (kpeak > 0.0f) kdelta = kpeak / 127.0f;
        a.kdelta[bk * a.S + jj] = kdelta;
        uint32_t *dst = a.khat + (bk * a.S + jj) * a.d4;
        for (size_t w = 0; w < a.d4; w++) {
            int c4[4];
            for (int e = 0; e < 4; e++) {
                size_t c = 4 * w + e;
                c4[e] = c < a.d ? q8((kt[c] - km[c]) / kdelta) : 0;
            }
            dst[w] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
    }
    for (size_t c = threadIdx.x; c < a.dv; c += blockDim.x) {
        float vpeak = 0.0f;
        for (size_t jj = j0; jj < j1; jj++) {
            float x = V[jj * a.dv + c];
            float ax = x < 0.0f ? 0.0f - x : x;
            if (ax > vpeak) vpeak = ax;
        }
        float vd = vpeak > 0.0f ? vpeak / 127.0f : 1.0f;
        a.vd[(bk * a.nkb + kb) * a.dv + c] = vd;
        uint32_t *dst = a.vhat + ((bk * a.nkb + kb) * a.dv + c) * a.blk4;
        for (size_t w = 0; w < a.blk4; w++) {
            int c4[4];
            for (int e = 0; e < 4; e++) {
                size_t jj = j0 + 4 * w + e;
                c4[e] = jj < j1 ? q8(V[jj * a.dv + c] / vd) : 0;
            }
            dst[w] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
    }
}

// Main pass: gpu_attention.rs:89-396 for REF_ROWS consecutive query rows of
// one (batch, head); one row per lane.
__global__ void __launch_bounds__(REF_ROWS) sage_ref_main(RefArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
    const int tid = threadIdx.x;
    const size_t bh = blockIdx.y;
    const size_t b = bh / a.H, h = bh % a.H;
    const size_t bk = b * a.Hk + h / (a.H / a.Hk);
    const size_t i = (size_t)blockIdx.x * REF_ROWS + tid;
    const bool valid = i < a.S;
    const size_t row = bh * a.S + i;
    const size_t rows_total = a.B * a.H * a.S;
    const size_t d4 = a.d4, dv = a.dv;

    uint32_t *qs = smem;                                   // [d4][64]
    float *kms = (float *)(qs + d4 * REF_ROWS);            // [d]
    float *kdl = kms + d4 * 4;                             // [REF_CH]
    uint32_t *kc = (uint32_t *)(kdl + REF_CH);             // [REF_CH][d4]
    float *vdl = (float *)(kc + REF_CH * d4);              // [dv]
    uint32_t *vc = (uint32_t *)(vdl + dv);                 // [dv][REF_CH/4]
    float *lsc = (float *)(vc + dv * (REF_CH / 4));        // [REF_CH][64] if sc_lds
    uint32_t *lph = (uint32_t *)(lsc + (a.sc_lds ? REF_CH * REF_ROWS : 0));  // [16][64]
    float *lout = (float *)(lph + (a.sc_lds ? (REF_CH / 4) * REF_ROWS : 0)); // [dv][64]

    auto SC = [&](size_t kk) -> float & {
        return a.sc_lds ? lsc[kk * REF_ROWS + tid] : a.gsc[kk * rows_total + row];
    };
    auto PH = [&](size_t w) -> uint32_t & {
        return a.sc_lds ? lph[w * REF_ROWS + tid] : a.gph[w * rows_total + row];
    };
    auto OUT = [&](size_t c) -> float & {
        return a.out_lds ? lout[c * REF_ROWS + tid] : a.gout[c * rows_total + row];
    };

    // psi_Q (gpu_attention.rs:113-159)
    float qdelta = 1.0f;
    if (valid) {
        const float *qi = a.q + row * a.d;
        float qpeak = 0.0f;
        for (size_t c = 0; c < a.d; c++) {
            float x = qi[c] * a.inv_sqrt_d;
            float ax = x < 0.0f ? 0.0f - x : x;
            if (ax > qpeak) qpeak = ax;
        }
        if (qpeak > 0.0f) qdelta = qpeak / 127.0f;
        for (size_t w = 0; w < d4; w++) {
            int c4[4];
            for (int e = 0; e < 4; e++) {
                size_t c = 4 * w + e;
                c4[e] = c < a.d ? q8((qi[c] * a.inv_sqrt_d) / qdelta) : 0;
            }
            qs[w * REF_ROWS + tid] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
        for (size_t c = 0; c < dv; c++) OUT(c) = 0.0f;
    }
    size_t i1 = (i / a.block + 1) * a.block;
    if (i1 > a.S) i1 = a.S;
    const size_t j_stop = valid ? (a.causal ? i1 : a.S) : 0;
    size_t last = (size_t)blockIdx.x * REF_ROWS + REF_ROWS - 1;
    if (last > a.S - 1) last = a.S - 1;
    size_t jmax = a.S;
    if (a.causal) {
        jmax = (last / a.block + 1) * a.block;
        if (jmax > a.S) jmax = a.S;
    }

    float m = MASKED, ell = 0.0f;
    for (size_t j0 = 0; j0 < jmax; j0 += a.block) {
        const size_t j1 = j0 + a.block < a.S ? j0 + a.block : a.S;
        const size_t kj = j1 - j0, kb = j0 / a.block;
        const bool active = j0 < j_stop;
        __syncthreads();
        for (size_t c = tid; c < a.d; c += REF_ROWS) kms[c] = a.kmean[(bk * a.nkb + kb) * a.d + c];
        for (size_t c = tid; c < dv; c += REF_ROWS) vdl[c] = a.vd[(bk * a.nkb + kb) * dv + c];
        __syncthreads();
        // shift = sum_c (q^_c * dq) * kmean_c, element order (:253)
        float shift = 0.0f;
        if (active) {
            for (size_t w = 0; w < d4; w++) {
                uint32_t qw = qs[w * REF_ROWS + tid];
                for (int e = 0; e < 4; e++) {
                    size_t c = 4 * w + e;
                    if (c >= a.d) break;
                    int qc = (int)(int8_t)(qw >> (8 * e));
                    shift += ((float)qc * qdelta) * kms[c];
                }
            }
        }
        // scores (:209-262)
        for (size_t t0 = 0; t0 < kj; t0 += REF_CH) {
            const size_t tc = kj - t0 < REF_CH ? kj - t0 : REF_CH;
            __syncthreads();
            for (size_t t = tid; t < tc; t += REF_ROWS) kdl[t] = a.kdelta[bk * a.S + j0 + t0 + t];
            for (size_t x = tid; x < tc * d4; x += REF_ROWS)
                kc[x] = a.khat[(bk * a.S + j0 + t0) * d4 + x];
            __syncthreads();
            if (active) {
                for (size_t t = 0; t < tc; t++) {
                    int acc_i = 0;
                    for (size_t w = 0; w < d4; w++)
                        acc_i = __builtin_amdgcn_sdot4((int)qs[w * REF_ROWS + tid], (int)kc[t * d4 + w],
                                                       acc_i, false);
                    float s = (float)acc_i * qdelta * kdl[t] + shift;
                    size_t jj = j0 + t0 + t;
                    if (a.causal && jj > i) s = MASKED;
                    SC(t0 + t) = s;
                }
            }
        }
        // online softmax and psi_P (:264-342)
        float alpha = 0.0f;
        int live = 0;
        float m_new = m;
        if (active) {
            float rowmax = MASKED;
            for (size_t kk = 0; kk < kj; kk++) {
                float sv = SC(kk);
                if (sv > rowmax) rowmax = sv;
            }
            if (rowmax > m_new) m_new = rowmax;
            live = !(m_new < MASKED * 0.5f);
            if (live) alpha = qbk_expf(m - m_new);
            float esum = 0.0f;
            for (size_t w = 0; w < a.blk4; w++) {
                int c4[4];
                for (int e = 0; e < 4; e++) {
                    size_t kk = 4 * w + e;
                    int pc = 0;
                    if (kk < kj) {
                        float p = live ? qbk_expf(SC(kk) - m_new) : 0.0f;
                        esum += p;
                        float pr = __builtin_rintf(p * 127.0f);
                        pr = pr > 127.0f ? 127.0f : pr;
                        pr = pr < 0.0f ? 0.0f : pr;
                        pc = (int)pr;
                    }
                    c4[e] = pc;
                }
                PH(w) = pack4(c4[0], c4[1], c4[2], c4[3]);
            }
            ell = alpha * ell + esum;
        }
        // O = alpha*O + (P^ V^) * (1/127) * dv  (:344-381)
        const bool chunked = kj > REF_CH;
        for (size_t t0 = 0; t0 < kj; t0 += REF_CH) {
            const size_t tc = kj - t0 < REF_CH ? kj - t0 : REF_CH;
            const size_t tw = (tc + 3) / 4, w0 = t0 / 4;
            __syncthreads();
            for (size_t x = tid; x < dv * tw; x += REF_ROWS) {
                size_t c = x / tw, w = x % tw;
                vc[c * (REF_CH / 4) + w] = a.vhat[((bk * a.nkb + kb) * dv + c) * a.blk4 + w0 + w];
            }
            __syncthreads();
            if (active) {
                for (size_t c = 0; c < dv; c++) {
                    int pv = chunked && t0 > 0 ? a.gpv[c * rows_total + row] : 0;
                    for (size_t w = 0; w < tw; w++)
                        pv = __builtin_amdgcn_sdot4((int)PH(w0 + w), (int)vc[c * (REF_CH / 4) + w], pv,
                                                    false);
                    if (t0 + tc < kj) {
                        a.gpv[c * rows_total + row] = pv;
                    } else {
                        float prev = live ? OUT(c) : 0.0f;
                        OUT(c) = alpha * prev + (float)pv * (1.0f / 127.0f) * vdl[c];
                    }
                }
            }
        }
        if (active) m = m_new;
    }
    if (valid)
        for (size_t c = 0; c < dv; c++) a.out[row * dv + c] = OUT(c) / ell;
}

static std::string shape_debug(const qbk_attn_shape *s) {
    return fmt("AttentionShape { batch: %zu, n_heads: %zu, n_kv_heads: %zu, seq_q: %zu, seq_kv: "
               "%zu, head_dim: %zu, val_dim: %zu }",
               s->batch, s->n_heads, s->n_kv_heads, s->seq_q, s->seq_kv, s->head_dim, s->val_dim);
}

// gpu_attention.rs:598-651 validation, same messages and order.
static int validate_sage(const qbk_attn_shape *s, size_t block_size, const size_t *lens) {
    if (!s) return fail(QBK_ERR_VALIDATION, "null shape");
    if (s->batch == 0 || s->n_heads == 0 || s->n_kv_heads == 0)
        return fail(QBK_ERR_VALIDATION, "attention requires non-empty batch and head dimensions");
    if (s->n_heads % s->n_kv_heads != 0)
        return fail(QBK_ERR_VALIDATION, fmt("n_kv_heads must divide n_heads: n_heads=%zu, "
                                            "n_kv_heads=%zu",
                                            s->n_heads, s->n_kv_heads));
    if (s->seq_q == 0 || s->seq_kv == 0 || s->head_dim == 0 || s->val_dim == 0)
        return fail(QBK_ERR_VALIDATION,
                    "attention requires non-empty sequence and head dimensions");
    if (s->seq_q != s->seq_kv)
        return fail(QBK_ERR_VALIDATION,
                    fmt("sage attention is self-attention over one cache: seq_q=%zu, seq_kv=%zu",
                        s->seq_q, s->seq_kv));
    if (block_size == 0)
        return fail(QBK_ERR_VALIDATION,
                    "sage attention requires a positive block_size ([SA] \xc2\xa7"
                    "4's tile width)");
    if (lens) {
        size_t eq = s->batch * s->n_heads * s->seq_q * s->head_dim;
        size_t ek = s->batch * s->n_kv_heads * s->seq_kv * s->head_dim;
        size_t ev = s->batch * s->n_kv_heads * s->seq_kv * s->val_dim;
        if (lens[0] != eq)
            return fail(QBK_ERR_VALIDATION, fmt("query must hold %zu values for %s, got %zu", eq,
                                                shape_debug(s).c_str(), lens[0]));
        if (lens[1] != ek)
            return fail(QBK_ERR_VALIDATION, fmt("key must hold %zu values for %s, got %zu", ek,
                                                shape_debug(s).c_str(), lens[1]));
        if (lens[2] != ev)
            return fail(QBK_ERR_VALIDATION, fmt("value must hold %zu values for %s, got %zu", ev,
                                                shape_debug(s).c_str(), lens[2]));
    }
    if (s->head_dim > REF_MAXD || s->val_dim > REF_MAXD)
        return fail(QBK_ERR_VALIDATION,
                    fmt("sage attention on this device supports head_dim and val_dim up to %d, "
                        "got head_dim=%zu, val_dim=%zu",
                        REF_MAXD, s->head_dim, s->val_dim));
    return QBK_OK;
}

struct RefPlan {
    RefArgs a;
    size_t ws_bytes, lds_bytes;
    size_t off_kmean, off_kdelta, off_khat, off_vd, off_vhat, off_gsc, off_gph, off_gpv, off_gout;
};

static RefPlan ref_plan(const qbk_attn_shape *s, size_t block) {
    RefPlan P{};
    RefArgs &a = P.a;
    a.B = s->batch;
    a.H = s->n_heads;
    a.Hk = s->n_kv_heads;
    a.S = s->seq_q;
    a.d = s->head_dim;
    a.dv = s->val_dim;
    a.block = block;
    a.nkb = div_ceil(a.S, block);
    a.d4 = div_ceil(a.d, 4);
    a.blk4 = div_ceil(block < a.S ? block : a.S, 4);
    a.sc_lds = block <= REF_CH;
    a.out_lds = a.dv <= 64;
    const size_t rows = a.B * a.H * a.S, bk = a.B * a.Hk;
    size_t off = 0;
    auto take = [&](size_t n) {
        size_t o = off;
        off += round_up(n ? n : 4, 256);
        return o;
    };
    P.off_kmean = take(bk * a.nkb * a.d * 4);
    P.off_kdelta = take(bk * a.S * 4);
    P.off_khat = take(bk * a.S * a.d4 * 4);
    P.off_vd = take(bk * a.nkb * a.dv * 4);
    P.off_vhat = take(bk * a.nkb * a.dv * a.blk4 * 4);
    P.off_gsc = take(a.sc_lds ? 0 : a.blk4 * 4 * rows * 4);
    P.off_gph = take(a.sc_lds ? 0 : a.blk4 * rows * 4);
    P.off_gpv = take(block > REF_CH ? a.dv * rows * 4 : 0);
    P.off_gout = take(a.out_lds ? 0 : a.dv * rows * 4);
    P.ws_bytes = off;
    P.lds_bytes = 4 * (a.d4 * REF_ROWS + a.d4 * 4 + REF_CH + REF_CH * a.d4 + a.dv +
                       a.dv * (REF_CH / 4) + (a.sc_lds ? REF_CH * REF_ROWS + (REF_CH / 4) * REF_ROWS : 0) +
                       (a.out_lds ? a.dv * REF_ROWS : 0));
    return P;
}

static int run_ref(const qbk_attn_shape *s, const float *q, const float *k, const float *v,
                   int causal, size_t block, float *out, void *ws, hipStream_t st) {
    RefPlan P = ref_plan(s, block);
    RefArgs a = P.a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.causal = causal ? 1 : 0;
    a.inv_sqrt_d = 1.0f / sqrtf((float)a.d);
    char *w = (char *)ws;
    a.kmean = (float *)(w + P.off_kmean);
    a.kdelta = (float *)(w + P.off_kdelta);
    a.khat = (uint32_t *)(w + P.off_khat);
    a.vd = (float *)(w + P.off_vd);
    a.vhat = (uint32_t *)(w + P.off_vhat);
    a.gsc = (float *)(w + P.off_gsc);
    a.gph = (uint32_t *)(w + P.off_gph);
    a.gpv = (int *)(w + P.off_gpv);
    a.gout = (float *)(w + P.off_gout);
    hipLaunchKernelGGL(sage_ref_prep, dim3((unsigned)a.nkb, (unsigned)(a.B * a.Hk)), dim3(256), 0,
                       st, a);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(sage_ref_main, dim3((unsigned)div_ceil(a.S, REF_ROWS), (unsigned)(a.B * a.H)),
                       dim3(REF_ROWS), P.lds_bytes, st, a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

// ======================================================================
// 2. block-scaled scheme (INT8 MFMA Q.K^T, fp16 MFMA P.V)
// ======================================================================

#define BLK 64   // quantisation block and key tile (tokens)
#define BQ 128   // query rows per workgroup (4 waves x 32)
#define HD 128   // head_dim == val_dim
#define LOG2E_F 1.44269504088896341f
#define KS_PITCH 144  // bytes per K^ row in LDS (128 + 16 pad)
#define VS_PITCH 72   // fp16 per V^T row in LDS (64 + 8 pad)

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

struct BlkArgs {
    const uint16_t *q, *k, *v;  // bf16
    uint16_t *out;              // bf16
    size_t B, H, Hk, S, nblk, Sp;
    int causal;
    float inv_sqrt_d;
    float *kpart;     // [B*Hk][nblk][HD]
    float *kmean;     // [B*Hk][HD]
    int8_t *khat;     // [B*Hk][Sp][HD]
    float *kscale;    // [B*Hk][nblk]
    int8_t *qhat;     // [B*H][Sp][HD]
    float *qscale;    // [B*H][nblk]
    uint16_t *vt;     // [B*Hk][nblk][HD][BLK] fp16 (V^T per key block)
};

// chunk partial sums of K per channel, token order within the chunk
__global__ void __launch_bounds__(HD) blk_kpart(BlkArgs a) {
    const size_t blk = blockIdx.x, bk = blockIdx.y, c = threadIdx.x;
    const uint16_t *K = a.k + bk * a.S * HD;
    size_t t0 = blk * BLK, t1 = t0 + BLK < a.S ? t0 + BLK : a.S;
    float part = 0.0f;
    for (size_t t = t0; t < t1; t++) part += bf16_to_f32(K[t * HD + c]);
    a.kpart[(bk * a.nblk + blk) * HD + c] = part;
}

__device__ __forceinline__ float block_max(float v, float *red) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

// K: mean (chunk partials summed in chunk order), smoothing, block scale,
// codes; V: bf16 -> fp16, transposed per key block.  One workgroup per
// (kv head, block).
__global__ void __launch_bounds__(256) blk_kvquant(BlkArgs a) {
    __shared__ float mean[HD];
    __shared__ float red[4];
    const size_t blk = blockIdx.x, bk = blockIdx.y;
    const int tid = threadIdx.x;
    if (tid < HD) {
        float tot = 0.0f;
        for (size_t p = 0; p < a.nblk; p++) tot += a.kpart[(bk * a.nblk + p) * HD + tid];
        float mv = tot / (float)a.S;
        mean[tid] = mv;
        if (blk == 0) a.kmean[bk * HD + tid] = mv;
    }
    __syncthreads();
    const size_t t0 = blk * BLK;
    const uint16_t *K = a.k + bk * a.S * HD;
    // 64 tokens x 128 channels = 8192 elements, 32 per thread
    float peak = 0.0f;
    for (int e = tid; e < BLK * HD; e += 256) {
        size_t t = t0 + e / HD;
        int c = e % HD;
        if (t < a.S) peak = fmaxf(peak, fabsf(bf16_to_f32(K[t * HD + c]) - mean[c]));
    }
    peak = block_max(peak, red);
    const float inv = peak > 0.0f ? 127.0f / peak : 0.0f;
    if (tid == 0) a.kscale[bk * a.nblk + blk] = peak > 0.0f ? peak / 127.0f : 1.0f;
    int8_t *KH = a.khat + (bk * a.Sp + t0) * HD;
    for (int e4 = tid; e4 < BLK * HD / 4; e4 += 256) {
        int e = e4 * 4;
        size_t t = t0 + e / HD;
        int c = e % HD;
        int c4[4] = {0, 0, 0, 0};
        if (t < a.S)
            for (int u = 0; u < 4; u++) c4[u] = q8((bf16_to_f32(K[t * HD + c + u]) - mean[c + u]) * inv);
        *(uint32_t *)(KH + e) = pack4(c4[0], c4[1], c4[2], c4[3]);
    }
    // V^T block: vt[c][j] for j < 64 (zero beyond S)
    const uint16_t *V = a.v + bk * a.S * HD;
    uint16_t *VT = a.vt + (bk * a.nblk + blk) * HD * BLK;
    for (int e = tid; e < BLK * HD; e += 256) {
        int c = e / BLK, j = e % BLK;
        size_t t = t0 + j;
        _Float16 h = (_Float16)(t < a.S ? bf16_to_f32(V[t * HD + c]) : 0.0f);
        VT[c * BLK + j] = __builtin_bit_cast(uint16_t, h);
    }
}

// Q: 1/sqrt(d) folded, block scale, codes.  One workgroup per (head, block).
__global__ void __launch_bounds__(256) blk_qquant(BlkArgs a) {
    __shared__ float red[4];
    const size_t blk = blockIdx.x, bh = blockIdx.y;
    const int tid = threadIdx.x;
    const size_t t0 = blk * BLK;
    const uint16_t *Q = a.q + bh * a.S * HD;
    float peak = 0.0f;
    for (int e = tid; e < BLK * HD; e += 256) {
        size_t t = t0 + e / HD;
        if (t < a.S) peak = fmaxf(peak, fabsf(bf16_to_f32(Q[t * HD + e % HD]) * a.inv_sqrt_d));
    }
    peak = block_max(peak, red);
    const float inv = peak > 0.0f ? 127.0f / peak : 0.0f;
    if (tid == 0) a.qscale[bh * a.nblk + blk] = peak > 0.0f ? peak / 127.0f : 1.0f;
    int8_t *QH = a.qhat + (bh * a.Sp + t0) * HD;
    for (int e4 = tid; e4 < BLK * HD / 4; e4 += 256) {
        int e = e4 * 4;
        size_t t = t0 + e / HD;
        int c = e % HD;
        int c4[4] = {0, 0, 0, 0};
        if (t < a.S)
            for (int u = 0; u < 4; u++) c4[u] = q8((bf16_to_f32(Q[t * HD + c + u]) * a.inv_sqrt_d) * inv);
        *(uint32_t *)(QH + e) = pack4(c4[0], c4[1], c4[2], c4[3]);
    }
}

#pragma clang fp contract(fast)

// Main pass.  Workgroup: (128-query tile, batch*head); wave w owns queries
// q0 + 32w .. +31 (two 16-query MFMA tiles, one quantisation block).
// Per key block (64 keys, double-buffered in LDS: K^ 8 KB, V^T 16 KB):
//   S^T[64 x 32] = K^[64 x 128] . Q^T  -- 4 key tiles x 2 query tiles x 2
//                  d-chunks of i8 16x16x64; C lane l holds query l%16 and
//                  keys 4*(l/16)+i of its key tile;
//   online softmax per query column (4 lanes share a query: xor 16, 32);
//   O^T[128 x 32] += V^T[128 x 64] . P^T -- 8 channel tiles x 2 query tiles
//                  x 2 key chunks of f16 16x16x32, P^T taken straight from
//                  the S^T registers: fragment element e of lane l is key
//                  4*(l/16)+e of key tile 2c (e<4) or 16 + 4*(l/16)+(e-4)
//                  of key tile 2c+1, and V^T is read with the same map.
__global__ void __launch_bounds__(256) blk_attn(BlkArgs a) {
    // LDS rows padded to 144 bytes: the 16 lanes of a fragment read rows
    // 144 B apart, which lands them on disjoint bank groups.
    __shared__ __attribute__((aligned(16))) int8_t ks[2][BLK * KS_PITCH];
    __shared__ __attribute__((aligned(16))) uint16_t vs[2][HD * VS_PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const size_t bk = b * a.Hk + h / (a.H / a.Hk);
    const size_t q0 = (size_t)blockIdx.x * BQ;
    const size_t qw = q0 + 32 * wave;
    const int g = lane >> 4, col = lane & 15;

    // Q^ fragments (B operand): query col, 16 consecutive d per lane
    i32x4_t qf[2][2];
    for (int qt = 0; qt < 2; qt++)
        for (int dc = 0; dc < 2; dc++) {
            size_t qi = qw + 16 * qt + col;
            const int8_t *src = a.qhat + (bh * a.Sp + qi) * HD + dc * 64 + 16 * g;
            qf[qt][dc] = *(const i32x4_t *)src;
        }
    const bool wave_live = qw < a.S;
    const float qsc = wave_live ? a.qscale[bh * a.nblk + qw / BLK] : 0.0f;

    f32x4_t o[2][8];
    for (int qt = 0; qt < 2; qt++)
        for (int ct = 0; ct < 8; ct++) o[qt][ct] = f32x4_t{0, 0, 0, 0};
    float mrow[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};
    float lrow[2] = {0.0f, 0.0f};  // per-lane partial row sums

    size_t kb_end = a.nblk;
    if (a.causal) {
        size_t last = q0 + BQ - 1 < a.S - 1 ? q0 + BQ - 1 : a.S - 1;
        kb_end = last / BLK + 1;
    }
    size_t wlast = qw + 31 < a.S - 1 ? qw + 31 : a.S - 1;
    const size_t wave_kb_end = a.causal ? wlast / BLK + 1 : a.nblk;

    // Next tile staged in registers: the global loads are issued before the
    // block's math and written to LDS after it, so their latency overlaps
    // the MFMA/softmax work.  K^ tile: 512 x 16 B chunks (2 per thread),
    // V^T tile: 1024 x 16 B chunks (4 per thread).
    uint4 kreg[2], vreg[4];
    auto fetch_tile = [&](size_t kb) {
        const uint4 *ksrc = (const uint4 *)(a.khat + (bk * a.Sp + kb * BLK) * HD);
        for (int u = 0; u < 2; u++) kreg[u] = ksrc[tid + 256 * u];
        const uint4 *vsrc = (const uint4 *)(a.vt + (bk * a.nblk + kb) * HD * BLK);
        for (int u = 0; u < 4; u++) vreg[u] = vsrc[tid + 256 * u];
    };
    auto store_tile = [&](int buf) {
        for (int u = 0; u < 2; u++) {
            int x = tid + 256 * u;  // row x/8 (128 B = 8 chunks), chunk x%8
            *(uint4 *)&ks[buf][(x >> 3) * KS_PITCH + (x & 7) * 16] = kreg[u];
        }
        for (int u = 0; u < 4; u++) {
            int x = tid + 256 * u;  // row x/8 (64 fp16 = 8 chunks), chunk x%8
            *(uint4 *)&vs[buf][(x >> 3) * VS_PITCH + (x & 7) * 8] = vreg[u];
        }
    };

    fetch_tile(0);
    store_tile(0);
    __syncthreads();
    for (size_t kb = 0; kb < kb_end; kb++) {
        const int buf = kb & 1;
        const bool more = kb + 1 < kb_end;
        if (more) fetch_tile(kb + 1);
        if (wave_live && kb < wave_kb_end) {
            const float cs = (qsc * a.kscale[bk * a.nblk + kb]) * LOG2E_F;
            // ---- S^T = K^ Q^T
            i32x4_t st[4][2];
            for (int kt = 0; kt < 4; kt++)
                for (int qt = 0; qt < 2; qt++) st[kt][qt] = i32x4_t{0, 0, 0, 0};
            for (int kt = 0; kt < 4; kt++)
                for (int dc = 0; dc < 2; dc++) {
                    i32x4_t kf = *(const i32x4_t *)&ks[buf][(16 * kt + col) * KS_PITCH + dc * 64 + 16 * g];
                    for (int qt = 0; qt < 2; qt++)
                        st[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf, qf[qt][dc], st[kt][qt], 0, 0, 0);
                }
            // ---- softmax on the S^T columns
            const bool diag = a.causal && (kb * BLK + BLK - 1 > qw);
            const bool ragged = !a.causal && (kb * BLK + BLK > a.S);
            f16x8_t pf[2][2];  // [qt][key chunk]
            for (int qt = 0; qt < 2; qt++) {
                const size_t qi = qw + 16 * qt + col;
                float sv[4][4];
                float mx = -__builtin_huge_valf();
                for (int kt = 0; kt < 4; kt++)
                    for (int i = 0; i < 4; i++) {
                        float s = (float)st[kt][qt][i] * cs;
                        size_t kj = kb * BLK + 16 * kt + 4 * g + i;
                        if ((diag && kj > qi) || (ragged && kj >= a.S)) s = -__builtin_huge_valf();
                        sv[kt][i] = s;
                        mx = fmaxf(mx, s);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float mnew = fmaxf(mrow[qt], mx);
                const float alpha = __builtin_amdgcn_exp2f(mrow[qt] - mnew);
                mrow[qt] = mnew;
                float ls = 0.0f;
                for (int kt = 0; kt < 4; kt++)
                    for (int i = 0; i < 4; i++) {
                        float p = __builtin_amdgcn_exp2f(sv[kt][i] - mnew);
                        sv[kt][i] = p;
                        ls += p;
                    }
                lrow[qt] = alpha * lrow[qt] + ls;
                for (int ct = 0; ct < 8; ct++) o[qt][ct] *= alpha;
                for (int kc = 0; kc < 2; kc++) {
                    f16x8_t f;
                    for (int i = 0; i < 4; i++) {
                        f[i] = (_Float16)sv[2 * kc][i];
                        f[4 + i] = (_Float16)sv[2 * kc + 1][i];
                    }
                    pf[qt][kc] = f;
                }
            }
            // ---- O^T += V^T P^T
            for (int ct = 0; ct < 8; ct++)
                for (int kc = 0; kc < 2; kc++) {
                    const uint16_t *vrow = &vs[buf][(16 * ct + col) * VS_PITCH + 32 * kc];
                    uint2 lo = *(const uint2 *)(vrow + 4 * g);
                    uint2 hi = *(const uint2 *)(vrow + 16 + 4 * g);
                    uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    f16x8_t vf = __builtin_bit_cast(f16x8_t, vv);
                    for (int qt = 0; qt < 2; qt++)
                        o[qt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[qt][kc], o[qt][ct], 0, 0, 0);
                }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }
    if (!wave_live) return;
    // ---- normalise and store: lane holds query col, channels 4*(l/16)+i
    for (int qt = 0; qt < 2; qt++) {
        float l = lrow[qt];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float inv = 1.0f / l;
        const size_t qi = qw + 16 * qt + col;
        if (qi >= a.S) continue;
        uint16_t *dst = a.out + (bh * a.S + qi) * HD;
        for (int ct = 0; ct < 8; ct++) {
            uint32_t w0 = (uint32_t)f32_to_bf16(o[qt][ct][0] * inv) |
                          ((uint32_t)f32_to_bf16(o[qt][ct][1] * inv) << 16);
            uint32_t w1 = (uint32_t)f32_to_bf16(o[qt][ct][2] * inv) |
                          ((uint32_t)f32_to_bf16(o[qt][ct][3] * inv) << 16);
            *(uint2 *)(dst + 16 * ct + 4 * g) = make_uint2(w0, w1);
        }
    }
}

#pragma clang fp contract(off)

// export the pre-pass stages in natural layouts (parity checks)
__global__ void blk_export(BlkArgs a, int8_t *qhat, int8_t *khat, uint16_t *vh) {
    size_t x = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t nq = a.B * a.H * a.S * HD, nk = a.B * a.Hk * a.S * HD;
    if (x < nq) {
        size_t bh = x / (a.S * HD), rem = x % (a.S * HD);
        qhat[x] = a.qhat[bh * a.Sp * HD + rem];
    }
    if (x < nk) {
        size_t bk = x / (a.S * HD), rem = x % (a.S * HD);
        size_t t = rem / HD, c = rem % HD;
        khat[x] = a.khat[bk * a.Sp * HD + rem];
        vh[x] = a.vt[((bk * a.nblk + t / BLK) * HD + c) * BLK + t % BLK];
    }
}

struct BlkPlan {
    BlkArgs a;
    size_t ws;
    size_t o_kpart, o_kmean, o_khat, o_kscale, o_qhat, o_qscale, o_vt;
};

static BlkPlan blk_plan(const qbk_attn_shape *s) {
    BlkPlan P{};
    BlkArgs &a = P.a;
    a.B = s->batch;
    a.H = s->n_heads;
    a.Hk = s->n_kv_heads;
    a.S = s->seq_q;
    a.nblk = div_ceil(a.S, BLK);
    a.Sp = round_up(a.S, BQ);
    const size_t bk = a.B * a.Hk, bh = a.B * a.H;
    size_t off = 0;
    auto take = [&](size_t n) {
        size_t o = off;
        off += round_up(n ? n : 4, 256);
        return o;
    };
    P.o_kpart = take(bk * a.nblk * HD * 4);
    P.o_kmean = take(bk * HD * 4);
    P.o_khat = take(bk * a.Sp * HD);
    P.o_kscale = take(bk * a.nblk * 4);
    P.o_qhat = take(bh * a.Sp * HD);
    P.o_qscale = take(bh * a.nblk * 4);
    P.o_vt = take(bk * a.nblk * HD * BLK * 2);
    P.ws = off;
    return P;
}

static int validate_blk(const qbk_attn_shape *s) {
    int rc = validate_sage(s, 1, nullptr);
    if (rc) return rc;
    if (s->head_dim != HD || s->val_dim != HD)
        return fail(QBK_ERR_VALIDATION,
                    fmt("block-scaled sage attention needs head_dim == val_dim == %d, got "
                        "head_dim=%zu, val_dim=%zu",
                        HD, s->head_dim, s->val_dim));
    return QBK_OK;
}

static int run_blk_prepass(BlkPlan &P, const qbk_attn_shape *s, const uint16_t *q,
                           const uint16_t *k, const uint16_t *v, void *ws, hipStream_t st) {
    BlkArgs &a = P.a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.inv_sqrt_d = 1.0f / sqrtf((float)HD);
    char *w = (char *)ws;
    a.kpart = (float *)(w + P.o_kpart);
    a.kmean = (float *)(w + P.o_kmean);
    a.khat = (int8_t *)(w + P.o_khat);
    a.kscale = (float *)(w + P.o_kscale);
    a.qhat = (int8_t *)(w + P.o_qhat);
    a.qscale = (float *)(w + P.o_qscale);
    a.vt = (uint16_t *)(w + P.o_vt);
    // Query codes of tokens >= nblk*64 (up to the 128-row tile) are never
    // written: those queries are computed and discarded, and each query
    // column of the MFMA tiles is independent of the others.
    hipLaunchKernelGGL(blk_kpart, dim3((unsigned)a.nblk, (unsigned)(a.B * a.Hk)), dim3(HD), 0, st, a);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(blk_kvquant, dim3((unsigned)a.nblk, (unsigned)(a.B * a.Hk)), dim3(256), 0, st, a);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(blk_qquant, dim3((unsigned)a.nblk, (unsigned)(a.B * a.H)), dim3(256), 0, st, a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_attention_sage(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, size_t q_len,
                       const float *k, size_t k_len, const float *v, size_t v_len, int causal,
                       size_t block_size, float *out) {
    size_t lens[3] = {q_len, k_len, v_len};
    int rc;
    if ((rc = validate_sage(shape, block_size, lens))) return rc;
    if ((rc = bind(ctx))) return rc;
    RefPlan P = ref_plan(shape, block_size);
    CallStream cs;
    DevBuf dq, dk, dvb, dout, dws;
    size_t on = shape->batch * shape->n_heads * shape->seq_q * shape->val_dim;
    if ((rc = cs.create()) || (rc = dq.alloc(q_len * 4)) || (rc = dk.alloc(k_len * 4)) ||
        (rc = dvb.alloc(v_len * 4)) || (rc = dout.alloc(on * 4)) || (rc = dws.alloc(P.ws_bytes)))
        return rc;
    QBK_HIP(hipMemcpyAsync(dq.p, q, q_len * 4, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dk.p, k, k_len * 4, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dvb.p, v, v_len * 4, hipMemcpyHostToDevice, cs.s));
    if ((rc = run_ref(shape, (const float *)dq.p, (const float *)dk.p, (const float *)dvb.p, causal,
                      block_size, (float *)dout.p, dws.p, cs.s)))
        return rc;
    QBK_HIP(hipMemcpyAsync(out, dout.p, on * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_attention_sage_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q,
                           const float *k, const float *v, int causal, size_t block_size,
                           float *out, void *stream) {
    int rc;
    if ((rc = validate_sage(shape, block_size, nullptr))) return rc;
    if ((rc = bind(ctx))) return rc;
    // the reference scheme's per-(kv head, block) products live in a
    // per-call device buffer, freed once the stream has consumed it
    RefPlan P = ref_plan(shape, block_size);
    void *ws = nullptr;
    QBK_HIP(hipMallocAsync(&ws, P.ws_bytes, (hipStream_t)stream));
    rc = run_ref(shape, q, k, v, causal, block_size, out, ws, (hipStream_t)stream);
    QBK_HIP(hipFreeAsync(ws, (hipStream_t)stream));
    return rc;
}

size_t qbk_sage_blk_workspace_size(const qbk_attn_shape *shape) {
    if (!shape) return 0;
    return blk_plan(shape).ws;
}

int qbk_attention_sage_blk_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q,
                               const uint16_t *k, const uint16_t *v, int causal, uint16_t *out,
                               void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if ((rc = validate_blk(shape))) return rc;
    if ((rc = bind(ctx))) return rc;
    BlkPlan P = blk_plan(shape);
    if (workspace_size < P.ws)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs",
                        workspace_size, P.ws));
    hipStream_t st = (hipStream_t)stream;
    if ((rc = run_blk_prepass(P, shape, q, k, v, workspace, st))) return rc;
    P.a.out = out;
    P.a.causal = causal ? 1 : 0;
    hipLaunchKernelGGL(blk_attn, dim3((unsigned)div_ceil(P.a.S, BQ), (unsigned)(P.a.B * P.a.H)),
                       dim3(256), 0, st, P.a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int qbk_sage_blk_quantize_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q,
                              const uint16_t *k, const uint16_t *v, int8_t *qhat, float *qscale,
                              int8_t *khat, float *kscale, float *kmean, uint16_t *vh,
                              void *stream) {
    int rc;
    if ((rc = validate_blk(shape))) return rc;
    if ((rc = bind(ctx))) return rc;
    BlkPlan P = blk_plan(shape);
    hipStream_t st = (hipStream_t)stream;
    void *ws = nullptr;
    QBK_HIP(hipMallocAsync(&ws, P.ws, st));
    rc = run_blk_prepass(P, shape, q, k, v, ws, st);
    if (!rc) {
        const BlkArgs &a = P.a;
        size_t n = a.B * (a.H > a.Hk ? a.H : a.Hk) * a.S * HD;
        hipLaunchKernelGGL(blk_export, dim3((unsigned)div_ceil(n, 256)), dim3(256), 0, st, a, qhat,
                           khat, vh);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = fail(QBK_ERR_DEVICE, fmt("blk_export: %s", hipGetErrorString(e)));
    }
    if (!rc) {
        const BlkArgs &a = P.a;
        hipError_t e = hipMemcpyAsync(qscale, a.qscale, a.B * a.H * a.nblk * 4, hipMemcpyDeviceToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(kscale, a.kscale, a.B * a.Hk * a.nblk * 4, hipMemcpyDeviceToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(kmean, a.kmean, a.B * a.Hk * HD * 4, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) rc = fail(QBK_ERR_DEVICE, fmt("hipMemcpyAsync: %s", hipGetErrorString(e)));
    }
    QBK_HIP(hipFreeAsync(ws, st));
    return rc;
}

}  // extern "C"
