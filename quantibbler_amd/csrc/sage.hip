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
//    fp16, O^T += V^T.P^T on fp16 MFMA (16x16x32) with P kept in registers
//    and the softmax row sums l = sum of the fp16 P on the same MFMA.
#include <math.h>
#include <string.h>

#include <string>

#include "qbk_internal.h"
#include "q4_operand.h"

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

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

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
    // K / V element strides between consecutive tokens of one kv head and
    // between kv heads: head-major (B, Hk, S, d) by default; the decode
    // step reads a row-major cache (S, Hk, d) in place
    size_t k_tok, k_head, v_tok, v_head;
    // pre-pass products, laid out for pst tokens (pnkb key blocks) per kv
    // head: S (nkb) except for a decode state sized for a cache's capacity;
    // the pre-pass quantises key blocks kb0 .. nkb-1 (kb0 > 0 only when the
    // codes of the earlier, complete blocks are kept from a previous step)
    size_t pst, pnkb, kb0;
    float *kmean;     // [B*Hk*pnkb][d]
    float *kdelta;    // [B*Hk*pst]
    uint32_t *khat;   // [B*Hk*pst][d4]
    float *vd;        // [B*Hk*pnkb][dv]
    uint32_t *vhat;   // [B*Hk*pnkb][dv][blk4]
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
// The f32 operations are the reference's; the block's K (then V) is staged
// through LDS in chunks of REF_PREP_CH(maxd) tokens with coalesced loads --
// a block that fits is read from memory once -- and the work is spread so
// that every thread has some: a thread per channel for the sums and V, a
// wave per token for K (lane l holds channels 4l .. 4l+3 -- the peak is a
// max, so a wave reduction gives the reference's value -- and writes their
// code word).
#define REF_PREP_LDS 61440  // with the static arrays, within the 64 KiB a launch gets by default
__host__ __device__ __forceinline__ size_t ref_prep_ch(size_t maxd) {
    return (REF_PREP_LDS / (4 * maxd)) & ~(size_t)3;  // tokens per LDS chunk (a multiple of 4)
}

__global__ void __launch_bounds__(256) sage_ref_prep(RefArgs a) {
    extern __shared__ __attribute__((aligned(16))) float tile[];  // [ch][maxd]
    __shared__ float km[REF_MAXD];
    const size_t kb = a.kb0 + blockIdx.x, bk = blockIdx.y;
    const size_t j0 = kb * a.block;
    const size_t j1 = j0 + a.block < a.S ? j0 + a.block : a.S;
    const size_t kj = j1 - j0;
    const float *K = a.k + bk * a.k_head;
    const float *V = a.v + bk * a.v_head;
    const size_t maxd = a.d > a.dv ? a.d : a.dv, CH = ref_prep_ch(maxd);
    const bool one = kj <= CH;  // the whole block in one chunk: load once
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwave = nt >> 6;
    // tokens t0 .. t0+tc-1 (w channels each) into the tile: a wave per token,
    // four tokens a pass, every load of the pass issued before its stores
    // (indices clamped into the chunk, so the loads are unconditional)
    auto stage = [&](const float *X, size_t tok, size_t t0, size_t tc, size_t w) {
        __syncthreads();
        for (size_t tb = 0; tb < tc; tb += 4 * (size_t)nwave) {
            float v[4][4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                size_t t = tb + (size_t)(u * nwave + wave);
                t = t < tc ? t : tc - 1;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    size_t c = (size_t)(lane + 64 * e);
                    c = c < w ? c : w - 1;
                    v[u][e] = X[(t0 + t) * tok + c];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const size_t t = tb + (size_t)(u * nwave + wave);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const size_t c = (size_t)(lane + 64 * e);
                    if (t < tc && c < w) tile[t * maxd + c] = v[u][e];
                }
            }
        }
        __syncthreads();
    };
    // A block whose K and V each take at most 8 16-byte loads a thread (and
    // whose rows are 16-byte aligned): every load of the block is issued at
    // once, V held in registers while K is worked on -- one trip to memory
    // instead of one per staged pass.
    const uint32_t dq = (uint32_t)(a.d / 4), vq = (uint32_t)(a.dv / 4);
    const bool fast = one && a.d % 4 == 0 && a.dv % 4 == 0 && a.k_tok % 4 == 0 && a.v_tok % 4 == 0 &&
                      ((((uintptr_t)K) | ((uintptr_t)V)) & 15) == 0 && kj * dq <= 8 * (size_t)nt &&
                      kj * vq <= 8 * (size_t)nt;
    const uint32_t nkq = (uint32_t)kj * dq, nvq = (uint32_t)kj * vq;
    f32x4_t vr[8];
    if (fast) {
        f32x4_t kr[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t it = (uint32_t)(tid + u * nt), i = it < nkq ? it : nkq - 1;
            kr[u] = *(const f32x4_t *)(K + (j0 + i / dq) * a.k_tok + 4 * (i % dq));
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t it = (uint32_t)(tid + u * nt), i = it < nvq ? it : nvq - 1;
            vr[u] = *(const f32x4_t *)(V + (j0 + i / vq) * a.v_tok + 4 * (i % vq));
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t it = (uint32_t)(tid + u * nt);
            if (it < nkq) *(f32x4_t *)&tile[(it / dq) * maxd + 4 * (it % dq)] = kr[u];
        }
        __syncthreads();
    }
    // block mean of K, sequential over the tokens
    float ssum = 0.0f;
    for (size_t t0 = j0; t0 < j1; t0 += CH) {
        const size_t tc = j1 - t0 < CH ? j1 - t0 : CH;
        if (!fast) stage(K, a.k_tok, t0, tc, a.d);
        if ((size_t)tid < a.d)
#pragma unroll 8
            for (size_t t = 0; t < tc; t++) ssum += tile[t * maxd + tid];
    }
    if ((size_t)tid < a.d) {
        const float m = ssum / (float)kj;
        km[tid] = m;
        a.kmean[(bk * a.pnkb + kb) * a.d + tid] = m;
    }
    __syncthreads();
    // per-token peak, delta and codes: a wave per token, or a half-wave per
    // token when the codes fit in 32 words (d <= 128)
    const bool half = a.d4 <= 32;
    const int tpw = half ? 2 : 1, sub = half ? lane >> 5 : 0, wl = half ? lane & 31 : lane;
    const size_t c0 = 4 * (size_t)wl;  // this lane's channels
    for (size_t t0 = j0; t0 < j1; t0 += CH) {
        const size_t tc = j1 - t0 < CH ? j1 - t0 : CH;
        if (!one) stage(K, a.k_tok, t0, tc, a.d);
        for (size_t tb = (size_t)(wave * tpw); tb < tc; tb += (size_t)(nwave * tpw)) {
            const size_t t = tb + sub < tc ? tb + sub : tc - 1;  // a past-the-end half repeats a token
            const size_t jj = t0 + t;
            float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            float kpeak = 0.0f;
            for (int e = 0; e < 4; e++) {
                const size_t c = c0 + e;
                if (c < a.d) {
                    g[e] = tile[t * maxd + c] - km[c];
                    float ag = g[e] < 0.0f ? 0.0f - g[e] : g[e];
                    if (ag > kpeak) kpeak = ag;
                }
            }
            for (int o = half ? 16 : 32; o >= 1; o >>= 1) {
                const float w = __shfl_xor(kpeak, o, 64);
                kpeak = w > kpeak ? w : kpeak;
            }
            float kdelta = 1.0f;
            if (kpeak > 0.0f) kdelta = kpeak / 127.0f;
            if (wl == 0) a.kdelta[bk * a.pst + jj] = kdelta;
            if ((size_t)wl < a.d4) {
                int c4[4];
                for (int e = 0; e < 4; e++) c4[e] = c0 + e < a.d ? q8(g[e] / kdelta) : 0;
                a.khat[(bk * a.pst + jj) * a.d4 + wl] = pack4(c4[0], c4[1], c4[2], c4[3]);
            }
        }
    }
    // V: per-channel peak over the block, then codes four tokens a word
    float vpeak = 0.0f;
    for (size_t t0 = j0; t0 < j1; t0 += CH) {
        const size_t tc = j1 - t0 < CH ? j1 - t0 : CH;
        if (fast) {
            __syncthreads();  // every wave is done with K's tile
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t it = (uint32_t)(tid + u * nt);
                if (it < nvq) *(f32x4_t *)&tile[(it / vq) * maxd + 4 * (it % vq)] = vr[u];
            }
            __syncthreads();
        } else {
            stage(V, a.v_tok, t0, tc, a.dv);
        }
        if ((size_t)tid < a.dv)
#pragma unroll 8
            for (size_t t = 0; t < tc; t++) {
                float x = tile[t * maxd + tid];
                float ax = x < 0.0f ? 0.0f - x : x;
                if (ax > vpeak) vpeak = ax;
            }
    }
    if ((size_t)tid < a.dv) {
        const float vd = vpeak > 0.0f ? vpeak / 127.0f : 1.0f;
        km[tid] = vd;  // the K means are no longer needed
        a.vd[(bk * a.pnkb + kb) * a.dv + tid] = vd;
    }
    __syncthreads();
    // codes four tokens a word, the (channel, word) items over every thread
    const uint32_t dv = (uint32_t)a.dv;
    uint32_t *vrow = a.vhat + (bk * a.pnkb + kb) * a.dv * a.blk4;
    for (size_t t0 = j0; t0 < j1; t0 += CH) {
        const size_t tc = j1 - t0 < CH ? j1 - t0 : CH;
        if (!one) stage(V, a.v_tok, t0, tc, a.dv);
        const uint32_t tw = (uint32_t)((tc + 3) / 4);
        for (uint32_t x = tid; x < dv * tw; x += nt) {
            const uint32_t c = x % dv, w = x / dv;
            const float vd = km[c];
            int c4[4];
            for (int e = 0; e < 4; e++) {
                const size_t t = 4 * w + e;
                c4[e] = t < tc ? q8(tile[t * maxd + c] / vd) : 0;
            }
            vrow[c * a.blk4 + (t0 - j0) / 4 + w] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
    }
}

// LDS bytes of a sage_ref_prep launch
static size_t ref_prep_lds(size_t d, size_t dv, size_t block) {
    const size_t maxd = d > dv ? d : dv, ch = ref_prep_ch(maxd);
    return 4 * maxd * (block < ch ? block : ch);
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
        for (size_t c = tid; c < a.d; c += REF_ROWS) kms[c] = a.kmean[(bk * a.pnkb + kb) * a.d + c];
        for (size_t c = tid; c < dv; c += REF_ROWS) vdl[c] = a.vd[(bk * a.pnkb + kb) * dv + c];
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
            for (size_t t = tid; t < tc; t += REF_ROWS) kdl[t] = a.kdelta[bk * a.pst + j0 + t0 + t];
            for (size_t x = tid; x < tc * d4; x += REF_ROWS)
                kc[x] = a.khat[(bk * a.pst + j0 + t0) * d4 + x];
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
                vc[c * (REF_CH / 4) + w] = a.vhat[((bk * a.pnkb + kb) * dv + c) * a.blk4 + w0 + w];
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
        // gpu_attention.rs:652-669: the reference face's u32 index ceiling over
        // the operands and every per-row extent its kernel derives
        const uint64_t rows = (uint64_t)s->batch * s->n_heads * s->seq_q;
        uint64_t largest = eq > ek ? eq : ek;
        const uint64_t ext[5] = {ev, rows * s->head_dim, rows * s->val_dim, rows * block_size,
                                 rows * block_size + block_size};
        for (uint64_t x : ext) largest = x > largest ? x : largest;
        if (largest > 0xFFFFFFFFull)
            return fail(QBK_ERR_VALIDATION, "sage attention inputs exceed the device u32 index ceiling "
                                            "(4294967295); use the reference face");
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
    a.k_tok = a.d;
    a.k_head = a.S * a.d;
    a.v_tok = a.dv;
    a.v_head = a.S * a.dv;
    a.pst = a.S;
    a.pnkb = a.nkb;
    a.kb0 = 0;
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
    hipLaunchKernelGGL(sage_ref_prep, dim3((unsigned)a.nkb, (unsigned)(a.B * a.Hk)), dim3(256),
                       ref_prep_lds(a.d, a.dv, a.block), st, a);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(sage_ref_main, dim3((unsigned)div_ceil(a.S, REF_ROWS), (unsigned)(a.B * a.H)),
                       dim3(REF_ROWS), P.lds_bytes, st, a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

// ----------------------------------------------------------------------
// 1b. one decode step of the reference scheme over a KV cache
// ----------------------------------------------------------------------
//
// engine/mod.rs:984-1030 (gqa_attention_sage) pads the one query of a decode
// step into row 0 of a (pos + 1)-row problem, runs the scheme with causal =
// false and reads row 0.  Row i of the scheme depends only on query i and
// the cache (Q is quantised per row, K and V per key block), so row 0 alone
// is that step -- here in O(seq) instead of O(seq^2): the key-block loop
// that the main pass runs within one lane is spread over workgroups, each
// f32 value formed by the same operations in the same order (the sums that
// the main pass makes sequential stay sequential; the maxima and integer
// dot products are order-free).  The pre-pass reads the row-major cache
// (seq, n_kv_heads, d) in place -- the layout KvCache::head_major gathers
// from (engine/mod.rs:1236-1268).
//   sage_dec_scores  (key block, head): the block's shift, scores, max
//   sage_dec_pv      (key block, head): the running max, live flag and alpha
//                    of the block, p, their sum in key order, P codes, and
//                    each channel's (P^.V^)/127 * dv term of the block
//   sage_dec_combine (head): l and O over the blocks in order, then O / l

#define DEC_CH 4096  // keys of a block whose p and codes sit in LDS at once

// A workgroup barrier that orders LDS only: __syncthreads() also fences
// global memory, which waits for every load in flight -- the key or value
// codes a kernel issues ahead of the work that does not need them.
__device__ __forceinline__ void dec_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

struct DecArgs {
    RefArgs r;                           // shape (S = seq_kv), pre-pass products
    float *sc;                           // [H][S] scores, then p
    float *bmax, *balpha, *besum;        // [H][nkb]
    int *blive;                          // [H][nkb]
    float *pvt;                          // [H][nkb][dv]
    uint32_t *qsw;                       // [H][d4] the query's codes (grouped kernels)
    float *qdl;                          // [H] and its delta
    float *mprev;                        // [H][nkb] running max before each block, or null
    const float *op_s2;                  // combine: the next layer's s2, and where its operand goes
    uint8_t *op, *op_sc;                 //   (DecOpSink), or null
};

// Several sequences' decode steps in one set of launches: sequence s has
// S[s] cached tokens, the codes of its first kb0[s] key blocks kept from its
// last step, its query, output, caches and state at s times the strides
// past those of sequence 0.  n == 0: a launch for the one sequence its
// arguments describe.
struct DecSeqTab {
    uint32_t n;
    uint32_t S[QBK_DEC_MAXSEQ], kb0[QBK_DEC_MAXSEQ];
    size_t q_stride, o_stride, kv_stride;  // floats
    size_t st_stride;                      // bytes
    const uint32_t *pos;                   // device positions in place of S and kb0, or null
};

typedef __attribute__((address_space(4))) const uint32_t cu32_t;

template <class T>
__device__ __forceinline__ T *dec_shift(T *p, size_t bytes) {
    return p ? (T *)((char *)p + bytes) : p;
}

__device__ __forceinline__ void dec_seq_ref(RefArgs &a, const DecSeqTab &t, uint32_t s) {
    if (t.pos) {
        // written by an earlier kernel of the stream (scalar loads: the
        // scalar cache starts each kernel invalidated)
        const uint32_t p = ((cu32_t *)t.pos)[s];
        const bool ok = p < a.pst;
        a.S = ok ? p + 1 : 0;
        a.kb0 = ok ? p / a.block : 0;
    } else {
        a.S = t.S[s];
        a.kb0 = t.kb0[s];
    }
    a.nkb = (a.S + a.block - 1) / a.block;
    a.q += s * t.q_stride;
    a.out += s * t.o_stride;
    a.k += s * t.kv_stride;
    a.v += s * t.kv_stride;
    const size_t b = s * t.st_stride;
    a.kmean = dec_shift(a.kmean, b);
    a.kdelta = dec_shift(a.kdelta, b);
    a.khat = dec_shift(a.khat, b);
    a.vd = dec_shift(a.vd, b);
    a.vhat = dec_shift(a.vhat, b);
}

__device__ __forceinline__ void dec_seq(DecArgs &da, const DecSeqTab &t, uint32_t s) {
    dec_seq_ref(da.r, t, s);
    const size_t b = s * t.st_stride;
    da.sc = dec_shift(da.sc, b);
    da.bmax = dec_shift(da.bmax, b);
    da.balpha = dec_shift(da.balpha, b);
    da.besum = dec_shift(da.besum, b);
    da.blive = dec_shift(da.blive, b);
    da.pvt = dec_shift(da.pvt, b);
    da.qsw = dec_shift(da.qsw, b);
    da.qdl = dec_shift(da.qdl, b);
    da.mprev = dec_shift(da.mprev, b);
}

// max over the workgroup (blockDim.x a multiple of 64, <= 1024)
__device__ __forceinline__ float dec_wg_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    const int wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wv] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < nw; i++) m = red[i] > m ? red[i] : m;
    return m;
}

// Pre-pass of a decode step, for blocks that fit in LDS: the (key block, kv
// head) work of sage_ref_prep (the same f32 operations) spread over ks
// workgroups for K -- each forms the block's channel means (the first
// writes them) and then the deltas and codes of its share of the tokens --
// and vs for V, each a share of the channels (DPREP_KS and DPREP_VS for one
// sequence; one each when many sequences' (kv head, block) pairs fill the
// chip already).  Each workgroup issues all of its loads at once (up to
// DPREP_U 16-byte loads a thread), so a step's pre-pass costs about one trip
// to memory and a short serial tail instead of one workgroup's whole
// sequence.
#define DPREP_KS 4
#define DPREP_VS 4
#define DPREP_U 16
#define DPREP_LDS 61440

struct DPrepGeom {
    uint32_t ks, vs;                // workgroups per (kv head, block) for K / V
    uint32_t kq, kstep, vq, vstep;  // 16-byte columns and rows per pass of a K / V load
    size_t lds;
    bool ok;
};

static DPrepGeom dprep_geom(const RefArgs &a, const void *k, const void *v, uint32_t ks = DPREP_KS,
                            uint32_t vs = DPREP_VS) {
    DPrepGeom g{};
    g.ks = ks;
    g.vs = vs;
    const size_t kj = a.block < a.S ? a.block : a.S;
    if (a.d % 4 || a.dv % 4 || ((uintptr_t)k & 15) || ((uintptr_t)v & 15)) return g;
    g.kq = (uint32_t)(a.d / 4);
    g.kstep = 256 / g.kq;
    g.vq = (uint32_t)div_ceil(a.dv / 4, vs);
    g.vstep = 256 / g.vq;
    const size_t kjp = 4 * div_ceil(kj, 4);  // V is staged channel-major with rows of kjp tokens
    g.lds = 4 * (kj * a.d > 4 * (size_t)g.vq * kjp ? kj * a.d : 4 * (size_t)g.vq * kjp);
    g.ok = g.kstep > 0 && g.vstep > 0 && kj <= (size_t)DPREP_U * g.kstep && kj <= (size_t)DPREP_U * g.vstep &&
           g.lds <= DPREP_LDS && div_ceil(kj, ks) <= 256;
    return g;
}

// psi_Q of the step's query (gpu_attention.rs:113-159) for the heads of kv
// head bk: a wave per head, lane l holding channels 4l .. 4l+3 (d <= 256);
// the peak is a max, so a wave reduction gives the reference's value
//
// With rp.qkv, the heads are rotated here first (rope_head at position p,
// through the wave's lbuf region of d floats) instead of read from a.q.
__device__ void dec_query_codes(const RefArgs &a, uint32_t bk, uint32_t *qsw, float *qdl, const DecRope &rp,
                                uint32_t p, float *lbuf) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t G = (uint32_t)(a.H / a.Hk), d4 = (uint32_t)a.d / 4;
    for (uint32_t hg = wave; hg < G; hg += 4) {
        const uint32_t h = bk * G + hg;
        const float *qi = a.q + (size_t)h * a.d;
        if (rp.qkv) {
            float *lw = lbuf + wave * a.d;
            __builtin_amdgcn_wave_barrier();  // the wave's last head is read
            rope_head(rp.qkv + (size_t)h * a.d, rp.wq, rp.eps, rp.rope + (size_t)p * (a.d / 2), (int)a.d,
                      (int)lane, [&](int j, float v) { lw[j] = v; });
            __builtin_amdgcn_wave_barrier();
            qi = lw;
        }
        float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (lane < d4)
#pragma unroll
            for (int e = 0; e < 4; e++) x[e] = qi[4 * lane + e];
        float pk = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float v = x[e] * a.inv_sqrt_d;
            const float av = v < 0.0f ? 0.0f - v : v;
            if (av > pk) pk = av;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float w = __shfl_xor(pk, o, 64);
            pk = w > pk ? w : pk;
        }
        const float qdelta = pk > 0.0f ? pk / 127.0f : 1.0f;
        if (lane < d4) {
            int c4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) c4[e] = q8((x[e] * a.inv_sqrt_d) / qdelta);
            qsw[(size_t)h * d4 + lane] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
        if (lane == 0) qdl[h] = qdelta;
    }
}

// grid (max(nkb - kb0, 1), Hk, ks + vs + 1): the last slice
// forms the query's codes (once per kv head, when qsw is given).  Batched
// (t.n > 0): y runs over (sequence, kv head), x over the largest count of
// blocks to quantise.
__global__ void __launch_bounds__(256) sage_dec_prep(RefArgs a, DPrepGeom g, uint32_t *qsw, float *qdl,
                                                     DecSeqTab t, DecRope rp) {
    extern __shared__ __attribute__((aligned(16))) float tile[];  // [kj][row of this workgroup]
    __shared__ __attribute__((aligned(16))) float km[REF_MAXD];  // K means, then V scales
    __shared__ float kdl[256];                                    // deltas of this workgroup's tokens
    const uint32_t tid = threadIdx.x, z = blockIdx.z;
    uint32_t bky = blockIdx.y;
    if (t.n) {
        const uint32_t sq = blockIdx.y / (uint32_t)a.Hk;
        bky = blockIdx.y % (uint32_t)a.Hk;
        dec_seq_ref(a, t, sq);
        qsw = dec_shift(qsw, sq * t.st_stride);
        qdl = dec_shift(qdl, sq * t.st_stride);
    }
    // the step's position (one sequence): with rp.qkv its k and v rows are
    // formed here -- row p of the block that holds it, in place of the cache
    // row the loads bring, and written to the cache
    const uint32_t p = a.S ? (uint32_t)a.S - 1 : 0;
    if (z == g.ks + g.vs) {
        if (blockIdx.x == 0 && qsw && (a.S || !rp.qkv)) dec_query_codes(a, bky, qsw, qdl, rp, p, tile);
        return;
    }
    const uint32_t kb = (uint32_t)a.kb0 + blockIdx.x, bk = bky;
    if (kb >= a.nkb) return;
    const uint32_t j0 = kb * (uint32_t)a.block;
    const uint32_t kj = (uint32_t)(a.block < a.S - j0 ? a.block : a.S - j0);
    const uint32_t d = (uint32_t)a.d, d4 = d / 4;
    const uint32_t prow = rp.qkv && p >= j0 && p - j0 < kj ? p - j0 : 0xffffffffu;
    f32x4_t r[DPREP_U];
    if (z < g.ks) {
        const float *K = a.k + bk * a.k_head + (size_t)j0 * a.k_tok;
        const uint32_t q = tid % g.kq, r0 = tid / g.kq;
        const bool lane_ok = r0 < g.kstep;
#pragma unroll
        for (uint32_t u = 0; u < DPREP_U; u++) {
            const uint32_t row = r0 + u * g.kstep;
            r[u] = *(const f32x4_t *)(K + (size_t)(row < kj ? row : kj - 1) * a.k_tok + 4 * q);
        }
#pragma unroll
        for (uint32_t u = 0; u < DPREP_U; u++) {
            const uint32_t row = r0 + u * g.kstep;
            if (lane_ok && row < kj && row != prow) *(f32x4_t *)&tile[row * d + 4 * q] = r[u];
        }
        if (prow != 0xffffffffu && tid < 64) {
            float *crow = const_cast<float *>(K) + (size_t)prow * a.k_tok;
            const bool w0 = z == 0;  // one workgroup appends the row
            rope_head(rp.qkv + (size_t)(rp.H + bk) * d, rp.wk, rp.eps, rp.rope + (size_t)p * (d / 2), (int)d,
                      (int)tid, [&](int j, float v) {
                          tile[prow * d + j] = v;
                          if (w0) crow[j] = v;
                      });
        }
        __syncthreads();
        // the block's mean per channel, sequential over its tokens
        if (tid < d) {
            float ssum = 0.0f;
#pragma unroll 8
            for (uint32_t t = 0; t < kj; t++) ssum += tile[t * d + tid];
            const float m = ssum / (float)kj;
            km[tid] = m;
            if (z == 0) a.kmean[((size_t)bk * a.pnkb + kb) * d + tid] = m;
        }
        __syncthreads();
        // this workgroup's tokens
        const uint32_t per = (kj + g.ks - 1) / g.ks, t0 = z * per;
        const uint32_t t1 = t0 + per < kj ? t0 + per : kj;
        if (t0 >= t1) return;
        const uint32_t nt = t1 - t0;
        if ((d4 & (d4 - 1)) == 0) {
            // a token's d4 words in d4 consecutive lanes: its peak by a lane
            // reduction (a max), then each lane's word of codes
            const uint32_t lg = 31 - __builtin_clz(d4);
            for (uint32_t i0 = 0; i0 < nt * d4; i0 += 256) {
                const uint32_t it = i0 + tid;
                const bool ok = it < nt * d4;
                const uint32_t tt = ok ? it >> lg : 0, w = it & (d4 - 1), t = t0 + tt;
                const f32x4_t x = *(const f32x4_t *)&tile[t * d + 4 * w];
                const f32x4_t m = *(const f32x4_t *)&km[4 * w];
                float gv[4], kpeak = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    gv[e] = x[e] - m[e];
                    const float ag = gv[e] < 0.0f ? 0.0f - gv[e] : gv[e];
                    if (ag > kpeak) kpeak = ag;
                }
                for (uint32_t o = 1; o < d4; o <<= 1) {
                    const float wv = __shfl_xor(kpeak, o, 64);
                    kpeak = wv > kpeak ? wv : kpeak;
                }
                float kdelta = 1.0f;
                if (kpeak > 0.0f) kdelta = kpeak / 127.0f;
                if (ok) {
                    if (w == 0) a.kdelta[(size_t)bk * a.pst + j0 + t] = kdelta;
                    int c4[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) c4[e] = q8(gv[e] / kdelta);
                    a.khat[((size_t)bk * a.pst + j0 + t) * d4 + w] = pack4(c4[0], c4[1], c4[2], c4[3]);
                }
            }
            return;
        }
        // otherwise a thread per token for the peak, then (token, word) items
        if (tid < nt) {
            const uint32_t t = t0 + tid;
            float kpeak = 0.0f;
            for (uint32_t w = 0; w < d4; w++) {
                const f32x4_t x = *(const f32x4_t *)&tile[t * d + 4 * w];
                const f32x4_t m = *(const f32x4_t *)&km[4 * w];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float gv = x[e] - m[e];
                    const float ag = gv < 0.0f ? 0.0f - gv : gv;
                    if (ag > kpeak) kpeak = ag;
                }
            }
            float kdelta = 1.0f;
            if (kpeak > 0.0f) kdelta = kpeak / 127.0f;
            kdl[tid] = kdelta;
            a.kdelta[(size_t)bk * a.pst + j0 + t] = kdelta;
        }
        __syncthreads();
        for (uint32_t it = tid; it < nt * d4; it += 256) {
            const uint32_t tt = it / d4, w = it % d4, t = t0 + tt;
            const f32x4_t x = *(const f32x4_t *)&tile[t * d + 4 * w];
            const f32x4_t m = *(const f32x4_t *)&km[4 * w];
            const float kdelta = kdl[tt];
            int c4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) c4[e] = q8((x[e] - m[e]) / kdelta);
            a.khat[((size_t)bk * a.pst + j0 + t) * d4 + w] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
    } else {
        // V: channels 4 * c4_0 .. of this workgroup, all of the block's
        // tokens, staged channel-major ([cw][kjp], kjp = kj rounded up to 4)
        const uint32_t dv4 = (uint32_t)a.dv / 4, c4_0 = (z - g.ks) * g.vq;
        if (c4_0 >= dv4) return;
        const uint32_t cq = dv4 - c4_0 < g.vq ? dv4 - c4_0 : g.vq, cw = 4 * cq;
        const uint32_t step = 256 / cq, tw = (kj + 3) / 4, kjp = 4 * tw;
        const float *V = a.v + bk * a.v_head + (size_t)j0 * a.v_tok + 4 * c4_0;
        const uint32_t q = tid % cq, r0 = tid / cq;
        const bool lane_ok = r0 < step;
#pragma unroll
        for (uint32_t u = 0; u < DPREP_U; u++) {
            const uint32_t row = r0 + u * step;
            r[u] = *(const f32x4_t *)(V + (size_t)(row < kj ? row : kj - 1) * a.v_tok + 4 * q);
        }
#pragma unroll
        for (uint32_t u = 0; u < DPREP_U; u++) {
            const uint32_t row = r0 + u * step;
            if (lane_ok && row < kj && row != prow)
#pragma unroll
                for (int e = 0; e < 4; e++) tile[(4 * q + e) * kjp + row] = r[u][e];
        }
        if (prow != 0xffffffffu && tid < cw) {
            // this workgroup's channels of the new v row (no rotation)
            const float x = rp.qkv[(size_t)(rp.H + a.Hk + bk) * a.dv + 4 * c4_0 + tid];
            tile[tid * kjp + prow] = x;
            const_cast<float *>(V)[(size_t)prow * a.v_tok + tid] = x;
        }
        __syncthreads();
        uint32_t *vrow = a.vhat + ((size_t)bk * a.pnkb + kb) * a.dv * a.blk4;
        if ((tw & (tw - 1)) == 0 && tw <= 64) {
            // a channel's tw words in tw consecutive lanes: its peak over the
            // block by a lane reduction (a max), then each lane's word
            const uint32_t lg = 31 - __builtin_clz(tw);
            for (uint32_t i0 = 0; i0 < cw * tw; i0 += 256) {
                const uint32_t it = i0 + tid;
                const bool ok = it < cw * tw;
                const uint32_t c = ok ? it >> lg : 0, w = it & (tw - 1);
                const f32x4_t x = *(const f32x4_t *)&tile[c * kjp + 4 * w];
                float vpeak = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float xv = 4 * w + e < kj ? x[e] : 0.0f;
                    const float ax = xv < 0.0f ? 0.0f - xv : xv;
                    if (ax > vpeak) vpeak = ax;
                }
                for (uint32_t o = 1; o < tw; o <<= 1) {
                    const float wv = __shfl_xor(vpeak, o, 64);
                    vpeak = wv > vpeak ? wv : vpeak;
                }
                const float vd = vpeak > 0.0f ? vpeak / 127.0f : 1.0f;
                if (ok) {
                    if (w == 0) a.vd[((size_t)bk * a.pnkb + kb) * a.dv + 4 * c4_0 + c] = vd;
                    int c4[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) c4[e] = 4 * w + e < kj ? q8(x[e] / vd) : 0;
                    vrow[(size_t)(4 * c4_0 + c) * a.blk4 + w] = pack4(c4[0], c4[1], c4[2], c4[3]);
                }
            }
            return;
        }
        // otherwise a thread per channel for the peak, then (channel, word) items
        if (tid < cw) {
            float vpeak = 0.0f;
#pragma unroll 8
            for (uint32_t t = 0; t < kj; t++) {
                const float x = tile[tid * kjp + t];
                const float ax = x < 0.0f ? 0.0f - x : x;
                if (ax > vpeak) vpeak = ax;
            }
            const float vd = vpeak > 0.0f ? vpeak / 127.0f : 1.0f;
            km[tid] = vd;
            a.vd[((size_t)bk * a.pnkb + kb) * a.dv + 4 * c4_0 + tid] = vd;
        }
        __syncthreads();
        for (uint32_t it = tid; it < cw * tw; it += 256) {
            const uint32_t c = it % cw, w = it / cw;
            const float vd = km[c];
            int c4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t t = 4 * w + e;
                c4[e] = t < kj ? q8(tile[c * kjp + t] / vd) : 0;
            }
            vrow[(size_t)(4 * c4_0 + c) * a.blk4 + w] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
    }
}

__global__ void __launch_bounds__(256) sage_dec_scores(DecArgs da) {
    const RefArgs &a = da.r;
    __shared__ uint32_t qs[REF_MAXD / 4];
    __shared__ __attribute__((aligned(16))) float term[REF_MAXD];
    __shared__ float red[4];
    __shared__ float shv;
    const int tid = threadIdx.x;
    const size_t kb = blockIdx.x, h = blockIdx.y;
    const size_t bk = h / (a.H / a.Hk);
    const size_t j0 = kb * a.block, j1 = j0 + a.block < a.S ? j0 + a.block : a.S;
    // this thread's loads that do not wait on the query: its key's delta
    // and the block's mean of its channel
    const size_t jj0 = j0 + tid;
    const float kd0 = jj0 < j1 ? a.kdelta[bk * a.pst + jj0] : 0.0f;
    const float kmc = (size_t)tid < a.d ? a.kmean[(bk * a.pnkb + kb) * a.d + tid] : 0.0f;
    // and, for code rows of at most 8 whole 16-byte words (d <= 128), its
    // key's codes
    const bool vec = (a.d4 & 3) == 0;
    const size_t n4 = a.d4 >> 2;
    const bool pre = vec && n4 <= 8 && jj0 < j1;
    u32x4_t kv0[8];
    if (pre) {
        const u32x4_t *kc = (const u32x4_t *)(a.khat + (bk * a.pst + jj0) * a.d4);
#pragma unroll
        for (int u = 0; u < 8; u++) kv0[u] = (size_t)u < n4 ? kc[u] : u32x4_t{0, 0, 0, 0};
    }
    // psi_Q of the query (gpu_attention.rs:113-159; the peak is a max)
    const float *qi = a.q + h * a.d;
    float pk = 0.0f;
    for (size_t c = tid; c < a.d; c += blockDim.x) {
        const float x = qi[c] * a.inv_sqrt_d;
        const float ax = x < 0.0f ? 0.0f - x : x;
        if (ax > pk) pk = ax;
    }
    const float qpeak = dec_wg_max(pk, red);
    const float qdelta = qpeak > 0.0f ? qpeak / 127.0f : 1.0f;
    for (size_t w = tid; w < a.d4; w += blockDim.x) {
        int c4[4];
        for (int e = 0; e < 4; e++) {
            const size_t c = 4 * w + e;
            c4[e] = c < a.d ? q8((qi[c] * a.inv_sqrt_d) / qdelta) : 0;
        }
        qs[w] = pack4(c4[0], c4[1], c4[2], c4[3]);
    }
    // shift = sum_c (q^_c * dq) * kmean_c in element order (:253): the
    // products in parallel (d <= REF_MAXD <= the 256 threads), the sum by
    // one thread over them in order
    if ((size_t)tid < a.d) {
        const int qc = q8((qi[tid] * a.inv_sqrt_d) / qdelta);
        term[tid] = ((float)qc * qdelta) * kmc;
    }
    __syncthreads();
    if (tid == 0) {
        float shift = 0.0f;
        size_t c = 0;
#pragma unroll 4
        for (; c + 4 <= a.d; c += 4) {
            const float4 t4 = *(const float4 *)&term[c];
            shift += t4.x;
            shift += t4.y;
            shift += t4.z;
            shift += t4.w;
        }
        for (; c < a.d; c++) shift += term[c];
        shv = shift;
    }
    __syncthreads();
    const float shift = shv;
    float rm = MASKED;
    for (size_t jj = jj0; jj < j1; jj += blockDim.x) {
        const uint32_t *kc = a.khat + (bk * a.pst + jj) * a.d4;
        int acc = 0;
        if (pre && jj == jj0) {
#pragma unroll
            for (int u = 0; u < 8; u++)
                if ((size_t)u < n4) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        acc = __builtin_amdgcn_sdot4((int)qs[4 * u + e], (int)kv0[u][e], acc, false);
                }
        } else if (vec) {
            for (size_t w0 = 0; w0 < n4; w0 += 8) {
                u32x4_t kv[8];
#pragma unroll
                for (int u = 0; u < 8; u++)
                    kv[u] = w0 + u < n4 ? ((const u32x4_t *)kc)[w0 + u] : u32x4_t{0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (w0 + u < n4) {
                        const uint32_t *qw = qs + 4 * (w0 + u);
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acc = __builtin_amdgcn_sdot4((int)qw[e], (int)kv[u][e], acc, false);
                    }
            }
        } else {
            for (size_t w = 0; w < a.d4; w++) acc = __builtin_amdgcn_sdot4((int)qs[w], (int)kc[w], acc, false);
        }
        const float kdl = jj == jj0 ? kd0 : a.kdelta[bk * a.pst + jj];
        const float sv = (float)acc * qdelta * kdl + shift;
        da.sc[h * a.S + jj] = sv;
        if (sv > rm) rm = sv;
    }
    rm = dec_wg_max(rm, red);
    if (tid == 0) da.bmax[h * a.nkb + kb] = rm;
}

// :288-296's running max before each block, for caches of more than
// DEC_PMAX blocks (where each P.V workgroup reducing the earlier maxima
// itself would read O(nkb^2) values): mprev[kb] = max(MASKED, bmax[0..kb-1]),
// a max, so a parallel scan gives the reference's sequential value.  One
// workgroup per head, 8 blocks a thread, 2048 blocks a pass.
__global__ void __launch_bounds__(256) sage_dec_runmax(DecArgs da, DecSeqTab t) {
    __shared__ float wm[4];
    if (t.n) dec_seq(da, t, blockIdx.y);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t h = blockIdx.x, nkb = da.r.nkb;
    const float *bm = da.bmax + h * nkb;
    float *mp = da.mprev + h * nkb;
    float carry = MASKED;
    for (size_t base = 0; base < nkb; base += 2048) {
        float v[8], ex[8], run = MASKED;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t i = base + 8 * tid + u;
            v[u] = i < nkb ? bm[i] : MASKED;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            ex[u] = run;
            run = v[u] > run ? v[u] : run;
        }
        float incl = run;  // inclusive scan over the wave's lanes
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float w = __shfl_up(incl, o, 64);
            if ((int)lane >= o) incl = w > incl ? w : incl;
        }
        __syncthreads();
        if (lane == 63) wm[wave] = incl;
        __syncthreads();
        float before = carry;  // the earlier waves of this pass and the earlier passes
        for (uint32_t w2 = 0; w2 < wave; w2++) before = wm[w2] > before ? wm[w2] : before;
        const float up = __shfl_up(incl, 1, 64);
        const float tex = lane == 0 ? before : (up > before ? up : before);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t i = base + 8 * tid + u;
            if (i < nkb) mp[i] = ex[u] > tex ? ex[u] : tex;
        }
        for (int w2 = 0; w2 < 4; w2++) carry = wm[w2] > carry ? wm[w2] : carry;
    }
}

// :288-296 (the running max, live flag and alpha of this block), :297-316
// (p, esum in key order, codes) and :317-341 (P^.V^ per channel).  The
// running max before a block is the max of MASKED and the earlier blocks'
// maxima: a max, so the reference's scan and a reduction give one value
// (no score is -0.0: shift starts at +0.0).
__global__ void __launch_bounds__(256) sage_dec_pv(DecArgs da) {
    const RefArgs &a = da.r;
    __shared__ __attribute__((aligned(16))) float pf[DEC_CH];
    __shared__ uint32_t ph[DEC_CH / 4];
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const size_t kb = blockIdx.x, h = blockIdx.y, nkb = a.nkb;
    const size_t bk = h / (a.H / a.Hk);
    const size_t j0 = kb * a.block, j1 = j0 + a.block < a.S ? j0 + a.block : a.S;
    const uint32_t *vh = a.vhat + (bk * a.pnkb + kb) * a.dv * a.blk4;
    // loads that wait on nothing, issued first: this thread's four scores of
    // the first chunk and its channel's first code words (up to 8 16-byte
    // words) and scale, alongside the earlier blocks' maxima
    const size_t tc0 = j1 - j0 < DEC_CH ? j1 - j0 : DEC_CH, tw0 = (tc0 + 3) / 4;
    const bool spre = (size_t)tid < tw0 && tw0 <= blockDim.x;
    float sc0[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (spre)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const size_t t = 4 * (size_t)tid + e;
            sc0[e] = t < tc0 ? da.sc[h * a.S + j0 + t] : 0.0f;
        }
    const bool vvec = (a.blk4 & 3) == 0;  // whole 16-byte words (t0 - j0 is a multiple of DEC_CH)
    const size_t vn0 = (tw0 + 3) >> 2;
    const bool vpre = vvec && vn0 <= 8 && (size_t)tid < a.dv;
    u32x4_t vv0[8];
    if (vpre) {
        const u32x4_t *vc = (const u32x4_t *)(vh + tid * a.blk4);
#pragma unroll
        for (int u = 0; u < 8; u++) vv0[u] = (size_t)u < vn0 ? vc[u] : u32x4_t{0, 0, 0, 0};
    }
    const float vdc = (size_t)tid < a.dv ? a.vd[(bk * a.pnkb + kb) * a.dv + tid] : 0.0f;
    // the running max before this block: from sage_dec_runmax when the
    // cache has many blocks, else reduced here over the earlier maxima
    float pm = MASKED;
    if (!da.mprev)
        for (size_t i = tid; i < kb; i += blockDim.x) {
            const float x = da.bmax[h * nkb + i];
            pm = x > pm ? x : pm;
        }
    const float bx = da.bmax[h * nkb + kb];
    const float m = da.mprev ? da.mprev[h * nkb + kb] : dec_wg_max(pm, red);
    const float m_new = bx > m ? bx : m;
    const int live = !(m_new < MASKED * 0.5f);
    float esum = 0.0f;  // thread 0's running sum
    int pv = 0;         // thread c's P^.V^ over the block (dv <= the 256 threads)
    for (size_t t0 = j0; t0 < j1; t0 += DEC_CH) {
        const size_t tc = j1 - t0 < DEC_CH ? j1 - t0 : DEC_CH, tw = (tc + 3) / 4;
        const bool first = t0 == j0;
        __syncthreads();
        for (size_t w = tid; w < tw; w += blockDim.x) {
            int c4[4];
            for (int e = 0; e < 4; e++) {
                const size_t t = 4 * w + e;
                int pc = 0;
                if (t < tc) {
                    const float scv = first && spre ? sc0[e] : da.sc[h * a.S + t0 + t];
                    const float p = live ? qbk_expf(scv - m_new) : 0.0f;
                    pf[t] = p;
                    float pr = __builtin_rintf(p * 127.0f);
                    pr = pr > 127.0f ? 127.0f : pr;
                    pr = pr < 0.0f ? 0.0f : pr;
                    pc = (int)pr;
                }
                c4[e] = pc;
            }
            ph[w] = pack4(c4[0], c4[1], c4[2], c4[3]);
        }
        __syncthreads();
        if (tid == 0) {
            size_t t = 0;
#pragma unroll 4
            for (; t + 4 <= tc; t += 4) {
                const float4 p4 = *(const float4 *)&pf[t];
                esum += p4.x;
                esum += p4.y;
                esum += p4.z;
                esum += p4.w;
            }
            for (; t < tc; t++) esum += pf[t];
        }
        if ((size_t)tid < a.dv) {
            const uint32_t *vc = vh + tid * a.blk4 + (t0 - j0) / 4;
            if (first && vpre) {
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const size_t w = 4 * (size_t)u + e;
                        if (w < tw) pv = __builtin_amdgcn_sdot4((int)ph[w], (int)vv0[u][e], pv, false);
                    }
            } else if (vvec) {
                const size_t n4 = (tw + 3) >> 2;
                for (size_t w0 = 0; w0 < n4; w0 += 8) {
                    u32x4_t vv[8];
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        vv[u] = w0 + u < n4 ? ((const u32x4_t *)vc)[w0 + u] : u32x4_t{0, 0, 0, 0};
#pragma unroll
                    for (int u = 0; u < 8; u++)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const size_t w = 4 * (w0 + u) + e;
                            if (w < tw) pv = __builtin_amdgcn_sdot4((int)ph[w], (int)vv[u][e], pv, false);
                        }
                }
            } else {
                for (size_t w = 0; w < tw; w++) pv = __builtin_amdgcn_sdot4((int)ph[w], (int)vc[w], pv, false);
            }
        }
    }
    if (tid == 0) {
        da.besum[h * nkb + kb] = esum;
        da.blive[h * nkb + kb] = live;
        da.balpha[h * nkb + kb] = live ? qbk_expf(m - m_new) : 0.0f;
    }
    if ((size_t)tid < a.dv)
        da.pvt[(h * nkb + kb) * a.dv + tid] = (float)pv * (1.0f / 127.0f) * vdc;
}

// :315 and :337-338 over the blocks in order, then :346.  DEC_CB blocks at
// a time: every thread's P.V terms and the blocks' alpha, esum and live
// flags loaded at once (indices clamped into the chunk) and staged through
// LDS, then the recurrence reads them from there.  Indices are 32-bit and
// the code is kept short: a launch this small is bound by its serial
// instruction stream, fetches included.
#define DEC_CB 32
__global__ void __launch_bounds__(256) sage_dec_combine(DecArgs da, DecSeqTab t) {
    if (t.n) dec_seq(da, t, blockIdx.y);
    const RefArgs &a = da.r;
    __shared__ float sa[DEC_CB], se[DEC_CB];
    __shared__ int sl[DEC_CB];
    __shared__ float pvl[DEC_CB * REF_MAXD];
    const uint32_t h = blockIdx.x, nkb = (uint32_t)a.nkb, dv = (uint32_t)a.dv, tid = threadIdx.x;
    const bool act = tid < dv;
    const uint32_t c = act ? tid : 0;
    const float *pt = da.pvt + (size_t)h * nkb * dv + c;
    const float *pa = da.balpha + (size_t)h * nkb, *pe = da.besum + (size_t)h * nkb;
    const int *pl = da.blive + (size_t)h * nkb;
    float o = 0.0f, ell = 0.0f;
    for (uint32_t kb0 = 0; kb0 < nkb; kb0 += DEC_CB) {
        const uint32_t n = nkb - kb0 < DEC_CB ? nkb - kb0 : DEC_CB;
        float t[DEC_CB];
#pragma unroll
        for (uint32_t u = 0; u < DEC_CB; u++) t[u] = pt[(kb0 + (u < n ? u : n - 1)) * dv];
        const uint32_t i = kb0 + (tid < n ? tid : n - 1);
        const float ra = pa[i], re = pe[i];
        const int rl = pl[i];
        __syncthreads();
        if (tid < DEC_CB) {
            sa[tid] = ra;
            se[tid] = re;
            sl[tid] = rl;
        }
#pragma unroll
        for (uint32_t u = 0; u < DEC_CB; u++) pvl[u * REF_MAXD + c] = t[u];
        __syncthreads();
        if (act) {
#pragma unroll 4
            for (uint32_t u = 0; u < n; u++) {
                const float alpha = sa[u];
                ell = alpha * ell + se[u];
                const float prev = sl[u] ? o : 0.0f;
                o = alpha * prev + pvl[u * REF_MAXD + c];
            }
        }
    }
    // no key block (a device position at or past the capacity): 0, not 0/0
    const float val = act && nkb ? o / ell : 0.0f;
    if (act) a.out[(size_t)h * dv + c] = val;
    if (da.op) {
        // the output as the next layer's operand: a run of 16 channels a
        // lane of wave 0 (dv a multiple of 128: the head's runs fill whole
        // slices, lanes past them shadow the last slice's)
        __shared__ float ov[REF_MAXD];
        if (act) ov[c] = val;
        __syncthreads();
        if (tid < 64) {
            const uint32_t nr = dv / 16, rl = tid < nr ? tid : nr - 8 + (tid & 7);
            const float *s2 = da.op_s2 + (size_t)h * dv + 16 * rl;
            float z[16];
#pragma unroll
            for (int e = 0; e < 16; e++) z[e] = bf16_to_f32(f32_to_bf16(s2[e] * ov[16 * rl + e]));
            uint32_t hw[4], lw[4];
            int e_hi, e_lo;
            q4_run_operand(z, hw, lw, e_hi, e_lo);
            if (tid < nr) {
                const size_t t = (size_t)h * nr + rl;
                const int r = (int)(t & 7);
                const size_t slot = q4_run_slot(t >> 3, r, 2, 0), byte = 16 * (r & 1);
                *(uint4 *)(da.op + slot * 32 + byte) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                *(uint4 *)(da.op + (slot + 1) * 32 + byte) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
                if ((r & 2) == 0)
                    *(uint16_t *)(da.op_sc + q4_run_scale(t >> 3, r, 2, 0)) =
                        (uint16_t)((e_hi + 127) | ((e_lo + 127) << 8));
            }
        }
    }
}

// Grouped form of sage_dec_scores and sage_dec_pv: one workgroup per (key
// block, kv head) for the G = n_heads / n_kv_heads query heads that share
// the kv head, a wave per head, so a block's key codes are read once per
// group and a step launches G times fewer workgroups; the query's codes
// come from the pre-pass.  The same f32 operations in the same order as
// the per-head kernels.  Used when G <= DEC_GMAX, a block has at most
// DEC_KMAX keys, and d and the code rows are whole 16-byte words.  Up to
// DEC_PMAX blocks each P.V workgroup reduces the earlier blocks' maxima
// itself; beyond, sage_dec_runmax scans them first.
#define DEC_GMAX 16
#define DEC_KMAX 256
#define DEC_PMAX 512

// GM, DM: the largest group and head_dim a kernel serves (register and LDS
// arrays sized by them: the config-5 shape's 4 and 128 leave room for twice
// the waves of the general 16 and 256).
template <int GM, int DM>
__global__ void __launch_bounds__(256) sage_dec_scores_g(DecArgs da, DecSeqTab t) {
    if (t.n) dec_seq(da, t, blockIdx.z);
    const RefArgs &a = da.r;
    if (blockIdx.x >= a.nkb) return;  // a batched launch covers the longest sequence's blocks
    __shared__ uint32_t qs[GM * (DM / 4)];
    __shared__ float qd[GM];
    __shared__ float kms[DM];
    __shared__ __attribute__((aligned(16))) float term[GM * DM];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kb = blockIdx.x, bk = blockIdx.y, G = (uint32_t)(a.H / a.Hk);
    const uint32_t d = (uint32_t)a.d, d4 = d / 4, n4 = d4 / 4;
    const uint32_t j0 = kb * (uint32_t)a.block;
    const uint32_t kj = (uint32_t)(a.block < a.S - j0 ? a.block : a.S - j0);
    // the loads that wait on nothing, first: the group's query codes and
    // deltas, the block's means, this lane's first key's codes and delta
    for (uint32_t i = tid; i < G * d4; i += 256) qs[i] = da.qsw[(size_t)bk * G * d4 + i];
    if (tid < G) qd[tid] = da.qdl[bk * G + tid];
    if (tid < d) kms[tid] = a.kmean[((size_t)bk * a.pnkb + kb) * d + tid];
    const uint32_t jl = lane < kj ? lane : kj - 1;
    const u32x4_t *krow = (const u32x4_t *)(a.khat + ((size_t)bk * a.pst + j0 + jl) * d4);
    u32x4_t kv[DM / 16];
#pragma unroll
    for (uint32_t u = 0; u < DM / 16; u++)
        if (u < n4) kv[u] = krow[u];
    const float kd0 = a.kdelta[(size_t)bk * a.pst + j0 + jl];
    __syncthreads();
    // the shift's terms (q^_c * dq) * kmean_c, every (head, channel) at once
    for (uint32_t i = tid; i < G * d; i += 256) {
        const uint32_t hg = i / d, c = i % d;
        const int qc = (int)(int8_t)(qs[hg * d4 + c / 4] >> (8 * (c % 4)));
        term[i] = ((float)qc * qd[hg]) * kms[c];
    }
    __syncthreads();
    for (uint32_t hg = wave; hg < G; hg += 4) {
        // shift: the terms summed in channel order (:253) by lane 0
        float shift = 0.0f;
        if (lane == 0) {
            const float *t = term + hg * d;
#pragma unroll 4
            for (uint32_t c = 0; c < d; c += 4) {
                const f32x4_t t4 = *(const f32x4_t *)&t[c];
                shift += t4[0];
                shift += t4[1];
                shift += t4[2];
                shift += t4[3];
            }
        }
        shift = __shfl(shift, 0, 64);
        const float qdh = qd[hg];
        const uint32_t *qh = qs + hg * d4;
        const size_t h = (size_t)bk * G + hg;
        float rm = MASKED;
        for (uint32_t j = lane; j < kj; j += 64) {
            int acc = 0;
            float kdl;
            if (j == lane) {
#pragma unroll
                for (uint32_t u = 0; u < DM / 16; u++)
                    if (u < n4)
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acc = __builtin_amdgcn_sdot4((int)qh[4 * u + e], (int)kv[u][e], acc, false);
                kdl = kd0;
            } else {
                const u32x4_t *kr = (const u32x4_t *)(a.khat + ((size_t)bk * a.pst + j0 + j) * d4);
                for (uint32_t u = 0; u < n4; u++) {
                    const u32x4_t k4 = kr[u];
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        acc = __builtin_amdgcn_sdot4((int)qh[4 * u + e], (int)k4[e], acc, false);
                }
                kdl = a.kdelta[(size_t)bk * a.pst + j0 + j];
            }
            const float sv = (float)acc * qdh * kdl + shift;
            da.sc[h * a.S + j0 + j] = sv;
            if (sv > rm) rm = sv;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float w = __shfl_xor(rm, o, 64);
            rm = w > rm ? w : rm;
        }
        if (lane == 0) da.bmax[h * a.nkb + kb] = rm;
    }
}

// GM, KM: the largest group and key block a kernel serves; HALVES: the
// instance for groups of exactly four heads at dv 128 (below).
template <int GM, int KM, bool HALVES = false>
__global__ void __launch_bounds__(256) sage_dec_pv_g(DecArgs da, DecSeqTab t) {
    if (t.n) dec_seq(da, t, blockIdx.z);
    const RefArgs &a = da.r;
    if (blockIdx.x >= a.nkb) return;
    __shared__ __attribute__((aligned(16))) float pf[GM * KM];
    __shared__ __attribute__((aligned(16))) uint8_t ph[GM * KM];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kb = blockIdx.x, bk = blockIdx.y, nkb = (uint32_t)a.nkb;
    const uint32_t G = HALVES ? 4u : (uint32_t)(a.H / a.Hk), dv = HALVES ? 128u : (uint32_t)a.dv;
    const uint32_t j0 = kb * (uint32_t)a.block;
    const uint32_t kj = (uint32_t)(a.block < a.S - j0 ? a.block : a.S - j0);
    const uint32_t tw = (kj + 3) / 4, vn4 = (tw + 3) / 4;
    // first, this thread's channel's V codes and scale (256 / dv threads a
    // channel, each for every (256 / dv)-th head of the group).  A group of
    // four at dv 128 and blocks of at most 64 keys: the two threads of a
    // channel take half of its code words each, for all four heads, so the
    // codes are fetched once per workgroup (their integer sums added after).
    constexpr bool halves = HALVES;  // the launch checks G == 4 and dv == 128
    static_assert(!HALVES || (GM == 4 && KM == 64), "the halves instance serves groups of four, 64-key blocks");
    const uint32_t hstep = 256 / dv, c = tid % dv, hs = tid / dv;
    const size_t vb = ((size_t)bk * a.pnkb + kb) * dv + c;
    const u32x4_t *vrow = (const u32x4_t *)(a.vhat + vb * a.blk4);
    // The L2-resident operands first -- the scores of this wave's first
    // head at this lane's first key and (two halves: the wave's one head) the
    // earlier blocks' maxima -- then the V codes from HBM, unconditional
    // (indices clamped), so that the probabilities and their key-order sum
    // below are formed while the codes are in flight (the barriers order LDS
    // only).
    float sc0, mp0 = MASKED, bx0 = MASKED;
    if (halves) {  // four waves, a head each: every load unconditional, selected after
        const size_t h = (size_t)bk * G + wave;
        const float *bm = da.bmax + h * nkb;
        const float scr = da.sc[h * a.S + j0 + (lane < kj ? lane : 0)];
        // a global load (a pointer chosen between two reads as a flat load,
        // which counts against both wait counters)
        const float *mpa = da.mprev ? da.mprev + h * nkb + kb : bm + (lane < kb ? lane : kb);
        const float mpr = *(const __attribute__((address_space(1))) float *)mpa;
        bx0 = bm[kb];
        sc0 = lane < kj ? scr : 0.0f;
        mp0 = da.mprev || lane < kb ? mpr : MASKED;
    } else {
        sc0 = wave < G && lane < kj ? da.sc[((size_t)bk * G + wave) * a.S + j0 + lane] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);  // the value loads stay behind these
    u32x4_t vv[KM / 16];
    if (halves) {
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) vv[u] = vrow[2 * hs + u < vn4 ? 2 * hs + u : vn4 - 1];
    } else {
#pragma unroll
        for (uint32_t u = 0; u < KM / 16; u++)
            if (u < vn4) vv[u] = vrow[u];
    }
    const float vdc = a.vd[vb];
    // a wave per head: the running max before and after this block (a max
    // of MASKED and the earlier blocks' maxima: the reference's scan and a
    // reduction give one value), its live flag and alpha, p and its codes
    for (uint32_t hg = wave; hg < G; hg += 4) {
        const size_t h = (size_t)bk * G + hg;
        const float *bm = da.bmax + h * nkb;
        float pm = halves ? mp0 : MASKED;
        if (halves && da.mprev) {
        } else if (da.mprev) {
            pm = da.mprev[h * nkb + kb];
        } else {
            for (uint32_t i = halves ? lane + 64 : lane; i < kb; i += 64) {  // halves: blocks past the first 64
                const float x = bm[i];
                pm = x > pm ? x : pm;
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float w = __shfl_xor(pm, o, 64);
                pm = w > pm ? w : pm;
            }
        }
        const float bx = halves ? bx0 : bm[kb];
        const float m_new = bx > pm ? bx : pm;
        const int live = !(m_new < MASKED * 0.5f);
        for (uint32_t j = lane; j < 4 * tw; j += 64) {
            float p = 0.0f;
            int pc = 0;
            if (j < kj) {
                const float scv = hg == wave && j == lane ? sc0 : da.sc[h * a.S + j0 + j];
                p = live ? qbk_expf(scv - m_new) : 0.0f;
                float pr = __builtin_rintf(p * 127.0f);
                pr = pr > 127.0f ? 127.0f : pr;
                pr = pr < 0.0f ? 0.0f : pr;
                pc = (int)pr;
            }
            pf[hg * KM + j] = p;
            ph[hg * KM + j] = (uint8_t)pc;
        }
        if (lane == 0) {
            da.blive[h * nkb + kb] = live;
            da.balpha[h * nkb + kb] = live ? qbk_expf(pm - m_new) : 0.0f;
        }
    }
    dec_lds_barrier();
    // esum: p summed in key order (:315), by lane 0 of the head's wave
    for (uint32_t hg = wave; hg < G; hg += 4)
        if (lane == 0) {
            const float *pp = pf + hg * KM;
            float esum = 0.0f;
            uint32_t t = 0;
#pragma unroll 4
            for (; t + 4 <= kj; t += 4) {
                const f32x4_t p4 = *(const f32x4_t *)&pp[t];
                esum += p4[0];
                esum += p4[1];
                esum += p4[2];
                esum += p4[3];
            }
            for (; t < kj; t++) esum += pp[t];
            da.besum[((size_t)bk * G + hg) * nkb + kb] = esum;
        }
    // P^.V^ per (head, channel) (:317-341)
    if (halves) {
        __shared__ int red[2][4][128];
#pragma unroll
        for (uint32_t hg = 0; hg < 4; hg++) {
            const uint32_t *pw = (const uint32_t *)(ph + hg * KM);
            int pv = 0;
#pragma unroll
            for (uint32_t u = 0; u < 2; u++)
                if (2 * hs + u < vn4)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (4 * (2 * hs + u) + e < tw)
                            pv = __builtin_amdgcn_sdot4((int)pw[4 * (2 * hs + u) + e], (int)vv[u][e], pv, false);
            red[hs][hg][c] = pv;
        }
        dec_lds_barrier();
#pragma unroll
        for (uint32_t hg = hs; hg < 4; hg += 2) {
            const int pv = red[0][hg][c] + red[1][hg][c];
            da.pvt[(((size_t)bk * G + hg) * nkb + kb) * dv + c] = (float)pv * (1.0f / 127.0f) * vdc;
        }
        return;
    }
    if (hs < hstep)
        for (uint32_t hg = hs; hg < G; hg += hstep) {
            const uint32_t *pw = (const uint32_t *)(ph + hg * KM);
            int pv = 0;
#pragma unroll
            for (uint32_t u = 0; u < KM / 16; u++)
                if (u < vn4)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (4 * u + e < tw) pv = __builtin_amdgcn_sdot4((int)pw[4 * u + e], (int)vv[u][e], pv, false);
            da.pvt[(((size_t)bk * G + hg) * nkb + kb) * dv + c] = (float)pv * (1.0f / 127.0f) * vdc;
        }
}


// sage_dec_scores_g for groups of exactly four heads, head_dim 128 and key
// blocks of at most 64: two key blocks a workgroup (two waves each), a
// lane per key for two heads of the group -- so that a block's key codes are
// fetched once per workgroup (the two lanes of a key read the same words),
// and a batched step's grid holds half the workgroups, each no longer; the
// same f32 operations in the same order (each shift summed sequentially by
// its own lane, the scores' products as above).
__global__ void __launch_bounds__(256) sage_dec_scores_g4(DecArgs da, DecSeqTab t) {
    if (t.n) dec_seq(da, t, blockIdx.z);
    const RefArgs &a = da.r;
    const uint32_t kbA = 2 * blockIdx.x;
    if (kbA >= a.nkb) return;  // a batched launch covers the longest sequence's blocks
    __shared__ uint32_t qs[4 * 32];
    __shared__ float qd[4], shs[2][4], wmax[4][4];
    __shared__ float kms[2][128];
    __shared__ __attribute__((aligned(16))) float term[2][4 * 128];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t bk = blockIdx.y, bi = wave >> 1, kb = kbA + bi;
    const bool bval = kb < (uint32_t)a.nkb;  // the workgroup's second block may be past the end
    constexpr uint32_t d = 128, d4 = d / 4, n4 = d4 / 4;  // the launch checks head_dim == 128
    const uint32_t kbc = bval ? kb : kbA;
    const uint32_t j0 = kbc * (uint32_t)a.block;
    const uint32_t kj = (uint32_t)(a.block < a.S - j0 ? a.block : a.S - j0);
    const uint32_t hp = lane >> 5, kk = 32 * (wave & 1) + (lane & 31);  // heads hp, hp + 2; key kk
    // The L2-resident operands first (the group's query codes and deltas,
    // the blocks' means), then this lane's key codes and delta from HBM,
    // every load unconditional (indices clamped) so that the wait before
    // the LDS writes counts only the first ones: the shifts below are formed
    // while the key codes are in flight, and the barriers order LDS only.
    const uint32_t qv = da.qsw[(size_t)bk * 4 * d4 + (tid < 4 * d4 ? tid : 0)];
    const float qdv = da.qdl[bk * 4 + (tid & 3)];
    const uint32_t b2m = tid / d < 2 ? tid / d : 1, cm = tid % d;
    const uint32_t kb2 = kbA + b2m < (uint32_t)a.nkb ? kbA + b2m : kbA;
    const float kmv = a.kmean[((size_t)bk * a.pnkb + kb2) * d + cm];
    __builtin_amdgcn_sched_barrier(0);  // the key loads stay behind these
    const uint32_t jl = kk < kj ? kk : kj - 1;
    const u32x4_t *krow = (const u32x4_t *)(a.khat + ((size_t)bk * a.pst + j0 + jl) * d4);
    u32x4_t kv[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; u++) kv[u] = krow[u];
    const float kdl = a.kdelta[(size_t)bk * a.pst + j0 + jl];
    if (tid < 4 * d4) qs[tid] = qv;
    if (tid < 4) qd[tid] = qdv;
    if (tid < 2 * d) kms[b2m][cm] = kmv;
    dec_lds_barrier();
    // the shift's terms (q^_c * dq) * kmean_c, every (block, head, channel)
#pragma unroll
    for (uint32_t k = 0; k < 8 * d / 256; k++) {
        const uint32_t i = tid + 256 * k;
        const uint32_t b2 = i / (4 * d), r = i % (4 * d), h4 = r / d, c = r % d;
        const int qc = (int)(int8_t)(qs[h4 * d4 + c / 4] >> (8 * (c % 4)));
        term[b2][r] = ((float)qc * qd[h4]) * kms[b2][c];
    }
    dec_lds_barrier();
    // each (block, head)'s shift: its terms summed in channel order (:253)
    if (tid < 8) {
        const float *tt = term[tid >> 2] + (tid & 3) * d;
        float shift = 0.0f;
#pragma unroll 4
        for (uint32_t c = 0; c < d; c += 4) {
            const f32x4_t t4 = *(const f32x4_t *)&tt[c];
            shift += t4[0];
            shift += t4[1];
            shift += t4[2];
            shift += t4[3];
        }
        shs[tid >> 2][tid & 3] = shift;
    }
    dec_lds_barrier();
    const bool ok = bval && kk < kj;
#pragma unroll
    for (uint32_t e2 = 0; e2 < 2; e2++) {
        const uint32_t hg = hp + 2 * e2;
        const uint32_t *qh = qs + hg * d4;
        int acc = 0;
#pragma unroll
        for (uint32_t u = 0; u < 8; u++)
            if (u < n4)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc = __builtin_amdgcn_sdot4((int)qh[4 * u + e], (int)kv[u][e], acc, false);
        const float sv = (float)acc * qd[hg] * kdl + shs[bi][hg];
        if (ok) da.sc[((size_t)bk * 4 + hg) * a.S + j0 + kk] = sv;
        // the block max of the head: over the wave's 32 keys, then its two waves
        float rm = ok ? sv : MASKED;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) {
            const float w = __shfl_xor(rm, o, 64);
            rm = w > rm ? w : rm;
        }
        if ((lane & 31) == 0) wmax[wave][hg] = rm;
    }
    dec_lds_barrier();
    if (tid < 8) {
        const uint32_t b2 = tid >> 2, hg = tid & 3;
        const float m0 = wmax[2 * b2][hg], m1 = wmax[2 * b2 + 1][hg];
        if (kbA + b2 < (uint32_t)a.nkb) da.bmax[((size_t)bk * 4 + hg) * a.nkb + kbA + b2] = m1 > m0 ? m1 : m0;
    }
}

// The grouped kernels' instances: the config-5 shape's (group 4, head_dim
// 128, 64-key blocks) and the general bounds.
static void dec_launch_scores(dim3 g, const DecArgs &da, const DecSeqTab &t, hipStream_t st) {
    const RefArgs &a = da.r;
    if (a.H / a.Hk == 4 && a.d == 128 && a.block <= 64)
        hipLaunchKernelGGL(sage_dec_scores_g4, dim3((g.x + 1) / 2, g.y, g.z), dim3(256), 0, st, da, t);
    else if (a.H / a.Hk <= 4 && a.d <= 128)
        hipLaunchKernelGGL((sage_dec_scores_g<4, 128>), g, dim3(256), 0, st, da, t);
    else
        hipLaunchKernelGGL((sage_dec_scores_g<DEC_GMAX, REF_MAXD>), g, dim3(256), 0, st, da, t);
}

static void dec_launch_pv(dim3 g, const DecArgs &da, const DecSeqTab &t, hipStream_t st) {
    const RefArgs &a = da.r;
    if (a.H / a.Hk == 4 && a.dv == 128 && a.block <= 64)
        hipLaunchKernelGGL((sage_dec_pv_g<4, 64, true>), g, dim3(256), 0, st, da, t);
    else if (a.H / a.Hk <= 4 && a.block <= 64)
        hipLaunchKernelGGL((sage_dec_pv_g<4, 64>), g, dim3(256), 0, st, da, t);
    else
        hipLaunchKernelGGL((sage_dec_pv_g<DEC_GMAX, DEC_KMAX>), g, dim3(256), 0, st, da, t);
}

struct DecPlan {
    DecArgs da;
    size_t ws;
    size_t o_kmean, o_kdelta, o_khat, o_vd, o_vhat, o_sc, o_bmax, o_balpha, o_besum, o_blive, o_pvt, o_qsw, o_qdl,
        o_mprev;
};

// The workspace is laid out for a cache of cap tokens (cap >= seq_kv): the
// pre-pass products of the complete key blocks stay where they are as the
// cache grows, so a later step can keep them.
static DecPlan dec_plan(const qbk_attn_shape *s, size_t block, size_t cap) {
    DecPlan P{};
    RefArgs &a = P.da.r;
    a.B = 1;
    a.H = s->n_heads;
    a.Hk = s->n_kv_heads;
    a.S = s->seq_kv;
    a.d = s->head_dim;
    a.dv = s->val_dim;
    a.block = block;
    a.causal = 0;
    a.inv_sqrt_d = 1.0f / sqrtf((float)a.d);
    a.nkb = div_ceil(a.S, block);
    a.d4 = div_ceil(a.d, 4);
    a.blk4 = div_ceil(block < cap ? block : cap, 4);
    // the cache's row-major layout (seq, n_kv_heads, d)
    a.k_tok = a.Hk * a.d;
    a.k_head = a.d;
    a.v_tok = a.Hk * a.dv;
    a.v_head = a.dv;
    a.pst = cap;
    a.pnkb = div_ceil(cap, block);
    a.kb0 = 0;
    const size_t bk = a.Hk, H = a.H, cb = a.pnkb;
    size_t off = 0;
    auto take = [&](size_t n) {
        size_t o = off;
        off += round_up(n ? n : 4, 256);
        return o;
    };
    P.o_kmean = take(bk * cb * a.d * 4);
    P.o_kdelta = take(bk * cap * 4);
    P.o_khat = take(bk * cap * a.d4 * 4);
    P.o_vd = take(bk * cb * a.dv * 4);
    P.o_vhat = take(bk * cb * a.dv * a.blk4 * 4);
    P.o_sc = take(H * cap * 4);
    P.o_bmax = take(H * cb * 4);
    P.o_balpha = take(H * cb * 4);
    P.o_besum = take(H * cb * 4);
    P.o_blive = take(H * cb * 4);
    P.o_pvt = take(H * cb * a.dv * 4);
    P.o_qsw = take(H * a.d4 * 4);
    P.o_qdl = take(H * 4);
    P.o_mprev = take(H * cb * 4);
    P.ws = off;
    return P;
}

// A decode step's shape: batch 1, the step's one query, the cache's keys.
static int validate_decode(const qbk_attn_shape *s, size_t block_size, const size_t *lens) {
    if (!s) return fail(QBK_ERR_VALIDATION, "null shape");
    if (s->batch != 1)
        return fail(QBK_ERR_VALIDATION, fmt("sage decode takes one sequence: batch must be 1, got %zu", s->batch));
    if (s->n_heads == 0 || s->n_kv_heads == 0)
        return fail(QBK_ERR_VALIDATION, "attention requires non-empty batch and head dimensions");
    if (s->n_heads % s->n_kv_heads != 0)
        return fail(QBK_ERR_VALIDATION, fmt("n_kv_heads must divide n_heads: n_heads=%zu, "
                                            "n_kv_heads=%zu",
                                            s->n_heads, s->n_kv_heads));
    if (s->seq_q != 1)
        return fail(QBK_ERR_VALIDATION,
                    fmt("sage decode takes the step's one query: seq_q must be 1, got %zu", s->seq_q));
    if (s->seq_kv == 0 || s->head_dim == 0 || s->val_dim == 0)
        return fail(QBK_ERR_VALIDATION,
                    "attention requires non-empty sequence and head dimensions");
    if (block_size == 0)
        return fail(QBK_ERR_VALIDATION,
                    "sage attention requires a positive block_size ([SA] \xc2\xa7"
                    "4's tile width)");
    if (lens) {
        const size_t eq = s->n_heads * s->head_dim, ek = s->seq_kv * s->n_kv_heads * s->head_dim,
                     ev = s->seq_kv * s->n_kv_heads * s->val_dim, eo = s->n_heads * s->val_dim;
        if (lens[0] != eq)
            return fail(QBK_ERR_VALIDATION, fmt("query must hold %zu values for %s, got %zu", eq,
                                                shape_debug(s).c_str(), lens[0]));
        if (lens[1] != ek)
            return fail(QBK_ERR_VALIDATION, fmt("key cache must hold %zu values for %s, got %zu", ek,
                                                shape_debug(s).c_str(), lens[1]));
        if (lens[2] != ev)
            return fail(QBK_ERR_VALIDATION, fmt("value cache must hold %zu values for %s, got %zu", ev,
                                                shape_debug(s).c_str(), lens[2]));
        if (lens[3] != eo)
            return fail(QBK_ERR_VALIDATION, fmt("out must hold %zu values for %s, got %zu", eo,
                                                shape_debug(s).c_str(), lens[3]));
    }
    if (s->head_dim > REF_MAXD || s->val_dim > REF_MAXD)
        return fail(QBK_ERR_VALIDATION,
                    fmt("sage attention on this device supports head_dim and val_dim up to %d, "
                        "got head_dim=%zu, val_dim=%zu",
                        REF_MAXD, s->head_dim, s->val_dim));
    return QBK_OK;
}

static const DecSeqTab kNoSeqs{};

// Binds a decode plan's workspace pointers to ws.
static void dec_bind(const DecPlan &P, DecArgs &da, void *ws) {
    RefArgs &a = da.r;
    char *w = (char *)ws;
    a.kmean = (float *)(w + P.o_kmean);
    a.kdelta = (float *)(w + P.o_kdelta);
    a.khat = (uint32_t *)(w + P.o_khat);
    a.vd = (float *)(w + P.o_vd);
    a.vhat = (uint32_t *)(w + P.o_vhat);
    da.sc = (float *)(w + P.o_sc);
    da.bmax = (float *)(w + P.o_bmax);
    da.balpha = (float *)(w + P.o_balpha);
    da.besum = (float *)(w + P.o_besum);
    da.blive = (int *)(w + P.o_blive);
    da.pvt = (float *)(w + P.o_pvt);
    da.qsw = (uint32_t *)(w + P.o_qsw);
    da.qdl = (float *)(w + P.o_qdl);
    da.mprev = nullptr;
    da.op_s2 = nullptr;
    da.op = da.op_sc = nullptr;
}

// One step over seq_kv cached tokens with a workspace laid out for cap; the
// products of the key blocks that were complete at cached tokens are taken
// as they are (the caller guarantees that those cache rows are the ones the
// workspace's earlier step quantised) and the rest are quantised again.
static int run_decode(const qbk_attn_shape *s, const float *q, const float *k, const float *v,
                      size_t block, float *out, void *ws, size_t cap, size_t cached, hipStream_t st,
                      const DecOpSink *sink = nullptr, const DecRope *rope = nullptr) {
    DecPlan P = dec_plan(s, block, cap);
    DecArgs da = P.da;
    RefArgs &a = da.r;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    char *w = (char *)ws;
    dec_bind(P, da, ws);
    if (sink) {
        da.op_s2 = sink->s2;
        da.op = sink->op;
        da.op_sc = sink->sc;
    }
    const unsigned nkb = (unsigned)a.nkb, H = (unsigned)a.H;
    a.kb0 = cached / block;
    const DPrepGeom g = dprep_geom(a, k, v);
    const size_t G = a.H / a.Hk, kjm = a.block < a.S ? a.block : a.S;
    const bool grouped = g.ok && G <= DEC_GMAX && kjm <= DEC_KMAX && a.d % 16 == 0 && a.blk4 % 4 == 0;
    if (rope && !grouped)
        return fail(QBK_ERR_VALIDATION, "sage decode: the RoPE fold needs the grouped decode kernels");
    if (g.ok && (a.kb0 < a.nkb || grouped)) {
        const unsigned nx = (unsigned)(a.kb0 < a.nkb ? a.nkb - a.kb0 : 1);
        const size_t lds = rope && g.lds < 16 * a.d ? 16 * a.d : g.lds;  // the query's rotated heads
        hipLaunchKernelGGL(sage_dec_prep, dim3(nx, (unsigned)a.Hk, g.ks + g.vs + (grouped ? 1 : 0)),
                           dim3(256), lds, st, a, g, grouped ? da.qsw : nullptr, grouped ? da.qdl : nullptr,
                           kNoSeqs, rope ? *rope : DecRope{});
        QBK_HIP(hipGetLastError());
    } else if (a.kb0 < a.nkb) {
        hipLaunchKernelGGL(sage_ref_prep, dim3((unsigned)(a.nkb - a.kb0), (unsigned)a.Hk), dim3(256),
                           ref_prep_lds(a.d, a.dv, a.block), st, a);
        QBK_HIP(hipGetLastError());
    }
    if (grouped) {
        dec_launch_scores(dim3(nkb, (unsigned)a.Hk), da, kNoSeqs, st);
        QBK_HIP(hipGetLastError());
        if (a.nkb > DEC_PMAX) {
            da.mprev = (float *)(w + P.o_mprev);
            hipLaunchKernelGGL(sage_dec_runmax, dim3(H), dim3(256), 0, st, da, kNoSeqs);
            QBK_HIP(hipGetLastError());
        }
        dec_launch_pv(dim3(nkb, (unsigned)a.Hk), da, kNoSeqs, st);
        QBK_HIP(hipGetLastError());
        hipLaunchKernelGGL(sage_dec_combine, dim3(H), dim3(256), 0, st, da, kNoSeqs);
        QBK_HIP(hipGetLastError());
        return QBK_OK;
    }
    hipLaunchKernelGGL(sage_dec_scores, dim3(nkb, H), dim3(256), 0, st, da);
    QBK_HIP(hipGetLastError());
    if (a.nkb > DEC_PMAX) {
        da.mprev = (float *)(w + P.o_mprev);
        hipLaunchKernelGGL(sage_dec_runmax, dim3(H), dim3(256), 0, st, da, kNoSeqs);
        QBK_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(sage_dec_pv, dim3(nkb, H), dim3(256), 0, st, da);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(sage_dec_combine, dim3(H), dim3(256), 0, st, da, kNoSeqs);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

// The grouped kernels' batched form (sequences along the grid's last
// dimension) fits a shape when its widest block does: the geometry at
// seq_kv = cap bounds every sequence's.
static bool dec_batch_plan(const qbk_attn_shape *one, size_t block, size_t cap, const float *k, const float *v,
                           size_t kv_stride, DecPlan &P, DPrepGeom &g) {
    qbk_attn_shape sh = *one;
    sh.seq_kv = cap;
    P = dec_plan(&sh, block, cap);
    const RefArgs &a = P.da.r;
    g = dprep_geom(a, k, v);
    const size_t G = a.H / a.Hk, kjm = block < cap ? block : cap;
    return g.ok && G <= DEC_GMAX && kjm <= DEC_KMAX && a.d % 16 == 0 && a.blk4 % 4 == 0 && kv_stride % 4 == 0;
}

bool sage_decode_batchable(const qbk_attn_shape *one, size_t block, size_t cap, const float *k, const float *v,
                           size_t kv_stride) {
    DecPlan P;
    DPrepGeom g;
    return one && block && cap && dec_batch_plan(one, block, cap, k, v, kv_stride, P, g);
}

int sage_decode_batch(const qbk_attn_shape *one, const float *q, size_t q_stride, const float *k, const float *v,
                      size_t kv_stride, size_t block, float *out, size_t o_stride, void *state, size_t st_stride,
                      size_t cap, const size_t *seq_kv, const size_t *cached, size_t n, hipStream_t st,
                      const uint32_t *pos_dev, const DecOpSink *sink, const DecRope *rope) {
    DecPlan P;
    DPrepGeom g;
    if (n == 0 || n > QBK_DEC_MAXSEQ || !dec_batch_plan(one, block, cap, k, v, kv_stride, P, g))
        return fail(QBK_ERR_VALIDATION, "sage decode: no batched form for this shape");
    if ((sink || rope) && n != 1)
        return fail(QBK_ERR_VALIDATION, "sage decode: an operand sink or a RoPE fold serves one sequence");
    DecArgs da = P.da;
    RefArgs &a = da.r;
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    dec_bind(P, da, state);
    if (sink) {
        da.op_s2 = sink->s2;
        da.op = sink->op;
        da.op_sc = sink->sc;
    }
    DecSeqTab t{};
    t.n = (uint32_t)n;
    t.q_stride = q_stride;
    t.o_stride = o_stride;
    t.kv_stride = kv_stride;
    t.st_stride = st_stride;
    t.pos = pos_dev;
    size_t mkb = 0, mx = 1;
    if (pos_dev) mkb = a.pnkb;  // the capacity's blocks; one block (the position's) to quantise
    for (size_t i = 0; !pos_dev && i < n; i++) {
        if (seq_kv[i] == 0 || seq_kv[i] > cap || cached[i] > seq_kv[i])
            return fail(QBK_ERR_VALIDATION, fmt("sage decode: sequence %zu holds %zu tokens (%zu kept) in a "
                                                "capacity of %zu", i, seq_kv[i], cached[i], cap));
        const size_t nkb = div_ceil(seq_kv[i], block), kb0 = cached[i] / block;
        t.S[i] = (uint32_t)seq_kv[i];
        t.kb0[i] = (uint32_t)kb0;
        mkb = nkb > mkb ? nkb : mkb;
        mx = nkb - kb0 > mx ? nkb - kb0 : mx;
    }
    const unsigned Hk = (unsigned)a.Hk, H = (unsigned)a.H, ns = (unsigned)n;
    // one workgroup each for K and V per (sequence, kv head, block) once the
    // pairs alone fill the chip (the split only shortens one sequence's step)
    if (Hk * ns >= 64) {
        const DPrepGeom g1 = dprep_geom(a, k, v, 1, 1);
        if (g1.ok) g = g1;
    }
    const size_t lds = rope && g.lds < 16 * a.d ? 16 * a.d : g.lds;  // the query's rotated heads
    hipLaunchKernelGGL(sage_dec_prep, dim3((unsigned)mx, Hk * ns, g.ks + g.vs + 1), dim3(256), lds, st, a, g,
                       da.qsw, da.qdl, t, rope ? *rope : DecRope{});
    QBK_HIP(hipGetLastError());
    dec_launch_scores(dim3((unsigned)mkb, Hk, ns), da, t, st);
    QBK_HIP(hipGetLastError());
    if (mkb > DEC_PMAX) {
        da.mprev = (float *)((char *)state + P.o_mprev);
        hipLaunchKernelGGL(sage_dec_runmax, dim3(H, ns), dim3(256), 0, st, da, t);
        QBK_HIP(hipGetLastError());
    }
    dec_launch_pv(dim3((unsigned)mkb, Hk, ns), da, t, st);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(sage_dec_combine, dim3(H, ns), dim3(256), 0, st, da, t);
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

typedef int i32x4_t __attribute__((ext_vector_type(4)));
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
    uint16_t *vt;     // [B*Hk][nblk][HD][BLK] fp16, V^T per key block, keys in PV order
    int8_t *qhat_out; // quantize-only launch: Q codes [B*H][S][HD] and scales [B*H][nblk]
    float *qscale_out;
    int hpx;          // heads per XCD of the XCD-aware tile order (0: plain order)
    int out_rows;     // 1: out token-major [B][S][H][HD] (the o projection's rows), 0: [B][H][S][HD]
};

// Key order of a V^T block: within each 32-key chunk, position 8g + e holds
// key 4g + (e & 3) + 16 (e >> 2) -- the keys lane group g of an S^T 16x16
// C tile pair holds, in the order that lane feeds them to the P.V MFMA as
// its 8 fp16 B elements.  So every V^T fragment is one 16-byte read.
__host__ __device__ __forceinline__ int vt_key(int pos) {
    const int kc = pos >> 5, g = (pos >> 3) & 3, e = pos & 7;
    return 32 * kc + 4 * g + (e & 3) + 16 * (e >> 2);
}

// chunk partial sums of K per channel, token order within the chunk: one
// workgroup per (block, kv head), two channels per thread
__global__ void __launch_bounds__(64) blk_kpart(BlkArgs a) {
    const size_t blk = blockIdx.x, bk = blockIdx.y;
    const int c = 2 * threadIdx.x;
    const uint32_t *K = (const uint32_t *)(a.k + bk * a.S * HD + c);
    const size_t t0 = blk * BLK, t1 = t0 + BLK < a.S ? t0 + BLK : a.S;
    float p0 = 0.0f, p1 = 0.0f;
    size_t t = t0;
    for (; t + 8 <= t1; t += 8) {
        uint32_t w[8];
#pragma unroll
        for (int u = 0; u < 8; u++) w[u] = K[(t + u) * (HD / 2)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            p0 += __uint_as_float(w[u] << 16);
            p1 += __uint_as_float(w[u] & 0xffff0000u);
        }
    }
    for (; t < t1; t++) {
        const uint32_t w = K[t * (HD / 2)];
        p0 += __uint_as_float(w << 16);
        p1 += __uint_as_float(w & 0xffff0000u);
    }
    *(float2 *)&a.kpart[(bk * a.nblk + blk) * HD + c] = make_float2(p0, p1);
}

// K channel mean of channel c of kv head bk: the chunk partials summed in
// chunk order, / S.
__device__ __forceinline__ float blk_mean_of(const BlkArgs &a, size_t bk, int c) {
    const float *part = a.kpart + bk * a.nblk * HD + c;
    float tot = 0.0f;
    size_t p = 0;
    for (; p + 16 <= a.nblk; p += 16) {  // loads in flight together, sums in chunk order
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = part[(p + u) * HD];
#pragma unroll
        for (int u = 0; u < 16; u++) tot += v[u];
    }
    for (; p < a.nblk; p++) tot += part[p * HD];
    return tot / (float)a.S;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// K: smoothing by the channel mean, block scale, codes; V: bf16 -> fp16,
// transposed per key block into PV order.  One workgroup per (block, kv
// head); thread t holds token t/4, channels 32 (t%4) .. +31.  Each
// workgroup forms the channel means itself from the chunk partials (the
// first of a kv head also stores them): a separate launch cost more than
// the redundant sums, which stay in L2.
__global__ void __launch_bounds__(256) blk_kvquant(BlkArgs a) {
    __shared__ float mean[HD];
    __shared__ float red[4];
    __shared__ uint16_t vs[BLK][HD + 2];  // fp16 V, token-major
    const size_t blk = blockIdx.x, bk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < HD) {
        const float m = blk_mean_of(a, bk, tid);
        mean[tid] = m;
        if (blk == 0) a.kmean[bk * HD + tid] = m;
    }
    __syncthreads();
    const size_t t0 = blk * BLK;
    const int tt = tid >> 2, c0 = 32 * (tid & 3);
    const bool live = t0 + tt < a.S;
    float g[32];
    float peak = 0.0f;
    {
        const u32x4_t *src = (const u32x4_t *)(a.k + (bk * a.S + t0 + tt) * HD + c0);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const u32x4_t w = live ? src[u] : u32x4_t{0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                g[8 * u + 2 * e] = __uint_as_float(w[e] << 16) - mean[c0 + 8 * u + 2 * e];
                g[8 * u + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u) - mean[c0 + 8 * u + 2 * e + 1];
            }
        }
        if (live)
#pragma unroll
            for (int e = 0; e < 32; e++) peak = fmaxf(peak, fabsf(g[e]));
    }
    peak = wave_max(peak);
    if (lane == 0) red[wave] = peak;
    // V: fp16, token-major into LDS
    {
        const u32x4_t *src = (const u32x4_t *)(a.v + (bk * a.S + t0 + tt) * HD + c0);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const u32x4_t w = live ? src[u] : u32x4_t{0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const f32x2_t f = {__uint_as_float(w[e] << 16), __uint_as_float(w[e] & 0xffff0000u)};
                *(uint32_t *)&vs[tt][c0 + 8 * u + 2 * e] =
                    __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2_t));
            }
        }
    }
    __syncthreads();
    peak = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float inv = peak > 0.0f ? 127.0f / peak : 0.0f;
    if (tid == 0) a.kscale[bk * a.nblk + blk] = peak > 0.0f ? peak / 127.0f : 1.0f;
    {
        uint32_t w[8];
#pragma unroll
        for (int u = 0; u < 8; u++)
            w[u] = live ? pack4(q8(g[4 * u] * inv), q8(g[4 * u + 1] * inv), q8(g[4 * u + 2] * inv),
                                q8(g[4 * u + 3] * inv))
                        : 0u;
        u32x4_t *dst = (u32x4_t *)(a.khat + (bk * a.Sp + t0 + tt) * HD + c0);
        dst[0] = u32x4_t{w[0], w[1], w[2], w[3]};
        dst[1] = u32x4_t{w[4], w[5], w[6], w[7]};
    }
    // V^T [HD][BLK] in PV key order: 1024 16-byte pieces (channel d, 8 positions), four per thread
    u32x4_t *VT = (u32x4_t *)(a.vt + (bk * a.nblk + blk) * HD * BLK);
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int x = tid + 256 * u, d = x >> 3, p0 = (x & 7) * 8;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            w[e] = (uint32_t)vs[vt_key(p0 + 2 * e)][d] | ((uint32_t)vs[vt_key(p0 + 2 * e + 1)][d] << 16);
        VT[x] = u32x4_t{w[0], w[1], w[2], w[3]};
    }
}

// max over lanes l, l ^ 16, l ^ 32, l ^ 48 -- the four lanes that share a
// query column of a 16x16 C tile -- with v_permlane16/32_swap: swapping a
// register with itself hands each lane the other row's (half's) value in
// one of the two results, in the VALU, with no LDS round trip.
__device__ __forceinline__ int lanes_max4(int v) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    const int a = max((int)r16[0], (int)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(a, a, false, false);
    return max((int)r32[0], (int)r32[1]);
}

#pragma clang fp contract(fast)

// LDS tiles: K^ [64 keys][128 B], V^T [128 d][128 B], Q codes [128
// queries][128 B]; each 128-byte row keeps its eight 16-byte chunks
// XOR-swizzled by the row (chunk c at c ^ (row & 7)), so that the eight
// lanes of a 16-byte-read phase -- eight consecutive rows, one chunk -- hit
// disjoint banks.
__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

// Main pass.  Workgroup: (128-query tile, batch*head); wave w owns queries
// qw = q0 + 32w .. +31 (two 16-query MFMA tiles, one quantisation block of
// two waves).  Prologue: Q codes of the tile, block scale over the wave
// pair.  Per key block (64 keys, double-buffered in LDS, loads for the next
// block issued unconditionally -- the last one reloaded -- ahead of the
// math):
//   S^T[64 x 32] = K^[64 x 128] . Q^T  -- i8 16x16x64, 4 key tiles x 2 query
//                  tiles x 2 d-chunks; C lane l holds query l%16, keys
//                  4(l/16) + i of its key tile;
//   online softmax per query column on the integer scores: block max by
//   v_max3 (the scale is positive), one cvt + fma + exp2 per score, masks
//   only on the causal diagonal and the ragged last block, and a reference
//   max that moves (rescaling O and l) only when a block max exceeds it by
//   more than 8 in log2 units;
//   O^T[128 x 32] += V^T . P^T and l += 1 . P^T -- f16 16x16x32, P^T taken
//                  straight from the S^T registers (PV key order above), the
//                  row sums from a ninth tile of ones.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) blk_attn(BlkArgs a) {
    // K^ and V^T tiles, double buffered -- four separate objects, so that the
    // compiler can tell a read of one from the direct loads into another
    __shared__ __attribute__((aligned(16))) uint8_t kl0[BLK * 128], kl1[BLK * 128];
    __shared__ __attribute__((aligned(16))) uint8_t vl0[HD * 128], vl1[HD * 128];
#define KL(B) ((B) ? kl1 : kl0)
#define VL(B) ((B) ? vl1 : vl0)
    // the prologue's block-peak exchange; V^T buffer 1 is first loaded after
    // the barrier that ends the prologue
    float *red = (float *)vl1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, col = lane & 15;
    const size_t nq = (a.S + BQ - 1) / BQ, BH = a.B * a.H;
    size_t bh, qi;
    {
        const size_t L = blockIdx.x;
        if (a.hpx) {  // XCD x = L % 8 runs heads x*hpx .. +hpx-1, heaviest tiles first
            const size_t s = L / 8;
            bh = (L % 8) * a.hpx + s % a.hpx;
            qi = nq - 1 - s / a.hpx;
        } else {
            bh = L % BH;
            qi = nq - 1 - L / BH;
        }
    }
    const size_t b = bh / a.H, h = bh % a.H;
    const size_t bk = b * a.Hk + h / (a.H / a.Hk);
    const size_t q0 = qi * BQ, qw = q0 + 32 * wave;

    // ---- Q codes (B operand): query qw + 16 qt + col, d = 64 dc + 16 g + e,
    // kept in registers for every key block
    float qsc;
    i32x4_t qf[2][2];
    {
        float x[2][2][16];
        float pk = 0.0f;
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            const size_t q = qw + 16 * qt + col;
            const bool ok = q < a.S;
#pragma unroll
            for (int dc = 0; dc < 2; dc++) {
                const u32x4_t *src = (const u32x4_t *)(a.q + (bh * a.S + (ok ? q : 0)) * HD + 64 * dc + 16 * g);
                const u32x4_t w0 = ok ? src[0] : u32x4_t{0, 0, 0, 0};
                const u32x4_t w1 = ok ? src[1] : u32x4_t{0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[qt][dc][2 * e] = __uint_as_float(w0[e] << 16) * a.inv_sqrt_d;
                    x[qt][dc][2 * e + 1] = __uint_as_float(w0[e] & 0xffff0000u) * a.inv_sqrt_d;
                    x[qt][dc][8 + 2 * e] = __uint_as_float(w1[e] << 16) * a.inv_sqrt_d;
                    x[qt][dc][8 + 2 * e + 1] = __uint_as_float(w1[e] & 0xffff0000u) * a.inv_sqrt_d;
                }
#pragma unroll
                for (int e = 0; e < 16; e++) pk = fmaxf(pk, fabsf(x[qt][dc][e]));
            }
        }
        pk = wave_max(pk);
        if (lane == 0) red[wave] = pk;
        __syncthreads();
        const float peak = fmaxf(red[wave & ~1], red[wave | 1]);  // the wave pair's 64-query block
        const float inv = peak > 0.0f ? 127.0f / peak : 0.0f;
        qsc = peak > 0.0f ? peak / 127.0f : 1.0f;
#pragma unroll
        for (int qt = 0; qt < 2; qt++)
#pragma unroll
            for (int dc = 0; dc < 2; dc++)
#pragma unroll
                for (int w = 0; w < 4; w++)
                    qf[qt][dc][w] = (int)pack4(q8(x[qt][dc][4 * w] * inv), q8(x[qt][dc][4 * w + 1] * inv),
                                               q8(x[qt][dc][4 * w + 2] * inv), q8(x[qt][dc][4 * w + 3] * inv));
        if (a.qhat_out) {  // quantize-only launch: export the codes and scales
#pragma unroll
            for (int qt = 0; qt < 2; qt++) {
                const size_t q = qw + 16 * qt + col;
                if (q >= a.S) continue;
#pragma unroll
                for (int dc = 0; dc < 2; dc++)
                    *(i32x4_t *)(a.qhat_out + (bh * a.S + q) * HD + 64 * dc + 16 * g) = qf[qt][dc];
            }
            if ((wave & 1) == 0 && lane == 0 && qw < a.S) a.qscale_out[bh * a.nblk + qw / BLK] = qsc;
            return;
        }
    }

    // ---- key blocks
    const size_t qlast = q0 + BQ - 1 < a.S - 1 ? q0 + BQ - 1 : a.S - 1;
    const size_t kb_end = a.causal ? qlast / BLK + 1 : a.nblk;
    const bool wave_live = qw < a.S;
    const size_t wlast = qw + 31 < a.S - 1 ? qw + 31 : a.S - 1;
    const size_t wave_kb_end = !wave_live ? 0 : a.causal ? wlast / BLK + 1 : a.nblk;

    f32x4_t o[2][8], lt[2];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        lt[qt] = f32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int ct = 0; ct < 8; ct++) o[qt][ct] = f32x4_t{0, 0, 0, 0};
    }
    float mrow[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};
    const f16x8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};

    // K^ tiles load two blocks ahead and V^T tiles one, into double buffers
    // (issued at the top of an iteration, waited for at its end), straight
    // into LDS: a K^ tile is 8 and a V^T tile 16 1-KB pieces of eight
    // 128-byte rows, and lane i of a global_load_lds_dwordx4 fills bytes
    // 16 i .. of its piece, so it fetches the source chunk that the swizzle
    // puts there.  Every LDS fragment is read a phase before its MFMAs: the
    // next block's Q and K^ fragments at the end of an iteration (they wait
    // out the barrier in registers), the first key chunk's V^T fragments at
    // the top, the second chunk's under the first chunk's P.V MFMAs.
    const int lr = lane >> 3, lcs = ((lane & 7) ^ lr) * 16;
    // the K block scales through the constant address space: scalar loads,
    // counted apart from the tile loads in flight
    const __attribute__((address_space(4))) float *kscl =
        (const __attribute__((address_space(4))) float *)(a.kscale + bk * a.nblk);
    const uint8_t *ksrc0 = (const uint8_t *)a.khat + bk * a.Sp * HD;
    const uint8_t *vsrc0 = (const uint8_t *)a.vt + bk * a.nblk * HD * BLK * 2;
    // a lane's byte offset within tile piece wave + 4 u: row 8 (wave + 4 u) + lr,
    // swizzled chunk (the uniform tile base stays in SGPRs)
    const uint32_t loff = (uint32_t)(8 * wave + lr) * 128 + lcs;
#define BLK_LOAD_K(KB, BUF)                                                                     \
    {                                                                                           \
        const uint8_t *kb_ = ksrc0 + (KB) * (BLK * HD);                                         \
        _Pragma("unroll") for (int u = 0; u < 2; u++)                                           \
            __builtin_amdgcn_global_load_lds((const void *)(kb_ + (loff + u * 4096u)),           \
                                             (__attribute__((address_space(3))) void *)&KL(BUF)[(wave + 4 * u) * 1024], 16, 0, 0);\
    }
#define BLK_LOAD_V(KB, BUF)                                                                     \
    {                                                                                           \
        const uint8_t *vb_ = vsrc0 + (KB) * (HD * BLK * 2);                                     \
        _Pragma("unroll") for (int u = 0; u < 4; u++)                                           \
            __builtin_amdgcn_global_load_lds((const void *)(vb_ + (loff + u * 4096u)),           \
                                             (__attribute__((address_space(3))) void *)&VL(BUF)[(wave + 4 * u) * 1024], 16, 0, 0);\
    }
    // the K^ fragments of the block whose K^ tile is in buffer BUF
#define BLK_FRAGS(BUF)                                                                          \
    {                                                                                           \
        _Pragma("unroll") for (int kt = 0; kt < 4; kt++)                                        \
        _Pragma("unroll") for (int dc = 0; dc < 2; dc++)                                        \
            kf[kt][dc] = *(const i32x4_t *)&KL(BUF)[swz(16 * kt + col, 4 * dc + g)];            \
    }
    // Softmax of one block's scores st into pf / alpha / moved; MASKED (a
    // constant) zeroes the p of the keys set in mbits.  A lane moves its
    // reference max only when the block max exceeds it by more than 8
    // (log2): below that p = exp2(s - m) <= 256, and O / l does not depend on
    // which reference max the accumulators share, so most blocks skip the O
    // rescale.
#define BLK_SOFTMAX(MASKED)                                                                     \
    _Pragma("unroll") for (int qt = 0; qt < 2; qt++) {                                          \
        int mi = INT32_MIN;                                                                     \
        _Pragma("unroll") for (int kt = 0; kt < 4; kt++)                                        \
            mi = max(max(mi, st[kt][qt][0]), max(st[kt][qt][1], max(st[kt][qt][2], st[kt][qt][3])));\
        mi = lanes_max4(mi);                                                                    \
        const float mb = mi == INT32_MIN ? -__builtin_huge_valf() : (float)mi * cs;             \
        const bool up = mb > mrow[qt] + 8.0f;                                                   \
        alpha[qt] = up ? __builtin_amdgcn_exp2f(mrow[qt] - mb) : 1.0f;                          \
        moved |= up;                                                                            \
        mrow[qt] = up ? mb : mrow[qt];                                                          \
        const float nm = mrow[qt] == -__builtin_huge_valf() ? 0.0f : -mrow[qt];                 \
        _Pragma("unroll") for (int kc = 0; kc < 2; kc++) {                                      \
            float p[8];                                                                         \
            _Pragma("unroll") for (int i = 0; i < 4; i++) {                                     \
                p[i] = __builtin_amdgcn_exp2f((float)st[2 * kc][qt][i] * cs + nm);              \
                p[4 + i] = __builtin_amdgcn_exp2f((float)st[2 * kc + 1][qt][i] * cs + nm);      \
                if (MASKED) {                                                                   \
                    p[i] = (mbits[qt] >> (8 * kc + i)) & 1 ? 0.0f : p[i];                       \
                    p[4 + i] = (mbits[qt] >> (8 * kc + 4 + i)) & 1 ? 0.0f : p[4 + i];           \
                }                                                                               \
            }                                                                                   \
            _Pragma("unroll") for (int i = 0; i < 4; i++) {                                     \
                const f32x2_t pp = {p[2 * i], p[2 * i + 1]};                                    \
                const f16x2_t hh = __builtin_convertvector(pp, f16x2_t);                        \
                pf[qt][kc][2 * i] = hh[0];                                                      \
                pf[qt][kc][2 * i + 1] = hh[1];                                                  \
            }                                                                                   \
        }                                                                                       \
    }
    // One key block KB from buffer B (masks only on the causal diagonal and
    // the ragged last block).
#define BLK_ITER(KB, B)                                                                         \
    {                                                                                           \
        const size_t k1 = (KB) + 1 < kb_end ? (KB) + 1 : kb_end - 1;                            \
        const size_t k2 = (KB) + 2 < kb_end ? (KB) + 2 : kb_end - 1;                            \
        BLK_LOAD_K(k2, B)                                                                       \
        BLK_LOAD_V(k1, (B) ^ 1)                                                                 \
        __builtin_amdgcn_sched_barrier(0);                                                      \
        if ((KB) < wave_kb_end) {                                                               \
            const float cs = (qsc * kscl[KB]) * LOG2E_F;                                        \
            const uint8_t *VT = VL(B);                                                          \
            f16x8_t vf0[8];                                                                     \
            _Pragma("unroll") for (int ct = 0; ct < 8; ct++)                                    \
                vf0[ct] = *(const f16x8_t *)&VT[swz(16 * ct + col, g)];                         \
            i32x4_t st[4][2];                                                                   \
            _Pragma("unroll") for (int kt = 0; kt < 4; kt++)                                    \
            _Pragma("unroll") for (int qt = 0; qt < 2; qt++) {                                  \
                st[kt][qt] = i32x4_t{0, 0, 0, 0};                                               \
                _Pragma("unroll") for (int dc = 0; dc < 2; dc++)                                \
                    st[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[kt][dc], qf[qt][dc], st[kt][qt], 0, 0, 0);\
            }                                                                                   \
            const bool masked = (a.causal && (KB) * BLK + BLK - 1 > qw) || (KB) * BLK + BLK > a.S;\
            f16x8_t pf[2][2];                                                                   \
            bool moved = false;                                                                 \
            float alpha[2];                                                                     \
            if (masked) {                                                                       \
                uint32_t mbits[2] = {0u, 0u};                                                   \
                _Pragma("unroll") for (int qt = 0; qt < 2; qt++) {                              \
                    const int qrel = (int)(qw + 16 * qt + col - (KB) * BLK);                    \
                    const int klim = (int)(a.S - (KB) * BLK);                                   \
                    _Pragma("unroll") for (int kt = 0; kt < 4; kt++)                            \
                    _Pragma("unroll") for (int i = 0; i < 4; i++) {                             \
                        const int kr = 16 * kt + 4 * g + i;                                     \
                        if ((a.causal && kr > qrel) || kr >= klim) {                            \
                            st[kt][qt][i] = INT32_MIN;                                          \
                            mbits[qt] |= 1u << (4 * kt + i);                                    \
                        }                                                                       \
                    }                                                                           \
                }                                                                               \
                BLK_SOFTMAX(true)                                                               \
            } else {                                                                            \
                const uint32_t mbits[2] = {0u, 0u};                                             \
                BLK_SOFTMAX(false)                                                              \
            }                                                                                   \
            if (__builtin_amdgcn_ballot_w64(moved)) {                                           \
                _Pragma("unroll") for (int qt = 0; qt < 2; qt++) {                              \
                    lt[qt] *= alpha[qt];                                                        \
                    _Pragma("unroll") for (int ct = 0; ct < 8; ct++) o[qt][ct] *= alpha[qt];    \
                }                                                                               \
            }                                                                                   \
            f16x8_t vf1[8];                                                                     \
            _Pragma("unroll") for (int ct = 0; ct < 8; ct++) {                                  \
                vf1[ct] = *(const f16x8_t *)&VT[swz(16 * ct + col, 4 + g)];                     \
                _Pragma("unroll") for (int qt = 0; qt < 2; qt++)                                \
                    o[qt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf0[ct], pf[qt][0], o[qt][ct], 0, 0, 0);\
            }                                                                                   \
            _Pragma("unroll") for (int qt = 0; qt < 2; qt++)                                    \
                lt[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[qt][0], lt[qt], 0, 0, 0);\
            _Pragma("unroll") for (int ct = 0; ct < 8; ct++)                                    \
            _Pragma("unroll") for (int qt = 0; qt < 2; qt++)                                    \
                o[qt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf1[ct], pf[qt][1], o[qt][ct], 0, 0, 0);\
            _Pragma("unroll") for (int qt = 0; qt < 2; qt++)                                    \
                lt[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[qt][1], lt[qt], 0, 0, 0);\
        }                                                                                       \
        __builtin_amdgcn_sched_barrier(0);                                                      \
        BLK_FRAGS((B) ^ 1)                                                                      \
        __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): the next tiles have landed */        \
        __syncthreads();                                                                        \
    }
    i32x4_t kf[4][2];
    BLK_LOAD_K(0, 0)
    BLK_LOAD_K(kb_end > 1 ? 1 : 0, 1)
    BLK_LOAD_V(0, 0)
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    BLK_FRAGS(0)
    __syncthreads();  // every wave has read K^ buffer 0 before block 2 loads into it
    size_t kb = 0;
    for (; kb + 2 <= kb_end; kb += 2) {
        BLK_ITER(kb, 0)
        BLK_ITER(kb + 1, 1)
    }
    if (kb < kb_end) BLK_ITER(kb, 0)
#undef BLK_ITER
#undef BLK_SOFTMAX
#undef BLK_LOAD_K
#undef BLK_LOAD_V
#undef BLK_FRAGS
#undef KL
#undef VL
    if (!wave_live) return;
    // ---- normalise and store: lane holds query col, channels 16 ct + 4 g + i
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const float inv = 1.0f / lt[qt][0];
        const size_t q = qw + 16 * qt + col;
        if (q >= a.S) continue;
        uint16_t *dst = a.out + (a.out_rows ? ((b * a.S + q) * a.H + h) * HD : (bh * a.S + q) * HD);
#pragma unroll
        for (int ct = 0; ct < 8; ct++) {
            const uint32_t w0 = f32x2_to_bf16x2(o[qt][ct][0] * inv, o[qt][ct][1] * inv);
            const uint32_t w1 = f32x2_to_bf16x2(o[qt][ct][2] * inv, o[qt][ct][3] * inv);
            *(uint2 *)(dst + 16 * ct + 4 * g) = make_uint2(w0, w1);
        }
    }
}

#pragma clang fp contract(off)

// export the K codes and V (fp16) of the pre-pass in natural layouts (parity checks)
__global__ void blk_export(BlkArgs a, int8_t *khat, uint16_t *vh) {
    const size_t x = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nk = a.B * a.Hk * a.S * HD;
    if (x >= nk) return;
    const size_t bk = x / (a.S * HD), rem = x % (a.S * HD);
    const size_t t = rem / HD, c = rem % HD;
    khat[x] = a.khat[bk * a.Sp * HD + rem];
    // key t % 64 of its block sits at the position whose vt_key is it
    const int kr = (int)(t % BLK), kc = kr >> 5, j = kr & 31, tt = j >> 4, r = j & 15;
    const int pos = 32 * kc + 8 * (r >> 2) + 4 * tt + (r & 3);
    vh[x] = a.vt[((bk * a.nblk + t / BLK) * HD + c) * BLK + pos];
}

struct BlkPlan {
    BlkArgs a;
    size_t ws;
    size_t o_kpart, o_kmean, o_khat, o_kscale, o_vt;
};

static BlkPlan blk_plan(const qbk_attn_shape *s) {
    BlkPlan P{};
    BlkArgs &a = P.a;
    a.B = s->batch;
    a.H = s->n_heads;
    a.Hk = s->n_kv_heads;
    a.S = s->seq_q;
    a.nblk = div_ceil(a.S, BLK);
    a.Sp = a.nblk * BLK;
    const size_t bk = a.B * a.Hk, bh = a.B * a.H;
    a.hpx = bh % 8 == 0 ? (int)(bh / 8) : 0;
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

static void blk_bind(BlkPlan &P, const uint16_t *q, const uint16_t *k, const uint16_t *v, void *ws) {
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
    a.vt = (uint16_t *)(w + P.o_vt);
}

// K mean, K codes and V^T (fp16) of every (kv head, block): three launches
static int run_blk_prepass(BlkPlan &P, hipStream_t st) {
    const BlkArgs &a = P.a;
    hipLaunchKernelGGL(blk_kpart, dim3((unsigned)a.nblk, (unsigned)(a.B * a.Hk)), dim3(64), 0, st, a);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(blk_kvquant, dim3((unsigned)a.nblk, (unsigned)(a.B * a.Hk)), dim3(256), 0, st, a);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

static int run_blk_attn(const BlkPlan &P, hipStream_t st) {
    const BlkArgs &a = P.a;
    const size_t n = div_ceil(a.S, BQ) * a.B * a.H;
    hipLaunchKernelGGL(blk_attn, dim3((unsigned)n), dim3(256), 0, st, a);
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

size_t qbk_sage_decode_workspace_size(const qbk_attn_shape *shape, size_t block_size) {
    if (!shape || block_size == 0 || shape->n_kv_heads == 0) return 0;
    return dec_plan(shape, block_size, shape->seq_kv).ws;
}

int qbk_attention_sage_decode(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, size_t q_len,
                              const float *k, size_t k_len, const float *v, size_t v_len,
                              size_t block_size, float *out, size_t out_len) {
    int rc;
    const size_t lens[4] = {q_len, k_len, v_len, out_len};
    if ((rc = validate_decode(shape, block_size, lens))) return rc;
    if (!q || !k || !v || !out) return fail(QBK_ERR_VALIDATION, "null buffer");
    if ((rc = bind(ctx))) return rc;
    CallStream cs;
    if ((rc = cs.create())) return rc;
    DevBuf dq, dk, dvb, dout, dws;
    if ((rc = dq.alloc(q_len * 4)) || (rc = dk.alloc(k_len * 4)) || (rc = dvb.alloc(v_len * 4)) ||
        (rc = dout.alloc(out_len * 4)) || (rc = dws.alloc(dec_plan(shape, block_size, shape->seq_kv).ws)))
        return rc;
    QBK_HIP(hipMemcpyAsync(dq.p, q, q_len * 4, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dk.p, k, k_len * 4, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dvb.p, v, v_len * 4, hipMemcpyHostToDevice, cs.s));
    if ((rc = run_decode(shape, (const float *)dq.p, (const float *)dk.p, (const float *)dvb.p, block_size,
                         (float *)dout.p, dws.p, shape->seq_kv, 0, cs.s)))
        return rc;
    QBK_HIP(hipMemcpyAsync(out, dout.p, out_len * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_attention_sage_decode_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, const float *k,
                                  const float *v, size_t block_size, float *out, void *workspace,
                                  size_t workspace_size, void *stream) {
    int rc;
    if ((rc = validate_decode(shape, block_size, nullptr))) return rc;
    if ((rc = bind(ctx))) return rc;
    const size_t need = dec_plan(shape, block_size, shape->seq_kv).ws;
    if (workspace_size < need)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs", workspace_size, need));
    return run_decode(shape, q, k, v, block_size, out, workspace, shape->seq_kv, 0, (hipStream_t)stream);
}

int qbk_attention_sage_decode_step_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q,
                                       const float *k, const float *v, size_t block_size, float *out,
                                       void *state, size_t state_size, size_t capacity, size_t cached_tokens,
                                       void *stream) {
    return sage_decode_step_sink(ctx, shape, q, k, v, block_size, out, state, state_size, capacity,
                                 cached_tokens, nullptr, stream);
}

}  // extern "C"

int qbk::sage_decode_step_sink(qbk_ctx *ctx, const qbk_attn_shape *shape, const float *q, const float *k,
                               const float *v, size_t block_size, float *out, void *state, size_t state_size,
                               size_t capacity, size_t cached_tokens, const DecOpSink *sink, void *stream,
                               const DecRope *rope) {
    int rc;
    if ((rc = validate_decode(shape, block_size, nullptr))) return rc;
    if (shape->seq_kv > capacity)
        return fail(QBK_ERR_VALIDATION, fmt("the cache holds %zu tokens, beyond the state's capacity of %zu",
                                            shape->seq_kv, capacity));
    if (cached_tokens > shape->seq_kv)
        return fail(QBK_ERR_VALIDATION,
                    fmt("cached_tokens (%zu) exceeds the %zu tokens of the cache; a shorter cache "
                        "starts again from cached_tokens = 0",
                        cached_tokens, shape->seq_kv));
    const size_t need = dec_plan(shape, block_size, capacity).ws;
    if (state_size < need)
        return fail(QBK_ERR_VALIDATION, fmt("decode state of %zu bytes is smaller than the %zu a capacity of "
                                            "%zu tokens needs",
                                            state_size, need, capacity));
    if (!q || !k || !v || !out || !state) return fail(QBK_ERR_VALIDATION, "null buffer");
    if ((rc = bind(ctx))) return rc;
    if (sink && (shape->val_dim % 128 != 0 || !sink->s2 || !sink->op || !sink->sc))
        return fail(QBK_ERR_VALIDATION, "an operand sink needs val_dim a multiple of 128 and its three buffers");
    return run_decode(shape, q, k, v, block_size, out, state, capacity, cached_tokens, (hipStream_t)stream, sink,
                      rope);
}

extern "C" {

size_t qbk_sage_blk_workspace_size(const qbk_attn_shape *shape) {
    if (!shape) return 0;
    return blk_plan(shape).ws;
}

int qbk_attention_sage_blk_dev(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q,
                               const uint16_t *k, const uint16_t *v, int causal, uint16_t *out,
                               void *workspace, size_t workspace_size, void *stream) {
    return sage_blk_run(ctx, shape, q, k, v, causal, out, false, workspace, workspace_size, stream);
}
}  // extern "C"

namespace qbk {
int sage_blk_run(qbk_ctx *ctx, const qbk_attn_shape *shape, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                 int causal, uint16_t *out, bool out_rows, void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if ((rc = validate_blk(shape))) return rc;
    if ((rc = bind(ctx))) return rc;
    BlkPlan P = blk_plan(shape);
    if (workspace_size < P.ws)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs",
                        workspace_size, P.ws));
    hipStream_t st = (hipStream_t)stream;
    blk_bind(P, q, k, v, workspace);
    if ((rc = run_blk_prepass(P, st))) return rc;
    P.a.out = out;
    P.a.out_rows = out_rows ? 1 : 0;
    P.a.causal = causal ? 1 : 0;
    return run_blk_attn(P, st);
}
}  // namespace qbk

extern "C" {

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
    blk_bind(P, q, k, v, ws);
    rc = run_blk_prepass(P, st);
    if (!rc) {
        // Q codes come from the attention kernel's own prologue, run in its
        // quantize-only mode
        P.a.qhat_out = qhat;
        P.a.qscale_out = qscale;
        rc = run_blk_attn(P, st);
    }
    if (!rc) {
        const BlkArgs &a = P.a;
        const size_t n = a.B * a.Hk * a.S * HD;
        hipLaunchKernelGGL(blk_export, dim3((unsigned)div_ceil(n, 256)), dim3(256), 0, st, a, khat, vh);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = fail(QBK_ERR_DEVICE, fmt("blk_export: %s", hipGetErrorString(e)));
    }
    if (!rc) {
        const BlkArgs &a = P.a;
        hipError_t e = hipMemcpyAsync(kscale, a.kscale, a.B * a.Hk * a.nblk * 4, hipMemcpyDeviceToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(kmean, a.kmean, a.B * a.Hk * HD * 4, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) rc = fail(QBK_ERR_DEVICE, fmt("hipMemcpyAsync: %s", hipGetErrorString(e)));
    }
    QBK_HIP(hipFreeAsync(ws, st));
    return rc;
}

}  // extern "C"
