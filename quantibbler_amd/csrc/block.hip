// block.hip -- one decoder block of the server's transformer at one position.
//
// engine/mod.rs:878-945 (Engine::transformer, the body of its block loop)
// at bf16 serving with the sage decode attention (engine/mod.rs:984-1030):
//
//   x  = bf16(rmsnorm(bf16(h)) * w_in)                 (:837-852, :1154-1166)
//   q, k, v = apply_bf16(x)                             (:901-906)
//   q, k per-head RMSNorm when the block has q/k norms  (:907-910, :854-876)
//   q, k rotated by RoPE at position pos                (:911-912, :1169-1187)
//   k, v appended to the block's cache                  (:913)
//   a  = attention of q over the cache's pos + 1 rows   (:918)
//   h1 = apply_bf16(a; o) + h                           (:919-923)
//   x2 = bf16(rmsnorm(bf16(h1)) * w_post)               (:926)
//   g, u = apply_bf16(x2; gate), apply_bf16(x2; up)     (:928-929)
//   h' = apply_bf16(g u / (1 + exp(-g)); down) + h1     (:930-942)
//
// The projections are the device factor linears (q/k/v as one layer set,
// gate/up as another), the attention is the decode step on the block's kept
// state (bit-identical to the reference's padded call), RoPE's angles come
// from a table the host builds with the reference's f64 formula, and the
// norms, SwiGLU and residual adds are small kernels here.  Two of those
// differ from the reference's sequence in rounding, not in formula: the
// norm's sum of squares is a tree (the reference's is one 4096-long chain)
// and exp is the device's.  The block is checked against the oracle's
// restatement to a stated tolerance; its parts that are bit-exact stay so.
// The per-head q/k norms (Qwen-style blocks) are optional.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "factor_internal.h"
#include "q4_operand.h"

#pragma clang fp contract(off)

struct qbk_block {
    int device;
    size_t d, H, Hk, hd, ffn, cap, block;
    float eps;
    const qbk_factor *lay[7];  // q, k, v, o, gate, up, down
    const qbk_factor *o, *down;
    qbk_factor_set *qkv, *gu;
    float *w_in, *w_post;     // d each
    float *ones_ffn;          // ffn ones: the down projection's s2 once the prefill's SwiGLU has applied it
    float *w_q, *w_k;         // head_dim each, or null (no per-head q/k norms)
    float2 *rope;             // [cap][hd / 2] (cos, sin) in f32, from f64
    float *kc, *vc;           // [nseq][cap][Hk * hd] the block's KV caches
    void *state;              // [nseq] the attention's kept decode states
    size_t state_bytes;
    size_t nseq;              // independent sequences: caches and states, sequence s at offset s
    std::vector<size_t> tokens;  // per sequence: cache rows the attention state's codes cover
    std::vector<size_t> filled;  // per sequence: cache rows holding its keys and values
    int face;                    // QBK_ATTN_SAGE (the sage decode attention) or QBK_ATTN_EXACT
    int serving;                 // QBK_BF16, or QBK_F32 (apply's f64 products, f32 norms)
    float *xf;                   // fp32 serving: the normalised row, f32 [d] (null until set)
    double *f64s;                // fp32 serving: the f64 products' scratch
    // per-call buffers
    uint16_t *xcat;           // bf16 [3 d] (q, k, v inputs), then [2 d] (gate, up)
    float *ycat;              // f32 [(H + 2 Hk) hd], then [2 ffn]
    float *qrot, *attn, *oout, *h1, *hid, *dout;
    void *ws;
    size_t ws_bytes;
    std::vector<void *> allocs;
};

namespace qbk {

#define BLKD_NORM_THREADS 1024

__device__ __forceinline__ uint16_t blkd_bf16(float x) {  // RNE (finite x)
    const uint32_t u = __float_as_uint(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// hsum = a (+ r when r); optionally stored to hout; x = bf16 of the
// RMS-normalised bf16(hsum) times w, written nrep times, one copy a d
__global__ void __launch_bounds__(BLKD_NORM_THREADS) blkd_norm(const float *a, const float *r, float *hout,
                                                              const float *w, float eps, uint16_t *x, int nrep,
                                                              int d) {
    __shared__ float red[BLKD_NORM_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.0f;
    for (int i = tid; i < d; i += BLKD_NORM_THREADS) {
        float v = a[i];
        if (r) v = v + r[i];
        if (hout) hout[i] = v;
        const float b = __uint_as_float((uint32_t)blkd_bf16(v) << 16);
        ss += b * b;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < BLKD_NORM_THREADS / 64; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    for (int i = tid; i < d; i += BLKD_NORM_THREADS) {
        float v = a[i];
        if (r) v = v + r[i];
        const float b = __uint_as_float((uint32_t)blkd_bf16(v) << 16);
        const uint16_t o = blkd_bf16(b * inv * w[i]);
        for (int k = 0; k < nrep; k++) x[k * d + i] = o;
    }
}

// blkd_norm at fp32 serving (norm_apply's Fp32 arm, engine/mod.rs:837-852):
// x = RMS-normalised hsum times w in f32, no bf16 roundings; x f32 [d].
__global__ void __launch_bounds__(BLKD_NORM_THREADS) blkd_norm_f32(const float *a, const float *r, float *hout,
                                                                  const float *w, float eps, float *x, int d) {
    __shared__ float red[BLKD_NORM_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.0f;
    for (int i = tid; i < d; i += BLKD_NORM_THREADS) {
        float v = a[i];
        if (r) v = v + r[i];
        if (hout) hout[i] = v;
        ss += v * v;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < BLKD_NORM_THREADS / 64; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    for (int i = tid; i < d; i += BLKD_NORM_THREADS) {
        float v = a[i];
        if (r) v = v + r[i];
        x[i] = v * inv * w[i];
    }
}

// Per-head RMSNorm (optional) and RoPE of q and k at position pos: one wave
// per head, q heads first, then k heads (which also copy their v head to
// the cache).  qkv = [q (H hd) | k (Hk hd) | v (Hk hd)] as the projections
// wrote them; q goes to qrot, k and v to cache row pos.  The norm is
// norm_apply at bf16 serving over one head (engine/mod.rs:854-876): the
// head's values rounded to bf16, their mean square (a tree here), then
// bf16(v * inv * w).  RoPE pairs (i, i + hd/2) (engine/mod.rs:1169-1187).
template <bool F32 = false>
__global__ void __launch_bounds__(64) blkd_qk_rope(const float *qkv, const float2 *rope, size_t pos,
                                                   const uint32_t *pos_dev, size_t cap, const float *wq,
                                                   const float *wk, float eps, float *qrot, float *kc, float *vc,
                                                   int H, int Hk, int hd) {
    const int head = blockIdx.x, lane = threadIdx.x, half = hd / 2;
    if (pos_dev) {
        pos = *(const __attribute__((address_space(4))) uint32_t *)pos_dev;
        if (pos >= cap) return;  // past the cache: nothing is written
    }
    const bool is_q = head < H;
    const int hh = is_q ? head : head - H;
    const float *src = is_q ? qkv + (size_t)hh * hd : qkv + (size_t)H * hd + (size_t)hh * hd;
    float *dst = is_q ? qrot + (size_t)hh * hd : kc + pos * (size_t)Hk * hd + (size_t)hh * hd;
    auto put = [&](int j, float v) { dst[j] = v; };
    rope_head<decltype(put), F32>(src, is_q ? wq : wk, eps, rope + pos * (size_t)half, hd, lane, put);
    if (!is_q) {
        const float *v = qkv + (size_t)(H + Hk) * hd + (size_t)hh * hd;
        float *vr = vc + pos * (size_t)Hk * hd + (size_t)hh * hd;
        for (int j = lane; j < hd; j += 64) vr[j] = v[j];
    }
}

// hidden = g u / (1 + exp(-g)); gu = [g (ffn) | u (ffn)]
__global__ void blkd_swiglu(const float *gu, float *hid, int ffn) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < ffn) {
        const float g = gu[i], u = gu[ffn + i];
        hid[i] = g * u / (1.0f + expf(0.0f - g));
    }
}

__global__ void blkd_add(const float *a, const float *b, float *out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// blkd_norm writing, in place of x, the stage-1 operand of the layer set
// that x feeds (a workgroup per token, ncol = 2 x the batch) (nrep layers each reading x: every din == d, d a multiple
// of 128; q4_operand.h's flat runs over nrep copies of x, the bytes
// q4_prep_flat_kernel writes from them).  The row, the residual, w and the
// first runs' s2 are loaded up front (one memory round trip before the
// reduction), the sums run in blkd_norm's order, x goes through LDS.
#define BLKD_OP_PER 8  // row elements a thread holds: d <= 8192
__global__ void __launch_bounds__(BLKD_NORM_THREADS) blkd_norm_op(const float *a, const float *r, float *hout,
                                                                 const float *w, float eps, int d, int nrep,
                                                                 const float *s2cat, uint8_t *op, uint8_t *sc,
                                                                 int ncol) {
    __shared__ float red[BLKD_NORM_THREADS / 64];
    __shared__ __attribute__((aligned(16))) uint16_t xs[BLKD_NORM_THREADS * BLKD_OP_PER];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // token tok = blockIdx.x of a batch: its row, and its columns 2 tok, 2 tok + 1 of the operand's ncol
    const int tok = (int)blockIdx.x;
    a += (size_t)tok * d;
    if (r) r += (size_t)tok * d;
    if (hout) hout += (size_t)tok * d;
    const uint32_t n_runs = (uint32_t)(nrep * d / 16), rpl = (uint32_t)(d / 16);
    // a run past the end shadows one of the last slice (n_runs is a multiple
    // of 8, so its shuffle partner at lane distance 2 does too)
    auto run_of = [&](uint32_t tt) { return tt < n_runs ? tt : n_runs - 8 + (tt & 7); };
    u32x4_t sr[4];
    {
        const u32x4_t *ss = (const u32x4_t *)(s2cat + (size_t)run_of((uint32_t)tid) * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) sr[q] = ss[q];
    }
    float va[BLKD_OP_PER], wv[BLKD_OP_PER];
#pragma unroll
    for (int k = 0; k < BLKD_OP_PER; k++) {
        const int i = tid + k * BLKD_NORM_THREADS;
        va[k] = 0.0f;
        wv[k] = 0.0f;
        if (i < d) {
            float v = a[i];
            if (r) v = v + r[i];
            va[k] = v;
            wv[k] = w[i];
        }
    }
    float ss2 = 0.0f;
#pragma unroll
    for (int k = 0; k < BLKD_OP_PER; k++) {
        const int i = tid + k * BLKD_NORM_THREADS;
        if (i < d) {
            if (hout) hout[i] = va[k];
            const float b = __uint_as_float((uint32_t)blkd_bf16(va[k]) << 16);
            ss2 += b * b;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss2 += __shfl_xor(ss2, o, 64);
    if (lane == 0) red[wave] = ss2;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < BLKD_NORM_THREADS / 64; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
#pragma unroll
    for (int k = 0; k < BLKD_OP_PER; k++) {
        const int i = tid + k * BLKD_NORM_THREADS;
        if (i < d) {
            const float b = __uint_as_float((uint32_t)blkd_bf16(va[k]) << 16);
            xs[i] = blkd_bf16(b * inv * wv[k]);
        }
    }
    __syncthreads();
    for (uint32_t t0 = 0; t0 < n_runs; t0 += BLKD_NORM_THREADS) {  // uniform: every lane shuffles
        const uint32_t tt = t0 + (uint32_t)tid, t = run_of(tt);
        if (t0 > 0) {
            const u32x4_t *ss = (const u32x4_t *)(s2cat + (size_t)t * 16);
#pragma unroll
            for (int q = 0; q < 4; q++) sr[q] = ss[q];
        }
        const uint32_t e0 = (t % rpl) * 16;
        const u32x4_t xr[2] = {*(const u32x4_t *)(xs + e0), *(const u32x4_t *)(xs + e0 + 8)};
        float z[16];
        q4_run_z(xr, sr, z);
        uint32_t hw[4], lw[4];
        int e_hi, e_lo;
        q4_run_operand(z, hw, lw, e_hi, e_lo);
        if (tt >= n_runs) continue;
        const int rr = (int)(t & 7);
        const size_t slot = q4_run_slot(t >> 3, rr, ncol, tok), byte = 16 * (rr & 1);
        *(uint4 *)(op + slot * 32 + byte) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *(uint4 *)(op + (slot + 1) * 32 + byte) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        if ((rr & 2) == 0)
            *(uint16_t *)(sc + q4_run_scale(t >> 3, rr, ncol, tok)) = (uint16_t)((e_hi + 127) | ((e_lo + 127) << 8));
    }
}

// blkd_swiglu written as the stage-1 operand of the layer it feeds (din =
// ffn, a multiple of 128): a thread per run of 16, hid as blkd_swiglu forms
// it, z = bf16(s2 hid) as q4_prep_kernel's f32 path.  Token tok =
// blockIdx.y of a batch: rows gp + tok ffn, up + tok ffn, columns 2 tok,
// 2 tok + 1 of the operand's ncol.
__global__ void __launch_bounds__(256) blkd_swiglu_op(const float *gp, const float *up, int ffn, const float *s2,
                                                      uint8_t *op, uint8_t *sc, int ncol) {
    const uint32_t n_runs = (uint32_t)ffn / 16;
    const uint32_t tt = blockIdx.x * 256 + threadIdx.x;
    const uint32_t t = tt < n_runs ? tt : n_runs - 8 + (tt & 7);
    const int tok = (int)blockIdx.y;
    gp += (size_t)tok * ffn;
    up += (size_t)tok * ffn;
    const size_t k0 = (size_t)t * 16;
    float z[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 g4 = *(const float4 *)(gp + k0 + 4 * q), u4 = *(const float4 *)(up + k0 + 4 * q);
        const float4 s4 = *(const float4 *)(s2 + k0 + 4 * q);
        const float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w},
                    sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float hid = g[e] * u[e] / (1.0f + expf(0.0f - g[e]));
            z[4 * q + e] = bf16_to_f32(f32_to_bf16(sv[e] * hid));
        }
    }
    uint32_t hw[4], lw[4];
    int e_hi, e_lo;
    q4_run_operand(z, hw, lw, e_hi, e_lo);
    if (tt >= n_runs) return;
    const int rr = (int)(t & 7);
    const size_t slot = q4_run_slot(t >> 3, rr, ncol, tok), byte = 16 * (rr & 1);
    *(uint4 *)(op + slot * 32 + byte) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(op + (slot + 1) * 32 + byte) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if ((rr & 2) == 0)
        *(uint16_t *)(sc + q4_run_scale(t >> 3, rr, ncol, tok)) = (uint16_t)((e_hi + 127) | ((e_lo + 127) << 8));
}

// ---- prefill (n tokens at positions 0 .. n - 1) ---------------------------

// Per row of d: hsum = a (+ r), optionally stored to hout; x = bf16 of the
// RMS-normalised bf16(hsum) times w (the decode's blkd_norm, a row per
// workgroup), written nrep times: copy k of the n rows at x + k n d (the
// input of a layer set whose layers share x).  Rows up to NT NE elements
// are read once, all their loads issued before any store.
template <int NT, int NE = 8192 / NT>
__global__ void __launch_bounds__(NT) blkp_norm(const float *__restrict__ a, const float *__restrict__ r,
                                                float *__restrict__ hout, const float *__restrict__ w, float eps,
                                                uint16_t *__restrict__ x, int d, int nrep) {
    __shared__ float red[NT / 64];
    const size_t off = (size_t)blockIdx.x * d;
    const int tid = threadIdx.x;
    if (d > NT * NE) {  // a longer row: two passes over it
        float ss = 0.0f;
        for (int i = tid; i < d; i += NT) {
            float v = a[off + i];
            if (r) v = v + r[off + i];
            if (hout) hout[off + i] = v;
            const float b = __uint_as_float((uint32_t)blkd_bf16(v) << 16);
            ss += b * b;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < NT / 64; i++) tot += red[i];
        const float inv = 1.0f / sqrtf(tot / (float)d + eps);
        for (int i = tid; i < d; i += NT) {
            float v = a[off + i];
            if (r) v = v + r[off + i];
            const float b = __uint_as_float((uint32_t)blkd_bf16(v) << 16);
            const uint16_t o = blkd_bf16(b * inv * w[i]);
            for (int c = 0; c < nrep; c++) x[c * (size_t)gridDim.x * d + off + i] = o;
        }
        return;
    }
    // the row once: every load first, then the sums, then the stores
    float va[NE], wa[NE];
#pragma unroll
    for (int k = 0; k < NE; k++) {
        const int i = tid + k * NT;
        va[k] = i < d ? a[off + i] : 0.0f;
        wa[k] = i < d ? w[i] : 0.0f;
    }
    if (r) {
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int i = tid + k * NT;
            if (i < d) va[k] = va[k] + r[off + i];
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NE; k++) {
        const int i = tid + k * NT;
        if (i < d) {
            const float b = __uint_as_float((uint32_t)blkd_bf16(va[k]) << 16);
            ss += b * b;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    if (hout) {
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int i = tid + k * NT;
            if (i < d) hout[off + i] = va[k];
        }
    }
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NT / 64; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
#pragma unroll
    for (int k = 0; k < NE; k++) {
        const int i = tid + k * NT;
        if (i < d) {
            const float b = __uint_as_float((uint32_t)blkd_bf16(va[k]) << 16);
            const uint16_t o = blkd_bf16(b * inv * wa[k]);
            for (int c = 0; c < nrep; c++) x[c * (size_t)gridDim.x * d + off + i] = o;  // copy c: [n][d] at c n d
        }
    }
}

// blkp_norm over n rows: 1024 threads a row for a few rows (a batched decode
// step: the row's latency is the step's), 256 for many (a prefill).
static void blkp_norm_launch(size_t n, const float *a, const float *r, float *hout, const float *w, float eps,
                             uint16_t *x, int d, int nrep, hipStream_t s) {
    if (n <= 64)
        hipLaunchKernelGGL(blkp_norm<BLKD_NORM_THREADS>, dim3((unsigned)n), dim3(BLKD_NORM_THREADS), 0, s, a, r,
                           hout, w, eps, x, d, nrep);
    else
        hipLaunchKernelGGL(blkp_norm<256>, dim3((unsigned)n), dim3(256), 0, s, a, r, hout, w, eps, x, d, nrep);
}

// Row t's q, k, v (token-major f32, as the projections wrote them): per-head
// q/k norm (optional) and RoPE at position t, as blkd_qk_rope; k and v also
// to cache row t.  The attention operands go out head-major in bf16:
// qb [H][n][hd], kb / vb [Hk][n][hd].  Grid (ceil((H + Hk) / 4), n), a wave
// per head (one-wave workgroups, 40 a token at config 5, measured 30 us a
// 2048-token block: dispatch-bound).
__global__ void __launch_bounds__(256) blkp_qk_rope(const float *q, const float *k, const float *v, const float2 *rope,
                                                    const float *wq, const float *wk, float eps, float *kc, float *vc,
                                                    uint16_t *qb, uint16_t *kb, uint16_t *vb, int H, int Hk, int hd,
                                                    int n) {
    const int head = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), t = blockIdx.y, lane = threadIdx.x & 63,
              half = hd / 2;
    if (head >= H + Hk) return;  // a wave of the last workgroup past the heads (no barrier follows)
    const bool is_q = head < H;
    const int hh = is_q ? head : head - H;
    const float *src = is_q ? q + ((size_t)t * H + hh) * hd : k + ((size_t)t * Hk + hh) * hd;
    const float *w = is_q ? wq : wk;
    float inv = 1.0f;
    if (w) {
        float ss = 0.0f;
        for (int j = lane; j < hd; j += 64) {
            const float b = bf16_to_f32(f32_to_bf16(src[j]));
            ss += b * b;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        inv = 1.0f / sqrtf(ss / (float)hd + eps);
    }
    const float2 *cs = rope + (size_t)t * half;
    uint16_t *ob = is_q ? qb + ((size_t)hh * n + t) * hd : kb + ((size_t)hh * n + t) * hd;
    float *crow = kc + ((size_t)t * Hk + hh) * hd;
    for (int j = lane; j < half; j += 64) {
        float a = src[j], b = src[j + half];
        if (w) {
            a = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(a)) * inv * w[j]));
            b = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(b)) * inv * w[j + half]));
        }
        const float2 c = cs[j];
        const float ra = a * c.x - b * c.y, rb = b * c.x + a * c.y;
        ob[j] = f32_to_bf16(ra);
        ob[j + half] = f32_to_bf16(rb);
        if (!is_q) {
            crow[j] = ra;
            crow[j + half] = rb;
        }
    }
    if (!is_q) {
        const float *vs = v + ((size_t)t * Hk + hh) * hd;
        float *vr = vc + ((size_t)t * Hk + hh) * hd;
        uint16_t *vo = vb + ((size_t)hh * n + t) * hd;
        for (int j = lane; j < hd; j += 64) {
            vr[j] = vs[j];
            vo[j] = f32_to_bf16(vs[j]);
        }
    }
}

// hidden = g u / (1 + exp(-g)), elementwise over n rows of ffn
__global__ void blkp_swiglu(const float *g, const float *u, float *hid, size_t count) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) {
        const float gv = g[i], uv = u[i];
        hid[i] = gv * uv / (1.0f + expf(0.0f - gv));
    }
}

// blkp_swiglu followed by the down projection's z = bf16(s2 hid) (the
// GEMM's f32-x conversion, the same f32 product and rounding), written as
// bf16: the GEMM then reads it at s2 = 1, where bf16(1 * z) = z.  Half the
// bytes of the f32 hidden row on both sides.  Four elements a thread (ffn a
// multiple of 4).
__global__ void blkp_swiglu_z(const float *g, const float *u, const float *s2, uint16_t *z, size_t count,
                              uint32_t ffn) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= count) return;
    const float4 gv = *(const float4 *)(g + i), uv = *(const float4 *)(u + i);
    const float4 sv = *(const float4 *)(s2 + i % ffn);
    const float ga[4] = {gv.x, gv.y, gv.z, gv.w}, ua[4] = {uv.x, uv.y, uv.z, uv.w}, sa[4] = {sv.x, sv.y, sv.z, sv.w};
    uint16_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float hid = ga[e] * ua[e] / (1.0f + expf(0.0f - ga[e]));
        o[e] = f32_to_bf16(sa[e] * hid);
    }
    *(uint2 *)(z + i) = make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
}

__global__ void blkp_add(const float *a, const float *b, float *out, size_t count) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = a[i] + b[i];
}

// A projection of n rows: the decode GEMV up to its batch limit, the GEMM
// beyond; y f32.
static size_t blkp_proj_ws(const qbk_factor *L, size_t n) {
    return n <= Q4_MAXB ? q4_workspace(L, n) : gemm_workspace(L, n);
}
static int blkp_proj(const qbk_factor *L, size_t n, const void *x, bool xf32, float *y, void *ws, hipStream_t s) {
    return n <= Q4_MAXB ? q4_run(L, n, x, xf32, y, false, ws, s) : gemm_run(L, x, xf32, n, y, false, ws, s);
}

// Prefill workspace regions (256-byte aligned), for n rows.
struct BlkpPlan {
    size_t o_x, o_q, o_k, o_v, o_qb, o_kb, o_vb, o_sage, o_arow, o_oo, o_h1, o_g, o_u, o_z, o_gemm, bytes;
    size_t sage_bytes, gemm_bytes;
};

static BlkpPlan blkp_plan(const qbk_block *B, const qbk_factor *const L[7], size_t n) {
    BlkpPlan p{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += round_up(bytes ? bytes : 4, 256);
        return o;
    };
    const size_t d = B->d, qd = B->H * B->hd, kd = B->Hk * B->hd;
    p.o_x = take(n * (d > qd ? d : qd) * 2);
    p.o_q = take(n * qd * 4);
    p.o_k = take(n * kd * 4);
    p.o_v = take(n * kd * 4);
    p.o_qb = take(n * qd * 2);
    p.o_kb = take(n * kd * 2);
    p.o_vb = take(n * kd * 2);
    const qbk_attn_shape sh{1, B->H, B->Hk, n, n, B->hd, B->hd};
    p.sage_bytes = qbk_sage_blk_workspace_size(&sh);
    p.o_sage = take(p.sage_bytes);
    p.o_arow = take(n * qd * 2);
    p.o_oo = take(n * d * 4);
    p.o_h1 = take(n * d * 4);
    p.o_g = take(n * B->ffn * 4);
    p.o_u = take(n * B->ffn * 4);
    p.o_z = take(n * B->ffn * 2);
    size_t g = 0;
    for (int i = 0; i < 7; i++) {
        const size_t w = blkp_proj_ws(L[i], n);
        g = w > g ? w : g;
    }
    p.gemm_bytes = g;
    p.o_gemm = take(g);
    p.bytes = off;
    return p;
}

// ---- batched decode (one position of each of n sequences) -----------------

#define BLKB_MAXSEQ QBK_DEC_MAXSEQ
struct BlkbPos {
    uint32_t p[BLKB_MAXSEQ];
};

// Row t (sequence t): per-head q/k norm and RoPE at pos.p[t] as blkd_qk_rope;
// q to qr [n][H hd], k and v to row pos.p[t] of sequence t's cache.
__global__ void __launch_bounds__(64) blkb_qk_rope(const float *q, const float *k, const float *v, const float2 *rope,
                                                   BlkbPos pos, const uint32_t *pos_dev, size_t cap, const float *wq,
                                                   const float *wk, float eps, float *kc, float *vc, size_t kvs,
                                                   float *qr, int H, int Hk, int hd) {
    const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x, half = hd / 2;
    const size_t p = pos_dev ? ((const __attribute__((address_space(4))) uint32_t *)pos_dev)[t] : pos.p[t];
    if (p >= cap) return;  // a device position past the cache: nothing is written
    const bool is_q = head < H;
    const int hh = is_q ? head : head - H;
    const float *src = is_q ? q + ((size_t)t * H + hh) * hd : k + ((size_t)t * Hk + hh) * hd;
    float *dst = is_q ? qr + ((size_t)t * H + hh) * hd : kc + t * kvs + (p * Hk + hh) * hd;
    rope_head(src, is_q ? wq : wk, eps, rope + p * (size_t)half, hd, lane, [&](int j, float x) { dst[j] = x; });
    if (!is_q) {
        const float *vs = v + ((size_t)t * Hk + hh) * hd;
        float *vr = vc + t * kvs + (p * Hk + hh) * hd;
        for (int j = lane; j < hd; j += 64) vr[j] = vs[j];
    }
}

// Up to Q4_MAXB sequences the projections run on the fp4 decode GEMV, q/k/v
// and gate/up as the block's layer sets (one launch per stage for each set,
// x written once per layer of the set); beyond, layer by layer on the
// prefill GEMM, which is the faster of the two there (at config 3's q shape:
// 20-21 us a layer at batch 9-32 against the GEMV's 19-40 us).
struct BlkbPlan {
    bool sets;
    size_t o_x, o_qkv, o_qr, o_at, o_oo, o_h1, o_gu, o_gemm, bytes;
};

static BlkbPlan blkb_plan(const qbk_block *B, size_t n) {
    BlkbPlan p{};
    p.sets = n <= Q4_MAXB;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += round_up(bytes ? bytes : 4, 256);
        return o;
    };
    const size_t d = B->d, qd = B->H * B->hd, kd = B->Hk * B->hd;
    p.o_x = take(3 * n * d * 2);
    p.o_qkv = take(n * (qd + 2 * kd) * 4);  // q [n][qd], then k and v [n][kd]
    p.o_qr = take(n * qd * 4);
    p.o_at = take(n * qd * 4);
    p.o_oo = take(n * d * 4);
    p.o_h1 = take(n * d * 4);
    p.o_gu = take(2 * n * B->ffn * 4);      // g [n][ffn], then u
    size_t g = 0;
    if (p.sets) {
        const size_t w[4] = {q4_set_workspace_batch(B->qkv, n), q4_set_workspace_batch(B->gu, n),
                             q4_workspace(B->o, n), q4_workspace(B->down, n)};
        for (int i = 0; i < 4; i++) g = w[i] > g ? w[i] : g;
    } else {
        for (int i = 0; i < 7; i++) {
            const size_t w = blkp_proj_ws(B->lay[i], n);
            g = w > g ? w : g;
        }
        for (const qbk_factor_set *S : {B->qkv, B->gu})
            if (q4_set_gemm_fits(S, n)) {
                const size_t w = q4_set_gemm_workspace(S, n);
                g = w > g ? w : g;
            }
    }
    p.o_gemm = take(g);
    p.bytes = off;
    return p;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

void qbk_block_destroy(qbk_block *B) {
    if (!B) return;
    (void)hipSetDevice(B->device);
    (void)hipDeviceSynchronize();
    if (B->qkv) qbk_factor_set_destroy(B->qkv);
    if (B->gu) qbk_factor_set_destroy(B->gu);
    for (void *p : B->allocs) (void)hipFree(p);
    delete B;
}

int qbk_block_create_seqs(qbk_ctx *ctx, const qbk_factor *const *layers, const float *input_norm,
                          size_t input_norm_len, const float *post_norm, size_t post_norm_len, const float *q_norm,
                          const float *k_norm, size_t qk_norm_len, size_t n_heads, size_t n_kv_heads,
                          size_t head_dim, double rope_theta, double rms_norm_eps, size_t capacity,
                          size_t block_size, size_t n_seqs, qbk_block **out) {
    int rc;
    if (n_seqs == 0 || n_seqs > BLKB_MAXSEQ)
        return fail(QBK_ERR_VALIDATION, fmt("decoder block holds 1 to %d sequences, got %zu", BLKB_MAXSEQ, n_seqs));
    if (!layers || !input_norm || !post_norm || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    if (!q_norm != !k_norm)
        return fail(QBK_ERR_VALIDATION, "decoder block: q_norm and k_norm come together or not at all");
    for (int i = 0; i < 7; i++)
        if (!layers[i]) return fail(QBK_ERR_VALIDATION, "null layer");
    size_t dims[7][3];
    for (int i = 0; i < 7; i++) qbk_factor_dims(layers[i], &dims[i][0], &dims[i][1], &dims[i][2]);
    const size_t d = dims[0][1], H = n_heads, Hk = n_kv_heads, hd = head_dim, ffn = dims[4][0];
    if (H == 0 || Hk == 0 || hd == 0 || hd % 2 || H % Hk)
        return fail(QBK_ERR_VALIDATION, "decoder block needs n_kv_heads dividing n_heads and an even head_dim");
    // q (H hd x d), k, v (Hk hd x d), o (d x H hd), gate, up (ffn x d), down (d x ffn)
    const size_t want[7][2] = {{H * hd, d}, {Hk * hd, d}, {Hk * hd, d}, {d, H * hd}, {ffn, d}, {ffn, d}, {d, ffn}};
    static const char *names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
    for (int i = 0; i < 7; i++)
        if (dims[i][0] != want[i][0] || dims[i][1] != want[i][1])
            return fail(QBK_ERR_VALIDATION, fmt("decoder block: %s is %zux%zu, expected %zux%zu", names[i],
                                                dims[i][0], dims[i][1], want[i][0], want[i][1]));
    if (input_norm_len != d || post_norm_len != d)
        return fail(QBK_ERR_VALIDATION, fmt("decoder block: norm weights of %zu and %zu floats; d_model is %zu",
                                            input_norm_len, post_norm_len, d));
    if (q_norm && qk_norm_len != hd)
        return fail(QBK_ERR_VALIDATION,
                    fmt("decoder block: q/k norm weights of %zu floats; head_dim is %zu", qk_norm_len, hd));
    if (capacity == 0 || block_size == 0) return fail(QBK_ERR_VALIDATION, "decoder block needs a capacity and a block size");
    if ((rc = bind(ctx))) return rc;
    qbk_block *B = new qbk_block();
    B->device = ctx->device;
    B->d = d;
    B->H = H;
    B->Hk = Hk;
    B->hd = hd;
    B->ffn = ffn;
    B->cap = capacity;
    B->block = block_size;
    B->eps = (float)rms_norm_eps;
    B->nseq = n_seqs;
    B->face = QBK_ATTN_SAGE;
    B->serving = QBK_BF16;
    B->xf = nullptr;
    B->f64s = nullptr;
    B->tokens.assign(n_seqs, 0);
    B->filled.assign(n_seqs, 0);
    for (int i = 0; i < 7; i++) B->lay[i] = layers[i];
    B->o = layers[3];
    B->down = layers[6];
    auto alloc = [&](void **p, size_t n) -> int {
        hipError_t e = hipMalloc(p, n ? n : 4);
        if (e != hipSuccess) return fail(QBK_ERR_DEVICE, fmt("hipMalloc(%zu): %s", n, hipGetErrorString(e)));
        B->allocs.push_back(*p);
        return QBK_OK;
    };
    const qbk_factor *qkv[3] = {layers[0], layers[1], layers[2]}, *gu[2] = {layers[4], layers[5]};
    qbk_attn_shape sh{1, H, Hk, 1, capacity, hd, hd};
    B->state_bytes = qbk_sage_decode_workspace_size(&sh, block_size);
    const size_t kv = capacity * Hk * hd * 4;
    if ((rc = qbk_factor_set_create(ctx, qkv, 3, &B->qkv)) || (rc = qbk_factor_set_create(ctx, gu, 2, &B->gu)) ||
        (rc = alloc((void **)&B->w_in, d * 4)) || (rc = alloc((void **)&B->w_post, d * 4)) ||
        (q_norm && ((rc = alloc((void **)&B->w_q, hd * 4)) || (rc = alloc((void **)&B->w_k, hd * 4)))) ||
        (rc = alloc((void **)&B->rope, capacity * (hd / 2) * 8)) || (rc = alloc((void **)&B->kc, kv * n_seqs)) ||
        (rc = alloc((void **)&B->vc, kv * n_seqs)) || (rc = alloc(&B->state, B->state_bytes * n_seqs)) ||
        (rc = alloc((void **)&B->xcat, 3 * d * 2)) ||
        (rc = alloc((void **)&B->ycat, ((H + 2 * Hk) * hd > 2 * ffn ? (H + 2 * Hk) * hd : 2 * ffn) * 4)) ||
        (rc = alloc((void **)&B->qrot, H * hd * 4)) || (rc = alloc((void **)&B->attn, H * hd * 4)) ||
        (rc = alloc((void **)&B->oout, d * 4)) || (rc = alloc((void **)&B->h1, d * 4)) ||
        (rc = alloc((void **)&B->hid, ffn * 4)) || (rc = alloc((void **)&B->dout, d * 4)) ||
        (rc = alloc((void **)&B->ones_ffn, ffn * 4))) {
        qbk_block_destroy(B);
        return rc;
    }
    size_t ws = q4_set_workspace(B->qkv);
    const size_t wss[3] = {q4_set_workspace(B->gu), q4_workspace(B->o, 1), q4_workspace(B->down, 1)};
    for (size_t w : wss) ws = w > ws ? w : ws;
    B->ws_bytes = ws;
    if ((rc = alloc(&B->ws, ws))) {
        qbk_block_destroy(B);
        return rc;
    }
    // RoPE angles as rope_rotate forms them (engine/mod.rs:1169-1187): f64
    // inv_freq = theta^(-2i / hd), (sin, cos) of pos * inv_freq, then f32
    std::vector<float2> tab(capacity * (hd / 2));
    for (size_t p = 0; p < capacity; p++)
        for (size_t i = 0; i < hd / 2; i++) {
            const double inv_freq = pow(rope_theta, -(2.0 * (double)i) / (double)hd);
            const double ang = (double)p * inv_freq;
            tab[p * (hd / 2) + i] = make_float2((float)cos(ang), (float)sin(ang));
        }
    hipError_t e = hipMemcpy(B->rope, tab.data(), tab.size() * 8, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(B->w_in, input_norm, d * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(B->w_post, post_norm, d * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        const std::vector<float> ones(ffn, 1.0f);
        e = hipMemcpy(B->ones_ffn, ones.data(), ffn * 4, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess && q_norm) e = hipMemcpy(B->w_q, q_norm, hd * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess && k_norm) e = hipMemcpy(B->w_k, k_norm, hd * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        qbk_block_destroy(B);
        return fail(QBK_ERR_DEVICE, fmt("hipMemcpy: %s", hipGetErrorString(e)));
    }
    *out = B;
    return QBK_OK;
}

int qbk_block_create(qbk_ctx *ctx, const qbk_factor *const *layers, const float *input_norm,
                     size_t input_norm_len, const float *post_norm, size_t post_norm_len, const float *q_norm,
                     const float *k_norm, size_t qk_norm_len, size_t n_heads, size_t n_kv_heads,
                     size_t head_dim, double rope_theta, double rms_norm_eps, size_t capacity,
                     size_t block_size, qbk_block **out) {
    return qbk_block_create_seqs(ctx, layers, input_norm, input_norm_len, post_norm, post_norm_len, q_norm, k_norm,
                                 qk_norm_len, n_heads, n_kv_heads, head_dim, rope_theta, rms_norm_eps, capacity,
                                 block_size, 1, out);
}

int qbk_block_cache(const qbk_block *B, float **k_cache, float **v_cache) {
    if (!B) return fail(QBK_ERR_VALIDATION, "null block");
    if (k_cache) *k_cache = B->kc;
    if (v_cache) *v_cache = B->vc;
    return QBK_OK;
}

}  // extern "C"

static int block_mlp_one(qbk_block *B, float *h, hipStream_t s);

static const char *const kExactFaceOnly =
    "the exact attention face serves one sequence at host positions (qbk_block_decode_dev, "
    "qbk_block_prefill_dev); the batched and device-position steps run the sage face";
static const char *const kF32Only =
    "fp32 serving runs one sequence at host positions (qbk_block_decode_dev, qbk_block_prefill_dev); the "
    "batched and device-position steps serve bf16";

// One position of sequence 0 at fp32 serving (engine/mod.rs:886-941 with
// ServingDtype::Fp32): norms in f32 without bf16 roundings (:837-876), the
// seven projections as apply's f64 products (:393-436), q/k norms and RoPE,
// the cache append, the block's attention face over rows 0 .. pos, SwiGLU,
// the residuals.  A parity face: a few launches a projection.
static int block_decode_f32(qbk_ctx *ctx, qbk_block *B, float *h, size_t pos, hipStream_t s) {
    int rc;
    const int d = (int)B->d, hd = (int)B->hd, H = (int)B->H, Hk = (int)B->Hk, ffn = (int)B->ffn;
    auto proj = [&](int li, const float *x, float *y) {
        return factor_apply_f64_dev(ctx, B->lay[li], x, y, B->f64s, s);
    };
    hipLaunchKernelGGL(blkd_norm_f32, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, h, (const float *)nullptr,
                       (float *)nullptr, B->w_in, B->eps, B->xf, d);
    QBK_HIP(hipGetLastError());
    float *q = B->ycat, *k = q + (size_t)H * hd, *v = k + (size_t)Hk * hd;
    if ((rc = proj(0, B->xf, q)) || (rc = proj(1, B->xf, k)) || (rc = proj(2, B->xf, v))) return rc;
    hipLaunchKernelGGL(blkd_qk_rope<true>, dim3(H + Hk), dim3(64), 0, s, B->ycat, B->rope, pos,
                       (const uint32_t *)nullptr, B->cap, B->w_q, B->w_k, B->eps, B->qrot, B->kc, B->vc, H, Hk, hd);
    QBK_HIP(hipGetLastError());
    if (B->face == QBK_ATTN_EXACT) {
        if ((rc = attention_exact_cache(B->qrot, B->kc, B->vc, B->H, B->Hk, B->hd, pos + 1, B->attn, s))) return rc;
        if (B->tokens[0] > pos) B->tokens[0] = pos;
    } else {
        const qbk_attn_shape sh{1, B->H, B->Hk, 1, pos + 1, B->hd, B->hd};
        const size_t cached = B->tokens[0] <= pos ? B->tokens[0] : 0;
        if ((rc = sage_decode_step_sink(ctx, &sh, B->qrot, B->kc, B->vc, B->block, B->attn, B->state,
                                        B->state_bytes, B->cap, cached, nullptr, s)))
            return rc;
        B->tokens[0] = pos + 1;
    }
    B->filled[0] = pos + 1;
    if ((rc = proj(3, B->attn, B->oout))) return rc;
    hipLaunchKernelGGL(blkd_norm_f32, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, B->oout, (const float *)h, B->h1,
                       B->w_post, B->eps, B->xf, d);
    QBK_HIP(hipGetLastError());
    if ((rc = proj(4, B->xf, B->ycat)) || (rc = proj(5, B->xf, B->ycat + ffn))) return rc;
    hipLaunchKernelGGL(blkd_swiglu, dim3((ffn + 255) / 256), dim3(256), 0, s, B->ycat, B->hid, ffn);
    QBK_HIP(hipGetLastError());
    if ((rc = proj(6, B->hid, B->dout))) return rc;
    hipLaunchKernelGGL(blkd_add, dim3((d + 255) / 256), dim3(256), 0, s, B->dout, B->h1, h, d);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

// The decode of one position of sequence 0: at pos (host), or with pos_dev
// at the position that device word holds when the step runs (the host
// record of cached positions is then left to the caller).
static int block_decode_one(qbk_ctx *ctx, qbk_block *B, float *h, size_t pos, const uint32_t *pos_dev,
                            void *stream) {
    int rc;
    if (!B || !h) return fail(QBK_ERR_VALIDATION, "null argument");
    if (!pos_dev && pos >= B->cap)
        return fail(QBK_ERR_VALIDATION, fmt("position %zu is past the block's cache capacity of %zu", pos, B->cap));
    if (!pos_dev && pos > B->filled[0])
        return fail(QBK_ERR_VALIDATION,
                    fmt("position %zu skips cache rows: the block holds %zu positions", pos, B->filled[0]));
    if ((rc = bind(ctx))) return rc;
    if (B->device != ctx->device) return fail(QBK_ERR_VALIDATION, "block lives on another device than the context");
    const bool exact = B->face == QBK_ATTN_EXACT;
    if (pos_dev && exact) return fail(QBK_ERR_VALIDATION, kExactFaceOnly);
    if (B->serving == QBK_F32) {
        if (pos_dev) return fail(QBK_ERR_VALIDATION, kF32Only);
        return block_decode_f32(ctx, B, h, pos, (hipStream_t)stream);
    }
    const qbk_attn_shape one{1, B->H, B->Hk, 1, B->cap, B->hd, B->hd};
    const size_t kvs = B->cap * B->Hk * B->hd;
    if (pos_dev && !sage_decode_batchable(&one, B->block, B->cap, B->kc, B->vc, kvs))
        return fail(QBK_ERR_VALIDATION, "a device-position step needs the grouped sage decode kernels "
                                        "(head_dim a multiple of 16, groups of up to 16 heads, blocks of up to "
                                        "64 tokens)");
    hipStream_t s = (hipStream_t)stream;
    const int d = (int)B->d, hd = (int)B->hd, H = (int)B->H, Hk = (int)B->Hk, ffn = (int)B->ffn;
    // the norms and SwiGLU write the operand of the projections they feed
    // when those have the flat batch-1 layout (every din a multiple of 128)
    const bool fits = d <= BLKD_NORM_THREADS * BLKD_OP_PER;
    uint8_t *op, *sc;
    const float *s2c;
    // attention sublayer
    if (fits && q4_set_flat_operand(B->qkv, B->ws, &op, &sc, &s2c)) {
        hipLaunchKernelGGL(blkd_norm_op, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, h, (const float *)nullptr,
                           (float *)nullptr, B->w_in, B->eps, d, 3, s2c, op, sc, 2);
        QBK_HIP(hipGetLastError());
        if ((rc = q4_set_run_staged(B->qkv, B->ycat, false, B->ws, s))) return rc;
    } else {
        hipLaunchKernelGGL(blkd_norm, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, h, (const float *)nullptr,
                           (float *)nullptr, B->w_in, B->eps, B->xcat, 3, d);
        QBK_HIP(hipGetLastError());
        if ((rc = q4_set_run(B->qkv, B->xcat, false, B->ycat, false, B->ws, s))) return rc;
    }
    // the q/k norms, RoPE and the cache append run in the attention's
    // pre-pass when the grouped decode kernels serve the shape (one launch
    // fewer), else in a kernel of their own
    const bool fold = !exact && sage_decode_batchable(&one, B->block, B->cap, B->kc, B->vc, kvs);
    const DecRope rp{B->ycat, B->rope, B->w_q, B->w_k, B->eps, H};
    if (!fold) {
        hipLaunchKernelGGL(blkd_qk_rope<false>, dim3(H + Hk), dim3(64), 0, s, B->ycat, B->rope, pos, pos_dev, B->cap,
                           B->w_q, B->w_k, B->eps, B->qrot, B->kc, B->vc, H, Hk, hd);
        QBK_HIP(hipGetLastError());
    }
    // the exact face (engine/mod.rs:1041-1067 gqa_attention_tiled): f32
    // attention of the rotated query over cache rows 0 .. pos, read in place;
    // the o projection from its f32 output
    if (exact) {
        if ((rc = attention_exact_cache(B->qrot, B->kc, B->vc, B->H, B->Hk, B->hd, pos + 1, B->attn, s))) return rc;
        if (B->tokens[0] > pos) B->tokens[0] = pos;  // the sage state covers the rows before pos at most
        B->filled[0] = pos + 1;
        if ((rc = q4_run(B->o, 1, B->attn, true, B->oout, false, B->ws, s))) return rc;
        return block_mlp_one(B, h, s);
    }
    // the attention's combine writes the o projection's operand directly
    DecOpSink sink{B->o->s2, nullptr, nullptr};
    const bool osink = B->hd % 128 == 0 && q4_flat_operand(B->o, B->ws, &sink.op, &sink.sc);
    if (pos_dev) {
        const size_t qs = B->H * B->hd;
        if ((rc = sage_decode_batch(&one, B->qrot, qs, B->kc, B->vc, kvs, B->block, B->attn, qs, B->state,
                                    B->state_bytes, B->cap, nullptr, nullptr, 1, s, pos_dev,
                                    osink ? &sink : nullptr, fold ? &rp : nullptr)))
            return rc;
    } else {
        const qbk_attn_shape sh{1, B->H, B->Hk, 1, pos + 1, B->hd, B->hd};
        const size_t cached = B->tokens[0] <= pos ? B->tokens[0] : 0;
        if ((rc = sage_decode_step_sink(ctx, &sh, B->qrot, B->kc, B->vc, B->block, B->attn, B->state,
                                        B->state_bytes, B->cap, cached, osink ? &sink : nullptr, stream,
                                        fold ? &rp : nullptr)))
            return rc;
        B->tokens[0] = pos + 1;
        B->filled[0] = pos + 1;
    }
    if ((rc = osink ? q4_run_staged(B->o, B->oout, false, nullptr, B->ws, s)
                    : q4_run(B->o, 1, B->attn, true, B->oout, false, B->ws, s)))
        return rc;
    return block_mlp_one(B, h, s);
}

// The MLP sublayer of one position of sequence 0, from the o projection's
// output B->oout: h1 = o + h, its norm, gate / up, SwiGLU, down + h1 -> h.
static int block_mlp_one(qbk_block *B, float *h, hipStream_t s) {
    int rc;
    const int d = (int)B->d, ffn = (int)B->ffn;
    const bool fits = d <= BLKD_NORM_THREADS * BLKD_OP_PER;
    uint8_t *op, *sc;
    const float *s2c;
    if (fits && q4_set_flat_operand(B->gu, B->ws, &op, &sc, &s2c)) {
        hipLaunchKernelGGL(blkd_norm_op, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, B->oout, (const float *)h, B->h1,
                           B->w_post, B->eps, d, 2, s2c, op, sc, 2);
        QBK_HIP(hipGetLastError());
        if ((rc = q4_set_run_staged(B->gu, B->ycat, false, B->ws, s))) return rc;
    } else {
        hipLaunchKernelGGL(blkd_norm, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, B->oout, (const float *)h, B->h1,
                           B->w_post, B->eps, B->xcat, 2, d);
        QBK_HIP(hipGetLastError());
        if ((rc = q4_set_run(B->gu, B->xcat, false, B->ycat, false, B->ws, s))) return rc;
    }
    // h' = down(SwiGLU) + h1: the residual added in the down projection's
    // epilogue when it runs from a flat operand
    if (q4_flat_operand(B->down, B->ws, &op, &sc)) {
        hipLaunchKernelGGL(blkd_swiglu_op, dim3((unsigned)div_ceil((size_t)ffn / 16, 256)), dim3(256), 0, s,
                           (const float *)B->ycat, (const float *)B->ycat + ffn, ffn, B->down->s2, op, sc, 2);
        QBK_HIP(hipGetLastError());
        return q4_run_staged(B->down, h, false, B->h1, B->ws, s);
    }
    hipLaunchKernelGGL(blkd_swiglu, dim3((ffn + 255) / 256), dim3(256), 0, s, B->ycat, B->hid, ffn);
    QBK_HIP(hipGetLastError());
    if ((rc = q4_run(B->down, 1, B->hid, true, B->dout, false, B->ws, s))) return rc;
    hipLaunchKernelGGL(blkd_add, dim3((d + 255) / 256), dim3(256), 0, s, B->dout, B->h1, h, d);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

extern "C" {

int qbk_block_decode_dev(qbk_ctx *ctx, qbk_block *B, float *h, size_t pos, void *stream) {
    return block_decode_one(ctx, B, h, pos, nullptr, stream);
}

}  // extern "C"

// A device-position step reads the kept attention state for every complete
// key block before its position, so each sequence's state must cover the
// cached rows -- not so after a prefill or qbk_block_set_filled, whose state
// is rebuilt by the next eager step.
static int pos_state_ready(const qbk_block *B, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (B->tokens[i] < B->filled[i])
            return fail(QBK_ERR_VALIDATION,
                        fmt("sequence %zu: the attention state covers %zu of its %zu cached positions; a "
                            "device-position step needs an eager step first", i, B->tokens[i], B->filled[i]));
    return QBK_OK;
}

extern "C" {

int qbk_block_decode_pos_dev(qbk_ctx *ctx, qbk_block *B, float *h, const uint32_t *pos, void *stream) {
    if (!pos || !B) return fail(QBK_ERR_VALIDATION, "null argument");
    if (B->face == QBK_ATTN_EXACT) return fail(QBK_ERR_VALIDATION, kExactFaceOnly);
    if (B->serving == QBK_F32) return fail(QBK_ERR_VALIDATION, kF32Only);
    int rc;
    if ((rc = pos_state_ready(B, 1))) return rc;
    return block_decode_one(ctx, B, h, 0, pos, stream);
}

int qbk_block_set_positions(qbk_block *B, const size_t *pos, size_t n) {
    if (!B || !pos) return fail(QBK_ERR_VALIDATION, "null argument");
    if (n == 0 || n > B->nseq)
        return fail(QBK_ERR_VALIDATION, fmt("%zu sequences on a block holding %zu", n, B->nseq));
    for (size_t i = 0; i < n; i++)
        if (pos[i] > B->cap)
            return fail(QBK_ERR_VALIDATION,
                        fmt("sequence %zu: %zu positions exceed the block's cache capacity of %zu", i, pos[i], B->cap));
    for (size_t i = 0; i < n; i++) B->tokens[i] = B->filled[i] = pos[i];
    return QBK_OK;
}

int qbk_block_set_filled(qbk_block *B, const size_t *rows, size_t n) {
    if (!B || !rows) return fail(QBK_ERR_VALIDATION, "null argument");
    if (n == 0 || n > B->nseq)
        return fail(QBK_ERR_VALIDATION, fmt("%zu sequences on a block holding %zu", n, B->nseq));
    for (size_t i = 0; i < n; i++)
        if (rows[i] > B->cap)
            return fail(QBK_ERR_VALIDATION,
                        fmt("sequence %zu: %zu rows exceed the block's cache capacity of %zu", i, rows[i], B->cap));
    for (size_t i = 0; i < n; i++) {
        B->filled[i] = rows[i];
        B->tokens[i] = 0;  // the attention state rebuilds its codes from the cache
    }
    return QBK_OK;
}

int qbk_block_set_attention_face(qbk_block *B, int face) {
    if (!B) return fail(QBK_ERR_VALIDATION, "null block");
    if (face != QBK_ATTN_SAGE && face != QBK_ATTN_EXACT)
        return fail(QBK_ERR_VALIDATION,
                    fmt("attention face must be QBK_ATTN_SAGE (0) or QBK_ATTN_EXACT (1), got %d", face));
    B->face = face;
    return QBK_OK;
}

int qbk_block_set_serving(qbk_ctx *ctx, qbk_block *B, int serving) {
    int rc;
    if (!B) return fail(QBK_ERR_VALIDATION, "null block");
    if (serving != QBK_F32 && serving != QBK_BF16)
        return fail(QBK_ERR_VALIDATION, "serving dtype must be QBK_F32 or QBK_BF16");
    if (serving == QBK_F32 && !B->xf) {
        if ((rc = bind(ctx))) return rc;
        if (B->device != ctx->device)
            return fail(QBK_ERR_VALIDATION, "block lives on another device than the context");
        size_t nd = 0;
        for (const qbk_factor *L : B->lay) nd = std::max(nd, L->din + L->r + L->dout);
        void *xf = nullptr, *sc = nullptr;
        QBK_HIP(hipMalloc(&xf, B->d * sizeof(float)));
        B->allocs.push_back(xf);
        QBK_HIP(hipMalloc(&sc, nd * sizeof(double)));
        B->allocs.push_back(sc);
        for (const qbk_factor *L : B->lay)
            if ((rc = factor_rows_ready(L, nullptr))) return rc;
        B->xf = (float *)xf;
        B->f64s = (double *)sc;
    }
    B->serving = serving;
    return QBK_OK;
}

int qbk_block_reset(qbk_block *B) {
    if (!B) return fail(QBK_ERR_VALIDATION, "null block");
    for (size_t i = 0; i < B->nseq; i++) B->tokens[i] = B->filled[i] = 0;
    return QBK_OK;
}

size_t qbk_block_prefill_workspace_size(const qbk_block *B, size_t n_tokens) {
    if (!B || n_tokens == 0) return 0;
    return blkp_plan(B, B->lay, n_tokens).bytes;
}

int qbk_block_prefill_seq_dev(qbk_ctx *ctx, qbk_block *B, size_t seq, float *h, size_t n, void *workspace,
                              size_t workspace_size, void *stream) {
    int rc;
    if (!B || !h) return fail(QBK_ERR_VALIDATION, "null argument");
    if (seq >= B->nseq)
        return fail(QBK_ERR_VALIDATION, fmt("sequence %zu of a block holding %zu", seq, B->nseq));
    if (n == 0) return fail(QBK_ERR_VALIDATION, "prefill needs at least one token");
    if (n > B->cap)
        return fail(QBK_ERR_VALIDATION, fmt("prefill of %zu tokens exceeds the block's cache capacity of %zu", n, B->cap));
    if (B->face == QBK_ATTN_EXACT || B->serving == QBK_F32) {
        // forward_prefill's per-token loop (engine/mod.rs:811-822) on the
        // exact face or at fp32 serving: row t through the decode step at
        // position t
        if (seq != 0) return fail(QBK_ERR_VALIDATION, B->serving == QBK_F32 ? kF32Only : kExactFaceOnly);
        for (size_t t = 0; t < n; t++)
            if ((rc = block_decode_one(ctx, B, h + t * B->d, t, nullptr, stream))) return rc;
        return QBK_OK;
    }
    if (B->hd != 128)
        return fail(QBK_ERR_VALIDATION,
                    fmt("block prefill runs the block-scaled SageAttention, which needs head_dim 128; got %zu", B->hd));
    const BlkpPlan P = blkp_plan(B, B->lay, n);
    if (!workspace || workspace_size < P.bytes)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this prefill needs", workspace_size, P.bytes));
    if ((rc = bind(ctx))) return rc;
    if (B->device != ctx->device) return fail(QBK_ERR_VALIDATION, "block lives on another device than the context");
    hipStream_t s = (hipStream_t)stream;
    char *w = (char *)workspace;
    uint16_t *x = (uint16_t *)(w + P.o_x), *qb = (uint16_t *)(w + P.o_qb), *kb = (uint16_t *)(w + P.o_kb),
             *vb = (uint16_t *)(w + P.o_vb), *arow = (uint16_t *)(w + P.o_arow);
    float *q = (float *)(w + P.o_q), *k = (float *)(w + P.o_k), *v = (float *)(w + P.o_v),
          *oo = (float *)(w + P.o_oo), *h1 = (float *)(w + P.o_h1), *g = (float *)(w + P.o_g),
          *u = (float *)(w + P.o_u);
    void *ws = w + P.o_gemm;
    const int d = (int)B->d, hd = (int)B->hd, H = (int)B->H, Hk = (int)B->Hk;
    const size_t nd = n * B->d, nf = n * B->ffn;
    // attention sublayer: norm, q/k/v at batch n, q/k norms + RoPE + cache
    blkp_norm_launch(n, h, nullptr, nullptr, B->w_in, B->eps, x, d, 1, s);
    QBK_HIP(hipGetLastError());
    if ((rc = blkp_proj(B->lay[0], n, x, false, q, ws, s)) || (rc = blkp_proj(B->lay[1], n, x, false, k, ws, s)) ||
        (rc = blkp_proj(B->lay[2], n, x, false, v, ws, s)))
        return rc;
    const size_t kvs = B->cap * B->Hk * B->hd;  // one sequence's cache floats
    hipLaunchKernelGGL(blkp_qk_rope, dim3((H + Hk + 3) / 4, (unsigned)n), dim3(256), 0, s, q, k, v, B->rope, B->w_q, B->w_k,
                       B->eps, B->kc + seq * kvs, B->vc + seq * kvs, qb, kb, vb, H, Hk, hd, (int)n);
    QBK_HIP(hipGetLastError());
    // causal block-scaled SageAttention over the n tokens
    const qbk_attn_shape sh{1, B->H, B->Hk, n, n, B->hd, B->hd};
    // written token-major: the o projection's rows
    if ((rc = sage_blk_run(ctx, &sh, qb, kb, vb, 1, arow, true, w + P.o_sage, P.sage_bytes, stream))) return rc;
    // o + residual, norm, gate / up, SwiGLU, down + residual
    if ((rc = blkp_proj(B->o, n, arow, false, oo, ws, s))) return rc;
    blkp_norm_launch(n, oo, h, h1, B->w_post, B->eps, x, d, 1, s);
    QBK_HIP(hipGetLastError());
    if ((rc = blkp_proj(B->lay[4], n, x, false, g, ws, s)) || (rc = blkp_proj(B->lay[5], n, x, false, u, ws, s)))
        return rc;
    if (n > Q4_MAXB && q4g_use(B->down, n) && B->ffn % 4 == 0) {
        // SwiGLU writes the down projection's z in bf16 (read at s2 = 1), and
        // h = down + h1, the residual added in the GEMM's epilogue
        uint16_t *z = (uint16_t *)(w + P.o_z);
        hipLaunchKernelGGL(blkp_swiglu_z, dim3((unsigned)div_ceil(nf / 4, 256)), dim3(256), 0, s, g, u,
                           B->down->s2, z, nf, (uint32_t)B->ffn);
        QBK_HIP(hipGetLastError());
        if ((rc = q4g_run(B->down, z, false, n, h, false, (uint16_t *)ws, s, h1, B->ones_ffn))) return rc;
    } else {
        hipLaunchKernelGGL(blkp_swiglu, dim3((unsigned)div_ceil(nf, 256)), dim3(256), 0, s, g, u, g, nf);
        QBK_HIP(hipGetLastError());
        if ((rc = blkp_proj(B->down, n, g, true, oo, ws, s))) return rc;
        hipLaunchKernelGGL(blkp_add, dim3((unsigned)div_ceil(nd, 256)), dim3(256), 0, s, oo, h1, h, nd);
        QBK_HIP(hipGetLastError());
    }
    B->filled[seq] = n;
    B->tokens[seq] = 0;  // the decode attention state rebuilds its codes from the cache
    return QBK_OK;
}

int qbk_block_prefill_dev(qbk_ctx *ctx, qbk_block *B, float *h, size_t n, void *workspace, size_t workspace_size,
                          void *stream) {
    return qbk_block_prefill_seq_dev(ctx, B, 0, h, n, workspace, workspace_size, stream);
}

size_t qbk_block_decode_batch_workspace_size(const qbk_block *B, size_t n) {
    if (!B || n == 0) return 0;
    return blkb_plan(B, n).bytes;
}

// One position of each of sequences 0 .. n - 1 (sequence i at pos[i]): the
// projections batched over the n rows (the GEMV up to batch 8, the GEMM
// beyond), RoPE and the cache append per sequence, the sage decode
// attention stepping every sequence's kept state.
}  // extern "C"

// With pos_dev (device, n entries) in place of pos: each sequence at the
// position its word holds when the step runs; the host record of cached
// positions is then left to the caller.
static int block_decode_batch(qbk_ctx *ctx, qbk_block *B, float *h, const size_t *pos, const uint32_t *pos_dev,
                              size_t n, void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if (!B || !h || (!pos && !pos_dev)) return fail(QBK_ERR_VALIDATION, "null argument");
    if (B->face == QBK_ATTN_EXACT) return fail(QBK_ERR_VALIDATION, kExactFaceOnly);
    if (B->serving == QBK_F32) return fail(QBK_ERR_VALIDATION, kF32Only);
    if (n == 0 || n > B->nseq)
        return fail(QBK_ERR_VALIDATION, fmt("batch of %zu sequences on a block holding %zu", n, B->nseq));
    for (size_t i = 0; !pos_dev && i < n; i++) {
        if (pos[i] >= B->cap)
            return fail(QBK_ERR_VALIDATION,
                        fmt("position %zu is past the block's cache capacity of %zu", pos[i], B->cap));
        if (pos[i] > B->filled[i])
            return fail(QBK_ERR_VALIDATION, fmt("sequence %zu: position %zu skips cache rows: the block holds %zu "
                                                "positions", i, pos[i], B->filled[i]));
    }
    const BlkbPlan P = blkb_plan(B, n);
    if (!workspace || workspace_size < P.bytes)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this step needs", workspace_size, P.bytes));
    if ((rc = bind(ctx))) return rc;
    if (B->device != ctx->device) return fail(QBK_ERR_VALIDATION, "block lives on another device than the context");
    hipStream_t s = (hipStream_t)stream;
    char *w = (char *)workspace;
    uint16_t *x = (uint16_t *)(w + P.o_x);
    const size_t qd = B->H * B->hd, kd = B->Hk * B->hd;
    float *q = (float *)(w + P.o_qkv), *k = q + n * qd, *v = k + n * kd, *qr = (float *)(w + P.o_qr),
          *at = (float *)(w + P.o_at), *oo = (float *)(w + P.o_oo), *h1 = (float *)(w + P.o_h1),
          *g = (float *)(w + P.o_gu), *u = g + n * B->ffn;
    void *ws = w + P.o_gemm;
    const int d = (int)B->d, hd = (int)B->hd, H = (int)B->H, Hk = (int)B->Hk;
    const size_t nd = n * B->d, nf = n * B->ffn, kvs = B->cap * B->Hk * B->hd;
    // From 2 tokens on the layer-set GEMV, the norms and SwiGLU write their
    // projections' stage-1 operands themselves (no prep launch) and the down
    // projection's epilogue adds the residual.
    const bool fits = P.sets && n >= 2 && d <= BLKD_NORM_THREADS * BLKD_OP_PER;
    uint8_t *op, *sc;
    const float *s2c;
    const bool qkv_op = fits && q4_set_flat_operand_batch(B->qkv, n, ws, &op, &sc, &s2c);
    if (qkv_op)
        hipLaunchKernelGGL(blkd_norm_op, dim3((unsigned)n), dim3(BLKD_NORM_THREADS), 0, s, h, (const float *)nullptr,
                           (float *)nullptr, B->w_in, B->eps, d, 3, s2c, op, sc, (int)(2 * n));
    else
        blkp_norm_launch(n, h, nullptr, nullptr, B->w_in, B->eps, x, d, P.sets ? 3 : 1, s);
    QBK_HIP(hipGetLastError());
    if (qkv_op) {
        if ((rc = q4_set_run_batch_staged(B->qkv, n, q, false, ws, s))) return rc;
    } else if (P.sets) {
        if ((rc = q4_set_run_batch(B->qkv, n, x, false, q, false, ws, s))) return rc;
    } else if (q4_set_gemm_fits(B->qkv, n)) {
        // q, k, v as one set on the GEMM (y [layer][n][dout]: q, then k, v)
        if ((rc = q4_set_gemm_run(B->qkv, n, x, false, q, false, ws, s))) return rc;
    } else if ((rc = blkp_proj(B->lay[0], n, x, false, q, ws, s)) ||
               (rc = blkp_proj(B->lay[1], n, x, false, k, ws, s)) ||
               (rc = blkp_proj(B->lay[2], n, x, false, v, ws, s))) {
        return rc;
    }
    BlkbPos bp{};
    for (size_t i = 0; !pos_dev && i < n; i++) bp.p[i] = (uint32_t)pos[i];
    hipLaunchKernelGGL(blkb_qk_rope, dim3(H + Hk, (unsigned)n), dim3(64), 0, s, q, k, v, B->rope, bp, pos_dev,
                       B->cap, B->w_q, B->w_k, B->eps, B->kc, B->vc, kvs, qr, H, Hk, hd);
    QBK_HIP(hipGetLastError());
    const qbk_attn_shape one{1, B->H, B->Hk, 1, B->cap, B->hd, B->hd};
    const size_t qs = B->H * B->hd;
    if (pos_dev) {
        if ((rc = sage_decode_batch(&one, qr, qs, B->kc, B->vc, kvs, B->block, at, qs, B->state, B->state_bytes,
                                    B->cap, nullptr, nullptr, n, s, pos_dev)))
            return rc;
    } else if (sage_decode_batchable(&one, B->block, B->cap, B->kc, B->vc, kvs)) {
        size_t skv[BLKB_MAXSEQ], kept[BLKB_MAXSEQ];
        for (size_t i = 0; i < n; i++) {
            skv[i] = pos[i] + 1;
            kept[i] = B->tokens[i] <= pos[i] ? B->tokens[i] : 0;
        }
        if ((rc = sage_decode_batch(&one, qr, qs, B->kc, B->vc, kvs, B->block, at, qs, B->state, B->state_bytes,
                                    B->cap, skv, kept, n, s)))
            return rc;
    } else {
        for (size_t i = 0; i < n; i++) {
            const qbk_attn_shape sh{1, B->H, B->Hk, 1, pos[i] + 1, B->hd, B->hd};
            const size_t cached = B->tokens[i] <= pos[i] ? B->tokens[i] : 0;
            if ((rc = qbk_attention_sage_decode_step_dev(ctx, &sh, qr + i * qs, B->kc + i * kvs, B->vc + i * kvs,
                                                         B->block, at + i * qs,
                                                         (char *)B->state + i * B->state_bytes, B->state_bytes,
                                                         B->cap, cached, stream)))
                return rc;
        }
    }
    for (size_t i = 0; !pos_dev && i < n; i++) B->tokens[i] = B->filled[i] = pos[i] + 1;
    if ((rc = P.sets ? q4_run(B->o, n, at, true, oo, false, ws, s) : blkp_proj(B->o, n, at, true, oo, ws, s)))
        return rc;
    const bool gu_op = fits && q4_set_flat_operand_batch(B->gu, n, ws, &op, &sc, &s2c);
    if (gu_op)
        hipLaunchKernelGGL(blkd_norm_op, dim3((unsigned)n), dim3(BLKD_NORM_THREADS), 0, s, (const float *)oo,
                           (const float *)h, h1, B->w_post, B->eps, d, 2, s2c, op, sc, (int)(2 * n));
    else
        blkp_norm_launch(n, oo, h, h1, B->w_post, B->eps, x, d, P.sets ? 2 : 1, s);
    QBK_HIP(hipGetLastError());
    if (gu_op) {
        if ((rc = q4_set_run_batch_staged(B->gu, n, g, false, ws, s))) return rc;
    } else if (P.sets) {
        if ((rc = q4_set_run_batch(B->gu, n, x, false, g, false, ws, s))) return rc;
    } else if (q4_set_gemm_fits(B->gu, n)) {
        if ((rc = q4_set_gemm_run(B->gu, n, x, false, g, false, ws, s))) return rc;
    } else if ((rc = blkp_proj(B->lay[4], n, x, false, g, ws, s)) ||
               (rc = blkp_proj(B->lay[5], n, x, false, u, ws, s))) {
        return rc;
    }
    if (fits && q4_flat_operand_batch(B->down, n, ws, &op, &sc)) {
        hipLaunchKernelGGL(blkd_swiglu_op, dim3((unsigned)div_ceil(B->ffn / 16, 256), (unsigned)n), dim3(256), 0, s,
                           (const float *)g, (const float *)u, (int)B->ffn, B->down->s2, op, sc, (int)(2 * n));
        QBK_HIP(hipGetLastError());
        return q4_run_staged_batch(B->down, n, h, false, h1, ws, s);  // h = down(hid) + h1
    }
    hipLaunchKernelGGL(blkp_swiglu, dim3((unsigned)div_ceil(nf, 256)), dim3(256), 0, s, g, u, g, nf);
    QBK_HIP(hipGetLastError());
    if ((rc = P.sets ? q4_run(B->down, n, g, true, oo, false, ws, s) : blkp_proj(B->down, n, g, true, oo, ws, s)))
        return rc;
    hipLaunchKernelGGL(blkp_add, dim3((unsigned)div_ceil(nd, 256)), dim3(256), 0, s, oo, h1, h, nd);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

extern "C" {

int qbk_block_decode_batch_dev(qbk_ctx *ctx, qbk_block *B, float *h, const size_t *pos, size_t n, void *workspace,
                               size_t workspace_size, void *stream) {
    if (!pos) return fail(QBK_ERR_VALIDATION, "null argument");
    return block_decode_batch(ctx, B, h, pos, nullptr, n, workspace, workspace_size, stream);
}

int qbk_block_decode_batch_pos_dev(qbk_ctx *ctx, qbk_block *B, float *h, const uint32_t *pos, size_t n,
                                   void *workspace, size_t workspace_size, void *stream) {
    if (!pos) return fail(QBK_ERR_VALIDATION, "null argument");
    if (B && B->face == QBK_ATTN_EXACT) return fail(QBK_ERR_VALIDATION, kExactFaceOnly);
    if (B && B->serving == QBK_F32) return fail(QBK_ERR_VALIDATION, kF32Only);
    if (B && n && n <= B->nseq) {
        int rc;
        if ((rc = pos_state_ready(B, n))) return rc;
        const qbk_attn_shape one{1, B->H, B->Hk, 1, B->cap, B->hd, B->hd};
        if (!sage_decode_batchable(&one, B->block, B->cap, B->kc, B->vc, B->cap * B->Hk * B->hd))
            return fail(QBK_ERR_VALIDATION, "a device-position step needs the grouped sage decode kernels "
                                            "(head_dim a multiple of 16, groups of up to 16 heads, blocks of up "
                                            "to 64 tokens)");
    }
    return block_decode_batch(ctx, B, h, nullptr, pos, n, workspace, workspace_size, stream);
}

}  // extern "C"
