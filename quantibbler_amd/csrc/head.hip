// head.hip -- the language-model head on gfx950.
//
// engine/mod.rs:781-800 (Engine::logits; the prefill path, :1131-1147, is
// the same loop per position): logits[v] = sum_t hidden[t] * head[v][t],
// one f32 sum per vocabulary row in t order, each term a separate f32
// multiply and add.  Every row's sum stays in one lane, in that order, so
// the logits are bit-identical to the reference's; the parallelism is the
// rows (128256 for a Llama-3 vocabulary).
//
// Layout: the head is stored transposed per wave and grouped four steps a
// lane, [vocab_p / RW][d_p / 4][64 lanes][4 steps] dwords, with RW the rows
// one wave covers (vocab_p = vocab rounded up to the rows of a workgroup,
// d_p = d_model rounded up to 4, both zero-padded): a lane's four steps are
// one 16-byte load, a wave's four steps one contiguous KiB, and a wave's
// steps follow each other in memory, so every wave streams one contiguous
// region (the plain [d_model][vocab] transpose made each step 256 KB from
// the last and read at 4.6 TB/s; one dword a lane a step, 5.4 TB/s: a wave
// can have at most 63 loads in flight, 16 KiB of dwords).  When every
// element is a bf16 value (the reference's bf16 serving quantises the head
// so, engine/mod.rs:695-706) it is stored as bf16 -- 1.05 GB instead of 2.1
// for 128256 x 4096 -- and widened exactly on use; otherwise as f32.
//
// At one hidden row the dot product is HBM-bound (one pass over the head
// per call; the row rides in SGPRs through scalar loads).  From two rows a
// wave on, the rows' values come through LDS (head_logits_lds_kernel), and
// beyond eight rows two or four waves share each block of head words (the
// block fetched once from memory), so that a batch's products (two VALU ops
// a term: the reference rounds the product and the sum separately) spread
// over more SIMDs.  A lane covers two vocabulary rows (bf16: one dword
// holds both) or one (f32), reads a dword per step, and keeps two chunks
// of loads in flight (alternating register sets, so no in-flight register
// is ever copied).
#include <string.h>

#include "qbk_internal.h"

#pragma clang fp contract(off)

struct qbk_head {
    int device;
    size_t vocab, d_model, vocab_p;
    int bf16;    // elements stored as bf16 (all were bf16 values), else f32
    void *w;     // [vocab_p / RW][d_p / 4][64][4] dwords, RW = head_rows_per_wave(bf16)
};

namespace qbk {

#define HEAD_THREADS 256
#define HEAD_CHUNK 64   // steps per load chunk
#define HEAD_MAXB 8     // hidden rows per launch
#define HEAD_LDS_CH 32  // steps per load chunk of the LDS-fed kernel (16: 3-5 % slower at 8-32 rows)

typedef __attribute__((address_space(1))) const uint32_t g32_t;
typedef __attribute__((address_space(4))) const float cf32_t;

// rows one wave / one workgroup covers
__host__ __device__ static inline size_t head_rows_per_wave(int bf16) { return bf16 ? 128 : 64; }
static inline size_t head_rows_per_wg(int bf16) { return (HEAD_THREADS / 64) * head_rows_per_wave(bf16); }

// one chunk of CH steps from t0 on, words in W: the lane's
// rows += hidden[b][t] * w (bf16: the word's low half is row 2c, high half
// row 2c + 1)
template <bool BF16, int NB, int CH>
__device__ __forceinline__ void head_chunk(float acc[NB][2], const uint32_t W[CH], const cf32_t *const h[NB],
                                           size_t t0) {
    float w0[CH], w1[CH];
#pragma unroll
    for (int u = 0; u < CH; u++) {
        w0[u] = BF16 ? __uint_as_float(W[u] << 16) : __uint_as_float(W[u]);
        w1[u] = BF16 ? __uint_as_float(W[u] & 0xffff0000u) : 0.0f;
    }
    // hidden row by hidden row (each row's steps in order), so that only one
    // row's values of the chunk are live in SGPRs at a time
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const float hv = h[b][t0 + u];
            acc[b][0] = acc[b][0] + hv * w0[u];
            if (BF16) acc[b][1] = acc[b][1] + hv * w1[u];
        }
}

typedef uint32_t hu32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const hu32x4_t g128_t;

// steps t0 .. t0 + CH - 1 (t0 a multiple of 4) of the lane's column, four
// a load; q4last = the last four-step group
template <int CH>
__device__ __forceinline__ void head_load(uint32_t W[CH], const uint32_t *col, size_t t0, size_t q4last) {
#pragma unroll
    for (int u = 0; u < CH / 4; u++) {
        size_t q = t0 / 4 + u;
        q = q < q4last ? q : q4last;  // past the end: a repeated (unused) group
        const hu32x4_t v = __builtin_nontemporal_load((g128_t *)(col + q * 256));
#pragma unroll
        for (int e = 0; e < 4; e++) W[4 * u + e] = v[e];
    }
}

// logits[b][v] for up to NB hidden rows a wave.  w: the per-wave blocked
// layout, bf16 (dwords of two rows) or f32; lane l of wave block wb reads
// dword ((wb * d_p / 4 + t / 4) * 64 + l) * 4 + t % 4 at step t.  The four
// waves of a workgroup cover 4 / chunks wave blocks; the waves of one block
// take consecutive chunks of NB of the batch rows (the last chunk may hold
// fewer) -- the same head words, fetched once from memory and re-read from
// the CU's cache, so a batch of up to 4 NB rows keeps four waves a SIMD
// busy where one wave of 4 NB accumulators would run alone.
template <bool BF16, int NB>
__global__ void __launch_bounds__(HEAD_THREADS) head_logits_kernel(const uint32_t *w, size_t vocab_p, size_t vocab,
                                                                  size_t d, const float *hidden, float *logits,
                                                                  int chunks, int batch) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ci = wave % chunks;  // wave-uniform
    const size_t wb = (size_t)blockIdx.x * (HEAD_THREADS / 64 / chunks) + wave / chunks;
    const size_t lane = threadIdx.x & 63;
    const size_t dq = (d + 3) / 4;  // four-step groups
    const uint32_t *col = w + wb * dq * 256 + lane * 4;
    const int nb = batch - ci * NB < NB ? batch - ci * NB : NB;  // rows of this wave's chunk (>= 1)
    hidden += (size_t)ci * NB * d;
    logits += (size_t)ci * NB * vocab;
    const cf32_t *h[NB];  // the chunk's rows; rows past nb repeat the last (not stored)
#pragma unroll
    for (int b = 0; b < NB; b++) h[b] = (const cf32_t *)hidden + (size_t)(b < nb ? b : nb - 1) * d;
    float acc[NB][2];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b][0] = acc[b][1] = 0.0f;
    constexpr int CH = HEAD_CHUNK;
    const size_t dmain = d / (2 * CH) * (2 * CH);
    uint32_t A[CH], Bw[CH];
    if (dmain) {
        head_load<CH>(A, col, 0, dq - 1);
        for (size_t t0 = 0; t0 < dmain; t0 += 2 * CH) {
            head_load<CH>(Bw, col, t0 + CH, dq - 1);
            head_chunk<BF16, NB, CH>(acc, A, h, t0);
            head_load<CH>(A, col, t0 + 2 * CH, dq - 1);
            head_chunk<BF16, NB, CH>(acc, Bw, h, t0 + CH);
        }
    }
    for (size_t t = dmain; t < d; t++) {  // the last d % (2 CH) steps, in order
        const uint32_t wv = col[(t / 4) * 256 + t % 4];
        const float w0 = BF16 ? __uint_as_float(wv << 16) : __uint_as_float(wv);
        const float w1 = BF16 ? __uint_as_float(wv & 0xffff0000u) : 0.0f;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float hv = h[b][t];
            acc[b][0] = acc[b][0] + hv * w0;
            if (BF16) acc[b][1] = acc[b][1] + hv * w1;
        }
    }
    const size_t v0 = wb * head_rows_per_wave(BF16) + (BF16 ? 2 * lane : lane);
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b >= nb) break;
        if (v0 < vocab) logits[(size_t)b * vocab + v0] = acc[b][0];
        if (BF16 && v0 + 1 < vocab) logits[(size_t)b * vocab + v0 + 1] = acc[b][1];
    }
}

// The same logits for NB >= 2 hidden rows a wave, the rows' values read
// from LDS instead of scalar loads: each wave stages its rows' next CH steps
// ([step][8] floats, lane u loading step u of every row) one chunk ahead,
// and the products run step by step, a step's row values two broadcast
// reads (all lanes one address).  Each (row, vocabulary row) sum still runs
// over t in order.  (With the rows in SGPRs, eight rows a wave waited on a
// scalar memory round trip every sixteen values and ran at a third of the
// VALU rate the products need.)
typedef __attribute__((address_space(1))) const float gf32h_t;

template <bool BF16, int NB, int CH>
__global__ void __launch_bounds__(HEAD_THREADS) head_logits_lds_kernel(const uint32_t *w, size_t vocab_p,
                                                                      size_t vocab, size_t d, const float *hidden,
                                                                      float *logits, int chunks, int batch) {
    static_assert(NB >= 2 && NB <= 8 && CH <= 64 && CH % 4 == 0, "rows and chunk");
    __shared__ __attribute__((aligned(16))) float hs[HEAD_THREADS / 64][2][CH][8];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ci = wave % chunks;  // wave-uniform
    const size_t wb = (size_t)blockIdx.x * (HEAD_THREADS / 64 / chunks) + wave / chunks;
    const size_t lane = threadIdx.x & 63;
    const size_t dq = (d + 3) / 4;
    const uint32_t *col = w + wb * dq * 256 + lane * 4;
    const int nb = batch - ci * NB < NB ? batch - ci * NB : NB;  // rows of this wave's chunk (>= 1)
    hidden += (size_t)ci * NB * d;
    logits += (size_t)ci * NB * vocab;
    const gf32h_t *hr[NB];  // rows past nb repeat the last (not stored)
#pragma unroll
    for (int b = 0; b < NB; b++) hr[b] = (const gf32h_t *)hidden + (size_t)(b < nb ? b : nb - 1) * d;
    float acc[NB][2];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b][0] = acc[b][1] = 0.0f;
    float(*hw)[CH][8] = hs[wave];
    const size_t dmain = d / (2 * CH) * (2 * CH);
    const size_t us = lane % CH;  // the step this lane stages (lanes past CH repeat it, not stored)
    auto hload = [&](float H[NB], size_t t0) {
        size_t t = t0 + us;
        t = t < d ? t : d - 1;
#pragma unroll
        for (int b = 0; b < NB; b++) H[b] = hr[b][t];
    };
    auto hstore = [&](const float H[NB], int buf) {
        if (lane < CH) {
            float v[8];
#pragma unroll
            for (int b = 0; b < 8; b++) v[b] = b < NB ? H[b] : 0.0f;
            *(float4 *)&hw[buf][us][0] = make_float4(v[0], v[1], v[2], v[3]);
            if (NB > 4) *(float4 *)&hw[buf][us][4] = make_float4(v[4], v[5], v[6], v[7]);
        }
        __builtin_amdgcn_wave_barrier();
    };
    // a chunk in groups of HG steps: the next group's row values are read
    // while this group's products run (the empty asm statements, which take
    // the sums and fence memory, keep the compiler from hoisting every read
    // of the chunk ahead of the products, which held a register per value)
    constexpr int HG = 4;
    auto hread = [&](float4 R[HG][2], int buf, int u0) {
#pragma unroll
        for (int i = 0; i < HG; i++) {
            R[i][0] = *(const float4 *)&hw[buf][u0 + i][0];
            if (NB > 4) R[i][1] = *(const float4 *)&hw[buf][u0 + i][4];
        }
    };
    auto chunk = [&](const uint32_t W[CH], int buf) {
        float4 R[2][HG][2];
        hread(R[0], buf, 0);
#pragma unroll
        for (int g = 0; g < CH / HG; g++) {
            if (g + 1 < CH / HG) hread(R[(g + 1) & 1], buf, (g + 1) * HG);
#pragma unroll
            for (int i = 0; i < HG; i++) {
                const int u = g * HG + i;
                const float4 h0 = R[g & 1][i][0], h1 = R[g & 1][i][1];
                const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
                const float w0 = BF16 ? __uint_as_float(W[u] << 16) : __uint_as_float(W[u]);
                const float w1 = BF16 ? __uint_as_float(W[u] & 0xffff0000u) : 0.0f;
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    acc[b][0] = acc[b][0] + hv[b] * w0;
                    if (BF16) acc[b][1] = acc[b][1] + hv[b] * w1;
                }
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                __asm__ volatile("" : "+v"(acc[b][0]));
                if (BF16) __asm__ volatile("" : "+v"(acc[b][1]));
            }
            __asm__ volatile("" ::: "memory");
        }
    };
    uint32_t A[CH], Bw[CH];
    float HA[NB], HB[NB];
    if (dmain) {
        head_load<CH>(A, col, 0, dq - 1);
        hload(HA, 0);
#pragma unroll 1
        for (size_t t0 = 0; t0 < dmain; t0 += 2 * CH) {
            head_load<CH>(Bw, col, t0 + CH, dq - 1);
            hstore(HA, 0);
            hload(HB, t0 + CH);
            chunk(A, 0);
            head_load<CH>(A, col, t0 + 2 * CH, dq - 1);
            hstore(HB, 1);
            hload(HA, t0 + 2 * CH);
            chunk(Bw, 1);
        }
    }
    for (size_t t = dmain; t < d; t++) {  // the last d % (2 CH) steps, in order
        const uint32_t wv = col[(t / 4) * 256 + t % 4];
        const float w0 = BF16 ? __uint_as_float(wv << 16) : __uint_as_float(wv);
        const float w1 = BF16 ? __uint_as_float(wv & 0xffff0000u) : 0.0f;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float hv = hr[b][t];
            acc[b][0] = acc[b][0] + hv * w0;
            if (BF16) acc[b][1] = acc[b][1] + hv * w1;
        }
    }
    const size_t v0 = wb * head_rows_per_wave(BF16) + (BF16 ? 2 * lane : lane);
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (b >= nb) break;
        if (v0 < vocab) logits[(size_t)b * vocab + v0] = acc[b][0];
        if (BF16 && v0 + 1 < vocab) logits[(size_t)b * vocab + v0 + 1] = acc[b][1];
    }
}

// any element of src (f32, n of them) not a bf16 value -> *flag = 1
__global__ void head_bf16_check(const float *src, size_t n, uint32_t *flag) {
    uint32_t bad = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        bad |= __float_as_uint(src[i]) & 0xffffu;
    if (__builtin_amdgcn_ballot_w64(bad != 0) && (threadIdx.x & 63) == 0) atomicOr(flag, 1u);
}

// [vocab][d] f32 -> the per-wave blocked layout (bf16 halves or f32), zero
// padding; 32 x 32 tiles through LDS
template <bool BF16>
__global__ void __launch_bounds__(256) head_transpose(const float *src, size_t vocab, size_t d, size_t vocab_p,
                                                      void *dst) {
    __shared__ float tile[32][33];
    const size_t v0 = (size_t)blockIdx.x * 32, t0 = (size_t)blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const size_t v = v0 + r, t = t0 + tx;
        tile[r][tx] = v < vocab && t < d ? src[v * d + t] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const size_t t = t0 + r, v = v0 + tx;
        if (t >= d || v >= vocab_p) continue;
        const float x = tile[tx][r];
        const size_t rw = head_rows_per_wave(BF16), rr = v % rw, dq = (d + 3) / 4;
        const size_t lane = BF16 ? rr / 2 : rr;
        const size_t dw = (((v / rw) * dq + t / 4) * 64 + lane) * 4 + t % 4;  // the dword
        if (BF16)
            ((uint16_t *)dst)[2 * dw + rr % 2] = (uint16_t)(__float_as_uint(x) >> 16);
        else
            ((float *)dst)[dw] = x;
    }
}

static int head_build(qbk_ctx *ctx, const float *src_dev, size_t vocab, size_t d_model, qbk_head **out) {
    qbk_head *H = new qbk_head();
    H->device = ctx->device;
    H->vocab = vocab;
    H->d_model = d_model;
    uint32_t *flag = nullptr;
    hipError_t e = hipMalloc((void **)&flag, 4);
    if (e == hipSuccess) e = hipMemset(flag, 0, 4);
    if (e == hipSuccess) {
        const size_t n = vocab * d_model;
        hipLaunchKernelGGL(head_bf16_check, dim3((unsigned)(div_ceil(n, 256) < 4096 ? div_ceil(n, 256) : 4096)),
                           dim3(256), 0, 0, src_dev, n, flag);
        e = hipGetLastError();
    }
    uint32_t f = 1;
    if (e == hipSuccess) e = hipMemcpy(&f, flag, 4, hipMemcpyDeviceToHost);
    if (flag) (void)hipFree(flag);
    H->bf16 = f == 0;
    H->vocab_p = round_up(vocab, head_rows_per_wg(H->bf16));
    const size_t bytes = round_up(d_model, 4) * H->vocab_p * (H->bf16 ? 2 : 4);
    if (e == hipSuccess) e = hipMalloc(&H->w, bytes);
    if (e == hipSuccess) e = hipMemset(H->w, 0, bytes);  // the padded steps
    if (e == hipSuccess) {
        dim3 g((unsigned)div_ceil(H->vocab_p, 32), (unsigned)div_ceil(d_model, 32));
        if (H->bf16)
            hipLaunchKernelGGL(head_transpose<true>, g, dim3(256), 0, 0, src_dev, vocab, d_model, H->vocab_p, H->w);
        else
            hipLaunchKernelGGL(head_transpose<false>, g, dim3(256), 0, 0, src_dev, vocab, d_model, H->vocab_p, H->w);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (H->w) (void)hipFree(H->w);
        delete H;
        return fail(QBK_ERR_DEVICE, fmt("lm_head upload failed: %s", hipGetErrorString(e)));
    }
    *out = H;
    return QBK_OK;
}

// Up to 4 HEAD_MAXB rows a launch: 1, 2 or 4 chunks of at most HEAD_MAXB
// rows, a wave each, over the same head words.
static int head_run(const qbk_head *H, const float *hidden, size_t batch, float *logits, hipStream_t s) {
    const size_t rpw = head_rows_per_wg(H->bf16);
    for (size_t b0 = 0; b0 < batch; b0 += 4 * HEAD_MAXB) {
        const size_t rows = batch - b0 < 4 * HEAD_MAXB ? batch - b0 : 4 * HEAD_MAXB;
        // (four waves of two rows each for a batch of 8 took 452 us against
        // 338 for one wave of eight: the waves sharing a block re-read its
        // words from the caches, and at two rows a wave that traffic bounds)
        const int chunks = rows <= HEAD_MAXB ? 1 : rows <= 2 * HEAD_MAXB ? 2 : 4;
        const size_t nb = div_ceil(rows, (size_t)chunks);
        const dim3 g((unsigned)(H->vocab_p / (rpw / chunks)));
        const float *hb = hidden + b0 * H->d_model;
        float *lb = logits + b0 * H->vocab;
        const uint32_t *w = (const uint32_t *)H->w;
#define HEAD_LAUNCH(BF, NB)                                                                                   \
    if (NB == 1)                                                                                              \
        hipLaunchKernelGGL((head_logits_kernel<BF, 1>), g, dim3(HEAD_THREADS), 0, s, w, H->vocab_p, H->vocab,  \
                           H->d_model, hb, lb, chunks, (int)rows);                                            \
    else                                                                                                      \
        hipLaunchKernelGGL((head_logits_lds_kernel<BF, (NB > 1 ? NB : 2), HEAD_LDS_CH>), g, dim3(HEAD_THREADS), \
                           0, s, w, H->vocab_p, H->vocab, H->d_model, hb, lb, chunks, (int)rows)
#define HEAD_BATCH(BF)                                                                                        \
    switch (nb) {                                                                                             \
        case 1: HEAD_LAUNCH(BF, 1); break;                                                                    \
        case 2: HEAD_LAUNCH(BF, 2); break;                                                                    \
        case 3: HEAD_LAUNCH(BF, 3); break;                                                                    \
        case 4: HEAD_LAUNCH(BF, 4); break;                                                                    \
        case 5: HEAD_LAUNCH(BF, 5); break;                                                                    \
        case 6: HEAD_LAUNCH(BF, 6); break;                                                                    \
        case 7: HEAD_LAUNCH(BF, 7); break;                                                                    \
        default: HEAD_LAUNCH(BF, 8); break;                                                                   \
    }
        if (H->bf16) {
            HEAD_BATCH(true)
        } else {
            HEAD_BATCH(false)
        }
#undef HEAD_BATCH
#undef HEAD_LAUNCH
        QBK_HIP(hipGetLastError());
    }
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_head_create(qbk_ctx *ctx, const float *head, size_t head_len, size_t vocab, size_t d_model,
                    qbk_head **out) {
    int rc;
    if (!out) return fail(QBK_ERR_VALIDATION, "null output handle");
    *out = nullptr;
    if (vocab == 0 || d_model == 0) return fail(QBK_ERR_VALIDATION, "lm_head requires non-empty vocab and d_model");
    if (head_len != vocab * d_model)
        return fail(QBK_ERR_VALIDATION, fmt("lm_head is %zu floats; expected %zux%zu = %zu", head_len, vocab,
                                            d_model, vocab * d_model));
    if (!head) return fail(QBK_ERR_VALIDATION, "null buffer");
    if ((rc = bind(ctx))) return rc;
    DevBuf src;
    if ((rc = src.alloc(head_len * 4))) return rc;
    QBK_HIP(hipMemcpy(src.p, head, head_len * 4, hipMemcpyHostToDevice));
    return head_build(ctx, (const float *)src.p, vocab, d_model, out);
}

int qbk_head_create_dev(qbk_ctx *ctx, const float *head, size_t vocab, size_t d_model, qbk_head **out) {
    int rc;
    if (!out) return fail(QBK_ERR_VALIDATION, "null output handle");
    *out = nullptr;
    if (vocab == 0 || d_model == 0) return fail(QBK_ERR_VALIDATION, "lm_head requires non-empty vocab and d_model");
    if ((rc = bind(ctx))) return rc;
    return head_build(ctx, head, vocab, d_model, out);
}

void qbk_head_destroy(qbk_head *H) {
    if (!H) return;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(H->device);
    (void)hipFree(H->w);
    (void)hipSetDevice(cur);
    delete H;
}

int qbk_head_info(const qbk_head *H, size_t *vocab, size_t *d_model, int *bf16) {
    if (!H) return fail(QBK_ERR_VALIDATION, "null lm_head");
    if (vocab) *vocab = H->vocab;
    if (d_model) *d_model = H->d_model;
    if (bf16) *bf16 = H->bf16;
    return QBK_OK;
}

int qbk_head_logits(qbk_ctx *ctx, const qbk_head *H, const float *hidden, size_t hidden_len, float *logits,
                    size_t logits_len) {
    int rc;
    if (!H) return fail(QBK_ERR_VALIDATION, "null lm_head");
    if (hidden_len == 0 || hidden_len % H->d_model != 0)
        return fail(QBK_ERR_VALIDATION, fmt("hidden must hold rows of d_model = %zu values, got %zu", H->d_model,
                                            hidden_len));
    const size_t batch = hidden_len / H->d_model;
    if (logits_len != batch * H->vocab)
        return fail(QBK_ERR_VALIDATION, fmt("logits must hold %zu values (%zu rows x vocab %zu), got %zu",
                                            batch * H->vocab, batch, H->vocab, logits_len));
    if (!hidden || !logits) return fail(QBK_ERR_VALIDATION, "null buffer");
    if ((rc = bind(ctx))) return rc;
    if (H->device != ctx->device) return fail(QBK_ERR_VALIDATION, "lm_head lives on another device");
    CallStream cs;
    if ((rc = cs.create())) return rc;
    DevBuf dh, dl;
    if ((rc = dh.alloc(hidden_len * 4)) || (rc = dl.alloc(logits_len * 4))) return rc;
    QBK_HIP(hipMemcpyAsync(dh.p, hidden, hidden_len * 4, hipMemcpyHostToDevice, cs.s));
    if ((rc = head_run(H, (const float *)dh.p, batch, (float *)dl.p, cs.s))) return rc;
    QBK_HIP(hipMemcpyAsync(logits, dl.p, logits_len * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_head_logits_dev(qbk_ctx *ctx, const qbk_head *H, const float *hidden, size_t batch, float *logits,
                        void *stream) {
    int rc;
    if (!H) return fail(QBK_ERR_VALIDATION, "null lm_head");
    if (batch == 0) return fail(QBK_ERR_VALIDATION, "batch must be at least 1");
    if ((rc = bind(ctx))) return rc;
    if (H->device != ctx->device) return fail(QBK_ERR_VALIDATION, "lm_head lives on another device");
    return head_run(H, hidden, batch, logits, (hipStream_t)stream);
}

}  // extern "C"
