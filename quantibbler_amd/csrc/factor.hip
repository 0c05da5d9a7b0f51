// factor.hip -- the binary latent-factor linear on gfx950.
//
//   y = s1 . (Ub (Vb^T (s2 . x))) + b           (engine/mod.rs:393-481)
//
// bf16 serving composite (apply_bf16, engine/mod.rs:449-460), per token:
//   z = bf16(s2*x);  t = bf16(Vb^T z);  u = bf16(Ub t);  y = f32(u)*s1 + b
// with f32 accumulation of the +-1 products.
//
// This file: layer upload and repack, the prefill GEMM (batch > 8), and the
// host faces.  The decode GEMV (batch 1-8) and layer sets are in decode.hip.
//
// A layer is uploaded once and repacked into three device layouts:
//   * ref rows   : the engine's per-row bitplanes (ub_rows, vb_t_rows) for
//                  the f64 serving path (sequential, bit-identical);
//   * q4 words   : (64-row group, 128-k slice) blocks of 64 lane x 4 words
//                  in the fp4 operand order of the scaled MFMA (decode);
//   * mfma frags : the sign matrix cut into (64-row group, 32-k slice)
//                  blocks of 64 lane words, each word holding the bits one
//                  MFMA lane needs for four 16x16x32 bf16 A fragments, so the
//                  kernel expands a fragment with two VALU ops per VGPR and
//                  the wave's 256-byte block load is fully coalesced
//                  (prefill GEMM).
//
// Padded rows of Vb^T produce garbage t values; every consumer of t masks
// k >= r to zero, so padding never reaches the output.
#include <string.h>

#include <vector>

#include "factor_internal.h"

namespace qbk {

// ------------------------------------------------------------------------
// host-side repack
// ------------------------------------------------------------------------

static inline int rbit(const uint8_t *rows, size_t row_words, size_t i, size_t k) {
    return (rows[i * row_words + (k >> 3)] >> (k & 7)) & 1;
}

// mfma fragment word for (group g, slice s, lane l): rows 64g + 16*rt + l%16
// (rt = 0..3), columns 32s + 8*(l/16) + e (e = 0..7); element e of row tile
// rt sits at bit 4*rt + e/2 + 16*(e%2).
static void repack_frag(const uint8_t *rows, size_t n_rows, size_t n_bits, size_t rows_p,
                        size_t bits_p, uint32_t *out) {
    size_t rw = div_ceil(n_bits, 8);
    size_t ns = bits_p / 32, ng = rows_p / 64;
    memset(out, 0, ng * ns * 64 * 4);
    for (size_t g = 0; g < ng; g++)
        for (size_t s = 0; s < ns; s++)
            for (int l = 0; l < 64; l++) {
                uint32_t w = 0;
                for (int rt = 0; rt < 4; rt++) {
                    size_t i = 64 * g + 16 * rt + (l & 15);
                    if (i >= n_rows) continue;
                    for (int e = 0; e < 8; e++) {
                        size_t k = 32 * s + 8 * (l >> 4) + e;
                        if (k < n_bits && rbit(rows, rw, i, k))
                            w |= 1u << (4 * rt + (e >> 1) + 16 * (e & 1));
                    }
                }
                out[(g * ns + s) * 64 + l] = w;
            }
}

// fp4 decode layout.  The scaled 16x16x128 MFMA with an fp4 A operand gives
// lane group g = l/16 the 32 elements k = kq4(g, e) of a 128-k slice, and an
// fp8 B operand gives group g the elements 32g .. 32g+31 (measured pairing).
__host__ __device__ inline int kq4(int g, int e) {
    return 16 * (g >> 1) + 64 * (g & 1) + (e & 15) + 32 * (e >> 4);
}
// Word for (row group rg, slice s, lane l, row tile rt): element e of row
// 64rg + 16rt + l%16 is stored at bit 4*(e%8) + e/8, set when the sign is -1,
// so VGPR v of the fp4 operand is one v_bfi of (word << (3 - v)) into
// 0x22222222 (fp4 e2m1 +1.0 = 0x2, -1.0 = 0xA).
static void repack_q4(const uint8_t *rows, size_t n_rows, size_t n_bits, size_t rows_p,
                      size_t bits_q, uint32_t *out) {
    size_t rw = div_ceil(n_bits, 8);
    size_t ns = bits_q / 128, ng = rows_p / 64;
    memset(out, 0, ng * ns * 64 * 4 * 4);
    for (size_t rg = 0; rg < ng; rg++)
        for (size_t s = 0; s < ns; s++)
            for (int l = 0; l < 64; l++)
                for (int rt = 0; rt < 4; rt++) {
                    size_t i = 64 * rg + 16 * rt + (l & 15);
                    if (i >= n_rows) continue;
                    uint32_t w = 0;
                    for (int e = 0; e < 32; e++) {
                        size_t k = 128 * s + kq4(l >> 4, e);
                        if (k < n_bits && !rbit(rows, rw, i, k)) w |= 1u << (4 * (e & 7) + (e >> 3));
                    }
                    out[((rg * ns + s) * 64 + l) * 4 + rt] = w;
                }
}

// engine/mod.rs:258-289 container_to_rows / container_to_rows_transposed.
static void container_to_rows(const uint8_t *packed, size_t n_rows, size_t r, uint8_t *out) {
    size_t rw = div_ceil(r, 8);
    memset(out, 0, n_rows * rw);
    for (size_t i = 0; i < n_rows; i++)
        for (size_t j = 0; j < r; j++) {
            size_t b = i * r + j;
            if ((packed[b >> 3] >> (b & 7)) & 1) out[i * rw + (j >> 3)] |= (uint8_t)(1u << (j & 7));
        }
}

static void container_to_rows_transposed(const uint8_t *packed, size_t din, size_t r,
                                         uint8_t *out) {
    size_t rw = div_ceil(din, 8);
    memset(out, 0, r * rw);
    for (size_t j = 0; j < din; j++)
        for (size_t k = 0; k < r; k++) {
            size_t b = j * r + k;
            if ((packed[b >> 3] >> (b & 7)) & 1) out[k * rw + (j >> 3)] |= (uint8_t)(1u << (j & 7));
        }
}

static int dev_upload(qbk_factor *L, void **dst, const void *src, size_t n) {
    void *p = nullptr;
    QBK_HIP(hipMalloc(&p, n ? n : 16));
    L->allocs.push_back(p);
    if (n) QBK_HIP(hipMemcpy(p, src, n, hipMemcpyHostToDevice));
    *dst = p;
    return QBK_OK;
}

static void destroy_layer(qbk_factor *L) {
    if (!L) return;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(L->device);
    for (void *p : L->allocs) (void)hipFree(p);
    (void)hipSetDevice(cur);
    delete L;
}

static int build_layer(qbk_ctx *ctx, size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                       const uint8_t *vbt_rows, const float *s1, const float *s2,
                       const float *bias, qbk_factor **out) {
    int rc;
    if ((rc = bind(ctx))) return rc;
    qbk_factor *L = new qbk_factor();
    L->device = ctx->device;
    L->num_cus = ctx->num_cus;
    L->dout = dout;
    L->din = din;
    L->r = r;
    L->din_p = round_up(din, 64);
    L->r_p = round_up(r, 128);
    L->dout_p = round_up(dout, 128);
    std::vector<uint32_t> vf(L->r_p / 64 * L->din_p / 32 * 64), uf(L->dout_p / 64 * L->r_p / 32 * 64);
    repack_frag(vbt_rows, r, din, L->r_p, L->din_p, vf.data());
    repack_frag(ub_rows, dout, r, L->dout_p, L->r_p, uf.data());
    L->din_q = round_up(din, 128);
    L->r_q = round_up(r, 128);
    std::vector<uint32_t> vq(L->r_p / 64 * L->din_q / 128 * 256), uq(L->dout_p / 64 * L->r_q / 128 * 256);
    repack_q4(vbt_rows, r, din, L->r_p, L->din_q, vq.data());
    repack_q4(ub_rows, dout, r, L->dout_p, L->r_q, uq.data());
    std::vector<float> zb(dout, 0.0f);
    void *p;
#define UP(field, src, n)                                                  \
    if ((rc = dev_upload(L, &p, src, n))) {                                \
        destroy_layer(L);                                                  \
        return rc;                                                         \
    }                                                                      \
    L->field = (decltype(L->field))p;
    UP(ub_rows, ub_rows, dout * div_ceil(r, 8));
    UP(vbt_rows, vbt_rows, r * div_ceil(din, 8));
    UP(vt_frag, vf.data(), vf.size() * 4);
    UP(u_frag, uf.data(), uf.size() * 4);
    UP(vt_q4, vq.data(), vq.size() * 4);
    UP(u_q4, uq.data(), uq.size() * 4);
    UP(s1, s1, dout * 4);
    UP(s2, s2, din * 4);
    UP(bias, bias ? bias : zb.data(), dout * 4);
    Q4Layer qtab[2];
    q4_layer_entries(L, qtab);
    UP(q4_tab, qtab, sizeof qtab);
#undef UP
    *out = L;
    return QBK_OK;
}

// ------------------------------------------------------------------------
// prefill GEMM (batch > 1), bf16 MFMA 16x16x32, f32 accumulation
// ------------------------------------------------------------------------
//
// C[M x N] = S[M x K] (+-1) . Act[K x N], Act token-major (Act^T[n][k]).
// Block: 4 waves as WM x WN, wave tile 64 x (BN/WN); BK = 64.
// A: each wave streams its own 64-row group's fragment words straight from
//    HBM into registers (256 B per 32-k slice, coalesced) and expands them
//    (two VALU ops per VGPR) -- no LDS round trip for the sign tiles.
// B: the activation tile is staged through LDS (double buffered, padded
//    rows, conflict-free 16-byte fragment reads), converted on the way in
//    (stage 1: bf16(s2*x); stage 2: bf16(sum of split-K partials), k >= r
//    masked).
// Stage 1 may split K; each split writes f32 partials [split][n][row] that
// stage 2's loader sums in split order before rounding t to bf16.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#define GBK 64
#define BPAD 8  // bf16 elements of padding per LDS row

struct GemmArgs {
    const uint32_t *frag;  // [M_p/64][K_p/32][64]
    size_t M_p, K_p, M_valid, N;
    size_t k_valid;         // columns >= k_valid of Act are zero
    // stage 1 source
    const void *x;          // [N][ldx] bf16 or f32
    size_t ldx;
    const float *s2;
    int vec_ok;             // x rows and s2 allow 16-byte loads
    // stage 2 source: t bf16 [N][ldt], zero for k >= r
    const uint16_t *t_in;
    size_t ldt;
    // outputs
    float *part_out;        // stage 1: [split][N][M_p]
    void *y_out;            // stage 2: [N][ldy]
    size_t ldy;
    const float *s1, *bias;
    int y_bf16;
    size_t k_per_split;     // stage 1 split-K extent (multiple of GBK)
};

__device__ __forceinline__ uint32_t sign_pair(uint32_t nw, int bitpos) {
    uint32_t t = nw << (15 - bitpos);
    return (t & 0x80008000u) | 0x3F803F80u;
}

template <int STAGE, bool XF32, int WM, int WN, int BN>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs A) {
    constexpr int BM = 64 * WM;
    constexpr int WTN = BN / WN;       // wave tile width (tokens)
    constexpr int NT = WTN / 16;       // 16-wide n tiles per wave
    constexpr int LDS_ROW = GBK + BPAD;  // bf16 elements
    __shared__ __attribute__((aligned(16))) uint16_t bs[2][BN * LDS_ROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const size_t n0 = (size_t)blockIdx.x * BN;
    const size_t m0 = (size_t)blockIdx.y * BM;
    const int split = blockIdx.z;
    size_t kb = 0, ke = A.K_p;
    if (STAGE == 1) {
        kb = (size_t)split * A.k_per_split;
        ke = kb + A.k_per_split;
        if (ke > A.K_p) ke = A.K_p;
    }
    const size_t ns = A.K_p / 32;
    const size_t g = m0 / 64 + wm;
    const uint32_t *fr = A.frag + (g * ns) * 64 + lane;

    // B tile loader: BN x GBK elements, 256 threads, 8 elements per chunk.
    constexpr int CHUNKS = BN * GBK / 8;
    constexpr int CPT = (CHUNKS + 255) / 256;
    uint32_t breg[CPT][4];

    auto load_b = [&](size_t k0) {
#pragma unroll
        for (int c = 0; c < CPT; c++) {
            int ci = tid + c * 256;
            if (ci >= CHUNKS) break;
            int nn = ci / (GBK / 8), kk = (ci % (GBK / 8)) * 8;
            size_t n = n0 + nn, k = k0 + kk;
            if (n >= A.N) {
                breg[c][0] = breg[c][1] = breg[c][2] = breg[c][3] = 0;
                continue;
            }
            if (STAGE == 2) {
                // t (bf16, zero beyond r) written by the split-K reduction
                uint4 tv = *(const uint4 *)(A.t_in + n * A.ldt + k);
                breg[c][0] = tv.x;
                breg[c][1] = tv.y;
                breg[c][2] = tv.z;
                breg[c][3] = tv.w;
                continue;
            }
            float xv[8], sv[8];
            if (A.vec_ok && k + 8 <= A.k_valid) {
                if (XF32) {
                    const float4 *xp = (const float4 *)((const float *)A.x + n * A.ldx + k);
                    float4 a0 = xp[0], a1 = xp[1];
                    xv[0] = a0.x; xv[1] = a0.y; xv[2] = a0.z; xv[3] = a0.w;
                    xv[4] = a1.x; xv[5] = a1.y; xv[6] = a1.z; xv[7] = a1.w;
                } else {
                    uint4 xb = *(const uint4 *)((const uint16_t *)A.x + n * A.ldx + k);
                    uint32_t w4[4] = {xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        xv[2 * e] = __uint_as_float(w4[e] << 16);
                        xv[2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
                    }
                }
                const float4 *sp = (const float4 *)(A.s2 + k);
                float4 b0 = sp[0], b1 = sp[1];
                sv[0] = b0.x; sv[1] = b0.y; sv[2] = b0.z; sv[3] = b0.w;
                sv[4] = b1.x; sv[5] = b1.y; sv[6] = b1.z; sv[7] = b1.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    size_t kk2 = k + e;
                    bool ok = kk2 < A.k_valid;
                    xv[e] = !ok ? 0.0f
                                : XF32 ? ((const float *)A.x)[n * A.ldx + kk2]
                                       : bf16_to_f32(((const uint16_t *)A.x)[n * A.ldx + kk2]);
                    sv[e] = ok ? A.s2[kk2] : 0.0f;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
                breg[c][e] = (uint32_t)f32_to_bf16(sv[2 * e] * xv[2 * e]) |
                             ((uint32_t)f32_to_bf16(sv[2 * e + 1] * xv[2 * e + 1]) << 16);
        }
    };
    auto store_b = [&](int buf) {
#pragma unroll
        for (int c = 0; c < CPT; c++) {
            int ci = tid + c * 256;
            if (ci >= CHUNKS) break;
            int nn = ci / (GBK / 8), kk = (ci % (GBK / 8)) * 8;
            uint4 *dst = (uint4 *)&bs[buf][nn * LDS_ROW + kk];
            *dst = make_uint4(breg[c][0], breg[c][1], breg[c][2], breg[c][3]);
        }
    };

    f32x4_t acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[i][j] = f32x4_t{0, 0, 0, 0};

    int buf = 0;
    uint32_t aw[2] = {0, 0};
    if (kb < ke) {
        load_b(kb);
        store_b(0);
        aw[0] = fr[(kb / 32) * 64];
        aw[1] = fr[(kb / 32 + 1) * 64];
    }
    __syncthreads();

    for (size_t k0 = kb; k0 < ke; k0 += GBK) {
        const bool more = k0 + GBK < ke;
        uint32_t an[2] = {0, 0};
        if (more) {
            load_b(k0 + GBK);
            an[0] = fr[((k0 + GBK) / 32) * 64];
            an[1] = fr[((k0 + GBK) / 32 + 1) * 64];
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint32_t nw = ~aw[s];
            bf16x8_t af[4];
#pragma unroll
            for (int rt = 0; rt < 4; rt++) {
                uint32_t v0 = sign_pair(nw, 4 * rt + 0), v1 = sign_pair(nw, 4 * rt + 1);
                uint32_t v2 = sign_pair(nw, 4 * rt + 2), v3 = sign_pair(nw, 4 * rt + 3);
                uint4 u = make_uint4(v0, v1, v2, v3);
                af[rt] = __builtin_bit_cast(bf16x8_t, u);
            }
#pragma unroll
            for (int j = 0; j < NT; j++) {
                int nn = wn * WTN + j * 16 + (lane & 15);
                int kk = s * 32 + (lane >> 4) * 8;
                uint4 bv = *(const uint4 *)&bs[buf][nn * LDS_ROW + kk];
                bf16x8_t bf = __builtin_bit_cast(bf16x8_t, bv);
#pragma unroll
                for (int rt = 0; rt < 4; rt++)
                    acc[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], bf, acc[rt][j], 0, 0, 0);
            }
        }
        if (more) {
            store_b(buf ^ 1);
            aw[0] = an[0];
            aw[1] = an[1];
        }
        __syncthreads();
        buf ^= 1;
    }

    // epilogue: lane holds C[row = 4*(lane/16) + i][col = lane%16] per tile
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            size_t n = n0 + wn * WTN + j * 16 + (lane & 15);
            size_t row = m0 + wm * 64 + rt * 16 + (lane >> 4) * 4;
            if (n >= A.N) continue;
            if (STAGE == 1) {
                float *dst = A.part_out + ((size_t)split * A.N + n) * A.M_p + row;
                *(f32x4_t *)dst = acc[rt][j];
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    size_t rr = row + i;
                    if (rr >= A.M_valid) continue;
                    float u = bf16_to_f32(f32_to_bf16(acc[rt][j][i]));
                    float y = u * A.s1[rr] + A.bias[rr];
                    if (A.y_bf16)
                        ((uint16_t *)A.y_out)[n * A.ldy + rr] = f32_to_bf16(y);
                    else
                        ((float *)A.y_out)[n * A.ldy + rr] = y;
                }
            }
        }
}

// ------------------------------------------------------------------------
// host orchestration
// ------------------------------------------------------------------------

static int splitk_for(const qbk_factor *L, size_t batch, int num_cus) {
    // enough stage-1 blocks to cover the chip: tiles = (r_p/128)*(ceil(N/128))
    size_t tiles = (L->r_p / 128) * div_ceil(batch, 128);
    int s = 1;
    while (tiles * s < (size_t)num_cus && s < 8 && L->din_p / (GBK * 2 * s) >= 4) s *= 2;
    return s;
}

// batch <= Q4_MAXB: the fp4 decode's operand buffers (decode.hip).  Larger
// batches: f32 partials [split][batch][r_p], then t bf16 [batch][r_p].
static size_t ws_bytes(const qbk_factor *L, size_t batch, int split) {
    if (batch <= Q4_MAXB) return q4_workspace(L, batch);
    return round_up((size_t)split * batch * L->r_p * 4, 256) + batch * L->r_p * 2 + 256;
}

// Sum the split-K partials in split order, round to bf16, zero k >= r.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float *__restrict__ part,
                                                            int split, size_t stride,
                                                            size_t ld, size_t r,
                                                            uint16_t *__restrict__ t,
                                                            size_t chunks) {
    size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    size_t e0 = c * 8, k0 = e0 % ld;
    float v[8];
    const float4 *p0 = (const float4 *)(part + e0);
    float4 a = p0[0], b = p0[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    for (int s = 1; s < split; s++) {
        const float4 *ps = (const float4 *)(part + (size_t)s * stride + e0);
        float4 c0 = ps[0], c1 = ps[1];
        v[0] += c0.x; v[1] += c0.y; v[2] += c0.z; v[3] += c0.w;
        v[4] += c1.x; v[5] += c1.y; v[6] += c1.z; v[7] += c1.w;
    }
    uint32_t w[4];
    for (int e = 0; e < 4; e++) {
        uint32_t lo = k0 + 2 * e < r ? f32_to_bf16(v[2 * e]) : 0;
        uint32_t hi = k0 + 2 * e + 1 < r ? f32_to_bf16(v[2 * e + 1]) : 0;
        w[e] = lo | (hi << 16);
    }
    *(uint4 *)(t + e0) = make_uint4(w[0], w[1], w[2], w[3]);
}


template <int STAGE, bool XF32>
static void launch_gemm_cfg(const GemmArgs &a, size_t N, int split, hipStream_t s) {
    if (N <= 32) {
        dim3 g((unsigned)div_ceil(N, 32), (unsigned)(a.M_p / 256), split);
        hipLaunchKernelGGL((gemm_kernel<STAGE, XF32, 4, 1, 32>), g, dim3(256), 0, s, a);
    } else {
        dim3 g((unsigned)div_ceil(N, 128), (unsigned)(a.M_p / 128), split);
        hipLaunchKernelGGL((gemm_kernel<STAGE, XF32, 2, 2, 128>), g, dim3(256), 0, s, a);
    }
}

static int run_gemm(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16,
                    void *ws, int split, hipStream_t s) {
    // M tiles of 256 (small N) need M_p % 256 == 0: r_p/dout_p are multiples
    // of 128, so small-N launches fall back to the 128-row config when odd.
    GemmArgs a{};
    a.frag = L->vt_frag;
    a.M_p = L->r_p;
    a.K_p = L->din_p;
    a.M_valid = L->r;
    a.N = N;
    a.k_valid = L->din;
    a.x = x;
    a.ldx = L->din;
    a.s2 = L->s2;
    a.vec_ok = (L->din % 8) == 0;
    a.part_out = (float *)ws;
    a.k_per_split = round_up(div_ceil(L->din_p, split), GBK);
    bool small = N <= 32;
    if (small && (L->r_p % 256 != 0 || L->dout_p % 256 != 0)) small = false;
    if (small) {
        if (xf32) launch_gemm_cfg<1, true>(a, N, split, s);
        else launch_gemm_cfg<1, false>(a, N, split, s);
    } else {
        dim3 g((unsigned)div_ceil(N, 128), (unsigned)(a.M_p / 128), split);
        if (xf32)
            hipLaunchKernelGGL((gemm_kernel<1, true, 2, 2, 128>), g, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((gemm_kernel<1, false, 2, 2, 128>), g, dim3(256), 0, s, a);
    }
    QBK_HIP(hipGetLastError());
    // t = bf16(sum of the split partials), zero for k >= r
    uint16_t *tb = (uint16_t *)((char *)ws + round_up((size_t)split * N * L->r_p * 4, 256));
    size_t chunks = N * L->r_p / 8;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)div_ceil(chunks, 256)), dim3(256), 0, s,
                       (const float *)ws, split, N * L->r_p, L->r_p, L->r, tb, chunks);
    QBK_HIP(hipGetLastError());
    GemmArgs b{};
    b.frag = L->u_frag;
    b.M_p = L->dout_p;
    b.K_p = L->r_p;
    b.M_valid = L->dout;
    b.N = N;
    b.k_valid = L->r;
    b.t_in = tb;
    b.ldt = L->r_p;
    b.y_out = y;
    b.ldy = L->dout;
    b.s1 = L->s1;
    b.bias = L->bias;
    b.y_bf16 = ybf16;
    if (small) {
        launch_gemm_cfg<2, false>(b, N, 1, s);
    } else {
        dim3 g((unsigned)div_ceil(N, 128), (unsigned)(b.M_p / 128), 1);
        hipLaunchKernelGGL((gemm_kernel<2, false, 2, 2, 128>), g, dim3(256), 0, s, b);
    }
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_factor_from_rows(qbk_ctx *ctx, size_t dout, size_t din, size_t r, const uint8_t *ub_rows,
                         const uint8_t *vb_t_rows, const float *s1, const float *s2,
                         const float *bias, qbk_factor **out) {
    if (!out) return fail(QBK_ERR_VALIDATION, "null output pointer");
    *out = nullptr;
    if (dout == 0 || din == 0 || r == 0)
        return fail(QBK_ERR_VALIDATION,
                    fmt("dout, din and r must all be >= 1, got (%zu, %zu, %zu)", dout, din, r));
    if (!ub_rows || !vb_t_rows || !s1 || !s2) return fail(QBK_ERR_VALIDATION, "null layer field");
    return build_layer(ctx, dout, din, r, ub_rows, vb_t_rows, s1, s2, bias, out);
}

// quantibbler-qpk1 lib.rs:229-320 parse, then engine/mod.rs:342-381 from_layer.
int qbk_factor_from_qpk1(qbk_ctx *ctx, const uint8_t *b, size_t len, qbk_factor **out) {
    if (!out) return fail(QBK_ERR_VALIDATION, "null output pointer");
    *out = nullptr;
    if (len < 24)
        return fail(QBK_ERR_VALIDATION,
                    fmt("stream is %zu bytes; shorter than the 24-byte header", len));
    if (memcmp(b, "QPK1", 4) != 0)
        return fail(QBK_ERR_VALIDATION, fmt("bad magic [%u, %u, %u, %u]; expected [81, 80, 75, 49]",
                                            b[0], b[1], b[2], b[3]));
    auto rd = [&](size_t o) {
        return (uint32_t)b[o] | ((uint32_t)b[o + 1] << 8) | ((uint32_t)b[o + 2] << 16) |
               ((uint32_t)b[o + 3] << 24);
    };
    uint32_t version = rd(4), tag = rd(8);
    if (version != 1 && version != 2)
        return fail(QBK_ERR_VALIDATION,
                    fmt("unsupported representation version %u; this reader implements version 1 "
                        "(pre-bias legacy) and version 2 (current, with bias)",
                        version));
    if (tag != 1 && tag != 2)
        return fail(QBK_ERR_VALIDATION,
                    fmt("unknown dtype tag %u; expected 1 (float16) or 2 (float32)", tag));
    size_t dout = rd(12), din = rd(16), r = rd(20);
    if (dout == 0 || din == 0 || r == 0)
        return fail(QBK_ERR_VALIDATION,
                    fmt("dout, din and r must all be >= 1, got (%zu, %zu, %zu)", dout, din, r));
    size_t item = tag == 1 ? 2 : 4;
    bool has_bias = version >= 2;
    size_t floats = has_bias ? 2 * dout + din : dout + din;
    size_t expected = 24 + floats * item + div_ceil(dout * r, 8) + div_ceil(din * r, 8);
    if (len < expected)
        return fail(QBK_ERR_VALIDATION,
                    fmt("truncated stream: %zu bytes; header declares %zu", len, expected));
    if (len > expected)
        return fail(QBK_ERR_VALIDATION,
                    fmt("trailing garbage: %zu bytes; one layer at this header is %zu", len,
                        expected));
    auto decode = [&](size_t off, size_t n, std::vector<float> &dst) {
        dst.resize(n);
        for (size_t i = 0; i < n; i++) {
            if (item == 2) {
                uint16_t h = (uint16_t)(b[off + 2 * i] | (b[off + 2 * i + 1] << 8));
                uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
                float v;
                if (e == 0) {
                    v = (float)m * 5.9604644775390625e-08f;
                    if (sign) v = -v;
                } else {
                    uint32_t u = sign | (e == 31 ? (0x7f800000u | (m << 13)) : (((e + 112u) << 23) | (m << 13)));
                    memcpy(&v, &u, 4);
                }
                dst[i] = v;
            } else {
                uint32_t u = rd(off + 4 * i);
                float v;
                memcpy(&v, &u, 4);
                dst[i] = v;
            }
        }
    };
    std::vector<float> s1, s2, bias;
    size_t off = 24;
    decode(off, dout, s1);
    off += dout * item;
    decode(off, din, s2);
    off += din * item;
    if (has_bias) {
        decode(off, dout, bias);
        off += dout * item;
    }
    const uint8_t *ub = b + off;
    const uint8_t *vb = ub + div_ceil(dout * r, 8);
    std::vector<uint8_t> ub_rows(dout * div_ceil(r, 8)), vbt_rows(r * div_ceil(din, 8));
    container_to_rows(ub, dout, r, ub_rows.data());
    container_to_rows_transposed(vb, din, r, vbt_rows.data());
    return build_layer(ctx, dout, din, r, ub_rows.data(), vbt_rows.data(), s1.data(), s2.data(),
                       has_bias ? bias.data() : nullptr, out);
}

void qbk_factor_destroy(qbk_factor *layer) { destroy_layer(layer); }

int qbk_factor_dims(const qbk_factor *L, size_t *dout, size_t *din, size_t *r) {
    if (!L) return fail(QBK_ERR_VALIDATION, "null layer");
    if (dout) *dout = L->dout;
    if (din) *din = L->din;
    if (r) *r = L->r;
    return QBK_OK;
}

size_t qbk_factor_workspace_size(const qbk_factor *L, size_t batch) {
    if (!L) return 0;
    return ws_bytes(L, batch, batch <= 1 ? 1 : splitk_for(L, batch, L->num_cus));
}

int qbk_factor_linear_dev(qbk_ctx *ctx, const qbk_factor *L, const uint16_t *x, size_t batch,
                          void *y, int y_dtype, void *workspace, size_t workspace_size,
                          void *stream) {
    int rc;
    if (!L) return fail(QBK_ERR_VALIDATION, "null layer");
    if (y_dtype != QBK_F32 && y_dtype != QBK_BF16)
        return fail(QBK_ERR_VALIDATION, "y_dtype must be QBK_F32 or QBK_BF16");
    if (batch == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    if (L->device != ctx->device)
        return fail(QBK_ERR_VALIDATION, "layer lives on another device than the context");
    int split = batch <= 1 ? 1 : splitk_for(L, batch, ctx->num_cus);
    size_t need = ws_bytes(L, batch, split);
    if (workspace_size < need)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs",
                        workspace_size, need));
    hipStream_t s = (hipStream_t)stream;
    if (batch <= Q4_MAXB) return q4_run(L, batch, x, false, y, y_dtype == QBK_BF16, workspace, s);
    return run_gemm(L, x, false, batch, y, y_dtype == QBK_BF16, workspace, split, s);
}

// engine/mod.rs:393-460 apply / apply_bf16 with host buffers.
int qbk_factor_apply(qbk_ctx *ctx, const qbk_factor *L, int serving, const float *x, size_t batch,
                     float *y) {
    int rc;
    if (!L) return fail(QBK_ERR_VALIDATION, "null layer");
    if (serving != QBK_F32 && serving != QBK_BF16)
        return fail(QBK_ERR_VALIDATION, "serving dtype must be QBK_F32 or QBK_BF16");
    if (batch == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    CallStream cs;
    if ((rc = cs.create())) return rc;
    if (serving == QBK_F32) {
        // z = f64(s2*x) on the host (f32 multiply, widen), then the two f64
        // matvecs in element order on the device, y = f32(u)*s1 + b.
        std::vector<float> s1(L->dout), s2(L->din), bias(L->dout);
        QBK_HIP(hipMemcpy(s1.data(), L->s1, L->dout * 4, hipMemcpyDeviceToHost));
        QBK_HIP(hipMemcpy(s2.data(), L->s2, L->din * 4, hipMemcpyDeviceToHost));
        QBK_HIP(hipMemcpy(bias.data(), L->bias, L->dout * 4, hipMemcpyDeviceToHost));
        DevBuf dz, dt, du;
        if ((rc = dz.alloc(L->din * 8)) || (rc = dt.alloc(L->r * 8)) || (rc = du.alloc(L->dout * 8)))
            return rc;
        std::vector<double> z(L->din), u(L->dout);
        for (size_t bb = 0; bb < batch; bb++) {
            const float *xb = x + bb * L->din;
            for (size_t j = 0; j < L->din; j++) z[j] = (double)(s2[j] * xb[j]);
            QBK_HIP(hipMemcpyAsync(dz.p, z.data(), L->din * 8, hipMemcpyHostToDevice, cs.s));
            if ((rc = qbk_packed_matvec_dev(ctx, QBK_F64, L->vbt_rows, L->r, L->din, dz.p, dt.p, cs.s)))
                return rc;
            if ((rc = qbk_packed_matvec_dev(ctx, QBK_F64, L->ub_rows, L->dout, L->r, dt.p, du.p, cs.s)))
                return rc;
            QBK_HIP(hipMemcpyAsync(u.data(), du.p, L->dout * 8, hipMemcpyDeviceToHost, cs.s));
            QBK_HIP(hipStreamSynchronize(cs.s));
            float *yb = y + bb * L->dout;
            for (size_t i = 0; i < L->dout; i++) yb[i] = ((float)u[i]) * s1[i] + bias[i];
        }
        return QBK_OK;
    }
    int split = batch <= 1 ? 1 : splitk_for(L, batch, ctx->num_cus);
    DevBuf dx, dy, dws;
    if ((rc = dx.alloc(batch * L->din * 4)) || (rc = dy.alloc(batch * L->dout * 4)) ||
        (rc = dws.alloc(ws_bytes(L, batch, split))))
        return rc;
    QBK_HIP(hipMemcpyAsync(dx.p, x, batch * L->din * 4, hipMemcpyHostToDevice, cs.s));
    if (batch <= Q4_MAXB)
        rc = q4_run(L, batch, dx.p, true, dy.p, false, dws.p, cs.s);
    else
        rc = run_gemm(L, dx.p, true, batch, dy.p, false, dws.p, split, cs.s);
    if (rc) return rc;
    QBK_HIP(hipMemcpyAsync(y, dy.p, batch * L->dout * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

}  // extern "C"
