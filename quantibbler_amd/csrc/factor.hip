// factor.hip -- the binary latent-factor linear on gfx950.
//
//   y = s1 . (Ub (Vb^T (s2 . x))) + b           (engine/mod.rs:393-481)
//
// bf16 serving composite (apply_bf16, engine/mod.rs:449-460), per token:
//   z = bf16(s2*x);  t = bf16(Vb^T z);  u = bf16(Ub t);  y = f32(u)*s1 + b
// with f32 accumulation of the +-1 products.
//
// A layer is uploaded once and repacked into three device layouts:
//   * ref rows   : the engine's per-row bitplanes (ub_rows, vb_t_rows) for
//                  the f64 serving path (sequential, bit-identical);
//   * gemv words : rows of 32-bit words, K padded to a multiple of 256 bits,
//                  the bits of each word pair-permuted so one v_bfi builds a
//                  bf16 +-1 pair for v_dot2_f32_bf16 (decode, batch 1);
//   * mfma frags : the sign matrix cut into (64-row group, 32-k slice)
//                  blocks of 64 lane words, each word holding the bits one
//                  MFMA lane needs for four 16x16x32 bf16 A fragments, so the
//                  kernel expands a fragment with two VALU ops per VGPR and
//                  the wave's 256-byte block load is fully coalesced
//                  (prefill GEMM, batch > 1).
//
// Padded rows of Vb^T produce garbage t values; every consumer of t masks
// k >= r to zero, so padding never reaches the output.
#include <string.h>

#include <vector>

#include "qbk_internal.h"

namespace qbk {
// Per-layer operands of one decode GEMV stage (bits in the fp4 decode
// layout): an entry of a device-side table, so one launch covers any number
// of layers of one shape.
struct Q4Layer {
    const uint32_t *bits;
    const float *s_in;
    const float *s_out;
    const float *bias;
};

}  // namespace qbk

struct qbk_factor {
    int device, num_cus;
    size_t dout, din, r;
    size_t din_p, r_p, dout_p;  // padded for the MFMA tiles (64 / 128 / 128)
    uint8_t *ub_rows, *vbt_rows;      // reference per-row bitplanes
    uint32_t *vt_frag, *u_frag;       // [r_p/64][din_p/32][64], [dout_p/64][r_p/32][64]
    size_t din_q, r_q;                // K of the fp4 decode layout: multiples of 128
    uint32_t *vt_q4, *u_q4;           // [r_p/64][din_q/128][64][4], [dout_p/64][r_q/128][64][4]
    float *s1, *s2, *bias;            // dout, din, dout (zeros when absent)
    void *q4_tab;              // device Q4Layer[2]: [0] stage 1, [1] stage 2
    std::vector<void *> allocs;
};

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
    Q4Layer qtab[2] = {{L->vt_q4, L->s2, nullptr, nullptr}, {L->u_q4, nullptr, L->s1, L->bias}};
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
// decode GEMV on the scaled fp4 x fp8 MFMA (batch 1..8)
// ------------------------------------------------------------------------
//
// out[i] = sum_k s(i,k) a_k as C = A.B with v_mfma_scale_f32_16x16x128_f8f6f4:
// A = the +-1 signs as fp4 e2m1 (exact), built from the bits with one shift
// and one v_bfi per 8 weights; B = the activations split exactly into two
// fp8 e4m3 columns, a = hi*2^e_hi + lo*2^e_lo, with one E8M0 scale per
// 32-element block and column (a bf16 value has 8 significant bits: hi keeps
// the top 4, lo the rest).  Token b of a decode batch uses columns 2b, 2b+1;
// the product sums exactly-represented terms in f32, and out = C[.,2b] +
// C[.,2b+1].  Each 128-k slice of a 16-row tile is one MFMA over 256 bytes
// of packed signs.

#define Q4_MAXB 8
#define Q4_U 8  // slices whose sign loads a wave issues together
#define Q4_PHASES 3  // prep x, stage 1 (+ stage 2's operand), stage 2

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Pointers read from a layer table are generic to the compiler; loading
// through an address_space(1) pointer keeps them global loads (flat loads
// count against both vmcnt and lgkmcnt and defeat per-load waits).
typedef __attribute__((address_space(1))) const u32x4_t gu32x4_t;
typedef __attribute__((address_space(1))) const float gf32_t;
// The layer tables are never written by a kernel: reading them through the
// constant address space lets the compiler use scalar loads even after the
// kernel's own stores (a vector load of a pointer would wait on vmcnt).
typedef __attribute__((address_space(4))) const Q4Layer cq4layer_t;

// B operand of one (layer, slice, lane group, column): 32 fp8 bytes + scale.
struct Q4Args {
    const Q4Layer *layers;
    size_t rows_p, rows_valid, k_valid, ns;  // ns = K_q / 128
    int batch, ncol;                          // ncol = 2 * batch
    const void *act;                          // stage 1: x bf16 [layer][batch][ldx]; stage 2: t bf16
    size_t act_ld, act_layer;                 // elements per token row, per layer
    uint8_t *bop;                             // [layer][ns][4][ncol][32]
    uint8_t *bsc;                             // [layer][ns][4][ncol]
    void *out;                                // stage 2: y [layer][batch][out_ld]
    size_t out_ld, out_layer;
    int y_bf16;
    int vec_ok;                               // act rows allow 4-element vector loads
    uint32_t c7;                              // 0x77777777 (fp4 sign build)
    uint8_t *tb_op, *tb_sc;                   // stage 1: stage 2's operand and scales
    size_t tb_ns;                             // stage 2's slices per layer
    uint32_t wg_per_layer, n_layers;          // GEMV grid: workgroups per layer, layers
};

__device__ __forceinline__ int e8m0_of(float amax) {
    // exponent so that amax * 2^-e lies in [128, 256): e = floor(log2 amax) - 7
    int ex = (int)((__float_as_uint(amax) >> 23) & 0xff) - 127;
    int e = ex - 7;
    return e < -126 ? -126 : (e > 126 ? 126 : e);
}

__device__ __forceinline__ float pow2f(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// x -> stage 1's fp8 operand.  One thread per run of 16 activations:
// (layer, token, slice s, run r) covers k = 128s + 16r .. +15.  The E8M0
// scale given by MFMA lane group G covers the activations k = 128s +
// kq4(G, e) (measured on gfx950): the two runs 16(G>>1) + 64(G&1) + {0, 32},
// i.e. runs r and r^2 with G = 2(r&1) + (r>>2), so the block max is one
// shuffle away.  Run r's bytes go to B lane group 2(r>>2) + ((r>>1)&1) at
// byte offset 16(r&1): one uint4 for hi (column 2b), one for lo (2b + 1).
// z = bf16(s2 * x) splits exactly into hi + lo: each fp8 e4m3 part keeps 4
// significant bits relative to the block max's exponent.
template <bool XF32>
__global__ void __launch_bounds__(256) q4_prep_kernel(Q4Args a, size_t n_runs) {
    const size_t it = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = it < n_runs;  // dead threads still join the shuffle
    const size_t itc = live ? it : 0;
    const int r = (int)(itc & 7);
    size_t rest = itc >> 3;
    const size_t s = rest % a.ns;
    rest /= a.ns;
    const int b = (int)(rest % a.batch);
    const size_t li = rest / a.batch;
    const size_t k0 = 128 * s + 16 * r;
    float z[16];
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    if (live) {
        const size_t off = li * a.act_layer + (size_t)b * a.act_ld;
        const uint16_t *src = (const uint16_t *)a.act + off;
        const float *srcf = (const float *)a.act + off;
        const float *s2 = ((const cq4layer_t *)a.layers + li)->s_in;
        if (a.vec_ok && k0 + 15 < a.k_valid) {
            float v[16];
            if (XF32) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 f = *(const float4 *)(srcf + k0 + 4 * q);
                    v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const uint4 u = *(const uint4 *)(src + k0 + 8 * q);
                    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int h = 0; h < 4; h++) {
                        v[8 * q + 2 * h] = bf16_to_f32(w[h] & 0xffff);
                        v[8 * q + 2 * h + 1] = bf16_to_f32(w[h] >> 16);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 f = *(const float4 *)(s2 + k0 + 4 * q);
                z[4 * q] = bf16_to_f32(f32_to_bf16(f.x * v[4 * q]));
                z[4 * q + 1] = bf16_to_f32(f32_to_bf16(f.y * v[4 * q + 1]));
                z[4 * q + 2] = bf16_to_f32(f32_to_bf16(f.z * v[4 * q + 2]));
                z[4 * q + 3] = bf16_to_f32(f32_to_bf16(f.w * v[4 * q + 3]));
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const size_t k = k0 + e;
                if (k >= a.k_valid) continue;
                const float v = XF32 ? srcf[k] : bf16_to_f32(src[k]);
                z[e] = bf16_to_f32(f32_to_bf16(s2[k] * v));
            }
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(z[e]));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    const int e_hi = amax > 0.0f ? e8m0_of(amax) : 0;
    const float inv_hi = pow2f(-e_hi), sc_hi = pow2f(e_hi);
    uint32_t hw[4], lw[4];
    float rmax = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(z[4 * q] * inv_hi, z[4 * q + 1] * inv_hi, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(z[4 * q + 2] * inv_hi, z[4 * q + 3] * inv_hi, w, true);
        hw[q] = (uint32_t)w;
        z[4 * q] -= __builtin_amdgcn_cvt_f32_fp8(w, 0) * sc_hi;  // exact residuals
        z[4 * q + 1] -= __builtin_amdgcn_cvt_f32_fp8(w, 1) * sc_hi;
        z[4 * q + 2] -= __builtin_amdgcn_cvt_f32_fp8(w, 2) * sc_hi;
        z[4 * q + 3] -= __builtin_amdgcn_cvt_f32_fp8(w, 3) * sc_hi;
#pragma unroll
        for (int u = 0; u < 4; u++) rmax = fmaxf(rmax, fabsf(z[4 * q + u]));
    }
    rmax = fmaxf(rmax, __shfl_xor(rmax, 2, 64));
    const int e_lo = rmax > 0.0f ? e8m0_of(rmax) : 0;
    const float inv_lo = pow2f(-e_lo);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(z[4 * q] * inv_lo, z[4 * q + 1] * inv_lo, 0, false);
        lw[q] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(z[4 * q + 2] * inv_lo, z[4 * q + 3] * inv_lo, w, true);
    }
    if (!live) return;
    const size_t gb = 2 * (r >> 2) + ((r >> 1) & 1);
    const size_t slot = ((li * a.ns + s) * 4 + gb) * a.ncol + 2 * b;  // hi column; lo is slot + 1
    const size_t byte = 16 * (r & 1);
    *(uint4 *)(a.bop + slot * 32 + byte) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(a.bop + (slot + 1) * 32 + byte) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if ((r & 2) == 0) {
        const size_t sc = ((li * a.ns + s) * 4 + 2 * (r & 1) + (r >> 2)) * a.ncol + 2 * b;
        a.bsc[sc] = (uint8_t)(e_hi + 127);
        a.bsc[sc + 1] = (uint8_t)(e_lo + 127);
    }
}

// Signs of one 16-row tile as fp4 e2m1: nibble e of VGPR j carries bit
// 4e + 3 - j of the word in its sign bit, and OR-ing 0x7 into every nibble
// forces the other three bits to 1 whatever the shift brought in, so each
// element is exactly +-6 (e2m1 0111 = 1.5 * 2^2).  One VALU op per VGPR
// (v_lshl_or_b32 with c7 = 0x77777777 in an SGPR; v_or_b32 for j = 3).  The
// MFMA's A scale 2^-2 (E8M0 125) makes the elements +-1.5, and the epilogue
// divides by 1.5: exact whenever the f32 sum is (1.5 * sum then needs one
// more significant bit).
#define Q4_SCALE_A 125
__device__ __forceinline__ i32x8_t q4_signs(uint32_t w, uint32_t c7) {
    i32x8_t av;
    av[0] = (int)((w << 3) | c7);
    av[1] = (int)((w << 2) | c7);
    av[2] = (int)((w << 1) | c7);
    av[3] = (int)(w | c7);
    av[4] = av[5] = av[6] = av[7] = 0;
    return av;
}

// One 128-k slice of a 64-row group: the four row tiles' MFMAs against the
// fp8 operand held in LDS at byte offset bo (scale byte at so).
__device__ __forceinline__ void q4_slice_lds(f32x4_t acc[4], const uint4 &w4, const uint8_t *lds,
                                             uint32_t bo, uint32_t so, uint32_t c7) {
    const uint4 *bq = (const uint4 *)(lds + bo);
    const uint4 b0 = bq[0], b1 = bq[1];
    const i32x8_t bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                        (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    const int bs = lds[so];
    const uint32_t wr[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
        acc[rt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q4_signs(wr[rt], c7), bv, acc[rt],
                                                                  4, 0, 0, Q4_SCALE_A, 0, bs);
}

// Epilogue of one 64-row group, one row per lane: the accumulators are
// transposed through the wave's LDS region T [ncol][64] (lane (col, g) holds
// rows 16rt + 4g + i of column col), then lane l finishes row rg*64 + l of
// every token: v = (hi + lo) / 1.5 (the A scale of q4_signs).
//
// Stage 1 writes t = bf16(v) (0 past rows_valid) as stage 2's fp8 operand:
// row l of the group is element e = (l & 15) + 16 (l >> 5) of scale group
// G = 2((l >> 4) & 1) + (rg & 1) of stage-2 slice rg/2 (the 32 rows sharing
// G differ in lane bits 0-3 and 5, so the block max is five xor shuffles);
// its bytes go to B lane group 2(rg & 1) + (l >> 5), byte 16((l >> 4) & 1) +
// (l & 15), hi to column 2b and lo to 2b + 1.
//
// Stage 2 writes y = bf16(v) * s1 + bias (so / bi: this lane's row).
template <int STAGE>
__device__ __forceinline__ void q4_epilogue(const f32x4_t acc[4], float *T, const Q4Args &a, int ncol,
                                            size_t li, size_t rg, int lane, float so, float bi) {
    const int col = lane & 15, g = lane >> 4;
    if (col < ncol) {
#pragma unroll
        for (int rt = 0; rt < 4; rt++) *(f32x4_t *)(T + col * 64 + 16 * rt + 4 * g) = acc[rt];
    }
    __builtin_amdgcn_wave_barrier();
    const size_t row = rg * 64 + lane;
    const bool valid = row < a.rows_valid;
    for (int b = 0; b < (ncol >> 1); b++) {
        const float v = (T[(2 * b) * 64 + lane] + T[(2 * b + 1) * 64 + lane]) / 1.5f;
        const float t = valid ? bf16_to_f32(f32_to_bf16(v)) : 0.0f;
        if (STAGE == 2) {
            if (valid) {
                const float y = t * so + bi;
                const size_t o = li * a.out_layer + (size_t)b * a.out_ld + row;
                if (a.y_bf16)
                    ((uint16_t *)a.out)[o] = f32_to_bf16(y);
                else
                    ((float *)a.out)[o] = y;
            }
            continue;
        }
        float amax = fabsf(t);
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 8, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
        const int e_hi = amax > 0.0f ? e8m0_of(amax) : 0;
        const int hw = __builtin_amdgcn_cvt_pk_fp8_f32(t * pow2f(-e_hi), 0.0f, 0, false);
        const float r = t - __builtin_amdgcn_cvt_f32_fp8(hw, 0) * pow2f(e_hi);  // exact residual
        float rmax = fabsf(r);
        rmax = fmaxf(rmax, __shfl_xor(rmax, 1, 64));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 2, 64));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 4, 64));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 8, 64));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
        const int e_lo = rmax > 0.0f ? e8m0_of(rmax) : 0;
        const int lw = __builtin_amdgcn_cvt_pk_fp8_f32(r * pow2f(-e_lo), 0.0f, 0, false);
        const int q = (lane >> 4) & 1, h = lane >> 5;
        const size_t base = (li * a.tb_ns + (rg >> 1)) * 4;
        const size_t slot = (base + 2 * (rg & 1) + h) * ncol + 2 * b;  // hi column; lo = +1
        const size_t byte = 16 * q + (lane & 15);
        a.tb_op[slot * 32 + byte] = (uint8_t)hw;
        a.tb_op[(slot + 1) * 32 + byte] = (uint8_t)lw;
        if ((lane & 47) == 0) {  // lanes 0 and 16: scale groups 2q + (rg & 1)
            const size_t sc = (base + 2 * q + (rg & 1)) * ncol + 2 * b;
            a.tb_sc[sc] = (uint8_t)(e_hi + 127);
            a.tb_sc[sc + 1] = (uint8_t)(e_lo + 127);
        }
    }
}

// Slice j of a step: the fp8 operand from the wave's staged LDS region
// (NCOL > 0) or from global memory (NCOL == 0), then the four MFMAs.
template <int NCOL>
__device__ __forceinline__ void q4_step(f32x4_t acc[4], const uint4 &w4u, uint32_t j, const uint8_t *wl,
                                        uint32_t bo0, uint32_t bstep, uint32_t so0, uint32_t sstep,
                                        const uint8_t *gb, const uint8_t *gs, size_t sb, int g, int ncol,
                                        int col, bool bcol, uint32_t c7) {
    if (NCOL > 0) {
        q4_slice_lds(acc, w4u, wl, bo0 + j * bstep, so0 + j * sstep, c7);
        return;
    }
    i32x8_t bv = {0, 0, 0, 0, 0, 0, 0, 0};
    int bs = 127;
    if (bcol) {
        const size_t slot = ((sb + j) * 4 + g) * ncol + col;
        const uint4 *bq = (const uint4 *)(gb + slot * 32);
        const uint4 b0 = bq[0], b1 = bq[1];
        bv = i32x8_t{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        bs = gs[slot];
    }
    const uint32_t wr[4] = {w4u.x, w4u.y, w4u.z, w4u.w};
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
        acc[rt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q4_signs(wr[rt], c7), bv, acc[rt], 4, 0, 0,
                                                                  Q4_SCALE_A, 0, bs);
}

// LDS bytes of one wave's region: the staged operand of Q4_U slices (NCOL
// columns), their scales (one dword per lane), a zero slot, and room for the
// epilogue's transpose.
__host__ __device__ constexpr uint32_t q4_wave_lds(int ncol) {
    return ncol > 0 ? (uint32_t)(Q4_U * 4 * ncol * 32 + 256 + 48) : 16 * 64 * 4;
}

// Decode GEMV.  Workgroup = 4 waves; KSPLIT waves share a 64-row group and
// split its slices (4/KSPLIT row groups per workgroup).  Lane l loads the 16
// bytes of its four row tiles' sign words per slice (1 KiB per wave per
// slice, contiguous over the slices); Q4_U slices are loaded per step.
//
// NCOL > 0 (batch 1-2): each wave stages the fp8 operand of its own slices
// through registers into its LDS region -- operand loads issued first, sign
// loads right behind them, no workgroup barrier -- and reads it per slice;
// lanes past the batch's columns read a zero slot.  NCOL == 0 (batch 3-8):
// lanes read the operand of each slice from global memory (L2).
//
// Loads are unconditional (indices clamped into the layer; the MFMAs of
// clamped slices are skipped) so that the compiler's wait counts stay exact:
// each slice's MFMAs start as soon as its own load lands.
template <int STAGE, int KSPLIT, int NCOL>
__global__ void __launch_bounds__(256) q4_gemv_kernel(Q4Args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t q4_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
    const int ncol = NCOL > 0 ? NCOL : a.ncol;
    // XCD-aware 1D grid: workgroup i runs on XCD i % 8; XCD x takes the
    // contiguous workgroup range [x*per_x, (x+1)*per_x) of the (layer, row
    // group) order, so that one layer's operand is fetched into one L2.
    const uint32_t xcd = blockIdx.x & 7, per_x = gridDim.x >> 3;
    const size_t wgi = (size_t)xcd * per_x + (blockIdx.x >> 3);
    if (wgi >= (size_t)a.wg_per_layer * a.n_layers) return;  // padding workgroup
    const size_t li = wgi / a.wg_per_layer;
    const cq4layer_t *lp = (const cq4layer_t *)a.layers + li;
    const Q4Layer L = {lp->bits, lp->s_in, lp->s_out, lp->bias};
    constexpr int RG_PER_WG = 4 / KSPLIT;
    const size_t rg = (wgi - li * a.wg_per_layer) * RG_PER_WG + wave / KSPLIT;
    const int ks = wave % KSPLIT;
    const size_t n_rg = a.rows_p / 64;
    const size_t per = (a.ns + KSPLIT - 1) / KSPLIT;
    const size_t s0 = ks * per < a.ns ? ks * per : a.ns;
    const size_t s1 = s0 + per < a.ns ? s0 + per : a.ns;
    const int col = lane & 15, g = lane >> 4;
    const bool bcol = col < ncol;
    const bool live = rg < n_rg;
    const size_t rgc = live ? rg : n_rg - 1;
    const uint32_t c7 = a.c7;
    const uint32_t wreg = q4_wave_lds(NCOL);  // the launch allocates 4 * this (+ red)
    uint8_t *wl = q4_lds + wave * wreg;
    const size_t opl = a.ns * 4 * ncol * 32, scl = a.ns * 4 * ncol;  // per layer
    const uint8_t *gb = a.bop + li * opl;
    const uint8_t *gs = a.bsc + li * scl;

    // staged operand offsets within the wave's region (slice j of the step)
    constexpr uint32_t OPB = NCOL > 0 ? Q4_U * 4 * NCOL * 32 : 0;
    constexpr uint32_t ZS = OPB + 256;
    const uint32_t slot0 = (uint32_t)(g * ncol + col);
    const uint32_t bo0 = bcol ? slot0 * 32 : ZS, bstep = bcol ? 4 * ncol * 32 : 0;
    const uint32_t so0 = bcol ? OPB + slot0 : ZS + 32, sstep = bcol ? 4 * ncol : 0;
    if (NCOL > 0) {
        if (lane < 2) *(uint4 *)(wl + ZS + 16 * lane) = make_uint4(0, 0, 0, 0);
        if (lane == 2) wl[ZS + 32] = 127;
    }

    // stage 2: this lane's row of the group, for the epilogue
    float so = 0.0f, bi = 0.0f;
    if (STAGE == 2) {
        const size_t row = rgc * 64 + lane;
        const size_t rc = row < a.rows_valid ? row : a.rows_valid - 1;
        so = ((gf32_t *)L.s_out)[rc];
        bi = ((gf32_t *)L.bias)[rc];
    }

    const uint4 *wp = (const uint4 *)L.bits + (rgc * a.ns) * 64 + lane;
    f32x4_t acc[4];
#pragma unroll
    for (int rt = 0; rt < 4; rt++) acc[rt] = f32x4_t{0, 0, 0, 0};
    for (size_t sb = s0; sb < s1; sb += Q4_U) {
        const uint32_t nsl = (uint32_t)(s1 - sb < Q4_U ? s1 - sb : Q4_U);
        uint4 stg[NCOL > 0 ? NCOL : 1];
        uint32_t stgs = 0;
        if (NCOL > 0) {
            // operand of slices sb..sb+nsl-1: NCOL uint4 + one dword of scales per lane
            const uint32_t ob = nsl * 4 * NCOL * 32, os = nsl * 4 * NCOL;
            const uint8_t *gbs = gb + sb * 4 * NCOL * 32, *gss = gs + sb * 4 * NCOL;
#pragma unroll
            for (int q = 0; q < (NCOL > 0 ? NCOL : 1); q++) {
                uint32_t o = (lane + 64 * q) * 16;
                o = o < ob ? o : ob - 16;
                stg[q] = *(const uint4 *)(gbs + o);
            }
            uint32_t o = lane * 4;
            o = o < os ? o : os - 4;
            stgs = *(const uint32_t *)(gss + o);
        }
        uint4 w4[Q4_U];
#pragma unroll
        for (int u = 0; u < Q4_U; u++) {
            const size_t sl = sb + (u < (int)nsl ? u : nsl - 1);
            const u32x4_t q = __builtin_nontemporal_load((gu32x4_t *)(wp + sl * 64));
            w4[u] = make_uint4(q[0], q[1], q[2], q[3]);
        }
        if (NCOL > 0) {
#pragma unroll
            for (int q = 0; q < (NCOL > 0 ? NCOL : 1); q++) *(uint4 *)(wl + (lane + 64 * q) * 16) = stg[q];
            *(uint32_t *)(wl + OPB + lane * 4) = stgs;  // lanes past the scales fill the padding
            __builtin_amdgcn_wave_barrier();
        }
        if (nsl == Q4_U) {
#pragma unroll
            for (int u = 0; u < Q4_U; u++)
                q4_step<NCOL>(acc, w4[u], u, wl, bo0, bstep, so0, sstep, gb, gs, sb, g, ncol, col, bcol, c7);
        } else {
#pragma unroll
            for (int u = 0; u < Q4_U; u++)
                if (u < (int)nsl)
                    q4_step<NCOL>(acc, w4[u], u, wl, bo0, bstep, so0, sstep, gb, gs, sb, g, ncol, col, bcol, c7);
        }
        if (NCOL > 0) __builtin_amdgcn_wave_barrier();  // the next step overwrites the region
    }
    if (KSPLIT > 1) {
        f32x4_t *red = (f32x4_t *)(q4_lds + 4 * wreg);  // [4 waves][4 tiles][64 lanes]
#pragma unroll
        for (int rt = 0; rt < 4; rt++) red[(wave * 4 + rt) * 64 + lane] = acc[rt];
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int rt = 0; rt < 4; rt++) {
            f32x4_t v = red[(wave * 4 + rt) * 64 + lane];
            for (int q = 1; q < KSPLIT; q++) v += red[((wave + q) * 4 + rt) * 64 + lane];
            acc[rt] = v;
        }
    }
    if (!live) return;
    q4_epilogue<STAGE>(acc, (float *)wl, a, ncol, li, rg, lane, so, bi);
}

// LDS bytes of a q4_gemv_kernel workgroup.
static size_t q4_gemv_lds(int ncol_t, int ksplit) {
    return 4 * (size_t)q4_wave_lds(ncol_t) + (ksplit > 1 ? 4 * 4 * 64 * 16 : 0);
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

// batch 1: t bf16 [r_p].  batch > 1: f32 partials [split][batch][r_p], then
// t bf16 [batch][r_p].
static size_t q4_ws(const qbk_factor *L, size_t n_layers, size_t batch);

// batch <= Q4_MAXB: the fp4 decode's operand buffers (q4_plan).  Larger
// batches: f32 partials [split][batch][r_p], then t bf16 [batch][r_p].
static size_t ws_bytes(const qbk_factor *L, size_t batch, int split) {
    if (batch <= Q4_MAXB) return q4_ws(L, 1, batch);
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


// Workspace of the fp4 decode for n_layers layers of L's shape at `batch`:
// [bop1 | bsc1 | bop2 | bsc2] (the fp8 operands and E8M0 scales of the two
// stages), each region 256-byte aligned.
struct Q4Plan {
    size_t ns1, ns2, ncol;
    size_t o_bop1, o_bsc1, o_bop2, o_bsc2, bytes;
};

static Q4Plan q4_plan(const qbk_factor *L, size_t n_layers, size_t batch) {
    Q4Plan p{};
    p.ns1 = L->din_q / 128;
    p.ns2 = L->r_q / 128;
    p.ncol = 2 * batch;
    size_t off = 0;
    auto take = [&](size_t n) {
        size_t o = off;
        off += round_up(n, 256);
        return o;
    };
    p.o_bop1 = take(n_layers * p.ns1 * 4 * p.ncol * 32);
    p.o_bsc1 = take(n_layers * p.ns1 * 4 * p.ncol);
    p.o_bop2 = take(n_layers * p.ns2 * 4 * p.ncol * 32);
    p.o_bsc2 = take(n_layers * p.ns2 * 4 * p.ncol);
    p.bytes = off;
    return p;
}

static size_t q4_ws(const qbk_factor *L, size_t n_layers, size_t batch) {
    return q4_plan(L, n_layers, batch).bytes;
}

// Waves that share a 64-row group split its slices: one load step (Q4_U
// slices) per wave where the group has more, and further while the launch is
// too small to fill the chip (a single layer).
static int q4_ksplit(size_t ns, size_t n_rg_total, int num_cus) {
    int k = 1;
    while (k < 4 && ns > (size_t)(Q4_U * k)) k *= 2;
    while (k < 4 && ns >= (size_t)(2 * k) && n_rg_total * k < (size_t)num_cus * 8) k *= 2;
    return k;
}

// Workgroups per CU of the stream kernel at this LDS size (cached per variant).
// phase 1: x -> stage 1's fp8 operand; 2: stage-1 MFMA GEMV, whose epilogue
// writes t = bf16(Vb^T z) as stage 2's fp8 operand; 3: stage-2 MFMA GEMV -> y.
// x: [n][batch][din] (bf16, or f32 when xf32), y: [n][batch][dout].
static int q4_phase(int phase, const qbk_factor *L, const Q4Layer *tab, size_t n_layers,
                    size_t batch, const void *x, bool xf32, void *y, bool ybf16, void *ws,
                    hipStream_t s) {
    Q4Plan p = q4_plan(L, n_layers, batch);
    char *w = (char *)ws;
    Q4Args a{};
    a.c7 = 0x77777777u;
    a.batch = (int)batch;
    a.ncol = (int)p.ncol;
    a.y_bf16 = ybf16;
    if (phase <= 2) {
        a.layers = tab;
        a.rows_p = L->r_p;
        a.rows_valid = L->r;
        a.k_valid = L->din;
        a.ns = p.ns1;
        a.act = x;
        a.act_ld = L->din;
        a.act_layer = batch * L->din;
        a.bop = (uint8_t *)(w + p.o_bop1);
        a.bsc = (uint8_t *)(w + p.o_bsc1);
        a.tb_op = (uint8_t *)(w + p.o_bop2);
        a.tb_sc = (uint8_t *)(w + p.o_bsc2);
        a.tb_ns = p.ns2;
    } else {
        a.layers = tab + n_layers;
        a.rows_p = L->dout_p;
        a.rows_valid = L->dout;
        a.k_valid = L->r;
        a.ns = p.ns2;
        a.bop = (uint8_t *)(w + p.o_bop2);
        a.bsc = (uint8_t *)(w + p.o_bsc2);
        a.out = y;
        a.out_ld = L->dout;
        a.out_layer = batch * L->dout;
    }
    if (phase == 1) {
        // 16-element vector loads need 16-aligned rows (32 or 64 bytes)
        a.vec_ok = a.act_ld % 16 == 0 && (uintptr_t)a.act % 16 == 0;
        const size_t runs = n_layers * batch * a.ns * 8;
        dim3 g((unsigned)div_ceil(runs, 256));
        if (xf32)
            hipLaunchKernelGGL((q4_prep_kernel<true>), g, dim3(256), 0, s, a, runs);
        else
            hipLaunchKernelGGL((q4_prep_kernel<false>), g, dim3(256), 0, s, a, runs);
        QBK_HIP(hipGetLastError());
        return QBK_OK;
    }
    const size_t n_rg = a.rows_p / 64;
    const int ksplit = q4_ksplit(a.ns, n_layers * n_rg, L->num_cus);
    const size_t rg_per_wg = 4 / ksplit;
    a.wg_per_layer = (uint32_t)div_ceil(n_rg, rg_per_wg);
    a.n_layers = (uint32_t)n_layers;
    dim3 g((unsigned)round_up((size_t)a.wg_per_layer * n_layers, 8));  // a multiple of the 8 XCDs
    const int ncol_t = batch <= 2 ? (int)p.ncol : 0;  // staged operand at batch 1-2
    const size_t lds = q4_gemv_lds(ncol_t, ksplit);
#define Q4_LAUNCH(ST, KS)                                                                        \
    if (ncol_t == 2) hipLaunchKernelGGL((q4_gemv_kernel<ST, KS, 2>), g, dim3(256), lds, s, a);  \
    else if (ncol_t == 4) hipLaunchKernelGGL((q4_gemv_kernel<ST, KS, 4>), g, dim3(256), lds, s, a); \
    else hipLaunchKernelGGL((q4_gemv_kernel<ST, KS, 0>), g, dim3(256), lds, s, a);
#define Q4_LAUNCH_KS(ST)                                                                         \
    if (ksplit == 4) { Q4_LAUNCH(ST, 4) }                                                        \
    else if (ksplit == 2) { Q4_LAUNCH(ST, 2) }                                                   \
    else { Q4_LAUNCH(ST, 1) }
    if (phase == 2) {
        Q4_LAUNCH_KS(1)
    } else {
        Q4_LAUNCH_KS(2)
    }
#undef Q4_LAUNCH_KS
#undef Q4_LAUNCH
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

static int run_q4(const qbk_factor *L, size_t batch, const void *x, bool xf32, void *y,
                  bool ybf16, void *ws, hipStream_t s) {
    // a single layer's table is {stage 1, stage 2}: tab + n_layers is stage 2
    const Q4Layer *tab = (const Q4Layer *)L->q4_tab;
    for (int ph = 1; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, L, tab, 1, batch, x, xf32, y, ybf16, ws, s);
        if (rc) return rc;
    }
    return QBK_OK;
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

struct qbk_factor_set {
    int device;
    size_t n, dout, din, r, r_p;
    Q4Layer *d1, *d2;  // device table: [0, n) stage 1 entries, [n, 2n) stage 2 (d2 = d1 + n)
    const qbk_factor *first;
};

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
    if (batch <= Q4_MAXB) return run_q4(L, batch, x, false, y, y_dtype == QBK_BF16, workspace, s);
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
        rc = run_q4(L, batch, dx.p, true, dy.p, false, dws.p, cs.s);
    else
        rc = run_gemm(L, dx.p, true, batch, dy.p, false, dws.p, split, cs.s);
    if (rc) return rc;
    QBK_HIP(hipMemcpyAsync(y, dy.p, batch * L->dout * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_factor_set_create(qbk_ctx *ctx, const qbk_factor *const *layers, size_t n,
                          qbk_factor_set **out) {
    int rc;
    if (!out || !layers || n == 0) return fail(QBK_ERR_VALIDATION, "empty layer set");
    *out = nullptr;
    const qbk_factor *f = layers[0];
    for (size_t i = 0; i < n; i++) {
        const qbk_factor *L = layers[i];
        if (!L || L->dout != f->dout || L->din != f->din || L->r != f->r)
            return fail(QBK_ERR_VALIDATION,
                        fmt("layer %zu of the set does not share (dout, din, r) = (%zu, %zu, %zu)",
                            i, f->dout, f->din, f->r));
    }
    if ((rc = bind(ctx))) return rc;
    std::vector<Q4Layer> h(2 * n);
    for (size_t i = 0; i < n; i++) {
        const qbk_factor *L = layers[i];
        if (L->device != ctx->device)
            return fail(QBK_ERR_VALIDATION, fmt("layer %zu lives on another device", i));
        h[i] = Q4Layer{L->vt_q4, L->s2, nullptr, nullptr};
        h[n + i] = Q4Layer{L->u_q4, nullptr, L->s1, L->bias};
    }
    qbk_factor_set *S = new qbk_factor_set();
    S->device = ctx->device;
    S->n = n;
    S->dout = f->dout;
    S->din = f->din;
    S->r = f->r;
    S->r_p = f->r_p;
    S->first = f;
    hipError_t e1 = hipMalloc((void **)&S->d1, 2 * n * sizeof(Q4Layer));
    if (e1 != hipSuccess) {
        delete S;
        return fail(QBK_ERR_DEVICE, fmt("hipMalloc failed: %s", hipGetErrorString(e1)));
    }
    S->d2 = S->d1 + n;
    e1 = hipMemcpy(S->d1, h.data(), 2 * n * sizeof(Q4Layer), hipMemcpyHostToDevice);
    if (e1 != hipSuccess) {
        (void)hipFree(S->d1);
        delete S;
        return fail(QBK_ERR_DEVICE, fmt("hipMemcpy failed: %s", hipGetErrorString(e1)));
    }
    *out = S;
    return QBK_OK;
}

void qbk_factor_set_destroy(qbk_factor_set *S) {
    if (!S) return;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(S->device);
    (void)hipFree(S->d1);
    (void)hipSetDevice(cur);
    delete S;
}

size_t qbk_factor_set_workspace_size(const qbk_factor_set *S) {
    return S ? q4_ws(S->first, S->n, 1) : 0;
}

// x [n][din] bf16 -> y [n][dout] bf16 in three phases (see q4_phase).
int qbk_factor_set_stage_dev(qbk_ctx *ctx, const qbk_factor_set *S, int stage, const uint16_t *x,
                             uint16_t *y, void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if (!S) return fail(QBK_ERR_VALIDATION, "null layer set");
    if (stage < 1 || stage > Q4_PHASES)
        return fail(QBK_ERR_VALIDATION, fmt("stage must be 1..%d, got %d", Q4_PHASES, stage));
    if ((rc = bind(ctx))) return rc;
    if (workspace_size < qbk_factor_set_workspace_size(S))
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs",
                        workspace_size, qbk_factor_set_workspace_size(S)));
    return q4_phase(stage, S->first, (const Q4Layer *)S->d1, S->n, 1, x, false, y, true, workspace,
                    (hipStream_t)stream);
}

int qbk_factor_set_decode_dev(qbk_ctx *ctx, const qbk_factor_set *S, const uint16_t *x,
                              uint16_t *y, void *workspace, size_t workspace_size, void *stream) {
    for (int ph = 1; ph <= Q4_PHASES; ph++) {
        int rc = qbk_factor_set_stage_dev(ctx, S, ph, x, y, workspace, workspace_size, stream);
        if (rc) return rc;
    }
    return QBK_OK;
}

}  // extern "C"
