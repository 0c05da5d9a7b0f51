// prefill.hip -- the factor linear's prefill GEMM (batch > 8) on gfx950.
//
//   t = bf16(Vb^T z), z = bf16(s2 * x);  y = bf16(Ub t) * s1 + bias
//                              (engine/mod.rs:449-460, apply_bf16, per token)
//
// Both stages are C[M x N] = S[M x K] (+-1) . Act[K x N] with the
// activations token-major (Act^T [N][K], bf16) and f32 accumulation on
// v_mfma_f32_32x32x16_bf16:
//   * workgroup tile 256 (rows) x 128 (tokens), 8 waves as 4 (rows) x 2
//     (tokens), wave tile 64 x 64 = 2 x 2 MFMA tiles: 64 accumulator
//     registers, so two waves share each SIMD and one's LDS and barrier
//     waits are covered by the other's MFMAs;
//   * A (signs): each wave loads one uint2 per lane per 64-k stage -- its
//     64 rows x 64 k bits -- from the g32 layout (g32_repack) and expands a
//     32x16 fragment with two VALU ops per VGPR, reused by both n-tiles;
//   * B (activations): 128 tokens x 64 k staged through LDS, double
//     buffered, rows padded to 144 bytes (the 32 lanes of a fragment read
//     rows 144 B apart: conflict-free 16-byte reads);
//   * stage 1 forms z = bf16(s2 * x) (zero past din) while staging x through
//     LDS -- g32_prep_kernel writes it beforehand only for rows that are not
//     16-byte chunks -- splits K to fill the chip and writes f32 partials that
//     g32_reduce_kernel sums in split order into t bf16 (zero past r); with
//     no split the epilogue writes t directly;
//   * stage 2 reads t and writes y = bf16(u) * s1 + bias, u = bf16(acc).
#include <string.h>

#include <mutex>

#include "factor_internal.h"

namespace qbk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define G_BK 64
#define G_PITCH 72    // bf16 per LDS row of the activation tile: 64 + 8 of padding
#define G_TPITCH 68   // f32 per token row of the epilogue transpose: 64 + 4

// g32 sign layout: blocks of (128-row group g, 64-k slice s), 64 lanes x 4
// words.  Word j of lane l holds row 128g + 32j + l%32 at
// k = 64s + 16q + 8(l/32) + e for k16 step q (0..3) and element e (0..7):
// element 2v at bit 4q + v, element 2v + 1 at bit 4q + v + 16, set when the
// sign is -1 (0 in the rows' bitplanes).  Rows >= n_rows and k >= n_bits
// hold +1 (0): padded k meets zero activations.
void g32_repack(const uint8_t *rows, size_t n_rows, size_t n_bits, size_t rows_p, size_t bits_p,
                uint32_t *out) {
    const size_t rw = div_ceil(n_bits, 8);
    const size_t ng = rows_p / 128, nsk = bits_p / 64;
    memset(out, 0, ng * nsk * 64 * 4 * 4);
    for (size_t g = 0; g < ng; g++)
        for (size_t s = 0; s < nsk; s++)
            for (int l = 0; l < 64; l++)
                for (int j = 0; j < 4; j++) {
                    const size_t i = 128 * g + 32 * j + (l & 31);
                    if (i >= n_rows) continue;
                    uint32_t w = 0;
                    for (int q = 0; q < 4; q++)
                        for (int e = 0; e < 8; e++) {
                            const size_t k = 64 * s + 16 * q + 8 * (l >> 5) + e;
                            if (k < n_bits && !((rows[i * rw + (k >> 3)] >> (k & 7)) & 1))
                                w |= 1u << (4 * q + (e >> 1) + 16 * (e & 1));
                        }
                    out[((g * nsk + s) * 64 + l) * 4 + j] = w;
                }
}

struct G32Args {
    const uint32_t *sg;    // g32 layout [M_p/128][K_p/64][64][4]
    size_t M_p, K_p, M_valid, N;
    const uint16_t *act;   // bf16 [N][K_p] (z or t), zero for k past the valid K (XM 0)
    const void *x;         // stage 1, XM 1 / 2: x [N][din] bf16 / f32, s2 [din]; din % 8 == 0
    const float *s2;
    size_t din;
    float *part;           // [split][N][ld_out] f32 (split > 1, either stage)
    size_t k_per_split;
    int split;
    size_t ld_out, ld_act; // row strides of part / t_out and of the activation (XM 0)
    // a layer set (null for one layer): the layers of this stage, found by
    // row tile (128-row tiles), each at its own rows of the concatenated
    // partials / t (stage 1) or columns of t and block of y (stage 2)
    const G32SetLayer *set;
    uint32_t n_set;
    // stage 1
    uint16_t *t_out;       // [N][M_p] bf16 (split == 1), zero for rows >= M_valid
    // stage 2
    void *y;               // [N][M_valid] bf16 or f32
    const float *s1, *bias;
    int y_bf16, vec_y;     // vec_y: y rows allow 16-byte stores (M_valid % 8 == 0, y aligned)
    uint32_t sign_mask, one_pair;  // 0x80008000, 0x3F803F80 (see g32_frag)
};

// Expand sign word w for k16 step q into the 32x16 A fragment: VGPR v holds
// elements 2v, 2v + 1 as bf16 +-1 (0x3F80 | sign << 15).  The mask and the
// +1 pair come in as registers (m = 0x80008000, one = 0x3F803F80) so that
// each VGPR costs a shift and one v_and_or_b32 (VOP3 takes no literal).
__device__ __forceinline__ bf16x8_t g32_frag(uint32_t w, int q, uint32_t m, uint32_t one) {
    u32x4_t u;
    u.x = ((w << (15 - (4 * q + 0))) & m) | one;
    u.y = ((w << (15 - (4 * q + 1))) & m) | one;
    u.z = ((w << (15 - (4 * q + 2))) & m) | one;
    u.w = ((w << (15 - (4 * q + 3))) & m) | one;
    return __builtin_bit_cast(bf16x8_t, u);
}

// XM: the activation operand -- 0: bf16 rows of K_p (z or t); 1 / 2: stage 1
// forms z = bf16(s2 * x) itself from bf16 / f32 x while staging it.
// Wave grid WM (rows) x WN (tokens), wave tile 64 rows x 32 NT tokens, so
// the workgroup tile is 64 WM x 32 NT WN with 64 WM WN threads; the tile
// staging gives each thread two 8-element chunks, which needs BN = threads/4
// (WM = 2 NT).  Shapes: 4 x 2 x 2 (256 x 128, 8 waves) for grids that fill the
// chip; 2 x 2 x 1 (128 x 64, 4 waves) for the others.
template <int WM, int WN, int NT>
struct G32Shape {
    static constexpr int THREADS = 64 * WM * WN, BM = 64 * WM, BN = 32 * NT * WN;
    static constexpr int LDS_TILES = 2 * BN * G_PITCH * 2, LDS_EPI = WM * WN * 32 * G_TPITCH * 4;
    static constexpr int LDS = LDS_TILES > LDS_EPI ? LDS_TILES : LDS_EPI;
    static_assert(BN == THREADS / 4 && WM % 2 == 0, "two staged chunks per thread, 128-row sign groups");
};

template <int STAGE, int XM, int WM, int WN, int NT>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(1, 2))) g32_kernel(G32Args a0) {
    using SH = G32Shape<WM, WN, NT>;
    G32Args a = a0;
    size_t by = blockIdx.y, col0 = 0;
    if (a.set) {
        // this workgroup's layer: the last whose first tile is at or before it
        const __attribute__((address_space(4))) G32SetLayer *ls =
            (const __attribute__((address_space(4))) G32SetLayer *)a.set;
        uint32_t li = 0;
        for (uint32_t i = 1; i < a.n_set; i++)
            if (by >= ls[i].tile0) li = i;
        by -= ls[li].tile0;
        a.sg = ls[li].sg;
        a.M_p = ls[li].M_p;
        a.M_valid = ls[li].M_valid;
        a.K_p = ls[li].K_p;
        a.s2 = ls[li].s2;
        a.s1 = ls[li].s1;
        a.bias = ls[li].bias;
        col0 = ls[li].col0;
        if (STAGE == 2) {
            a.act += col0;
            a.y = (char *)a.y + ls[li].y0 * a.N * (a.y_bf16 ? 2 : 4);
        }
    }
    constexpr int BN = SH::BN, BM = SH::BM, TPB8 = SH::THREADS / 8;
    // [2 tile buffers of BN x G_PITCH bf16] during the loop; [waves][32 x
    // G_TPITCH f32] in the epilogue
    extern __shared__ __attribute__((aligned(16))) uint8_t g32_lds[];
    uint16_t(*bs)[BN * G_PITCH] = (uint16_t(*)[BN * G_PITCH])g32_lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave % WM, wc = wave / WM;  // 64-row block, 32 NT-token block
    const size_t n0 = (size_t)blockIdx.x * BN, m0 = by * BM;
    size_t kb = 0, ke = a.K_p;
    if (STAGE == 1 || a.split > 1) {
        kb = (size_t)blockIdx.z * a.k_per_split;
        ke = kb + a.k_per_split < a.K_p ? kb + a.k_per_split : a.K_p;
    }
    const size_t ng = a.M_p / 128, nsk = a.K_p / G_BK;
    const size_t g = m0 / 128 + (wr >> 1);          // this wave's 128-row group
    const size_t gc = g < ng ? g : ng - 1;          // clamped: loads stay in bounds
    // words 2h, 2h + 1 of each lane's record: this wave's 64 rows
    const uint2 *sp = (const uint2 *)a.sg + ((gc * nsk) * 64 + lane) * 2 + (wr & 1);
    // the +1 pair in a VGPR, the mask in an SGPR: one v_and_or_b32 can read both
    const uint32_t m_sign = a.sign_mask;
    uint32_t one;
    asm volatile("v_mov_b32 %0, %1" : "=v"(one) : "s"(a.one_pair));

    // B tile: BN tokens x 64 k = 8 BN chunks of 8 elements, two per thread
    // (tokens tid/8 + (threads/8) u, k chunk tid%8).  Every load is issued
    // unconditionally -- tokens past N are clamped to N - 1 and only feed
    // output columns the epilogue does not store; with XM, chunks past din
    // read chunk 0 and store zeros -- so that the wait for the prefetch can
    // be a counted one at the LDS store.
    const size_t kc = (tid & 7) * 8, ld = XM ? a.din : a.ld_act;
    const char *brow[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const size_t n = n0 + (tid >> 3) + TPB8 * u;
        const size_t off = (n < a.N ? n : a.N - 1) * ld + kc;
        brow[u] = XM == 2 ? (const char *)((const float *)a.x + off)
                          : (const char *)((XM ? (const uint16_t *)a.x : a.act) + off);
    }
    constexpr int NB = XM == 2 ? 4 : 2;  // staged 16-byte pieces per thread
    u32x4_t breg[NB];
    float4 s2r[2];                       // XM: s2 of the staged chunk
    bool bval = true;                    // XM: the staged chunk lies below din
#define G32_LOAD_ACT(K)                                                                         \
    {                                                                                           \
        size_t ko = (K);                                                                        \
        if (XM) {                                                                               \
            bval = ko + kc < a.din;                                                             \
            ko = bval ? ko : 0;                                                                 \
            s2r[0] = *(const float4 *)(a.s2 + ko + kc);                                         \
            s2r[1] = *(const float4 *)(a.s2 + ko + kc + 4);                                     \
        }                                                                                       \
        _Pragma("unroll") for (int u = 0; u < 2; u++) {                                         \
            if (XM == 2) {                                                                      \
                breg[2 * u] = *(const u32x4_t *)((const float *)brow[u] + ko);                  \
                breg[2 * u + 1] = *(const u32x4_t *)((const float *)brow[u] + ko + 4);          \
            } else {                                                                            \
                breg[u] = *(const u32x4_t *)((const uint16_t *)brow[u] + ko);                   \
            }                                                                                   \
        }                                                                                       \
    }
    // XM: z = bf16(s2 * x) of the staged chunk, formed as it is stored
#define G32_STORE_ACT(B)                                                                        \
    _Pragma("unroll") for (int u = 0; u < 2; u++) {                                             \
        u32x4_t zv;                                                                             \
        if (XM == 0) {                                                                          \
            zv = breg[u];                                                                       \
        } else {                                                                                \
            const float sv[8] = {s2r[0].x, s2r[0].y, s2r[0].z, s2r[0].w,                        \
                                 s2r[1].x, s2r[1].y, s2r[1].z, s2r[1].w};                       \
            float xv[8];                                                                        \
            _Pragma("unroll") for (int e = 0; e < 4; e++) {                                     \
                if (XM == 2) {                                                                  \
                    xv[2 * e] = __uint_as_float(breg[2 * u + (e >> 1)][2 * (e & 1)]);          \
                    xv[2 * e + 1] = __uint_as_float(breg[2 * u + (e >> 1)][2 * (e & 1) + 1]);  \
                } else {                                                                        \
                    xv[2 * e] = __uint_as_float(breg[u][e] << 16);                             \
                    xv[2 * e + 1] = __uint_as_float(breg[u][e] & 0xffff0000u);                 \
                }                                                                               \
            }                                                                                   \
            _Pragma("unroll") for (int e = 0; e < 4; e++)                                       \
                zv[e] = bval ? f32x2_to_bf16x2(sv[2 * e] * xv[2 * e], sv[2 * e + 1] * xv[2 * e + 1]) : 0u;\
        }                                                                                       \
        *(u32x4_t *)&bs[B][((tid >> 3) + TPB8 * u) * G_PITCH + kc] = zv;                        \
    }

    f32x16_t acc[2][NT];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[j][nt][i] = 0.0f;

    // Three-stage pipeline over the 64-k stages i.  Activations: stage
    // i + 2's tile is in flight from global memory, stage i + 1's sits in
    // registers until it is stored to LDS at the top of stage i and read
    // back (after the barrier) under stage i's MFMAs.  Signs: stage i + 2's
    // words load during stage i and stage i + 1's fragments are expanded
    // between stage i's MFMAs, so that no MFMA waits on a VALU result or an
    // LDS read of its own stage.  Stages past the end reload the last one (in
    // bounds, never used).  The loop is unrolled by two so that words,
    // fragments and tiles alternate between two register sets (a copy of a
    // value still in flight would wait for it).
    const size_t k_last = ke > kb ? ke - G_BK : kb;
    uint2 awA = make_uint2(0, 0), awB = make_uint2(0, 0);
    bf16x8_t afA[4][2], afB[4][2], bfA[4][NT], bfB[4][NT];
#define G32_READ_FRAGS(B, F)                                                                    \
    _Pragma("unroll") for (int q = 0; q < 4; q++)                                               \
    _Pragma("unroll") for (int nt = 0; nt < NT; nt++)                                           \
        F[q][nt] = __builtin_bit_cast(                                                          \
            bf16x8_t, *(const u32x4_t *)&bs[B][(wc * 32 * NT + nt * 32 + (lane & 31)) * G_PITCH + \
                                              16 * q + 8 * (lane >> 5)]);
    // one stage: K0 its first k, B its LDS buffer, AFC/BFC its sign and
    // activation fragments, AFN/BFN the next stage's, AWU the next stage's
    // sign words, AWL the register set for stage i + 2's
#define G32_STAGE(K0, B, AFC, AFN, BFC, BFN, AWU, AWL)                                          \
    {                                                                                           \
        G32_STORE_ACT((B) ^ 1)                                                                  \
        const size_t k2 = (K0) + 2 * G_BK < ke ? (K0) + 2 * G_BK : k_last;                      \
        AWL = sp[(k2 / G_BK) * 128];                                                            \
        G32_LOAD_ACT(k2)                                                                        \
        __builtin_amdgcn_sched_barrier(0);                                                      \
        __syncthreads();                                                                        \
        __builtin_amdgcn_sched_barrier(0);                                                      \
        G32_READ_FRAGS((B) ^ 1, BFN)                                                            \
        __builtin_amdgcn_sched_barrier(0);                                                      \
        _Pragma("unroll") for (int q = 0; q < 4; q++) {                                         \
            AFN[q][0] = g32_frag(AWU.x, q, m_sign, one);                                        \
            AFN[q][1] = g32_frag(AWU.y, q, m_sign, one);                                        \
            _Pragma("unroll") for (int j = 0; j < 2; j++)                                       \
            _Pragma("unroll") for (int nt = 0; nt < NT; nt++)                                   \
                acc[j][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(AFC[q][j], BFC[q][nt], acc[j][nt], 0, 0, 0);\
        }                                                                                       \
    }
    if (kb < ke) {
        const size_t k1 = kb + G_BK < ke ? kb + G_BK : k_last;
        G32_LOAD_ACT(kb)
        const uint2 aw0 = sp[(kb / G_BK) * 128];
        awB = sp[(k1 / G_BK) * 128];
        G32_STORE_ACT(0)
        G32_LOAD_ACT(k1)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            afA[q][0] = g32_frag(aw0.x, q, m_sign, one);
            afA[q][1] = g32_frag(aw0.y, q, m_sign, one);
        }
    }
    __syncthreads();
    G32_READ_FRAGS(0, bfA)
    size_t k0 = kb;
    for (; k0 + G_BK < ke; k0 += 2 * G_BK) {
        G32_STAGE(k0, 0, afA, afB, bfA, bfB, awB, awA)
        G32_STAGE(k0 + G_BK, 1, afB, afA, bfB, bfA, awA, awB)
    }
    if (k0 < ke) G32_STAGE(k0, 0, afA, afB, bfA, bfB, awB, awA)  // an odd stage count's last
#undef G32_STAGE
#undef G32_READ_FRAGS
#undef G32_STORE_ACT
#undef G32_LOAD_ACT
    __syncthreads();  // the epilogue reuses the tile buffers
    // Epilogue, one 32-token n-tile at a time, through the wave's LDS region
    // T [32 tokens][G_TPITCH] f32 (the tile buffers are free: the loop ended
    // with a barrier): lanes write their accumulators -- acc[j][nt][4h + p]
    // is row 32j + 8h + 4(l/32) + p of token l%32 -- then read whole
    // token rows back, so that consecutive lanes store consecutive 16-byte
    // pieces of one token's output row.
    float *T = (float *)(g32_lds + wave * (32 * G_TPITCH * 4));
    const bool gvalid = g < ng;
    const size_t row0 = m0 + 64 * wr;  // this wave's first row
    // stage 2: s1 and bias of rows 8c .. 8c + 7 of the wave (c = lane % 8)
    float s1v[8], biv[8];
    if (STAGE == 2 && gvalid && a.split == 1) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const size_t rr = row0 + 8 * (lane & 7) + e;
            s1v[e] = rr < a.M_valid ? a.s1[rr] : 0.0f;
            biv[e] = rr < a.M_valid ? a.bias[rr] : 0.0f;
        }
    }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int h = 0; h < 4; h++)
                *(float4 *)&T[(lane & 31) * G_TPITCH + 32 * j + 8 * h + 4 * (lane >> 5)] =
                    make_float4(acc[j][nt][4 * h], acc[j][nt][4 * h + 1], acc[j][nt][4 * h + 2],
                                acc[j][nt][4 * h + 3]);
        __builtin_amdgcn_wave_barrier();
        const size_t nb = n0 + wc * 32 * NT + nt * 32;  // first token of the n-tile
        if (gvalid) {
            if (a.split > 1) {
                // f32 partials: 16 lanes per token (4 rows each), four tokens per store
#pragma unroll 4
                for (int k = 0; k < 8; k++) {
                    const int tt = 4 * k + (lane >> 4), c = lane & 15;
                    const size_t n = nb + tt;
                    float4 v = *(const float4 *)&T[tt * G_TPITCH + 4 * c];
                    const size_t rv = row0 + 4 * c;  // rows past the valid ones contribute zeros
                    if (rv >= a.M_valid) v.x = 0.0f;
                    if (rv + 1 >= a.M_valid) v.y = 0.0f;
                    if (rv + 2 >= a.M_valid) v.z = 0.0f;
                    if (rv + 3 >= a.M_valid) v.w = 0.0f;
                    if (n < a.N) *(float4 *)(a.part + ((size_t)blockIdx.z * a.N + n) * a.ld_out + col0 + rv) = v;
                }
            } else {
                // bf16 rows: 8 lanes per token (8 rows each), eight tokens per store
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int tt = 8 * k + (lane >> 3), c = lane & 7;
                    const size_t n = nb + tt;
                    const float4 v0 = *(const float4 *)&T[tt * G_TPITCH + 8 * c];
                    const float4 v1 = *(const float4 *)&T[tt * G_TPITCH + 8 * c + 4];
                    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                    const size_t rb = row0 + 8 * c;
                    if (n >= a.N) continue;
                    if (STAGE == 1) {
                        // t = bf16(acc), zero past r (split == 1)
                        uint32_t w[4];
#pragma unroll
                        for (int p = 0; p < 4; p++) {
                            w[p] = f32x2_to_bf16x2(v[2 * p], v[2 * p + 1]);
                            if (rb + 2 * p >= a.M_valid) w[p] &= 0xffff0000u;
                            if (rb + 2 * p + 1 >= a.M_valid) w[p] &= 0x0000ffffu;
                        }
                        *(uint4 *)(a.t_out + n * a.ld_out + col0 + rb) = make_uint4(w[0], w[1], w[2], w[3]);
                    } else {
                        float y[8];
#pragma unroll
                        for (int p = 0; p < 4; p++) {
                            const uint32_t u = f32x2_to_bf16x2(v[2 * p], v[2 * p + 1]);
                            y[2 * p] = __uint_as_float(u << 16) * s1v[2 * p] + biv[2 * p];
                            y[2 * p + 1] = __uint_as_float(u & 0xffff0000u) * s1v[2 * p + 1] + biv[2 * p + 1];
                        }
                        if (a.y_bf16 && a.vec_y && rb + 8 <= a.M_valid) {
                            uint32_t w[4];
#pragma unroll
                            for (int p = 0; p < 4; p++) w[p] = f32x2_to_bf16x2(y[2 * p], y[2 * p + 1]);
                            *(uint4 *)((uint16_t *)a.y + n * a.M_valid + rb) = make_uint4(w[0], w[1], w[2], w[3]);
                        } else {
#pragma unroll
                            for (int p = 0; p < 8; p++) {
                                if (rb + p >= a.M_valid) continue;
                                if (a.y_bf16)
                                    ((uint16_t *)a.y)[n * a.M_valid + rb + p] = f32_to_bf16(y[p]);
                                else
                                    ((float *)a.y)[n * a.M_valid + rb + p] = y[p];
                            }
                        }
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the next n-tile overwrites T
    }
}

// z[n][k] = bf16(s2[k] * x[n][k]) for k < din, 0 for din <= k < K_p, eight
// elements per thread: the staging for inputs whose rows stage 1 cannot
// read in 16-byte chunks (din % 8 != 0 or x unaligned).
template <bool XF32>
__global__ void __launch_bounds__(256) g32_prep_kernel(const void *x, const float *s2, size_t din,
                                                        size_t K_p, size_t N, uint16_t *z) {
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_row = K_p / 8;
    if (c >= N * per_row) return;
    const size_t n = c / per_row, k0 = (c % per_row) * 8;
    float v[8], sv[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const size_t k = k0 + e;
        const bool ok = k < din;
        v[e] = !ok ? 0.0f : XF32 ? ((const float *)x)[n * din + k] : bf16_to_f32(((const uint16_t *)x)[n * din + k]);
        sv[e] = ok ? s2[k] : 0.0f;
    }
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) w[e] = f32x2_to_bf16x2(sv[2 * e] * v[2 * e], sv[2 * e + 1] * v[2 * e + 1]);
    *(uint4 *)(z + n * K_p + k0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// t = bf16(sum of the split partials in split order), zero for rows >= r;
// eight rows per thread.
__global__ void __launch_bounds__(256) g32_reduce_kernel(const float *__restrict__ part, int split,
                                                          size_t stride, size_t ld, size_t r,
                                                          uint16_t *__restrict__ t, size_t chunks) {
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const size_t e0 = c * 8, k0 = e0 % ld;
    float v[8];
    const float4 *p0 = (const float4 *)(part + e0);
    const float4 a0 = p0[0], a1 = p0[1];
    v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
    v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    for (int s = 1; s < split; s++) {
        const float4 *ps = (const float4 *)(part + (size_t)s * stride + e0);
        const float4 c0 = ps[0], c1 = ps[1];
        v[0] += c0.x; v[1] += c0.y; v[2] += c0.z; v[3] += c0.w;
        v[4] += c1.x; v[5] += c1.y; v[6] += c1.z; v[7] += c1.w;
    }
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        w[e] = f32x2_to_bf16x2(v[2 * e], v[2 * e + 1]);
        if (k0 + 2 * e >= r) w[e] &= 0xffff0000u;
        if (k0 + 2 * e + 1 >= r) w[e] &= 0x0000ffffu;
    }
    *(uint4 *)(t + e0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Stage 2 split over K: y = bf16(sum of the split partials in split order)
// * s1 + bias for rows < dout (the stage-2 epilogue's arithmetic on the whole
// sum); eight rows per thread over [N][M_p].
__global__ void __launch_bounds__(256) g32_reduce_y_kernel(const float *__restrict__ part, int split,
                                                            size_t stride, size_t ld, size_t dout,
                                                            const float *__restrict__ s1,
                                                            const float *__restrict__ bias, void *y, int y_bf16,
                                                            int vec_y, size_t chunks) {
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const size_t e0 = c * 8, n = e0 / ld, r0 = e0 % ld;
    if (r0 >= dout) return;
    float v[8];
    const float4 *p0 = (const float4 *)(part + e0);
    const float4 a0 = p0[0], a1 = p0[1];
    v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
    v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    for (int s = 1; s < split; s++) {
        const float4 *ps = (const float4 *)(part + (size_t)s * stride + e0);
        const float4 c0 = ps[0], c1 = ps[1];
        v[0] += c0.x; v[1] += c0.y; v[2] += c0.z; v[3] += c0.w;
        v[4] += c1.x; v[5] += c1.y; v[6] += c1.z; v[7] += c1.w;
    }
    float yv[8];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t u = f32x2_to_bf16x2(v[2 * p], v[2 * p + 1]);
        const size_t ra = r0 + 2 * p < dout ? r0 + 2 * p : 0, rb = r0 + 2 * p + 1 < dout ? r0 + 2 * p + 1 : 0;
        yv[2 * p] = __uint_as_float(u << 16) * s1[ra] + bias[ra];
        yv[2 * p + 1] = __uint_as_float(u & 0xffff0000u) * s1[rb] + bias[rb];
    }
    if (y_bf16 && vec_y && r0 + 8 <= dout) {
        uint32_t w[4];
#pragma unroll
        for (int p = 0; p < 4; p++) w[p] = f32x2_to_bf16x2(yv[2 * p], yv[2 * p + 1]);
        *(uint4 *)((uint16_t *)y + n * dout + r0) = make_uint4(w[0], w[1], w[2], w[3]);
        return;
    }
#pragma unroll
    for (int p = 0; p < 8; p++) {
        if (r0 + p >= dout) continue;
        if (y_bf16)
            ((uint16_t *)y)[n * dout + r0 + p] = f32_to_bf16(yv[p]);
        else
            ((float *)y)[n * dout + r0 + p] = yv[p];
    }
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

// The two workgroup shapes: 256 x 128 tiles (8 waves) and 128 x 64 tiles
// (4 waves).  Stage 2 takes the large ones when they alone give every CU a
// workgroup.
typedef G32Shape<4, 2, 2> G32Big;
typedef G32Shape<2, 2, 1> G32Small;
typedef G32Shape<2, 1, 1> G32Tiny;  // 128 x 32 tiles (2 waves): batches of up to 32 tokens

static bool g32_big(size_t M_p, size_t N, int num_cus) {
    return div_ceil(N, G32Big::BN) * div_ceil(M_p, G32Big::BM) >= (size_t)num_cus;
}

// Stage-1 K split, only where even the small tiles leave CUs idle: enough
// workgroups to cover every CU, at least four 64-k stages per split.
// Stage 1 shape: the 256 x 128 tiles, split over K, while they alone cover
// a quarter of the CUs (measured at B = 2048: 56.6 us for the layer, against
// 60-82 us for every 128 x 64 choice); below that the 128 x 64 tiles (at
// B <= 512: 21-31 us, against 38-45 us).  Either way the K split brings the
// workgroups up to the CU count, at least four 64-k stages per split.
static bool g32_big1(const qbk_factor *L, size_t N) {
    return div_ceil(N, G32Big::BN) * div_ceil(L->r_p, G32Big::BM) * 4 >= (size_t)L->num_cus;
}

static int g32_split(const qbk_factor *L, size_t N) {
    const bool big = g32_big1(L, N);
    const size_t tiles = big ? div_ceil(N, G32Big::BN) * div_ceil(L->r_p, G32Big::BM)
                             : div_ceil(N, G32Small::BN) * div_ceil(L->r_p, G32Small::BM);
    int s = 1;
    // up to 8 splits of at least four 64-k stages; a long K (the down
    // projection's 224 stages) up to 16 of at least twelve
    const size_t st = L->din_p / G_BK;
    while (tiles * s < (size_t)L->num_cus && ((s < 8 && st / (2 * s) >= 4) || (s < 16 && st / (2 * s) >= 12)))
        s *= 2;
    return s;
}

// Stage-2 K split, by the same rule, where the stage's own tiles (one row
// block a workgroup, no split of its own) leave CUs idle: a decode batch
// of 9-64 tokens gives q/o 32 workgroups of 18 64-k stages each, a chain of
// dependent stages per workgroup, without it.
static int g32_split2(const qbk_factor *L, size_t N) {
    if (g32_big(L->dout_p, N, L->num_cus)) return 1;
    const size_t tiles = div_ceil(N, G32Small::BN) * div_ceil(L->dout_p, G32Small::BM);
    int s = 1;
    while (tiles * s < (size_t)L->num_cus && s < 8 && L->r_p / (G_BK * 2 * s) >= 4) s *= 2;
    return s;
}

// Workspace: z bf16 [N][din_p] (written only when stage 1 cannot form z from x
// itself) | partials f32 [split][N][r_p] | t bf16 [N][r_p] | stage 2's
// partials f32 [split2][N][dout_p].
struct G32Plan {
    int split, split2;
    size_t o_z, o_part, o_t, o_part2, bytes;
};

static G32Plan g32_plan(const qbk_factor *L, size_t N) {
    G32Plan p{};
    p.split = g32_split(L, N);
    p.split2 = g32_split2(L, N);
    size_t off = 0;
    auto take = [&](size_t n) {
        size_t o = off;
        off += round_up(n, 256);
        return o;
    };
    p.o_z = take(N * L->din_p * 2);
    p.o_part = take(p.split > 1 ? (size_t)p.split * N * L->r_p * 4 : 0);
    p.o_t = take(N * L->r_p * 2);
    p.o_part2 = take(p.split2 > 1 ? (size_t)p.split2 * N * L->dout_p * 4 : 0);
    p.bytes = off;
    return p;
}

template <int STAGE, int XM, class SH, int WM, int WN, int NT>
static void g32_launch(const G32Args &a, size_t M_p, int split, hipStream_t s) {
    dim3 g((unsigned)div_ceil(a.N, SH::BN), (unsigned)div_ceil(M_p, SH::BM), split);
    hipLaunchKernelGGL((g32_kernel<STAGE, XM, WM, WN, NT>), g, dim3(SH::THREADS), SH::LDS, s, a);
}

template <int STAGE, int XM>
static void g32_launch_any(const G32Args &a, size_t M_p, int split, bool big, hipStream_t s) {
    if (big)
        g32_launch<STAGE, XM, G32Big, 4, 2, 2>(a, M_p, split, s);
    else if (a.N <= (size_t)G32Tiny::BN)
        g32_launch<STAGE, XM, G32Tiny, 2, 1, 1>(a, M_p, split, s);
    else
        g32_launch<STAGE, XM, G32Small, 2, 2, 1>(a, M_p, split, s);
}

size_t g32_workspace(const qbk_factor *L, size_t N) { return g32_plan(L, N).bytes; }

// ---- layer sets (a decode step's batch beyond the GEMV) -----------------
//
// The layers of a set share x (so din); one launch per stage covers them
// all: stage 1's row tiles of every layer in one grid, K split as one layer
// would be, the partials and t of the layers side by side ([.][N][sum r_p],
// rows past a layer's r written as zeros); stage 2's row tiles of every
// layer in one grid, each reading its own columns of t, no K split.  Three
// launches for the set where the layers alone take three or four each.

void g32_set_tables(const qbk_factor *const *L, size_t n, G32SetLayer *t1, G32SetLayer *t2) {
    size_t tile1 = 0, tile2 = 0, rcol = 0, ycol = 0;
    for (size_t i = 0; i < n; i++) {
        t1[i] = G32SetLayer{L[i]->vt_g32, L[i]->s2, nullptr, nullptr, L[i]->r_p, L[i]->r, L[i]->din_p,
                            (uint32_t)tile1, rcol, 0};
        t2[i] = G32SetLayer{L[i]->u_g32, nullptr, L[i]->s1, L[i]->bias, L[i]->dout_p, L[i]->dout, L[i]->r_p,
                            (uint32_t)tile2, rcol, ycol};
        tile1 += L[i]->r_p / 128;
        tile2 += L[i]->dout_p / 128;
        rcol += L[i]->r_p;
        ycol += L[i]->dout;
    }
}

bool g32_set_fits(const qbk_factor *const *L, size_t n, size_t N) {
    if (N == 0 || N > (size_t)G32Small::BN) return false;
    for (size_t i = 0; i < n; i++)
        if (L[i]->din != L[0]->din || L[i]->din % 8 != 0) return false;
    return true;
}

struct G32SetPlan {
    int split;
    size_t rtot, tiles1, tiles2, o_part, o_t, bytes;
};

static G32SetPlan g32_set_plan(const qbk_factor *const *L, size_t n, size_t N) {
    G32SetPlan p{};
    for (size_t i = 0; i < n; i++) {
        p.rtot += L[i]->r_p;
        p.tiles2 += L[i]->dout_p / 128;
    }
    p.tiles1 = p.rtot / 128;
    const size_t bn = N <= (size_t)G32Tiny::BN ? G32Tiny::BN : G32Small::BN;
    const size_t tiles = div_ceil(N, bn) * p.tiles1;
    p.split = 1;
    while (tiles * p.split < (size_t)L[0]->num_cus && p.split < 8 && L[0]->din_p / (G_BK * 2 * p.split) >= 4)
        p.split *= 2;
    size_t off = 0;
    auto take = [&](size_t b) {
        const size_t o = off;
        off += round_up(b ? b : 4, 256);
        return o;
    };
    p.o_part = take(p.split > 1 ? (size_t)p.split * N * p.rtot * 4 : 0);
    p.o_t = take(N * p.rtot * 2);
    p.bytes = off;
    return p;
}

size_t g32_set_workspace(const qbk_factor *const *L, size_t n, size_t N) { return g32_set_plan(L, n, N).bytes; }

int g32_set_run(const qbk_factor *const *L, size_t n, const G32SetLayer *tab1, const G32SetLayer *tab2, size_t N,
                const void *x, bool xf32, void *y, bool ybf16, void *ws, hipStream_t s) {
    const G32SetPlan p = g32_set_plan(L, n, N);
    char *w = (char *)ws;
    float *part = (float *)(w + p.o_part);
    uint16_t *t = (uint16_t *)(w + p.o_t);
    G32Args a{};
    a.K_p = L[0]->din_p;
    a.N = N;
    a.x = x;
    a.din = L[0]->din;
    a.split = p.split;
    a.part = part;
    a.t_out = t;
    a.k_per_split = round_up(div_ceil(L[0]->din_p, p.split), G_BK);
    a.ld_out = p.rtot;
    a.ld_act = L[0]->din_p;
    a.set = tab1;
    a.n_set = (uint32_t)n;
    a.sign_mask = 0x80008000u;
    a.one_pair = 0x3F803F80u;
    if (xf32)
        g32_launch_any<1, 2>(a, p.tiles1 * 128, p.split, false, s);
    else
        g32_launch_any<1, 1>(a, p.tiles1 * 128, p.split, false, s);
    QBK_HIP(hipGetLastError());
    if (p.split > 1) {
        const size_t chunks = N * p.rtot / 8;
        hipLaunchKernelGGL(g32_reduce_kernel, dim3((unsigned)div_ceil(chunks, 256)), dim3(256), 0, s,
                           (const float *)part, p.split, N * p.rtot, p.rtot, p.rtot, t, chunks);
        QBK_HIP(hipGetLastError());
    }
    bool vec = (uintptr_t)y % 16 == 0;
    for (size_t i = 0; i < n; i++) vec = vec && L[i]->dout % 8 == 0;
    G32Args b{};
    b.N = N;
    b.act = t;
    b.y = y;
    b.y_bf16 = ybf16;
    b.vec_y = vec;
    b.split = 1;
    b.ld_act = p.rtot;
    b.set = tab2;
    b.n_set = (uint32_t)n;
    b.sign_mask = 0x80008000u;
    b.one_pair = 0x3F803F80u;
    g32_launch_any<2, 0>(b, p.tiles2 * 128, 1, false, s);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int g32_run(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16, void *ws,
            hipStream_t s) {
    const G32Plan p = g32_plan(L, N);
    {
        // the epilogue's 68 KiB exceed the 64 KiB default; the attribute is
        // per device, set once on each under a lock (callers may share a ctx)
        static std::mutex mu;
        static uint64_t done = 0;
        int dev = 0;
        QBK_HIP(hipGetDevice(&dev));
        std::lock_guard<std::mutex> lock(mu);
        if (dev < 64 && !((done >> dev) & 1)) {
            for (const void *k : {(const void *)g32_kernel<1, 0, 4, 2, 2>, (const void *)g32_kernel<1, 1, 4, 2, 2>,
                                  (const void *)g32_kernel<1, 2, 4, 2, 2>, (const void *)g32_kernel<2, 0, 4, 2, 2>})
                QBK_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, G32Big::LDS));
            done |= 1ull << dev;
        }
    }
    char *w = (char *)ws;
    uint16_t *z = (uint16_t *)(w + p.o_z), *t = (uint16_t *)(w + p.o_t);
    float *part = (float *)(w + p.o_part);
    // Stage 1 forms z itself from 16-byte chunks of x when they line up
    // (din % 8 == 0, x aligned); otherwise g32_prep_kernel stages z first.
    const bool fused = L->din % 8 == 0 && (uintptr_t)x % 16 == 0;
    if (!fused) {
        const size_t chunks = N * L->din_p / 8;
        dim3 g((unsigned)div_ceil(chunks, 256));
        if (xf32)
            hipLaunchKernelGGL((g32_prep_kernel<true>), g, dim3(256), 0, s, x, (const float *)L->s2, L->din,
                               L->din_p, N, z);
        else
            hipLaunchKernelGGL((g32_prep_kernel<false>), g, dim3(256), 0, s, x, (const float *)L->s2, L->din,
                               L->din_p, N, z);
        QBK_HIP(hipGetLastError());
    }
    G32Args a{};
    a.sg = L->vt_g32;
    a.M_p = L->r_p;
    a.K_p = L->din_p;
    a.M_valid = L->r;
    a.N = N;
    a.act = z;
    a.x = x;
    a.s2 = L->s2;
    a.din = L->din;
    a.split = p.split;
    a.part = part;
    a.t_out = t;
    a.ld_out = L->r_p;
    a.ld_act = L->din_p;
    a.k_per_split = round_up(div_ceil(L->din_p, p.split), G_BK);
    a.sign_mask = 0x80008000u;
    a.one_pair = 0x3F803F80u;
    const bool big1 = g32_big1(L, N);
    if (!fused)
        g32_launch_any<1, 0>(a, L->r_p, p.split, big1, s);
    else if (xf32)
        g32_launch_any<1, 2>(a, L->r_p, p.split, big1, s);
    else
        g32_launch_any<1, 1>(a, L->r_p, p.split, big1, s);
    QBK_HIP(hipGetLastError());
    if (p.split > 1) {
        const size_t chunks = N * L->r_p / 8;
        hipLaunchKernelGGL(g32_reduce_kernel, dim3((unsigned)div_ceil(chunks, 256)), dim3(256), 0, s,
                           (const float *)part, p.split, N * L->r_p, L->r_p, L->r, t, chunks);
        QBK_HIP(hipGetLastError());
    }
    G32Args b{};
    b.sg = L->u_g32;
    b.M_p = L->dout_p;
    b.K_p = L->r_p;
    b.M_valid = L->dout;
    b.N = N;
    b.act = t;
    b.y = y;
    b.s1 = L->s1;
    b.bias = L->bias;
    b.y_bf16 = ybf16;
    b.vec_y = L->dout % 8 == 0 && (uintptr_t)y % 16 == 0;
    b.sign_mask = 0x80008000u;
    b.one_pair = 0x3F803F80u;
    b.split = p.split2;
    b.part = (float *)(w + p.o_part2);
    b.ld_out = L->dout_p;
    b.ld_act = L->r_p;
    b.k_per_split = round_up(div_ceil(L->r_p, p.split2), G_BK);
    g32_launch_any<2, 0>(b, L->dout_p, p.split2, g32_big(L->dout_p, N, L->num_cus), s);
    QBK_HIP(hipGetLastError());
    if (p.split2 > 1) {
        const size_t chunks = N * L->dout_p / 8;
        hipLaunchKernelGGL(g32_reduce_y_kernel, dim3((unsigned)div_ceil(chunks, 256)), dim3(256), 0, s,
                           (const float *)b.part, p.split2, N * L->dout_p, L->dout_p, L->dout, L->s1, L->bias, y,
                           ybf16 ? 1 : 0, b.vec_y, chunks);
        QBK_HIP(hipGetLastError());
    }
    return QBK_OK;
}

}  // namespace qbk
