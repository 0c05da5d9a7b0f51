// gemm.hip -- the factor linear's prefill GEMM on the fp4 x fp8 scaled MFMA,
// both stages in one launch.
//
//   t = bf16(Vb^T z), z = bf16(s2 * x);  y = bf16(Ub t) * s1 + bias
//                              (engine/mod.rs:449-460, apply_bf16, per token)
//
// The decode GEMV's arithmetic (decode.hip) at any number of tokens: the
// +-1 signs are the fp4 A operand of v_mfma_scale_f32_16x16x128_f8f6f4, built
// in registers from the decode's sign layout (four VALU ops per 32 weights);
// the activations are the B operand, each split exactly into two fp8 e4m3
// columns (hi, lo) with E8M0 scales per 32-element block -- token b of a
// column group takes columns 2b, 2b + 1 of one MFMA, 8 tokens a group.
//
// One workgroup owns one column group (8 tokens) and all of the layer's rows:
//   1. x of its tokens becomes stage 1's operand chunk by chunk (16 slices of
//      128 k a chunk, double buffered in LDS): z = bf16(s2 * x) and its
//      hi/lo split, formed once per token;
//   2. stage 1: each wave takes 64-row groups of Vb^T (r) round robin and
//      accumulates them over all chunks, two row groups sharing each B
//      fragment;
//   3. its epilogue forms t = bf16(acc) and writes it as stage 2's operand
//      into LDS (the 32 rows of a scale block lie in one wave's row group, so
//      the block maxima are two lane shuffles);
//   4. stage 2: each wave takes 64-row groups of Ub (dout) round robin, two
//      at a time, over t's slices in LDS, and writes y = bf16(acc) * s1 + bias.
// Nothing between the stages leaves the CU: no operand prep launch, no split
// K partials, no t round trip through memory.  Every workgroup reads all of
// the layer's signs; they stay in the XCD's L2 (a config-2 layer is 1 MiB).
// Sign words stream through per-wave register rings, several slices ahead
// of the MFMAs that use them.
//
// Where the time goes (config 2, B = 2048, measured per wave): an MFMA of
// this shape holds a SIMD 32 cycles, but the SIMD's VALU ops do not overlap
// it freely -- each VALU op costs about 4 cycles on top past the first few
// in an MFMA's shadow -- so the VALU work per MFMA (4 ops building the signs,
// plus the operand conversion and the epilogues) sets the pace as much as
// the MFMAs do.  Hence: scaled fp8 conversions (one op for multiply and
// convert), pair sums folded into DPP adds, and wave priorities that keep the
// waves of a SIMD level so that none is left to run alone at the end.
#include <mutex>

#include "factor_internal.h"
#include "q4_operand.h"

namespace qbk {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4_t gu4_t;

#define Q4G_WAVES 16
#define Q4G_CH 16         // slices of x per LDS chunk (2048 k)
#define Q4G_SLICE 2112    // LDS bytes of one slice's operand: 2 KiB of fp8 + 64 scale bytes
#define Q4G_SC 2048       // offset of the scale bytes within a slice
#define Q4G_MAX_RG1 32    // stage-1 row groups (r_p / 64) the accumulators hold: 2 a wave
#define Q4G_SCALE_A 125   // the fp4 signs' E8M0 scale 2^-2 (decode.hip's q4_signs)

struct Q4GArgs {
    const uint32_t *bits1, *bits2;  // Vb^T and Ub in the decode layout [rows_p/64][K/128][64][4]
    const float *s2, *s1, *bias;
    const void *x;                  // [N][din] bf16 or f32
    void *y;                        // [N][dout] bf16 or f32
    uint32_t N, din, ns1;           // tokens, din, stage-1 slices (din_q / 128)
    uint32_t r, n_rg1, ns2;         // rank, stage-1 row groups (r_p / 64), stage-2 slices (r_q / 128)
    uint32_t dout, n_rg2;           // dout, stage-2 row groups (dout_p / 64)
    int vec_x, vec_y;               // x rows allow 16-byte loads; y rows allow 4-element stores
    uint32_t c7;                    // 0x77777777
    uint16_t *t_out;                // t bf16 [N][r_p] as well (zero past r), or null
    uint32_t r_p;
    const float *resid;             // f32 [N][dout] added to an f32 y (the block's residual), or null
};

__device__ __forceinline__ i32x8_t q4g_signs(uint32_t w, uint32_t c7) {
    i32x8_t av;
    av[0] = (int)((w << 3) | c7);
    av[1] = (int)((w << 2) | c7);
    av[2] = (int)((w << 1) | c7);
    av[3] = (int)(w | c7);
    av[4] = av[5] = av[6] = av[7] = 0;
    return av;
}

// A workgroup barrier that orders LDS only: HIP's __syncthreads() also
// fences global memory, which waits for every load in flight -- the sign
// words the rings hold ahead -- at each barrier.
__device__ __forceinline__ void q4g_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The B fragment and scale byte of lane (col, G) for one slice in LDS.
__device__ __forceinline__ void q4g_bfrag(const uint8_t *slice, int lane, i32x8_t &bv, int &bs) {
    const uint4 b0 = *(const uint4 *)(slice + lane * 16);
    const uint4 b1 = *(const uint4 *)(slice + 1024 + lane * 16);
    bv = i32x8_t{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    bs = slice[Q4G_SC + lane];
}

__device__ __forceinline__ void q4g_mfma4(f32x4_t acc[4], const u32x4_t &w, const i32x8_t &bv, int bs, uint32_t c7) {
    acc[0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q4g_signs(w.x, c7), bv, acc[0], 4, 0, 0, Q4G_SCALE_A, 0, bs);
    acc[1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q4g_signs(w.y, c7), bv, acc[1], 4, 0, 0, Q4G_SCALE_A, 0, bs);
    acc[2] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q4g_signs(w.z, c7), bv, acc[2], 4, 0, 0, Q4G_SCALE_A, 0, bs);
    acc[3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q4g_signs(w.w, c7), bv, acc[3], 4, 0, 0, Q4G_SCALE_A, 0, bs);
}

// One run of 16 activations of x in registers (the loads of a chunk are
// issued a chunk ahead of their conversion).
template <bool XF32>
struct Q4GRun {
    u32x4_t xr[XF32 ? 4 : 2];
    u32x4_t sr[4];
};

template <bool XF32>
__device__ __forceinline__ void q4g_load_run(const Q4GArgs &a, size_t n, size_t k0, Q4GRun<XF32> &R) {
    if (n < a.N && a.vec_x && k0 + 16 <= a.din) {
        const gu4_t *xs = (const gu4_t *)((const char *)a.x + (n * a.din + k0) * (XF32 ? 4 : 2));
#pragma unroll
        for (int q = 0; q < (XF32 ? 4 : 2); q++) {
            R.xr[q] = xs[q];
        }
        const gu4_t *ss = (const gu4_t *)(a.s2 + k0);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            R.sr[q] = ss[q];
        }
        return;
    }
    // the last run of a row, a token past N, or rows without 16-byte
    // pieces: element by element, zero past din (x) and past N (token)
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const size_t k = k0 + e;
        const bool ok = n < a.N && k < a.din;
        uint32_t xv = 0, sv = 0;
        if (ok) {
            xv = XF32 ? ((const uint32_t *)a.x)[n * a.din + k] : ((const uint16_t *)a.x)[n * a.din + k];
            sv = __float_as_uint(a.s2[k]);
        }
        if constexpr (XF32)
            R.xr[e >> 2][e & 3] = xv;
        else if (e & 1)
            R.xr[e >> 3][(e & 7) >> 1] |= xv << 16;
        else
            R.xr[e >> 3][(e & 7) >> 1] = xv;
        R.sr[e >> 2][e & 3] = sv;
    }
}

// Run (b, j, r) of a chunk -> the LDS operand: hi bytes to column 2b, lo to
// 2b + 1 of B lane group r / 2, half r % 2; the scale pair of the run's
// block from the runs with r & 2 == 0 (decode.hip's layout with 16 columns).
template <bool XF32>
__device__ __forceinline__ void q4g_store_run(const Q4GRun<XF32> &R, uint8_t *slice, int b, int r) {
    float z[16];
    if constexpr (XF32) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int u = 0; u < 4; u++)
                z[4 * q + u] = bf16_to_f32(f32_to_bf16(__uint_as_float(R.sr[q][u]) * __uint_as_float(R.xr[q][u])));
    } else {
        q4_run_z(R.xr, R.sr, z);
    }
    uint32_t hw[4], lw[4];
    int e_hi, e_lo;
    q4_run_operand(z, hw, lw, e_hi, e_lo);
    uint8_t *p = slice + (r & 1) * 1024 + ((r >> 1) * 16 + 2 * b) * 16;
    *(uint4 *)p = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(p + 16) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if ((r & 2) == 0)
        *(uint16_t *)(slice + Q4G_SC + (2 * (r & 1) + (r >> 2)) * 16 + 2 * b) =
            (uint16_t)((e_hi + 127) | ((e_lo + 127) << 8));
}

// The value of the lane's column partner (lane ^ 1: the other half of a
// token's hi / lo pair) -- a DPP quad permutation, no LDS round trip.
// Every source lane of a quad permutation exists, so bound_ctrl changes
// nothing here (all lanes are active where it is called); set, it lets the
// compiler fold the move into the add that uses it (v_add_f32_dpp).
__device__ __forceinline__ float q4g_pair(float a) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0xB1, 0xF, 0xF, true));
}

// max over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lane groups holding a
// column) of non-negative values: v_permlane16/32_swap of a register with
// itself hands each lane the other half's value in one of its two results,
// in the VALU.
__device__ __forceinline__ float q4g_max4(float v) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float a = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// Stage 1's epilogue for row group g (acc: its four row tiles): t =
// bf16((hi + lo) / 1.5), zero past r, written as stage 2's operand.  Lane
// (col, G) of row tile rt holds rows 64g + 16rt + 4G + i of column col; both
// lanes of a column pair form the same t.  Stage-2 slice g / 2, run 4(g & 1)
// + rt, element 4G + i: lane (col, G) writes four consecutive bytes -- the hi
// bytes from an even column, the lo bytes from an odd one.  Row tiles rt and
// rt + 2 form one scale block (runs u, u ^ 2): its maxima are over the lane's
// eight values and the lanes 16, 32 and 48 apart (q4g_max4).
__device__ __forceinline__ void q4g_epilogue1(const f32x4_t acc[4], uint8_t *tbuf, size_t g, uint32_t r,
                                              int lane, uint16_t *t_out, size_t n, uint32_t r_p) {
    const int col = lane & 15, G = lane >> 4;
    uint8_t *slice = tbuf + (g >> 1) * Q4G_SLICE;
    const int half = (int)(g & 1);
#pragma unroll
    for (int pr = 0; pr < 2; pr++) {
        float t[2][4];
        uint32_t tw[2][2];
        float amax = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const int rt = pr + 2 * tt;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = q4_unscale(acc[rt][i] + q4g_pair(acc[rt][i]));
            const uint32_t row0 = (uint32_t)(64 * g) + 16 * rt + 4 * G;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint32_t w = f32x2_to_bf16x2(v[2 * h], v[2 * h + 1]);
                if (row0 + 2 * h >= r) w &= 0xffff0000u;
                if (row0 + 2 * h + 1 >= r) w &= 0x0000ffffu;
                tw[tt][h] = w;
                t[tt][2 * h] = __uint_as_float(w << 16);
                t[tt][2 * h + 1] = __uint_as_float(w & 0xffff0000u);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(t[tt][i]));
        }
        if (t_out && !(col & 1)) {
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
                *(uint2 *)(t_out + n * r_p + 64 * g + 16 * (pr + 2 * tt) + 4 * G) = make_uint2(tw[tt][0], tw[tt][1]);
        }
        amax = q4g_max4(amax);
        const int e_hi = amax > 0.0f ? e8m0_of(amax) : 0;
        const float sc_hi = pow2f(e_hi);
        uint32_t hw[2];
        float rmax = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            hw[tt] = q4_fp8x4(t[tt][0], t[tt][1], t[tt][2], t[tt][3], sc_hi);
            float b[4];
            q4_f32x4(hw[tt], sc_hi, b);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                t[tt][i] -= b[i];  // exact residuals
                rmax = fmaxf(rmax, fabsf(t[tt][i]));
            }
        }
        rmax = q4g_max4(rmax);
        const int e_lo = rmax > 0.0f ? e8m0_of(rmax) : 0;
        const float sc_lo = pow2f(e_lo);
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const int rt = pr + 2 * tt, u = 4 * half + rt;
            uint32_t w = hw[tt];
            if (col & 1) w = q4_fp8x4(t[tt][0], t[tt][1], t[tt][2], t[tt][3], sc_lo);
            *(uint32_t *)(slice + (u & 1) * 1024 + ((u >> 1) * 16 + col) * 16 + 4 * G) = w;
        }
        if (G == 0) slice[Q4G_SC + (2 * pr + half) * 16 + col] = (uint8_t)((col & 1 ? e_lo : e_hi) + 127);
    }
}

// Stage 2's epilogue for row group g: y = bf16((hi + lo) / 1.5) * s1 + bias,
// s1 and bias of the group's 64 rows read from the wave's LDS region sb
// ([64] s1 then [64] bias).  Lane (col, G) of row tile rt holds rows 16rt +
// 4G + i, i < 4, of column col.  The two lanes of a column pair split the
// work: both form the four pair sums by DPP adds, the even lane finishes
// rows 0, 1 and the odd lane rows 2, 3 of token col / 2; the odd lane then
// hands its two results back and the even lane stores all four (stores from
// all 64 lanes of two rows each measured 2 us slower at config 2, B = 2048).
__device__ __forceinline__ void q4g_y2(const f32x4_t acc[4], int rt, bool odd, const float *sb, int r2, float y[2]) {
    const float2 s1v = *(const float2 *)(sb + r2);
    const float2 biv = *(const float2 *)(sb + 64 + r2);
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = acc[rt][i] + q4g_pair(acc[rt][i]);
    const float v0 = q4_unscale(odd ? x[2] : x[0]), v1 = q4_unscale(odd ? x[3] : x[1]);
    const uint32_t u = f32x2_to_bf16x2(v0, v1);
    y[0] = __uint_as_float(u << 16) * s1v.x + biv.x;
    y[1] = __uint_as_float(u & 0xffff0000u) * s1v.y + biv.y;
}

__device__ __forceinline__ uint32_t q4g_pair_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);
}

// VECY: y rows take 4-element stores (dout a multiple of 4, y aligned), so
// a lane pair's four rows are all in or all out; otherwise element by
// element.  The two are separate kernels: one store per row tile keeps the
// count of memory operations in flight the same on every path, which the
// waits on the sign ring rely on.
template <bool VECY>
__device__ __forceinline__ void q4g_epilogue2(const f32x4_t acc[4], const Q4GArgs &a, size_t g, const float *sb,
                                              size_t n0, int lane, bool ybf16) {
    const int col = lane & 15, G = lane >> 4, odd = col & 1;
    const size_t n = n0 + (col >> 1);
#pragma unroll
    for (int rt = 0; rt < 4; rt++) {
        const int r2 = 16 * rt + 4 * G + 2 * odd;  // this lane's first row within the group
        float y[2];
        q4g_y2(acc, rt, odd != 0, sb, r2, y);
        // the odd lane's rows 2, 3, handed to the even lane (all lanes active)
        const uint32_t w = f32x2_to_bf16x2(y[0], y[1]);
        const uint32_t wp = q4g_pair_u(w);
        const float y2 = __uint_as_float(q4g_pair_u(__float_as_uint(y[0])));
        const float y3 = __uint_as_float(q4g_pair_u(__float_as_uint(y[1])));
        const size_t row0 = 64 * g + r2;
        if (odd || n >= a.N || row0 >= a.dout) continue;
        if constexpr (VECY) {
            if (ybf16) {
                *(uint2 *)((uint16_t *)a.y + n * a.dout + row0) = make_uint2(w, wp);
            } else {
                float4 o = make_float4(y[0], y[1], y2, y3);
                if (a.resid) {
                    const float4 rv = *(const float4 *)(a.resid + n * a.dout + row0);
                    o = make_float4(o.x + rv.x, o.y + rv.y, o.z + rv.z, o.w + rv.w);
                }
                *(float4 *)((float *)a.y + n * a.dout + row0) = o;
            }
        } else {
            const float yy[4] = {y[0], y[1], y2, y3};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (row0 + i >= a.dout) break;
                if (ybf16)
                    ((uint16_t *)a.y)[n * a.dout + row0 + i] = f32_to_bf16(yy[i]);
                else
                    ((float *)a.y)[n * a.dout + row0 + i] =
                        a.resid ? yy[i] + a.resid[n * a.dout + row0 + i] : yy[i];
            }
        }
    }
}

// The wave's issue priority, 0 (lowest) to 3: lowered as a wave gets ahead
// so that the SIMD's scheduler, which otherwise favours the oldest wave,
// keeps the waves of a SIMD level and they finish together -- a wave left
// alone at the end runs its MFMAs and VALU work with nothing to overlap.
__device__ __forceinline__ void q4g_prio(uint32_t level) {
    switch (level) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
    }
}

// Sign words stream through a ring of Q4G_RING units per wave, all in
// flight: a unit's loads are issued Q4G_RING units before its MFMAs.
// Loads are unconditional (indices clamped into the layer) so that the
// compiler's waits stay counted ones; only MFMAs sit under branches.
#define Q4G_RING 4

// NG1: stage-1 row groups a wave accumulates (1: r_p <= 1024, 2: r_p <=
// 2048).  Stage 1's unit: one slice of the wave's NG1 row groups (their B
// fragment read once); stage 2's unit: one slice of a pair of row groups.
template <bool XF32, bool YBF16, int NG1, bool VECY>
__global__ void __launch_bounds__(64 * Q4G_WAVES) q4g_kernel(Q4GArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t q4g_lds[];
    uint8_t *xbuf = q4g_lds;                             // [2][Q4G_CH slices]
    uint8_t *tbuf = q4g_lds + 2 * Q4G_CH * Q4G_SLICE;    // [ns2 slices]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t n0 = (size_t)blockIdx.x * 8;
    const uint32_t c7 = a.c7;
    const gu4_t *b1 = (const gu4_t *)a.bits1, *b2 = (const gu4_t *)a.bits2;

    // ---- stage 1 --------------------------------------------------------
    // this wave's row groups: wave + 8q, q < NG1 (those past the rank padded
    // to 128 load a clamped group and skip their MFMAs)
    const uint32_t nrg1 = a.n_rg1, ns1 = a.ns1;
    const int ng1 = wave < (int)nrg1 ? (int)((nrg1 - 1 - wave) / Q4G_WAVES) + 1 : 0;
    const uint32_t nch = (ns1 + Q4G_CH - 1) / Q4G_CH, nu1 = nch * Q4G_CH;
    // x conversion: thread (token b, slice j, run r) of each chunk, two waves a token
    const int xb = tid >> 7, xj = (tid >> 3) & 15, xr = tid & 7;
    Q4GRun<XF32> run;
    const gu4_t *g1p[NG1];
#pragma unroll
    for (int q = 0; q < NG1; q++) {
        uint32_t g = (uint32_t)wave + Q4G_WAVES * q;
        g = g < nrg1 ? g : nrg1 - 1;
        g1p[q] = b1 + (size_t)g * ns1 * 64 + lane;
    }
    f32x4_t acc1[NG1][4];
#pragma unroll
    for (int q = 0; q < NG1; q++)
#pragma unroll
        for (int rt = 0; rt < 4; rt++) acc1[q][rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // stage 1's ring: eight slices ahead for one group a wave, two for two
    // groups (four slices ahead of two groups held 128 VGPRs and spilled
    // 27 of them to scratch inside the chunk loop, 73 with f32 x; two
    // slices spill none with bf16 x: config 3's prefill 0.539-0.541 ->
    // 0.493-0.511 ms a decoder layer, three slices 0.506-0.507)
    constexpr int R1 = NG1 == 1 ? 8 : 2;
    u32x4_t ring1[R1][NG1];
#define Q4G_ISSUE1(U, SLOT)                                                             \
    {                                                                                   \
        uint32_t s_ = (U);                                                              \
        s_ = s_ < ns1 ? s_ : ns1 - 1;                                                   \
        _Pragma("unroll") for (int q = 0; q < NG1; q++) ring1[SLOT][q] = g1p[q][(size_t)s_ * 64]; \
    }

    // chunk 0 into buffer 0; the first units' sign words in flight
    q4g_load_run<XF32>(a, n0 + xb, 128 * xj + 16 * xr, run);
#pragma unroll
    for (int k = 0; k < R1; k++) Q4G_ISSUE1((uint32_t)k, k)
    q4g_store_run<XF32>(run, xbuf + xj * Q4G_SLICE, xb, xr);
    q4g_lds_barrier();

    for (uint32_t c = 0; c < nch; c++) {
        const bool more = c + 1 < nch;
        if (more) q4g_load_run<XF32>(a, n0 + xb, (size_t)(c + 1) * (128 * Q4G_CH) + 128 * xj + 16 * xr, run);
        const uint8_t *xs = xbuf + (c & 1) * (Q4G_CH * Q4G_SLICE);
        // B fragments one slice ahead (within the chunk: the next chunk's
        // buffer is written behind the barrier that ends this one)
        i32x8_t bvq[2];
        int bsq[2];
        q4g_bfrag(xs, lane, bvq[0], bsq[0]);
#pragma unroll
        for (int j = 0; j < Q4G_CH; j++) {
            const int slot = j % R1, cur = j & 1;
            const uint32_t s = c * Q4G_CH + j;
            // the chunk ends at a barrier: keep the waves level up to it
            if (j % (Q4G_CH / 4) == 0) q4g_prio(3 - j / (Q4G_CH / 4));
            if (j + 1 < Q4G_CH) q4g_bfrag(xs + (j + 1) * Q4G_SLICE, lane, bvq[cur ^ 1], bsq[cur ^ 1]);
            if (s < ns1) {
#pragma unroll
                for (int q = 0; q < NG1; q++)
                    if (q < ng1) q4g_mfma4(acc1[q], ring1[slot][q], bvq[cur], bsq[cur], c7);
            }
            Q4G_ISSUE1(s + R1, slot)
        }
        if (more) q4g_store_run<XF32>(run, xbuf + ((c + 1) & 1) * (Q4G_CH * Q4G_SLICE) + xj * Q4G_SLICE, xb, xr);
        q4g_lds_barrier();
    }
#undef Q4G_ISSUE1
    (void)nu1;

    // ---- stage 2 --------------------------------------------------------
    // this wave's row groups wave + 16q, two at a time; a pair's units are
    // its slices, rounded up to the ring depth so that each unit's ring slot
    // is fixed at compile time (units past ns2 load a clamped slice and skip
    // their MFMAs).  The ring runs on across pairs: (pi, si) is the unit
    // issued.  The epilogue, with the only stores and s1 / bias loads, sits
    // between pairs, outside the unit loop, so the waits on the ring keep
    // their counts.  s1 and bias of a pair's rows are loaded one pair ahead
    // and staged through the wave's LDS region.
    const uint32_t nrg2 = a.n_rg2, ns2 = a.ns2, dout = a.dout;
    const int ng2 = wave < (int)nrg2 ? (int)((nrg2 - 1 - wave) / Q4G_WAVES) + 1 : 0;
    const uint32_t np2 = (uint32_t)(ng2 + 1) >> 1;
    const uint32_t nsr = (ns2 + Q4G_RING - 1) / Q4G_RING * Q4G_RING;
    float *sb = (float *)(tbuf + ns2 * Q4G_SLICE) + wave * 256;  // [2 groups][s1 64 | bias 64]
    f32x4_t acc2[2][4];
    u32x4_t ring2[Q4G_RING][2];
    uint32_t pi = 0, si = 0;
#define Q4G_ISSUE2(SLOT)                                                                \
    {                                                                                   \
        const uint32_t p_ = pi < np2 ? pi : np2 - 1;                                    \
        const uint32_t s_ = si < ns2 ? si : ns2 - 1;                                    \
        _Pragma("unroll") for (int w = 0; w < 2; w++) {                                 \
            uint32_t g = (uint32_t)wave + Q4G_WAVES * (2 * p_ + w);                     \
            g = g < nrg2 ? g : nrg2 - 1;                                                \
            ring2[SLOT][w] = b2[((size_t)g * ns2 + s_) * 64 + lane];                    \
        }                                                                               \
        if (++si == nsr) {                                                              \
            si = 0;                                                                     \
            ++pi;                                                                       \
        }                                                                               \
    }
    // s1 and bias of lane l's row in pair P's two groups
    float sv[2][2];
#define Q4G_SCALES2(P)                                                                  \
    _Pragma("unroll") for (int w = 0; w < 2; w++) {                                     \
        size_t row = ((size_t)wave + Q4G_WAVES * (2 * (P) + w)) * 64 + lane;            \
        row = row < dout ? row : dout - 1;                                              \
        sv[w][0] = a.s1[row];                                                           \
        sv[w][1] = a.bias[row];                                                         \
    }
    // the first units' sign words and pair 0's scales in flight under
    // stage 1's epilogue
    if (np2 > 0) {
        Q4G_SCALES2(0u)
#pragma unroll
        for (int k = 0; k < Q4G_RING; k++) Q4G_ISSUE2(k)
    }

    // stage 1's epilogue: t -> stage 2's operand in LDS
#pragma unroll
    for (int q = 0; q < NG1; q++)
        if (q < ng1) {
            // tokens past N keep t to themselves
            const size_t n = n0 + ((lane & 15) >> 1);
            q4g_epilogue1(acc1[q], tbuf, (size_t)wave + Q4G_WAVES * q, a.r, lane, n < a.N ? a.t_out : nullptr, n,
                          a.r_p);
        }
    q4g_lds_barrier();

    for (uint32_t p = 0; p < np2; p++) {
        const bool two = 2 * p + 1 < (uint32_t)ng2;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int rt = 0; rt < 4; rt++) acc2[h][rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        i32x8_t bvq[2];
        int bsq[2];
        q4g_bfrag(tbuf, lane, bvq[0], bsq[0]);
        for (uint32_t s0 = 0; s0 < nsr; s0 += Q4G_RING) {
            q4g_prio(3 - 4 * (p * nsr + s0) / (np2 * nsr));
#pragma unroll
            for (int k = 0; k < Q4G_RING; k++) {
                const int cur = k & 1;
                const uint32_t s = s0 + k, sn = s + 1 < ns2 ? s + 1 : ns2 - 1;
                q4g_bfrag(tbuf + sn * Q4G_SLICE, lane, bvq[cur ^ 1], bsq[cur ^ 1]);
                if (s < ns2) {
                    q4g_mfma4(acc2[0], ring2[k][0], bvq[cur], bsq[cur], c7);
                    if (two) q4g_mfma4(acc2[1], ring2[k][1], bvq[cur], bsq[cur], c7);
                }
                Q4G_ISSUE2(k)
            }
        }
        // the pair is complete: its scales through LDS, then the next pair's in flight
#pragma unroll
        for (int w = 0; w < 2; w++) {
            sb[128 * w + lane] = sv[w][0];
            sb[128 * w + 64 + lane] = sv[w][1];
        }
        __builtin_amdgcn_wave_barrier();
        Q4G_SCALES2(p + 1 < np2 ? p + 1 : p)
        const size_t g0 = (size_t)wave + Q4G_WAVES * (2 * p);
        q4g_epilogue2<VECY>(acc2[0], a, g0, sb, n0, lane, YBF16);
        if (two) q4g_epilogue2<VECY>(acc2[1], a, g0 + Q4G_WAVES, sb + 128, n0, lane, YBF16);
        __builtin_amdgcn_wave_barrier();
    }
#undef Q4G_ISSUE2
#undef Q4G_SCALES2
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

// Every instantiation, indexed by xf32 << 3 | ybf16 << 2 | (NG1 == 2) << 1 | vecy.
#define Q4G_K(XF, YB, NG, VY) (const void *)q4g_kernel<XF, YB, NG, VY>
static const void *const q4g_kernels[16] = {
    Q4G_K(false, false, 1, false), Q4G_K(false, false, 1, true), Q4G_K(false, false, 2, false),
    Q4G_K(false, false, 2, true),  Q4G_K(false, true, 1, false), Q4G_K(false, true, 1, true),
    Q4G_K(false, true, 2, false),  Q4G_K(false, true, 2, true),  Q4G_K(true, false, 1, false),
    Q4G_K(true, false, 1, true),   Q4G_K(true, false, 2, false), Q4G_K(true, false, 2, true),
    Q4G_K(true, true, 1, false),   Q4G_K(true, true, 1, true),   Q4G_K(true, true, 2, false),
    Q4G_K(true, true, 2, true)};
#undef Q4G_K

// x chunks, stage 2's operand, each wave's s1 / bias staging (1 KiB)
static uint32_t q4g_lds_bytes(const qbk_factor *L) {
    return (uint32_t)((2 * Q4G_CH + L->r_q / 128) * Q4G_SLICE + Q4G_WAVES * 1024);
}

bool q4g_fits(const qbk_factor *L, size_t N) {
    return N > 0 && N <= 0x7fffffff && L->r > 0 && L->r_p / 64 <= Q4G_MAX_RG1 && L->din > 0 &&
           L->din <= 0x7fffffff && L->dout > 0 && L->dout <= 0x7fffffff;
}

// The smallest batch the one-launch GEMM takes over from the two-stage one:
// its workgroups (8 tokens each) each stream all of a layer's signs, so its
// time barely depends on the batch; the two-stage GEMM's grows with it
// (measured at config 2, one-launch against two-stage: B = 256, 28.9 against
// 33.0 us; 512, 29.8 against 31.1; 768, 30.8 against 40.1; 2048, 35.5
// against 56); below, the two-stage GEMM splits each stage over row tiles
// and K.
#define Q4G_MIN_N 256

bool q4g_use(const qbk_factor *L, size_t N) { return N >= Q4G_MIN_N && q4g_fits(L, N); }

size_t gemm_workspace(const qbk_factor *L, size_t N) {
    return q4g_use(L, N) ? N * L->r_p * 2 : g32_workspace(L, N);
}

int gemm_run(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16, void *ws,
             hipStream_t s) {
    if (q4g_use(L, N)) return q4g_run(L, x, xf32, N, y, ybf16, (uint16_t *)ws, s);
    return g32_run(L, x, xf32, N, y, ybf16, ws, s);
}

int q4g_run(const qbk_factor *L, const void *x, bool xf32, size_t N, void *y, bool ybf16, uint16_t *t_out,
            hipStream_t s, const float *resid, const float *s2) {
    if (resid && ybf16) return fail(QBK_ERR_VALIDATION, "the GEMM adds a residual to an f32 output only");
    const uint32_t lds = q4g_lds_bytes(L);
    {
        // up to 67.5 KiB of LDS, past the 64 KiB default: the attribute is
        // per device, set once on each under a lock (callers may share a ctx)
        static std::mutex mu;
        static uint64_t done = 0;
        int dev = 0;
        QBK_HIP(hipGetDevice(&dev));
        std::lock_guard<std::mutex> lock(mu);
        if (dev < 64 && !((done >> dev) & 1)) {
            const uint32_t most = (2 * Q4G_CH + Q4G_MAX_RG1 / 2) * Q4G_SLICE + Q4G_WAVES * 1024;
            for (const void *k : q4g_kernels)
                QBK_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)most));
            done |= 1ull << dev;
        }
    }
    Q4GArgs a{};
    a.bits1 = L->vt_q4;
    a.bits2 = L->u_q4;
    a.s2 = s2 ? s2 : L->s2;
    a.s1 = L->s1;
    a.bias = L->bias;
    a.x = x;
    a.y = y;
    a.N = (uint32_t)N;
    a.din = (uint32_t)L->din;
    a.ns1 = (uint32_t)(L->din_q / 128);
    a.r = (uint32_t)L->r;
    a.n_rg1 = (uint32_t)(L->r_p / 64);
    a.ns2 = (uint32_t)(L->r_q / 128);
    a.dout = (uint32_t)L->dout;
    a.n_rg2 = (uint32_t)(L->dout_p / 64);
    a.vec_x = L->din % (xf32 ? 4 : 8) == 0 && (uintptr_t)x % 16 == 0;
    a.vec_y = L->dout % 4 == 0 && (uintptr_t)y % (ybf16 ? 8 : 16) == 0;
    a.c7 = 0x77777777u;
    a.t_out = t_out;
    a.r_p = (uint32_t)L->r_p;
    a.resid = resid;
    const dim3 grid((unsigned)div_ceil(N, 8)), block(64 * Q4G_WAVES);
    // one row group a wave in stage 1 up to 16 groups (r_p <= 1024), two up to 32
    const bool two = a.n_rg1 > Q4G_WAVES;
    const void *k = q4g_kernels[(xf32 ? 8 : 0) | (ybf16 ? 4 : 0) | (two ? 2 : 0) | (a.vec_y ? 1 : 0)];
    void *args[] = {&a};
    QBK_HIP(hipLaunchKernel(k, grid, block, args, lds, s));
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // namespace qbk
