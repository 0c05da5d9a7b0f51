// decode.hip -- the factor linear's decode GEMV (batch 1..32) on gfx950.
//
//   t = bf16(Vb^T z), z = bf16(s2 * x);  y = bf16(Ub t) * s1 + bias
//                                        (engine/mod.rs:449-460, apply_bf16)
//
// out[i] = sum_k s(i,k) a_k runs on v_mfma_scale_f32_16x16x128_f8f6f4:
// A = the +-1 signs as fp4 e2m1, built in registers from the packed words;
// B = the activations split into two fp8 e4m3 columns, a = hi*2^e_hi +
// lo*2^e_lo, one E8M0 scale per 32-element block and column (a bf16 value
// has 8 significant bits: hi keeps the top 4, lo the rest).  Token b of a
// decode batch uses columns 2b, 2b+1.  Each 128-k slice of a 16-row tile is
// one MFMA over 256 bytes of packed signs per 16 columns (8 tokens): batches
// beyond 8 run column groups of 16 against the same sign registers, so the
// signs are still read once.
//
// A launch covers any set of layers (any shapes): each stage reads a device
// table of Q4Layer entries (factor_internal.h) and finds its layer from the
// workgroup index.  Three launches per decode:
//   1. q4_prep_kernel (q4_prep_flat_kernel at batch 1 when every din is a
//      multiple of 128): x -> stage 1's fp8 operand;
//   2. q4_gemv_kernel<1>: t = bf16(Vb^T z), written by the epilogue straight
//      into stage 2's fp8 operand;
//   3. q4_gemv_kernel<2>: y = bf16(Ub t) * s1 + bias.
#include <string.h>

#include <algorithm>
#include <vector>

#include "factor_internal.h"
#include "q4_operand.h"

namespace qbk {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
// Pointers read from a layer table are generic to the compiler; loading
// through an address_space(1) pointer keeps them global loads (flat loads
// count against both vmcnt and lgkmcnt and defeat per-load waits).
typedef __attribute__((address_space(1))) const u32x4_t gu32x4_t;
typedef __attribute__((address_space(1))) const float gf32_t;
// The layer tables are never written by a kernel: reading them through the
// constant address space lets the compiler use scalar loads even after the
// kernel's own stores (a vector load of a pointer would wait on vmcnt).
typedef __attribute__((address_space(4))) const Q4Layer cq4layer_t;

#define Q4_U 8       // slices whose sign loads a wave issues together
// waves of a GEMV workgroup: four, or eight when eight waves split one row
// group's K (a lone layer of long K at batch 1)
#define Q4_NW(ks) ((ks) > 4 ? (ks) : 4)
#define Q4_PHASES 3  // prep x, stage 1 (+ stage 2's operand), stage 2

// One launch over a set of layers.
struct Q4Args {
    const Q4Layer *layers;       // this stage's table entries
    const uint32_t *wg_layer;    // GEMV: (layer, first row group) of each workgroup (null for one layer)
    uint32_t n_layers, n_wg;     // layers; workgroups doing work (GEMV)
    int batch, ncol;             // ncol = 2 * batch
    const void *act;             // stage 1 prep: x (bf16, or f32)
    void *out;                   // stage 2: y (bf16 or f32)
    uint8_t *op, *sc;            // this stage's fp8 operand [slice][4][ncol][32] and scales [slice][4][ncol]
    uint8_t *tb_op, *tb_sc;      // stage 1: stage 2's operand and scales
    int y_bf16, vec_ok;          // vec_ok: x rows allow 16-element vector loads
    uint32_t c7;                 // 0x77777777 (fp4 sign build)
    const float *resid;          // stage 2, f32 y: added to y (y = (t s1 + bias) + resid), or null
};

// The table entry of layer li (scalar loads).
__device__ __forceinline__ Q4Layer q4_entry(const Q4Args &a, uint32_t li) {
    const cq4layer_t *lp = (const cq4layer_t *)a.layers + li;
    Q4Layer L;
    L.bits = lp->bits;
    L.s_in = lp->s_in;
    L.s_out = lp->s_out;
    L.bias = lp->bias;
    L.s_out_h = lp->s_out_h;
    L.bias_h = lp->bias_h;
    L.rows_p = lp->rows_p;
    L.rows_valid = lp->rows_valid;
    L.ns = lp->ns;
    L.k_valid = lp->k_valid;
    L.slice0 = lp->slice0;
    L.tb_ns = lp->tb_ns;
    L.tb_slice0 = lp->tb_slice0;
    L.wg0 = lp->wg0;
    L.act0 = lp->act0;
    L.out0 = lp->out0;
    return L;
}

// The layer and first row group of workgroup wgi: one scalar load from the
// per-workgroup table (so that a workgroup's sign loads wait on two
// dependent scalar loads, not on a search); one layer: its row groups in
// order.
__device__ __forceinline__ void q4_work_of(const Q4Args &a, uint32_t wgi, uint32_t rg_per_wg, uint32_t &li,
                                           uint32_t &rg0) {
    if (a.n_layers == 1) {
        li = 0;
        rg0 = wgi * rg_per_wg;
        return;
    }
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t e = ((__attribute__((address_space(4))) const u32x2_t *)a.wg_layer)[wgi];
    li = e[0];
    rg0 = e[1];
}

// x -> stage 1's fp8 operand.  Workgroup (x, layer); one thread per run of
// 16 activations: (token b, slice s, run r) covers k = 128s + 16r .. +15.
template <bool XF32>
__global__ void __launch_bounds__(256) q4_prep_kernel(Q4Args a) {
    const uint32_t li = blockIdx.y;
    const Q4Layer L = q4_entry(a, li);
    const size_t n_runs = (size_t)a.batch * L.ns * 8;
    const size_t it = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = it < n_runs;  // dead threads still join the shuffle
    const size_t itc = live ? it : 0;
    const int r = (int)(itc & 7);
    const size_t s = (itc >> 3) % L.ns;
    const int b = (int)((itc >> 3) / L.ns);
    const size_t k0 = 128 * s + 16 * r;
    float z[16];
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    if (live) {
        const size_t off = L.act0 * (size_t)a.batch + (size_t)b * L.k_valid;
        const uint16_t *src = (const uint16_t *)a.act + off;
        const float *srcf = (const float *)a.act + off;
        const float *s2 = L.s_in;
        if (a.vec_ok && k0 + 15 < L.k_valid) {
            u32x4_t sr[4];
#pragma unroll
            for (int q = 0; q < 4; q++) sr[q] = *(const u32x4_t *)(s2 + k0 + 4 * q);
            if (XF32) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 f = *(const float4 *)(srcf + k0 + 4 * q);
                    const float v[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        z[4 * q + u] = bf16_to_f32(f32_to_bf16(__uint_as_float(sr[q][u]) * v[u]));
                }
            } else {
                const u32x4_t xr[2] = {*(const u32x4_t *)(src + k0), *(const u32x4_t *)(src + k0 + 8)};
                q4_run_z(xr, sr, z);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const size_t k = k0 + e;
                if (k >= L.k_valid) continue;
                const float v = XF32 ? srcf[k] : bf16_to_f32(src[k]);
                z[e] = bf16_to_f32(f32_to_bf16(s2[k] * v));
            }
        }
    }
    uint32_t hw[4], lw[4];
    int e_hi, e_lo;
    q4_run_operand(z, hw, lw, e_hi, e_lo);
    if (!live) return;
    const size_t slot = q4_run_slot(L.slice0 + s, r, a.ncol, b);  // hi column; lo is slot + 1
    const size_t byte = 16 * (r & 1);
    *(uint4 *)(a.op + slot * 32 + byte) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(a.op + (slot + 1) * 32 + byte) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if ((r & 2) == 0) {
        const size_t sc = q4_run_scale(L.slice0 + s, r, a.ncol, b);
        a.sc[sc] = (uint8_t)(e_hi + 127);
        a.sc[sc + 1] = (uint8_t)(e_lo + 127);
    }
}

// The same at batch 1 when every din is a multiple of 128: x is then the
// concatenation of the layers' inputs and stage 1's slices follow the same
// order, so run t (k = 16t .. 16t + 15 of the concatenated x) belongs to
// global slice t / 8, and s2cat holds the layers' s2 concatenated the same
// way -- no per-layer table lookup ahead of the loads (one dependent memory
// round trip instead of two).
template <bool S2H>
__global__ void __launch_bounds__(256) q4_prep_flat_kernel(const uint16_t *x, const void *s2cat, uint8_t *op,
                                                           uint8_t *sc, uint32_t n_runs) {
    const uint32_t t0 = blockIdx.x * 256 + threadIdx.x;
    const bool live = t0 < n_runs;
    // lanes past the end shadow the last slice's runs (n_runs is a multiple
    // of 8, so a shuffle partner at distance 2 shadows the same slice)
    const uint32_t t = live ? t0 : n_runs - 8 + (t0 & 7);
    const size_t k0 = (size_t)t * 16;
    const gu32x4_t *xs = (const gu32x4_t *)(x + k0);
    const u32x4_t xr[2] = {xs[0], xs[1]};
    u32x4_t sr[4];
    if (S2H) {  // fp16 s2, widened exactly
        const gu32x4_t *ss = (const gu32x4_t *)((const uint16_t *)s2cat + k0);
        const u32x4_t h[2] = {ss[0], ss[1]};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t w0 = h[q >> 1][2 * (q & 1)], w1 = h[q >> 1][2 * (q & 1) + 1];
            sr[q] = u32x4_t{__float_as_uint(h16_to_f32(w0 & 0xffff)), __float_as_uint(h16_to_f32(w0 >> 16)),
                            __float_as_uint(h16_to_f32(w1 & 0xffff)), __float_as_uint(h16_to_f32(w1 >> 16))};
        }
    } else {
        const gu32x4_t *ss = (const gu32x4_t *)((const float *)s2cat + k0);
        sr[0] = ss[0];
        sr[1] = ss[1];
        sr[2] = ss[2];
        sr[3] = ss[3];
    }
    float z[16];
    q4_run_z(xr, sr, z);
    uint32_t hw[4], lw[4];
    int e_hi, e_lo;
    q4_run_operand(z, hw, lw, e_hi, e_lo);
    if (!live) return;
    const int r = (int)(t & 7);
    const size_t slot = q4_run_slot(t >> 3, r, 2, 0), byte = 16 * (r & 1);
    *(uint4 *)(op + slot * 32 + byte) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(op + (slot + 1) * 32 + byte) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if ((r & 2) == 0)
        *(uint16_t *)(sc + q4_run_scale(t >> 3, r, 2, 0)) = (uint16_t)((e_hi + 127) | ((e_lo + 127) << 8));
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

// sched_barrier mask: SALU, VALU, LDS and transcendental instructions may
// cross; MFMAs and vector memory loads and stores may not.
#define Q4_SCHED_PIN 0x486
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

// Slice j of a step: the fp8 operand from the wave's staged LDS region
// (NCOL > 0) or from global memory (NCOL == 0; gb/gs point at the step's
// first slice), then the four MFMAs.
template <int NCOL>
__device__ __forceinline__ void q4_step(f32x4_t acc[4], const uint4 &w4u, uint32_t j, const uint8_t *wl,
                                        uint32_t bo0, uint32_t bstep, uint32_t so0, uint32_t sstep,
                                        const uint8_t *gb, const uint8_t *gs, int g, int ncol, int col,
                                        bool bcol, uint32_t c7) {
    if (NCOL > 0) {
        q4_slice_lds(acc, w4u, wl, bo0 + j * bstep, so0 + j * sstep, c7);
        return;
    }
    i32x8_t bv = {0, 0, 0, 0, 0, 0, 0, 0};
    int bs = 127;
    if (bcol) {
        const size_t slot = ((size_t)j * 4 + g) * ncol + col;
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

// The maximum of v over the 32 lanes whose ids differ from this lane's only
// in bits 0-3 and 5 (one scale block of stage 2's operand), with no LDS
// round trip: the quad by two DPP quad permutations (l ^ 1, l ^ 2), the
// 16-lane row by two DPP row rotations (by 4 and by 8 lanes, which between
// them reach every quad of the row), and the lane 32 apart by
// v_permlane32_swap.  Every lane of the wave must be active.
#define Q4_DPP_MAX(v, ctrl) fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false)))
__device__ __forceinline__ float q4_block_max32(float v) {
    v = Q4_DPP_MAX(v, 0xB1);   // quad_perm [1, 0, 3, 2]
    v = Q4_DPP_MAX(v, 0x4E);   // quad_perm [2, 3, 0, 1]
    v = Q4_DPP_MAX(v, 0x124);  // row_ror 4
    v = Q4_DPP_MAX(v, 0x128);  // row_ror 8
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
}
#undef Q4_DPP_MAX

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
//
// acc holds columns c0 .. c0 + 15 (tokens c0 / 2 on): a column group of a
// batch beyond 8 (c0 = 16 cg), or the whole batch (c0 = 0).
template <int STAGE>
__device__ __forceinline__ void q4_epilogue(const f32x4_t acc[4], float *T, const Q4Args &a,
                                            const Q4Layer &L, int ncol, size_t rg, int lane, float so,
                                            float bi, int c0 = 0) {
    const int col = lane & 15, g = lane >> 4;
    const int nc = ncol - c0 < 16 ? ncol - c0 : 16;
    if (col < nc) {
#pragma unroll
        for (int rt = 0; rt < 4; rt++) *(f32x4_t *)(T + col * 64 + 16 * rt + 4 * g) = acc[rt];
    }
    __builtin_amdgcn_wave_barrier();
    const size_t row = rg * 64 + lane;
    const bool valid = row < L.rows_valid;
    for (int bb = 0; bb < (nc >> 1); bb++) {
        const int b = (c0 >> 1) + bb;
        const float v = q4_unscale(T[(2 * bb) * 64 + lane] + T[(2 * bb + 1) * 64 + lane]);
        const float t = valid ? bf16_to_f32(f32_to_bf16(v)) : 0.0f;
        if (STAGE == 2) {
            if (valid) {
                float y = t * so + bi;
                const size_t o = L.out0 * (size_t)a.batch + (size_t)b * L.rows_valid + row;
                if (a.resid) y = y + a.resid[o];
                if (a.y_bf16)
                    ((uint16_t *)a.out)[o] = f32_to_bf16(y);
                else
                    ((float *)a.out)[o] = y;
            }
            continue;
        }
        const float amax = q4_block_max32(fabsf(t));
        const int e_hi = amax > 0.0f ? e8m0_of(amax) : 0;
        const float sc_hi = pow2f(e_hi);
        const int hw = (int)q4_fp8x1(t, sc_hi);
        const float r = t - q4_f32x1((uint32_t)hw, sc_hi);  // exact residual
        const float rmax = q4_block_max32(fabsf(r));
        const int e_lo = rmax > 0.0f ? e8m0_of(rmax) : 0;
        const int lw = (int)q4_fp8x1(r, pow2f(e_lo));
        const int q = (lane >> 4) & 1, h = lane >> 5;
        const size_t base = ((size_t)L.tb_slice0 + (rg >> 1)) * 4;
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

// LDS bytes of one wave's region.  NCOL > 0: two buffers, each the staged
// operand of Q4_U slices (NCOL columns) and their scales (one dword per
// lane), then a zero slot; the epilogue's transpose and the K split's
// partial sums (4 KiB a wave) reuse the buffers.  NCOL == 0: the transpose.
__host__ __device__ constexpr uint32_t q4_wave_lds(int ncol) {
    return ncol > 0 ? (uint32_t)(2 * (Q4_U * 4 * ncol * 32 + 256) + 48) : 16 * 64 * 4;
}
static_assert(q4_wave_lds(2) >= 4 * 64 * 16, "a wave's partial sums fit its region");

// Decode GEMV.  Workgroup = 4 waves (8 at KSPLIT 8); KSPLIT waves share a
// 64-row group and split its slices (Q4_NW / KSPLIT row groups per
// workgroup).  Lane l loads the 16 bytes of its four row tiles' sign words
// per slice (1 KiB per wave per slice, contiguous over the slices); Q4_U
// slices are loaded per step.
//
// NCOL > 0 (batch 1-2): each wave stages the fp8 operand of its own slices
// through registers into its LDS region -- operand loads issued first, sign
// loads right behind them, no workgroup barrier -- and reads it per slice;
// lanes past the batch's columns read a zero slot.  NCOL == 0 (batch 3-8):
// lanes read the operand of each slice from global memory (L2).
//
// Loads are unconditional (indices clamped into the layer; the MFMAs of
// clamped slices are skipped) so that the compiler's wait counts stay
// counted ones: a slice's MFMAs wait for the loads issued up to its own, not
// for every load in flight (at batch 1-2 the compiler issues the operand's
// loads behind six of the sign loads, so the first MFMA of a step waits for
// those six).
//
// XCD-aware 1-D grid: workgroup i runs on XCD i % 8; XCD x takes the
// contiguous range [x*per_x, (x+1)*per_x) of the (layer, row group) work, so
// that one layer's operand is fetched into one L2.
template <int STAGE, int KSPLIT, int NCOL>
__global__ void __launch_bounds__(64 * Q4_NW(KSPLIT)) q4_gemv_kernel(Q4Args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t q4_lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
    const int ncol = NCOL > 0 ? NCOL : a.ncol;
    const uint32_t xcd = blockIdx.x & 7, per_x = gridDim.x >> 3;
    const uint32_t wgi = xcd * per_x + (blockIdx.x >> 3);
    if (wgi >= a.n_wg) return;  // padding workgroup (the whole group leaves)
    constexpr int RG_PER_WG = Q4_NW(KSPLIT) / KSPLIT;
    uint32_t li, rg0;
    q4_work_of(a, wgi, RG_PER_WG, li, rg0);
    const Q4Layer L = q4_entry(a, li);
    const size_t rg = (size_t)rg0 + wave / KSPLIT;
    const int ks = wave % KSPLIT;
    const size_t n_rg = L.rows_p / 64, ns = L.ns;
    const size_t per = (ns + KSPLIT - 1) / KSPLIT;
    const size_t s0 = ks * per < ns ? ks * per : ns;
    const size_t s1 = s0 + per < ns ? s0 + per : ns;
    const int col = lane & 15, g = lane >> 4;
    // NCOL == 0, one column group a workgroup (batches 9-32): the grid's y
    // index picks the workgroup's 16 columns (8 tokens)
    const int c0 = NCOL == 0 ? 16 * (int)blockIdx.y : 0;
    const bool bcol = c0 + col < ncol;
    const bool live = rg < n_rg;
    const size_t rgc = live ? rg : n_rg - 1;
    const uint32_t c7 = a.c7;
    const uint32_t wreg = q4_wave_lds(NCOL);  // the launch allocates 4 * this (+ red)
    uint8_t *wl = q4_lds + wave * wreg;
    const uint8_t *gb = a.op + (size_t)L.slice0 * 4 * ncol * 32;  // this layer's operand
    const uint8_t *gs = a.sc + (size_t)L.slice0 * 4 * ncol;

    // staged operand offsets within the wave's region (slice j of the step;
    // buffer b at b * RB)
    constexpr uint32_t OPB = NCOL > 0 ? Q4_U * 4 * NCOL * 32 : 0;
    constexpr uint32_t RB = OPB + 256;
    constexpr uint32_t ZS = 2 * RB;
    const uint32_t slot0 = (uint32_t)(g * ncol + col);
    const uint32_t bo0 = bcol ? slot0 * 32 : ZS, bstep = bcol ? 4 * ncol * 32 : 0;
    const uint32_t so0 = bcol ? OPB + slot0 : ZS + 32, sstep = bcol ? 4 * ncol : 0;
    if (NCOL > 0) {
        if (lane < 2) *(uint4 *)(wl + ZS + 16 * lane) = make_uint4(0, 0, 0, 0);
        if (lane == 2) wl[ZS + 32] = 127;
    }

    // stage 2: this lane's row of the group, for the epilogue (a layer
    // without a bias, or with an all +0.0 one, has no bias pointer: y adds
    // +0.0 all the same)
    float so = 0.0f, bi = 0.0f;
    if (STAGE == 2) {
        const size_t row = rgc * 64 + lane;
        const size_t rc = row < L.rows_valid ? row : L.rows_valid - 1;
        if (L.s_out_h) {  // fp16 scales (the layer's are fp16 values): half the bytes
            so = h16_to_f32(((const __attribute__((address_space(1))) uint16_t *)L.s_out_h)[rc]);
            if (L.bias_h) bi = h16_to_f32(((const __attribute__((address_space(1))) uint16_t *)L.bias_h)[rc]);
        } else {
            so = ((gf32_t *)L.s_out)[rc];
            if (L.bias) bi = ((gf32_t *)L.bias)[rc];
        }
    }

    // Padding is not streamed.  A row group wholly past the valid rows (the
    // rank padded to 128 in stage 1) loads nothing: its accumulators stay 0
    // and the epilogue writes t = 0.  In a slice that ends past the valid K
    // (the last one of a padded rank in stage 2), a lane group whose k run
    // lies wholly past it (first k 16(g>>1) + 64(g&1) of the slice) reads
    // lane group 0's words of the same slice instead -- lines the wave
    // fetches anyway -- since its activations there are zero.
    const uint4 *wp = (const uint4 *)L.bits + (rgc * ns) * 64 + lane;
    const uint32_t kmin = 16 * (g >> 1) + 64 * (g & 1);
    const size_t sdead = L.k_valid > kmin ? (L.k_valid - kmin + 127) / 128 : 0;  // first slice all past K
    const uint32_t dead_off = (uint32_t)(lane & 48);
    const bool rows_dead = rgc * 64 >= L.rows_valid;
    f32x4_t acc[4];
#pragma unroll
    for (int rt = 0; rt < 4; rt++) acc[rt] = f32x4_t{0, 0, 0, 0};
    if constexpr (NCOL == 2 && KSPLIT <= 4) {
        // Batch 1, up to four waves a row group.  (At batch 2 the ring's
        // registers went to scratch, and eight waves a group needed 124 VGPRs
        // against 94: those keep the step loop below.)  A ring of Q4_U sign
        // words a lane: the slot of slice j is refilled
        // with slice j + Q4_U as soon as slice j's signs are expanded, so
        // Q4_U - 1 to Q4_U sign loads stay in flight through the MFMAs.  The
        // staged operand of group G (slices s0 + Q4_U G ...) sits in buffer
        // G & 1: group G + 1's operand loads are issued at the start of group
        // G and written to the other buffer at its end (the buffer group G - 1
        // read; one wave's LDS operations complete in order).  The groups
        // before the last issue their successors' loads unconditionally
        // (clamped into the layer, as in a partial last group), so the
        // compiler's wait counts stay exact counts; the last group issues
        // none.
        const size_t n = rows_dead ? 0 : s1 - s0;
        const uint32_t n_grp = (uint32_t)((n + Q4_U - 1) / Q4_U);
        constexpr int SQ = Q4_U * NCOL / 8;  // 16-byte operand words a lane per group
        static_assert(Q4_U * NCOL % 8 == 0, "whole 16-byte words per lane");
        struct Staged {
            uint4 w[SQ];
            uint32_t s;
        };
        auto op_load = [&](uint32_t grp) {
            Staged st;
            const size_t sb = s0 + (size_t)grp * Q4_U;
            const uint32_t nsl = (uint32_t)(s1 - sb < Q4_U ? s1 - sb : Q4_U);
            const uint32_t ob = nsl * 4 * NCOL * 32, os = nsl * 4 * NCOL;
            const uint8_t *gbs = gb + sb * 4 * NCOL * 32, *gss = gs + sb * 4 * NCOL;
#pragma unroll
            for (int q = 0; q < SQ; q++) {
                uint32_t o = (lane + 64 * q) * 16;
                o = o < ob ? o : ob - 16;
                st.w[q] = *(const uint4 *)(gbs + o);
            }
            uint32_t o = lane * 4;
            o = o < os ? o : os - 4;
            st.s = *(const uint32_t *)(gss + o);
            return st;
        };
        auto op_store = [&](uint32_t grp, const Staged &st) {
            uint8_t *buf = wl + (grp & 1) * RB;
#pragma unroll
            for (int q = 0; q < SQ; q++) *(uint4 *)(buf + (lane + 64 * q) * 16) = st.w[q];
            *(uint32_t *)(buf + OPB + lane * 4) = st.s;  // lanes past the scales fill the padding
            __builtin_amdgcn_wave_barrier();
        };
        auto sign_load = [&](size_t j) {
            const size_t sl = j < s1 ? j : s1 - 1;
            const u32x4_t q = __builtin_nontemporal_load((gu32x4_t *)(wp + sl * 64 - (sl >= sdead ? dead_off : 0)));
            return make_uint4(q[0], q[1], q[2], q[3]);
        };
        if (n_grp > 0) {
            uint4 w4[Q4_U];
            const Staged st0 = op_load(0);
#pragma unroll
            for (int u = 0; u < Q4_U; u++) w4[u] = sign_load(s0 + u);
            op_store(0, st0);
            uint32_t grp = 0;
            for (; grp + 1 < n_grp; grp++) {
                const Staged st = op_load(grp + 1);
                __builtin_amdgcn_sched_barrier(Q4_SCHED_PIN);
                const size_t sb = s0 + (size_t)grp * Q4_U;
                const uint32_t rb = bcol ? (grp & 1) * RB : 0;
                // each refill stays behind its own slice's MFMAs and ahead of
                // the next slice's (the scheduler would otherwise sink the
                // loads below the group's MFMAs)
#pragma unroll
                for (int u = 0; u < Q4_U; u++) {
                    q4_slice_lds(acc, w4[u], wl, bo0 + rb + u * bstep, so0 + rb + u * sstep, c7);
                    w4[u] = sign_load(sb + Q4_U + u);
                    __builtin_amdgcn_sched_barrier(Q4_SCHED_PIN);
                }
                op_store(grp + 1, st);
            }
            const size_t sb = s0 + (size_t)grp * Q4_U;
            const uint32_t nsl = (uint32_t)(s1 - sb), rb = bcol ? (grp & 1) * RB : 0;
#pragma unroll
            for (int u = 0; u < Q4_U; u++)
                if (u < (int)nsl) q4_slice_lds(acc, w4[u], wl, bo0 + rb + u * bstep, so0 + rb + u * sstep, c7);
        }
    } else {
        for (size_t sb = s0; sb < (rows_dead ? s0 : s1); sb += Q4_U) {
            const uint32_t nsl = (uint32_t)(s1 - sb < Q4_U ? s1 - sb : Q4_U);
            // a step's operand: Q4_U slices x 4 lane groups x NCOL columns x 32 B,
            // SQ 16-byte words per lane
            constexpr int SQ = NCOL > 0 ? Q4_U * NCOL / 8 : 1;
            static_assert(NCOL == 0 || Q4_U * NCOL % 8 == 0, "whole 16-byte words per lane");
            uint4 stg[SQ];
            uint32_t stgs = 0;
            if (NCOL > 0) {
                // operand of slices sb..sb+nsl-1: SQ uint4 + one dword of scales per lane
                const uint32_t ob = nsl * 4 * NCOL * 32, os = nsl * 4 * NCOL;
                const uint8_t *gbs = gb + sb * 4 * NCOL * 32, *gss = gs + sb * 4 * NCOL;
    #pragma unroll
                for (int q = 0; q < SQ; q++) {
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
                const u32x4_t q = __builtin_nontemporal_load((gu32x4_t *)(wp + sl * 64 - (sl >= sdead ? dead_off : 0)));
                w4[u] = make_uint4(q[0], q[1], q[2], q[3]);
            }
            if (NCOL > 0) {
    #pragma unroll
                for (int q = 0; q < SQ; q++) *(uint4 *)(wl + (lane + 64 * q) * 16) = stg[q];
                *(uint32_t *)(wl + OPB + lane * 4) = stgs;  // lanes past the scales fill the padding
                __builtin_amdgcn_wave_barrier();
            }
            const uint8_t *gbs = gb + sb * 4 * ncol * 32, *gss = gs + sb * 4 * ncol;
            // one form for whole and partial steps (a uniform branch per slice): a
            // second, unguarded copy of the step kept its own accumulator
            // registers -- 122 VGPRs a wave against 94 at batch 1 (four waves a
            // SIMD instead of five)
    #pragma unroll
            for (int u = 0; u < Q4_U; u++)
                if (u < (int)nsl)
                    q4_step<NCOL>(acc, w4[u], u, wl, bo0, bstep, so0, sstep, gbs, gss, g, ncol, c0 + col, bcol, c7);
            if (NCOL > 0) __builtin_amdgcn_wave_barrier();  // the next step overwrites the region
        }
    }
    if (KSPLIT > 1) {
        // the partial sums through [4 tiles][64 lanes] a wave: in the wave's
        // own region (NCOL > 0: no wave reads another's region before the
        // barrier) or past the regions
        auto red = [&](int w, int rt) {
            return NCOL > 0 ? (f32x4_t *)(q4_lds + w * wreg) + rt * 64 + lane
                            : (f32x4_t *)(q4_lds + Q4_NW(KSPLIT) * wreg) + (w * 4 + rt) * 64 + lane;
        };
#pragma unroll
        for (int rt = 0; rt < 4; rt++) *red(wave, rt) = acc[rt];
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int rt = 0; rt < 4; rt++) {
            f32x4_t v = *red(wave, rt);
            for (int q = 1; q < KSPLIT; q++) v += *red(wave + q, rt);
            acc[rt] = v;
        }
    }
    if (!live) return;
    q4_epilogue<STAGE>(acc, (float *)wl, a, L, ncol, rg, lane, so, bi, c0);
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

// LDS bytes of a q4_gemv_kernel workgroup.
static size_t q4_gemv_lds(int ncol_t, int ksplit) {
    const size_t nw = Q4_NW(ksplit);
    return nw * (size_t)q4_wave_lds(ncol_t) + (ksplit > 1 && ncol_t == 0 ? nw * 4 * 64 * 16 : 0);
}

// Waves that share a 64-row group split its slices: one load step (Q4_U
// slices) per wave where the group has more, and further while the launch
// is too small to fill the chip (a single layer).
static int q4_ksplit(size_t max_ns, size_t min_ns, size_t n_rg_total, int num_cus, size_t batch) {
    int k = 1;
    while (k < 4 && max_ns > (size_t)(2 * Q4_U * k)) k *= 2;
    while (k < 4 && min_ns >= (size_t)(2 * k) && n_rg_total * k < (size_t)num_cus * 8) k *= 2;
    // eight waves a row group (one workgroup of 512 threads) where four
    // would each run more than two load steps and the launch holds few row
    // groups (a lone long-K layer at batch 1: config 3's down projection, 112
    // slices over 28 row groups, 10.7 -> 8.4 us; sixteen waves, 8.6)
    if (k == 4 && batch == 1 && min_ns > (size_t)(2 * Q4_U * 4) && n_rg_total * 8 <= (size_t)num_cus * 4) k = 8;
    return k;
}

// Launch geometry of one set of layers (or one layer) at a batch.
struct Q4Geom {
    size_t n_layers, batch, ncol;
    size_t ns1_tot, ns2_tot, max_ns1;
    bool din_mult8;  // every layer's din % 8 == 0: x blocks and rows start 16-byte aligned
    bool din_mult128;  // every layer's din % 128 == 0: stage 1's slices are all valid
    int ks1, ks2;
    uint32_t n_wg1, n_wg2;
    size_t o_op1, o_sc1, o_op2, o_sc2, bytes;  // workspace regions
};

// Fill stage-1 / stage-2 entries (tab[i], tab[n + i]) for layers[0..n) and
// the launch geometry; x and y of layer i start at batch times the running
// sums of din and dout (the entries hold the sums, so one table serves
// every batch).
static void q4_build(const qbk_factor *const *layers, size_t n, size_t batch, int num_cus,
                     Q4Layer *tab, Q4Geom &G) {
    G = Q4Geom{};
    G.n_layers = n;
    G.batch = batch;
    G.ncol = 2 * batch;
    size_t max1 = 0, min1 = SIZE_MAX, max2 = 0, min2 = SIZE_MAX, rg1 = 0, rg2 = 0;
    for (size_t i = 0; i < n; i++) {
        const qbk_factor *L = layers[i];
        const size_t ns1 = L->din_q / 128, ns2 = L->r_q / 128;
        max1 = ns1 > max1 ? ns1 : max1;
        min1 = ns1 < min1 ? ns1 : min1;
        max2 = ns2 > max2 ? ns2 : max2;
        min2 = ns2 < min2 ? ns2 : min2;
        rg1 += L->r_p / 64;
        rg2 += L->dout_p / 64;
    }
    G.max_ns1 = max1;
    G.din_mult8 = true;
    G.din_mult128 = true;
    for (size_t i = 0; i < n; i++) {
        G.din_mult8 = G.din_mult8 && layers[i]->din % 8 == 0;
        G.din_mult128 = G.din_mult128 && layers[i]->din % 128 == 0;
    }
    G.ks1 = q4_ksplit(max1, min1, rg1, num_cus, batch);
    G.ks2 = q4_ksplit(max2, min2, rg2, num_cus, batch);
    const size_t rpw1 = Q4_NW(G.ks1) / G.ks1, rpw2 = Q4_NW(G.ks2) / G.ks2;
    size_t s1 = 0, s2 = 0, wg1 = 0, wg2 = 0, act = 0, out = 0;
    for (size_t i = 0; i < n; i++) {
        const qbk_factor *L = layers[i];
        const size_t ns1 = L->din_q / 128, ns2 = L->r_q / 128;
        Q4Layer &a = tab[i];
        Q4Layer &b = tab[n + i];
        a = Q4Layer{};
        b = Q4Layer{};
        a.bits = L->vt_q4;
        a.s_in = L->s2;
        a.rows_p = (uint32_t)L->r_p;
        a.rows_valid = (uint32_t)L->r;
        a.ns = (uint32_t)ns1;
        a.k_valid = (uint32_t)L->din;
        a.slice0 = (uint32_t)s1;
        a.tb_ns = (uint32_t)ns2;
        a.tb_slice0 = (uint32_t)s2;
        a.wg0 = (uint32_t)wg1;
        a.act0 = act;
        b.bits = L->u_q4;
        b.s_out = L->s1;
        b.bias = L->bias_zero ? nullptr : L->bias;
        b.s_out_h = L->scales_f16 ? L->s1h : nullptr;
        b.bias_h = L->scales_f16 && !L->bias_zero ? L->biash : nullptr;
        b.rows_p = (uint32_t)L->dout_p;
        b.rows_valid = (uint32_t)L->dout;
        b.ns = (uint32_t)ns2;
        b.k_valid = (uint32_t)L->r;
        b.slice0 = (uint32_t)s2;
        b.wg0 = (uint32_t)wg2;
        b.out0 = out;
        s1 += ns1;
        s2 += ns2;
        wg1 += div_ceil(L->r_p / 64, rpw1);
        wg2 += div_ceil(L->dout_p / 64, rpw2);
        act += L->din;
        out += L->dout;
    }
    G.ns1_tot = s1;
    G.ns2_tot = s2;
    G.n_wg1 = (uint32_t)wg1;
    G.n_wg2 = (uint32_t)wg2;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += round_up(bytes, 256);
        return o;
    };
    G.o_op1 = take(s1 * 4 * G.ncol * 32);
    G.o_sc1 = take(s1 * 4 * G.ncol);
    G.o_op2 = take(s2 * 4 * G.ncol * 32);
    G.o_sc2 = take(s2 * 4 * G.ncol);
    G.bytes = off;
}

// One phase of a decode over the table `tab` (device; stage-1 entries
// [0, n), stage-2 entries [n, 2n)) and, for several layers, the per-
// workgroup layer tables wg1 (stage 1) and wg2.  Phase 1: x -> stage 1's
// operand; 2: stage 1 (writes stage 2's operand); 3: stage 2 -> y.  s2cat:
// the layers' s2 concatenated (null when some din is not a multiple of 128).
static int q4_phase(int phase, const Q4Geom &G, const Q4Layer *tab, const uint32_t *wg1,
                    const uint32_t *wg2, const float *s2cat, const void *x, bool xf32, void *y, bool ybf16,
                    void *ws, hipStream_t s, const float *resid = nullptr, const uint16_t *s2cat_h = nullptr) {
    char *w = (char *)ws;
    Q4Args a{};
    a.c7 = 0x77777777u;
    a.batch = (int)G.batch;
    a.ncol = (int)G.ncol;
    a.n_layers = (uint32_t)G.n_layers;
    a.y_bf16 = ybf16;
    if (phase <= 2) {
        a.layers = tab;
        a.act = x;
        a.op = (uint8_t *)(w + G.o_op1);
        a.sc = (uint8_t *)(w + G.o_sc1);
        a.tb_op = (uint8_t *)(w + G.o_op2);
        a.tb_sc = (uint8_t *)(w + G.o_sc2);
        a.n_wg = G.n_wg1;
        a.wg_layer = wg1;
    } else {
        a.layers = tab + G.n_layers;
        a.op = (uint8_t *)(w + G.o_op2);
        a.sc = (uint8_t *)(w + G.o_sc2);
        a.out = y;
        a.resid = ybf16 ? nullptr : resid;
        a.n_wg = G.n_wg2;
        a.wg_layer = wg2;
    }
    if (phase == 1) {
        if (s2cat && !xf32 && G.batch == 1 && G.din_mult128 && (uintptr_t)x % 16 == 0) {
            const uint32_t n_runs = (uint32_t)(G.ns1_tot * 8);
            if (s2cat_h)
                hipLaunchKernelGGL(q4_prep_flat_kernel<true>, dim3((unsigned)div_ceil(n_runs, 256)), dim3(256), 0,
                                   s, (const uint16_t *)x, (const void *)s2cat_h, a.op, a.sc, n_runs);
            else
                hipLaunchKernelGGL(q4_prep_flat_kernel<false>, dim3((unsigned)div_ceil(n_runs, 256)), dim3(256), 0,
                                   s, (const uint16_t *)x, (const void *)s2cat, a.op, a.sc, n_runs);
            QBK_HIP(hipGetLastError());
            return QBK_OK;
        }
        // 16-byte vector loads of x: every layer's x block and token row
        // start 16-byte aligned when x is and every din is a multiple of 8
        a.vec_ok = G.din_mult8 && (uintptr_t)x % 16 == 0;
        const size_t runs = G.batch * G.max_ns1 * 8;
        dim3 g((unsigned)div_ceil(runs, 256), (unsigned)G.n_layers);
        if (xf32)
            hipLaunchKernelGGL((q4_prep_kernel<true>), g, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((q4_prep_kernel<false>), g, dim3(256), 0, s, a);
        QBK_HIP(hipGetLastError());
        return QBK_OK;
    }
    const int ksplit = phase == 2 ? G.ks1 : G.ks2;
    const int ncol_t = G.batch <= 2 ? (int)G.ncol : 0;  // staged operand at batch 1-2
    const int ncg = (int)div_ceil(G.ncol, 16);           // column groups (batch > 8)
    const size_t lds = q4_gemv_lds(ncol_t, ksplit);
    dim3 g((unsigned)round_up((size_t)a.n_wg, 8));  // a multiple of the 8 XCDs
    if (ksplit > 4) {  // batch 1 only (q4_ksplit)
        if (phase == 2)
            hipLaunchKernelGGL((q4_gemv_kernel<1, 8, 2>), g, dim3(512), lds, s, a);
        else
            hipLaunchKernelGGL((q4_gemv_kernel<2, 8, 2>), g, dim3(512), lds, s, a);
        QBK_HIP(hipGetLastError());
        return QBK_OK;
    }
#define Q4_LAUNCH(ST, KS)                                                                             \
    if (ncol_t == 2) hipLaunchKernelGGL((q4_gemv_kernel<ST, KS, 2>), g, dim3(256), lds, s, a);       \
    else if (ncol_t == 4) hipLaunchKernelGGL((q4_gemv_kernel<ST, KS, 4>), g, dim3(256), lds, s, a);  \
    else hipLaunchKernelGGL((q4_gemv_kernel<ST, KS, 0>), dim3(g.x, (unsigned)ncg), dim3(256), lds, s, a);
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

void q4_layer_entries(const qbk_factor *L, Q4Layer out[2]) {
    Q4Geom G;
    q4_build(&L, 1, 1, L->num_cus, out, G);
}

size_t q4_workspace(const qbk_factor *L, size_t batch) {
    Q4Layer tab[2];
    Q4Geom G;
    q4_build(&L, 1, batch, L->num_cus, tab, G);
    return G.bytes;
}

int q4_run(const qbk_factor *L, size_t batch, const void *x, bool xf32, void *y, bool ybf16, void *ws,
           hipStream_t s) {
    Q4Layer tab[2];
    Q4Geom G;
    q4_build(&L, 1, batch, L->num_cus, tab, G);  // geometry; the device table is L->q4_tab
    const float *s2cat = G.din_mult128 ? L->s2 : nullptr;  // one layer: its own s2
    for (int ph = 1; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, G, L->q4_tab, nullptr, nullptr, s2cat, x, xf32, y, ybf16, ws, s, nullptr,
                          s2cat && L->scales_f16 ? L->s2h : nullptr);
        if (rc) return rc;
    }
    return QBK_OK;
}

bool q4_flat_operand(const qbk_factor *L, void *ws, uint8_t **op, uint8_t **sc) {
    Q4Layer tab[2];
    Q4Geom G;
    q4_build(&L, 1, 1, L->num_cus, tab, G);
    if (!G.din_mult128) return false;
    *op = (uint8_t *)ws + G.o_op1;
    *sc = (uint8_t *)ws + G.o_sc1;
    return true;
}

bool q4_flat_operand_batch(const qbk_factor *L, size_t n, void *ws, uint8_t **op, uint8_t **sc) {
    Q4Layer tab[2];
    Q4Geom G;
    q4_build(&L, 1, n, L->num_cus, tab, G);
    if (!G.din_mult128) return false;
    *op = (uint8_t *)ws + G.o_op1;
    *sc = (uint8_t *)ws + G.o_sc1;
    return true;
}

int q4_run_staged_batch(const qbk_factor *L, size_t n, void *y, bool ybf16, const float *resid, void *ws,
                        hipStream_t s) {
    Q4Layer tab[2];
    Q4Geom G;
    q4_build(&L, 1, n, L->num_cus, tab, G);
    for (int ph = 2; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, G, L->q4_tab, nullptr, nullptr, nullptr, nullptr, false, y, ybf16, ws, s, resid);
        if (rc) return rc;
    }
    return QBK_OK;
}

int q4_run_staged(const qbk_factor *L, void *y, bool ybf16, const float *resid, void *ws, hipStream_t s) {
    Q4Layer tab[2];
    Q4Geom G;
    q4_build(&L, 1, 1, L->num_cus, tab, G);
    for (int ph = 2; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, G, L->q4_tab, nullptr, nullptr, nullptr, nullptr, false, y, ybf16, ws, s, resid);
        if (rc) return rc;
    }
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

// A decode set: layers of any shapes, one table, three launches.
struct qbk_factor_set {
    int device, num_cus;
    size_t n;
    Q4Layer *tab;          // device: [0, n) stage 1, [n, 2n) stage 2; then the
    uint32_t *wg1, *wg2;   // per-workgroup layer tables (same allocation)
    float *s2cat;          // device: the layers' s2 concatenated (every din % 128 == 0), else null
    uint16_t *s2cat_h;     // device: the same as fp16 when every layer's scales are fp16 values, else null
    G32SetLayer *g32tab;   // device: the set on the prefill GEMM, [n] stage 1 then [n] stage 2
    Q4Geom geom;           // batch 1
    std::vector<const qbk_factor *> layers;
};

namespace qbk {

// A set's decode with the x and y dtypes of the caller's choice (the C ABI's
// form is bf16 in and out): x the concatenation of the layers' inputs.
int q4_set_run(const qbk_factor_set *S, const void *x, bool xf32, void *y, bool ybf16, void *ws, hipStream_t s) {
    for (int ph = 1; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, S->geom, S->tab, S->wg1, S->wg2, S->s2cat, x, xf32, y, ybf16, ws, s, nullptr,
                          S->s2cat_h);
        if (rc) return rc;
    }
    return QBK_OK;
}

size_t q4_set_workspace(const qbk_factor_set *S) { return S->geom.bytes; }

bool q4_set_gemm_fits(const qbk_factor_set *S, size_t N) { return g32_set_fits(S->layers.data(), S->n, N); }

size_t q4_set_gemm_workspace(const qbk_factor_set *S, size_t N) {
    return g32_set_workspace(S->layers.data(), S->n, N);
}

int q4_set_gemm_run(const qbk_factor_set *S, size_t N, const void *x, bool xf32, void *y, bool ybf16, void *ws,
                    hipStream_t s) {
    return g32_set_run(S->layers.data(), S->n, S->g32tab, S->g32tab + S->n, N, x, xf32, y, ybf16, ws, s);
}

bool q4_set_flat_operand(const qbk_factor_set *S, void *ws, uint8_t **op, uint8_t **sc, const float **s2cat) {
    if (!S->s2cat || !S->geom.din_mult128) return false;
    *op = (uint8_t *)ws + S->geom.o_op1;
    *sc = (uint8_t *)ws + S->geom.o_sc1;
    *s2cat = S->s2cat;
    return true;
}

int q4_set_run_staged(const qbk_factor_set *S, void *y, bool ybf16, void *ws, hipStream_t s) {
    for (int ph = 2; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, S->geom, S->tab, S->wg1, S->wg2, nullptr, nullptr, false, y, ybf16, ws, s);
        if (rc) return rc;
    }
    return QBK_OK;
}

// The set at a batch of n tokens: the device tables are the batch-1 ones
// (their offsets are per token); the geometry is the batch's.
static void q4_set_geom(const qbk_factor_set *S, size_t n, Q4Geom &G) {
    std::vector<Q4Layer> h(2 * S->n);
    q4_build(S->layers.data(), S->n, n, S->num_cus, h.data(), G);
}

size_t q4_set_workspace_batch(const qbk_factor_set *S, size_t n) {
    Q4Geom G;
    q4_set_geom(S, n, G);
    return G.bytes;
}

// The per-workgroup table of a set's GEMV launch: (layer, first row group)
// of each workgroup.  The kernel hands XCD x the contiguous workgroups [x
// per_x, (x + 1) per_x) (per_x = the grid's eighth); inside each such range
// the workgroups are ordered by the slices they stream, longest first (at
// config 3 the down projection's row groups stream 112 slices, the others'
// 32, and in layer order the last of them started when most of the launch
// had ended), ties kept in layer order; row groups wholly past a layer's
// valid rows stream nothing and go last.
static void q4_wg_table(const Q4Layer *tab, size_t n, uint32_t n_wg, uint32_t rg_per_wg, uint32_t *out) {
    struct Unit {
        uint32_t li, rg0;
        uint64_t cost;
    };
    std::vector<Unit> u(n_wg);
    for (size_t i = 0; i < n; i++) {
        const uint32_t e = i + 1 < n ? tab[i + 1].wg0 : n_wg;
        for (uint32_t w = tab[i].wg0; w < e; w++) {
            const uint32_t rg0 = (w - tab[i].wg0) * rg_per_wg;
            uint64_t live = 0;
            for (uint32_t r = rg0; r < rg0 + rg_per_wg && r < tab[i].rows_p / 64; r++)
                live += (uint64_t)r * 64 < tab[i].rows_valid;
            u[w] = Unit{(uint32_t)i, rg0, live * tab[i].ns};
        }
    }
    const uint32_t per_x = (uint32_t)(round_up(n_wg, 8) / 8);
    for (uint32_t x = 0; x < 8; x++) {
        const uint32_t b = x * per_x, e = b + per_x < n_wg ? b + per_x : n_wg;
        if (b < e)
            std::stable_sort(u.begin() + b, u.begin() + e, [](const Unit &p, const Unit &q) { return p.cost > q.cost; });
    }
    for (uint32_t w = 0; w < n_wg; w++) {
        out[2 * w] = u[w].li;
        out[2 * w + 1] = u[w].rg0;
    }
}

bool q4_set_flat_operand_batch(const qbk_factor_set *S, size_t n, void *ws, uint8_t **op, uint8_t **sc,
                               const float **s2cat) {
    if (!S->s2cat || !S->geom.din_mult128) return false;
    Q4Geom G;
    q4_set_geom(S, n, G);
    *op = (uint8_t *)ws + G.o_op1;
    *sc = (uint8_t *)ws + G.o_sc1;
    *s2cat = S->s2cat;
    return true;
}

int q4_set_run_batch_staged(const qbk_factor_set *S, size_t n, void *y, bool ybf16, void *ws, hipStream_t s) {
    Q4Geom G;
    q4_set_geom(S, n, G);
    for (int ph = 2; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, G, S->tab, S->wg1, S->wg2, nullptr, nullptr, false, y, ybf16, ws, s);
        if (rc) return rc;
    }
    return QBK_OK;
}

int q4_set_run_batch(const qbk_factor_set *S, size_t n, const void *x, bool xf32, void *y, bool ybf16, void *ws,
                     hipStream_t s) {
    if (n == 1) return q4_set_run(S, x, xf32, y, ybf16, ws, s);
    Q4Geom G;
    q4_set_geom(S, n, G);
    for (int ph = 1; ph <= Q4_PHASES; ph++) {
        int rc = q4_phase(ph, G, S->tab, S->wg1, S->wg2, nullptr, x, xf32, y, ybf16, ws, s);
        if (rc) return rc;
    }
    return QBK_OK;
}

}  // namespace qbk

extern "C" {

int qbk_factor_set_create(qbk_ctx *ctx, const qbk_factor *const *layers, size_t n,
                          qbk_factor_set **out) {
    int rc;
    if (!out || !layers || n == 0) return fail(QBK_ERR_VALIDATION, "empty layer set");
    *out = nullptr;
    if ((rc = bind(ctx))) return rc;
    for (size_t i = 0; i < n; i++) {
        if (!layers[i]) return fail(QBK_ERR_VALIDATION, fmt("layer %zu of the set is null", i));
        if (layers[i]->device != ctx->device)
            return fail(QBK_ERR_VALIDATION, fmt("layer %zu lives on another device", i));
    }
    std::vector<Q4Layer> h(2 * n);
    qbk_factor_set *S = new qbk_factor_set();
    S->device = ctx->device;
    S->num_cus = ctx->num_cus;
    S->n = n;
    S->layers.assign(layers, layers + n);
    q4_build(layers, n, 1, ctx->num_cus, h.data(), S->geom);
    if (S->geom.n_wg1 == 0 || S->geom.n_wg2 == 0 || S->geom.ns1_tot >= (1ull << 31)) {
        delete S;
        return fail(QBK_ERR_VALIDATION, "layer set too large for one decode launch");
    }
    // (layer, first row group) of every workgroup of the two GEMV launches
    std::vector<uint32_t> wl(2 * (S->geom.n_wg1 + S->geom.n_wg2));
    q4_wg_table(h.data(), n, S->geom.n_wg1, Q4_NW(S->geom.ks1) / S->geom.ks1, wl.data());
    q4_wg_table(h.data() + n, n, S->geom.n_wg2, Q4_NW(S->geom.ks2) / S->geom.ks2, wl.data() + 2 * S->geom.n_wg1);
    const size_t tab_bytes = 2 * n * sizeof(Q4Layer);
    hipError_t e1 = hipMalloc((void **)&S->tab, tab_bytes + wl.size() * 4);
    if (e1 != hipSuccess) {
        delete S;
        return fail(QBK_ERR_DEVICE, fmt("hipMalloc failed: %s", hipGetErrorString(e1)));
    }
    S->wg1 = (uint32_t *)((char *)S->tab + tab_bytes);
    S->wg2 = S->wg1 + 2 * S->geom.n_wg1;
    S->s2cat = nullptr;
    S->s2cat_h = nullptr;
    e1 = hipMemcpy(S->tab, h.data(), tab_bytes, hipMemcpyHostToDevice);
    if (e1 == hipSuccess) e1 = hipMemcpy(S->wg1, wl.data(), wl.size() * 4, hipMemcpyHostToDevice);
    if (e1 == hipSuccess && S->geom.din_mult128) {
        // the layers' s2 in x's order, for the batch-1 flat prep
        size_t n_in = 0;
        for (size_t i = 0; i < n; i++) n_in += layers[i]->din;
        e1 = hipMalloc((void **)&S->s2cat, n_in * sizeof(float));
        if (e1 != hipSuccess) S->s2cat = nullptr;
        for (size_t i = 0, o = 0; e1 == hipSuccess && i < n; o += layers[i]->din, i++)
            e1 = hipMemcpy(S->s2cat + o, layers[i]->s2, layers[i]->din * sizeof(float), hipMemcpyDeviceToDevice);
        // and as fp16 when every layer's scales are fp16 values
        bool f16 = true;
        for (size_t i = 0; i < n; i++) f16 = f16 && layers[i]->scales_f16;
        if (e1 == hipSuccess && f16) {
            e1 = hipMalloc((void **)&S->s2cat_h, n_in * sizeof(uint16_t));
            if (e1 != hipSuccess) S->s2cat_h = nullptr;
            for (size_t i = 0, o = 0; e1 == hipSuccess && i < n; o += layers[i]->din, i++)
                e1 = hipMemcpy(S->s2cat_h + o, layers[i]->s2h, layers[i]->din * sizeof(uint16_t),
                               hipMemcpyDeviceToDevice);
        }
    }
    S->g32tab = nullptr;
    if (e1 == hipSuccess) {
        std::vector<G32SetLayer> gt(2 * n);
        g32_set_tables(layers, n, gt.data(), gt.data() + n);
        e1 = hipMalloc((void **)&S->g32tab, gt.size() * sizeof(G32SetLayer));
        if (e1 != hipSuccess) S->g32tab = nullptr;
        if (e1 == hipSuccess)
            e1 = hipMemcpy(S->g32tab, gt.data(), gt.size() * sizeof(G32SetLayer), hipMemcpyHostToDevice);
    }
    if (e1 != hipSuccess) {
        (void)hipFree(S->tab);
        if (S->s2cat) (void)hipFree(S->s2cat);
        if (S->s2cat_h) (void)hipFree(S->s2cat_h);
        if (S->g32tab) (void)hipFree(S->g32tab);
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
    (void)hipFree(S->tab);
    if (S->s2cat) (void)hipFree(S->s2cat);
    if (S->s2cat_h) (void)hipFree(S->s2cat_h);
    if (S->g32tab) (void)hipFree(S->g32tab);
    (void)hipSetDevice(cur);
    delete S;
}

size_t qbk_factor_set_workspace_size(const qbk_factor_set *S) { return S ? S->geom.bytes : 0; }

int qbk_factor_set_stage_dev(qbk_ctx *ctx, const qbk_factor_set *S, int stage, const uint16_t *x,
                             uint16_t *y, void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if (!S) return fail(QBK_ERR_VALIDATION, "null layer set");
    if (stage < 1 || stage > Q4_PHASES)
        return fail(QBK_ERR_VALIDATION, fmt("stage must be 1..%d, got %d", Q4_PHASES, stage));
    if ((rc = bind(ctx))) return rc;
    if (workspace_size < S->geom.bytes)
        return fail(QBK_ERR_VALIDATION, fmt("workspace of %zu bytes is smaller than the %zu this call needs",
                                            workspace_size, S->geom.bytes));
    return q4_phase(stage, S->geom, S->tab, S->wg1, S->wg2, S->s2cat, x, false, y, true, workspace,
                    (hipStream_t)stream, nullptr, S->s2cat_h);
}

size_t qbk_factor_set_workspace_size_batch(const qbk_factor_set *S, size_t n) {
    if (!S || n == 0 || n > Q4_MAXB_KERNEL) return 0;
    return q4_set_workspace_batch(S, n);
}

int qbk_factor_set_decode_batch_dev(qbk_ctx *ctx, const qbk_factor_set *S, size_t n, const uint16_t *x,
                                    uint16_t *y, void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if (!S) return fail(QBK_ERR_VALIDATION, "null layer set");
    if (n == 0 || n > Q4_MAXB_KERNEL)
        return fail(QBK_ERR_VALIDATION, fmt("batched set decode takes 1 to %zu tokens, got %zu", Q4_MAXB_KERNEL, n));
    if (!x || !y) return fail(QBK_ERR_VALIDATION, "null buffer");
    if ((rc = bind(ctx))) return rc;
    if (S->device != ctx->device) return fail(QBK_ERR_VALIDATION, "layer set lives on another device");
    const size_t need = q4_set_workspace_batch(S, n);
    if (!workspace || workspace_size < need)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs", workspace_size, need));
    return q4_set_run_batch(S, n, x, false, y, true, workspace, (hipStream_t)stream);
}

size_t qbk_factor_set_shared_workspace_size(const qbk_factor_set *S, size_t n) {
    if (!S || !q4_set_gemm_fits(S, n)) return 0;
    return q4_set_gemm_workspace(S, n);
}

int qbk_factor_set_shared_dev(qbk_ctx *ctx, const qbk_factor_set *S, size_t n, const uint16_t *x, uint16_t *y,
                              void *workspace, size_t workspace_size, void *stream) {
    int rc;
    if (!S) return fail(QBK_ERR_VALIDATION, "null layer set");
    if (n == 0 || n > 64)
        return fail(QBK_ERR_VALIDATION, fmt("shared-input set on the GEMM takes 1 to 64 tokens, got %zu", n));
    if (!q4_set_gemm_fits(S, n))
        return fail(QBK_ERR_VALIDATION, "shared-input set: every layer's din must be equal and a multiple of 8");
    if (!x || !y) return fail(QBK_ERR_VALIDATION, "null buffer");
    if ((uintptr_t)x % 16 != 0) return fail(QBK_ERR_VALIDATION, "shared-input set: x must be 16-byte aligned");
    if ((rc = bind(ctx))) return rc;
    if (S->device != ctx->device) return fail(QBK_ERR_VALIDATION, "layer set lives on another device");
    const size_t need = q4_set_gemm_workspace(S, n);
    if (!workspace || workspace_size < need)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs", workspace_size, need));
    return q4_set_gemm_run(S, n, x, false, y, true, workspace, (hipStream_t)stream);
}

int qbk_factor_set_decode_dev(qbk_ctx *ctx, const qbk_factor_set *S, const uint16_t *x, uint16_t *y,
                              void *workspace, size_t workspace_size, void *stream) {
    for (int ph = 1; ph <= Q4_PHASES; ph++) {
        int rc = qbk_factor_set_stage_dev(ctx, S, ph, x, y, workspace, workspace_size, stream);
        if (rc) return rc;
    }
    return QBK_OK;
}

}  // extern "C"
