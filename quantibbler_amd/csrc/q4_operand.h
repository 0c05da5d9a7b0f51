// q4_operand.h -- the decode GEMV's stage-1 operand: activations z =
// bf16(s2 * x) as two fp8 e4m3 columns (hi, lo) with E8M0 block scales, in
// the layout the fp4 x fp8 scaled MFMA reads.  Shared by the decode's prep
// kernels (decode.hip) and the decoder block's kernels that write the
// operand of the projection they feed directly (block.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qbk_internal.h"

namespace qbk {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int e8m0_of(float amax) {
    // exponent so that amax * 2^-e lies in [128, 256): e = floor(log2 amax) - 7
    int ex = (int)((__float_as_uint(amax) >> 23) & 0xff) - 127;
    int e = ex - 7;
    return e < -126 ? -126 : (e > 126 ? 126 : e);
}

__device__ __forceinline__ float pow2f(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// fp8 e4m3 of a / sc, b / sc, c / sc, d / sc (sc a power of two), bytes 0-3,
// round to nearest even, saturating: the scaled conversion divides by sc
// exactly, in the one instruction -- bit for bit cvt_pk_fp8_f32(a * 2^-e,
// ...) for sc = 2^e, e in [-126, 126] (checked on gfx950 over 2^20 values).
typedef short q4_s16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t q4_fp8x4(float a, float b, float c, float d, float sc) {
    q4_s16x2_t w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q4_s16x2_t{0, 0}, a, b, sc, false);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, c, d, sc, true);
    return __builtin_bit_cast(uint32_t, w);
}

// fp8 e4m3 of a / sc in byte 0 (byte 1 zero), as q4_fp8x4.
__device__ __forceinline__ uint32_t q4_fp8x1(float a, float sc) {
    const q4_s16x2_t w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(q4_s16x2_t{0, 0}, a, 0.0f, sc, false);
    return (uint32_t)(uint16_t)w[0];
}

// fp8 byte 0 of w times sc (a power of two): exact.
__device__ __forceinline__ float q4_f32x1(uint32_t w, float sc) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, sc, false)[0];
}

// The four fp8 bytes of w times sc (a power of two): exact.
__device__ __forceinline__ void q4_f32x4(uint32_t w, float sc, float out[4]) {
    const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, sc, false);
    const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, sc, true);
    out[0] = lo[0];
    out[1] = lo[1];
    out[2] = hi[0];
    out[3] = hi[1];
}

// fp16 bits (the low half of h) -> f32, exact.
__device__ __forceinline__ float h16_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// The fp4 signs enter the MFMA as +-1.5 (e2m1 6 at E8M0 scale 2^-2), so a
// sum s comes out as 1.5 s.  Multiplying by c = 11184811 * 2^-24, the float
// nearest 2/3, undoes it: 1.5 c = 1 + 2^-25, so for any float s, (1.5 s) * c
// = s (1 + 2^-25) rounds back to s exactly -- what a division by 1.5 gives,
// in one multiply; a sum that is not 1.5 times a float lands within one ulp
// of the division's quotient.
__device__ __forceinline__ float q4_unscale(float v) { return v * 0.666666686534881591796875f; }

// One run of 16 activations z = bf16(s2 * x) as stage 1's fp8 operand:
// z splits exactly into hi + lo, each fp8 e4m3 part keeping 4 significant
// bits relative to its block's E8M0 exponent (e_hi from the block max of z,
// e_lo from the block max of the residual).  The E8M0 scale given by MFMA
// lane group G covers the activations k = 128s + kq4(G, e) (measured on
// gfx950): the two runs 16(G>>1) + 64(G&1) + {0, 32}, i.e. runs r and r^2, so
// the block max is one shuffle away -- the calling lanes must hold runs r
// and r^2 of a slice at lane distance 2.
__device__ __forceinline__ void q4_run_operand(float z[16], uint32_t hw[4], uint32_t lw[4], int &e_hi,
                                               int &e_lo) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(z[e]));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    e_hi = amax > 0.0f ? e8m0_of(amax) : 0;
    const float sc_hi = pow2f(e_hi);
    float rmax = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        hw[q] = q4_fp8x4(z[4 * q], z[4 * q + 1], z[4 * q + 2], z[4 * q + 3], sc_hi);
        float b[4];
        q4_f32x4(hw[q], sc_hi, b);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            z[4 * q + u] -= b[u];  // exact residuals
            rmax = fmaxf(rmax, fabsf(z[4 * q + u]));
        }
    }
    rmax = fmaxf(rmax, __shfl_xor(rmax, 2, 64));
    e_lo = rmax > 0.0f ? e8m0_of(rmax) : 0;
    const float sc_lo = pow2f(e_lo);
#pragma unroll
    for (int q = 0; q < 4; q++) lw[q] = q4_fp8x4(z[4 * q], z[4 * q + 1], z[4 * q + 2], z[4 * q + 3], sc_lo);
}

// z = bf16(s2 * x) of 16 bf16 activations (two 16-byte words) and their s2.
__device__ __forceinline__ void q4_run_z(const u32x4_t xr[2], const u32x4_t sr[4], float z[16]) {
#pragma unroll
    for (int q = 0; q < 2; q++) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
            z[8 * q + 2 * h] = bf16_to_f32(xr[q][h] & 0xffff);
            z[8 * q + 2 * h + 1] = bf16_to_f32(xr[q][h] >> 16);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
            const uint32_t w = f32x2_to_bf16x2(__uint_as_float(sr[q][u]) * z[4 * q + u],
                                               __uint_as_float(sr[q][u + 1]) * z[4 * q + u + 1]);
            z[4 * q + u] = __uint_as_float(w << 16);
            z[4 * q + u + 1] = __uint_as_float(w & 0xffff0000u);
        }
    }
}

// Where run r (of slice u, token b) of a step's operand lives in the layout
// [slice][4 lane groups][ncol][32 B]: lane group 2(r>>2) + ((r>>1)&1), byte
// offset 16(r&1); hi in column 2b, lo in 2b + 1.  Its two scale bytes (hi,
// lo) sit in [slice][4][ncol] at group 2(r&1) + (r>>2) when r & 2 == 0.
__device__ __forceinline__ size_t q4_run_slot(size_t slice, int r, int ncol, int b) {
    return (slice * 4 + 2 * (r >> 2) + ((r >> 1) & 1)) * ncol + 2 * b;
}
__device__ __forceinline__ size_t q4_run_scale(size_t slice, int r, int ncol, int b) {
    return (slice * 4 + 2 * (r & 1) + (r >> 2)) * ncol + 2 * b;
}

}  // namespace qbk
