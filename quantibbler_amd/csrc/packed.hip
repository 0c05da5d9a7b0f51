// packed.hip -- the dtype-tagged packed products behind packed_matvec[_dtype]
// and packed_matmul[_dtype] (core.rs:202-317, dispatch.rs:81-109,
// gpu.rs:116-185).
//
// These are the drop-in faces of the reference's generic products, whose
// contract pins a strictly sequential accumulation in element order
// (core.rs:202-221; gpu.rs module note: "Reordering the loop ... is NOT
// sanctioned").  Each output element is therefore owned by one thread that
// sums in element order, so f64/f32/bf16 results are bit-identical to the
// CPU rlib face.  (The sign multiply is exact, so fused multiply-add gives
// the same value as the separate multiply and add.)  The bandwidth-optimised
// kernels of the factor linear live in factor.hip.
#include <string.h>

#include "qbk_internal.h"

namespace qbk {

template <int DT>
struct Dt;
template <>
struct Dt<QBK_F64> {
    using T = double;
    using Acc = double;
    static __device__ Acc load(const T *p, size_t i) { return p[i]; }
    static __device__ void store(T *p, size_t i, Acc a) { p[i] = a; }
};
template <>
struct Dt<QBK_F32> {
    using T = float;
    using Acc = float;
    static __device__ Acc load(const T *p, size_t i) { return p[i]; }
    static __device__ void store(T *p, size_t i, Acc a) { p[i] = a; }
};
template <>
struct Dt<QBK_BF16> {
    using T = uint16_t;
    using Acc = float;
    static __device__ Acc load(const T *p, size_t i) { return bf16_to_f32(p[i]); }
    static __device__ void store(T *p, size_t i, Acc a) { p[i] = f32_to_bf16(a); }
};

// One thread per row; bits decoded LSB-first, one byte load per 8 elements.
template <int DT>
__global__ void __launch_bounds__(256) seq_matvec_kernel(const uint8_t *__restrict__ packed,
                                                         size_t n_rows, size_t n_bits,
                                                         size_t row_words,
                                                         const typename Dt<DT>::T *__restrict__ vec,
                                                         typename Dt<DT>::T *__restrict__ out) {
    using D = Dt<DT>;
    size_t row = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n_rows) return;
    const uint8_t *p = packed + row * row_words;
    typename D::Acc acc = 0;
    for (size_t k0 = 0; k0 < n_bits; k0 += 8) {
        unsigned byte = p[k0 >> 3];
        size_t k1 = k0 + 8 < n_bits ? k0 + 8 : n_bits;
        for (size_t k = k0; k < k1; k++) {
            typename D::Acc v = D::load(vec, k);
            acc = ((byte >> (k - k0)) & 1u) ? acc + v : acc - v;
        }
    }
    D::store(out, row, acc);
}

// One thread per output element (i, j); the packed row is shared by the
// block's threads of one i (broadcast loads), mat rows are read coalesced.
template <int DT>
__global__ void __launch_bounds__(256) seq_matmul_kernel(const uint8_t *__restrict__ packed,
                                                         size_t n_rows, size_t n_bits,
                                                         size_t row_words,
                                                         const typename Dt<DT>::T *__restrict__ mat,
                                                         size_t k_cols, size_t n_cols,
                                                         typename Dt<DT>::T *__restrict__ out) {
    using D = Dt<DT>;
    size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t i = (size_t)blockIdx.y * blockDim.y + threadIdx.y;
    if (i >= n_rows || j >= k_cols) return;
    const uint8_t *p = packed + i * row_words;
    typename D::Acc acc = 0;
    for (size_t t0 = 0; t0 < n_bits; t0 += 8) {
        unsigned byte = p[t0 >> 3];
        size_t t1 = t0 + 8 < n_bits ? t0 + 8 : n_bits;
        for (size_t t = t0; t < t1; t++) {
            typename D::Acc v = D::load(mat, t * n_cols + j);
            acc = ((byte >> (t - t0)) & 1u) ? acc + v : acc - v;
        }
    }
    D::store(out, i * k_cols + j, acc);
}

static size_t dtype_size(int dt) { return dt == QBK_F64 ? 8 : dt == QBK_F32 ? 4 : 2; }

static int check_dtype(int dt) {
    if (dt != QBK_F64 && dt != QBK_F32 && dt != QBK_BF16)
        return fail(QBK_ERR_VALIDATION, fmt("unknown dtype tag %d; expected 0 (float64), 1 "
                                            "(float32) or 2 (bfloat16)",
                                            dt));
    return QBK_OK;
}

static int launch_matvec(int dt, const uint8_t *packed, size_t n_rows, size_t n_bits,
                         const void *vec, void *out, hipStream_t s) {
    size_t w = div_ceil(n_bits, 8);
    dim3 grid((unsigned)div_ceil(n_rows, 256)), block(256);
    switch (dt) {
        case QBK_F64:
            hipLaunchKernelGGL(seq_matvec_kernel<QBK_F64>, grid, block, 0, s, packed, n_rows,
                               n_bits, w, (const double *)vec, (double *)out);
            break;
        case QBK_F32:
            hipLaunchKernelGGL(seq_matvec_kernel<QBK_F32>, grid, block, 0, s, packed, n_rows,
                               n_bits, w, (const float *)vec, (float *)out);
            break;
        default:
            hipLaunchKernelGGL(seq_matvec_kernel<QBK_BF16>, grid, block, 0, s, packed, n_rows,
                               n_bits, w, (const uint16_t *)vec, (uint16_t *)out);
    }
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

static int launch_matmul(int dt, const uint8_t *packed, size_t n_rows, size_t n_bits,
                         const void *mat, size_t k_cols, size_t n_cols, void *out,
                         hipStream_t s) {
    size_t w = div_ceil(n_bits, 8);
    dim3 block(64, 4);
    dim3 grid((unsigned)div_ceil(k_cols, 64), (unsigned)div_ceil(n_rows, 4));
    switch (dt) {
        case QBK_F64:
            hipLaunchKernelGGL(seq_matmul_kernel<QBK_F64>, grid, block, 0, s, packed, n_rows,
                               n_bits, w, (const double *)mat, k_cols, n_cols, (double *)out);
            break;
        case QBK_F32:
            hipLaunchKernelGGL(seq_matmul_kernel<QBK_F32>, grid, block, 0, s, packed, n_rows,
                               n_bits, w, (const float *)mat, k_cols, n_cols, (float *)out);
            break;
        default:
            hipLaunchKernelGGL(seq_matmul_kernel<QBK_BF16>, grid, block, 0, s, packed, n_rows,
                               n_bits, w, (const uint16_t *)mat, k_cols, n_cols,
                               (uint16_t *)out);
    }
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_packed_matvec(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t packed_len,
                      size_t n_rows, size_t n_bits, const void *vec, size_t vec_len, void *out) {
    int rc;
    if ((rc = check_dtype(dtype))) return rc;
    size_t w;
    if ((rc = validate_packed(packed_len, n_rows, n_bits, &w))) return rc;
    if (vec_len != n_bits)
        return fail(QBK_ERR_VALIDATION,
                    fmt("vec must have length %zu, got %zu", n_bits, vec_len));
    // gpu.rs:127-137: the f64 device face's u32 index ceiling, after the
    // shape checks and before any device use (checked without overflow:
    // n_rows * w == packed_len already holds)
    const size_t ceiling = 0xFFFFFFFFull;
    if (dtype == QBK_F64 && (packed_len > ceiling || n_rows > ceiling))
        return fail(QBK_ERR_VALIDATION,
                    fmt("packed shape %zu x %zu words exceeds the device u32 index ceiling (%zu); "
                        "use the CPU rlib face", n_rows, w, ceiling));
    size_t es = dtype_size(dtype);
    if (n_rows == 0) return QBK_OK;
    if (n_bits == 0) {  // zero logical bits: every row's sum is empty
        memset(out, 0, n_rows * es);
        return QBK_OK;
    }
    if ((rc = bind(ctx))) return rc;
    CallStream cs;
    DevBuf dp, dv, dout;
    if ((rc = cs.create()) || (rc = dp.alloc(packed_len)) || (rc = dv.alloc(vec_len * es)) ||
        (rc = dout.alloc(n_rows * es)))
        return rc;
    QBK_HIP(hipMemcpyAsync(dp.p, packed, packed_len, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dv.p, vec, vec_len * es, hipMemcpyHostToDevice, cs.s));
    if ((rc = launch_matvec(dtype, (const uint8_t *)dp.p, n_rows, n_bits, dv.p, dout.p, cs.s)))
        return rc;
    QBK_HIP(hipMemcpyAsync(out, dout.p, n_rows * es, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_packed_matmul(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t packed_len,
                      size_t n_rows, size_t n_bits, const void *mat, size_t mat_len,
                      size_t n_cols, void *out) {
    int rc;
    if ((rc = check_dtype(dtype))) return rc;
    size_t w;
    if ((rc = validate_packed(packed_len, n_rows, n_bits, &w))) return rc;
    if (n_bits != 0 && mat_len % n_bits != 0)
        return fail(QBK_ERR_VALIDATION,
                    fmt("mat length %zu is not a multiple of n_bits %zu", mat_len, n_bits));
    size_t k = mat_len / (n_bits ? n_bits : 1);
    size_t es = dtype_size(dtype);
    if (n_rows == 0 || k == 0) return QBK_OK;
    if (n_bits == 0) {
        memset(out, 0, n_rows * k * es);
        return QBK_OK;
    }
    if ((n_bits - 1) * n_cols + (k - 1) >= mat_len)
        return fail(QBK_ERR_VALIDATION,
                    fmt("mat index out of range: n_cols %zu with %zu columns over %zu rows",
                        n_cols, k, n_bits));
    if ((rc = bind(ctx))) return rc;
    CallStream cs;
    DevBuf dp, dm, dout;
    if ((rc = cs.create()) || (rc = dp.alloc(packed_len)) || (rc = dm.alloc(mat_len * es)) ||
        (rc = dout.alloc(n_rows * k * es)))
        return rc;
    QBK_HIP(hipMemcpyAsync(dp.p, packed, packed_len, hipMemcpyHostToDevice, cs.s));
    QBK_HIP(hipMemcpyAsync(dm.p, mat, mat_len * es, hipMemcpyHostToDevice, cs.s));
    if ((rc = launch_matmul(dtype, (const uint8_t *)dp.p, n_rows, n_bits, dm.p, k, n_cols,
                            dout.p, cs.s)))
        return rc;
    QBK_HIP(hipMemcpyAsync(out, dout.p, n_rows * k * es, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

int qbk_packed_matvec_dev(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t n_rows,
                          size_t n_bits, const void *vec, void *out, void *stream) {
    int rc;
    if ((rc = check_dtype(dtype))) return rc;
    if (n_rows == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (n_bits == 0) {
        QBK_HIP(hipMemsetAsync(out, 0, n_rows * dtype_size(dtype), s));
        return QBK_OK;
    }
    return launch_matvec(dtype, packed, n_rows, n_bits, vec, out, s);
}

int qbk_packed_matmul_dev(qbk_ctx *ctx, int dtype, const uint8_t *packed, size_t n_rows,
                          size_t n_bits, const void *mat, size_t k_cols, size_t n_cols, void *out,
                          void *stream) {
    int rc;
    if ((rc = check_dtype(dtype))) return rc;
    if (n_rows == 0 || k_cols == 0) return QBK_OK;
    if ((rc = bind(ctx))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (n_bits == 0) {
        QBK_HIP(hipMemsetAsync(out, 0, n_rows * k_cols * dtype_size(dtype), s));
        return QBK_OK;
    }
    if (n_cols < k_cols)
        return fail(QBK_ERR_VALIDATION,
                    fmt("n_cols %zu is narrower than the %zu output columns", n_cols, k_cols));
    return launch_matmul(dtype, packed, n_rows, n_bits, mat, k_cols, n_cols, out, s);
}

}  // extern "C"
