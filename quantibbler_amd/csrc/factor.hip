// factor.hip -- the binary latent-factor linear on gfx950.
//
//   y = s1 . (Ub (Vb^T (s2 . x))) + b           (engine/mod.rs:393-481)
//
// bf16 serving composite (apply_bf16, engine/mod.rs:449-460), per token:
//   z = bf16(s2*x);  t = bf16(Vb^T z);  u = bf16(Ub t);  y = f32(u)*s1 + b
// with f32 accumulation of the +-1 products.
//
// This file: layer upload and repack, and the host faces.  The decode GEMV
// (batch 1-8) and layer sets are in decode.hip, the prefill GEMM (batch > 8)
// in prefill.hip.
//
// A layer is uploaded once and repacked into three device layouts:
//   * ref rows   : the engine's per-row bitplanes (ub_rows, vb_t_rows) for
//                  the f64 serving path (sequential, bit-identical);
//   * q4 words   : (64-row group, 128-k slice) blocks of 64 lane x 4 words
//                  in the fp4 operand order of the scaled MFMA (decode);
//   * g32 words  : (128-row group, 64-k slice) blocks of 64 lane x 4 words,
//                  the bits one lane needs for the 32x32x16 bf16 A fragments
//                  of four row tiles (prefill GEMM, prefill.hip).
//
// Padded rows of Vb^T produce garbage t values; every consumer of t masks
// k >= r to zero, so padding never reaches the output.
#include <string.h>

#include <vector>

#include <mutex>

#include "factor_internal.h"

namespace qbk {

// ------------------------------------------------------------------------
// host-side repack
// ------------------------------------------------------------------------

static inline int rbit(const uint8_t *rows, size_t row_words, size_t i, size_t k) {
    return (rows[i * row_words + (k >> 3)] >> (k & 7)) & 1;
}

// fp4 decode layout.  The scaled 16x16x128 MFMA with an fp4 A operand gives
// lane group g = l/16 the 32 elements k = kq4(g, e) of a 128-k slice, and an
// fp8 B operand gives group g the elements 32g .. 32g+31 (measured pairing).
__host__ __device__ inline int kq4(int g, int e) {
    return 16 * (g >> 1) + 64 * (g & 1) + (e & 15) + 32 * (e >> 4);
}
// Word for (row group rg, slice s, lane l, row tile rt): element e of row
// 64rg + 16rt + l%16 is stored at bit 4*(e%8) + e/8, set when the sign is -1,
// so VGPR v of the fp4 operand is one v_lshl_or_b32: (word << (3 - v)) |
// 0x77777777, every nibble then e2m1 0111 = +6 with the sign bit on top (the
// MFMA's A scale 2^-2 makes it +-1.5, which the epilogue divides out).
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

// The reference's per-row bitplanes (bit k of row i at byte k/8, LSB first,
// set for +1) rebuilt from the fp4 decode layout: one thread per row byte,
// each of its bits read from the word and bit repack_q4 put it at (the
// inverse of kq4: k % 128 = 64 (g & 1) + 32 (e >> 4) + 16 (g >> 1) + e % 16).
__global__ void q4_to_rows(const uint32_t *q4, size_t n_rows, size_t n_bits, size_t bits_q, uint8_t *rows) {
    const size_t rw = (n_bits + 7) / 8, idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * rw) return;
    const size_t i = idx / rw, j = idx % rw, ns = bits_q / 128;
    const size_t rg = i / 64, rt = (i % 64) / 16, l15 = i % 16;
    uint32_t byte = 0;
    for (int b = 0; b < 8; b++) {
        const size_t k = 8 * j + b;
        if (k >= n_bits) break;
        const uint32_t kk = (uint32_t)(k % 128), s = (uint32_t)(k / 128);
        const uint32_t g = 2 * ((kk >> 4) & 1) + ((kk >> 6) & 1), e = 16 * ((kk >> 5) & 1) + (kk & 15);
        const uint32_t w = q4[((rg * ns + s) * 64 + 16 * g + l15) * 4 + rt];
        if (!((w >> (4 * (e & 7) + (e >> 3))) & 1)) byte |= 1u << b;
    }
    rows[idx] = (uint8_t)byte;
}

// v's fp16 bits when v is an fp16 value (zero, a normal or subnormal fp16
// magnitude, or an infinity), else false.  The conversion is exact, so no
// rounding is involved.
static bool f32_to_f16_exact(float v, uint16_t *out) {
    uint32_t u;
    memcpy(&u, &v, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, ex = (u >> 23) & 0xff, man = u & 0x7fffffu;
    if (ex == 0xff) {
        if (man) return false;  // NaN: kept in f32
        *out = (uint16_t)(sign | 0x7c00u);
        return true;
    }
    if (ex == 0 && man == 0) {
        *out = (uint16_t)sign;
        return true;
    }
    if (ex == 0) return false;  // f32 subnormals lie below fp16's range
    const int e = (int)ex - 127;
    if (e > 15) return false;
    if (e >= -14) {
        if (man & 0x1fffu) return false;
        *out = (uint16_t)(sign | (uint32_t)(e + 15) << 10 | (man >> 13));
        return true;
    }
    if (e < -24) return false;
    // fp16 subnormal: m * 2^-24 with the implicit bit shifted in
    const uint32_t full = man | 0x800000u, shift = (uint32_t)(13 + (-14 - e));
    if (full & ((1u << shift) - 1)) return false;
    *out = (uint16_t)(sign | (full >> shift));
    return true;
}

static bool f16_copy(const float *v, size_t n, std::vector<uint16_t> &h) {
    h.resize(n);
    for (size_t i = 0; i < n; i++)
        if (!f32_to_f16_exact(v[i], &h[i])) return false;
    return true;
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
    std::vector<uint32_t> vf(L->r_p * L->din_p / 32), uf(L->dout_p * L->r_p / 32);
    g32_repack(vbt_rows, r, din, L->r_p, L->din_p, vf.data());
    g32_repack(ub_rows, dout, r, L->dout_p, L->r_p, uf.data());
    L->din_q = round_up(din, 128);
    L->r_q = round_up(r, 128);
    std::vector<uint32_t> vq(L->r_p / 64 * L->din_q / 128 * 256), uq(L->dout_p / 64 * L->r_q / 128 * 256);
    repack_q4(vbt_rows, r, din, L->r_p, L->din_q, vq.data());
    repack_q4(ub_rows, dout, r, L->dout_p, L->r_q, uq.data());
    std::vector<float> zb(dout, 0.0f);
    L->bias_zero = true;  // no bias, or every entry +0.0: y = v * s1 + 0.0 needs no load
    for (size_t i = 0; bias && i < dout; i++) {
        uint32_t u;
        memcpy(&u, bias + i, 4);
        if (u != 0) {
            L->bias_zero = false;
            break;
        }
    }
    void *p;
#define UP(field, src, n)                                                  \
    if ((rc = dev_upload(L, &p, src, n))) {                                \
        destroy_layer(L);                                                  \
        return rc;                                                         \
    }                                                                      \
    L->field = (decltype(L->field))p;
    L->ub_rows = L->vbt_rows = nullptr;  // formed on the first f64-face call (q4_to_rows)
    UP(vt_g32, vf.data(), vf.size() * 4);
    UP(u_g32, uf.data(), uf.size() * 4);
    UP(vt_q4, vq.data(), vq.size() * 4);
    UP(u_q4, uq.data(), uq.size() * 4);
    UP(s1, s1, dout * 4);
    UP(s2, s2, din * 4);
    UP(bias, bias ? bias : zb.data(), dout * 4);
    // fp16 copies where the scales are fp16 values (v2 qpk1 streams): the
    // decode GEMV then streams half the scale bytes
    {
        std::vector<uint16_t> h1, h2, hb;
        L->scales_f16 = f16_copy(s1, dout, h1) && f16_copy(s2, din, h2) &&
                        f16_copy(bias ? bias : zb.data(), dout, hb);
        L->s1h = L->s2h = L->biash = nullptr;
        if (L->scales_f16) {
            UP(s1h, h1.data(), dout * 2);
            UP(s2h, h2.data(), din * 2);
            UP(biash, hb.data(), dout * 2);
        }
    }
    Q4Layer qtab[2];
    q4_layer_entries(L, qtab);
    UP(q4_tab, qtab, sizeof qtab);
#undef UP
    *out = L;
    return QBK_OK;
}

// ------------------------------------------------------------------------
// host orchestration
// ------------------------------------------------------------------------

// batch <= Q4_MAXB: the fp4 decode's operand buffers (decode.hip).  Larger
// batches: the fused GEMM's t (gemm.hip), or the two-stage GEMM's z, split
// partials and t (prefill.hip).
static size_t ws_bytes(const qbk_factor *L, size_t batch) {
    return batch <= Q4_MAXB ? q4_workspace(L, batch) : gemm_workspace(L, batch);
}

// ---- the no-allocation form of qbk_factor_linear_dev --------------------
//
// For callers that cannot allocate (code under graph capture, serving loops
// that forbid hipMalloc): the workspace is this file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol); it passes the device address hipGetSymbolAddress returns, looked
// up once per device with that device current and kept per device.
// Every call on a GPU shares that GPU's array, so calls that overlap on one
// GPU race; the kernels write every byte they later read, so nothing needs
// clearing between calls.
static __device__ __align__(256) uint8_t scratch[QBK_NOALLOC_SCRATCH_BYTES];

static int scratch_address(int device, void **out) {
    static std::mutex mu;
    static void *addr[64] = {};
    if (device < 0 || device >= 64) return fail(QBK_ERR_DEVICE, fmt("device index %d out of range", device));
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        void *p = nullptr;
        QBK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        addr[device] = p;
    }
    *out = addr[device];
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
    return ws_bytes(L, batch);
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
    size_t need = ws_bytes(L, batch);
    if (workspace_size < need)
        return fail(QBK_ERR_VALIDATION,
                    fmt("workspace of %zu bytes is smaller than the %zu this call needs",
                        workspace_size, need));
    hipStream_t s = (hipStream_t)stream;
    if (batch <= Q4_MAXB) return q4_run(L, batch, x, false, y, y_dtype == QBK_BF16, workspace, s);
    return gemm_run(L, x, false, batch, y, y_dtype == QBK_BF16, workspace, s);
}

int qbk_factor_linear_noalloc_dev(qbk_ctx *ctx, const qbk_factor *L, const uint16_t *x, size_t batch, void *y,
                                  int y_dtype, void *stream) {
    int rc;
    if (!L) return fail(QBK_ERR_VALIDATION, "null layer");
    if (batch == 0) return QBK_OK;
    const size_t need = ws_bytes(L, batch);
    if (need > QBK_NOALLOC_SCRATCH_BYTES)
        return fail(QBK_ERR_VALIDATION,
                    fmt("this call needs %zu bytes of workspace; the no-allocation entry point holds %zu "
                        "(use qbk_factor_linear_dev with a workspace)",
                        need, (size_t)QBK_NOALLOC_SCRATCH_BYTES));
    if ((rc = bind(ctx))) return rc;
    void *ws = nullptr;
    if ((rc = scratch_address(ctx->device, &ws))) return rc;
    return qbk_factor_linear_dev(ctx, L, x, batch, y, y_dtype, ws, need, stream);
}

// The f64 serving path's two elementwise ends (engine/mod.rs:419-436):
// z = f64(s2 * x), an f32 product widened; y = f32(u) * s1 + b, a multiply
// then an add (the file is built without contraction).
__global__ void factor_f64_in(const float *x, const float *s2, double *z, size_t n) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) z[i] = (double)(s2[i] * x[i]);
}

__global__ void factor_f64_out(const double *u, const float *s1, const float *bias, float *y, size_t n) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) y[i] = ((float)u[i]) * s1[i] + bias[i];
}

}  // extern "C"

namespace qbk {

// The reference's row bitplanes of L (ub_rows, vbt_rows), formed from the
// decode layout on first use and kept with the layer.
int factor_rows_ready(const qbk_factor *L, hipStream_t s) {
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    if (L->ub_rows) return QBK_OK;
    qbk_factor *M = const_cast<qbk_factor *>(L);
    void *pu = nullptr, *pv = nullptr;
    const size_t nu = L->dout * div_ceil(L->r, 8), nv = L->r * div_ceil(L->din, 8);
    QBK_HIP(hipMalloc(&pu, nu));
    M->allocs.push_back(pu);
    QBK_HIP(hipMalloc(&pv, nv));
    M->allocs.push_back(pv);
    hipLaunchKernelGGL(q4_to_rows, dim3((unsigned)div_ceil(nu, 256)), dim3(256), 0, s, L->u_q4, L->dout, L->r,
                       L->r_q, (uint8_t *)pu);
    QBK_HIP(hipGetLastError());
    hipLaunchKernelGGL(q4_to_rows, dim3((unsigned)div_ceil(nv, 256)), dim3(256), 0, s, L->vt_q4, L->r, L->din,
                       L->din_q, (uint8_t *)pv);
    QBK_HIP(hipGetLastError());
    QBK_HIP(hipStreamSynchronize(s));
    M->vbt_rows = (uint8_t *)pv;
    M->ub_rows = (uint8_t *)pu;
    return QBK_OK;
}

// apply's fp32 serving (engine/mod.rs:393-436) of one token on the device:
// z = f64(s2 x), t = Vb^T z and u = Ub t as f64 matvecs in element order
// (the packed f64 product), y = f32(u) s1 + b.  x, y f32 device vectors;
// scratch holds din + r + dout doubles; the rows must be formed
// (factor_rows_ready).
int factor_apply_f64_dev(qbk_ctx *ctx, const qbk_factor *L, const float *x, float *y, double *scratch,
                         hipStream_t s) {
    int rc;
    double *z = scratch, *t = z + L->din, *u = t + L->r;
    hipLaunchKernelGGL(factor_f64_in, dim3((unsigned)((L->din + 255) / 256)), dim3(256), 0, s, x,
                       (const float *)L->s2, z, L->din);
    QBK_HIP(hipGetLastError());
    if ((rc = qbk_packed_matvec_dev(ctx, QBK_F64, L->vbt_rows, L->r, L->din, z, t, s))) return rc;
    if ((rc = qbk_packed_matvec_dev(ctx, QBK_F64, L->ub_rows, L->dout, L->r, t, u, s))) return rc;
    hipLaunchKernelGGL(factor_f64_out, dim3((unsigned)((L->dout + 255) / 256)), dim3(256), 0, s, (const double *)u,
                       (const float *)L->s1, (const float *)L->bias, y, L->dout);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

}  // namespace qbk

extern "C" {

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
        // per token: z = f64(s2*x), the two f64 matvecs in element order,
        // y = f32(u)*s1 + b -- all on the device.  The matvecs read the
        // reference's row layout, which the layer forms from its decode
        // layout on the first such call (a third copy of the signs only for
        // layers that use this face).
        if ((rc = factor_rows_ready(L, cs.s))) return rc;
        DevBuf dx, dy, dsc;
        if ((rc = dx.alloc(batch * L->din * 4)) || (rc = dy.alloc(batch * L->dout * 4)) ||
            (rc = dsc.alloc((L->din + L->r + L->dout) * 8)))
            return rc;
        QBK_HIP(hipMemcpyAsync(dx.p, x, batch * L->din * 4, hipMemcpyHostToDevice, cs.s));
        for (size_t bb = 0; bb < batch; bb++)
            if ((rc = factor_apply_f64_dev(ctx, L, (const float *)dx.p + bb * L->din, (float *)dy.p + bb * L->dout,
                                           (double *)dsc.p, cs.s)))
                return rc;
        QBK_HIP(hipMemcpyAsync(y, dy.p, batch * L->dout * 4, hipMemcpyDeviceToHost, cs.s));
        QBK_HIP(hipStreamSynchronize(cs.s));
        return QBK_OK;
    }
    DevBuf dx, dy, dws;
    if ((rc = dx.alloc(batch * L->din * 4)) || (rc = dy.alloc(batch * L->dout * 4)) ||
        (rc = dws.alloc(ws_bytes(L, batch))))
        return rc;
    QBK_HIP(hipMemcpyAsync(dx.p, x, batch * L->din * 4, hipMemcpyHostToDevice, cs.s));
    if (batch <= Q4_MAXB)
        rc = q4_run(L, batch, dx.p, true, dy.p, false, dws.p, cs.s);
    else
        rc = gemm_run(L, dx.p, true, batch, dy.p, false, dws.p, cs.s);
    if (rc) return rc;
    QBK_HIP(hipMemcpyAsync(y, dy.p, batch * L->dout * 4, hipMemcpyDeviceToHost, cs.s));
    QBK_HIP(hipStreamSynchronize(cs.s));
    return QBK_OK;
}

}  // extern "C"
