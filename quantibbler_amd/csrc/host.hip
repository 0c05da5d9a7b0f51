// host.hip -- host-side pieces of libqbk: errors, the device context, and the
// bit-layout functions of core.rs (pack/unpack/validate/sign_estimate), which
// the reference also runs on the host.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "qbk_internal.h"

namespace qbk {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

std::string fmt(const char *f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return std::string(buf);
}

int bind(qbk_ctx *ctx) {
    if (!ctx) return fail(QBK_ERR_VALIDATION, "null qbk_ctx");
    QBK_HIP(hipSetDevice(ctx->device));
    return QBK_OK;
}

// core.rs:223-240
int validate_packed(size_t packed_len, size_t n_rows, size_t n_bits, size_t *n_words) {
    if (n_bits == 0 && packed_len != 0 && n_rows != 0)
        return fail(QBK_ERR_VALIDATION, "n_bits=0 with non-empty packed rows");
    size_t w = div_ceil(n_bits, 8);
    if (n_rows * w != packed_len)
        return fail(QBK_ERR_VALIDATION,
                    fmt("packed length %zu does not match %zu rows x %zu bitplanes", packed_len,
                        n_rows, w));
    if (n_words) *n_words = w;
    return QBK_OK;
}

}  // namespace qbk

using namespace qbk;

extern "C" {

const char *qbk_backend_version(void) { return "0.1.0-gfx950"; }

const char *qbk_last_error(void) { return g_last_error.c_str(); }

// dtype.rs:110-119
int qbk_dtype_from_name(const char *name, int *dtype_out) {
    if (!name) return fail(QBK_ERR_VALIDATION, "null dtype name");
    if (!strcmp(name, "float64")) *dtype_out = QBK_F64;
    else if (!strcmp(name, "float32")) *dtype_out = QBK_F32;
    else if (!strcmp(name, "bfloat16")) *dtype_out = QBK_BF16;
    else
        return fail(QBK_ERR_VALIDATION,
                    fmt("unknown kernel dtype \"%s\"; expected one of \"float64\", \"float32\", "
                        "\"bfloat16\"",
                        name));
    return QBK_OK;
}

// core.rs:129-162 -- LSB-first bitplanes.  The inner loop packs one byte from
// eight sign tests; validation order (first bad value in row-major order)
// matches the reference so the same element is named.
int qbk_pack_bits(const int8_t *factor, size_t factor_len, size_t n_rows, size_t n_cols,
                  uint8_t *out) {
    if (n_rows * n_cols != factor_len)
        return fail(QBK_ERR_VALIDATION,
                    fmt("factor length %zu does not match %zux%zu", factor_len, n_rows, n_cols));
    for (size_t i = 0; i < factor_len; i++) {
        int8_t v = factor[i];
        if (v != 1 && v != -1)
            return fail(QBK_ERR_VALIDATION,
                        fmt("pack_bits expects values in {-1, +1}; got %d at row %zu, column %zu",
                            (int)v, i / n_cols, i % n_cols));
    }
    size_t w = div_ceil(n_cols, 8);
    for (size_t i = 0; i < n_rows; i++) {
        const int8_t *row = factor + i * n_cols;
        for (size_t j = 0; j < w; j++) {
            unsigned byte = 0;
            size_t k1 = (j * 8 + 8 < n_cols) ? 8 : n_cols - j * 8;
            for (size_t k = 0; k < k1; k++) byte |= (unsigned)(row[j * 8 + k] == 1) << k;
            out[i * w + j] = (uint8_t)byte;
        }
    }
    return QBK_OK;
}

// core.rs:166-189
int qbk_unpack_bits(const uint8_t *packed, size_t packed_len, size_t n_rows, size_t n_bits,
                    int8_t *out) {
    size_t w = div_ceil(n_bits, 8);
    if (n_rows * w != packed_len)
        return fail(QBK_ERR_VALIDATION,
                    fmt("packed length %zu does not match %zu rows x %zu bitplanes", packed_len,
                        n_rows, w));
    for (size_t i = 0; i < n_rows; i++) {
        const uint8_t *row = packed + i * w;
        int8_t *o = out + i * n_bits;
        for (size_t k = 0; k < n_bits; k++) o[k] = (int8_t)(((row[k >> 3] >> (k & 7)) & 1) * 2 - 1);
    }
    return QBK_OK;
}

int qbk_validate_packed(size_t packed_len, size_t n_rows, size_t n_bits, size_t *n_words) {
    return validate_packed(packed_len, n_rows, n_bits, n_words);
}

void qbk_sign_estimate(const double *x, size_t n, int8_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = x[i] >= 0.0 ? 1 : -1;
}

// gpu.rs:85-101 GpuContext::init_at: fail-closed with an actionable hint.
static const char *kInitHint =
    "no usable HIP/ROCm device; libqbk needs an AMD Instinct MI355X (gfx950) visible "
    "through /dev/kfd and /dev/dri/renderD* with the ROCm runtime (libamdhip64.so) "
    "on the library path";

int qbk_ctx_create(int device_index, qbk_ctx **out) {
    if (!out) return fail(QBK_ERR_VALIDATION, "null output pointer");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return fail(QBK_ERR_INIT, fmt("%s; device probe failed at index %d: %s", kInitHint,
                                      device_index,
                                      e != hipSuccess ? hipGetErrorString(e) : "no devices"));
    if (device_index < 0 || device_index >= n)
        return fail(QBK_ERR_INIT, fmt("%s; device probe failed at index %d: %d device(s) visible",
                                      kInitHint, device_index, n));
    qbk_ctx *c = new qbk_ctx();
    c->device = device_index;
    e = hipGetDeviceProperties(&c->props, device_index);
    if (e != hipSuccess) {
        delete c;
        return fail(QBK_ERR_INIT, fmt("%s; hipGetDeviceProperties failed: %s", kInitHint,
                                      hipGetErrorString(e)));
    }
    if (strncmp(c->props.gcnArchName, "gfx950", 6) != 0) {
        std::string arch = c->props.gcnArchName;
        delete c;
        return fail(QBK_ERR_INIT, fmt("%s; device %d is %s, this build targets gfx950", kInitHint,
                                      device_index, arch.c_str()));
    }
    c->num_cus = c->props.multiProcessorCount;
    *out = c;
    return QBK_OK;
}

void qbk_ctx_destroy(qbk_ctx *ctx) { delete ctx; }

int qbk_gpu_available(void) {
    qbk_ctx *c = nullptr;
    int rc = qbk_ctx_create(0, &c);
    if (rc == QBK_OK) qbk_ctx_destroy(c);
    return rc == QBK_OK;
}

}  // extern "C"
