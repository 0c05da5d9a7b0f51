// block.hip -- one decoder block of the server's transformer at one position.
//
// engine/mod.rs:878-945 (Engine::transformer, the body of its block loop)
// at bf16 serving with the sage decode attention (engine/mod.rs:984-1030):
//
//   x  = bf16(rmsnorm(bf16(h)) * w_in)                 (:837-852, :1154-1166)
//   q, k, v = apply_bf16(x)                             (:901-906)
//   q, k rotated by RoPE at position pos                (:911-912, :1169-1187)
//   k, v appended to the block's cache                  (:913)
//   a  = attention of q over the cache's pos + 1 rows   (:918)
//   h1 = apply_bf16(a; o) + h                           (:919-923)
//   x2 = bf16(rmsnorm(bf16(h1)) * w_post)               (:926)
//   g, u = apply_bf16(x2; gate), apply_bf16(x2; up)     (:928-929)
//   h' = apply_bf16(g u / (1 + exp(-g)); down) + h1     (:930-942)
//
// The projections are the device factor linears (q/k/v as one layer set,
// gate/up as another), the attention is the decode step on the block's kept
// state (bit-identical to the reference's padded call), RoPE's angles come
// from a table the host builds with the reference's f64 formula, and the
// norms, SwiGLU and residual adds are small kernels here.  Two of those
// differ from the reference's sequence in rounding, not in formula: the
// norm's sum of squares is a tree (the reference's is one 4096-long chain)
// and exp is the device's.  The block is checked against the oracle's
// restatement to a stated tolerance; its parts that are bit-exact stay so.
// No per-head q/k norms (Llama-style blocks).
#include <math.h>
#include <string.h>

#include <vector>

#include "factor_internal.h"

#pragma clang fp contract(off)

struct qbk_block {
    int device;
    size_t d, H, Hk, hd, ffn, cap, block;
    float eps;
    const qbk_factor *o, *down;
    qbk_factor_set *qkv, *gu;
    float *w_in, *w_post;     // d each
    float2 *rope;             // [cap][hd / 2] (cos, sin) in f32, from f64
    float *kc, *vc;           // [cap][Hk * hd] the block's KV cache
    void *state;              // the attention's kept decode state
    size_t state_bytes;
    size_t tokens;            // cache rows the state's codes cover
    // per-call buffers
    uint16_t *xcat;           // bf16 [3 d] (q, k, v inputs), then [2 d] (gate, up)
    float *ycat;              // f32 [(H + 2 Hk) hd], then [2 ffn]
    float *qrot, *attn, *oout, *h1, *hid, *dout;
    void *ws;
    size_t ws_bytes;
    std::vector<void *> allocs;
};

namespace qbk {

#define BLKD_NORM_THREADS 1024

__device__ __forceinline__ uint16_t blkd_bf16(float x) {  // RNE (finite x)
    const uint32_t u = __float_as_uint(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// hsum = a (+ r when r); optionally stored to hout; x = bf16 of the
// RMS-normalised bf16(hsum) times w, written nrep times, one copy a d
__global__ void __launch_bounds__(BLKD_NORM_THREADS) blkd_norm(const float *a, const float *r, float *hout,
                                                              const float *w, float eps, uint16_t *x, int nrep,
                                                              int d) {
    __shared__ float red[BLKD_NORM_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.0f;
    for (int i = tid; i < d; i += BLKD_NORM_THREADS) {
        float v = a[i];
        if (r) v = v + r[i];
        if (hout) hout[i] = v;
        const float b = __uint_as_float((uint32_t)blkd_bf16(v) << 16);
        ss += b * b;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < BLKD_NORM_THREADS / 64; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    for (int i = tid; i < d; i += BLKD_NORM_THREADS) {
        float v = a[i];
        if (r) v = v + r[i];
        const float b = __uint_as_float((uint32_t)blkd_bf16(v) << 16);
        const uint16_t o = blkd_bf16(b * inv * w[i]);
        for (int k = 0; k < nrep; k++) x[k * d + i] = o;
    }
}

// RoPE (rotate_half pairs (i, i + hd/2)) of q and k at position pos, q to
// qrot, k and v to cache row pos; qkv = [q (H hd) | k (Hk hd) | v (Hk hd)]
__global__ void blkd_rope_append(const float *qkv, const float2 *rope, size_t pos, float *qrot, float *kc,
                                 float *vc, int H, int Hk, int hd) {
    const int half = hd / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int nq = H * half, nk = Hk * half;
    const float2 cs = rope[pos * (size_t)half + (i < nq ? i % half : (i - nq) % half)];
    if (i < nq) {
        const int head = i / half, j = i % half, base = head * hd;
        const float a = qkv[base + j], b = qkv[base + half + j];
        qrot[base + j] = a * cs.x - b * cs.y;
        qrot[base + half + j] = b * cs.x + a * cs.y;
    } else if (i < nq + nk) {
        const int t = i - nq, head = t / half, j = t % half, base = head * hd;
        const float *k = qkv + (size_t)H * hd, *v = k + (size_t)Hk * hd;
        float *kr = kc + pos * (size_t)Hk * hd, *vr = vc + pos * (size_t)Hk * hd;
        const float a = k[base + j], b = k[base + half + j];
        kr[base + j] = a * cs.x - b * cs.y;
        kr[base + half + j] = b * cs.x + a * cs.y;
        vr[base + j] = v[base + j];
        vr[base + half + j] = v[base + half + j];
    }
}

// hidden = g u / (1 + exp(-g)); gu = [g (ffn) | u (ffn)]
__global__ void blkd_swiglu(const float *gu, float *hid, int ffn) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < ffn) {
        const float g = gu[i], u = gu[ffn + i];
        hid[i] = g * u / (1.0f + expf(0.0f - g));
    }
}

__global__ void blkd_add(const float *a, const float *b, float *out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

}  // namespace qbk

using namespace qbk;

extern "C" {

void qbk_block_destroy(qbk_block *B) {
    if (!B) return;
    (void)hipSetDevice(B->device);
    (void)hipDeviceSynchronize();
    if (B->qkv) qbk_factor_set_destroy(B->qkv);
    if (B->gu) qbk_factor_set_destroy(B->gu);
    for (void *p : B->allocs) (void)hipFree(p);
    delete B;
}

int qbk_block_create(qbk_ctx *ctx, const qbk_factor *const *layers, const float *input_norm,
                     const float *post_norm, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                     double rope_theta, double rms_norm_eps, size_t capacity, size_t block_size,
                     qbk_block **out) {
    int rc;
    if (!layers || !input_norm || !post_norm || !out) return fail(QBK_ERR_VALIDATION, "null argument");
    for (int i = 0; i < 7; i++)
        if (!layers[i]) return fail(QBK_ERR_VALIDATION, "null layer");
    size_t dims[7][3];
    for (int i = 0; i < 7; i++) qbk_factor_dims(layers[i], &dims[i][0], &dims[i][1], &dims[i][2]);
    const size_t d = dims[0][1], H = n_heads, Hk = n_kv_heads, hd = head_dim, ffn = dims[4][0];
    if (H == 0 || Hk == 0 || hd == 0 || hd % 2 || H % Hk)
        return fail(QBK_ERR_VALIDATION, "decoder block needs n_kv_heads dividing n_heads and an even head_dim");
    // q (H hd x d), k, v (Hk hd x d), o (d x H hd), gate, up (ffn x d), down (d x ffn)
    const size_t want[7][2] = {{H * hd, d}, {Hk * hd, d}, {Hk * hd, d}, {d, H * hd}, {ffn, d}, {ffn, d}, {d, ffn}};
    static const char *names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
    for (int i = 0; i < 7; i++)
        if (dims[i][0] != want[i][0] || dims[i][1] != want[i][1])
            return fail(QBK_ERR_VALIDATION, fmt("decoder block: %s is %zux%zu, expected %zux%zu", names[i],
                                                dims[i][0], dims[i][1], want[i][0], want[i][1]));
    if (capacity == 0 || block_size == 0) return fail(QBK_ERR_VALIDATION, "decoder block needs a capacity and a block size");
    if ((rc = bind(ctx))) return rc;
    qbk_block *B = new qbk_block();
    B->device = ctx->device;
    B->d = d;
    B->H = H;
    B->Hk = Hk;
    B->hd = hd;
    B->ffn = ffn;
    B->cap = capacity;
    B->block = block_size;
    B->eps = (float)rms_norm_eps;
    B->o = layers[3];
    B->down = layers[6];
    auto alloc = [&](void **p, size_t n) -> int {
        hipError_t e = hipMalloc(p, n ? n : 4);
        if (e != hipSuccess) return fail(QBK_ERR_DEVICE, fmt("hipMalloc(%zu): %s", n, hipGetErrorString(e)));
        B->allocs.push_back(*p);
        return QBK_OK;
    };
    const qbk_factor *qkv[3] = {layers[0], layers[1], layers[2]}, *gu[2] = {layers[4], layers[5]};
    qbk_attn_shape sh{1, H, Hk, 1, capacity, hd, hd};
    B->state_bytes = qbk_sage_decode_workspace_size(&sh, block_size);
    const size_t kv = capacity * Hk * hd * 4;
    if ((rc = qbk_factor_set_create(ctx, qkv, 3, &B->qkv)) || (rc = qbk_factor_set_create(ctx, gu, 2, &B->gu)) ||
        (rc = alloc((void **)&B->w_in, d * 4)) || (rc = alloc((void **)&B->w_post, d * 4)) ||
        (rc = alloc((void **)&B->rope, capacity * (hd / 2) * 8)) || (rc = alloc((void **)&B->kc, kv)) ||
        (rc = alloc((void **)&B->vc, kv)) || (rc = alloc(&B->state, B->state_bytes)) ||
        (rc = alloc((void **)&B->xcat, 3 * d * 2)) ||
        (rc = alloc((void **)&B->ycat, ((H + 2 * Hk) * hd > 2 * ffn ? (H + 2 * Hk) * hd : 2 * ffn) * 4)) ||
        (rc = alloc((void **)&B->qrot, H * hd * 4)) || (rc = alloc((void **)&B->attn, H * hd * 4)) ||
        (rc = alloc((void **)&B->oout, d * 4)) || (rc = alloc((void **)&B->h1, d * 4)) ||
        (rc = alloc((void **)&B->hid, ffn * 4)) || (rc = alloc((void **)&B->dout, d * 4))) {
        qbk_block_destroy(B);
        return rc;
    }
    size_t ws = q4_set_workspace(B->qkv);
    const size_t wss[3] = {q4_set_workspace(B->gu), q4_workspace(B->o, 1), q4_workspace(B->down, 1)};
    for (size_t w : wss) ws = w > ws ? w : ws;
    B->ws_bytes = ws;
    if ((rc = alloc(&B->ws, ws))) {
        qbk_block_destroy(B);
        return rc;
    }
    // RoPE angles as rope_rotate forms them (engine/mod.rs:1169-1187): f64
    // inv_freq = theta^(-2i / hd), (sin, cos) of pos * inv_freq, then f32
    std::vector<float2> tab(capacity * (hd / 2));
    for (size_t p = 0; p < capacity; p++)
        for (size_t i = 0; i < hd / 2; i++) {
            const double inv_freq = pow(rope_theta, -(2.0 * (double)i) / (double)hd);
            const double ang = (double)p * inv_freq;
            tab[p * (hd / 2) + i] = make_float2((float)cos(ang), (float)sin(ang));
        }
    hipError_t e = hipMemcpy(B->rope, tab.data(), tab.size() * 8, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(B->w_in, input_norm, d * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(B->w_post, post_norm, d * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        qbk_block_destroy(B);
        return fail(QBK_ERR_DEVICE, fmt("hipMemcpy: %s", hipGetErrorString(e)));
    }
    *out = B;
    return QBK_OK;
}

int qbk_block_cache(const qbk_block *B, float **k_cache, float **v_cache) {
    if (!B) return fail(QBK_ERR_VALIDATION, "null block");
    if (k_cache) *k_cache = B->kc;
    if (v_cache) *v_cache = B->vc;
    return QBK_OK;
}

int qbk_block_decode_dev(qbk_ctx *ctx, qbk_block *B, float *h, size_t pos, void *stream) {
    int rc;
    if (!B || !h) return fail(QBK_ERR_VALIDATION, "null argument");
    if (pos >= B->cap)
        return fail(QBK_ERR_VALIDATION, fmt("position %zu is past the block's cache capacity of %zu", pos, B->cap));
    if ((rc = bind(ctx))) return rc;
    if (B->device != ctx->device) return fail(QBK_ERR_VALIDATION, "block lives on another device than the context");
    hipStream_t s = (hipStream_t)stream;
    const int d = (int)B->d, hd = (int)B->hd, H = (int)B->H, Hk = (int)B->Hk, ffn = (int)B->ffn;
    // attention sublayer
    hipLaunchKernelGGL(blkd_norm, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, h, (const float *)nullptr,
                       (float *)nullptr, B->w_in, B->eps, B->xcat, 3, d);
    QBK_HIP(hipGetLastError());
    if ((rc = q4_set_run(B->qkv, B->xcat, false, B->ycat, false, B->ws, s))) return rc;
    const int nr = (H + Hk) * (hd / 2);
    hipLaunchKernelGGL(blkd_rope_append, dim3((nr + 255) / 256), dim3(256), 0, s, B->ycat, B->rope, pos, B->qrot,
                       B->kc, B->vc, H, Hk, hd);
    QBK_HIP(hipGetLastError());
    const qbk_attn_shape sh{1, B->H, B->Hk, 1, pos + 1, B->hd, B->hd};
    const size_t cached = B->tokens <= pos ? B->tokens : 0;
    if ((rc = qbk_attention_sage_decode_step_dev(ctx, &sh, B->qrot, B->kc, B->vc, B->block, B->attn, B->state,
                                                 B->state_bytes, B->cap, cached, stream)))
        return rc;
    B->tokens = pos + 1;
    if ((rc = q4_run(B->o, 1, B->attn, true, B->oout, false, B->ws, s))) return rc;
    // MLP sublayer: h1 = o + h, then its norm
    hipLaunchKernelGGL(blkd_norm, dim3(1), dim3(BLKD_NORM_THREADS), 0, s, B->oout, (const float *)h, B->h1,
                       B->w_post, B->eps, B->xcat, 2, d);
    QBK_HIP(hipGetLastError());
    if ((rc = q4_set_run(B->gu, B->xcat, false, B->ycat, false, B->ws, s))) return rc;
    hipLaunchKernelGGL(blkd_swiglu, dim3((ffn + 255) / 256), dim3(256), 0, s, B->ycat, B->hid, ffn);
    QBK_HIP(hipGetLastError());
    if ((rc = q4_run(B->down, 1, B->hid, true, B->dout, false, B->ws, s))) return rc;
    hipLaunchKernelGGL(blkd_add, dim3((d + 255) / 256), dim3(256), 0, s, B->dout, B->h1, h, d);
    QBK_HIP(hipGetLastError());
    return QBK_OK;
}

int qbk_block_reset(qbk_block *B) {
    if (!B) return fail(QBK_ERR_VALIDATION, "null block");
    B->tokens = 0;
    return QBK_OK;
}

}  // extern "C"
