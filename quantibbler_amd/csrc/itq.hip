// itq.hip -- joint_itq (core.rs:318-424), the compressor's alternating
// Procrustes over Z = [u_hat; v_hat] ([LB2] 4.4, Algorithm 1 lines 6-11).
// Host code: the reference runs it on the CPU too (the PyO3 face's
// joint_itq over core.rs; off the kernels' hot path).
//
//   R0 = modified Gram-Schmidt of a splitmix64 matrix (core.rs:47-95);
//   loop: B = sign(Z R); B^T Z = Phi Sigma Psi^T; R = Psi Phi^T;
//   stop when ||R_new - R||_F <= tol (tol > 0) or after max_iter.
//
// Every product and norm accumulates left to right in f64 element order, as
// core.rs's matmul_lr / matmul_at_b_lr / Gram-Schmidt do.  The SVD is this
// file's own one-sided Jacobi (Hestenes) on B^T Z, not nalgebra's: R = Psi
// Phi^T is the orthogonal polar factor of (B^T Z)^T, unique when the
// singular values are distinct, so it does not depend on which SVD computes
// it beyond the last bits -- and the iterates are the sign matrices B, which
// those bits do not move unless an entry of Z R sits at zero.  Once B
// repeats, R repeats bit for bit and the loop stops with a zero delta, so
// n_iter follows B's sequence as the reference's does.
#include <math.h>
#include <string.h>

#include <vector>

#include "qbk_internal.h"

namespace qbk {

static uint64_t itq_splitmix64(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

typedef std::vector<double> Mat;  // row-major

// Hestenes one-sided Jacobi on the r x r matrix M: W = M V with orthogonal
// columns, V orthogonal; then Phi[:, k] = W[:, k] / ||W[:, k]|| (completed to
// an orthonormal basis where a column vanished) and Psi = V, so that
// M = Phi Sigma Psi^T.
static void itq_svd(const Mat &M, size_t r, Mat &phi, Mat &psi) {
    Mat W = M;
    psi.assign(r * r, 0.0);
    for (size_t i = 0; i < r; i++) psi[i * r + i] = 1.0;
    for (int sweep = 0; sweep < 60; sweep++) {
        double off = 0.0;
        for (size_t p = 0; p + 1 < r; p++)
            for (size_t q = p + 1; q < r; q++) {
                double a = 0.0, b = 0.0, g = 0.0;
                for (size_t i = 0; i < r; i++) {
                    const double wp = W[i * r + p], wq = W[i * r + q];
                    a += wp * wp;
                    b += wq * wq;
                    g += wp * wq;
                }
                if (g == 0.0 || fabs(g) <= 1e-16 * sqrt(a * b)) continue;
                off = fmax(off, fabs(g) / sqrt(a * b));
                const double zeta = (b - a) / (2.0 * g);
                const double t = (zeta >= 0.0 ? 1.0 : -1.0) / (fabs(zeta) + sqrt(1.0 + zeta * zeta));
                const double c = 1.0 / sqrt(1.0 + t * t), s = c * t;
                for (size_t i = 0; i < r; i++) {
                    const double wp = W[i * r + p], wq = W[i * r + q];
                    W[i * r + p] = c * wp - s * wq;
                    W[i * r + q] = s * wp + c * wq;
                    const double vp = psi[i * r + p], vq = psi[i * r + q];
                    psi[i * r + p] = c * vp - s * vq;
                    psi[i * r + q] = s * vp + c * vq;
                }
            }
        if (off <= 1e-15) break;
    }
    phi.assign(r * r, 0.0);
    std::vector<bool> done(r, false);
    for (size_t k = 0; k < r; k++) {
        double n2 = 0.0;
        for (size_t i = 0; i < r; i++) n2 += W[i * r + k] * W[i * r + k];
        const double n = sqrt(n2);
        if (n > 0.0) {
            for (size_t i = 0; i < r; i++) phi[i * r + k] = W[i * r + k] / n;
            done[k] = true;
        }
    }
    // complete vanished columns from the unit vectors, orthogonal to the rest
    size_t e = 0;
    for (size_t k = 0; k < r; k++) {
        if (done[k]) continue;
        for (; e < r; e++) {
            std::vector<double> v(r, 0.0);
            v[e] = 1.0;
            for (size_t j = 0; j < r; j++) {
                if (!done[j]) continue;
                double dot = 0.0;
                for (size_t i = 0; i < r; i++) dot += phi[i * r + j] * v[i];
                for (size_t i = 0; i < r; i++) v[i] -= dot * phi[i * r + j];
            }
            double n2 = 0.0;
            for (size_t i = 0; i < r; i++) n2 += v[i] * v[i];
            if (n2 > 1e-6) {
                const double n = sqrt(n2);
                for (size_t i = 0; i < r; i++) phi[i * r + k] = v[i] / n;
                done[k] = true;
                e++;
                break;
            }
        }
    }
}

}  // namespace qbk

using namespace qbk;

extern "C" {

int qbk_joint_itq(const double *u_hat, size_t u_len, const double *v_hat, size_t v_len, size_t dout, size_t din,
                  size_t rank, size_t max_iter, double tol, uint64_t seed, int8_t *u_t, int8_t *v_t,
                  size_t *n_iter_out, int *converged_out) {
    if (rank == 0 || dout + din == 0) return fail(QBK_ERR_VALIDATION, "joint_itq expects non-empty factors");
    if (u_len != dout * rank || v_len != din * rank)
        return fail(QBK_ERR_VALIDATION, fmt("joint_itq shape mismatch: u_hat %zux%zu, v_hat %zux%zu", dout,
                                            u_len / (dout ? dout : 1), din, rank));
    const size_t r = rank, nz = dout + din;
    Mat Z(nz * r);
    if (dout) memcpy(Z.data(), u_hat, dout * r * sizeof(double));
    if (din) memcpy(Z.data() + dout * r, v_hat, din * r * sizeof(double));
    // R0: splitmix64 fill in [-1, 1), then modified Gram-Schmidt by columns
    Mat R(r * r);
    uint64_t st = seed;
    for (size_t i = 0; i < r * r; i++) {
        const uint64_t z = itq_splitmix64(&st);
        R[i] = (double)(z >> 11) / 9007199254740992.0 * 2.0 - 1.0;
    }
    for (size_t j = 0; j < r; j++) {
        std::vector<double> v(r);
        for (size_t i = 0; i < r; i++) v[i] = R[i * r + j];
        for (size_t k = 0; k < j; k++) {
            double d = 0.0;
            for (size_t i = 0; i < r; i++) d += R[i * r + k] * v[i];
            for (size_t i = 0; i < r; i++) v[i] -= d * R[i * r + k];
        }
        double s = 0.0;
        for (size_t i = 0; i < r; i++) s += v[i] * v[i];
        const double nrm = sqrt(s);
        if (nrm == 0.0) return fail(QBK_ERR_VALIDATION, "joint_itq produced a degenerate zero column building R0");
        for (size_t i = 0; i < r; i++) R[i * r + j] = v[i] / nrm;
    }
    auto sign_zr = [&](Mat &B) {  // B = sign(Z R), >= 0 -> +1
        B.assign(nz * r, 0.0);
        for (size_t i = 0; i < nz; i++)
            for (size_t j = 0; j < r; j++) {
                double acc = 0.0;
                for (size_t t = 0; t < r; t++) acc += Z[i * r + t] * R[t * r + j];
                B[i * r + j] = acc >= 0.0 ? 1.0 : -1.0;
            }
    };
    size_t n_iter = 0;
    int converged = 0;
    Mat B, M(r * r), phi, psi, Rn(r * r);
    for (size_t it = 1; it <= max_iter; it++) {
        sign_zr(B);
        for (size_t i = 0; i < r; i++)  // B^T Z
            for (size_t j = 0; j < r; j++) {
                double acc = 0.0;
                for (size_t t = 0; t < nz; t++) acc += B[t * r + i] * Z[t * r + j];
                M[i * r + j] = acc;
            }
        itq_svd(M, r, phi, psi);
        double dsq = 0.0;
        for (size_t i = 0; i < r; i++)  // R_new = Psi Phi^T
            for (size_t j = 0; j < r; j++) {
                double acc = 0.0;
                for (size_t t = 0; t < r; t++) acc += psi[i * r + t] * phi[j * r + t];
                Rn[i * r + j] = acc;
            }
        for (size_t i = 0; i < r * r; i++) {
            const double d = Rn[i] - R[i];
            dsq += d * d;
        }
        R.swap(Rn);
        n_iter = it;
        if (tol > 0.0 && sqrt(dsq) <= tol) {
            converged = 1;
            break;
        }
    }
    sign_zr(B);
    for (size_t i = 0; i < nz; i++)
        for (size_t j = 0; j < r; j++) {
            const int8_t sgn = B[i * r + j] > 0.0 ? 1 : -1;
            if (i < dout)
                u_t[i * r + j] = sgn;
            else
                v_t[(i - dout) * r + j] = sgn;
        }
    if (n_iter_out) *n_iter_out = n_iter;
    if (converged_out) *converged_out = converged;
    return QBK_OK;
}

}  // extern "C"
