/*
 * CPU oracle: Sinkhorn-Knopp forward and its exact adjoint, in double.
 *
 * Test infrastructure only (loaded by tests/ through ctypes as a checker);
 * nothing in the product links or calls it.
 *
 * Forward (ops_pytorch_backward.py:9-33): num_iters times
 *     A = X / (rowsum(X) + eps);   Y = A / (colsum(A) + eps);   X = Y.
 * The reference's backward kernel (sinkhorn_knopp.cpp:1608-1814) stores a
 * per-iteration history and reverses it, but its row step is approximate
 * (1773-1795).  This file writes the exact adjoint from the calculus of the
 * two steps, independently of any autograd, so that tests can pin the
 * PyTorch oracle's autograd backward and the HIP kernel against it:
 *     column step  dA[r][c] = (dY[r][c] - sum_r' dY[r'][c] Y[r'][c]) / cs[c]
 *     row step     dX[r][c] = (dA[r][c] - sum_c' dA[r][c'] A[r][c']) / rs[r]
 * with rs = rowsum + eps and cs = colsum + eps of that iteration.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* One matrix, forward, recording A_t, Y_t, rs_t, cs_t when hist != NULL.
 * hist layout per iteration: A (n*n), Y (n*n), rs (n), cs (n). */
static void sk_one_fwd(const double* in, double* out, int n, int iters, double eps, double* hist)
{
    double* x = (double*)malloc(sizeof(double) * n * n);
    memcpy(x, in, sizeof(double) * n * n);
    const size_t step = (size_t)(2 * n * n + 2 * n);
    for (int t = 0; t < iters; ++t) {
        double* A = hist ? hist + t * step : NULL;
        double* Y = hist ? A + n * n : NULL;
        double* rs = hist ? Y + n * n : NULL;
        double* cs = hist ? rs + n : NULL;
        for (int r = 0; r < n; ++r) {
            double s = 0.0;
            for (int c = 0; c < n; ++c) s += x[r * n + c];
            s += eps;
            if (rs) rs[r] = s;
            for (int c = 0; c < n; ++c) x[r * n + c] /= s;
        }
        if (A) memcpy(A, x, sizeof(double) * n * n);
        for (int c = 0; c < n; ++c) {
            double s = 0.0;
            for (int r = 0; r < n; ++r) s += x[r * n + c];
            s += eps;
            if (cs) cs[c] = s;
            for (int r = 0; r < n; ++r) x[r * n + c] /= s;
        }
        if (Y) memcpy(Y, x, sizeof(double) * n * n);
    }
    memcpy(out, x, sizeof(double) * n * n);
    free(x);
}

int oracle_sinkhorn_fwd(const double* in, double* out, int64_t batch, int n, int iters, double eps)
{
    if (n <= 0 || iters < 0 || batch < 0) return -1;
    for (int64_t b = 0; b < batch; ++b)
        sk_one_fwd(in + b * n * n, out + b * n * n, n, iters, eps, NULL);
    return 0;
}

int oracle_sinkhorn_bwd(const double* grad_out, const double* in, double* grad_in, int64_t batch, int n,
                        int iters, double eps)
{
    if (n <= 0 || iters < 0 || batch < 0) return -1;
    const size_t step = (size_t)(2 * n * n + 2 * n);
    double* hist = (double*)malloc(sizeof(double) * step * (iters > 0 ? iters : 1));
    double* out = (double*)malloc(sizeof(double) * n * n);
    double* dy = (double*)malloc(sizeof(double) * n * n);
    double* da = (double*)malloc(sizeof(double) * n * n);
    for (int64_t b = 0; b < batch; ++b) {
        sk_one_fwd(in + b * n * n, out, n, iters, eps, hist);
        memcpy(dy, grad_out + b * n * n, sizeof(double) * n * n);
        for (int t = iters - 1; t >= 0; --t) {
            const double* A = hist + t * step;
            const double* Y = A + n * n;
            const double* rs = Y + n * n;
            const double* cs = rs + n;
            for (int c = 0; c < n; ++c) {
                double dot = 0.0;
                for (int r = 0; r < n; ++r) dot += dy[r * n + c] * Y[r * n + c];
                for (int r = 0; r < n; ++r) da[r * n + c] = (dy[r * n + c] - dot) / cs[c];
            }
            for (int r = 0; r < n; ++r) {
                double dot = 0.0;
                for (int c = 0; c < n; ++c) dot += da[r * n + c] * A[r * n + c];
                for (int c = 0; c < n; ++c) dy[r * n + c] = (da[r * n + c] - dot) / rs[r];
            }
        }
        memcpy(grad_in + b * n * n, dy, sizeof(double) * n * n);
    }
    free(hist);
    free(out);
    free(dy);
    free(da);
    return 0;
}
