/*
 * Scalar float64 restatement of the reference selective-scan kernels
 * (test infrastructure only: the oracle, never the product).
 *
 * Forward follows csrc/selective_scan/forward_kernel.cu:174-310:
 *   delta' = delta + bias; softplus with the threshold-20 rule (:216-221);
 *   a_t = exp(delta'_t * A_n) (:228,264); b_t = delta'_t * u_t * B_n,t (:265);
 *   h_t = a_t * h_{t-1} + b_t (scan operator common.h:75-81);
 *   y_t = sum_n C_n,t h_t + D * u_t (:223,287-293).
 * z gate (caller side, modules/mamba_simple.py:143-146): out = y * silu(z).
 *
 * Backward follows csrc/selective_scan/backward_kernel.cu:276-585:
 *   g_t = a_{t+1} g_{t+1} + dy_t C_t (reverse scan, :386-431);
 *   du_t = D dy_t + sum_n g B delta' (:334,437-438);
 *   ddelta'_t = sum_n (g B u + g A a_t h_{t-1}) (:439-440);
 *   dA_n += g delta' a_t h_{t-1} (:441); dB += g delta' u (:451);
 *   dC += dy h_t (:454); dD += dy u (:339);
 *   softplus': ddelta = ddelta' * sigmoid(delta + bias) below 20 (:499-517);
 *   dbias += ddelta (:519-521).
 * With a z gate, dy = dout * silu(z) and dz = dout * y * silu'(z).
 *
 * Layouts (all contiguous): u, delta, z, dout, out: (Bt, D, L); A: (D, N);
 * variable B/C: (Bt, G, N, L); constant B/C: (D, N); D, bias: (D).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static double softplus20(double x) { return x <= 20.0 ? log1p(exp(x)) : x; }
static double sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

static double bval(const double* M, int var, int64_t b, int64_t g, int64_t d,
                   int64_t n, int64_t t, int64_t G, int64_t N, int64_t L) {
    if (var) return M[((b * G + g) * N + n) * L + t];
    return M[d * N + n];
}

/* Forward. last_state (Bt, D, N) may be NULL. Returns 0, or -1 on bad shape. */
int ss_oracle_fwd(int64_t Bt, int64_t D, int64_t L, int64_t N, int64_t G,
                  int var_B, int var_C, int softplus,
                  const double* u, const double* delta, const double* A,
                  const double* B, const double* C, const double* Dv,
                  const double* bias, const double* z,
                  double* out, double* last_state) {
    if (G <= 0 || D % G != 0) return -1;
    double* h = (double*)calloc((size_t)(N > 0 ? N : 1), sizeof(double));
    if (!h) return -1;
    const int64_t dpg = D / G;
    for (int64_t b = 0; b < Bt; ++b) {
        for (int64_t d = 0; d < D; ++d) {
            const int64_t g = d / dpg;
            const int64_t row = (b * D + d) * L;
            memset(h, 0, sizeof(double) * (size_t)N);
            for (int64_t t = 0; t < L; ++t) {
                double dt = delta[row + t] + (bias ? bias[d] : 0.0);
                if (softplus) dt = softplus20(dt);
                const double uu = u[row + t];
                double y = Dv ? Dv[d] * uu : 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    const double a = exp(dt * A[d * N + n]);
                    const double bb = dt * uu * bval(B, var_B, b, g, d, n, t, G, N, L);
                    h[n] = a * h[n] + bb;
                    y += bval(C, var_C, b, g, d, n, t, G, N, L) * h[n];
                }
                if (z) {
                    const double zz = z[row + t];
                    y *= zz * sigmoid(zz);
                }
                out[row + t] = y;
            }
            if (last_state)
                for (int64_t n = 0; n < N; ++n) last_state[(b * D + d) * N + n] = h[n];
        }
    }
    free(h);
    return 0;
}

/*
 * Backward. dB/dC have the shape of B/C; dA (D, N); dD, dbias (D); dz like z.
 * dD, dbias, dz may be NULL when D, bias, z are absent. All outputs are
 * overwritten (not accumulated into).
 */
int ss_oracle_bwd(int64_t Bt, int64_t D, int64_t L, int64_t N, int64_t G,
                  int var_B, int var_C, int softplus,
                  const double* u, const double* delta, const double* A,
                  const double* B, const double* C, const double* Dv,
                  const double* bias, const double* z, const double* dout,
                  double* du, double* ddelta, double* dA, double* dB,
                  double* dC, double* dD, double* dbias, double* dz) {
    if (G <= 0 || D % G != 0) return -1;
    const int64_t dpg = D / G;
    const int64_t LN = (L > 0 ? L : 1) * (N > 0 ? N : 1);
    double* hs = (double*)malloc(sizeof(double) * (size_t)LN);   /* h_t,n */
    double* as = (double*)malloc(sizeof(double) * (size_t)LN);   /* a_t,n */
    double* dts = (double*)malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
    double* dys = (double*)malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
    double* gs = (double*)calloc((size_t)(N > 0 ? N : 1), sizeof(double));
    if (!hs || !as || !dts || !dys || !gs) { free(hs); free(as); free(dts); free(dys); free(gs); return -1; }
    memset(dA, 0, sizeof(double) * (size_t)(D * N));
    memset(dB, 0, sizeof(double) * (size_t)(var_B ? Bt * G * N * L : D * N));
    memset(dC, 0, sizeof(double) * (size_t)(var_C ? Bt * G * N * L : D * N));
    if (dD) memset(dD, 0, sizeof(double) * (size_t)D);
    if (dbias) memset(dbias, 0, sizeof(double) * (size_t)D);
    for (int64_t b = 0; b < Bt; ++b) {
        for (int64_t d = 0; d < D; ++d) {
            const int64_t g = d / dpg;
            const int64_t row = (b * D + d) * L;
            /* recompute the forward states and the pre-gate output */
            for (int64_t n = 0; n < N; ++n) gs[n] = 0.0;  /* h_{-1} */
            for (int64_t t = 0; t < L; ++t) {
                double dt = delta[row + t] + (bias ? bias[d] : 0.0);
                if (softplus) dt = softplus20(dt);
                dts[t] = dt;
                const double uu = u[row + t];
                double y = Dv ? Dv[d] * uu : 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    const double a = exp(dt * A[d * N + n]);
                    const double prev = t > 0 ? hs[(t - 1) * N + n] : 0.0;
                    const double hv = a * prev + dt * uu * bval(B, var_B, b, g, d, n, t, G, N, L);
                    as[t * N + n] = a;
                    hs[t * N + n] = hv;
                    y += bval(C, var_C, b, g, d, n, t, G, N, L) * hv;
                }
                double dy = dout[row + t];
                if (z) {
                    const double zz = z[row + t];
                    const double sg = sigmoid(zz);
                    dz[row + t] = dout[row + t] * y * sg * (1.0 + zz * (1.0 - sg));
                    dy = dout[row + t] * zz * sg;
                }
                dys[t] = dy;
            }
            /* reverse adjoint scan */
            for (int64_t n = 0; n < N; ++n) gs[n] = 0.0;
            for (int64_t t = L - 1; t >= 0; --t) {
                const double uu = u[row + t];
                const double dt = dts[t];
                const double dy = dys[t];
                double s_du = Dv ? Dv[d] * dy : 0.0;
                double s_ddt = 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    const double a_next = t + 1 < L ? as[(t + 1) * N + n] : 1.0;
                    const double Bn = bval(B, var_B, b, g, d, n, t, G, N, L);
                    const double Cn = bval(C, var_C, b, g, d, n, t, G, N, L);
                    gs[n] = a_next * gs[n] + dy * Cn;
                    const double gv = gs[n];
                    const double prev = t > 0 ? hs[(t - 1) * N + n] : 0.0;
                    const double ah = as[t * N + n] * prev;
                    s_du += gv * Bn * dt;
                    s_ddt += gv * Bn * uu + gv * A[d * N + n] * ah;
                    dA[d * N + n] += gv * dt * ah;
                    if (var_B) dB[((b * G + g) * N + n) * L + t] += gv * dt * uu;
                    else dB[d * N + n] += gv * dt * uu;
                    if (var_C) dC[((b * G + g) * N + n) * L + t] += dy * hs[t * N + n];
                    else dC[d * N + n] += dy * hs[t * N + n];
                }
                double pre = delta[row + t] + (bias ? bias[d] : 0.0);
                double dd = s_ddt;
                if (softplus && pre <= 20.0) dd = s_ddt * sigmoid(pre);
                du[row + t] = s_du;
                ddelta[row + t] = dd;
                if (dD) dD[d] += dy * uu;
                if (dbias) dbias[d] += dd;
            }
        }
    }
    free(hs); free(as); free(dts); free(dys); free(gs);
    return 0;
}
