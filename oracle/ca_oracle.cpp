// ca_oracle.cpp — TEST INFRASTRUCTURE: a straight double-precision CPU
// restatement of Slime's multi-head neural-CA step (stages S1-S7) and its
// fitness (E1-E5). It exists to check the HIP library and to be timed as the
// CPU baseline; the product library never links or calls it.
//
// Reference sources each function follows (paths under the J0pari/Slime tree):
//   S1 projections   slime/core/pseudopod.cu:29-32 (per-head weight tensors),
//                    :94 (ReLU), :106-108 (tanh GELU); buildplan.md:572-591
//                    (P, I, V all from the neighbourhood input); the chained
//                    forms of :98-119, with the 3x3 neighbourhood sum of :62-91
//                    before the perception product in chain mode 2
//   S2 potential     slime/core/pseudopod.cu:168-180 (per-head 3x3 flow kernel),
//                    toroidal wrap as slime/kernels/warp_ca.cu:305-310 and
//                    slime/kernels/triton_impl.cu:90-105
//   S3 growth        failed_attempts/warp_ca.cu:49-56; variants: the Gaussian of
//                    failed_attempts/pseudopod.cu:46-48 and the shipped U exp(-U^2)
//                    of slime/core/pseudopod.cu:183
//   S4 activation    failed_attempts/pseudopod.cu:208-251 (query = centre
//                    perception, key = neighbour interaction, /sqrt(dim),
//                    max-subtracted softmax)
//   S5 propagation   failed_attempts/pseudopod.cu:295-311
//   S6 update + mix  slime/core/pseudopod.cu:186-187 (X + dt*update),
//                    slime/core/organism.cu:659 (dt = 0.1),
//                    failed_attempts/pseudopod.cu:330 (dt*(growth*value)),
//                    slime/core/pseudopod.cu:231-251 (head mixing M[o][h])
//   S7 conservation  failed_attempts/warp_ca.cu:401-450 (global sum rescale),
//                    slime/core/pseudopod.cu:21,198 (|mass| > 1e-6 guard); variant:
//                    the shipped per-cell, per-head renormalisation of
//                    slime/core/pseudopod.cu:160-165,196-203
//   E1 Gram          failed_attempts/pseudopod.cu:366-384 (d x d correlation
//                    over all cells; here per head, not averaged over heads)
//   E2 Jacobi        failed_attempts/pseudopod.cu:391-436 (cyclic two-sided
//                    Jacobi, skip |a_pq| <= tol, stop when sum|a_pq| < tol*n)
//   E3 eff. rank     slime/kernels/warp_ca.cu:118-143 (EPSILON 1e-7 at :21)
//   E4 coherence     lag-1 Pearson correlation mapped (rho+1)/2 as
//                    slime/core/organism.cu:256-257
//   E5 fitness       slime/kernels/warp_ca.cu:219
//   field adapters   slime/core/organism.cu:691-720 and :723-743
//   backward         no reference source: the reference declares gradients
//                    (slime/proto/model.cu:7,13) but never computes them. The
//                    step's chain rule is written out below, stage by stage,
//                    and pinned by finite differences of this file's forward.
#include "ca_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

struct Dims {
    int B, G, H, D, C, pods, per_pod;
    long cells;  // G*G
};

bool dims_of(const oracle_ca_cfg* cfg, Dims* d) {
    if (!cfg || cfg->B <= 0 || cfg->G <= 0 || cfg->H <= 0 || cfg->D <= 0 || cfg->pods <= 0)
        return false;
    if (cfg->growth_fn < 0 || cfg->growth_fn > 2 || cfg->conservation < 0 || cfg->conservation > 1)
        return false;
    if (cfg->B % cfg->pods != 0) return false;
    d->B = cfg->B;
    d->G = cfg->G;
    d->H = cfg->H;
    d->D = cfg->D;
    d->C = cfg->H * cfg->D;
    d->pods = cfg->pods;
    d->per_pod = cfg->B / cfg->pods;
    d->cells = (long)cfg->G * cfg->G;
    return true;
}

inline int wrap(int v, int G) { return v < 0 ? v + G : (v >= G ? v - G : v); }

inline double gelu_tanh(double x) {
    return 0.5 * x * (1.0 + std::tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
}

// out[b][cell][n] = act(sum_k in[b][cell][k] * W[pod][k][n]), with C x C weights.
// act: 0 none, 1 ReLU, 2 tanh-GELU.
void project(const Dims& d, const double* in, const float* W, int act, double* out) {
    const int C = d.C;
    const long rows = (long)d.B * d.cells;
    std::vector<double> Wd((size_t)d.pods * C * C);
    for (size_t i = 0; i < Wd.size(); ++i) Wd[i] = W[i];
    const int RB = 16;
#pragma omp parallel for schedule(static)
    for (long r0 = 0; r0 < rows; r0 += RB) {
        const int nr = (int)std::min<long>(RB, rows - r0);
        std::vector<double> acc((size_t)RB * C, 0.0);
        for (int k = 0; k < C; ++k) {
            for (int i = 0; i < nr; ++i) {
                const long r = r0 + i;
                const int pod = (int)(r / d.cells) / d.per_pod;
                const double* wrow = Wd.data() + ((size_t)pod * C + k) * C;
                const double xk = in[(size_t)r * C + k];
                double* a = acc.data() + (size_t)i * C;
                for (int n = 0; n < C; ++n) a[n] += xk * wrow[n];
            }
        }
        for (int i = 0; i < nr; ++i) {
            double* o = out + (size_t)(r0 + i) * C;
            const double* a = acc.data() + (size_t)i * C;
            for (int n = 0; n < C; ++n) {
                double v = a[n];
                if (act == 1) v = v > 0.0 ? v : 0.0;
                else if (act == 2) v = gelu_tanh(v);
                o[n] = v;
            }
        }
    }
}

// The perception input of multi_head_ca_kernel (slime/core/pseudopod.cu:62-91): each
// channel summed over the 3x3 neighbourhood before the product, the border wrapped
// (toroidal, as S2) where the reference clamps. Taps in the order k = 3(dy+1)+(dx+1).
void neighbourhood_sum(const Dims& d, const double* X, double* S) {
    const int G = d.G, C = d.C;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < d.B; ++b)
        for (int y = 0; y < G; ++y)
            for (int x = 0; x < G; ++x) {
                double* s = S + (((size_t)b * G + y) * G + x) * C;
                for (int ch = 0; ch < C; ++ch) s[ch] = 0.0;
                for (int dy = -1; dy <= 1; ++dy)
                    for (int dx = -1; dx <= 1; ++dx) {
                        const double* xn =
                            X + (((size_t)b * G + wrap(y + dy, G)) * G + wrap(x + dx, G)) * C;
                        for (int ch = 0; ch < C; ++ch) s[ch] += xn[ch];
                    }
            }
}

// chain: 0 P, I, V all from X; 1 I from P, V from I; 2 as 1 with P from the
// neighbourhood sum of X.
void project_all(const Dims& d, int chain, const double* X, const float* WP, const float* WI,
                 const float* WV, double* P, double* I, double* V) {
    if (chain == 2) {
        std::vector<double> S((size_t)d.B * d.cells * d.C);
        neighbourhood_sum(d, X, S.data());
        project(d, S.data(), WP, 1, P);
    } else {
        project(d, X, WP, 1, P);
    }
    project(d, chain ? P : X, WI, 2, I);
    project(d, chain ? I : X, WV, 0, V);
}

void potential(const Dims& d, const double* X, const float* K, double* U) {
    const int G = d.G, C = d.C, D = d.D;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < d.B; ++b)
        for (int y = 0; y < G; ++y) {
            const int pod = b / d.per_pod;
            for (int x = 0; x < G; ++x) {
                double* u = U + (((size_t)b * G + y) * G + x) * C;
                for (int ch = 0; ch < C; ++ch) u[ch] = 0.0;
                for (int dy = -1; dy <= 1; ++dy)
                    for (int dx = -1; dx <= 1; ++dx) {
                        const int k = 3 * (dy + 1) + (dx + 1);
                        const double* xn =
                            X + (((size_t)b * G + wrap(y + dy, G)) * G + wrap(x + dx, G)) * C;
                        for (int h = 0; h < d.H; ++h) {
                            const double w = K[((size_t)pod * d.H + h) * 9 + k];
                            for (int c = 0; c < D; ++c) u[h * D + c] += w * xn[h * D + c];
                        }
                    }
            }
        }
}

// fn 0: the bell 2 exp(-((U - mu) / (sigma + 1e-7))^2) - 1 (failed_attempts/warp_ca.cu:49-56);
// fn 1: the Gaussian exp(-(U - mu)^2 / (2 sigma^2)) (failed_attempts/pseudopod.cu:46-48);
// fn 2: the shipped kernel's U exp(-U^2), no mu or sigma (slime/core/pseudopod.cu:183).
double growth_of(int fn, double u, double m, double s) {
    if (fn == 1) return std::exp(-(u - m) * (u - m) / (2.0 * s * s));
    if (fn == 2) return u * std::exp(-u * u);
    const double z = (u - m) / (s + 1e-7);
    return 2.0 * std::exp(-z * z) - 1.0;
}

void growth(const Dims& d, int per_cell, int fn, const double* U, const float* mu, const float* sigma,
            double* g) {
    const int C = d.C, D = d.D;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)d.B * d.cells; ++r) {
        const int b = (int)(r / d.cells);
        const long cell = r % d.cells;
        const int pod = b / d.per_pod;
        for (int h = 0; h < d.H; ++h) {
            const size_t pi = per_cell ? ((size_t)pod * d.cells + cell) * d.H + h
                                       : (size_t)pod * d.H + h;
            const double m = mu[pi], s = sigma[pi];
            for (int c = 0; c < D; ++c)
                g[(size_t)r * C + h * D + c] = growth_of(fn, U[(size_t)r * C + h * D + c], m, s);
        }
    }
}

void attention(const Dims& d, const double* P, const double* I, double* A) {
    const int G = d.G, C = d.C, D = d.D, H = d.H;
    const double inv_sqrt_d = 1.0 / std::sqrt((double)D);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < d.B; ++b)
        for (int y = 0; y < G; ++y)
            for (int x = 0; x < G; ++x) {
                const size_t r = ((size_t)b * G + y) * G + x;
                for (int h = 0; h < H; ++h) {
                    double s[9];
                    for (int dy = -1; dy <= 1; ++dy)
                        for (int dx = -1; dx <= 1; ++dx) {
                            const int k = 3 * (dy + 1) + (dx + 1);
                            const double* in =
                                I + (((size_t)b * G + wrap(y + dy, G)) * G + wrap(x + dx, G)) * C +
                                h * D;
                            const double* pc = P + r * C + h * D;
                            double acc = 0.0;
                            for (int c = 0; c < D; ++c) acc += pc[c] * in[c];
                            s[k] = acc * inv_sqrt_d;
                        }
                    double mx = s[0];
                    for (int k = 1; k < 9; ++k) mx = std::max(mx, s[k]);
                    double sum = 0.0;
                    for (int k = 0; k < 9; ++k) {
                        s[k] = std::exp(s[k] - mx);
                        sum += s[k];
                    }
                    double* a = A + (r * H + h) * 9;
                    for (int k = 0; k < 9; ++k) a[k] = s[k] / sum;
                }
            }
}

void propagate(const Dims& d, const double* A, const double* V, double* Vt) {
    const int G = d.G, C = d.C, D = d.D, H = d.H;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < d.B; ++b)
        for (int y = 0; y < G; ++y)
            for (int x = 0; x < G; ++x) {
                const size_t r = ((size_t)b * G + y) * G + x;
                double* o = Vt + r * C;
                for (int ch = 0; ch < C; ++ch) o[ch] = 0.0;
                for (int dy = -1; dy <= 1; ++dy)
                    for (int dx = -1; dx <= 1; ++dx) {
                        const int k = 3 * (dy + 1) + (dx + 1);
                        const double* vn =
                            V + (((size_t)b * G + wrap(y + dy, G)) * G + wrap(x + dx, G)) * C;
                        for (int h = 0; h < H; ++h) {
                            const double a = A[(r * H + h) * 9 + k];
                            for (int c = 0; c < D; ++c) o[h * D + c] += a * vn[h * D + c];
                        }
                    }
            }
}

void mix(const Dims& d, double dt, const double* X, const double* g, const double* Vt,
         const float* M, double* Y) {
    const int C = d.C, D = d.D, H = d.H;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)d.B * d.cells; ++r) {
        const int pod = (int)(r / d.cells) / d.per_pod;
        std::vector<double> z(C);
        for (int ch = 0; ch < C; ++ch) {
            const size_t i = (size_t)r * C + ch;
            z[ch] = X[i] + dt * g[i] * Vt[i];
        }
        for (int o = 0; o < H; ++o)
            for (int c = 0; c < D; ++c) {
                double acc = 0.0;
                for (int h = 0; h < H; ++h)
                    acc += (double)M[((size_t)pod * H + o) * H + h] * z[h * D + c];
                Y[(size_t)r * C + o * D + c] = acc;
            }
    }
}

// Per (cell, head o), the shipped kernel's renormalisation (slime/core/pseudopod.cu:
// 160-165, 196-203): Y_o(cell) *= sum_c X_o(cell) / sum_c Y_o(cell) unless the
// latter is at most 1e-6 in magnitude. Applied to the mixed output, so that each
// cell's head sums equal its input's.
void conserve_cells(const Dims& d, const double* X, double* Y) {
    const int C = d.C, D = d.D, H = d.H;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)d.B * d.cells; ++r)
        for (int o = 0; o < H; ++o) {
            const size_t base = (size_t)r * C + o * D;
            double sx = 0.0, sy = 0.0;
            for (int c = 0; c < D; ++c) {
                sx += X[base + c];
                sy += Y[base + c];
            }
            if (std::fabs(sy) > 1e-6)
                for (int c = 0; c < D; ++c) Y[base + c] *= sx / sy;
        }
}

// Per (b, head o): Y_o *= sum(X_o) / sum(Y_o) unless |sum(Y_o)| <= 1e-6. With
// per_cell set, the per-cell renormalisation runs first (the global factor is then
// 1 up to rounding, unless a cell's sum took the guard).
void conserve(const Dims& d, int per_cell, const double* X, double* Y, double* mass_in,
              double* mass_out) {
    const int C = d.C, D = d.D, H = d.H;
    if (per_cell) conserve_cells(d, X, Y);
    for (int b = 0; b < d.B; ++b)
        for (int o = 0; o < H; ++o) {
            double sx = 0.0, sy = 0.0;
            for (long cell = 0; cell < d.cells; ++cell) {
                const size_t base = ((size_t)b * d.cells + cell) * C + o * D;
                for (int c = 0; c < D; ++c) {
                    sx += X[base + c];
                    sy += Y[base + c];
                }
            }
            const double scale = std::fabs(sy) > 1e-6 ? sx / sy : 1.0;
            double so = 0.0;
            for (long cell = 0; cell < d.cells; ++cell) {
                const size_t base = ((size_t)b * d.cells + cell) * C + o * D;
                for (int c = 0; c < D; ++c) {
                    Y[base + c] *= scale;
                    so += Y[base + c];
                }
            }
            if (mass_in) mass_in[b * H + o] = sx;
            if (mass_out) mass_out[b * H + o] = so;
        }
}

std::vector<double> to_d(const float* p, size_t n) {
    std::vector<double> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = p[i];
    return v;
}
void to_f(const std::vector<double>& v, float* p) {
    for (size_t i = 0; i < v.size(); ++i) p[i] = (float)v[i];
}

}  // namespace

extern "C" {

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

int oracle_project(const oracle_ca_cfg* cfg, const float* X, const float* WP, const float* WI,
                   const float* WV, float* P, float* I, float* V) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> xd = to_d(X, n), p(n), i(n), v(n);
    project_all(d, cfg->pvi_chain, xd.data(), WP, WI, WV, p.data(), i.data(), v.data());
    to_f(p, P);
    to_f(i, I);
    to_f(v, V);
    return 0;
}

int oracle_potential(const oracle_ca_cfg* cfg, const float* X, const float* K, float* U) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> xd = to_d(X, n), u(n);
    potential(d, xd.data(), K, u.data());
    to_f(u, U);
    return 0;
}

int oracle_growth(const oracle_ca_cfg* cfg, const float* U, const float* mu, const float* sigma,
                  float* g) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> ud = to_d(U, n), gd(n);
    growth(d, cfg->growth_per_cell, cfg->growth_fn, ud.data(), mu, sigma, gd.data());
    to_f(gd, g);
    return 0;
}

int oracle_attention(const oracle_ca_cfg* cfg, const float* P, const float* I, float* A) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> pd = to_d(P, n), id = to_d(I, n), ad((size_t)d.B * d.cells * d.H * 9);
    attention(d, pd.data(), id.data(), ad.data());
    to_f(ad, A);
    return 0;
}

int oracle_propagate(const oracle_ca_cfg* cfg, const float* A, const float* V, float* Vt) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> ad = to_d(A, (size_t)d.B * d.cells * d.H * 9), vd = to_d(V, n), o(n);
    propagate(d, ad.data(), vd.data(), o.data());
    to_f(o, Vt);
    return 0;
}

int oracle_mix(const oracle_ca_cfg* cfg, const float* X, const float* g, const float* Vt,
               const float* M, float* Y) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> xd = to_d(X, n), gd = to_d(g, n), vd = to_d(Vt, n), y(n);
    mix(d, cfg->dt, xd.data(), gd.data(), vd.data(), M, y.data());
    to_f(y, Y);
    return 0;
}

int oracle_conserve(const oracle_ca_cfg* cfg, const float* X, float* Y, double* mass_in,
                    double* mass_out) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> xd = to_d(X, n), yd = to_d(Y, n);
    conserve(d, cfg->conservation, xd.data(), yd.data(), mass_in, mass_out);
    to_f(yd, Y);
    return 0;
}

int oracle_step(const oracle_ca_cfg* cfg, const float* X_in, const float* WP, const float* WI,
                const float* WV, const float* K, const float* mu, const float* sigma,
                const float* M, float* X_out, int n_steps, double* mass_in, double* mass_out) {
    Dims d;
    if (!dims_of(cfg, &d) || n_steps < 0) return -1;
    const size_t n = (size_t)d.B * d.cells * d.C;
    std::vector<double> x = to_d(X_in, n), P(n), I(n), V(n), U(n), g(n), Vt(n), Y(n);
    std::vector<double> A((size_t)d.B * d.cells * d.H * 9);
    for (int s = 0; s < n_steps; ++s) {
        project_all(d, cfg->pvi_chain, x.data(), WP, WI, WV, P.data(), I.data(), V.data());
        potential(d, x.data(), K, U.data());
        growth(d, cfg->growth_per_cell, cfg->growth_fn, U.data(), mu, sigma, g.data());
        attention(d, P.data(), I.data(), A.data());
        propagate(d, A.data(), V.data(), Vt.data());
        mix(d, cfg->dt, x.data(), g.data(), Vt.data(), M, Y.data());
        conserve(d, cfg->conservation, x.data(), Y.data(), mass_in, mass_out);
        // The state is carried between steps in fp32, as the fp32 device path does.
        for (size_t i = 0; i < n; ++i) x[i] = (double)(float)Y[i];
    }
    to_f(x, X_out);
    return 0;
}

int oracle_gram(const oracle_ca_cfg* cfg, const float* X, double* A) {
    Dims d;
    if (!dims_of(cfg, &d)) return -1;
    const int D = d.D, C = d.C;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < d.B; ++b)
        for (int h = 0; h < d.H; ++h) {
            std::vector<double> acc((size_t)D * D, 0.0);
            for (long cell = 0; cell < d.cells; ++cell) {
                const float* v = X + ((size_t)b * d.cells + cell) * C + h * D;
                for (int i = 0; i < D; ++i) {
                    const double vi = v[i];
                    for (int j = 0; j < D; ++j) acc[(size_t)i * D + j] += vi * (double)v[j];
                }
            }
            double* out = A + ((size_t)b * d.H + h) * D * D;
            for (int i = 0; i < D * D; ++i) out[i] = acc[i] / (double)d.cells;
        }
    return 0;
}

int oracle_jacobi_eigs(const double* Ain, int n, double* eig_desc, int max_sweeps, double tol) {
    if (n <= 0) return -1;
    std::vector<double> A(Ain, Ain + (size_t)n * n);
    int sweeps = 0;
    for (int sweep = 0; sweep < max_sweeps; ++sweep) {
        ++sweeps;
        double off = 0.0;
        for (int p = 0; p < n - 1; ++p)
            for (int q = p + 1; q < n; ++q) {
                const double app = A[(size_t)p * n + p], aqq = A[(size_t)q * n + q];
                const double apq = A[(size_t)p * n + q];
                if (std::fabs(apq) > tol) {
                    const double tau = (aqq - app) / (2.0 * apq);
                    const double t = tau >= 0.0 ? 1.0 / (tau + std::sqrt(1.0 + tau * tau))
                                                : -1.0 / (-tau + std::sqrt(1.0 + tau * tau));
                    const double c = 1.0 / std::sqrt(1.0 + t * t), s = t * c;
                    for (int i = 0; i < n; ++i) {
                        const double aip = A[(size_t)i * n + p], aiq = A[(size_t)i * n + q];
                        A[(size_t)i * n + p] = c * aip - s * aiq;
                        A[(size_t)i * n + q] = s * aip + c * aiq;
                    }
                    for (int j = 0; j < n; ++j) {
                        const double apj = A[(size_t)p * n + j], aqj = A[(size_t)q * n + j];
                        A[(size_t)p * n + j] = c * apj - s * aqj;
                        A[(size_t)q * n + j] = s * apj + c * aqj;
                    }
                    A[(size_t)p * n + p] = c * c * app + s * s * aqq - 2.0 * c * s * apq;
                    A[(size_t)q * n + q] = s * s * app + c * c * aqq + 2.0 * c * s * apq;
                    A[(size_t)p * n + q] = 0.0;
                    A[(size_t)q * n + p] = 0.0;
                }
                off += std::fabs(apq);
            }
        if (off < tol * n) break;
    }
    for (int i = 0; i < n; ++i) eig_desc[i] = A[(size_t)i * n + i];
    std::sort(eig_desc, eig_desc + n, [](double a, double b) { return a > b; });
    return sweeps;
}

double oracle_effective_rank(const double* sv, int n) {
    double sum = 0.0;
    for (int i = 0; i < n; ++i) sum += sv[i];
    double ent = 0.0;
    for (int i = 0; i < n; ++i) {
        const double p = sv[i] / (sum + 1e-7);
        ent += -p * std::log(p + 1e-7);
    }
    return std::exp(ent);
}

int oracle_coherence(const oracle_ca_cfg* cfg, const float* hist, int T, double* coh) {
    Dims d;
    if (!dims_of(cfg, &d) || T < 2) return -1;
    const int D = d.D, C = d.C;
    const size_t state = (size_t)d.B * d.cells * C;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < d.B; ++b)
        for (int h = 0; h < d.H; ++h) {
            double rho_sum = 0.0;
            const double n = (double)d.cells * D;
            for (int t = 1; t < T; ++t) {
                const float* xa = hist + (size_t)(t - 1) * state + (size_t)b * d.cells * C + h * D;
                const float* xb = hist + (size_t)t * state + (size_t)b * d.cells * C + h * D;
                double ma = 0.0, mb = 0.0;
                for (long cell = 0; cell < d.cells; ++cell)
                    for (int c = 0; c < D; ++c) {
                        ma += xa[(size_t)cell * C + c];
                        mb += xb[(size_t)cell * C + c];
                    }
                ma /= n;
                mb /= n;
                double cov = 0.0, va = 0.0, vb = 0.0;
                for (long cell = 0; cell < d.cells; ++cell)
                    for (int c = 0; c < D; ++c) {
                        const double ea = xa[(size_t)cell * C + c] - ma;
                        const double eb = xb[(size_t)cell * C + c] - mb;
                        cov += ea * eb;
                        va += ea * ea;
                        vb += eb * eb;
                    }
                const double den = std::sqrt(va * vb);
                rho_sum += den > 0.0 ? cov / den : 0.0;
            }
            coh[b * d.H + h] = (rho_sum / (T - 1) + 1.0) * 0.5;
        }
    return 0;
}

int oracle_fitness(const oracle_ca_cfg* cfg, const float* hist, int T, double* erank,
                   double* coh, double* fitness) {
    Dims d;
    if (!dims_of(cfg, &d) || T < 2) return -1;
    const int D = d.D;
    const size_t state = (size_t)d.B * d.cells * d.C;
    std::vector<double> gram((size_t)d.B * d.H * D * D);
    oracle_gram(cfg, hist + (size_t)(T - 1) * state, gram.data());
    oracle_coherence(cfg, hist, T, coh);
    std::vector<double> eig(D), sv(D);
    for (int bh = 0; bh < d.B * d.H; ++bh) {
        oracle_jacobi_eigs(gram.data() + (size_t)bh * D * D, D, eig.data(), 30, 1e-6);
        for (int i = 0; i < D; ++i) sv[i] = std::sqrt(std::fabs(eig[i]));
        std::sort(sv.begin(), sv.end(), [](double a, double b) { return a > b; });
        erank[bh] = oracle_effective_rank(sv.data(), D);
        fitness[bh] = erank[bh] * coh[bh];
    }
    return 0;
}

// ---- one step with the MSE loss, and its gradient ---------------------------------------
// L = mean over all elements of (Y' - T)^2, Y' the conserved output of one step
// (parallel P/I/V projections). With gradient pointers NULL only the loss is
// computed. Chain rule, per (batch b, cell r, head h, channel c), k over the 9
// neighbours n_k(r) (all sums below also run over channels where indexed by c):
//   S7  r_o = A_o/B_o (A_o = sum X_o, B_o = sum Y_o; 1 when |B_o| <= 1e-6)
//       gY' = 2 (Y' - T)/N,  Q_o = sum gY' Y_o,  gY_o = r_o (gY' - Q_o/B_o),
//       gX_o += Q_o/B_o                       (both only when the guard passes)
//   S6  gZ_h = sum_o M[o][h] gY_o,  gM[o][h] += sum gY_o Z_h,  gX += gZ,
//       gg = dt gZ Vt,  gVt = dt gZ g
//   S3  t = (U - mu)/(sigma + 1e-7): gU = gg (-4 t e^{-t^2})/(sigma + 1e-7),
//       gmu += -gU,  gsigma += -gU t
//   S2  gX(n_k(r)) += K[h][k] gU(r),  gK[h][k] += sum gU(r) X(n_k(r))
//   S5  gV(n_k(r)) += a_k gVt(r),  ga_k = <gVt(r), V(n_k(r))>
//   S4  gs_k = a_k (ga_k - sum_j a_j ga_j),  gP(r) += sum_k gs_k I(n_k)/sqrt(D),
//       gI(n_k(r)) += gs_k P(r)/sqrt(D)
//   S1  gP~ = gP [P~ > 0],  gI~ = gI GELU'(I~),  gX += gP~ W_P^T + gI~ W_I^T + gV W_V^T,
//       gW_P += X^T gP~ (per pod), likewise W_I, W_V
// Scatters are evaluated as gathers (cell q collects from r = q - offset_k).
namespace {

inline double gelu_tanh_grad(double x) {
    const double c0 = 0.7978845608028654, c1 = 0.044715;
    const double th = std::tanh(c0 * (x + c1 * x * x * x));
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * c0 * (1.0 + 3.0 * c1 * x * x);
}

// out[r][k] += sum_n g[r][n] W[pod][k][n]   (gradient of x W through its input)
void project_back_input(const Dims& d, const double* g, const float* W, double* out) {
    const int C = d.C;
    const long rows = (long)d.B * d.cells;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; ++r) {
        const int pod = (int)(r / d.cells) / d.per_pod;
        const float* w = W + (size_t)pod * C * C;
        const double* gr = g + (size_t)r * C;
        double* o = out + (size_t)r * C;
        for (int k = 0; k < C; ++k) {
            double acc = 0.0;
            for (int n = 0; n < C; ++n) acc += gr[n] * (double)w[(size_t)k * C + n];
            o[k] += acc;
        }
    }
}

// gW[pod][k][n] = sum over the pod's rows r of x[r][k] g[r][n]
void project_back_weight(const Dims& d, const double* x, const double* g, float* gW) {
    const int C = d.C;
    for (int pod = 0; pod < d.pods; ++pod) {
        const long r0 = (long)pod * d.per_pod * d.cells, r1 = r0 + (long)d.per_pod * d.cells;
#pragma omp parallel for schedule(static)
        for (int k = 0; k < C; ++k) {
            std::vector<double> acc(C, 0.0);
            for (long r = r0; r < r1; ++r) {
                const double xk = x[(size_t)r * C + k];
                const double* gr = g + (size_t)r * C;
                for (int n = 0; n < C; ++n) acc[n] += xk * gr[n];
            }
            for (int n = 0; n < C; ++n) gW[((size_t)pod * C + k) * C + n] = (float)acc[n];
        }
    }
}

}  // namespace

int oracle_step_backward(const oracle_ca_cfg* cfg, const float* X_in, const float* WP,
                         const float* WI, const float* WV, const float* K, const float* mu,
                         const float* sigma, const float* M, const float* T, double* loss,
                         float* gX, float* gWP, float* gWI, float* gWV, float* gK, float* gmu,
                         float* gsigma, float* gM) {
    Dims d;
    if (!dims_of(cfg, &d) || cfg->pvi_chain || cfg->growth_fn || cfg->conservation || !loss) return -1;
    const int G = d.G, C = d.C, D = d.D, H = d.H;
    const int per_cell = cfg->growth_per_cell;
    const double dt = cfg->dt, inv_sqrt_d = 1.0 / std::sqrt((double)D);
    const size_t n = (size_t)d.B * d.cells * C;
    const size_t na = (size_t)d.B * d.cells * H * 9;
    std::vector<double> x = to_d(X_in, n), pt(n), it(n), P(n), I(n), V(n), U(n), g(n), Vt(n), Y(n);
    std::vector<double> A(na);
    // forward, keeping the pre-activations
    project(d, x.data(), WP, 0, pt.data());
    project(d, x.data(), WI, 0, it.data());
    project(d, x.data(), WV, 0, V.data());
    for (size_t i = 0; i < n; ++i) {
        P[i] = pt[i] > 0.0 ? pt[i] : 0.0;
        I[i] = gelu_tanh(it[i]);
    }
    potential(d, x.data(), K, U.data());
    growth(d, per_cell, 0, U.data(), mu, sigma, g.data());
    attention(d, P.data(), I.data(), A.data());
    propagate(d, A.data(), V.data(), Vt.data());
    mix(d, dt, x.data(), g.data(), Vt.data(), M, Y.data());
    // S7 and the loss
    std::vector<double> rs((size_t)d.B * H), sx((size_t)d.B * H), sy((size_t)d.B * H);
    std::vector<char> guard((size_t)d.B * H);
    for (int b = 0; b < d.B; ++b)
        for (int o = 0; o < H; ++o) {
            double ax = 0.0, by = 0.0;
            for (long cell = 0; cell < d.cells; ++cell)
                for (int c = 0; c < D; ++c) {
                    const size_t i = ((size_t)b * d.cells + cell) * C + o * D + c;
                    ax += x[i];
                    by += Y[i];
                }
            const size_t bo = (size_t)b * H + o;
            guard[bo] = std::fabs(by) > 1e-6;
            rs[bo] = guard[bo] ? ax / by : 1.0;
            sx[bo] = ax;
            sy[bo] = by;
        }
    const double N = (double)n;
    double L = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const size_t bo = (i / ((size_t)d.cells * C)) * H + (i % C) / D;
        const double e = rs[bo] * Y[i] - T[i];
        L += e * e;
    }
    *loss = L / N;
    if (!gX) return 0;

    // S7 backward
    std::vector<double> gY(n), gx(n, 0.0);
    std::vector<double> Q((size_t)d.B * H, 0.0);
    for (size_t i = 0; i < n; ++i) {
        const size_t bo = (i / ((size_t)d.cells * C)) * H + (i % C) / D;
        gY[i] = 2.0 * (rs[bo] * Y[i] - T[i]) / N;  // gY' for now
        Q[bo] += gY[i] * Y[i];
    }
    for (size_t i = 0; i < n; ++i) {
        const size_t bo = (i / ((size_t)d.cells * C)) * H + (i % C) / D;
        if (guard[bo]) {
            gY[i] = rs[bo] * (gY[i] - Q[bo] / sy[bo]);
            gx[i] += Q[bo] / sy[bo];
        }
    }
    // S6 backward
    std::vector<double> gZ(n, 0.0), gg(n), gVt(n), gU(n);
    std::vector<double> gMd((size_t)d.pods * H * H, 0.0);
    for (long r = 0; r < (long)d.B * d.cells; ++r) {
        const int pod = (int)(r / d.cells) / d.per_pod;
        for (int h = 0; h < H; ++h)
            for (int c = 0; c < D; ++c) {
                const size_t i = (size_t)r * C + h * D + c;
                double acc = 0.0;
                for (int o = 0; o < H; ++o)
                    acc += (double)M[((size_t)pod * H + o) * H + h] * gY[(size_t)r * C + o * D + c];
                gZ[i] = acc;
                const double z = x[i] + dt * g[i] * Vt[i];
                for (int o = 0; o < H; ++o)
                    gMd[((size_t)pod * H + o) * H + h] += gY[(size_t)r * C + o * D + c] * z;
                gx[i] += acc;
                gg[i] = dt * acc * Vt[i];
                gVt[i] = dt * acc * g[i];
            }
    }
    // S3 backward
    const size_t ng = per_cell ? (size_t)d.pods * d.cells * H : (size_t)d.pods * H;
    std::vector<double> gmud(ng, 0.0), gsgd(ng, 0.0);
    for (long r = 0; r < (long)d.B * d.cells; ++r) {
        const int b = (int)(r / d.cells);
        const long cell = r % d.cells;
        const int pod = b / d.per_pod;
        for (int h = 0; h < H; ++h) {
            const size_t pi = per_cell ? ((size_t)pod * d.cells + cell) * H + h : (size_t)pod * H + h;
            const double m = mu[pi], sp = (double)sigma[pi] + 1e-7;
            for (int c = 0; c < D; ++c) {
                const size_t i = (size_t)r * C + h * D + c;
                const double t = (U[i] - m) / sp;
                const double gu = gg[i] * (-4.0 * t * std::exp(-t * t)) / sp;
                gU[i] = gu;
                gmud[pi] += -gu;
                gsgd[pi] += -gu * t;
            }
        }
    }
    // S2, S5, S4 backward (gathers over the 9 neighbours)
    std::vector<double> gV(n, 0.0), gP(n, 0.0), gI(n, 0.0), gS(na);
    std::vector<double> gKd((size_t)d.pods * H * 9, 0.0);
    for (int b = 0; b < d.B; ++b) {
        const int pod = b / d.per_pod;
        for (int y = 0; y < G; ++y)
            for (int xx = 0; xx < G; ++xx) {
                const size_t r = ((size_t)b * G + y) * G + xx;
                for (int h = 0; h < H; ++h) {
                    const double* a = A.data() + (r * H + h) * 9;
                    double ga[9], sum = 0.0;
                    for (int k = 0; k < 9; ++k) {
                        const int dy = k / 3 - 1, dx = k % 3 - 1;
                        const size_t q = ((size_t)b * G + wrap(y + dy, G)) * G + wrap(xx + dx, G);
                        double acc = 0.0, acck = 0.0;
                        for (int c = 0; c < D; ++c) {
                            acc += gVt[r * C + h * D + c] * V[q * C + h * D + c];
                            acck += gU[r * C + h * D + c] * x[q * C + h * D + c];
                        }
                        ga[k] = acc;
                        sum += a[k] * acc;
                        gKd[((size_t)pod * H + h) * 9 + k] += acck;
                    }
                    for (int k = 0; k < 9; ++k) gS[(r * H + h) * 9 + k] = a[k] * (ga[k] - sum);
                    for (int k = 0; k < 9; ++k) {
                        const int dy = k / 3 - 1, dx = k % 3 - 1;
                        const size_t q = ((size_t)b * G + wrap(y + dy, G)) * G + wrap(xx + dx, G);
                        const double gs = gS[(r * H + h) * 9 + k] * inv_sqrt_d;
                        for (int c = 0; c < D; ++c) gP[r * C + h * D + c] += gs * I[q * C + h * D + c];
                    }
                }
            }
    }
    for (int b = 0; b < d.B; ++b) {
        const int pod = b / d.per_pod;
        for (int y = 0; y < G; ++y)
            for (int xx = 0; xx < G; ++xx) {
                const size_t q = ((size_t)b * G + y) * G + xx;
                for (int k = 0; k < 9; ++k) {
                    const int dy = k / 3 - 1, dx = k % 3 - 1;
                    const size_t r = ((size_t)b * G + wrap(y - dy, G)) * G + wrap(xx - dx, G);
                    for (int h = 0; h < H; ++h) {
                        const double a = A[(r * H + h) * 9 + k];
                        const double gs = gS[(r * H + h) * 9 + k] * inv_sqrt_d;
                        const double kw = K[((size_t)pod * H + h) * 9 + k];
                        for (int c = 0; c < D; ++c) {
                            const size_t iq = q * C + h * D + c, ir = r * C + h * D + c;
                            gV[iq] += a * gVt[ir];
                            gI[iq] += gs * P[ir];
                            gx[iq] += kw * gU[ir];
                        }
                    }
                }
            }
    }
    // S1 backward
    for (size_t i = 0; i < n; ++i) {
        gP[i] = pt[i] > 0.0 ? gP[i] : 0.0;
        gI[i] *= gelu_tanh_grad(it[i]);
    }
    project_back_input(d, gP.data(), WP, gx.data());
    project_back_input(d, gI.data(), WI, gx.data());
    project_back_input(d, gV.data(), WV, gx.data());
    to_f(gx, gX);
    if (gWP) project_back_weight(d, x.data(), gP.data(), gWP);
    if (gWI) project_back_weight(d, x.data(), gI.data(), gWI);
    if (gWV) project_back_weight(d, x.data(), gV.data(), gWV);
    if (gK) to_f(gKd, gK);
    if (gmu) to_f(gmud, gmu);
    if (gsigma) to_f(gsgd, gsigma);
    if (gM) to_f(gMd, gM);
    return 0;
}

int oracle_init_from_field(int G, int C, const float* conc, float* X) {
    if (G <= 0 || C <= 0) return -1;
    for (long cell = 0; cell < (long)G * G; ++cell)
        for (int c = 0; c < C; ++c)
            X[(size_t)cell * C + c] =
                (float)((double)conc[cell] * std::sin((double)((float)c * 0.1f)));
    return 0;
}

int oracle_field_from_state(int G, int C, const float* X, float* conc) {
    if (G <= 0 || C <= 0) return -1;
    for (long cell = 0; cell < (long)G * G; ++cell) {
        double s = 0.0;
        for (int c = 0; c < C; ++c) s += X[(size_t)cell * C + c];
        conc[cell] = (float)(s / C);
    }
    return 0;
}

}  // extern "C"
