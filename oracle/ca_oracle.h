/*
 * ca_oracle.h — CPU restatement of Slime's multi-head neural-CA step and its
 * fitness = effective_rank x coherence, used ONLY as a test checker and as the
 * bench's CPU baseline.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only to check or time against
 * it. The product library (libslime_ca.so) never links, loads or calls it.
 *
 * All arithmetic is double precision; tensors cross the interface as fp32
 * (callers that emulate bf16 round their inputs before the call).
 *
 * Layouts (channels-last, C = H*D):
 *   state X, P, I, V, U, Vt, Y : [B][G][G][C]
 *   attention A                : [B][G][G][H][9]   (k = 3*(dy+1)+(dx+1))
 *   W_P, W_I, W_V              : [pods][C][C]      (row k = input channel)
 *   K (flow kernels)           : [pods][H][9]
 *   mu, sigma                  : [pods][H] or, growth_per_cell=1, [pods][G][G][H]
 *   M (head mixing)            : [pods][H][H]      (M[o][h])
 *   batch b uses pod b / (B / pods)
 */
#ifndef SLIME_CA_ORACLE_H
#define SLIME_CA_ORACLE_H
#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int B, G, H, D;
    int pods;
    int growth_per_cell;
    int pvi_chain; /* 0 parallel; 1 chained; 2 chained, P from the 3x3 neighbourhood sum */
    float dt;
    int growth_fn;    /* 0 bell, 1 Gaussian, 2 shipped U exp(-U^2) */
    int conservation; /* 0 per (b, head); 1 per (cell, head), then per (b, head) */
} oracle_ca_cfg;

/* Each returns 0 on success, -1 on invalid configuration. */
int oracle_project(const oracle_ca_cfg* cfg, const float* X, const float* WP, const float* WI,
                   const float* WV, float* P, float* I, float* V);
int oracle_potential(const oracle_ca_cfg* cfg, const float* X, const float* K, float* U);
int oracle_growth(const oracle_ca_cfg* cfg, const float* U, const float* mu, const float* sigma,
                  float* g);
int oracle_attention(const oracle_ca_cfg* cfg, const float* P, const float* I, float* A);
int oracle_propagate(const oracle_ca_cfg* cfg, const float* A, const float* V, float* Vt);
int oracle_mix(const oracle_ca_cfg* cfg, const float* X, const float* g, const float* Vt,
               const float* M, float* Y);
int oracle_conserve(const oracle_ca_cfg* cfg, const float* X, float* Y, double* mass_in,
                    double* mass_out);
int oracle_step(const oracle_ca_cfg* cfg, const float* X_in, const float* WP, const float* WI,
                const float* WV, const float* K, const float* mu, const float* sigma,
                const float* M, float* X_out, int n_steps, double* mass_in, double* mass_out);

/* One step (parallel projections) and the loss L = mean (X_out - T)^2; with gX
 * non-NULL also dL/dX and, for each non-NULL pointer, the parameter gradients
 * (shapes as the parameters). Returns -1 for chained projections. */
int oracle_step_backward(const oracle_ca_cfg* cfg, const float* X, const float* WP,
                         const float* WI, const float* WV, const float* K, const float* mu,
                         const float* sigma, const float* M, const float* T, double* loss,
                         float* gX, float* gWP, float* gWI, float* gWV, float* gK, float* gmu,
                         float* gsigma, float* gM);

int oracle_gram(const oracle_ca_cfg* cfg, const float* X, double* A);
int oracle_jacobi_eigs(const double* A, int n, double* eig_desc, int max_sweeps, double tol);
double oracle_effective_rank(const double* sv, int n);
int oracle_coherence(const oracle_ca_cfg* cfg, const float* hist, int T, double* coh);
int oracle_fitness(const oracle_ca_cfg* cfg, const float* hist, int T, double* erank,
                   double* coh, double* fitness);

int oracle_init_from_field(int G, int C, const float* conc, float* X);
int oracle_field_from_state(int G, int C, const float* X, float* conc);

int oracle_num_threads(void);

/* Component pool (pool_oracle.cpp): host arrays in the layout of slime_pool. */
typedef struct {
    int capacity, genome_size;
    int* id;
    float* fitness;
    float* coherence;
    float* hunger;
    int* age;
    int* alive;
    float* genome;    /* [capacity][genome_size] */
    float* gradients; /* [capacity][genome_size] */
    int* counters;    /* active, spawned, culled */
} oracle_pool;
float oracle_xorshift_next(unsigned long long* s0, unsigned long long* s1);
float oracle_xorshift_gaussian(unsigned long long* s0, unsigned long long* s1);
void oracle_pool_init(oracle_pool* p);
void oracle_pool_set_fitness(oracle_pool* p, const float* fit, const float* coh, int n, int heads,
                             int generation, float* fit_hist, float* coh_hist);
void oracle_hunger(const float* coh, float* hunger, int n);
void oracle_pool_age(oracle_pool* p);
void oracle_pool_cull(oracle_pool* p, float fitness_threshold, float hunger_threshold);
void oracle_pool_spawn(oracle_pool* p, int parent, float rate);
float oracle_pool_spawn_wave(oracle_pool* p, float probability, int generation);
void oracle_pool_evolve(oracle_pool* p, const float* fit, const float* coh, int n, int heads,
                        int generation, float* fit_hist, float* coh_hist);

#ifdef __cplusplus
}
#endif
#endif
