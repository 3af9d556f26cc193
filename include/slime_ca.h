/*
 * slime_ca.h — C ABI of the MI355X (gfx950) multi-head neural-CA step.
 *
 * Drop-in for the CA hot path of J0pari/Slime. Each entry point names the
 * reference interface it replaces (paths under the reference tree):
 *
 *   slime_ca_create / slime_ca_destroy      buffer ownership of create_organism /
 *                                           destroy_organism for the CA state
 *                                           (slime/runtime.cu:66-94,173-182,453-461)
 *   slime_ca_set_params                     init_multihead_ca_kernel
 *                                           (slime/core/pseudopod.cu:386-444)
 *   slime_ca_project                        multi_head_ca_kernel
 *                                           (slime/core/pseudopod.cu:41-49)
 *   slime_ca_flow_lenia                     flow_lenia_dynamics_kernel + mix_heads_kernel
 *                                           (slime/core/pseudopod.cu:134-141,217-223)
 *   slime_ca_step                           the CA part of neural_ca_update_kernel
 *                                           (slime/core/organism.cu:639-669)
 *   slime_ca_mass                           mass_buffer (slime/core/pseudopod.cu:35,205-213)
 *   slime_ca_fitness                        fitness_fused_kernel
 *                                           (slime/kernels/warp_ca.cu:178-226)
 *   slime_ca_init_from_field /
 *   slime_ca_field_from_state               initialize_ca_from_field_kernel /
 *                                           update_field_from_ca_kernel
 *                                           (slime/core/organism.cu:691-743)
 *   slime_neural_ca_update                  neural_ca_update_kernel, the organism's
 *                                           per-generation CA call
 *                                           (slime/core/organism.cu:617-688)
 *   slime_ca_last_error                    the printed message of CUDA_CHECK
 *                                           (slime/runtime.cu:11-20), returned instead
 *                                           of exit(1)
 *
 * Conventions
 *   - Every function returns SLIME_OK (0) or a negative SLIME_E* code and never
 *     exits the process; slime_ca_last_error() describes the last failure on the
 *     calling thread.
 *   - State tensors are device pointers, channels-last [B][G][G][C] with
 *     C = H * D, element type = the handle's dtype (fp32, or bf16 as raw 16-bit
 *     words). Arithmetic is fp32 (fp64 for reductions and the Jacobi solve).
 *   - Parameters are host fp32 arrays, row-major:
 *       WP, WI, WV   [pods][C][C]   row k = input channel, column n = output channel
 *       K            [pods][H][9]   tap k = 3*(dy+1)+(dx+1), toroidal neighbours
 *       mu, sigma    [pods][H], or [pods][G][G][H] when growth_per_cell = 1
 *       M            [pods][H][H]   M[o][h]: weight of head h in output head o
 *     Batch entry b uses parameter set b / (B / pods).
 *   - stream is a hipStream_t passed as void* (NULL = default stream). Calls on
 *     one handle are stream-ordered and not thread-safe; use one stream per
 *     handle. No HIP types appear in this header.
 */
#ifndef SLIME_CA_H
#define SLIME_CA_H

#include <stddef.h> /* size_t */

#ifdef __cplusplus
extern "C" {
#endif

#define SLIME_OK 0
#define SLIME_EINVAL (-1)  /* invalid argument or configuration */
#define SLIME_ENOMEM (-2)  /* device allocation failed */
#define SLIME_EHIP (-3)    /* HIP runtime error */
#define SLIME_ENODEV (-4)  /* no usable gfx950 device */
#define SLIME_ESTATE (-5)  /* call out of order (e.g. step before set_params) */
#define SLIME_ENONFINITE (-6) /* a conserved sum is NaN or Inf: the state holds one */

#define SLIME_F32 0
#define SLIME_BF16 1

typedef struct slime_ca slime_ca;

typedef struct {
    int B;               /* batch entries */
    int G;               /* grid side (toroidal), multiple of 8, >= 8 */
    int H;               /* heads, must be 8 (NUM_HEADS, slime/core/pseudopod.cu:15) */
    int D;               /* head dim: 8, 16, 32 or 64 */
    int dtype;           /* SLIME_F32 or SLIME_BF16: storage of state and weights */
    float dt;            /* update step, 0.1 in the reference (slime/core/organism.cu:659) */
    int growth_per_cell; /* 0: mu, sigma per head; 1: per cell and head */
    int pods;            /* independent parameter sets; B % pods == 0 */
    int pvi_chain;       /* 0: P, I, V all from X;
                            1: I from P and V from I (the chained form of
                               slime/core/pseudopod.cu:98-119), P from X;
                            2: as 1, with P from the toroidal 3x3 neighbourhood sum
                               of X, the perception of multi_head_ca_kernel
                               (slime/core/pseudopod.cu:62-91, which clamps at the
                               border instead of wrapping) */
    int growth_fn;       /* S3: 0 the bell 2 exp(-((U-mu)/(sigma+1e-7))^2) - 1
                               (failed_attempts/warp_ca.cu:49-56);
                            1 the Gaussian exp(-(U-mu)^2 / (2 sigma^2))
                               (failed_attempts/pseudopod.cu:46-48; sigma != 0);
                            2 the shipped U exp(-U^2), mu and sigma unused
                               (slime/core/pseudopod.cu:183) */
    int conservation;    /* S7: 0 per (batch, head) over the grid
                               (failed_attempts/warp_ca.cu:401-450);
                            1 per (cell, head) first, the shipped kernel's
                               renormalisation (slime/core/pseudopod.cu:160-165,
                               196-203), then per (batch, head) as 0 (a factor of 1
                               up to rounding) */
} slime_ca_config;

typedef struct {
    const float* WP;
    const float* WI;
    const float* WV;
    const float* K;
    const float* mu;
    const float* sigma;
    const float* M;
} slime_ca_params;

/* Allocates every device buffer the step needs on the current device. */
int slime_ca_create(const slime_ca_config* config, slime_ca** out);
int slime_ca_destroy(slime_ca* ca);

/* Uploads parameters (host fp32, layouts above). Synchronous. Every array is
 * checked first (slime_ca_check_params): a NaN or Inf entry is SLIME_EINVAL and
 * leaves the handle's parameters as they were. */
int slime_ca_set_params(slime_ca* ca, const slime_ca_params* params);

/* The host-side checks of slime_ca_set_params for a configuration, without a handle
 * or a device: the config is valid, no pointer is NULL and every entry of the
 * arrays (sizes from the config) is finite. SLIME_OK or SLIME_EINVAL. The
 * reference uploads its parameters unchecked (init_multihead_ca_kernel,
 * slime/core/pseudopod.cu:386-444). */
int slime_ca_check_params(const slime_ca_config* config, const slime_ca_params* params);

/* S1: P = ReLU(X W_P) (X replaced by its 3x3 neighbourhood sum for pvi_chain 2),
 * I = GELU_tanh(X W_I) (or of P W_I when chained), V = X W_V (or I W_V). P, I, V
 * are [B][G][G][C] in the handle's dtype, distinct from x_in and from each other
 * (pvi_chain 2 uses V as scratch for the neighbourhood sum before V's product). */
int slime_ca_project(slime_ca* ca, const void* x_in, void* P, void* I, void* V, void* stream);

/* S2-S7 on given projections: 3x3 toroidal potential, bell growth, 3x3 CA
 * activation, value propagation, modulated update, head mixing and per-(b, head)
 * mass conservation. y_out must not alias x_in, P, I or V. */
int slime_ca_flow_lenia(slime_ca* ca, const void* x_in, const void* P, const void* I,
                        const void* V, void* y_out, void* stream);

/* n_steps full steps S1-S7 from x_in to x_out (x_out may equal x_in). After the
 * call the handle's mass buffer holds the last step's per-(b, head) sums. */
int slime_ca_step(slime_ca* ca, const void* x_in, void* x_out, int n_steps, void* stream);

/* Host copies of the last step's per-(b, head) input mass and output mass
 * (after conservation), B*H doubles each (either pointer may be NULL).
 * Synchronises the last stream used. SLIME_ENONFINITE, with the copies made, when
 * a sum is NaN or Inf: the step's input or output held a non-finite value. */
int slime_ca_mass(slime_ca* ca, double* h_mass_in, double* h_mass_out);

/* E1-E5 over a device history [T][B][G][G][C] (2 <= T <= 65): per (b, head)
 * effective rank of the last state's Gram matrix (64x64 Jacobi for D = 64),
 * lag-1 coherence over the T states and their product. Outputs are device
 * float arrays of B*H entries. */
int slime_ca_fitness(slime_ca* ca, const void* x_hist, int T, float* erank, float* coherence,
                     float* fitness, void* stream);

/* Parameter gradients of slime_ca_backward: device fp32 arrays in the layouts of
 * slime_ca_params (WP, WI, WV [pods][C][C]; K [pods][H][9]; mu, sigma [pods][H]
 * or [pods][G][G][H]; M [pods][H][H]). Any pointer may be NULL. */
typedef struct {
    float* WP;
    float* WI;
    float* WV;
    float* K;
    float* mu;
    float* sigma;
    float* M;
} slime_ca_grads;

/* One step from x_in (parallel projections) and the gradient of the loss
 * L = mean((x_out - target)^2) over all B*G*G*C elements (configuration c5),
 * x_out taken before its storage rounding: grad_x (device fp32 [B][G][G][C])
 * and, through grads (may be NULL), the parameter gradients. *loss (host, may be
 * NULL) receives L, which synchronises the stream. No counterpart in the
 * reference: it declares gradients (gradients_d and update_gradients,
 * slime/proto/model.cu:7,13) but never computes them. SLIME_EINVAL for chained
 * projections, growth_fn != 0 or conservation != 0. */
int slime_ca_backward(slime_ca* ca, const void* x_in, const void* target, float* grad_x,
                      const slime_ca_grads* grads, double* loss, void* hip_stream);

/* T-1 steps from hist[0] with every state kept: the organism's run of generations
 * whose last states the fitness scores (slime/core/organism.cu:679-683, the
 * effective-rank history; slime/kernels/warp_ca.cu:178-185 scores such a history).
 * hist (device, [T][B][G][G][C], the handle's dtype) holds the initial state in
 * hist[0] on entry; on return hist[t] holds state t as the step that produced it
 * stores it before its mass rescale, and scales (device fp64, [T][B][H]) the factor
 * that completes it: state t = scales[t][b][h] * hist[t] over head h of batch entry
 * b (scales[0] = 1). The next step reads each state that way, so no state is
 * rescaled in a pass of its own. Up to the storage rounding (once per state, before
 * rather than after the factor), the states are those of T-1 calls of
 * slime_ca_step(n_steps = 1); slime_ca_fitness_scaled scores the history. The
 * handle's mass sums are those of the last step. */
int slime_ca_rollout(slime_ca* ca, void* hist, int T, double* scales, void* stream);

/* slime_ca_fitness of a history stored with per-(state, batch, head) factors as
 * slime_ca_rollout leaves it: the moments and the last state's Gram are scaled in
 * fp64, so the result is that of the states scales[t] * hist[t]. */
int slime_ca_fitness_scaled(slime_ca* ca, const void* x_hist, const double* scales, int T,
                            float* erank, float* coherence, float* fitness, void* stream);

/* slime_ca_fitness without a handle and without allocating: no counterpart in the
 * reference. For callers that cannot call hipMalloc (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation). The partial sums go to a
 * static device buffer of 32 MiB per GPU that the library holds until the process
 * ends; B*H*chunks*(D*D + 3T) fp64 partials must fit, with the chunk count lowered
 * from slime_ca_fitness's when needed (which can change the last bits of the Gram
 * sums), else SLIME_EINVAL. Every call on a GPU shares that buffer: a call on
 * another stream than the previous call's waits for it (an event recorded after
 * each call), but under graph capture no event is used, and replays that overlap
 * on one GPU race. Loading the library reserves the buffer on every GPU it runs
 * on. The first call on a device looks up the buffer's address there and creates
 * its event (make it outside graph capture). config gives B, G, H, D and
 * dtype of the history (its other fields are validated but unused); outputs as
 * slime_ca_fitness; no sweep counts. */
int slime_ca_fitness_static(const slime_ca_config* config, const void* x_hist, int T,
                            float* erank, float* coherence, float* fitness, void* stream);

/* Jacobi sweeps used by the last slime_ca_fitness call, B*H ints (host copy). */
int slime_ca_fitness_sweeps(slime_ca* ca, int* h_sweeps);

/* Organism adapters for one G x G grid of C channels in the handle's dtype:
 * X[y][x][c] = conc[y][x] * sin(0.1 c), and conc[y][x] = mean_c X[y][x][c]. */
int slime_ca_init_from_field(slime_ca* ca, const float* conc, void* x, void* stream);
int slime_ca_field_from_state(slime_ca* ca, const void* x, float* conc, void* stream);

/* Read-back for visualisation; replaces get_ca_state (slime/runtime.cu:479-504, with
 * extract_ca_channel_kernel :506-518), which copies `size` floats of the organism's
 * chemical concentration to the host. After a generation that field is
 * update_field_from_ca of the CA output, so this computes conc = mean_c X of the
 * device state `x` (one G x G grid, handle dtype) and copies its first `size` values
 * (row-major, 0 <= size <= G*G, else SLIME_EINVAL) to the host array h_buffer.
 * Synchronous like the reference: it waits for all work on the device, so `x` may
 * come from any stream. */
int slime_ca_get_state(slime_ca* ca, const void* x, float* h_buffer, int size);

/* The buffers of the reference's MultiHeadCAState (slime/core/pseudopod.cu:29-38)
 * that one organism generation reads and writes, under the same field names. The
 * parameter fields of that struct (perception_weights, interaction_weights,
 * value_weights, head_mixing_weights, flow_kernels) are held by the handle and
 * uploaded by slime_ca_set_params, which replaces init_multihead_ca_kernel. */
typedef struct {
    float* mass_buffer; /* device, H floats: per-head mass after conservation (may be NULL) */
    void* ca_input;     /* device [G][G][C], handle dtype */
    void* ca_output;    /* device [G][G][C], handle dtype, distinct from ca_input */
} slime_multihead_ca_state;

/* One organism generation of the CA, launched from the host on `stream`; replaces
 * neural_ca_update_kernel (slime/core/organism.cu:617-688) for a handle with B = 1:
 *   ca_input  = initialize_ca_from_field(chemical_concentration)
 *   ca_output = one step S1-S7 of ca_input (projections, flow Lenia, head mixing and
 *               mass conservation)
 *   chemical_concentration = update_field_from_ca(ca_output)
 *   mass_buffer[h] = conserved mass of head h
 *   effective_rank_history[generation] = mean over heads of the effective rank of
 *               ca_output's per-head Gram matrix (E1-E3), in place of the
 *               weight-energy proxy compute_effective_rank_kernel
 *               (slime/core/pseudopod.cu:302-345).
 * chemical_concentration is device [G][G] fp32; effective_rank_history is a device
 * float array of more than `generation` entries. */
int slime_neural_ca_update(slime_ca* ca, const slime_multihead_ca_state* state,
                           float* chemical_concentration, float* effective_rank_history,
                           int generation, void* stream);

/* Kernel timing (no counterpart in the reference, which has no timers on this
 * path). While enabled, slime_ca_step records HIP events on its stream around
 * each projection GEMM and each fused stencil launch; slime_ca_timings returns
 * the summed device milliseconds and launch counts since timing was enabled
 * (it synchronises the last stream used). Enabling resets the sums. */
int slime_ca_set_timing(slime_ca* ca, int enable);
int slime_ca_timings(slime_ca* ca, double* gemm_ms, int* gemm_launches, double* stencil_ms,
                     int* stencil_launches);

/* ---- fitness consumers: the component pool -----------------------------------------
 * The reference's ComponentPool / PoolEntry (slime/memory/pool.cu:12-30) as a
 * structure of device arrays owned by the caller (nothing is allocated by these
 * calls). counters = {active_count, total_spawned, total_culled}. */
typedef struct {
    int capacity;      /* entries (MAX_POOL_SIZE = 256 in the reference) */
    int genome_size;   /* floats per genome (GENOME_SIZE = 512) */
    int* id;           /* [capacity] */
    float* fitness;    /* [capacity] */
    float* coherence;  /* [capacity] */
    float* hunger;     /* [capacity] */
    int* age;          /* [capacity] */
    int* alive;        /* [capacity], 0 or 1 */
    float* genome;     /* [capacity][genome_size] */
    float* gradients;  /* [capacity][genome_size] */
    int* counters;     /* [3]: active, spawned, culled */
} slime_pool;

/* Every entry dead with id -1, fitness 0, coherence 0, hunger 0.5, age 0, zero
 * genome and gradients; counters 0. Replaces init_pool_kernel
 * (slime/memory/pool.cu:300-320). */
int slime_pool_init(const slime_pool* pool, void* stream);

/* Alive entry i < n takes fitness = mean over `heads` of fitness[i*heads + h],
 * coherence likewise, hunger = 1 - coherence, and fitness_history /
 * coherence_history[generation * capacity + i] (either may be NULL). With the
 * per-(batch, head) outputs of slime_ca_fitness and batch entry = component, this
 * feeds the fused CA fitness to the pool in place of the genome-norm proxy of
 * fitness_computation_kernel (slime/core/organism.cu:204-289). */
int slime_pool_set_fitness(const slime_pool* pool, const float* fitness, const float* coherence, int n,
                           int heads, int generation, float* fitness_history,
                           float* coherence_history, void* stream);

/* hunger[i] = 1 - coherence[i] over n device floats: hunger_kernel
 * (slime/kernels/warp_ca.cu:229-240). */
int slime_ca_hunger(const float* coherence, float* hunger, int n, void* stream);

/* age += 1 for alive entries: age_components_kernel (slime/memory/pool.cu:162-168). */
int slime_pool_age(const slime_pool* pool, void* stream);

/* An alive entry dies when fitness < fitness_threshold * 0.1 or hunger >
 * hunger_threshold (active -1, culled +1 each): culling_kernel
 * (slime/core/organism.cu:590-614; the lifecycle passes 0.8 and 0.95). */
int slime_pool_cull(const slime_pool* pool, float fitness_threshold, float hunger_threshold,
                    void* stream);

/* One spawn into the first dead slot when active < capacity: spawn_component_kernel
 * (slime/memory/pool.cu:57-121). parent outside [0, capacity) draws a uniform
 * genome in [-1, 1). */
int slime_pool_spawn(const slime_pool* pool, int parent, float mutation_rate, void* stream);

/* The spawn wave of the lifecycle (slime/core/organism.cu:557-587): 32 draws in
 * lane order, each spawning from the first alive entry with fitness > 0.5 (rate
 * 0.01) when the draw is below `probability`. probability < 0 computes the
 * lifecycle's 0.1 * exp(-active / 256) on the device and skips the wave unless it
 * exceeds 0.01 (organism.cu:185-186). */
int slime_pool_spawn_wave(const slime_pool* pool, float probability, int generation, void* stream);

/* The fitness consumers of one lifecycle generation (component_evolution_kernel,
 * slime/core/organism.cu:144-201, without selection and archive): set_fitness,
 * spawn wave with the device-computed probability, cull at 0.8 / 0.95. */
int slime_pool_evolve(const slime_pool* pool, const float* fitness, const float* coherence, int n,
                      int heads, int generation, float* fitness_history, float* coherence_history,
                      void* stream);

/* One generation record of the reference's evolution.json (extract_system_state,
 * slime/extract_state.cu:64-184), written into buf (NUL-terminated):
 *   {"gen":G,"elapsed":E.EE,"chemical":{"concentration":[16x16 centre sample, %.4f],
 *    "size":16},"ca":{"flow_kernels":[[9 x %.4f] per head]},"agents":[],"voronoi":[],
 *    "archive":{"size":0,"elites":[]},"pool":{"active":A,"capacity":C,"spawned":S,
 *    "culled":K}}
 * with the keys in the reference's order. chemical_concentration is device [G][G]
 * fp32 (the sample is min(16, G) wide, centred); flow_kernels are pod 0's K of the
 * handle; pool (may be NULL: zeros) supplies the counters. The behavioural agents,
 * Voronoi cells and elite archive have no counterpart here and are written empty,
 * so the record stays valid JSON (the reference's archive object closes one brace
 * too many). *written receives the record's length; a buffer shorter than that
 * plus its NUL is SLIME_EINVAL. Synchronous, like the reference's extraction. */
int slime_snapshot_json(const slime_ca* ca, const float* chemical_concentration,
                        const slime_pool* pool, int generation, double elapsed, char* buf,
                        size_t cap, size_t* written);

/* 1 when this build runs S1 on the MFMA tile kernel for the handle's shape. */
int slime_ca_uses_mfma(const slime_ca* ca);

const char* slime_ca_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* SLIME_CA_H */
