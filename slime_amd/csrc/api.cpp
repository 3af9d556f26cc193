// api.cpp — the C ABI declared in include/slime_ca.h: handle ownership,
// argument validation and the host-ordered launch sequence of one CA step.
//
// The reference orchestrates the step from the device with dynamic parallelism
// (neural_ca_update_kernel, slime/core/organism.cu:617-688) and aborts the
// process on any CUDA error (CUDA_CHECK, slime/runtime.cu:11-20). Here the host
// enqueues the kernels on the caller's stream and every failure becomes a
// status code plus a thread-local message.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/slime_ca.h"
#include "kernels.hpp"

using namespace slime;

struct slime_ca {
    slime_ca_config cfg;
    int C = 0;
    int tiles = 0;
    int device = 0;
    size_t elem = 4;
    long long state_elems = 0;
    bool params_set = false;
    hipStream_t last_stream = nullptr;

    float* Wtm = nullptr;      // [pods][3C][C] fp32 masters, transposed (n-major)
    void* Wt = nullptr;        // [B][3C][C] per-batch scaled, transposed
    float* K = nullptr;        // [pods][H][9]
    float* mu = nullptr;       // [pods][H] or [pods][G][G][H]
    float* sigma = nullptr;
    float* M = nullptr;        // [pods][H][H]
    void* kband = nullptr;     // bf16, D = 64: the stencil's 3x3 band table (fill_stencil_kband)
    unsigned* sched = nullptr;  // bf16, D = 64: the stencil's 16 tile counters (StencilArgs::sched)
    void* P = nullptr;         // [B][G][G][C] work buffers for slime_ca_step
    void* I = nullptr;
    void* V = nullptr;
    void* S[2] = {nullptr, nullptr};  // unscaled step outputs (ping-pong)
    float* Sf = nullptr;       // unscaled fp32 output of a call's last step (bf16 state only)
    double* part_in = nullptr;  // [B*H][tiles]
    double* part_out = nullptr;
    float* scale[2] = {nullptr, nullptr};  // [2][B*H]: high parts, then low parts
    float* unit_scale = nullptr;           // [2][B*H]: 1.0, then 0.0
    double* mass_in = nullptr;             // [B*H]
    double* mass_out = nullptr;

    int fit_chunks = 0;
    int fit_T = 0;             // history length the fitness partials are sized for
    double* gram_part = nullptr;
    double* mom_part = nullptr;
    int* sweeps = nullptr;     // [B*H]
    float* org_fit = nullptr;  // [3][B*H] erank, coherence, fitness of slime_neural_ca_update
    float* view = nullptr;     // [G][G] field of slime_ca_get_state (allocated on its first call)

    // slime_ca_backward (allocated on its first call)
    void* Wcat = nullptr;      // [pods][C][3C] = [W_P | W_I | W_V] row k (input channel), dtype
    std::vector<float> wcat_host;
    void* Ipre = nullptr;      // I before the GELU, dtype
    double* bw_lpart = nullptr;
    float* bw_coef = nullptr;
    double* bw_loss = nullptr;
    float* bw_gU = nullptr;
    float* bw_gVt = nullptr;
    float* bw_att = nullptr;
    float* bw_gS = nullptr;
    void* bw_G3 = nullptr;
    float* bw_gXd = nullptr;
    float* bw_ppart = nullptr;
    float* bw_gcell = nullptr;
    void* bw_gXp = nullptr;
    float* bw_dwpart = nullptr;
    float* bw_y32 = nullptr;   // fp32 unscaled output of the taped step (fp32 state only)

    // Optional per-kernel timing: event pairs recorded around launches.
    bool timing = false;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_used = 0;
    std::vector<std::pair<size_t, size_t>> gemm_ev, stencil_ev;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                         \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return fail(e_ == hipErrorOutOfMemory ? SLIME_ENOMEM : SLIME_EHIP, "%s: %s (%s:%d)", \
                        #expr, hipGetErrorString(e_), __FILE__, __LINE__);                    \
    } while (0)

int dalloc(void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) return SLIME_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(SLIME_ENOMEM, "hipMalloc(%zu bytes): %s", bytes, hipGetErrorString(e));
    }
    return SLIME_OK;
}

template <typename P>
int dalloc_t(P** p, size_t bytes) {
    void* v = nullptr;
    int rc = dalloc(&v, bytes);
    *p = static_cast<P*>(v);
    return rc;
}

int validate(const slime_ca_config* c) {
    if (!c) return fail(SLIME_EINVAL, "config is NULL");
    if (c->B < 1) return fail(SLIME_EINVAL, "B=%d must be >= 1", c->B);
    if (c->G < 8 || c->G % 8 != 0) return fail(SLIME_EINVAL, "G=%d must be a multiple of 8", c->G);
    if (c->H != kHeads) return fail(SLIME_EINVAL, "H=%d unsupported (must be %d)", c->H, kHeads);
    if (c->D != 8 && c->D != 16 && c->D != 32 && c->D != 64)
        return fail(SLIME_EINVAL, "D=%d unsupported (8, 16, 32 or 64)", c->D);
    if (c->dtype != SLIME_F32 && c->dtype != SLIME_BF16)
        return fail(SLIME_EINVAL, "dtype=%d unsupported", c->dtype);
    if (c->pods < 1 || c->B % c->pods != 0)
        return fail(SLIME_EINVAL, "pods=%d must divide B=%d", c->pods, c->B);
    if (!std::isfinite(c->dt)) return fail(SLIME_EINVAL, "dt is not finite");
    if (c->growth_per_cell != 0 && c->growth_per_cell != 1)
        return fail(SLIME_EINVAL, "growth_per_cell must be 0 or 1");
    if (c->pvi_chain < 0 || c->pvi_chain > 2) return fail(SLIME_EINVAL, "pvi_chain must be 0, 1 or 2");
    if (c->growth_fn < 0 || c->growth_fn > 2) return fail(SLIME_EINVAL, "growth_fn must be 0, 1 or 2");
    if (c->conservation != 0 && c->conservation != 1)
        return fail(SLIME_EINVAL, "conservation must be 0 or 1");
    const double elems = (double)c->B * c->G * c->G * c->H * c->D;
    if (elems > 4.0e9) return fail(SLIME_EINVAL, "state of %.3g elements is too large", elems);
    // The stencils address one batch entry with 32-bit offsets: element offsets in
    // int and byte offsets in unsigned, the bytes of the widest array they read or
    // write (the fp32 output of a call's last step, also for a bf16 state).
    const double per_batch = (double)c->G * c->G * c->H * c->D;
    if (per_batch >= 2147483648.0 || per_batch * 4.0 >= 4294967296.0)
        return fail(SLIME_EINVAL,
                    "one batch entry of %.3g elements (G=%d, C=%d) exceeds the 32-bit per-batch "
                    "offsets of the stencil (G*G*C*4 bytes must stay below 2^32)",
                    per_batch, c->G, c->H * c->D);
    return SLIME_OK;
}

hipEvent_t next_event(slime_ca* h) {
    if (h->ev_used == h->ev_pool.size()) {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        h->ev_pool.push_back(e);
    }
    return h->ev_pool[h->ev_used++];
}

// Records an event pair around the launches in fn when timing is enabled.
template <typename Fn>
hipError_t timed(slime_ca* h, std::vector<std::pair<size_t, size_t>>& log, hipStream_t s, Fn fn) {
    if (!h->timing) return fn();
    hipEvent_t a = next_event(h);
    const size_t ia = h->ev_used - 1;
    hipEvent_t b = next_event(h);
    const size_t ib = h->ev_used - 1;
    if (!a || !b) return hipErrorOutOfMemory;
    hipError_t e = hipEventRecord(a, s);
    if (e == hipSuccess) e = fn();
    if (e == hipSuccess) e = hipEventRecord(b, s);
    if (e == hipSuccess) log.emplace_back(ia, ib);
    return e;
}

void release(slime_ca* h) {
    for (hipEvent_t e : h->ev_pool) (void)hipEventDestroy(e);
    h->ev_pool.clear();
    void* ptrs[] = {h->Wtm, h->Wt, h->K, h->mu, h->sigma, h->M, h->kband, h->sched, h->P, h->I, h->V,
                    h->S[0], h->S[1], h->Sf, h->part_in, h->part_out, h->scale[0], h->scale[1], h->unit_scale,
                    h->mass_in, h->mass_out, h->gram_part, h->mom_part, h->sweeps, h->org_fit, h->view,
                    h->Wcat, h->Ipre, h->bw_lpart, h->bw_coef, h->bw_loss, h->bw_gU, h->bw_gVt,
                    h->bw_att, h->bw_gS, h->bw_G3, h->bw_gXd, h->bw_ppart, h->bw_gcell, h->bw_gXp,
                    h->bw_dwpart, h->bw_y32};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
}

size_t n_param_growth(const slime_ca_config& c) {
    return c.growth_per_cell ? (size_t)c.pods * c.G * c.G * c.H : (size_t)c.pods * c.H;
}

// Makes the handle's device current for the rest of an entry point and gives the
// caller's current device back when the entry point returns.
class DeviceScope {
  public:
    DeviceScope() = default;
    DeviceScope(const DeviceScope&) = delete;
    DeviceScope& operator=(const DeviceScope&) = delete;
    ~DeviceScope() {
        if (restore_) (void)hipSetDevice(prev_);
    }
    int enter(const slime_ca* h) {
        if (!h) return fail(SLIME_EINVAL, "handle is NULL");
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        if (prev_ != h->device) {
            HIP_TRY(hipSetDevice(h->device));
            restore_ = prev_ >= 0;
        }
        return SLIME_OK;
    }

  private:
    int prev_ = -1;
    bool restore_ = false;
};

// S1 for one step: per-batch weights (scaled by the deferred mass scale of x),
// then the projection GEMM(s).
// With `pre` (parallel projections only), I before its GELU is also written there.
int run_project(slime_ca* h, const void* x, const float* x_scale, void* P, void* I, void* V,
                hipStream_t s, void* pre = nullptr) {
    const slime_ca_config& c = h->cfg;
    const int C = h->C;
    WeightPrepArgs w{};
    w.Wtm = h->Wtm;
    w.scale = x_scale;
    w.Wt = h->Wt;
    w.B = c.B;
    w.C = C;
    w.D = c.D;
    w.per_pod = c.B / c.pods;
    w.nplanes = 3;
    w.scaled_planes = c.pvi_chain ? 1u : 7u;
    HIP_TRY(launch_weight_prep(c.dtype, w, s));

    GemmArgs g{};
    g.rows_per_batch = c.G * c.G;
    g.M = c.B * c.G * c.G;
    g.K = C;
    g.ncol = C;
    g.bt_batch_stride = 3LL * C * C;
    if (!c.pvi_chain) {
        g.A = x;
        g.Bt = h->Wt;
        g.N = 3 * C;
        g.out[0] = P;
        g.out[1] = I;
        g.out[2] = V;
        g.act[0] = 1;
        g.act[1] = 2;
        g.act[2] = 0;
        if (pre && gemm_uses_mfma(c.dtype, g)) {
            HIP_TRY(timed(h, h->gemm_ev, s, [&] { return launch_gemm_tape(c.dtype, g, pre, s); }));
        } else {
            HIP_TRY(timed(h, h->gemm_ev, s, [&] { return launch_gemm(c.dtype, g, s); }));
            if (pre) {  // I before its GELU: the W_I plane again, identity
                g.Bt = static_cast<const char*>(h->Wt) + (size_t)C * C * h->elem;
                g.N = C;
                g.out[0] = pre;
                g.act[0] = 0;
                HIP_TRY(launch_gemm(c.dtype, g, s));
            }
        }
    } else {
        if (pre) return fail(SLIME_EINVAL, "the pre-activation output needs parallel projections");
        // pvi_chain 2: P reads the 3x3 neighbourhood sum of x, held in V until V's own
        // product overwrites it. The deferred mass scale of x is per (b, head), so it
        // scales the neighbourhood sum as it scales x, and plane 0 still carries it.
        if (c.pvi_chain == 2)
            HIP_TRY(launch_neighbourhood_sum(c.dtype, x, V, c.B, c.G, C, s));
        const void* ins[3] = {c.pvi_chain == 2 ? static_cast<const void*>(V) : x, P, I};
        void* outs[3] = {P, I, V};
        const int acts[3] = {1, 2, 0};
        g.N = C;
        for (int p = 0; p < 3; ++p) {
            g.A = ins[p];
            g.Bt = static_cast<const char*>(h->Wt) + (size_t)p * C * C * h->elem;
            g.out[0] = outs[p];
            g.act[0] = acts[p];
            HIP_TRY(timed(h, h->gemm_ev, s, [&] { return launch_gemm(c.dtype, g, s); }));
        }
    }
    return SLIME_OK;
}

// S2-S6 plus the mass partials and S7 finalize: y_raw gets the unscaled output,
// out_scale the per-(b, head) conservation factor.
// loss_T, loss_part: the backward's tape step on the MFMA stencil (bf16, D = 64), which
// also sums Y^2, Y T and T^2 per (b, head, tile) into loss_part (StencilArgs).
int run_stencil(slime_ca* h, const void* x, const float* x_scale, const void* P, const void* I,
                const void* V, void* y_raw, int y_f32, float* out_scale, hipStream_t s,
                double* out_scale64 = nullptr, const void* loss_T = nullptr, double* loss_part = nullptr) {
    const slime_ca_config& c = h->cfg;
    StencilArgs a{};
    a.X = x;
    a.scale_in = x_scale;
    a.P = P;
    a.I = I;
    a.V = V;
    a.Y = y_raw;
    a.y_f32 = y_f32;
    a.K = h->K;
    a.mu = h->mu;
    a.sigma = h->sigma;
    a.M = h->M;
    a.kband = h->kband;
    a.sched = h->sched;
    a.part_in = h->part_in;
    a.part_out = h->part_out;
    a.B = c.B;
    a.G = c.G;
    a.D = c.D;
    a.per_pod = c.B / c.pods;
    a.per_cell = c.growth_per_cell;
    a.dt = c.dt;
    a.growth_fn = c.growth_fn;
    a.T = loss_T;
    a.loss_part = loss_part;
    HIP_TRY(timed(h, h->stencil_ev, s, [&] { return launch_stencil(c.dtype, a, s); }));
    if (c.conservation == 1)
        HIP_TRY(launch_cell_conserve(c.dtype, x, x_scale, y_raw, y_f32, h->part_out, c.B, c.G, c.D, s));
    HIP_TRY(launch_mass_finalize(h->part_in, h->part_out, c.B * c.H, h->tiles, h->mass_in,
                                 h->mass_out, out_scale, out_scale64, s));
    return SLIME_OK;
}


// E1-E5 over T states, state t at x_hist + t * t_stride bytes.
int run_fitness(slime_ca* h, const void* x_hist, long long t_stride, int T, float* erank,
                float* coherence, float* fitness, hipStream_t s, const double* scales = nullptr) {
    const slime_ca_config& c = h->cfg;
    const size_t BH = (size_t)c.B * c.H;
    const int chunks = fitness_chunks(c.G);
    if (chunks < 1) return fail(SLIME_EINVAL, "grid too small for the fitness pass");
    int rc = SLIME_OK;
    if (!h->gram_part || h->fit_chunks != chunks) {
        if (h->gram_part) (void)hipFree(h->gram_part);
        h->gram_part = nullptr;
        rc = dalloc_t(&h->gram_part, BH * chunks * c.D * c.D * 8);
        if (rc) return rc;
        h->fit_chunks = chunks;
    }
    if (!h->mom_part || h->fit_T < T) {
        if (h->mom_part) (void)hipFree(h->mom_part);
        h->mom_part = nullptr;
        rc = dalloc_t(&h->mom_part, BH * chunks * (size_t)T * 3 * 8);
        if (rc) return rc;
        h->fit_T = T;
    }
    h->last_stream = s;
    FitnessArgs f{};
    f.hist = x_hist;
    f.t_stride = t_stride;
    f.T = T;
    f.B = c.B;
    f.G = c.G;
    f.D = c.D;
    f.gram_part = h->gram_part;
    f.mom_part = h->mom_part;
    f.chunks = chunks;
    f.erank = erank;
    f.coh = coherence;
    f.fitness = fitness;
    f.sweeps = h->sweeps;
    f.scales = scales;
    HIP_TRY(launch_fitness(c.dtype, f, s));
    return SLIME_OK;
}

}  // namespace

extern "C" {

const char* slime_ca_last_error(void) { return g_err.c_str(); }

int slime_ca_create(const slime_ca_config* config, slime_ca** out) {
    if (!out) return fail(SLIME_EINVAL, "out is NULL");
    *out = nullptr;
    int rc = validate(config);
    if (rc) return rc;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1)
        return fail(SLIME_ENODEV, "no HIP device visible");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(SLIME_ENODEV, "device %d is %s; this library is built for gfx950", dev,
                    prop.gcnArchName);

    slime_ca* h = new slime_ca();
    h->cfg = *config;
    h->device = dev;
    const slime_ca_config& c = h->cfg;
    h->C = c.H * c.D;
    h->elem = c.dtype == SLIME_BF16 ? 2 : 4;
    h->tiles = stencil_tiles_per_batch(c.G);
    h->state_elems = (long long)c.B * c.G * c.G * h->C;
    const size_t C = h->C, BH = (size_t)c.B * c.H;
    const size_t state_bytes = (size_t)h->state_elems * h->elem;

    rc = 0;
    rc = rc ? rc : dalloc_t(&h->Wtm, (size_t)c.pods * 3 * C * C * 4);
    rc = rc ? rc : dalloc(&h->Wt, (size_t)c.B * 3 * C * C * h->elem);
    rc = rc ? rc : dalloc_t(&h->K, (size_t)c.pods * c.H * 9 * 4);
    rc = rc ? rc : dalloc_t(&h->mu, n_param_growth(c) * 4);
    rc = rc ? rc : dalloc_t(&h->sigma, n_param_growth(c) * 4);
    rc = rc ? rc : dalloc_t(&h->M, (size_t)c.pods * c.H * c.H * 4);
    if (c.dtype == SLIME_BF16 && c.D == 64) {
        rc = rc ? rc : dalloc(&h->kband, stencil_kband_bytes(c.pods));
        rc = rc ? rc : dalloc_t(&h->sched, 16 * sizeof(unsigned));
    }
    rc = rc ? rc : dalloc(&h->P, state_bytes);
    rc = rc ? rc : dalloc(&h->I, state_bytes);
    rc = rc ? rc : dalloc(&h->V, state_bytes);
    rc = rc ? rc : dalloc(&h->S[0], state_bytes);
    rc = rc ? rc : dalloc(&h->S[1], state_bytes);
    if (c.dtype == SLIME_BF16) rc = rc ? rc : dalloc_t(&h->Sf, (size_t)h->state_elems * 4);
    rc = rc ? rc : dalloc_t(&h->part_in, BH * h->tiles * 8);
    rc = rc ? rc : dalloc_t(&h->part_out, BH * h->tiles * 8);
    // scales: [2][B*H] fp32, the high parts then the low parts (scale = hi + lo)
    rc = rc ? rc : dalloc_t(&h->scale[0], 2 * BH * 4);
    rc = rc ? rc : dalloc_t(&h->scale[1], 2 * BH * 4);
    rc = rc ? rc : dalloc_t(&h->unit_scale, 2 * BH * 4);
    rc = rc ? rc : dalloc_t(&h->mass_in, BH * 8);
    rc = rc ? rc : dalloc_t(&h->mass_out, BH * 8);
    rc = rc ? rc : dalloc_t(&h->sweeps, BH * sizeof(int));
    if (rc) {
        release(h);
        delete h;
        return rc;
    }
    float* ones = new float[2 * BH];
    for (size_t i = 0; i < 2 * BH; ++i) ones[i] = i < BH ? 1.0f : 0.0f;
    hipError_t e = hipMemcpy(h->unit_scale, ones, 2 * BH * 4, hipMemcpyHostToDevice);
    delete[] ones;
    if (e == hipSuccess) e = hipMemset(h->mass_in, 0, BH * 8);
    if (e == hipSuccess) e = hipMemset(h->mass_out, 0, BH * 8);
    if (e == hipSuccess && h->sched) e = hipMemset(h->sched, 0, 16 * sizeof(unsigned));
    if (e != hipSuccess) {
        release(h);
        delete h;
        return fail(SLIME_EHIP, "initialising handle buffers: %s", hipGetErrorString(e));
    }
    *out = h;
    return SLIME_OK;
}

int slime_ca_destroy(slime_ca* h) {
    if (!h) return SLIME_OK;
    DeviceScope scope;
    (void)scope.enter(h);
    (void)hipDeviceSynchronize();
    release(h);
    delete h;
    return SLIME_OK;
}

int slime_ca_check_params(const slime_ca_config* config, const slime_ca_params* p) {
    int rc = validate(config);
    if (rc) return rc;
    if (!p || !p->WP || !p->WI || !p->WV || !p->K || !p->mu || !p->sigma || !p->M)
        return fail(SLIME_EINVAL, "a parameter pointer is NULL");
    const slime_ca_config& c = *config;
    const size_t C = (size_t)c.H * c.D, CC = C * C;
    const size_t ng = n_param_growth(c);
    const struct {
        const char* name;
        const float* v;
        size_t n;
    } arrays[] = {{"WP", p->WP, (size_t)c.pods * CC}, {"WI", p->WI, (size_t)c.pods * CC},
                  {"WV", p->WV, (size_t)c.pods * CC}, {"K", p->K, (size_t)c.pods * c.H * 9},
                  {"M", p->M, (size_t)c.pods * c.H * c.H}, {"mu", p->mu, ng},
                  {"sigma", p->sigma, ng}};
    for (const auto& a : arrays)
        for (size_t i = 0; i < a.n; ++i)
            if (!std::isfinite(a.v[i]))
                return fail(SLIME_EINVAL, "%s entry %zu is not finite", a.name, i);
    if (c.growth_fn == 1)  // the Gaussian divides by 2 sigma^2
        for (size_t i = 0; i < ng; ++i)
            if (p->sigma[i] == 0.f)
                return fail(SLIME_EINVAL, "sigma entry %zu is zero (Gaussian growth)", i);
    return SLIME_OK;
}

int slime_ca_set_params(slime_ca* h, const slime_ca_params* p) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    const slime_ca_config& c = h->cfg;
    const size_t C = h->C, CC = C * C;
    const size_t ng = n_param_growth(c);
    // Every input is checked before the first upload, so a rejected call leaves the
    // handle's parameters as they were.
    rc = slime_ca_check_params(&c, p);
    if (rc) return rc;
    // From here a failed upload leaves a mix of old and new parameters: the handle
    // refuses to step until a later call succeeds.
    h->params_set = false;
    // Masters are kept transposed, [pods][p*C + n][k], so the per-step weight
    // preparation reads and writes along k.
    {
        std::vector<float> t(3 * CC);
        for (int q = 0; q < c.pods; ++q) {
            const float* src[3] = {p->WP + (size_t)q * CC, p->WI + (size_t)q * CC,
                                   p->WV + (size_t)q * CC};
            for (int pl = 0; pl < 3; ++pl)
                for (size_t k = 0; k < C; ++k)
                    for (size_t n = 0; n < C; ++n) t[(pl * C + n) * C + k] = src[pl][k * C + n];
            HIP_TRY(hipMemcpy(h->Wtm + (size_t)q * 3 * CC, t.data(), 3 * CC * 4,
                              hipMemcpyHostToDevice));
        }
    }
    // [W_P | W_I | W_V] by input channel, for the backward's dX GEMM (uploaded by
    // slime_ca_backward when first needed).
    h->wcat_host.assign((size_t)c.pods * C * 3 * C, 0.f);
    for (int q = 0; q < c.pods; ++q) {
        const float* src[3] = {p->WP + (size_t)q * CC, p->WI + (size_t)q * CC, p->WV + (size_t)q * CC};
        for (int pl = 0; pl < 3; ++pl)
            for (size_t k = 0; k < C; ++k)
                std::memcpy(&h->wcat_host[((size_t)q * C + k) * 3 * C + pl * C], src[pl] + k * C, C * 4);
    }
    if (h->Wcat) {
        (void)hipFree(h->Wcat);
        h->Wcat = nullptr;
    }
    HIP_TRY(hipMemcpy(h->K, p->K, (size_t)c.pods * c.H * 9 * 4, hipMemcpyHostToDevice));
    if (h->kband) {
        std::vector<uint32_t> kb(stencil_kband_bytes(c.pods) / 4);
        fill_stencil_kband(p->K, c.pods, kb.data());
        HIP_TRY(hipMemcpy(h->kband, kb.data(), kb.size() * 4, hipMemcpyHostToDevice));
    }
    HIP_TRY(hipMemcpy(h->mu, p->mu, ng * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(h->sigma, p->sigma, ng * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(h->M, p->M, (size_t)c.pods * c.H * c.H * 4, hipMemcpyHostToDevice));
    h->params_set = true;
    return SLIME_OK;
}

int slime_ca_project(slime_ca* h, const void* x_in, void* P, void* I, void* V, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h->params_set) return fail(SLIME_ESTATE, "slime_ca_set_params has not been called");
    if (!x_in || !P || !I || !V) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (P == x_in || I == x_in || V == x_in || P == I || P == V || I == V)
        return fail(SLIME_EINVAL, "P, I and V must be distinct from x_in and from each other");
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    return run_project(h, x_in, nullptr, P, I, V, s);
}

int slime_ca_flow_lenia(slime_ca* h, const void* x_in, const void* P, const void* I, const void* V,
                        void* y_out, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h->params_set) return fail(SLIME_ESTATE, "slime_ca_set_params has not been called");
    if (!x_in || !P || !I || !V || !y_out) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (y_out == x_in || y_out == P || y_out == I || y_out == V)
        return fail(SLIME_EINVAL, "y_out aliases an input");
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    const slime_ca_config& c = h->cfg;
    // The output is rescaled once from an fp32 copy, so a bf16 state is rounded once.
    void* raw = h->Sf ? static_cast<void*>(h->Sf) : h->S[0];
    rc = run_stencil(h, x_in, nullptr, P, I, V, raw, h->Sf != nullptr, h->scale[0], s);
    if (rc) return rc;
    HIP_TRY(launch_rescale(c.dtype, raw, h->Sf != nullptr, h->scale[0], y_out, c.B, c.G, h->C,
                           c.D, s));
    return SLIME_OK;
}

int slime_ca_step(slime_ca* h, const void* x_in, void* x_out, int n_steps, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h->params_set) return fail(SLIME_ESTATE, "slime_ca_set_params has not been called");
    if (!x_in || !x_out) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (n_steps < 0) return fail(SLIME_EINVAL, "n_steps=%d is negative", n_steps);
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    const slime_ca_config& c = h->cfg;
    if (n_steps == 0) {
        if (x_out != x_in)
            HIP_TRY(hipMemcpyAsync(x_out, x_in, (size_t)h->state_elems * h->elem,
                                   hipMemcpyDeviceToDevice, s));
        return SLIME_OK;
    }
    const void* cur = x_in;
    const float* cur_scale = h->unit_scale;
    // Intermediate outputs stay unscaled in the storage type: the next step applies
    // the conservation factor in fp32 as it reads them. The last step writes fp32
    // (bf16 state) so the final rescale rounds once.
    int cur_f32 = 0;
    for (int i = 0; i < n_steps; ++i) {
        const bool last = i == n_steps - 1;
        const int y_f32 = last && h->Sf != nullptr;
        void* y = y_f32 ? static_cast<void*>(h->Sf) : h->S[i & 1];
        float* ys = h->scale[i & 1];
        rc = run_project(h, cur, cur_scale, h->P, h->I, h->V, s);
        if (rc) return rc;
        rc = run_stencil(h, cur, cur_scale, h->P, h->I, h->V, y, y_f32, ys, s);
        if (rc) return rc;
        cur = y;
        cur_f32 = y_f32;
        cur_scale = ys;
    }
    HIP_TRY(launch_rescale(c.dtype, cur, cur_f32, cur_scale, x_out, c.B, c.G, h->C, c.D, s));
    return SLIME_OK;
}

int slime_ca_mass(slime_ca* h, double* h_in, double* h_out) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h_in && !h_out) return fail(SLIME_EINVAL, "both outputs are NULL");
    const size_t BH = (size_t)h->cfg.B * h->cfg.H;
    HIP_TRY(hipStreamSynchronize(h->last_stream));
    std::vector<double> in(BH), out(BH);
    HIP_TRY(hipMemcpy(in.data(), h->mass_in, BH * 8, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(out.data(), h->mass_out, BH * 8, hipMemcpyDeviceToHost));
    if (h_in) std::memcpy(h_in, in.data(), BH * 8);
    if (h_out) std::memcpy(h_out, out.data(), BH * 8);
    // A NaN or Inf anywhere in a (batch, head) block reaches its fp64 sums, so they
    // report a non-finite state (the reference detects and reports failures, CUDA_CHECK
    // at slime/runtime.cu:11-20; here with a status code).
    for (size_t i = 0; i < BH; ++i)
        if (!std::isfinite(in[i]) || !std::isfinite(out[i]))
            return fail(SLIME_ENONFINITE,
                        "mass of batch %zu head %zu is not finite (in %g, out %g): the state "
                        "holds NaN or Inf",
                        i / h->cfg.H, i % h->cfg.H, in[i], out[i]);
    return SLIME_OK;
}

int slime_ca_fitness(slime_ca* h, const void* x_hist, int T, float* erank, float* coherence,
                     float* fitness, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!x_hist || !erank || !coherence || !fitness)
        return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (T < 2 || T > 65) return fail(SLIME_EINVAL, "T=%d must be in [2, 65]", T);
    return run_fitness(h, x_hist, h->state_elems * (long long)h->elem, T, erank, coherence,
                       fitness, static_cast<hipStream_t>(stream));
}

int slime_ca_rollout(slime_ca* h, void* hist, int T, double* scales, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h->params_set) return fail(SLIME_ESTATE, "slime_ca_set_params has not been called");
    if (!hist || !scales) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (T < 2 || T > 65) return fail(SLIME_EINVAL, "T=%d must be in [2, 65]", T);
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    const slime_ca_config& c = h->cfg;
    const int BH = c.B * c.H;
    const size_t state_bytes = (size_t)h->state_elems * h->elem;
    char* base = static_cast<char*>(hist);
    HIP_TRY(launch_fill_f64(scales, BH, 1.0, s));
    // Step t reads state t-1 as stored, with its factor folded into the weights and
    // the stencil's loads, and stores state t before its own rescale; the factor goes
    // to the handle (for step t+1) and to scales[t].
    const float* cur_scale = h->unit_scale;
    for (int t = 1; t < T; ++t) {
        const void* cur = base + (size_t)(t - 1) * state_bytes;
        void* y = base + (size_t)t * state_bytes;
        float* ys = h->scale[t & 1];
        rc = run_project(h, cur, cur_scale, h->P, h->I, h->V, s);
        if (rc) return rc;
        rc = run_stencil(h, cur, cur_scale, h->P, h->I, h->V, y, 0, ys, s, scales + (size_t)t * BH);
        if (rc) return rc;
        cur_scale = ys;
    }
    return SLIME_OK;
}

int slime_ca_fitness_scaled(slime_ca* h, const void* x_hist, const double* scales, int T,
                            float* erank, float* coherence, float* fitness, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!x_hist || !scales || !erank || !coherence || !fitness)
        return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (T < 2 || T > 65) return fail(SLIME_EINVAL, "T=%d must be in [2, 65]", T);
    return run_fitness(h, x_hist, h->state_elems * (long long)h->elem, T, erank, coherence,
                       fitness, static_cast<hipStream_t>(stream), scales);
}

int slime_ca_fitness_static(const slime_ca_config* config, const void* x_hist, int T, float* erank,
                            float* coherence, float* fitness, void* stream) {
    int rc = validate(config);
    if (rc) return rc;
    if (!x_hist || !erank || !coherence || !fitness)
        return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (T < 2 || T > 65) return fail(SLIME_EINVAL, "T=%d must be in [2, 65]", T);
    const slime_ca_config& c = *config;
    if (fitness_chunks(c.G) < 1) return fail(SLIME_EINVAL, "grid too small for the fitness pass");
    const int chunks = fitness_static_chunks(c.B, c.G, c.D, T);
    if (chunks < 1)
        return fail(SLIME_EINVAL,
                    "B=%d, D=%d, T=%d needs %zu bytes of partial sums, more than the %zu-byte "
                    "static scratch of slime_ca_fitness_static (use slime_ca_fitness)",
                    c.B, c.D, T, fitness_partial_bytes(c.B, c.D, T, 1), kFitnessScratchBytes);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1)
        return fail(SLIME_ENODEV, "no HIP device visible");
    FitnessArgs f{};
    f.hist = x_hist;
    f.t_stride = (long long)c.B * c.G * c.G * c.H * c.D * (c.dtype == SLIME_BF16 ? 2 : 4);
    f.T = T;
    f.B = c.B;
    f.G = c.G;
    f.D = c.D;
    f.chunks = chunks;
    f.erank = erank;
    f.coh = coherence;
    f.fitness = fitness;
    f.sweeps = nullptr;
    const hipError_t e = launch_fitness_static(c.dtype, f, static_cast<hipStream_t>(stream));
    if (e == hipErrorNoBinaryForGpu) return fail(SLIME_ENODEV, "the current device is not a gfx950");
    HIP_TRY(e);
    return SLIME_OK;
}

int slime_ca_fitness_sweeps(slime_ca* h, int* h_sweeps) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h_sweeps) return fail(SLIME_EINVAL, "output is NULL");
    HIP_TRY(hipStreamSynchronize(h->last_stream));
    HIP_TRY(hipMemcpy(h_sweeps, h->sweeps, (size_t)h->cfg.B * h->cfg.H * sizeof(int),
                      hipMemcpyDeviceToHost));
    return SLIME_OK;
}

int slime_ca_init_from_field(slime_ca* h, const float* conc, void* x, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!conc || !x) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    HIP_TRY(launch_init_from_field(h->cfg.dtype, conc, x, h->cfg.G, h->C, s));
    return SLIME_OK;
}

int slime_ca_field_from_state(slime_ca* h, const void* x, float* conc, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!conc || !x) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    HIP_TRY(launch_field_from_state(h->cfg.dtype, x, conc, h->cfg.G, h->C, s));
    return SLIME_OK;
}

int slime_ca_get_state(slime_ca* h, const void* x, float* h_buffer, int size) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!x || !h_buffer) return fail(SLIME_EINVAL, "a pointer is NULL");
    const long long cells = (long long)h->cfg.G * h->cfg.G;
    if (size < 0 || size > cells)
        return fail(SLIME_EINVAL, "size=%d is outside [0, G*G = %lld]", size, cells);
    if (size == 0) return SLIME_OK;
    if (!h->view) {
        rc = dalloc_t(&h->view, (size_t)cells * 4);
        if (rc) return rc;
    }
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(launch_field_from_state(h->cfg.dtype, x, h->view, h->cfg.G, h->C, nullptr));
    HIP_TRY(hipMemcpy(h_buffer, h->view, (size_t)size * 4, hipMemcpyDeviceToHost));
    return SLIME_OK;
}

int slime_neural_ca_update(slime_ca* h, const slime_multihead_ca_state* st, float* conc,
                           float* erank_hist, int generation, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h->params_set) return fail(SLIME_ESTATE, "slime_ca_set_params has not been called");
    if (!st || !st->ca_input || !st->ca_output || !conc || !erank_hist)
        return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    if (st->ca_input == st->ca_output)
        return fail(SLIME_EINVAL, "ca_input and ca_output must be distinct buffers");
    if (h->cfg.B != 1) return fail(SLIME_EINVAL, "the organism update needs a handle with B=1");
    if (generation < 0) return fail(SLIME_EINVAL, "generation=%d is negative", generation);
    const long long t_stride =
        static_cast<const char*>(st->ca_output) - static_cast<const char*>(st->ca_input);
    if (t_stride % (long long)h->elem)
        return fail(SLIME_EINVAL, "ca_input and ca_output are not element-aligned to each other");
    const size_t BH = (size_t)h->cfg.B * h->cfg.H;
    if (!h->org_fit) {
        rc = dalloc_t(&h->org_fit, 3 * BH * 4);
        if (rc) return rc;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;
    HIP_TRY(launch_init_from_field(h->cfg.dtype, conc, st->ca_input, h->cfg.G, h->C, s));
    rc = slime_ca_step(h, st->ca_input, st->ca_output, 1, stream);
    if (rc) return rc;
    HIP_TRY(launch_field_from_state(h->cfg.dtype, st->ca_output, conc, h->cfg.G, h->C, s));
    rc = run_fitness(h, st->ca_input, t_stride, 2, h->org_fit, h->org_fit + BH,
                     h->org_fit + 2 * BH, s);
    if (rc) return rc;
    HIP_TRY(launch_organism_report(h->mass_out, h->org_fit, h->cfg.H, st->mass_buffer,
                                   erank_hist + generation, s));
    return SLIME_OK;
}

int slime_ca_backward(slime_ca* h, const void* x_in, const void* target, float* grad_x,
                      const slime_ca_grads* grads, double* loss, void* stream) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (!h->params_set) return fail(SLIME_ESTATE, "slime_ca_set_params has not been called");
    if (!x_in || !target || !grad_x) return fail(SLIME_EINVAL, "a tensor pointer is NULL");
    const slime_ca_config& c = h->cfg;
    if (c.pvi_chain) return fail(SLIME_EINVAL, "the backward supports parallel projections only");
    if (c.growth_fn || c.conservation)
        return fail(SLIME_EINVAL, "the backward supports the bell growth and global conservation only");
    const size_t C = h->C, BH = (size_t)c.B * c.H, n = (size_t)h->state_elems;
    const size_t cells = (size_t)c.B * c.G * c.G;
    // bf16, D = 64: the tape step runs on the MFMA stencil, which sums the loss terms per
    // tile itself (no loss-partial pass)
    const bool loss_fused = c.dtype == 1 && c.D == 64;
    const int lchunks = loss_fused ? h->tiles : backward_loss_chunks(c.G);
    const int nW = 1024;  // cell-pass workgroups per pod
    const long long rows_pod = (long long)(c.B / c.pods) * c.G * c.G;
    const int dw_chunks = backward_dw_chunks_per_pod(c.dtype, (int)C, rows_pod);
    const bool want_w = grads && (grads->WP || grads->WI || grads->WV);
    // work buffers, allocated on first use
    if (!h->Wcat) {
        rc = dalloc(&h->Wcat, h->wcat_host.size() * h->elem);
        if (rc) return rc;
        if (h->elem == 2) {
            std::vector<uint16_t> wb(h->wcat_host.size());
            for (size_t i = 0; i < wb.size(); ++i) {
                uint32_t u;
                std::memcpy(&u, &h->wcat_host[i], 4);
                u += 0x7FFFu + ((u >> 16) & 1u);  // round to nearest even, as the device cvt
                wb[i] = (uint16_t)(u >> 16);
            }
            HIP_TRY(hipMemcpy(h->Wcat, wb.data(), wb.size() * 2, hipMemcpyHostToDevice));
        } else {
            HIP_TRY(hipMemcpy(h->Wcat, h->wcat_host.data(), h->wcat_host.size() * 4, hipMemcpyHostToDevice));
        }
    }
    rc = 0;
    if (!h->Ipre) rc = rc ? rc : dalloc(&h->Ipre, n * h->elem);
    if (!h->bw_lpart) rc = rc ? rc : dalloc_t(&h->bw_lpart, BH * lchunks * 3 * 8);
    if (!h->bw_coef) rc = rc ? rc : dalloc_t(&h->bw_coef, BH * 3 * 4);
    if (!h->bw_loss) rc = rc ? rc : dalloc_t(&h->bw_loss, BH * 8);
    if (!h->bw_gU) rc = rc ? rc : dalloc_t(&h->bw_gU, n * 4);
    if (!h->bw_gVt) rc = rc ? rc : dalloc_t(&h->bw_gVt, n * 4);
    if (!h->bw_att) rc = rc ? rc : dalloc_t(&h->bw_att, cells * c.H * 9 * 4);
    if (!h->bw_gS) rc = rc ? rc : dalloc_t(&h->bw_gS, cells * c.H * 9 * 4);
    if (!h->bw_G3) rc = rc ? rc : dalloc(&h->bw_G3, n * 3 * h->elem);
    if (!h->bw_gXd) rc = rc ? rc : dalloc_t(&h->bw_gXd, n * 4);
    if (!h->bw_ppart)
        rc = rc ? rc : dalloc_t(&h->bw_ppart, (size_t)c.pods * c.H * nW * backward_part_floats() * 4);
    if (c.growth_per_cell && !h->bw_gcell) rc = rc ? rc : dalloc_t(&h->bw_gcell, cells * c.H * 2 * 4);
    if (!h->bw_gXp) rc = rc ? rc : dalloc(&h->bw_gXp, n * h->elem);
    if (want_w && !h->bw_dwpart)
        rc = rc ? rc : dalloc_t(&h->bw_dwpart, (size_t)c.pods * dw_chunks * C * 3 * C * 4);
    if (!h->Sf && !h->bw_y32) rc = rc ? rc : dalloc_t(&h->bw_y32, n * 4);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    h->last_stream = s;

    // forward tape: P, I, V and I before its GELU; the unscaled fp32 output and the scale
    rc = run_project(h, x_in, nullptr, h->P, h->I, h->V, s, h->Ipre);
    if (rc) return rc;
    float* y32 = h->Sf ? h->Sf : h->bw_y32;
    float* rs = h->scale[0];
    rc = run_stencil(h, x_in, nullptr, h->P, h->I, h->V, y32, 1, rs, s, nullptr,
                     loss_fused ? target : nullptr, loss_fused ? h->bw_lpart : nullptr);
    if (rc) return rc;

    // backward through S7..S2 and the activations
    BackwardArgs a{};
    a.X = x_in;
    a.P = h->P;
    a.I = h->I;
    a.V = h->V;
    a.Ipre = h->Ipre;
    a.Y = y32;
    a.T = target;
    a.scale = rs;
    a.K = h->K;
    a.mu = h->mu;
    a.sigma = h->sigma;
    a.M = h->M;
    a.B = c.B;
    a.G = c.G;
    a.D = c.D;
    a.per_pod = c.B / c.pods;
    a.pods = c.pods;
    a.per_cell = c.growth_per_cell;
    a.dt = c.dt;
    a.inv_n = (float)(1.0 / (double)n);
    a.lpart = h->bw_lpart;
    a.lchunks = lchunks;
    a.loss_fused = loss_fused;
    a.ysum_part = h->part_out;
    a.coef = h->bw_coef;
    a.loss_bh = h->bw_loss;
    a.gU = h->bw_gU;
    a.gVt = h->bw_gVt;
    a.att = h->bw_att;
    a.gS = h->bw_gS;
    a.G3 = h->bw_G3;
    a.gXd = h->bw_gXd;
    a.ppart = h->bw_ppart;
    a.nW = nW;
    a.gcell = h->bw_gcell;
    if (grads) {
        a.gK = grads->K;
        a.gmu = grads->mu;
        a.gsigma = grads->sigma;
        a.gM = grads->M;
    }
    HIP_TRY(launch_backward_stencil(c.dtype, a, s));
    // gX += [gP~ | gI~ | gV] [W_P | W_I | W_V]^T
    {
        GemmArgs g{};
        g.A = h->bw_G3;
        g.Bt = h->Wcat;
        g.bt_batch_stride = 3LL * C * C;
        g.rows_per_batch = (int)rows_pod;
        g.M = c.B * c.G * c.G;
        g.N = (int)C;
        g.K = (int)(3 * C);
        g.ncol = (int)C;
        g.act[0] = 0;
        if (gemm_uses_mfma(c.dtype, g)) {  // grad_x = gXd + the GEMM, from its epilogue
            g.out[0] = grad_x;
            HIP_TRY(launch_gemm_add_f32(c.dtype, g, h->bw_gXd, s));
        } else {
            g.out[0] = h->bw_gXp;
            HIP_TRY(launch_gemm(c.dtype, g, s));
            HIP_TRY(launch_backward_final(c.dtype, h->bw_gXd, h->bw_gXp, grad_x, (long long)n, s));
        }
    }
    if (want_w) {
        DwArgs d{};
        d.part = h->bw_dwpart;
        d.C = (int)C;
        d.pods = c.pods;
        d.chunks_per_pod = dw_chunks;
        d.rows_per_pod = rows_pod;
        d.rows_per_chunk = backward_dw_rows_per_chunk(c.dtype, (int)C, rows_pod);
        d.gWP = grads->WP;
        d.gWI = grads->WI;
        d.gWV = grads->WV;
        HIP_TRY(launch_backward_dw(c.dtype, a, d, s));
    }
    if (loss) {
        std::vector<double> l(BH);
        HIP_TRY(hipStreamSynchronize(s));
        HIP_TRY(hipMemcpy(l.data(), h->bw_loss, BH * 8, hipMemcpyDeviceToHost));
        double tot = 0.0;
        for (double v : l) tot += v;
        *loss = tot / (double)n;
    }
    return SLIME_OK;
}

int slime_ca_set_timing(slime_ca* h, int enable) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    if (h->last_stream || h->ev_used) HIP_TRY(hipStreamSynchronize(h->last_stream));
    h->timing = enable != 0;
    h->ev_used = 0;
    h->gemm_ev.clear();
    h->stencil_ev.clear();
    return SLIME_OK;
}

int slime_ca_timings(slime_ca* h, double* gemm_ms, int* gemm_n, double* stencil_ms, int* stencil_n) {
    DeviceScope scope;
    int rc = scope.enter(h);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(h->last_stream));
    auto sum = [&](const std::vector<std::pair<size_t, size_t>>& log, double* ms, int* n) -> int {
        double tot = 0.0;
        for (const auto& pr : log) {
            float t = 0.f;
            HIP_TRY(hipEventElapsedTime(&t, h->ev_pool[pr.first], h->ev_pool[pr.second]));
            tot += t;
        }
        if (ms) *ms = tot;
        if (n) *n = (int)log.size();
        return SLIME_OK;
    };
    rc = sum(h->gemm_ev, gemm_ms, gemm_n);
    if (rc) return rc;
    return sum(h->stencil_ev, stencil_ms, stencil_n);
}

// ---- component pool -------------------------------------------------------------------
static int pool_args(const slime_pool* p, PoolArgs* a) {
    if (!p) return fail(SLIME_EINVAL, "pool is NULL");
    if (p->capacity <= 0 || p->genome_size <= 0)
        return fail(SLIME_EINVAL, "pool capacity %d and genome_size %d must be positive", p->capacity,
                    p->genome_size);
    if (!p->id || !p->fitness || !p->coherence || !p->hunger || !p->age || !p->alive || !p->genome ||
        !p->gradients || !p->counters)
        return fail(SLIME_EINVAL, "a pool array is NULL");
    *a = PoolArgs{p->capacity, p->genome_size, p->id, p->fitness, p->coherence, p->hunger,
                  p->age, p->alive, p->genome, p->gradients, p->counters};
    return SLIME_OK;
}

int slime_pool_init(const slime_pool* pool, void* stream) {
    PoolArgs a;
    if (int rc = pool_args(pool, &a)) return rc;
    HIP_TRY(launch_pool_init(a, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_pool_set_fitness(const slime_pool* pool, const float* fitness, const float* coherence, int n,
                           int heads, int generation, float* fitness_history,
                           float* coherence_history, void* stream) {
    PoolArgs a;
    if (int rc = pool_args(pool, &a)) return rc;
    if (!fitness || !coherence) return fail(SLIME_EINVAL, "fitness or coherence is NULL");
    if (n < 0 || heads <= 0 || generation < 0)
        return fail(SLIME_EINVAL, "n %d, heads %d and generation %d must be >= 0, > 0, >= 0", n, heads,
                    generation);
    if (n == 0) return SLIME_OK;
    HIP_TRY(launch_pool_set_fitness(a, fitness, coherence, n, heads, generation, fitness_history,
                                    coherence_history, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_ca_hunger(const float* coherence, float* hunger, int n, void* stream) {
    if (n < 0) return fail(SLIME_EINVAL, "n %d < 0", n);
    if (n == 0) return SLIME_OK;
    if (!coherence || !hunger) return fail(SLIME_EINVAL, "coherence or hunger is NULL");
    HIP_TRY(launch_hunger(coherence, hunger, n, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_pool_age(const slime_pool* pool, void* stream) {
    PoolArgs a;
    if (int rc = pool_args(pool, &a)) return rc;
    HIP_TRY(launch_pool_age(a, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_pool_cull(const slime_pool* pool, float fitness_threshold, float hunger_threshold,
                    void* stream) {
    PoolArgs a;
    if (int rc = pool_args(pool, &a)) return rc;
    if (!std::isfinite(fitness_threshold) || !std::isfinite(hunger_threshold))
        return fail(SLIME_EINVAL, "cull thresholds must be finite");
    HIP_TRY(launch_pool_cull(a, fitness_threshold, hunger_threshold, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_pool_spawn(const slime_pool* pool, int parent, float mutation_rate, void* stream) {
    PoolArgs a;
    if (int rc = pool_args(pool, &a)) return rc;
    if (!std::isfinite(mutation_rate)) return fail(SLIME_EINVAL, "mutation_rate must be finite");
    HIP_TRY(launch_pool_spawn(a, parent, mutation_rate, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_pool_spawn_wave(const slime_pool* pool, float probability, int generation, void* stream) {
    PoolArgs a;
    if (int rc = pool_args(pool, &a)) return rc;
    if (std::isnan(probability) || generation < 0)
        return fail(SLIME_EINVAL, "probability is NaN or generation %d < 0", generation);
    HIP_TRY(launch_pool_spawn_wave(a, probability, generation, (hipStream_t)stream));
    return SLIME_OK;
}

int slime_pool_evolve(const slime_pool* pool, const float* fitness, const float* coherence, int n,
                      int heads, int generation, float* fitness_history, float* coherence_history,
                      void* stream) {
    if (int rc = slime_pool_set_fitness(pool, fitness, coherence, n, heads, generation, fitness_history,
                                        coherence_history, stream))
        return rc;
    if (int rc = slime_pool_spawn_wave(pool, -1.0f, generation, stream)) return rc;
    return slime_pool_cull(pool, 0.8f, 0.95f, stream);
}

int slime_snapshot_json(const slime_ca* h, const float* conc, const slime_pool* pool, int generation,
                        double elapsed, char* buf, size_t cap, size_t* written) {
    if (!h || !conc || !written) return fail(SLIME_EINVAL, "NULL handle, field or length pointer");
    if (!h->params_set) return fail(SLIME_ESTATE, "parameters not set");
    if (!std::isfinite(elapsed)) return fail(SLIME_EINVAL, "elapsed is not finite");
    const slime_ca_config& c = h->cfg;
    DeviceScope scope;
    if (int rc = scope.enter(h)) return rc;
    const int n = c.G < 16 ? c.G : 16, off = (c.G - n) / 2;
    std::vector<float> sample((size_t)n * n), K((size_t)c.H * 9);
    HIP_TRY(hipMemcpy2D(sample.data(), n * sizeof(float), conc + (size_t)off * c.G + off,
                        (size_t)c.G * sizeof(float), n * sizeof(float), n, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(K.data(), h->K, K.size() * sizeof(float), hipMemcpyDeviceToHost));
    int counters[3] = {0, 0, 0}, capacity = 0;
    if (pool) {
        PoolArgs pa;
        if (int rc = pool_args(pool, &pa)) return rc;
        HIP_TRY(hipMemcpy(counters, pool->counters, sizeof counters, hipMemcpyDeviceToHost));
        capacity = pool->capacity;
    }
    std::string r;
    char tmp[96];
    auto put = [&](const char* fmt, auto... v) {
        snprintf(tmp, sizeof tmp, fmt, v...);
        r += tmp;
    };
    put("{\"gen\":%d,\"elapsed\":%.2f,", generation, elapsed);
    r += "\"chemical\":{\"concentration\":[";
    for (size_t i = 0; i < sample.size(); ++i) put(i ? ",%.4f" : "%.4f", (double)sample[i]);
    put("],\"size\":%d},", n);
    r += "\"ca\":{\"flow_kernels\":[";
    for (int hh = 0; hh < c.H; ++hh) {
        r += hh ? ",[" : "[";
        for (int k = 0; k < 9; ++k) put(k ? ",%.4f" : "%.4f", (double)K[(size_t)hh * 9 + k]);
        r += "]";
    }
    r += "]},\"agents\":[],\"voronoi\":[],\"archive\":{\"size\":0,\"elites\":[]},";
    put("\"pool\":{\"active\":%d,\"capacity\":%d,", counters[0], capacity);
    put("\"spawned\":%d,\"culled\":%d}}", counters[1], counters[2]);
    *written = r.size();
    if (!buf || cap < r.size() + 1)
        return fail(SLIME_EINVAL, "snapshot needs %zu bytes, buffer has %zu", r.size() + 1, buf ? cap : 0);
    std::memcpy(buf, r.c_str(), r.size() + 1);
    return SLIME_OK;
}

int slime_ca_uses_mfma(const slime_ca* h) {
    if (!h) return 0;
    const slime_ca_config& c = h->cfg;
    GemmArgs g{};
    g.M = c.B * c.G * c.G;
    g.N = c.pvi_chain ? h->C : 3 * h->C;
    g.K = h->C;
    g.ncol = h->C;
    g.rows_per_batch = c.G * c.G;
    return gemm_uses_mfma(c.dtype, g) ? 1 : 0;
}

}  // extern "C"
