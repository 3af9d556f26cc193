// pool.hip — the consumers of the CA fitness: a device pool of components with
// hunger, ageing, culling and spawning (xorshift128+ / Box-Muller mutation).
//
// Reference kernels (paths under the reference tree):
//   init_pool_kernel          slime/memory/pool.cu:300-320
//   spawn_component_kernel    slime/memory/pool.cu:57-121
//   age_components_kernel     slime/memory/pool.cu:162-168
//   hunger_kernel             slime/kernels/warp_ca.cu:229-240
//   culling_kernel            slime/core/organism.cu:590-614
//   spawn_wave_kernel         slime/core/organism.cu:557-587
//   fitness_computation_kernel's writes of fitness, coherence, hunger and the
//   per-generation histories (slime/core/organism.cu:275-287); the values come
//   from the fused CA fitness (per (pod, head), averaged over heads) instead of
//   the genome-norm proxy of :219-272.
//
// The pool is a structure of arrays (slime_pool). Spawning is inherently serial:
// the slot search and the mutation draw one PRNG stream element by element, so
// one thread runs it; the reference launches up to 32 spawn grids from one wave
// that race on the slot search and the counters, here they run in lane order.
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

// xorshift128+ (shifts 23, 17, 26) with the reference's float mapping and
// Box-Muller transform (slime/memory/pool.cu:33-55).
struct Xorshift128p {
    uint64_t s0, s1;
    __device__ float next() {
        uint64_t x = s0;
        const uint64_t y = s1;
        s0 = y;
        x ^= x << 23;
        s1 = x ^ y ^ (x >> 17) ^ (y >> 26);
        return (float)(s1 + y) / 18446744073709551616.0f;
    }
    __device__ float gaussian() {
        const float u1 = next();
        const float u2 = next();
        const float r = sqrtf(-2.0f * logf(u1 + 1e-10f));
        const float theta = 2.0f * 3.14159265f * u2;
        return r * cosf(theta);
    }
};

constexpr uint64_t kSeedA = 0x9e3779b97f4a7c15ULL, kSeedB = 0xbf58476d1ce4e5b9ULL;
constexpr int kActive = 0, kSpawned = 1, kCulled = 2;

__global__ void pool_init_kernel(PoolArgs p) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long ng = (long long)p.capacity * p.genome_size;
    if (i < ng) {
        p.genome[i] = 0.0f;
        p.gradients[i] = 0.0f;
    }
    if (i < p.capacity) {
        p.id[i] = -1;
        p.alive[i] = 0;
        p.fitness[i] = 0.0f;
        p.coherence[i] = 0.0f;
        p.hunger[i] = 0.5f;
        p.age[i] = 0;
    }
    if (i < 3) p.counters[i] = 0;
}

// Alive entry i < n takes the mean over `heads` of fitness[i*heads ..] and
// coherence[i*heads ..] (fixed order), hunger = 1 - coherence, and the history
// rows of `generation`.
__global__ void pool_set_fitness_kernel(PoolArgs p, const float* fit, const float* coh, int n, int heads,
                                        int generation, float* fit_hist, float* coh_hist) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || i >= p.capacity || !p.alive[i]) return;
    float f = 0.f, c = 0.f;
    for (int h = 0; h < heads; ++h) {
        f += fit[i * heads + h];
        c += coh[i * heads + h];
    }
    f /= (float)heads;
    c /= (float)heads;
    p.fitness[i] = f;
    p.coherence[i] = c;
    p.hunger[i] = 1.0f - c;
    const long long hi = (long long)generation * p.capacity + i;
    if (fit_hist) fit_hist[hi] = f;
    if (coh_hist) coh_hist[hi] = c;
}

__global__ void hunger_kernel(const float* coh, float* hunger, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) hunger[i] = 1.0f - coh[i];
}

__global__ void pool_age_kernel(PoolArgs p) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.capacity && p.alive[i]) p.age[i] += 1;
}

__global__ void pool_cull_kernel(PoolArgs p, float fitness_threshold, float hunger_threshold) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= p.capacity || !p.alive[i]) return;
    if (p.fitness[i] < fitness_threshold * 0.1f || p.hunger[i] > hunger_threshold) {
        p.alive[i] = 0;
        atomicAdd(p.counters + kCulled, 1);
        atomicSub(p.counters + kActive, 1);
    }
}

// One spawn (single thread): the first dead slot takes id = spawned++, zero
// fitness and coherence, hunger 0.5, age 0, and a genome inherited from `parent`
// with per-element Gaussian mutation (or uniform in [-1, 1) without a parent).
__device__ void spawn_one(const PoolArgs& p, int parent, float rate) {
    if (p.counters[kActive] >= p.capacity) return;
    const int new_id = p.counters[kSpawned]++;
    for (int i = 0; i < p.capacity; ++i) {
        if (p.alive[i]) continue;
        p.id[i] = new_id;
        p.fitness[i] = 0.0f;
        p.coherence[i] = 0.0f;
        p.hunger[i] = 0.5f;
        p.age[i] = 0;
        p.alive[i] = 1;
        float* g = p.genome + (long long)i * p.genome_size;
        float* gr = p.gradients + (long long)i * p.genome_size;
        if (parent >= 0 && parent < p.capacity) {
            const float* pg = p.genome + (long long)parent * p.genome_size;
            const float* pgr = p.gradients + (long long)parent * p.genome_size;
            Xorshift128p rng{(uint64_t)new_id * kSeedA, (uint64_t)parent * kSeedB};
            for (int j = 0; j < p.genome_size; ++j) {
                float v = pg[j];
                if (rng.next() < rate) {
                    v += rng.gaussian() * 0.1f;
                    v = fmaxf(-1.0f, fminf(1.0f, v));
                }
                g[j] = v;
            }
            for (int j = 0; j < p.genome_size; ++j) gr[j] = pgr[j] * 0.9f;
        } else {
            Xorshift128p rng{(uint64_t)new_id * kSeedA, (uint64_t)new_id * kSeedB};
            for (int j = 0; j < p.genome_size; ++j) {
                g[j] = rng.next() * 2.0f - 1.0f;
                gr[j] = 0.0f;
            }
        }
        p.counters[kActive] += 1;
        return;
    }
}

__global__ void pool_spawn_kernel(PoolArgs p, int parent, float rate) {
    if (threadIdx.x == 0 && blockIdx.x == 0) spawn_one(p, parent, rate);
}

// The 32 lanes of the reference's spawn wave, in lane order: lane t draws
// u = LCG(t * generation * 1337) and spawns from the first alive entry with
// fitness > 0.5 when u < probability. probability < 0: use the lifecycle's
// 0.1 * exp(-active / 256), and skip the wave unless it exceeds 0.01
// (slime/core/organism.cu:185-186).
__global__ void pool_spawn_wave_kernel(PoolArgs p, float probability, int generation) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    if (probability < 0.0f) {
        probability = 0.1f * expf(-(float)p.counters[kActive] / 256.0f);
        if (!(probability > 0.01f)) return;
    }
    int parent = -1;
    for (int i = 0; i < p.capacity; ++i)
        if (p.alive[i] && p.fitness[i] > 0.5f) {
            parent = i;
            break;
        }
    for (int t = 0; t < 32; ++t) {
        unsigned seed = (unsigned)t * (unsigned)generation * 1337u;
        seed = seed * 1664525u + 1013904223u;
        const float u = (float)(seed & 0xFFFFFFu) / 16777216.0f;
        if (u < probability && parent >= 0) spawn_one(p, parent, 0.01f);
    }
}

unsigned blocks_for(long long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_pool_init(const PoolArgs& p, hipStream_t s) {
    const long long n = (long long)p.capacity * p.genome_size;
    hipLaunchKernelGGL(pool_init_kernel, dim3(blocks_for(n > p.capacity ? n : p.capacity)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_pool_set_fitness(const PoolArgs& p, const float* fit, const float* coh, int n, int heads,
                                   int generation, float* fit_hist, float* coh_hist, hipStream_t s) {
    hipLaunchKernelGGL(pool_set_fitness_kernel, dim3(blocks_for(n)), dim3(256), 0, s, p, fit, coh, n, heads,
                       generation, fit_hist, coh_hist);
    return hipGetLastError();
}

hipError_t launch_hunger(const float* coh, float* hunger, int n, hipStream_t s) {
    hipLaunchKernelGGL(hunger_kernel, dim3(blocks_for(n)), dim3(256), 0, s, coh, hunger, n);
    return hipGetLastError();
}

hipError_t launch_pool_age(const PoolArgs& p, hipStream_t s) {
    hipLaunchKernelGGL(pool_age_kernel, dim3(blocks_for(p.capacity)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_pool_cull(const PoolArgs& p, float fitness_threshold, float hunger_threshold, hipStream_t s) {
    hipLaunchKernelGGL(pool_cull_kernel, dim3(blocks_for(p.capacity)), dim3(256), 0, s, p, fitness_threshold,
                       hunger_threshold);
    return hipGetLastError();
}

hipError_t launch_pool_spawn(const PoolArgs& p, int parent, float rate, hipStream_t s) {
    hipLaunchKernelGGL(pool_spawn_kernel, dim3(1), dim3(64), 0, s, p, parent, rate);
    return hipGetLastError();
}

hipError_t launch_pool_spawn_wave(const PoolArgs& p, float probability, int generation, hipStream_t s) {
    hipLaunchKernelGGL(pool_spawn_wave_kernel, dim3(1), dim3(64), 0, s, p, probability, generation);
    return hipGetLastError();
}

}  // namespace slime
