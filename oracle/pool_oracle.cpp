// pool_oracle.cpp — CPU restatement of the component pool that consumes the CA
// fitness (hunger, ageing, culling, spawning with xorshift128+ / Box-Muller
// mutation). TEST INFRASTRUCTURE: only tests/ load it, to check
// slime_amd/csrc/pool.hip through the C ABI.
//
// Follows, in order of the functions below (paths under the reference tree):
//   init_pool_kernel            slime/memory/pool.cu:300-320
//   fitness_computation_kernel  slime/core/organism.cu:275-287 (the writes; values
//                               from the fused fitness, averaged over heads)
//   hunger_kernel               slime/kernels/warp_ca.cu:229-240
//   age_components_kernel       slime/memory/pool.cu:162-168
//   culling_kernel              slime/core/organism.cu:590-614
//   PRNGState                   slime/memory/pool.cu:33-55
//   spawn_component_kernel      slime/memory/pool.cu:57-121
//   spawn_wave_kernel           slime/core/organism.cu:557-587 (lanes in order)
//   component_evolution_kernel  slime/core/organism.cu:144-201 (without selection)
#include <cmath>
#include <cstdint>

#include "ca_oracle.h"

namespace {
constexpr uint64_t kSeedA = 0x9e3779b97f4a7c15ULL, kSeedB = 0xbf58476d1ce4e5b9ULL;

float rng_next(uint64_t* s0, uint64_t* s1) {
    uint64_t x = *s0;
    const uint64_t y = *s1;
    *s0 = y;
    x ^= x << 23;
    *s1 = x ^ y ^ (x >> 17) ^ (y >> 26);
    return (float)(*s1 + y) / 18446744073709551616.0f;
}

float rng_gaussian(uint64_t* s0, uint64_t* s1) {
    const float u1 = rng_next(s0, s1);
    const float u2 = rng_next(s0, s1);
    const float r = std::sqrt(-2.0f * std::log(u1 + 1e-10f));
    const float theta = 2.0f * 3.14159265f * u2;
    return r * std::cos(theta);
}
}  // namespace

extern "C" {

static_assert(sizeof(unsigned long long) == sizeof(uint64_t), "64-bit PRNG words");
float oracle_xorshift_next(unsigned long long* s0, unsigned long long* s1) {
    return rng_next(reinterpret_cast<uint64_t*>(s0), reinterpret_cast<uint64_t*>(s1));
}
float oracle_xorshift_gaussian(unsigned long long* s0, unsigned long long* s1) {
    return rng_gaussian(reinterpret_cast<uint64_t*>(s0), reinterpret_cast<uint64_t*>(s1));
}

void oracle_pool_init(oracle_pool* p) {
    for (int i = 0; i < p->capacity; ++i) {
        p->id[i] = -1;
        p->alive[i] = 0;
        p->fitness[i] = 0.0f;
        p->coherence[i] = 0.0f;
        p->hunger[i] = 0.5f;
        p->age[i] = 0;
        for (int j = 0; j < p->genome_size; ++j) {
            p->genome[(long long)i * p->genome_size + j] = 0.0f;
            p->gradients[(long long)i * p->genome_size + j] = 0.0f;
        }
    }
    p->counters[0] = p->counters[1] = p->counters[2] = 0;
}

void oracle_pool_set_fitness(oracle_pool* p, const float* fit, const float* coh, int n, int heads,
                             int generation, float* fit_hist, float* coh_hist) {
    for (int i = 0; i < n && i < p->capacity; ++i) {
        if (!p->alive[i]) continue;
        float f = 0.f, c = 0.f;
        for (int h = 0; h < heads; ++h) {
            f += fit[i * heads + h];
            c += coh[i * heads + h];
        }
        f /= (float)heads;
        c /= (float)heads;
        p->fitness[i] = f;
        p->coherence[i] = c;
        p->hunger[i] = 1.0f - c;
        const long long hi = (long long)generation * p->capacity + i;
        if (fit_hist) fit_hist[hi] = f;
        if (coh_hist) coh_hist[hi] = c;
    }
}

void oracle_hunger(const float* coh, float* hunger, int n) {
    for (int i = 0; i < n; ++i) hunger[i] = 1.0f - coh[i];
}

void oracle_pool_age(oracle_pool* p) {
    for (int i = 0; i < p->capacity; ++i)
        if (p->alive[i]) p->age[i] += 1;
}

void oracle_pool_cull(oracle_pool* p, float fitness_threshold, float hunger_threshold) {
    for (int i = 0; i < p->capacity; ++i) {
        if (!p->alive[i]) continue;
        if (p->fitness[i] < fitness_threshold * 0.1f || p->hunger[i] > hunger_threshold) {
            p->alive[i] = 0;
            p->counters[2] += 1;
            p->counters[0] -= 1;
        }
    }
}

void oracle_pool_spawn(oracle_pool* p, int parent, float rate) {
    if (p->counters[0] >= p->capacity) return;
    const int new_id = p->counters[1]++;
    for (int i = 0; i < p->capacity; ++i) {
        if (p->alive[i]) continue;
        p->id[i] = new_id;
        p->fitness[i] = 0.0f;
        p->coherence[i] = 0.0f;
        p->hunger[i] = 0.5f;
        p->age[i] = 0;
        p->alive[i] = 1;
        float* g = p->genome + (long long)i * p->genome_size;
        float* gr = p->gradients + (long long)i * p->genome_size;
        if (parent >= 0 && parent < p->capacity) {
            const float* pg = p->genome + (long long)parent * p->genome_size;
            const float* pgr = p->gradients + (long long)parent * p->genome_size;
            uint64_t s0 = (uint64_t)new_id * kSeedA, s1 = (uint64_t)parent * kSeedB;
            for (int j = 0; j < p->genome_size; ++j) {
                float v = pg[j];
                if (rng_next(&s0, &s1) < rate) {
                    v += rng_gaussian(&s0, &s1) * 0.1f;
                    v = std::fmax(-1.0f, std::fmin(1.0f, v));
                }
                g[j] = v;
            }
            for (int j = 0; j < p->genome_size; ++j) gr[j] = pgr[j] * 0.9f;
        } else {
            uint64_t s0 = (uint64_t)new_id * kSeedA, s1 = (uint64_t)new_id * kSeedB;
            for (int j = 0; j < p->genome_size; ++j) {
                g[j] = rng_next(&s0, &s1) * 2.0f - 1.0f;
                gr[j] = 0.0f;
            }
        }
        p->counters[0] += 1;
        return;
    }
}

// probability < 0: 0.1 exp(-active / 256), skipped unless > 0.01. The returned
// value is the probability used (0 when skipped).
float oracle_pool_spawn_wave(oracle_pool* p, float probability, int generation) {
    if (probability < 0.0f) {
        probability = 0.1f * std::exp(-(float)p->counters[0] / 256.0f);
        if (!(probability > 0.01f)) return 0.0f;
    }
    int parent = -1;
    for (int i = 0; i < p->capacity; ++i)
        if (p->alive[i] && p->fitness[i] > 0.5f) {
            parent = i;
            break;
        }
    for (int t = 0; t < 32; ++t) {
        unsigned seed = (unsigned)t * (unsigned)generation * 1337u;
        seed = seed * 1664525u + 1013904223u;
        const float u = (float)(seed & 0xFFFFFFu) / 16777216.0f;
        if (u < probability && parent >= 0) oracle_pool_spawn(p, parent, 0.01f);
    }
    return probability;
}

void oracle_pool_evolve(oracle_pool* p, const float* fit, const float* coh, int n, int heads,
                        int generation, float* fit_hist, float* coh_hist) {
    oracle_pool_set_fitness(p, fit, coh, n, heads, generation, fit_hist, coh_hist);
    oracle_pool_spawn_wave(p, -1.0f, generation);
    oracle_pool_cull(p, 0.8f, 0.95f);
}

}  // extern "C"
