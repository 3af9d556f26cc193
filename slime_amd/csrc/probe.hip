// probe.hip — measured ceilings of the MI355X the library runs on, for the
// roofline figures reported beside the datasheet peaks (libslime_probe.so, used by
// `python -m slime_amd.calibrate --ceilings`; not part of the CA library):
//   * bf16 MFMA: 16 independent v_mfma_f32_32x32x16_bf16 chains per wave on
//     register-resident operands, with random or all-zero data (the matrix cores
//     draw less power, and hold a higher clock, on zeros);
//   * HBM: 16-byte-per-lane streaming read, write and copy kernels over 2 GiB.
// It also checks on the device that the short fp64 division and square root of the
// Jacobi rotation (fp64.hpp) return the bits of IEEE `/` and `sqrt`.
// LDS bank probes (run under `rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT`, one
// dispatch per call): the projection GEMM's LDS access patterns, the kernel's own
// address functions (gemm_addr.hpp) beside the layouts it used before, and single-lane
// displacements of a conflict-free linear pattern, which give the bank model.
#include <hip/hip_runtime.h>

#include "fp64.hpp"
#include "gemm_addr.hpp"

#include <stdint.h>

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_v;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

__global__ __launch_bounds__(256, 1) void mfma_loop(const u32x4* src, float* out, int iters) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    u32x4 a[4], b[4];
    for (int i = 0; i < 4; ++i) {
        a[i] = src[(tid * 8 + i) & 65535];
        b[i] = src[(tid * 8 + 4 + i) & 65535];
    }
    f32x16 acc[4][4];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8_v, a[i]), __builtin_bit_cast(bf16x8_v, b[j]), acc[i][j], 0, 0, 0);
    }
    float s = 0.f;
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j)
            for (int e = 0; e < 16; ++e) s += acc[i][j][e];
    out[tid] = s;
}

__global__ __launch_bounds__(256) void hbm_read(const uint4* __restrict__ p, long long n, unsigned* out) {
    unsigned acc = 0;
    const long long stride = (long long)gridDim.x * 1024;
    for (long long i = (long long)blockIdx.x * 1024 + threadIdx.x; i + 768 < n; i += stride) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = p[i + u * 256];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x12345678u) out[0] = acc;
}

__global__ __launch_bounds__(256) void hbm_write(uint4* __restrict__ p, long long n) {
    const long long stride = (long long)gridDim.x * 1024;
    for (long long i = (long long)blockIdx.x * 1024 + threadIdx.x; i + 768 < n; i += stride) {
#pragma unroll
        for (int u = 0; u < 4; ++u) p[i + u * 256] = make_uint4((unsigned)i, u, 1, 2);
    }
}

__global__ __launch_bounds__(256) void hbm_copy(const uint4* __restrict__ s, uint4* __restrict__ d, long long n) {
    const long long stride = (long long)gridDim.x * 1024;
    for (long long i = (long long)blockIdx.x * 1024 + threadIdx.x; i + 768 < n; i += stride) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = s[i + u * 256];
#pragma unroll
        for (int u = 0; u < 4; ++u) d[i + u * 256] = v[u];
    }
}

uint32_t hash32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// splitmix64 finaliser: one 64-bit draw per (seed, index).
__device__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

// A double with a uniform 52-bit mantissa, sign from bit 63 when `sign`, and a
// binary exponent uniform in [lo, hi].
__device__ double draw(uint64_t r, int lo, int hi, bool sign) {
    const uint64_t e = (uint64_t)(1023 + lo + (int)((r >> 52) % (uint64_t)(hi - lo + 1)));
    const uint64_t bits = (sign ? (r & 0x8000000000000000ULL) : 0ULL) | (e << 52) | (r & 0xFFFFFFFFFFFFFULL);
    return __builtin_bit_cast(double, bits);
}

// Per index i: div_rn against / on (a, b) with exponents in [-60, 60], sqrt_ge1 and
// rcp_sqrt_ge1 against sqrt and 1 / sqrt on x in [1, 2^120), and the whole rotation (c, s) against its IEEE
// form on (app, aqq, apq) drawn like Gram entries, every eighth with app = aqq.
__global__ void fp64_core_check(long long n, uint64_t seed, unsigned long long* bad) {
    unsigned long long miss = 0;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        const uint64_t r0 = mix64(seed ^ (uint64_t)(4 * i)), r1 = mix64(seed ^ (uint64_t)(4 * i + 1));
        const uint64_t r2 = mix64(seed ^ (uint64_t)(4 * i + 2)), r3 = mix64(seed ^ (uint64_t)(4 * i + 3));
        const double a = draw(r0, -60, 60, true), b = draw(r1, -60, 60, true);
        if (__builtin_bit_cast(uint64_t, slime::div_rn(a, b)) != __builtin_bit_cast(uint64_t, a / b)) ++miss;
        const double x = draw(r2, 0, 119, false);
        if (__builtin_bit_cast(uint64_t, slime::sqrt_ge1(x)) != __builtin_bit_cast(uint64_t, sqrt(x))) ++miss;
        if (__builtin_bit_cast(uint64_t, slime::rcp_sqrt_ge1(x)) != __builtin_bit_cast(uint64_t, 1.0 / sqrt(x))) ++miss;
        const double app = draw(r0 ^ r3, -24, 8, false);
        const double aqq = (i % 8 == 0) ? app : draw(r1 ^ r3, -24, 8, false);
        const double apq = draw(r2 ^ (r3 << 7), -19, 8, true);  // |apq| > 1e-6 as in the solve
        double c0, s0, c1, s1;
        slime::jacobi_rotation<true>(app, aqq, apq, c0, s0);
        slime::jacobi_rotation<false>(app, aqq, apq, c1, s1);
        if (__builtin_bit_cast(uint64_t, c0) != __builtin_bit_cast(uint64_t, c1) ||
            __builtin_bit_cast(uint64_t, s0) != __builtin_bit_cast(uint64_t, s1))
            ++miss;
    }
    if (miss) atomicAdd(bad, miss);
}

typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

// One workgroup of 4 waves per CU, 256 workgroups, each running `iters` rounds of one
// access pattern over 64 KiB of LDS. kind: 0 linear 16-byte reads; 1 the GEMM's
// fragment reads (16 per round); 2 the same reads under the GEMM's earlier row
// swizzle ((r >> 1) ^ (r >> 3)) & 3; 3 the GEMM's epilogue staging writes (8 per
// round); 4 its staging reads (4 per round); 5 and 6 the earlier staging layout
// (144-byte rows, no swizzle) writes and reads. Every 8-byte write has its own
// address register, so no two are merged into one instruction.
template <int kKind>
__global__ __launch_bounds__(256) void lds_pattern(unsigned* sink, int iters) {
    using namespace slime::gemm_addr;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[65536];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 65536 / 16; i += 256) reinterpret_cast<u32x4*>(lds)[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
    __syncthreads();
    const int r32 = lane & 31, half = lane >> 5;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (int it = 0; it < iters; ++it) {
        asm volatile("" ::"v"(lds) : "memory");  // the stores are observable
        if constexpr (kKind == 0) {
#pragma unroll
            for (int j = 0; j < 16; ++j) acc += *reinterpret_cast<const u32x4*>(lds + wave * 1024 + lane * 16 + j * 4096);
        } else if constexpr (kKind == 1 || kKind == 2) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    unsigned x = frag_x_off(kk, lane, wave) + frag_block_off(q);
                    unsigned w = frag_w_off(kk, lane, wave) + frag_block_off(q) - kStageB / 2;  // inside 64 KiB
                    if constexpr (kKind == 2) {  // same rows, the earlier chunk permutation
                        const unsigned undo = (unsigned)(row_swz(r32) << 4);
                        const unsigned old = (unsigned)((((r32 >> 1) ^ (r32 >> 3)) & 3) << 4);
                        x = x ^ undo ^ old;
                        w = w ^ undo ^ old;
                    }
                    acc += *reinterpret_cast<const u32x4*>(lds + x);
                    acc += *reinterpret_cast<const u32x4*>(lds + w);
                }
        } else if constexpr (kKind == 3 || kKind == 5) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                unsigned a = kKind == 3 ? epi_w_piece(epi_w_off(wave, lane), k)
                                        : (unsigned)(wave * 32 * 144 + r32 * 144 + half * 8 + k * 16);
                asm volatile("" : "+v"(a));
                *reinterpret_cast<u32x2*>(lds + a) = u32x2{acc.x + (unsigned)it, (unsigned)k};
            }
        } else {
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const unsigned a = kKind == 4 ? epi_r_off(wave, lane) + s4 * 8 * kEpiRowB
                                              : (unsigned)(wave * 32 * 144 + ((lane >> 3) + 8 * s4) * 144 + (lane & 7) * 16);
                acc += *reinterpret_cast<const u32x4*>(lds + a);
            }
        }
    }
    asm volatile("" ::"v"(lds) : "memory");
    if (acc.x == 0xdeadbeefu) sink[0] = acc.y;
}

// One wave: every lane reads (write = 0) or writes (write = 1) its linear slot of
// `width` bytes (16 or 8), except lane `who`, which uses the slot of lane k moved by
// `delta` bytes. Conflict cycles appear when that address shares a bank group, but not
// the address, with a lane served in the same pass.
__global__ __launch_bounds__(64) void lds_pair(unsigned* sink, int iters, int width, int write, int who, int k,
                                               int delta) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[65536];
    const int lane = threadIdx.x;
    for (int i = lane; i < 65536 / 16; i += 64) reinterpret_cast<u32x4*>(lds)[i] = u32x4{(unsigned)i, 1u, 2u, 3u};
    __syncthreads();
    const unsigned off = (unsigned)((lane == who ? k * width + delta : lane * width) & 32767);
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (int it = 0; it < iters; ++it) {
        asm volatile("" ::"v"(lds) : "memory");  // the stores are observable
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            unsigned char* p = lds + off + j * 4096;
            if (width == 16 && !write) acc += *reinterpret_cast<const u32x4*>(p);
            else if (width == 16) *reinterpret_cast<u32x4*>(p) = acc + (unsigned)it;
            else if (!write) { const u32x2 v = *reinterpret_cast<const u32x2*>(p); acc.x += v.x; acc.y += v.y; }
            else *reinterpret_cast<u32x2*>(p) = u32x2{acc.x + (unsigned)it, (unsigned)j};
        }
    }
    asm volatile("" ::"v"(lds) : "memory");
    if (acc.x == 0xdeadbeefu) sink[0] = acc.y;
}

}  // namespace

extern "C" {

// LDS bank probes; 0 on success, -1 on error. slime_probe_lds_pattern runs kind 0..6
// of lds_pattern; slime_probe_lds_pair one displaced-lane pattern (width 16 or 8).
int slime_probe_lds_pattern(int kind) {
    unsigned* sink = nullptr;
    if (hipMalloc(&sink, 4) != hipSuccess) return -1;
    const dim3 g(256), b(256);
    const int iters = 500;
    switch (kind) {
        case 0: hipLaunchKernelGGL(lds_pattern<0>, g, b, 0, 0, sink, iters); break;
        case 1: hipLaunchKernelGGL(lds_pattern<1>, g, b, 0, 0, sink, iters); break;
        case 2: hipLaunchKernelGGL(lds_pattern<2>, g, b, 0, 0, sink, iters); break;
        case 3: hipLaunchKernelGGL(lds_pattern<3>, g, b, 0, 0, sink, iters); break;
        case 4: hipLaunchKernelGGL(lds_pattern<4>, g, b, 0, 0, sink, iters); break;
        case 5: hipLaunchKernelGGL(lds_pattern<5>, g, b, 0, 0, sink, iters); break;
        case 6: hipLaunchKernelGGL(lds_pattern<6>, g, b, 0, 0, sink, iters); break;
        default: (void)hipFree(sink); return -1;
    }
    const int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -1;
    (void)hipFree(sink);
    return rc;
}
int slime_probe_lds_pair(int width, int write, int who, int k, int delta) {
    if ((width != 8 && width != 16) || who < 0 || who > 63 || k < 0 || k > 63 || delta < 0 || delta > 16384) return -1;
    unsigned* sink = nullptr;
    if (hipMalloc(&sink, 4) != hipSuccess) return -1;
    hipLaunchKernelGGL(lds_pair, dim3(1), dim3(64), 0, 0, sink, 100, width, write, who, k, delta);
    const int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -1;
    (void)hipFree(sink);
    return rc;
}


// Achieved bf16 MFMA rate in TFLOP/s of a 1024-workgroup run; random != 0 fills
// the operands with finite bf16 values of magnitude < 2, else zeros. -1 on error.
double slime_probe_mfma_tflops(int random) {
    const int n = 65536 * 4, grid = 1024, iters = 2000;
    uint32_t* h = new uint32_t[n];
    for (int i = 0; i < n; ++i) h[i] = random ? (hash32((uint32_t)i) & 0xBFFFBFFFu) : 0u;
    void *src = nullptr, *out = nullptr;
    double r = -1.0;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc(&src, n * 4) == hipSuccess && hipMalloc(&out, grid * 256 * 4) == hipSuccess &&
        hipMemcpy(src, h, n * 4, hipMemcpyHostToDevice) == hipSuccess &&
        hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        hipLaunchKernelGGL(mfma_loop, dim3(grid), dim3(256), 0, 0, (const u32x4*)src, (float*)out, 10);
        (void)hipEventRecord(e0, 0);
        hipLaunchKernelGGL(mfma_loop, dim3(grid), dim3(256), 0, 0, (const u32x4*)src, (float*)out, iters);
        (void)hipEventRecord(e1, 0);
        float ms = 0.f;
        if (hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0.f)
            r = (double)grid * 4 * iters * 16 * 32768.0 / (ms * 1e-3) / 1e12;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (src) (void)hipFree(src);
    if (out) (void)hipFree(out);
    delete[] h;
    return r;
}

// Achieved HBM bandwidth in GB/s over 2 GiB buffers: kind 0 read, 1 write, 2 copy
// (read + write bytes). Best of 5 launches. -1 on error.
double slime_probe_hbm_gbs(int kind) {
    const long long bytes = 2LL << 30, n = bytes / 16;
    void *a = nullptr, *b = nullptr, *o = nullptr;
    double best = -1.0;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc(&a, bytes) == hipSuccess && hipMalloc(&b, bytes) == hipSuccess &&
        hipMalloc(&o, 64) == hipSuccess && hipMemset(a, 1, bytes) == hipSuccess &&
        hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        const int grid = 8192;
        for (int rep = 0; rep < 6; ++rep) {
            (void)hipEventRecord(e0, 0);
            if (kind == 0)
                hipLaunchKernelGGL(hbm_read, dim3(grid), dim3(256), 0, 0, (const uint4*)a, n, (unsigned*)o);
            else if (kind == 1)
                hipLaunchKernelGGL(hbm_write, dim3(grid), dim3(256), 0, 0, (uint4*)b, n);
            else
                hipLaunchKernelGGL(hbm_copy, dim3(grid), dim3(256), 0, 0, (const uint4*)a, (uint4*)b, n);
            (void)hipEventRecord(e1, 0);
            float ms = 0.f;
            if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) break;
            const double gbs = (kind == 2 ? 2.0 : 1.0) * bytes / (ms * 1e-3) / 1e9;
            if (rep > 0 && gbs > best) best = gbs;  // first launch is a warm-up
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (o) (void)hipFree(o);
    return best;
}

// Mismatches, out of 3 n comparisons, between the short fp64 division, square root
// and rotation of fp64.hpp and their IEEE forms, over n seeded draws. -1 on error.
long long slime_probe_fp64_core(long long n, unsigned long long seed) {
    unsigned long long* bad = nullptr;
    long long r = -1;
    if (n > 0 && hipMalloc(&bad, 8) == hipSuccess && hipMemset(bad, 0, 8) == hipSuccess) {
        hipLaunchKernelGGL(fp64_core_check, dim3(1024), dim3(256), 0, 0, n, (uint64_t)seed, bad);
        unsigned long long h = 0;
        if (hipGetLastError() == hipSuccess && hipMemcpy(&h, bad, 8, hipMemcpyDeviceToHost) == hipSuccess)
            r = (long long)h;
    }
    if (bad) (void)hipFree(bad);
    return r;
}

}  // extern "C"
