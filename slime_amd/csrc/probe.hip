// probe.hip — measured ceilings of the MI355X the library runs on, for the
// roofline figures reported beside the datasheet peaks (libslime_probe.so, used by
// `python -m slime_amd.calibrate --ceilings`; not part of the CA library):
//   * bf16 MFMA: 16 independent v_mfma_f32_32x32x16_bf16 chains per wave on
//     register-resident operands, with random or all-zero data (the matrix cores
//     draw less power, and hold a higher clock, on zeros);
//   * HBM: 16-byte-per-lane streaming read, write and copy kernels over 2 GiB.
#include <hip/hip_runtime.h>

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

}  // namespace

extern "C" {

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

}  // extern "C"
