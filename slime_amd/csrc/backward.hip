// backward.hip — gradient of one CA step under the MSE loss (configuration c5):
// L = mean over all elements of (Y' - T)^2, Y' the conserved output of one step
// with parallel P/I/V projections.
//
// The reference declares gradients (gradients_d, update_gradients,
// slime/proto/model.cu:7,13) but never computes any; the chain rule here follows
// the forward stages S1-S7 (slime/core/pseudopod.cu:41-253 and the sources listed
// in stencil.hip), stage by stage in reverse:
//   S7  gY' = 2 (Y' - T)/N;  Q_o = sum gY' Y_o;  gY_o = r_o (gY' - Q_o/B_o) and
//       gX_o += Q_o/B_o when |B_o| > 1e-6 (B_o = sum Y_o, r_o = A_o/B_o), else gY_o = gY'
//   S6  gZ_h = sum_o M[o][h] gY_o;  gM[o][h] += sum gY_o Z_h;  gX += gZ;
//       gg = dt gZ Vt;  gVt = dt gZ g
//   S3  gU = gg (-4 t e^{-t^2}) / (sigma + 1e-7);  gmu += -gU;  gsigma += -gU t
//   S2  gX(n_k(r)) += K[h][k] gU(r);  gK[h][k] += sum gU(r) X(n_k(r))
//   S5  gV(n_k(r)) += a_k gVt(r);  ga_k = <gVt(r), V(n_k(r))>
//   S4  gs_k = a_k (ga_k - sum_j a_j ga_j);  gP(r) += sum_k gs_k I(n_k) / sqrt(D);
//       gI(n_k(r)) += gs_k P(r) / sqrt(D)
//   S1  gP~ = gP [P > 0];  gI~ = gI GELU'(I~);  gX += [gP~|gI~|gV] [W_P|W_I|W_V]^T
//       (MFMA GEMM, gemm.hip);  gW_p = X^T gp (per pod)
// Scatters run as gathers: cell q collects from the cells r = q - offset_k whose
// neighbour k it is, so no atomics are needed and every sum has a fixed order.
//
// Work split: one lane per 4 channels of a (cell, head) (8- or 16-byte loads), the
// D/4 lanes of a (cell, head) adjacent; the per-(cell, head) dot products reduce
// over those lanes with DPP moves inside a 16-lane row.
// Parameter partial sums are kept per workgroup, each workgroup owning one
// (pod, head), and added in a fixed order by the finalize kernels.
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

__device__ __forceinline__ int wrapb(int v, int G) { return v < 0 ? v + G : (v >= G ? v - G : v); }

template <typename T>
__device__ __forceinline__ float ld(const void* p, long long i) {
    return Store<T>::to_f32(static_cast<const T*>(p)[i]);
}

struct F4 {
    float v[4];
};

template <typename T>
__device__ __forceinline__ F4 ld4(const void* p, long long i) {  // i: a multiple of 4
    F4 r;
    if constexpr (sizeof(T) == 2) {
        const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const T*>(p) + i);
        r.v[0] = bf16lo(w.x);
        r.v[1] = bf16hi(w.x);
        r.v[2] = bf16lo(w.y);
        r.v[3] = bf16hi(w.y);
    } else {
        const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        r.v[0] = f.x;
        r.v[1] = f.y;
        r.v[2] = f.z;
        r.v[3] = f.w;
    }
    return r;
}
// Four channels as loaded, converted at each use: two packed bf16 pairs or four floats.
template <typename T>
using Raw4 = std::conditional_t<sizeof(T) == 2, uint2, float4>;
template <typename T>
__device__ __forceinline__ Raw4<T> ldraw4(const void* p, long long i) {
    return *reinterpret_cast<const Raw4<T>*>(static_cast<const T*>(p) + i);
}
// Element `base` of p (a wave-uniform index), then `lane_bytes` further.
template <typename T>
__device__ __forceinline__ Raw4<T> ldraw4_at(const void* p, long long base, unsigned lane_bytes) {
    const char* q = reinterpret_cast<const char*>(static_cast<const T*>(p) + base);
    return *reinterpret_cast<const Raw4<T>*>(q + lane_bytes);
}
template <typename T>
__device__ __forceinline__ float raw_at(const Raw4<T>& r, int e) {
    if constexpr (sizeof(T) == 2) {
        const unsigned w = e < 2 ? r.x : r.y;
        return (e & 1) ? bf16hi(w) : bf16lo(w);
    } else {
        return e == 0 ? r.x : e == 1 ? r.y : e == 2 ? r.z : r.w;
    }
}
// Marks the loaded values as rewritten here, so the compiler converts them again at
// the next use instead of keeping the converted floats live in between.
template <typename T>
__device__ __forceinline__ void reuse_raw(Raw4<T> (&r)[9]) {
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        if constexpr (sizeof(T) == 2) asm volatile("" : "+v"(r[k].x), "+v"(r[k].y));
        else asm volatile("" : "+v"(r[k].x), "+v"(r[k].y), "+v"(r[k].z), "+v"(r[k].w));
    }
}
__device__ __forceinline__ F4 ld4f(const float* p, long long i) {
    const float4 f = *reinterpret_cast<const float4*>(p + i);
    return F4{{f.x, f.y, f.z, f.w}};
}
__device__ __forceinline__ void st4f(float* p, long long i, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p + i) = make_float4(v[0], v[1], v[2], v[3]);
}
template <typename T>
__device__ __forceinline__ void st4(void* p, long long i, const float (&v)[4]) {
    if constexpr (sizeof(T) == 2)
        *reinterpret_cast<uint2*>(static_cast<T*>(p) + i) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    else
        *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
}

// d/dx GELU_tanh(x) = d/dx [x sigma(2u)], u = c0 (x + c1 x^3):
//   sigma + 2 x sigma (1 - sigma) u',  u' = c0 (1 + 3 c1 x^2),
// the tanh form 0.5 (1 + th) + 0.5 x (1 - th^2) u' with th = 2 sigma - 1. With
// e = exp(-2u), sigma = 1 / (1 + e) and 1 - sigma = e sigma, so nothing cancels;
// the exponent is capped at 2^126, where sigma and the second term are negligible.
__device__ __forceinline__ float gelu_grad(float x) {
    constexpr float c0 = 0.7978845608028654f, c1 = 0.044715f, kLog2e = 1.4426950408889634f;
    const float x2 = x * x;
    const float u = c0 * x * __builtin_fmaf(c1, x2, 1.0f);
    const float e = exp2_fast(fminf(-2.0f * kLog2e * u, 126.0f));
    const float sg = rcp_fast(1.0f + e);
    const float du = c0 * __builtin_fmaf(3.0f * c1, x2, 1.0f);
    return sg * __builtin_fmaf(2.0f * x * du, e * sg, 1.0f);
}

// ---- S7: loss, Q_o, B_o partial sums ---------------------------------------------------
// Block (chunk, b) covers kLossCells cells of batch b; lane t of a cell slot owns
// channels 4t .. 4t+3 (one head) and accumulates in fp64; the block then adds the
// lanes of each head in a fixed tree order.
constexpr int kLossCells = 64;

template <typename T>
__global__ __launch_bounds__(256) void bw_loss_partial_kernel(BackwardArgs a) {
    const int b = blockIdx.y, chunk = blockIdx.x;
    const int C = kHeads * a.D, lanes = C / 4;      // lanes per cell
    const int slots = 256 / lanes;                  // cells per pass (C <= 1024)
    const int slot = threadIdx.x / lanes, t = threadIdx.x % lanes;
    const int h = 4 * t / a.D;
    const long long cells = (long long)a.G * a.G;
    const double N = (double)a.B * (double)cells * C;
    const int BH = a.B * kHeads;
    const double r = (double)a.scale[b * kHeads + h] + (double)a.scale[BH + b * kHeads + h];
    double l = 0.0, q = 0.0, bs = 0.0;
    if (slot < slots) {
        for (int c0 = slot; c0 < kLossCells; c0 += slots) {
            const long long cell = (long long)chunk * kLossCells + c0;
            if (cell >= cells) break;
            const long long base = ((long long)b * cells + cell) * C + 4 * t;
            const F4 y = ld4f(a.Y, base), tv = ld4<T>(a.T, base);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double yd = y.v[e];
                const double err = r * yd - (double)tv.v[e];
                l += err * err;
                q += err * yd;
                bs += yd;
            }
        }
    }
    // per-head sums over the block: lanes of head h are (slot, t) with 4t / D == h
    __shared__ double s[3][256];
    s[0][threadIdx.x] = l;
    s[1][threadIdx.x] = q * (2.0 / N);
    s[2][threadIdx.x] = bs;
    __syncthreads();
    if (threadIdx.x < 3 * kHeads) {
        const int qq = threadIdx.x / kHeads, hh = threadIdx.x % kHeads;
        const int per_head = a.D / 4;  // lanes of one head in one slot
        double sum = 0.0;
        for (int sl = 0; sl < slots; ++sl)
            for (int u = 0; u < per_head; ++u) sum += s[qq][sl * lanes + hh * per_head + u];
        a.lpart[(((long long)b * kHeads + hh) * a.lchunks + chunk) * 3 + qq] = sum;
    }
}

// One block per (b, head): fixed-order sums of the partials (strided per lane, then
// a tree), then the S7 chain coefficients: gY = cY (gY' - cQ), and cQ is also the
// uniform direct term of gX. With loss_fused the partials are the tape stencil's
// per-tile sums A = sum Y^2, B = sum Y T, C = sum T^2 and the mass partials' sum Y,
// and with r = hi + lo: L = r^2 A - 2 r B + C, Q = (2 / N)(r A - B), each sum of
// exact fp64 products, so only fp64 rounding separates them from the direct sums.
__global__ __launch_bounds__(256) void bw_loss_finalize_kernel(BackwardArgs a) {
    const int bh = blockIdx.x;
    __shared__ double s[4][256];
    double l = 0.0, q = 0.0, bs = 0.0, ys = 0.0;
    for (int c = threadIdx.x; c < a.lchunks; c += 256) {
        const double* p = a.lpart + ((long long)bh * a.lchunks + c) * 3;
        l += p[0];
        q += p[1];
        bs += p[2];
        if (a.loss_fused) ys += a.ysum_part[(long long)bh * a.lchunks + c];
    }
    s[0][threadIdx.x] = l;
    s[1][threadIdx.x] = q;
    s[2][threadIdx.x] = bs;
    s[3][threadIdx.x] = ys;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w)
#pragma unroll
            for (int k = 0; k < 4; ++k) s[k][threadIdx.x] += s[k][threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        double ls = s[0][0], qs = s[1][0], b_s = s[2][0];
        if (a.loss_fused) {
            const double r = (double)a.scale[bh] + (double)a.scale[gridDim.x + bh];
            const double A = s[0][0], Bt = s[1][0], Ct = s[2][0];
            const double N = (double)a.B * (double)a.G * (double)a.G * (double)(kHeads * a.D);
            ls = __builtin_fma(r, __builtin_fma(r, A, -2.0 * Bt), Ct);
            qs = (2.0 / N) * __builtin_fma(r, A, -Bt);
            b_s = s[3][0];
        }
        const bool guard = fabs(b_s) > 1e-6;
        a.coef[bh * 3 + 0] = guard ? a.scale[bh] : 1.0f;
        a.coef[bh * 3 + 1] = guard ? (float)(qs / b_s) : 0.0f;
        a.coef[bh * 3 + 2] = guard ? a.scale[gridDim.x + bh] : 0.0f;
        a.loss_bh[bh] = ls;
    }
}

// ---- per (cell, head): S7, S6, S3, S5, S4 backward and the tape for the gathers ------------
// Block (pod, w) walks cells w*kCpi .. +kCpi-1 (+ stride) of the pod's batches with all
// eight heads of each cell: group g of kL = D/4 lanes owns (cell slot g / 8, head
// g % 8), a lane 4 consecutive channels (8- or 16-byte loads), and the per-(cell,
// head) dot products reduce over the group with DPP lane moves. Each lane computes
// the loss gradient gY of its own head's 4 channels once and shares it through LDS,
// where every head of the cell reads the 8 output heads it mixes from (S6). Per-thread
// parameter partials (M column h, K row h, mu, sigma) are reduced per head over the
// block and written once.
constexpr int kPartF = kHeads + 9 + 2;  // gM[o][h] (8), gK[h][k] (9), gmu, gsigma

// Sum over groups of kL adjacent lanes (kL = 2 .. 16, inside one 16-lane DPP row),
// every lane of the group receiving the sum.
template <int kL>
__device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (kL >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (kL >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (kL >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror
    if constexpr (kL >= 16) v += dpp_f32<0x140>(v); // row_mirror
    return v;
}

// bf16: four waves per SIMD (128 VGPRs; a few bytes of spill), with the loaded
// neighbours kept packed, K and M in LDS and the parameter partials in LDS.
template <typename T, int kD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 4 : 2)))
void bw_cell_kernel(BackwardArgs a) {
    constexpr int H = kHeads, C = H * kD, kL = kD / 4, kGroups = 256 / kL, kCpi = kGroups / H;
    static_assert(kL >= 2 && kL <= 16, "4 channels per lane, groups inside a DPP row");
    __shared__ __attribute__((aligned(16))) float sgy[kCpi * C];  // gY of the block's cells
    const int G = a.G;
    const long long cells = (long long)G * G;
    const int pod = blockIdx.x / a.nW;
    const int grp = threadIdx.x / kL, li = threadIdx.x % kL;
    // When a cell's 8 heads fill whole waves (kD >= 32), the cell slot is the same in
    // every lane of a wave; saying so moves the cell's index and neighbour arithmetic
    // to the scalar unit.
    const int cs = kL * H >= 64 ? __builtin_amdgcn_readfirstlane(grp / H) : grp / H, h = grp % H;
    const int c0 = 4 * li;
    // pod_cells is a multiple of kCpi (G is a multiple of 8, kCpi <= 16), so every slot
    // of an iteration is a cell and all threads of the block run the same iterations
    // (they meet at barriers).
    const long long pod_cells = (long long)a.per_pod * cells;
    // Workgroups are dealt to the 8 XCDs in turn (blockIdx % 8); XCD x walks the x-th
    // eighth of the pod's cells, its workgroups on adjacent cell pairs, so a cell's
    // neighbours (the next row included) are read from the L2 of the XCD that read
    // them last. When the eighths are not whole iterations (small grids), one band.
    const bool banded = pod_cells % (8LL * kCpi) == 0;
    const int nWx = banded ? a.nW / 8 : a.nW;
    const int wx = banded ? (blockIdx.x % a.nW) / 8 : blockIdx.x % a.nW;
    const int xcd = banded ? blockIdx.x % 8 : 0;
    const long long band = banded ? pod_cells / 8 : pod_cells;
    const float inv_sqrt_d = 1.0f / __builtin_sqrtf((float)kD);
    const float dt = a.dt;
    // The pod's 3x3 weights K[h][k] and mixing columns M[o][h], read from LDS at each
    // use (registers are what limits the waves per SIMD here).
    __shared__ float skw[H * 9], smc[H * H];
    if (threadIdx.x < H * 9) skw[threadIdx.x] = a.K[pod * H * 9 + threadIdx.x];
    else if (threadIdx.x < H * 9 + H * H) {
        const int j = threadIdx.x - H * 9, hh = j / H, o = j % H;  // smc[hh * H + o] = M[o][hh]
        smc[j] = a.M[(pod * H + o) * H + hh];
    }
    __syncthreads();
    const float* kw = skw + h * 9;
    const float* mcol = smc + h * H;
    // Each thread's parameter partials, accumulated in its own LDS column:
    // gM[o][h] (8), gK[h][k] (9), gmu, gsigma.
    __shared__ float red[kPartF][256];
#pragma unroll
    for (int q = 0; q < kPartF; ++q) red[q][threadIdx.x] = 0.f;

    for (long long i0 = (long long)wx * kCpi; i0 < band; i0 += (long long)nWx * kCpi) {
        const long long i = xcd * band + i0 + cs;
        const int b = pod * a.per_pod + (int)(i / cells);
        const long long cell = i % cells;
        const int y = (int)(cell / G), x = (int)(cell % G);
        const long long r = (long long)b * cells + cell;
        const long long ir = r * C + h * kD + c0;
        // Neighbour k's first element, and this lane's channels within a cell: a
        // wave-uniform base and a 32-bit lane offset per load.
        const unsigned lane_b = (unsigned)((h * kD + c0) * sizeof(T));
        long long nb[9];
#pragma unroll
        for (int k = 0; k < 9; ++k)
            nb[k] = ((long long)b * cells + (long long)wrapb(y + k / 3 - 1, G) * G + wrapb(x + k % 3 - 1, G)) * C;
        // ---- forward locals of head h at r (4 channels) ----
        Raw4<T> xk[9], ik[9], vk[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            xk[k] = ldraw4_at<T>(a.X, nb[k], lane_b);
            ik[k] = ldraw4_at<T>(a.I, nb[k], lane_b);
            vk[k] = ldraw4_at<T>(a.V, nb[k], lane_b);
        }
        const F4 pc = ld4<T>(a.P, ir);
        const F4 yv = ld4f(a.Y, ir), tv = ld4<T>(a.T, ir);  // output head h of this cell
        float mu, sg;
        if (a.per_cell) {
            const long long pi = ((long long)pod * cells + cell) * H + h;
            mu = a.mu[pi];
            sg = a.sigma[pi];
        } else {
            mu = a.mu[pod * H + h];
            sg = a.sigma[pod * H + h];
        }
        const float inv_sp = 1.0f / (sg + 1e-7f);
        float t[4], et[4], g[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float u = 0.f;
#pragma unroll
            for (int k = 0; k < 9; ++k) u = __builtin_fmaf(kw[k], raw_at<T>(xk[k], e), u);
            t[e] = (u - mu) * inv_sp;
            et[e] = __expf(-t[e] * t[e]);
            g[e] = 2.0f * et[e] - 1.0f;
        }
        reuse_raw<T>(ik);
        float s[9], mx = -3.0e38f;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) d = __builtin_fmaf(pc.v[e], raw_at<T>(ik[k], e), d);
            s[k] = lanes_sum<kL>(d) * inv_sqrt_d;
            mx = fmaxf(mx, s[k]);
        }
        float den = 0.f;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            s[k] = __expf(s[k] - mx);
            den += s[k];
        }
        const float rden = 1.0f / den;
        reuse_raw<T>(vk);
        float vt[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            s[k] *= rden;  // a_k
#pragma unroll
            for (int e = 0; e < 4; ++e) vt[e] = __builtin_fmaf(s[k], raw_at<T>(vk[k], e), vt[e]);
        }
        float z[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) z[e] = __builtin_fmaf(dt * g[e], vt[e], raw_at<T>(xk[4], e));
        // ---- S7 -> gY of output head h at (r, c0..c0+3), shared; S6 -> gZ_h ----
        {
            const float rs = a.scale[b * H + h], rsl = a.scale[a.B * H + b * H + h];
            const float* cf = a.coef + (b * H + h) * 3;
            const float cy = cf[0], cq = cf[1], cyl = cf[2];
            float gyo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // y = (hi + lo) raw and gY = (cy_hi + cy_lo) u, each as an fma of the
                // high part over the product of the low part, as the forward scales
                const float u = 2.0f * (__builtin_fmaf(rs, yv.v[e], rsl * yv.v[e]) - tv.v[e]) * a.inv_n - cq;
                gyo[e] = __builtin_fmaf(cy, u, cyl * u);
            }
            *reinterpret_cast<float4*>(sgy + cs * C + h * kD + c0) = make_float4(gyo[0], gyo[1], gyo[2], gyo[3]);
        }
        __syncthreads();
        float gz[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < H; ++o) {
            const float4 gq = *reinterpret_cast<const float4*>(sgy + cs * C + o * kD + c0);
            const float gy[4] = {gq.x, gq.y, gq.z, gq.w};
            const float mo = mcol[o];
            float pm = red[o][threadIdx.x];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                gz[e] = __builtin_fmaf(mo, gy[e], gz[e]);
                pm = __builtin_fmaf(gy[e], z[e], pm);
            }
            red[o][threadIdx.x] = pm;
        }
        __syncthreads();  // sgy is rewritten by the next iteration
        // ---- S6, S3 ----
        float gu[4], gvt[4], gmu_l = 0.f, gsg_l = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float gg = dt * gz[e] * vt[e];
            gvt[e] = dt * gz[e] * g[e];
            gu[e] = gg * (-4.0f * t[e] * et[e]) * inv_sp;
            gmu_l -= gu[e];
            gsg_l -= gu[e] * t[e];
        }
        if (a.per_cell) {
            const float smu = lanes_sum<kL>(gmu_l), ssg = lanes_sum<kL>(gsg_l);
            if (li == 0) {
                a.gcell[(r * H + h) * 2 + 0] = smu;
                a.gcell[(r * H + h) * 2 + 1] = ssg;
            }
        } else {
            red[H + 9][threadIdx.x] += gmu_l;
            red[H + 10][threadIdx.x] += gsg_l;
        }
        reuse_raw<T>(xk);
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            float pk = red[H + k][threadIdx.x];
#pragma unroll
            for (int e = 0; e < 4; ++e) pk = __builtin_fmaf(gu[e], raw_at<T>(xk[k], e), pk);
            red[H + k][threadIdx.x] = pk;
        }
        // ---- S5, S4 ----
        reuse_raw<T>(vk);
        float ga[9], sa = 0.f;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) d = __builtin_fmaf(gvt[e], raw_at<T>(vk[k], e), d);
            ga[k] = lanes_sum<kL>(d);
            sa = __builtin_fmaf(s[k], ga[k], sa);
        }
        reuse_raw<T>(ik);
        float gp[4] = {0.f, 0.f, 0.f, 0.f};
        float tape_a = 0.f, tape_gs = 0.f;  // kL >= 9: lane li < 9 holds a_li and gs_li
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const float gs = s[k] * (ga[k] - sa);
#pragma unroll
            for (int e = 0; e < 4; ++e) gp[e] = __builtin_fmaf(gs * inv_sqrt_d, raw_at<T>(ik[k], e), gp[e]);
            // the tape for the gathers: a_k and gs_k per (r, h)
            if constexpr (kL >= 9) {
                tape_a = k == li ? s[k] : tape_a;
                tape_gs = k == li ? gs : tape_gs;
            } else if (k % kL == li) {
                a.att[(r * H + h) * 9 + k] = s[k];
                a.gS[(r * H + h) * 9 + k] = gs;
            }
        }
        if constexpr (kL >= 9) {  // one store of each per lane instead of one per k
            if (li < 9) {
                a.att[(r * H + h) * 9 + li] = tape_a;
                a.gS[(r * H + h) * 9 + li] = tape_gs;
            }
        }
        st4f(a.gU, ir, gu);
        st4f(a.gVt, ir, gvt);
        // gP~ -> plane 0 of G3; the direct part of gX
        float gpt[4], gxd[4];
        const float cqh = a.coef[(b * H + h) * 3 + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            gpt[e] = pc.v[e] > 0.f ? gp[e] : 0.f;
            gxd[e] = gz[e] + cqh;
        }
        st4<T>(a.G3, r * 3 * C + h * kD + c0, gpt);
        st4f(a.gXd, ir, gxd);
    }
    // block reduction of the parameter partials, fixed order
    __syncthreads();
    // per head h: the threads of groups g = cs * H + h, in the order (cs, lane)
    if ((int)threadIdx.x < H * kPartF) {
        const int hh = threadIdx.x / kPartF, q = threadIdx.x % kPartF;
        float sum = 0.f;
        for (int c2 = 0; c2 < kCpi; ++c2)
#pragma unroll
            for (int l2 = 0; l2 < kL; ++l2) sum += red[q][(c2 * H + hh) * kL + l2];
        a.ppart[((long long)(pod * H + hh) * a.nW + blockIdx.x % a.nW) * kPartF + q] = sum;
    }
}

// ---- the cell pass for bf16, D = 64: neighbours staged in an LDS ring along each row ----------
// The same per-(cell, head) sums as bw_cell_kernel, in the same order, for the c5 shape.
// Instead of 27 loads per lane from L2 per iteration (three planes, nine neighbours),
// a workgroup walks whole rows of cells, two cells per iteration, and keeps the
// neighbourhood columns of X, I and V (three rows, eight heads, 9 KiB per column) in a
// ring of six column slots: the two columns of the next iteration are staged by direct
// global->LDS loads while the current one computes, so each column crosses L2 once per
// row instead of once per neighbour, and its latency is hidden. The tape stores of an
// iteration are issued after the next iteration's barrier (their values wait in
// registers), so the wait for the staged columns at an iteration's start does not wait
// for the stores just issued.
namespace ring {
constexpr int kSlots = 6;                          // column slots (prefetch distance 1)
constexpr int kRowB = 128;                         // one (cell, head) row, bf16 D = 64
constexpr int kColB = 3 * 3 * kHeads * kRowB;      // [plane X, I, V][dy][head] rows: 9 KiB
constexpr int kInstPerCol = kColB / 1024;          // direct-load instructions per column (9)
}  // namespace ring

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void bw_cell_ring_kernel(BackwardArgs a) {
    using T = bf16_t;
    constexpr int kD = 64, H = kHeads, C = H * kD, kL = kD / 4, kCpi = 256 / kL / H;  // 2 cells
    __shared__ __attribute__((aligned(16))) unsigned char sring[ring::kSlots * ring::kColB];
    __shared__ __attribute__((aligned(16))) float sgy[kCpi * C];  // gY of the iteration's cells
    __shared__ float skw[H * 9], smc[H * H];
    __shared__ float red[kPartF][256];
    const int G = a.G;
    const long long cells = (long long)G * G;
    const int pod = blockIdx.x / a.nW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = tid / kL, li = tid % kL;
    const int cs = __builtin_amdgcn_readfirstlane(grp / H), h = grp % H;  // a wave holds one cell
    const int c0 = 4 * li;
    if (tid < H * 9) skw[tid] = a.K[pod * H * 9 + tid];
    else if (tid < H * 9 + H * H) {
        const int j = tid - H * 9, hh = j / H, o = j % H;  // smc[hh * H + o] = M[o][hh]
        smc[j] = a.M[(pod * H + o) * H + hh];
    }
#pragma unroll
    for (int q = 0; q < kPartF; ++q) red[q][tid] = 0.f;
    const float* kw = skw + h * 9;
    const float* mcol = smc + h * H;
    const float inv_sqrt_d = 1.0f / __builtin_sqrtf((float)kD);
    const float dt = a.dt;
    // Rows of the pod: XCD x (workgroups are dealt to the XCDs in turn) walks the x-th
    // eighth of them, its workgroups on adjacent rows, whose staged rows overlap in its L2.
    const int rows_pod = a.per_pod * G;
    const bool banded = rows_pod % 8 == 0 && a.nW % 8 == 0;
    const int nWx = banded ? a.nW / 8 : a.nW;
    const int wx = banded ? (blockIdx.x % a.nW) / 8 : blockIdx.x % a.nW;
    const int band = banded ? rows_pod / 8 : rows_pod;
    const int band0 = banded ? (blockIdx.x % 8) * band : 0;
    const unsigned sbase = lds_addr(sring);
    const unsigned char* sr = sring;
    // tape values of the previous iteration, stored after the next iteration's barrier
    float t_gu[4], t_gvt[4], t_gpt[4], t_gxd[4], t_a = 0.f, t_gs = 0.f;
    long long t_ir = -1, t_r = 0;
    auto store_tape = [&]() {
        if (t_ir < 0) return;
        st4f(a.gU, t_ir, t_gu);
        st4f(a.gVt, t_ir, t_gvt);
        st4<T>(a.G3, t_r * 3 * C + h * kD + c0, t_gpt);
        st4f(a.gXd, t_ir, t_gxd);
        if (li < 9) {
            a.att[(t_r * H + h) * 9 + li] = t_a;
            a.gS[(t_r * H + h) * 9 + li] = t_gs;
        }
    };

    for (int row = wx; row < band; row += nWx) {
        __syncthreads();  // LDS set up; the previous row's last iteration is done with its slots
        const int rr = band0 + row;                      // row of the pod
        const int b = pod * a.per_pod + rr / G, y = rr % G;
        const long long bb = (long long)b * cells * C * 2;  // bytes to batch entry b
        const char* srcX = reinterpret_cast<const char*>(a.X) + bb;
        const char* srcI = reinterpret_cast<const char*>(a.I) + bb;
        const char* srcV = reinterpret_cast<const char*>(a.V) + bb;
        // Stage column positions p0 .. p0 + kNp - 1 (position p is column p - 1, wrapped):
        // instruction j of a column covers plane j / 3, dy = j % 3, the eight heads (8
        // lanes of 16 bytes each); wave w issues instructions w, w + 4, ...
        const unsigned lane_off = (unsigned)(((lane >> 3) * kD + (lane & 7) * 8) * 2);
        const int yrow[3] = {wrapb(y - 1, G), y, wrapb(y + 1, G)};
        auto stage = [&](auto np_c, int p0) {
            constexpr int kNp = decltype(np_c)::value;
#pragma unroll
            for (int q = 0; q < kNp * ring::kInstPerCol; ++q) {
                if (q % 4 != wave) continue;
                const int p = p0 + q / ring::kInstPerCol, j = q % ring::kInstPerCol;
                const int pl = j / 3, dy = j % 3;
                const int col = wrapb(p - 1, G);
                const unsigned voff = (unsigned)(((long long)yrow[dy] * G + col) * C * 2) + lane_off;
                const char* src = pl == 0 ? srcX : (pl == 1 ? srcI : srcV);
                dma16_lds(src, voff, sbase + (p % ring::kSlots) * ring::kColB + j * 1024);
            }
        };
        stage(std::integral_constant<int, 4>{}, 0);  // the first iteration's four columns
        // The centre values of a cell (P, Y, T; mu and sigma when per cell) are loaded
        // one iteration ahead, into registers; the row's (batch, head) factors once.
        const long long row_r = (long long)b * cells + (long long)y * G;
        auto centre_pi = [&](int x) { return ((long long)pod * cells + (long long)y * G + x) * H + h; };
        Raw4<T> n_p = ldraw4<T>(a.P, (row_r + cs) * C + h * kD + c0);
        Raw4<T> n_t = ldraw4<T>(a.T, (row_r + cs) * C + h * kD + c0);
        F4 n_y = ld4f(a.Y, (row_r + cs) * C + h * kD + c0);
        float n_mu = 0.f, n_sg = 0.f;
        if (a.per_cell) {
            n_mu = a.mu[centre_pi(cs)];
            n_sg = a.sigma[centre_pi(cs)];
        }
        const float rs = a.scale[b * H + h], rsl = a.scale[a.B * H + b * H + h];
        const float cy = a.coef[(b * H + h) * 3 + 0], cq = a.coef[(b * H + h) * 3 + 1],
                    cyl = a.coef[(b * H + h) * 3 + 2];
        const float pod_mu = a.mu[pod * H + h], pod_sg = a.sigma[pod * H + h];
        for (int i = 0; i < G / 2; ++i) {
            const int x0 = 2 * i;
            wait_vm0();  // this wave's staging of the iteration's columns has landed
            __syncthreads();   // ... and every wave's; iteration i - 1 is done with its slots
            const Raw4<T> p_raw = n_p, t_raw = n_t;
            const F4 yv = n_y;
            const float mu = a.per_cell ? n_mu : pod_mu, sg = a.per_cell ? n_sg : pod_sg;
            store_tape();
            if (i + 1 < G / 2) {
                stage(std::integral_constant<int, 2>{}, x0 + 4);  // the next iteration's two new columns
                const long long in = (row_r + x0 + 2 + cs) * C + h * kD + c0;
                n_p = ldraw4<T>(a.P, in);
                n_t = ldraw4<T>(a.T, in);
                n_y = ld4f(a.Y, in);
                if (a.per_cell) {
                    n_mu = a.mu[centre_pi(x0 + 2 + cs)];
                    n_sg = a.sigma[centre_pi(x0 + 2 + cs)];
                }
            }
            const int x = x0 + cs;
            const long long r = row_r + x;
            const long long ir = r * C + h * kD + c0;
            // ---- forward locals of head h at r (4 channels) ----
            Raw4<T> xk[9], ik[9], vk[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const int dy = k / 3, dx = k % 3;  // neighbour (y + dy - 1, x + dx - 1)
                const unsigned char* base =
                    sr + ((x + dx) % ring::kSlots) * ring::kColB + (dy * H + h) * ring::kRowB + c0 * 2;
                xk[k] = *reinterpret_cast<const Raw4<T>*>(base);
                ik[k] = *reinterpret_cast<const Raw4<T>*>(base + 3 * H * ring::kRowB);
                vk[k] = *reinterpret_cast<const Raw4<T>*>(base + 6 * H * ring::kRowB);
            }
            const F4 pc{{raw_at<T>(p_raw, 0), raw_at<T>(p_raw, 1), raw_at<T>(p_raw, 2), raw_at<T>(p_raw, 3)}};
            const F4 tv{{raw_at<T>(t_raw, 0), raw_at<T>(t_raw, 1), raw_at<T>(t_raw, 2), raw_at<T>(t_raw, 3)}};
            const float inv_sp = 1.0f / (sg + 1e-7f);
            float t[4], et[4], g[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float u = 0.f;
#pragma unroll
                for (int k = 0; k < 9; ++k) u = __builtin_fmaf(kw[k], raw_at<T>(xk[k], e), u);
                t[e] = (u - mu) * inv_sp;
                et[e] = __expf(-t[e] * t[e]);
                g[e] = 2.0f * et[e] - 1.0f;
            }
            float s[9], mx = -3.0e38f;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) d = __builtin_fmaf(pc.v[e], raw_at<T>(ik[k], e), d);
                s[k] = lanes_sum<kL>(d) * inv_sqrt_d;
                mx = fmaxf(mx, s[k]);
            }
            float den = 0.f;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                s[k] = __expf(s[k] - mx);
                den += s[k];
            }
            const float rden = 1.0f / den;
            float vt[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                s[k] *= rden;  // a_k
#pragma unroll
                for (int e = 0; e < 4; ++e) vt[e] = __builtin_fmaf(s[k], raw_at<T>(vk[k], e), vt[e]);
            }
            float z[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) z[e] = __builtin_fmaf(dt * g[e], vt[e], raw_at<T>(xk[4], e));
            // ---- S7 -> gY of output head h at (r, c0..c0+3), shared; S6 -> gZ_h ----
            {
                float gyo[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float u = 2.0f * (__builtin_fmaf(rs, yv.v[e], rsl * yv.v[e]) - tv.v[e]) * a.inv_n - cq;
                    gyo[e] = __builtin_fmaf(cy, u, cyl * u);
                }
                *reinterpret_cast<float4*>(sgy + cs * C + h * kD + c0) = make_float4(gyo[0], gyo[1], gyo[2], gyo[3]);
            }
            __syncthreads();  // the next iteration's first barrier orders sgy's next writes
            float gz[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int o = 0; o < H; ++o) {
                const float4 gq = *reinterpret_cast<const float4*>(sgy + cs * C + o * kD + c0);
                const float gy[4] = {gq.x, gq.y, gq.z, gq.w};
                const float mo = mcol[o];
                float pm = red[o][tid];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    gz[e] = __builtin_fmaf(mo, gy[e], gz[e]);
                    pm = __builtin_fmaf(gy[e], z[e], pm);
                }
                red[o][tid] = pm;
            }
            // ---- S6, S3 ----
            float gu[4], gvt[4], gmu_l = 0.f, gsg_l = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float gg = dt * gz[e] * vt[e];
                gvt[e] = dt * gz[e] * g[e];
                gu[e] = gg * (-4.0f * t[e] * et[e]) * inv_sp;
                gmu_l -= gu[e];
                gsg_l -= gu[e] * t[e];
            }
            if (a.per_cell) {
                const float smu = lanes_sum<kL>(gmu_l), ssg = lanes_sum<kL>(gsg_l);
                if (li == 0) {
                    a.gcell[(r * H + h) * 2 + 0] = smu;
                    a.gcell[(r * H + h) * 2 + 1] = ssg;
                }
            } else {
                red[H + 9][tid] += gmu_l;
                red[H + 10][tid] += gsg_l;
            }
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                float pk = red[H + k][tid];
#pragma unroll
                for (int e = 0; e < 4; ++e) pk = __builtin_fmaf(gu[e], raw_at<T>(xk[k], e), pk);
                red[H + k][tid] = pk;
            }
            // ---- S5, S4 ----
            float ga[9], sa = 0.f;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) d = __builtin_fmaf(gvt[e], raw_at<T>(vk[k], e), d);
                ga[k] = lanes_sum<kL>(d);
                sa = __builtin_fmaf(s[k], ga[k], sa);
            }
            float gp[4] = {0.f, 0.f, 0.f, 0.f};
            float tape_a = 0.f, tape_gs = 0.f;  // lane li < 9 holds a_li and gs_li
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const float gs = s[k] * (ga[k] - sa);
#pragma unroll
                for (int e = 0; e < 4; ++e) gp[e] = __builtin_fmaf(gs * inv_sqrt_d, raw_at<T>(ik[k], e), gp[e]);
                tape_a = k == li ? s[k] : tape_a;
                tape_gs = k == li ? gs : tape_gs;
            }
            // the tape waits in registers until the next iteration's barrier
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                t_gu[e] = gu[e];
                t_gvt[e] = gvt[e];
                t_gpt[e] = pc.v[e] > 0.f ? gp[e] : 0.f;
                t_gxd[e] = gz[e] + cq;
            }
            t_a = tape_a;
            t_gs = tape_gs;
            t_ir = ir;
            t_r = r;
        }
    }
    __syncthreads();
    store_tape();
    // block reduction of the parameter partials, fixed order: per head h, the threads of
    // groups g = cs * H + h, in the order (cs, lane)
    if (tid < H * kPartF) {
        const int hh = tid / kPartF, q = tid % kPartF;
        float sum = 0.f;
        for (int c2 = 0; c2 < kCpi; ++c2)
#pragma unroll
            for (int l2 = 0; l2 < kL; ++l2) sum += red[q][(c2 * H + hh) * kL + l2];
        a.ppart[((long long)(pod * H + hh) * a.nW + blockIdx.x % a.nW) * kPartF + q] = sum;
    }
}

// ---- gathers: gV, gI~ (planes 2 and 1 of G3) and the potential's transpose -------------------
// One lane per 4 channels of one (cell q, head): cell q collects from the 9 cells
// r = q - offset_k whose neighbour k it is.
template <typename T, int kD>
__global__ __launch_bounds__(256) void bw_gather_kernel(BackwardArgs a) {
    constexpr int H = kHeads, C = H * kD;
    const int G = a.G;
    // Element offsets fit in 32 bits: the state holds at most 4e9 elements.
    const unsigned cells = (unsigned)G * (unsigned)G;
    const unsigned e4 = blockIdx.x * 256u + threadIdx.x;  // 4-channel unit
    if ((unsigned long long)e4 * 4 >= (unsigned long long)a.B * cells * C) return;
    const unsigned e = e4 * 4;
    const unsigned q = e4 / (C / 4);
    const int ch = (int)(e4 % (C / 4)) * 4, h = ch / kD;
    const unsigned b = q / cells;
    const unsigned cell = q - b * cells;
    const int y = (int)(cell / (unsigned)G), x = (int)(cell - (unsigned)y * (unsigned)G);
    const int pod = (int)b / a.per_pod;
    const float inv_sqrt_d = 1.0f / __builtin_sqrtf((float)kD);
    // All 9 neighbours' loads are issued before any use, so they are in flight together:
    // the empty asm statements (memory clobber) keep every load above them and take
    // the loaded registers as operands, so no arithmetic starts before the last load.
    float ak[9], gs[9], kw[9];
    f32x4 gvt[9], gu[9];
    u32x2 prw[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const unsigned r = b * cells + (unsigned)(wrapb(y - (k / 3 - 1), G) * G + wrapb(x - (k % 3 - 1), G));
        const unsigned ir = r * C + ch;
        const unsigned long long ai = ((unsigned long long)r * H + h) * 9 + k;  // may pass 2^32
        kw[k] = a.K[(pod * H + h) * 9 + k];
        ak[k] = a.att[ai];
        gs[k] = a.gS[ai];
        gvt[k] = *reinterpret_cast<const f32x4*>(a.gVt + ir);
        gu[k] = *reinterpret_cast<const f32x4*>(a.gU + ir);
        if constexpr (sizeof(T) == 2)
            prw[k] = *reinterpret_cast<const u32x2*>(static_cast<const T*>(a.P) + ir);
    }
    const F4 ip = ld4<T>(a.Ipre, e);
    const F4 gd = ld4f(a.gXd, e);
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        if constexpr (sizeof(T) == 2)
            asm volatile("" : "+v"(gvt[k]), "+v"(gu[k]), "+v"(prw[k]), "+v"(ak[k]), "+v"(gs[k]), "+v"(kw[k])::"memory");
        else
            asm volatile("" : "+v"(gvt[k]), "+v"(gu[k]), "+v"(ak[k]), "+v"(gs[k]), "+v"(kw[k])::"memory");
    }
    float gv[4] = {0.f, 0.f, 0.f, 0.f}, gi[4] = {0.f, 0.f, 0.f, 0.f}, gx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        F4 pr;
        if constexpr (sizeof(T) == 2) {
            pr = F4{{bf16lo(prw[k].x), bf16hi(prw[k].x), bf16lo(prw[k].y), bf16hi(prw[k].y)}};
        } else {
            const unsigned r = b * cells + (unsigned)(wrapb(y - (k / 3 - 1), G) * G + wrapb(x - (k % 3 - 1), G));
            pr = ld4<T>(a.P, r * C + ch);
        }
        const float gsk = gs[k] * inv_sqrt_d;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            gv[j] = __builtin_fmaf(ak[k], gvt[k][j], gv[j]);
            gi[j] = __builtin_fmaf(gsk, pr.v[j], gi[j]);
            gx[j] = __builtin_fmaf(kw[k], gu[k][j], gx[j]);
        }
    }
    float g1[4], gxd[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        g1[j] = gi[j] * gelu_grad(ip.v[j]);
        gxd[j] = gd.v[j] + gx[j];
    }
    const long long g3 = (long long)q * 3 * C + ch;  // G3 holds three planes: past 2^32
    st4<T>(a.G3, g3 + C, g1);
    st4<T>(a.G3, g3 + 2 * C, gv);
    st4f(a.gXd, e, gxd);
}

// ---- gathers for D = 64 through an LDS halo tile -----------------------------------------------
// The same sums as bw_gather_kernel, in the same order (k = 0..8), for one 4 x 8 cell
// tile of one (batch, head) per workgroup: the tile's 6 x 10 halo of gVt, gU (fp32),
// P (storage type) and the tape (a_k, gs_k) is read into LDS once, so each halo value
// crosses L2 once per tile instead of once per neighbour that uses it. Thread t owns
// cell t / 8 of the tile and channels 4 (t % 8) .. +3 and 32 + 4 (t % 8) .. +3; the
// eight lanes of a cell read one 128-byte half of a staged row per 16-byte read,
// cells of even column the first half first, cells of odd column the second. Under
// the LDS model of gfx950 (16 groups of 16 bytes, four 16-lane passes per wave of
// quads {0,3,5,6}, {1,2,4,7}, {9,10,12,15}, {8,11,13,14}), every pass then reads
// 16 distinct groups of unpadded 256-byte rows.
constexpr int kGTy = 4, kGTx = 8, kGHx = kGTx + 2, kGHalo = (kGTy + 2) * kGHx;  // 60 halo cells
constexpr int kGRowF = 64;  // floats per staged fp32 row

template <typename T>
__global__ __launch_bounds__(256) void bw_gather_tile_kernel(BackwardArgs a) {
    constexpr int H = kHeads, kD = 64, C = H * kD;
    __shared__ __attribute__((aligned(16))) float sV[kGHalo * kGRowF];   // gVt
    __shared__ __attribute__((aligned(16))) float sU[kGHalo * kGRowF];   // gU
    __shared__ __attribute__((aligned(16))) float sP[kGHalo * kGRowF];   // P, widened
    __shared__ float sA[kGHalo * 9], sS[kGHalo * 9];                     // a_k, gs_k
    const int G = a.G;
    const int tiles_x = G / kGTx, tpb = (G / kGTy) * tiles_x;
    const int h = blockIdx.x % H;
    const int tile = (blockIdx.x / H) % tpb;
    const int b = blockIdx.x / (H * tpb);
    const int ty0 = (tile / tiles_x) * kGTy, tx0 = (tile % tiles_x) * kGTx;
    const long long cells = (long long)G * G;
    const long long bcell = (long long)b * cells;
    const int tid = threadIdx.x;
    // ---- stage the halo: 60 cells x 64 channels, 4 channels per lane-step (the first
    // three steps cover every lane, so their loads are in flight together) ----
#pragma unroll
    for (int it = 0; it < (kGHalo * (kD / 4) + 255) / 256; ++it) {
        const int e = tid + 256 * it;
        if (256 * (it + 1) > kGHalo * (kD / 4) && e >= kGHalo * (kD / 4)) break;
        const int hc = e / (kD / 4), c4 = (e % (kD / 4)) * 4;
        const int gy = wrapb(ty0 + hc / kGHx - 1, G), gx = wrapb(tx0 + hc % kGHx - 1, G);
        const long long ir = (bcell + (long long)gy * G + gx) * C + h * kD + c4;
        *reinterpret_cast<float4*>(sV + hc * kGRowF + c4) = *reinterpret_cast<const float4*>(a.gVt + ir);
        *reinterpret_cast<float4*>(sU + hc * kGRowF + c4) = *reinterpret_cast<const float4*>(a.gU + ir);
        const F4 pv = ld4<T>(a.P, ir);
        *reinterpret_cast<float4*>(sP + hc * kGRowF + c4) = make_float4(pv.v[0], pv.v[1], pv.v[2], pv.v[3]);
    }
    for (int e = tid; e < kGHalo * 9; e += 256) {
        const int hc = e / 9, k = e % 9;
        const int gy = wrapb(ty0 + hc / kGHx - 1, G), gx = wrapb(tx0 + hc % kGHx - 1, G);
        const long long ai = ((bcell + (long long)gy * G + gx) * H + h) * 9 + k;
        sA[e] = a.att[ai];
        sS[e] = a.gS[ai];
    }
    const int cell = tid / 8;
    const int cy = cell / kGTx, cx = cell % kGTx;
    // this lane's channels: fa .. fa+3 (first read of a row) and fb .. fb+3 (second)
    const int fa = 4 * (tid % 8) + 32 * (cx & 1), fb = fa ^ 32;
    const long long q = bcell + (long long)(ty0 + cy) * G + tx0 + cx;
    const long long e0 = q * C + h * kD;
    const F4 ip0 = ld4<T>(a.Ipre, e0 + fa), ip1 = ld4<T>(a.Ipre, e0 + fb);
    const F4 gd0 = ld4f(a.gXd, e0 + fa), gd1 = ld4f(a.gXd, e0 + fb);
    const int pod = b / a.per_pod;
    float kw[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) kw[k] = a.K[(pod * H + h) * 9 + k];
    __syncthreads();
    const float inv_sqrt_d = 1.0f / __builtin_sqrtf((float)kD);
    float gv[8], gi[8], gx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) gv[j] = gi[j] = gx[j] = 0.f;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        // r = q - offset_k: halo cell (cy + 1 - dy_k, cx + 1 - dx_k)
        const int hc = (cy + 1 - (k / 3 - 1)) * kGHx + (cx + 1 - (k % 3 - 1));
        const float ak = sA[hc * 9 + k], gs = sS[hc * 9 + k] * inv_sqrt_d;
        const float4 v0 = *reinterpret_cast<const float4*>(sV + hc * kGRowF + fa);
        const float4 v1 = *reinterpret_cast<const float4*>(sV + hc * kGRowF + fb);
        const float4 p0 = *reinterpret_cast<const float4*>(sP + hc * kGRowF + fa);
        const float4 p1 = *reinterpret_cast<const float4*>(sP + hc * kGRowF + fb);
        const float4 u0 = *reinterpret_cast<const float4*>(sU + hc * kGRowF + fa);
        const float4 u1 = *reinterpret_cast<const float4*>(sU + hc * kGRowF + fb);
        const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            gv[j] = __builtin_fmaf(ak, vv[j], gv[j]);
            gi[j] = __builtin_fmaf(gs, pp[j], gi[j]);
            gx[j] = __builtin_fmaf(kw[k], uu[j], gx[j]);
        }
    }
    const float ipv[8] = {ip0.v[0], ip0.v[1], ip0.v[2], ip0.v[3], ip1.v[0], ip1.v[1], ip1.v[2], ip1.v[3]};
    const float gdv[8] = {gd0.v[0], gd0.v[1], gd0.v[2], gd0.v[3], gd1.v[0], gd1.v[1], gd1.v[2], gd1.v[3]};
    float g1a[4], g1b[4], gva[4], gvb[4], gxa[4], gxb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        g1a[j] = gi[j] * gelu_grad(ipv[j]);
        g1b[j] = gi[j + 4] * gelu_grad(ipv[j + 4]);
        gva[j] = gv[j];
        gvb[j] = gv[j + 4];
        gxa[j] = gdv[j] + gx[j];
        gxb[j] = gdv[j + 4] + gx[j + 4];
    }
    const long long g3 = q * 3 * C + h * kD;
    st4<T>(a.G3, g3 + C + fa, g1a);
    st4<T>(a.G3, g3 + C + fb, g1b);
    st4<T>(a.G3, g3 + 2 * C + fa, gva);
    st4<T>(a.G3, g3 + 2 * C + fb, gvb);
    st4f(a.gXd, e0 + fa, gxa);
    st4f(a.gXd, e0 + fb, gxb);
}

// ---- parameter finalize: fixed-order sums of the per-block partials ----------------------------
__global__ __launch_bounds__(256) void bw_param_finalize_kernel(BackwardArgs a) {
    // one block per (pod, head, quantity): thread t adds partials t, t + 256, ... in
    // order, then a fixed tree adds the 256 sums
    __shared__ float sm[256];
    const int idx = blockIdx.x;
    const int q = idx % kPartF, h = (idx / kPartF) % kHeads, pod = idx / (kPartF * kHeads);
    const float* src = a.ppart + (long long)(pod * kHeads + h) * a.nW * kPartF + q;
    float sum = 0.f;
    for (int w = threadIdx.x; w < a.nW; w += 256) sum += src[(long long)w * kPartF];
    sm[threadIdx.x] = sum;
    __syncthreads();
    for (int s2 = 128; s2 > 0; s2 >>= 1) {
        if ((int)threadIdx.x < s2) sm[threadIdx.x] += sm[threadIdx.x + s2];
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    sum = sm[0];
    if (q < kHeads) {
        if (a.gM) a.gM[(pod * kHeads + q) * kHeads + h] = sum;  // gM[o = q][h]
    } else if (q < kHeads + 9) {
        if (a.gK) a.gK[(pod * kHeads + h) * 9 + (q - kHeads)] = sum;
    } else if (!a.per_cell) {
        float* dst = q == kHeads + 9 ? a.gmu : a.gsigma;
        if (dst) dst[pod * kHeads + h] = sum;
    }
}

// per-cell growth parameters: sum over the pod's batches
__global__ __launch_bounds__(256) void bw_cell_param_finalize_kernel(BackwardArgs a) {
    const long long cells = (long long)a.G * a.G;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;  // (pod, cell, h)
    if (idx >= (long long)a.pods * cells * kHeads) return;
    const int pod = (int)(idx / (cells * kHeads));
    const long long ch = idx % (cells * kHeads);
    float smu = 0.f, ssg = 0.f;
    for (int j = 0; j < a.per_pod; ++j) {
        const long long r = (long long)(pod * a.per_pod + j) * cells * kHeads + ch;
        smu += a.gcell[r * 2 + 0];
        ssg += a.gcell[r * 2 + 1];
    }
    if (a.gmu) a.gmu[idx] = smu;
    if (a.gsigma) a.gsigma[idx] = ssg;
}

// ---- weight gradients gW_p[pod][k][j] = sum over the pod's rows of X[r][k] G_p[r][j] ----------
// Block (k tile, j tile, chunk): a 64 x 64 output tile over kWRows rows, 4 x 4
// per thread, operands staged through LDS 16 rows at a time; chunks are added in
// order by bw_dw_reduce_kernel.
constexpr int kWRows = 4096;

template <typename T>
__global__ __launch_bounds__(256) void bw_dw_partial_kernel(BackwardArgs a, DwArgs d) {
    const int C = d.C, N3 = 3 * C;
    const int kt = blockIdx.x, jt = blockIdx.y, chunk = blockIdx.z;
    const long long rows = d.rows_per_pod;
    const int pod = chunk / d.chunks_per_pod;
    const long long r0 = (long long)pod * rows + (long long)(chunk % d.chunks_per_pod) * d.rows_per_chunk;
    const long long r1 = min(r0 + d.rows_per_chunk, (long long)(pod + 1) * rows);
    __shared__ float sx[16][64], sg[16][64];
    const int tk = (threadIdx.x / 16) * 4, tj = (threadIdx.x % 16) * 4;
    float acc[4][4] = {};
    for (long long rb = r0; rb < r1; rb += 16) {
        for (int e = threadIdx.x; e < 16 * 64; e += 256) {
            const int rr = e / 64, cc = e % 64;
            const long long r = rb + rr;
            sx[rr][cc] = r < r1 ? ld<T>(a.X, r * C + kt * 64 + cc) : 0.f;
            sg[rr][cc] = r < r1 ? ld<T>(a.G3, r * N3 + jt * 64 + cc) : 0.f;
        }
        __syncthreads();
#pragma unroll 4
        for (int rr = 0; rr < 16; ++rr)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(sx[rr][tk + i], sg[rr][tj + j], acc[i][j]);
        __syncthreads();
    }
    float* out = d.part + (long long)chunk * C * N3;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) out[(long long)(kt * 64 + tk + i) * N3 + jt * 64 + tj + j] = acc[i][j];
}

// bf16: the same partial sums on the matrix cores. Block (k tile, j tile, chunk):
// a 128 x 128 output tile over rows_per_chunk rows in steps of 32, wave (wk, wj)
// owning 64 x 64 as 4 x 4 v_mfma_f32_16x16x32_bf16 blocks. Both operands are
// column slices of row-major tiles -- out[k][j] = sum_r X[r][k] G[r][j] -- staged
// as [32 rows][128 columns] (256-byte rows) by direct global->LDS loads through a
// 4-stage ring (three steps in flight), and read with ds_read_b64_tr_b16: in a
// 16-lane group, lane j reads 4 columns of row rbase + j / 4, and lane i then holds
// column i of rows rbase .. rbase + 3, the MFMA operand layout (8 consecutive rows
// of one column per lane, two reads). The 16-byte chunks of row r sit at chunk ^
// 2 (r % 4) ^ 8 ((r / 8) % 2): the four rows of a 16-lane group's read fall in
// disjoint banks, and so do the groups, whose rows are 8 apart.
constexpr int kDwT = 128, kDwStep = 32, kDwRowB = 2 * kDwT, kDwStages = 4;
constexpr int kDwStageB = 2 * kDwStep * kDwRowB;  // X and G tiles, 16 KiB
constexpr long long kDwRowsMfma = 16384;

typedef short dw_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) dw_v4i16 dw_lds_v4i16;

__device__ __forceinline__ uint2 dw_tr16(const unsigned char* p) {
    const dw_v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (dw_lds_v4i16*)(const __attribute__((address_space(3))) unsigned char*)(p));
    return __builtin_bit_cast(uint2, v);
}

// The ring's direct loads (dma16_lds, common.hpp) are waited for by dw_wait before the
// barrier that publishes a stage.
template <int N>
__device__ __forceinline__ void dw_wait() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | 0x0F70);
}
__device__ __forceinline__ void dw_barrier() {  // LDS data only (no vmcnt drain)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // s_waitcnt lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__global__ __launch_bounds__(256) void bw_dw_mfma_kernel(BackwardArgs a, DwArgs d) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kDwStages * kDwStageB];
    const int C = d.C, N3 = 3 * C;
    const int kt = blockIdx.x, jt = blockIdx.y, chunk = blockIdx.z;
    const int pod = chunk / d.chunks_per_pod;
    const long long r0 = (long long)pod * d.rows_per_pod + (long long)(chunk % d.chunks_per_pod) * d.rows_per_chunk;
    const long long r1 = min(r0 + d.rows_per_chunk, (long long)(pod + 1) * d.rows_per_pod);
    const int nsteps = (int)((r1 - r0) / kDwStep);  // rows are a multiple of kDwStep (host-checked)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wk = wave & 1, wj = wave >> 1;
    const char* Xs = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.X) + r0 * C + (long long)kt * kDwT);
    const char* Gs = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.G3) + r0 * N3 + (long long)jt * kDwT);
    // Direct loads: instruction q of a tile fills rows 4 q .. 4 q + 3; lane l lands in
    // row l / 16 of those, physical chunk l % 16, fetching logical chunk
    // (l % 16) ^ 2 (l / 16). Wave w issues instructions 2 w and 2 w + 1 of each tile.
    // Odd waves fill rows 8 .. 15 of every 16, whose chunk bit 3 is also flipped.
    const int drow = lane >> 4, dchunk = (lane & 15) ^ (2 * drow) ^ (8 * (wave & 1));
    const unsigned xoff = (unsigned)(drow * C * 2 + dchunk * 16), goff = (unsigned)(drow * N3 * 2 + dchunk * 16);
    auto issue = [&](int st, int stage) {  // step st (clamped: past the end refetch the last)
        const long long rb = (long long)(st < nsteps ? st : nsteps - 1) * kDwStep;
        const unsigned sb = lds_addr(lds + stage * kDwStageB);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int q = 2 * wave + u;
            dma16_lds(Xs + (rb + 4 * q) * C * 2, xoff, sb + q * 1024);
            dma16_lds(Gs + (rb + 4 * q) * N3 * 2, goff, sb + kDwStep * kDwRowB + q * 1024);
        }
    };
    // operand reads: 16-lane group g covers rows 8 g .. 8 g + 7 of a step (two reads)
    const int g = lane >> 4, i = lane & 15;
    auto rd = [&](int col0, int hf) {  // byte offset of this lane's 8 bytes in a tile
        const int row = 8 * g + 4 * hf + (i >> 2);
        const int chunk_l = col0 / 8 + ((i & 3) >> 1);
        return row * kDwRowB + ((chunk_l ^ (2 * (i >> 2)) ^ (8 * (g & 1))) << 4) + 8 * (i & 1);
    };
    int roff[2][4][2];  // [x/g][block][hf]
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            roff[0][b][hf] = rd(wk * 64 + b * 16, hf);
            roff[1][b][hf] = kDwStep * kDwRowB + rd(wj * 64 + b * 16, hf);
        }
    f32x4 acc[4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) acc[kb][jb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nsteps > 0) {
#pragma unroll
        for (int st = 0; st < kDwStages - 1; ++st) issue(st, st);
    }
    for (int st = 0; st < nsteps; ++st) {
        dw_wait<4 * (kDwStages - 2)>();  // this wave's loads of step st have landed
        dw_barrier();                    // ... and every wave's; step st-1's stage is free
        issue(st + kDwStages - 1, (st + kDwStages - 1) % kDwStages);
        const unsigned char* base = lds + (st % kDwStages) * kDwStageB;
        uint4 av[4], bv[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint2 x0 = dw_tr16(base + roff[0][b][0]), x1 = dw_tr16(base + roff[0][b][1]);
            const uint2 g0 = dw_tr16(base + roff[1][b][0]), g1 = dw_tr16(base + roff[1][b][1]);
            av[b] = make_uint4(x0.x, x0.y, x1.x, x1.y);
            bv[b] = make_uint4(g0.x, g0.y, g1.x, g1.y);
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
                acc[kb][jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_v, av[kb]), __builtin_bit_cast(bf16x8_v, bv[jb]), acc[kb][jb], 0, 0, 0);
    }
    dw_wait<0>();  // refetched steps may still be landing in LDS
    // C layout of a 16 x 16 block: lane l holds column l % 16 of rows 4 (l / 16) + e
    float* out = d.part + (long long)chunk * C * N3;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = kt * kDwT + wk * 64 + kb * 16 + 4 * g + e;
                const int j = jt * kDwT + wj * 64 + jb * 16 + i;
                out[(long long)k * N3 + j] = acc[kb][jb][e];
            }
}

// bf16 with C a multiple of 256: 256 x 256 output tiles, wave (wk, wj) owning
// 128 x 128 as 8 x 8 v_mfma_f32_16x16x32_bf16 blocks, so each staged byte feeds twice
// the matrix work of the 128-column tiles above. Each operand's 256 columns are staged
// as two [32 rows][128 columns] sub-tiles in the layout above, so the direct loads and
// the transposing reads are those of bw_dw_mfma_kernel plus a sub-tile offset; every
// output sums the same rows with the same instructions in the same order. (Without
// the swizzle's bit 3, the 16-lane groups of a read, rows 8 apart, shared banks: 2.0
// conflict cycles per LDS read.)
constexpr int kDw2T = 2 * kDwT, kDw2SubB = kDwStep * kDwRowB;  // 8 KiB per sub-tile
constexpr int kDw2StageB = 4 * kDw2SubB;                        // X0 X1 G0 G1: 32 KiB
constexpr int kDw2Stages = 4;                                   // 128 KiB

__global__ __launch_bounds__(256) void bw_dw_mfma2_kernel(BackwardArgs a, DwArgs d) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kDw2Stages * kDw2StageB];
    const int C = d.C, N3 = 3 * C;
    const int kt = blockIdx.x, jt = blockIdx.y, chunk = blockIdx.z;
    const int pod = chunk / d.chunks_per_pod;
    const long long r0 = (long long)pod * d.rows_per_pod + (long long)(chunk % d.chunks_per_pod) * d.rows_per_chunk;
    const long long r1 = min(r0 + d.rows_per_chunk, (long long)(pod + 1) * d.rows_per_pod);
    const int nsteps = (int)((r1 - r0) / kDwStep);  // rows are a multiple of kDwStep (host-checked)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wk = wave & 1, wj = wave >> 1;
    const char* Xs = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.X) + r0 * C + (long long)kt * kDw2T);
    const char* Gs = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.G3) + r0 * N3 + (long long)jt * kDw2T);
    // Odd waves fill rows 8 .. 15 of every 16, whose chunk bit 3 is also flipped.
    const int drow = lane >> 4, dchunk = (lane & 15) ^ (2 * drow) ^ (8 * (wave & 1));
    const unsigned xoff = (unsigned)(drow * C * 2 + dchunk * 16), goff = (unsigned)(drow * N3 * 2 + dchunk * 16);
    auto issue = [&](int st, int stage) {  // step st (clamped: past the end refetch the last)
        const long long rb = (long long)(st < nsteps ? st : nsteps - 1) * kDwStep;
        const unsigned sb = lds_addr(lds + stage * kDw2StageB);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int q = 2 * wave + u;
                dma16_lds(Xs + (rb + 4 * q) * C * 2 + sub * kDwRowB, xoff, sb + sub * kDw2SubB + q * 1024);
                dma16_lds(Gs + (rb + 4 * q) * N3 * 2 + sub * kDwRowB, goff, sb + (2 + sub) * kDw2SubB + q * 1024);
            }
    };
    // operand reads: as in bw_dw_mfma_kernel (16-lane group g reads rows 8 g .. 8 g + 7)
    const int g = lane >> 4, i = lane & 15;
    auto rd = [&](int col0, int hf) {
        const int row = 8 * g + 4 * hf + (i >> 2);
        const int chunk_l = col0 / 8 + ((i & 3) >> 1);
        return row * kDwRowB + ((chunk_l ^ (2 * (i >> 2)) ^ (8 * (g & 1))) << 4) + 8 * (i & 1);
    };
    int roff[2][8][2];  // [x/g][block][hf], with the wave's sub-tile offset
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            roff[0][b][hf] = wk * kDw2SubB + rd(b * 16, hf);
            roff[1][b][hf] = (2 + wj) * kDw2SubB + rd(b * 16, hf);
        }
    f32x4 acc[8][8];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) acc[kb][jb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // The fragments of step st + 1 are read while step st's MFMAs run (from registers),
    // so the matrix cores do not wait for each step's LDS reads: one wave per SIMD
    // has no other wave to cover them. A stage is refilled once every wave has read
    // its fragments (the barrier of the step after).
    auto read_frags = [&](int st, uint4 (&A)[8], uint4 (&Bv)[8]) {
        const unsigned char* base = lds + (st % kDw2Stages) * kDw2StageB;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint2 x0 = dw_tr16(base + roff[0][b][0]), x1 = dw_tr16(base + roff[0][b][1]);
            const uint2 g0 = dw_tr16(base + roff[1][b][0]), g1 = dw_tr16(base + roff[1][b][1]);
            A[b] = make_uint4(x0.x, x0.y, x1.x, x1.y);
            Bv[b] = make_uint4(g0.x, g0.y, g1.x, g1.y);
        }
    };
    uint4 av[8], bv[8];
    if (nsteps > 0) {
#pragma unroll
        for (int st = 0; st < kDw2Stages; ++st) issue(st, st);
        dw_wait<8 * (kDw2Stages - 1)>();  // this wave's loads of step 0 have landed
        dw_barrier();                     // ... and every wave's
        read_frags(0, av, bv);
    }
    for (int st = 0; st < nsteps; ++st) {
        dw_wait<8 * (kDw2Stages - 2)>();  // this wave's loads of step st + 1 have landed
        dw_barrier();                     // ... and every wave's; step st's stage is read
        issue(st + kDw2Stages, st % kDw2Stages);
        // each row of 8 MFMAs is followed by the reads of one block of step st + 1's
        // fragments (past the last step: the refetched last step, unused)
        const unsigned char* nbase = lds + ((st + 1) % kDw2Stages) * kDw2StageB;
        uint4 an[8], bn[8];
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
#pragma unroll
            for (int jb = 0; jb < 8; ++jb)
                acc[kb][jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_v, av[kb]), __builtin_bit_cast(bf16x8_v, bv[jb]), acc[kb][jb], 0, 0, 0);
            const uint2 x0 = dw_tr16(nbase + roff[0][kb][0]), x1 = dw_tr16(nbase + roff[0][kb][1]);
            const uint2 g0 = dw_tr16(nbase + roff[1][kb][0]), g1 = dw_tr16(nbase + roff[1][kb][1]);
            an[kb] = make_uint4(x0.x, x0.y, x1.x, x1.y);
            bn[kb] = make_uint4(g0.x, g0.y, g1.x, g1.y);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            av[b] = an[b];
            bv[b] = bn[b];
        }
    }
    dw_wait<0>();  // refetched steps may still be landing in LDS
    float* out = d.part + (long long)chunk * C * N3;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int jb = 0; jb < 8; ++jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = kt * kDw2T + wk * 128 + kb * 16 + 4 * g + e;
                const int j = jt * kDw2T + wj * 128 + jb * 16 + i;
                out[(long long)k * N3 + j] = acc[kb][jb][e];
            }
}

__global__ __launch_bounds__(256) void bw_dw_reduce_kernel(DwArgs d) {
    const int C = d.C, N3 = 3 * C;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;  // (pod, k, j)
    if (idx >= (long long)d.pods * C * N3) return;
    const int pod = (int)(idx / ((long long)C * N3));
    const long long kj = idx % ((long long)C * N3);
    float sum = 0.f;
    for (int c = 0; c < d.chunks_per_pod; ++c)
        sum += d.part[((long long)(pod * d.chunks_per_pod + c)) * C * N3 + kj];
    const int k = (int)(kj / N3), j = (int)(kj % N3), p = j / C;
    float* dst = p == 0 ? d.gWP : p == 1 ? d.gWI : d.gWV;
    if (dst) dst[((long long)pod * C + k) * C + (j - p * C)] = sum;
}

// grad_x = direct part + the projections' part (GEMM output, storage type)
template <typename T>
__global__ __launch_bounds__(256) void bw_final_kernel(const float* gXd, const void* gXp, float* gX,
                                                       long long n) {
    // 8 elements per thread (n is a multiple of 8: C >= 64)
    const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= n) return;
    const F4 d0 = ld4f(gXd, i), d1 = ld4f(gXd, i + 4);
    const F4 p0 = ld4<T>(gXp, i), p1 = ld4<T>(gXp, i + 4);
    float r0[4], r1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        r0[e] = d0.v[e] + p0.v[e];
        r1[e] = d1.v[e] + p1.v[e];
    }
    st4f(gX, i, r0);
    st4f(gX, i + 4, r1);
}

template <typename T, int kD>
hipError_t launch_dt(const BackwardArgs& a, hipStream_t s) {
    const long long cells = (long long)a.G * a.G;
    const long long n = (long long)a.B * cells * kHeads * kD;
    if (!a.loss_fused)
        hipLaunchKernelGGL((bw_loss_partial_kernel<T>), dim3(a.lchunks, a.B), dim3(256), 0, s, a);
    hipLaunchKernelGGL(bw_loss_finalize_kernel, dim3(a.B * kHeads), dim3(256), 0, s, a);
    if constexpr (sizeof(T) == 2 && kD == 64)  // G is a multiple of 8: whole cell pairs per row
        hipLaunchKernelGGL(bw_cell_ring_kernel, dim3(a.pods * a.nW), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((bw_cell_kernel<T, kD>), dim3(a.pods * a.nW), dim3(256), 0, s, a);
    if constexpr (kD == 64)
        hipLaunchKernelGGL((bw_gather_tile_kernel<T>),
                           dim3((unsigned)(a.B * (cells / (kGTy * kGTx)) * kHeads)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((bw_gather_kernel<T, kD>), dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, a);
    hipLaunchKernelGGL(bw_param_finalize_kernel, dim3(a.pods * kHeads * kPartF), dim3(256), 0, s, a);
    if (a.per_cell)
        hipLaunchKernelGGL(bw_cell_param_finalize_kernel,
                           dim3((unsigned)((a.pods * cells * kHeads + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const BackwardArgs& a, hipStream_t s) {
    switch (a.D) {
        case 8: return launch_dt<T, 8>(a, s);
        case 16: return launch_dt<T, 16>(a, s);
        case 32: return launch_dt<T, 32>(a, s);
        case 64: return launch_dt<T, 64>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int backward_loss_chunks(int G) { return (G * G + kLossCells - 1) / kLossCells; }
int backward_part_floats() { return kPartF; }
static bool dw_mfma(int dtype, int C, long long rows_per_pod) {
    return dtype == 1 && C % kDwT == 0 && rows_per_pod % kDwStep == 0;
}
long long backward_dw_rows_per_chunk(int dtype, int C, long long rows_per_pod) {
    if (!dw_mfma(dtype, C, rows_per_pod)) return kWRows;
    return rows_per_pod < kDwRowsMfma ? rows_per_pod : kDwRowsMfma;  // a multiple of kDwStep
}
int backward_dw_chunks_per_pod(int dtype, int C, long long rows_per_pod) {
    const long long r = backward_dw_rows_per_chunk(dtype, C, rows_per_pod);
    return (int)((rows_per_pod + r - 1) / r);
}

hipError_t launch_backward_stencil(int dtype, const BackwardArgs& a, hipStream_t s) {
    return dtype == 1 ? launch_t<bf16_t>(a, s) : launch_t<float>(a, s);
}

hipError_t launch_backward_dw(int dtype, const BackwardArgs& a, const DwArgs& d, hipStream_t s) {
    const dim3 grid(d.C / 64, 3 * d.C / 64, d.pods * d.chunks_per_pod);
    if (dw_mfma(dtype, d.C, d.rows_per_pod) && d.C % kDw2T == 0)
        hipLaunchKernelGGL(bw_dw_mfma2_kernel, dim3(d.C / kDw2T, 3 * d.C / kDw2T, d.pods * d.chunks_per_pod),
                           dim3(256), 0, s, a, d);
    else if (dw_mfma(dtype, d.C, d.rows_per_pod))
        hipLaunchKernelGGL(bw_dw_mfma_kernel, dim3(d.C / kDwT, 3 * d.C / kDwT, d.pods * d.chunks_per_pod),
                           dim3(256), 0, s, a, d);
    else if (dtype == 1)
        hipLaunchKernelGGL((bw_dw_partial_kernel<bf16_t>), grid, dim3(256), 0, s, a, d);
    else
        hipLaunchKernelGGL((bw_dw_partial_kernel<float>), grid, dim3(256), 0, s, a, d);
    const long long n = (long long)d.pods * d.C * 3 * d.C;
    hipLaunchKernelGGL(bw_dw_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d);
    return hipGetLastError();
}

hipError_t launch_backward_final(int dtype, const float* gXd, const void* gXp, float* gX, long long n,
                                 hipStream_t s) {
    const dim3 grid((unsigned)((n / 8 + 255) / 256));
    if (dtype == 1)
        hipLaunchKernelGGL((bw_final_kernel<bf16_t>), grid, dim3(256), 0, s, gXd, gXp, gX, n);
    else
        hipLaunchKernelGGL((bw_final_kernel<float>), grid, dim3(256), 0, s, gXd, gXp, gX, n);
    return hipGetLastError();
}

}  // namespace slime
