// ca_binding.cpp — a compiled C++ host of libslime_ca.so, written as the reference's
// runtime would call it (the binding a maintainer of the reference would add): the organism's CA
// engine is created next to the organism, its weights are the reference's per-head
// tensors embedded as dense matrices, and each generation calls
// slime_neural_ca_update from the host instead of the device-side launch of
// neural_ca_update_kernel (slime/core/organism.cu:113-120, 617-688).
//
// Built by tests/binding.py with g++ against include/slime_ca.h only (plus the HIP
// runtime API for the organism's own device buffers, as the reference's host uses
// the CUDA runtime for them). Two modes:
//
//   ca_binding checks
//       Status codes that need no GPU: NULL and invalid configurations are
//       SLIME_EINVAL, non-finite parameters fail slime_ca_check_params, and a valid
//       configuration is SLIME_OK on a gfx950 or SLIME_ENODEV / SLIME_EHIP without
//       one. Prints one line per check and "checks ok".
//
//   ca_binding generation <in.bin> <out.bin> <snapshot.json>
//       Runs `gens` organism generations on a G x G grid (B 1, 8 heads, D 64, fp32)
//       and writes the field, the mass buffer, the effective-rank history and the
//       last generation's CA input and output, plus the evolution.json record of the
//       last generation. The input file is little-endian:
//         int32 G, gens, pvi_chain
//         float32 perception [8][512][256], interaction [8][512][256],
//                 value [8][256][512], head_mixing [8][8], flow_kernels [8][3][3],
//                 mu [8], sigma [8], conc [G][G]
//       and the output file holds float32 conc [G][G], mass [8], erank [gens],
//       ca_input [G][G][512], ca_output [G][G][512].
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <vector>

#include "slime_ca.h"

namespace {

int g_failures = 0;

#define SLIME_CHECK(call)                                                                 \
    do {                                                                                  \
        int rc_ = (call);                                                                 \
        if (rc_ != SLIME_OK) {                                                            \
            std::fprintf(stderr, "slime_ca error %d at %s:%d: %s\n", rc_, __FILE__, __LINE__, \
                         slime_ca_last_error());                                          \
            std::exit(1); /* the reference's CUDA_CHECK behaviour */                      \
        }                                                                                 \
    } while (0)

#define HIP_CHECK(call)                                                                   \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) {                                                           \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_),        \
                         __FILE__, __LINE__);                                             \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

void expect(bool ok, const char* what) {
    std::printf("%s: %s\n", ok ? "ok  " : "FAIL", what);
    if (!ok) ++g_failures;
}

constexpr int kH = 8, kD = 64, kChannels = 512, kHidden = 256, kC = kH * kD;

// The reference's per-head tensors (MultiHeadCAState, slime/core/pseudopod.cu:29-38):
// perception/interaction [H][CHANNELS][HIDDEN], value [H][HIDDEN][CHANNELS],
// head_mixing [H][H], flow_kernels [H][3][3].
struct RefCAWeights {
    std::vector<float> perception, interaction, value, head_mixing, flow_kernels;
};

// multi_head_ca_kernel uses the D x D block at the top left of each per-head slab
// (pseudopod.cu:79-119), and its value loop reads interaction[j % D] for every
// j < HIDDEN, so the dense C x C matrices are block-diagonal with the value rows that
// share j % D added up.
void embed_reference_weights(const RefCAWeights& r, std::vector<float>& WP, std::vector<float>& WI,
                             std::vector<float>& WV, std::vector<float>& K, std::vector<float>& M) {
    WP.assign((size_t)kC * kC, 0.f);
    WI.assign((size_t)kC * kC, 0.f);
    WV.assign((size_t)kC * kC, 0.f);
    for (int h = 0; h < kH; ++h)
        for (int r0 = 0; r0 < kD; ++r0)
            for (int i = 0; i < kD; ++i) {
                const size_t dst = (size_t)(h * kD + r0) * kC + h * kD + i;  // row = input channel
                WP[dst] = r.perception[((size_t)h * kChannels + r0) * kHidden + i];
                WI[dst] = r.interaction[((size_t)h * kChannels + r0) * kHidden + i];
                double v = 0.0;
                for (int j = r0; j < kHidden; j += kD) v += r.value[((size_t)h * kHidden + j) * kChannels + i];
                WV[dst] = (float)v;
            }
    K.assign(r.flow_kernels.begin(), r.flow_kernels.end());  // [H][9], tap 3(dy+1)+(dx+1)
    M.assign(r.head_mixing.begin(), r.head_mixing.end());    // M[o][h]
}

slime_ca_config engine_config(int G, int pvi_chain) {
    slime_ca_config cfg{};
    cfg.B = 1;
    cfg.G = G;
    cfg.H = kH;
    cfg.D = kD;
    cfg.dtype = SLIME_F32;
    cfg.dt = 0.1f;  // organism.cu:659
    cfg.growth_per_cell = 0;
    cfg.pods = 1;
    cfg.pvi_chain = pvi_chain;
    return cfg;
}

int run_checks() {
    slime_ca* ca = nullptr;
    expect(slime_ca_create(nullptr, &ca) == SLIME_EINVAL && ca == nullptr, "create(NULL config) is EINVAL");
    slime_ca_config bad = engine_config(12, 2);
    expect(slime_ca_create(&bad, &ca) == SLIME_EINVAL && ca == nullptr, "create(G = 12) is EINVAL");
    expect(std::strlen(slime_ca_last_error()) > 0, "last_error describes the failure");
    bad = engine_config(32, 3);
    expect(slime_ca_create(&bad, &ca) == SLIME_EINVAL, "create(pvi_chain = 3) is EINVAL");
    expect(slime_ca_destroy(nullptr) == SLIME_OK, "destroy(NULL) is OK");
    expect(slime_ca_step(nullptr, nullptr, nullptr, 1, nullptr) == SLIME_EINVAL, "step(NULL) is EINVAL");

    // Parameter checks on the host: finite parameters pass, one NaN or Inf fails.
    const slime_ca_config cfg = engine_config(16, 2);
    std::vector<float> W((size_t)kC * kC, 0.01f), K(kH * 9, 0.1f), mu(kH, 0.2f), sigma(kH, 0.03f),
        M(kH * kH, 0.f);
    for (int h = 0; h < kH; ++h) M[h * kH + h] = 1.f;
    slime_ca_params p{W.data(), W.data(), W.data(), K.data(), mu.data(), sigma.data(), M.data()};
    expect(slime_ca_check_params(&cfg, &p) == SLIME_OK, "check_params accepts finite parameters");
    K[5] = std::numeric_limits<float>::quiet_NaN();
    expect(slime_ca_check_params(&cfg, &p) == SLIME_EINVAL, "check_params rejects a NaN flow-kernel tap");
    K[5] = 0.1f;
    W[(size_t)kC * kC - 1] = std::numeric_limits<float>::infinity();
    expect(slime_ca_check_params(&cfg, &p) == SLIME_EINVAL, "check_params rejects an Inf weight");

    const slime_ca_config good = engine_config(32, 2);
    const int rc = slime_ca_create(&good, &ca);
    int ndev = 0;
    const bool gpu = hipGetDeviceCount(&ndev) == hipSuccess && ndev > 0;
    if (gpu) {
        expect(rc == SLIME_OK && ca != nullptr, "create(valid) is OK on a GPU");
        expect(slime_ca_set_params(ca, &p) == SLIME_EINVAL, "set_params rejects the Inf weight");
        W[(size_t)kC * kC - 1] = 0.01f;
        expect(slime_ca_set_params(ca, &p) == SLIME_OK, "set_params accepts finite parameters");
        expect(slime_ca_destroy(ca) == SLIME_OK, "destroy is OK");
    } else {
        expect((rc == SLIME_ENODEV || rc == SLIME_EHIP) && ca == nullptr,
               "create(valid) without a GPU is ENODEV or EHIP");
        std::printf("      (%d: %s)\n", rc, slime_ca_last_error());
    }
    if (g_failures) return 1;
    std::printf("checks ok\n");
    return 0;
}

template <typename T>
void read_into(std::FILE* f, std::vector<T>& v, size_t n) {
    v.resize(n);
    if (std::fread(v.data(), sizeof(T), n, f) != n) {
        std::fprintf(stderr, "short input file\n");
        std::exit(1);
    }
}

void write_from(std::FILE* f, const float* d, size_t n) {
    std::vector<float> h(n);
    HIP_CHECK(hipMemcpy(h.data(), d, n * 4, hipMemcpyDeviceToHost));
    if (std::fwrite(h.data(), 4, n, f) != n) {
        std::fprintf(stderr, "short write\n");
        std::exit(1);
    }
}

int run_generations(const char* in_path, const char* out_path, const char* json_path) {
    std::FILE* f = std::fopen(in_path, "rb");
    if (!f) {
        std::fprintf(stderr, "cannot open %s\n", in_path);
        return 1;
    }
    std::vector<int> hdr;
    read_into(f, hdr, 3);
    const int G = hdr[0], gens = hdr[1], pvi_chain = hdr[2];
    RefCAWeights ref;
    std::vector<float> mu, sigma, conc;
    read_into(f, ref.perception, (size_t)kH * kChannels * kHidden);
    read_into(f, ref.interaction, (size_t)kH * kChannels * kHidden);
    read_into(f, ref.value, (size_t)kH * kHidden * kChannels);
    read_into(f, ref.head_mixing, (size_t)kH * kH);
    read_into(f, ref.flow_kernels, (size_t)kH * 9);
    read_into(f, mu, kH);
    read_into(f, sigma, kH);
    read_into(f, conc, (size_t)G * G);
    std::fclose(f);
    std::printf("generation: G=%d gens=%d pvi_chain=%d\n", G, gens, pvi_chain);

    // create_organism's part (slime/runtime.cu:66-94): the engine and its parameters.
    slime_ca_config cfg = engine_config(G, pvi_chain);
    slime_ca* ca = nullptr;
    SLIME_CHECK(slime_ca_create(&cfg, &ca));
    std::vector<float> WP, WI, WV, K, M;
    embed_reference_weights(ref, WP, WI, WV, K, M);
    slime_ca_params p{WP.data(), WI.data(), WV.data(), K.data(), mu.data(), sigma.data(), M.data()};
    SLIME_CHECK(slime_ca_set_params(ca, &p));

    // The organism's own buffers (MultiHeadCAState::ca_input, ca_output, mass_buffer;
    // the chemical field; the effective-rank history).
    const size_t state = (size_t)G * G * kC;
    float *ca_input = nullptr, *ca_output = nullptr, *mass = nullptr, *field = nullptr, *erank = nullptr;
    HIP_CHECK(hipMalloc((void**)&ca_input, state * 4));
    HIP_CHECK(hipMalloc((void**)&ca_output, state * 4));
    HIP_CHECK(hipMalloc((void**)&mass, kH * 4));
    HIP_CHECK(hipMalloc((void**)&field, (size_t)G * G * 4));
    HIP_CHECK(hipMalloc((void**)&erank, (size_t)gens * 4));
    HIP_CHECK(hipMemcpy(field, conc.data(), (size_t)G * G * 4, hipMemcpyHostToDevice));
    hipStream_t stream = nullptr;
    HIP_CHECK(hipStreamCreate(&stream));

    // run_organism's generation loop (slime/runtime.cu:396-409), the CA part on the host.
    slime_multihead_ca_state st{mass, ca_input, ca_output};
    for (int gen = 0; gen < gens; ++gen)
        SLIME_CHECK(slime_neural_ca_update(ca, &st, field, erank, gen, stream));
    HIP_CHECK(hipStreamSynchronize(stream));

    // get_ca_state (slime/runtime.cu:479): the field, read back by the library.
    std::vector<float> view((size_t)G * G);
    SLIME_CHECK(slime_ca_get_state(ca, ca_output, view.data(), G * G));
    // extract_system_state (slime/extract_state.cu:58): the generation's record.
    std::vector<char> json(1 << 16);
    size_t written = 0;
    SLIME_CHECK(slime_snapshot_json(ca, field, nullptr, gens - 1, 0.0, json.data(), json.size(), &written));

    std::FILE* o = std::fopen(out_path, "wb");
    if (!o) return 1;
    write_from(o, field, (size_t)G * G);
    write_from(o, mass, kH);
    write_from(o, erank, gens);
    write_from(o, ca_input, state);
    write_from(o, ca_output, state);
    std::fclose(o);
    std::FILE* j = std::fopen(json_path, "wb");
    if (!j) return 1;
    std::fwrite(json.data(), 1, written, j);
    std::fclose(j);

    std::vector<float> field_h((size_t)G * G);
    HIP_CHECK(hipMemcpy(field_h.data(), field, field_h.size() * 4, hipMemcpyDeviceToHost));
    expect(std::memcmp(view.data(), field_h.data(), view.size() * 4) == 0,
           "get_ca_state equals the organism's field after the last generation");

    HIP_CHECK(hipStreamDestroy(stream));
    for (float* d : {ca_input, ca_output, mass, field, erank}) HIP_CHECK(hipFree(d));
    SLIME_CHECK(slime_ca_destroy(ca));  // destroy_organism (slime/runtime.cu:417)
    if (g_failures) return 1;
    std::printf("generation ok\n");
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "checks") == 0) return run_checks();
    if (argc >= 5 && std::strcmp(argv[1], "generation") == 0)
        return run_generations(argv[2], argv[3], argv[4]);
    std::fprintf(stderr, "usage: %s checks | generation <in.bin> <out.bin> <snapshot.json>\n", argv[0]);
    return 2;
}
