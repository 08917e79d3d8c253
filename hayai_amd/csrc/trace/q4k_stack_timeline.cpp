// Timeline of the persistent Q4_K FFN stack (q4k_stack.hip) at the Llama-3-8B shape (d_model
// 4096, d_ff 14336, 32 chained residual blocks, random Q4_K blocks with small fixed d/dmin),
// from a code object built with HH_QSTK_TRACE: per workgroup and layer, the 100 MHz realtime
// counter at each phase of the layer (q4k_stack.hip names the events).  Prints the launch
// times (HIP events) and, for a few layers of the last launch, the earliest / median / latest
// workgroup of each event relative to the layer's first barrier A.
//
// Build: python -m hayai_amd.build --timeline
// Run:   hayai_amd/trace_build/q4k_stack_timeline hayai_amd/trace_build/hayai_kernels_trace.hsaco
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#define CK(x)                                                                                  \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess) {                                                                \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

// kernels/q4k_stack.hip: struct hh_qstk_args
struct QstkArgs {
    const uint8_t* pack;
    const float* norm;
    const float* x;
    float* y;
    uint64_t* hx;
    uint64_t* xx;
    unsigned* bar;
    uint64_t stride, off_g, off_u, off_d, rb1, rb2;
    uint32_t norm_stride, d_model, d_ff, n_layers, lds_wd, lds_hx;
    float eps;
    int32_t act;
};

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s <code object built with HH_QSTK_TRACE>\n", argv[0]);
        return 2;
    }
    const uint32_t DM = 4096, DF = 14336, L = 32, G = 256, EV = 10;
    const size_t rb1 = DM / 256 * 144, rb2 = DF / 256 * 144;
    const size_t off_u = DF * rb1, off_d = 2 * DF * rb1, stride = (off_d + DM * rb2 + 255) / 256 * 256;
    hipModule_t mod;
    CK(hipModuleLoad(&mod, argv[1]));
    hipFunction_t fn;
    CK(hipModuleGetFunction(&fn, mod, "hh_q4k_stk_d4_r3_t24"));
    void* trace;
    size_t trace_bytes;
    CK(hipModuleGetGlobal((hipDeviceptr_t*)&trace, &trace_bytes, mod, "hh_qstk_trace"));

    // Q4_K blocks: d = 2^-8, dmin = 2^-9 (f16), random scale and code bytes
    std::vector<uint8_t> host(stride);
    std::mt19937 rng(1);
    uint8_t* pack;
    CK(hipMalloc(&pack, stride * L));
    for (uint32_t l = 0; l < L; l++) {
        for (size_t o = 0; o + 144 <= stride; o += 144) {
            uint8_t* b = host.data() + o;
            b[0] = 0x00, b[1] = 0x1C, b[2] = 0x00, b[3] = 0x18;
            for (int i = 4; i < 144; i++) b[i] = (uint8_t)rng();
        }
        CK(hipMemcpy(pack + l * stride, host.data(), stride, hipMemcpyHostToDevice));
    }
    std::vector<float> nrm(DM * L, 1.0f), x(DM);
    for (auto& v : x) v = (float)((int)(rng() % 2001) - 1000) / 500.f;
    float *dn, *dx, *dy;
    uint64_t* ws;
    unsigned* bar;
    // exchange buffers as the engine pads them (enqueue_q4k_stack)
    const size_t hpad = (3 * (DF / 8) + 2687) / 2688 * 2688, xpad = DM + 64 * 22;
    CK(hipMalloc(&dn, 4 * DM * L));
    CK(hipMalloc(&dx, 4 * DM));
    CK(hipMalloc(&dy, 4 * DM));
    CK(hipMalloc(&ws, 8 * (hpad + xpad)));
    CK(hipMemset(ws, 0, 8 * (hpad + xpad)));
    CK(hipMalloc(&bar, 128 * 36));
    CK(hipMemset(bar, 0, 128 * 36));
    CK(hipMemcpy(dn, nrm.data(), 4 * DM * L, hipMemcpyHostToDevice));
    CK(hipMemcpy(dx, x.data(), 4 * DM, hipMemcpyHostToDevice));
    const size_t nrow_max = (DM + G - 1) / G, wpt2 = 4;
    const size_t lds_wd = (nrow_max * rb2 + 15) & ~(size_t)15;
    const size_t lds_hx =
        (std::max<size_t>(2 * DF + 2 * (DF / 8), ((2 * DM + (DM / 32) * 8 + 15) & ~(size_t)15) + 4 * DM) + 15) &
        ~(size_t)15;
    auto al4 = [](size_t n) { return (n + 3) & ~(size_t)3; };
    const size_t smem =
        lds_wd + lds_hx + 4 * (al4(16 * ((DF / 8 + G - 1) / G)) + al4(nrow_max * wpt2) + al4(3) + al4(2 * nrow_max));
    QstkArgs a{pack, dn, dx, dy, ws, ws + hpad, bar, stride, 0, off_u, off_d, rb1, rb2, DM, DM, DF, L,
               (uint32_t)lds_wd, (uint32_t)lds_hx, 1e-5f, 0};
    void* params[] = {&a};
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int r = 0; r < 6; r++) {
        CK(hipEventRecord(e0));
        CK(hipModuleLaunchKernel(fn, G, 1, 1, 12 * 64, 1, 1, (unsigned)smem, 0, params, nullptr));
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        printf("launch %d: %.1f us (%.2f us per layer)\n", r, ms * 1e3, ms * 1e3 / L);
    }
    unsigned err;
    CK(hipMemcpy(&err, (char*)bar + 128 * 33, 4, hipMemcpyDeviceToHost));
    printf("error word %u\n", err);
    std::vector<uint64_t> t(256 * 64 * EV);
    CK(hipMemcpy(t.data(), trace, t.size() * 8, hipMemcpyDeviceToHost));
    auto T = [&](int w, int l, int e) { return (double)t[((size_t)w * 64 + l) * EV + e]; };
    const char* name[EV] = {"A: x digits", "gate/up end", "B", "C: h + W_down", "E: down done", "h gathered",
                            "x_{l+1} gathered", "W_down landed", "down end", "h in registers"};
    const int order[] = {0, 1, 2, 5, 7, 3, 9, 8, 4, 6};
    for (int l : {0, 1, 15, 30}) {
        std::vector<double> a0;
        for (uint32_t w = 0; w < G; w++) a0.push_back(T(w, l, 0));
        const double base = *std::min_element(a0.begin(), a0.end());
        printf("layer %d (us after its first A):\n", l);
        auto row = [&](const char* nm, int ll, int e) {
            std::vector<double> v;
            for (uint32_t w = 0; w < G; w++) v.push_back((T(w, ll, e) - base) / 100.0);
            std::sort(v.begin(), v.end());
            printf("  %-18s min %7.2f  med %7.2f  max %7.2f\n", nm, v[0], v[G / 2], v[G - 1]);
        };
        for (int e : order) row(name[e], l, e);
        if (l + 1 < (int)L) row("next A", l + 1, 0);
    }
    return 0;
}
