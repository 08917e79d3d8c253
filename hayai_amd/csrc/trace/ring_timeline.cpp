// Phase timeline of the 8B ring FFN step (ring gate/up with RMSNorm + ring down with the
// residual, 32 layers chained on one residual stream, as bench.py's headline step runs them),
// from a code object built with HH_RING_TRACE: per workgroup, the 100 MHz realtime counter at
// kernel start, at "input ready" (x's digits / h's digits in LDS), at the end of the weight
// loop and at the end of the kernel.  Prints, per phase, the earliest / median / latest
// workgroup relative to the layer's first gate/up workgroup, averaged over the layers of the
// last step (the first two layers skipped), and the step time from HIP events.
//
// Build: python -m hayai_amd.build --timeline
// Run:   hayai_amd/trace_build/ring_timeline hayai_amd/trace_build/hayai_kernels_trace.hsaco
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define CK(x)                                                                                    \
    do {                                                                                         \
        hipError_t e_ = (x);                                                                     \
        if (e_ != hipSuccess) {                                                                  \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));   \
            exit(1);                                                                             \
        }                                                                                        \
    } while (0)

// kernels/q4k_ring.hip: struct hh_gur_args, struct hh_dnr_args
struct GurArgs {  // the gate/up kernel's scalar parameters
    const uint8_t *wg, *wu;
    const float* x;
    uint8_t* hx;
    const float* nw;
    uint32_t rb1;
    uint32_t dims;  // d_model | d_ff << 16
    uint32_t grid;
    int32_t act;
    float eps;
};
struct DnrArgs {
    const uint8_t* wd;
    const uint8_t* hx;
    float* y;
    const float* res;
    uint64_t rb2;
    uint32_t d_model, d_ff;
};

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s <code object built with HH_RING_TRACE> [layers] [steps]\n", argv[0]);
        return 2;
    }
    const int dm = 4096, df = 14336;
    const int L = argc > 2 ? std::max(4, std::min(64, atoi(argv[2]))) : 32;
    const int steps = argc > 3 ? std::max(2, atoi(argv[3])) : 5;
    hipModule_t mod;
    CK(hipModuleLoad(&mod, argv[1]));
    hipFunction_t fgu, fdn;
    CK(hipModuleGetFunction(&fgu, mod, "hh_q4k_gu_ring_g1_n"));
    CK(hipModuleGetFunction(&fdn, mod, "hh_q4k_dn_ring_d4"));
    const size_t rb1 = (dm / 256) * 144, rb2 = (df / 256) * 144;
    const size_t gsz = (size_t)df * rb1, dsz = (size_t)dm * rb2;
    const size_t stride = (2 * gsz + dsz + 255) / 256 * 256;

    // weights: every Q4_K superblock with d = dmin = 2^-11 and scale/quant bytes 0x11 (the
    // timeline does not depend on the values)
    uint8_t* w;
    CK(hipMalloc(&w, stride * L));
    std::vector<uint8_t> host(stride, 0);
    for (size_t i = 0; i + 144 <= 2 * gsz + dsz; i += 144) {
        memset(&host[i], 0x11, 144);
        host[i] = 0;
        host[i + 1] = 0x10;
        host[i + 2] = 0;
        host[i + 3] = 0x10;
    }
    for (int l = 0; l < L; l++) CK(hipMemcpy(w + (size_t)l * stride, host.data(), stride, hipMemcpyHostToDevice));
    float *x, *nw;
    uint8_t* hx;
    CK(hipMalloc(&x, dm * 4));
    CK(hipMalloc(&nw, (size_t)dm * 4 * L));
    CK(hipMalloc(&hx, 2 * df + (df / 8) * 4 + 64));
    std::vector<float> ones((size_t)dm * L, 1.0f), xv(dm);
    for (int i = 0; i < dm; i++) xv[i] = 0.01f * (float)((i % 17) - 8);
    CK(hipMemcpy(nw, ones.data(), (size_t)dm * 4 * L, hipMemcpyHostToDevice));
    CK(hipMemcpy(x, xv.data(), dm * 4, hipMemcpyHostToDevice));

    size_t sz;
    hipDeviceptr_t gbase, gstride, gtrace;
    CK(hipModuleGetGlobal(&gbase, &sz, mod, "hh_ring_trace_base"));
    CK(hipMemcpyHtoD(gbase, &w, sizeof(w)));
    CK(hipModuleGetGlobal(&gstride, &sz, mod, "hh_ring_trace_stride"));
    unsigned long long st = stride;
    CK(hipMemcpyHtoD(gstride, &st, sizeof(st)));
    size_t trace_bytes;
    CK(hipModuleGetGlobal(&gtrace, &trace_bytes, mod, "hh_ring_trace"));

    // launch shapes of engine.cpp (enqueue_ring_gu / launch_dn_ring), one workgroup per CU
    hipDeviceProp_t pr;
    CK(hipGetDeviceProperties(&pr, 0));
    const size_t cus = (size_t)pr.multiProcessorCount;
    const size_t rr_max = 2 * 8 * ((df / 8 + cus - 1) / cus);
    const size_t smem_gu = (((2 * dm + (dm / 32) * 8) + 15) & ~size_t(15)) + ((rr_max + 3) & ~size_t(3)) * 4 + 128;
    const size_t hb = ((2 * df + (df / 8) * 4) + 15) & ~size_t(15);
    const size_t smem_dn = hb + ((dm + cus - 1) / cus) * 4 * 64 * 4;

    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int s = 0; s < steps; s++) {
        if (s == steps - 1) CK(hipEventRecord(e0, 0));
        for (int l = 0; l < L; l++) {
            const uint8_t* base = w + (size_t)l * stride;
            GurArgs ga{base, base + gsz, x, hx, nw + (size_t)l * dm, (uint32_t)rb1, (uint32_t)(dm | (df << 16)), (uint32_t)cus, 0,
                       1e-5f};
            // the kernels take the blocks' fields as scalar parameters: pass the raw bytes
            size_t gsz = sizeof ga;
            void* c1[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &ga, HIP_LAUNCH_PARAM_BUFFER_SIZE, &gsz, HIP_LAUNCH_PARAM_END};
            CK(hipModuleLaunchKernel(fgu, (unsigned)cus, 1, 1, 512, 1, 1, (unsigned)smem_gu, 0, nullptr, c1));
            DnrArgs da{base + 2 * gsz, hx, x, x, rb2, (uint32_t)dm, (uint32_t)df};
            size_t dsz = sizeof da;
            void* c2[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &da, HIP_LAUNCH_PARAM_BUFFER_SIZE, &dsz, HIP_LAUNCH_PARAM_END};
            CK(hipModuleLaunchKernel(fdn, (unsigned)cus, 1, 1, 576, 1, 1, (unsigned)smem_dn, 0, nullptr, c2));
        }
        if (s == steps - 1) CK(hipEventRecord(e1, 0));
    }
    CK(hipDeviceSynchronize());
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    std::vector<unsigned long long> tr(trace_bytes / 8);
    CK(hipMemcpyDtoH(tr.data(), gtrace, trace_bytes));
    auto at = [&](int k, int l, size_t g, int p) { return tr[(((size_t)k * 64 + l) * 512 + g) * 4 + p]; };

    const char* names[2][4] = {{"start", "x digits in LDS", "weight loop done", "h digits stored"},
                               {"start", "h digits in LDS", "weight loop done", "y stored"}};
    double acc[2][4][3] = {};
    int nl = 0;
    for (int l = 2; l < L; l++) {
        unsigned long long t0 = ~0ull;
        for (size_t g = 0; g < cus; g++) t0 = std::min(t0, at(0, l, g, 0));
        for (int k = 0; k < 2; k++)
            for (int p = 0; p < 4; p++) {
                std::vector<double> v;
                for (size_t g = 0; g < cus; g++) v.push_back((double)(at(k, l, g, p) - t0) * 0.01);
                std::sort(v.begin(), v.end());
                acc[k][p][0] += v.front();
                acc[k][p][1] += v[v.size() / 2];
                acc[k][p][2] += v.back();
            }
        nl++;
    }
    printf("ring FFN step, %d layers (d_model %d, d_ff %d, Q4_K, RMSNorm + residual): %.1f us per step, %.2f us "
           "per layer (HIP events; trace stores included)\n",
           L, dm, df, ms * 1e3, ms * 1e3 / L);
    printf("per layer, us from the layer's first gate/up workgroup (mean over layers 2..%d of the last step):\n", L - 1);
    printf("%-9s %-18s %8s %8s %8s\n", "kernel", "phase", "first", "median", "last");
    for (int k = 0; k < 2; k++)
        for (int p = 0; p < 4; p++)
            printf("%-9s %-18s %8.2f %8.2f %8.2f\n", k ? "down" : "gate/up", names[k][p], acc[k][p][0] / nl,
                   acc[k][p][1] / nl, acc[k][p][2] / nl);
    return 0;
}
