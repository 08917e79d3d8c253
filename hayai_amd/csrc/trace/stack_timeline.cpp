// Timeline of the persistent FFN stack (small_stack.hip) at SmolLM2-135M's layer (d_model
// 576, d_ff 1536, Q4_0, 30 chained residual blocks, 8 rotated copies of the weights), from a
// code object built with HH_SSTK_TRACE: per workgroup and layer, the 100 MHz realtime counter
// when the exchange wave has x_l, when it has h_l, and when the compute waves pass barrier A,
// have published their h rows, pass barrier B and have published their x rows.  Prints the
// earliest / median / latest workgroup of each event for a few layers of the last launch,
// relative to the first barrier A of layer 0, and the launch time from HIP events.
//
// Build: python -m hayai_amd.build --timeline
// Run:   hayai_amd/trace_build/stack_timeline hayai_amd/trace_build/hayai_kernels_trace.hsaco
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#define CK(x)                                                                                    \
    do {                                                                                         \
        hipError_t e_ = (x);                                                                     \
        if (e_ != hipSuccess) {                                                                  \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));   \
            exit(1);                                                                             \
        }                                                                                        \
    } while (0)

// kernels/small_stack.hip: struct hh_sstk_args
struct SstkArgs {
    const uint8_t* pack;
    const float* norm;
    const float* x;
    float* y;
    uint64_t *hx, *xx, *spare;
    unsigned* bar;
    uint64_t stride, off_g, off_u, off_d, rb_in, rb_ff;
    uint32_t norm_stride, d_model, d_ff, n_layers;
    float eps;
    int32_t act;
};

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s <code object built with HH_SSTK_TRACE>\n", argv[0]);
        return 2;
    }
    const uint32_t DM = 576, DF = 1536, L = 30, COPIES = 8, G = 256;
    const size_t rb_in = DM / 32 * 18, rb_ff = DF / 32 * 18;
    const size_t off_u = DF * rb_in, off_d = 2 * DF * rb_in, stride = off_d + DM * rb_ff;
    hipModule_t mod;
    CK(hipModuleLoad(&mod, argv[1]));
    hipFunction_t fn;
    CK(hipModuleGetFunction(&fn, mod, "hh_sstk_q4_0_t32_64_r1"));
    void* trace;
    size_t trace_bytes;
    CK(hipModuleGetGlobal((hipDeviceptr_t*)&trace, &trace_bytes, mod, "hh_sstk_trace"));

    // Q4_0 blocks: d = 2^-7, random nibbles
    std::vector<uint8_t> host(stride * L);
    std::mt19937 rng(1);
    for (size_t b = 0; b < host.size() / 18; b++) {
        uint8_t* blk = host.data() + b * 18;
        blk[0] = 0x00;
        blk[1] = 0x20;
        for (int i = 2; i < 18; i++) blk[i] = (uint8_t)(rng() & 0xFF);
    }
    uint8_t* pack;
    float *norm, *x, *y;
    uint64_t* ws;
    unsigned* bar;
    CK(hipMalloc(&pack, stride * L * COPIES));
    for (uint32_t c = 0; c < COPIES; c++)
        CK(hipMemcpy(pack + c * stride * L, host.data(), host.size(), hipMemcpyHostToDevice));
    std::vector<float> nh(L * DM, 1.0f), xh(DM);
    for (auto& v : xh) v = (float)((int)(rng() % 2001) - 1000) / 1000.f;
    CK(hipMalloc(&norm, nh.size() * 4));
    CK(hipMemcpy(norm, nh.data(), nh.size() * 4, hipMemcpyHostToDevice));
    CK(hipMalloc(&x, DM * 4));
    CK(hipMemcpy(x, xh.data(), DM * 4, hipMemcpyHostToDevice));
    CK(hipMalloc(&y, DM * 4));
    const size_t words = DF + DM + 16 * G;
    CK(hipMalloc(&ws, words * 8));
    CK(hipMemset(ws, 0, words * 8));
    CK(hipMalloc(&bar, 128 * 36));
    CK(hipMemset(bar, 0, 128 * 36));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const int iters = 20;
    for (int it = 0; it < iters; it++) {
        SstkArgs a{};
        a.pack = pack + (size_t)(it % COPIES) * stride * L;
        a.norm = norm;
        a.x = x;
        a.y = y;
        a.hx = ws;
        a.xx = ws + DF;
        a.spare = ws + DF + DM;
        a.bar = bar;
        a.stride = stride;
        a.off_g = 0;
        a.off_u = off_u;
        a.off_d = off_d;
        a.rb_in = rb_in;
        a.rb_ff = rb_ff;
        a.norm_stride = DM;
        a.d_model = DM;
        a.d_ff = DF;
        a.n_layers = L;
        a.eps = 1e-5f;
        a.act = 0;
        void* params[] = {&a};
        if (it == iters - 1) CK(hipEventRecord(e0, 0));
        CK(hipModuleLaunchKernel(fn, G, 1, 1, 320, 1, 1, 0, 0, params, nullptr));
        if (it == iters - 1) CK(hipEventRecord(e1, 0));
    }
    CK(hipDeviceSynchronize());
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    unsigned err;
    CK(hipMemcpy(&err, bar + 33 * 32, 4, hipMemcpyDeviceToHost));
    std::vector<uint64_t> tr(256 * 64 * 8);
    CK(hipMemcpy(tr.data(), trace, std::min(trace_bytes, tr.size() * 8), hipMemcpyDeviceToHost));
    auto at = [&](uint32_t w, uint32_t l, int ev) { return tr[((size_t)w * 64 + l) * 8 + ev]; };
    printf("last launch %.1f us (%.2f us per layer), error word %u\n", ms * 1e3, ms * 1e3 / L, err);
    uint64_t t0 = ~0ull;
    for (uint32_t w = 0; w < G; w++) t0 = std::min(t0, at(w, 0, 2));
    const char* names[6] = {"X has x_l", "X has h_l", "C passed A", "C h rows out", "C passed B", "C x rows out"};
    printf("layer  event          first   median   last   (us from layer 0's first barrier A)\n");
    for (uint32_t l = 0; l < L; l++) {
        if (l > 3 && l != 15 && l + 2 < L) continue;
        for (int ev = 0; ev < 6; ev++) {
            if (l == 0 && ev == 0) continue;
            std::vector<double> v;
            for (uint32_t w = 0; w < G; w++) v.push_back(((double)at(w, l, ev) - (double)t0) / 100.0);
            std::sort(v.begin(), v.end());
            printf("%3u  %-13s %7.2f %7.2f %7.2f\n", l, names[ev], v[0], v[G / 2], v[G - 1]);
        }
    }
    return err ? 1 : 0;
}
