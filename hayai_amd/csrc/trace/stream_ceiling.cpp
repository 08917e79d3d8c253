// Streaming ceiling of one MI355X for the FFN's access sizes: plain read kernels with no
// math, one workgroup of 8 waves per CU, each wave streaming a contiguous share of the bytes
// (register loads in batches of U x 1 KB per wave; or global->LDS DMA into a per-wave LDS
// ring), over rotating windows of a 2 GiB buffer so no window is served from the 256 MB
// memory-side cache.  Prints the time per launch for 33 / 66 / 99 MB (one 8B-shape W_down,
// W_gate + W_up, and a whole layer), and the 66 + 33 MB pair as two dependent launches
// against 99 MB in one: the cost of the kernel boundary between gate/up and down.
//
// Build: python -m hayai_amd.build --timeline
// Run:   hayai_amd/trace_build/stream_ceiling
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define CK(x)                                                                                  \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess) {                                                                \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

// Each wave reads per_wave uint4 (a multiple of 64 * U) starting at its share.
template <int U>
__global__ void __launch_bounds__(512) read_regs(const uint4* __restrict__ p, size_t per_wave, uint32_t* out) {
    const uint32_t lane = threadIdx.x % 64, wv = blockIdx.x * 8 + threadIdx.x / 64;
    const uint4* q = p + (size_t)wv * per_wave;
    uint32_t acc = 0;
    for (size_t i = lane; i < per_wave; i += 64 * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = q[i + 64 * u];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x12345678u) out[wv] = acc;  // keeps the loads
}

// The same shares copied into a per-wave LDS ring of R KB (1 KB per instruction).
template <int U, int R>
__global__ void __launch_bounds__(512) read_lds(const uint4* __restrict__ p, size_t per_wave, uint32_t* out) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const uint32_t lane = threadIdx.x % 64, wv = blockIdx.x * 8 + threadIdx.x / 64, w = threadIdx.x / 64;
    const uint4* q = p + (size_t)wv * per_wave;
    char* ring = lds + (size_t)w * R * 1024;
    uint32_t slot = 0;
    for (size_t i = lane; i < per_wave; i += 64 * U) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(q + i + 64 * u),
                                             (__attribute__((address_space(3))) void*)(ring + (size_t)slot * 1024),
                                             16, 0, 0);
            slot = slot + 1 == R ? 0 : slot + 1;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const uint32_t acc = reinterpret_cast<uint32_t*>(ring)[lane];
    if (acc == 0x12345678u) out[wv] = acc;
}

int main() {
    const size_t TOT = 2ull << 30;
    uint4* buf;
    uint32_t* out;
    CK(hipMalloc(&buf, TOT));
    CK(hipMalloc(&out, 1 << 20));
    CK(hipMemset(buf, 1, TOT));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const int G = 256, reps = 60;
    auto elapsed_us = [&](auto&& body) {
        CK(hipEventRecord(e0));
        for (int r = 0; r < reps; r++) body(r);
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        return ms * 1e3 / reps;
    };
    auto run = [&](const char* name, auto kern, size_t bytes, unsigned lds) {
        const size_t per_wave = bytes / 16 / (G * 8), nwin = TOT / bytes;
        for (int r = 0; r < 3; r++)
            hipLaunchKernelGGL(kern, dim3(G), dim3(512), lds, 0, buf + (r % nwin) * (bytes / 16), per_wave, out);
        CK(hipDeviceSynchronize());
        const double us = elapsed_us([&](int r) {
            hipLaunchKernelGGL(kern, dim3(G), dim3(512), lds, 0, buf + (r % nwin) * (bytes / 16), per_wave, out);
        });
        printf("%-22s %6.1f MB  %7.2f us per launch  %5.2f TB/s\n", name, bytes / 1e6, us, bytes / us / 1e6);
    };
    // multiples of 256 workgroups x 8 waves x 64 lanes x 16 B x 8
    const size_t MB33 = 33030144, MB66 = 2 * MB33, MB99 = 3 * MB33;
    for (size_t b : {MB33, MB66, MB99}) {
        run("registers, 4 KB/wave", read_regs<4>, b, 0);
        run("registers, 8 KB/wave", read_regs<8>, b, 0);
        run("LDS DMA, 4 KB/wave", read_lds<4, 16>, b, 8 * 16 * 1024);
        run("LDS DMA, 8 KB/wave", read_lds<8, 16>, b, 8 * 16 * 1024);
    }
    const size_t pw33 = MB33 / 16 / (G * 8), pw66 = MB66 / 16 / (G * 8), pw99 = MB99 / 16 / (G * 8);
    const double two = elapsed_us([&](int r) {
        uint4* base = buf + (size_t)(r % 20) * (MB99 / 16);
        hipLaunchKernelGGL(read_regs<8>, dim3(G), dim3(512), 0, 0, base, pw66, out);
        hipLaunchKernelGGL(read_regs<8>, dim3(G), dim3(512), 0, 0, base + MB66 / 16, pw33, out);
    });
    const double one = elapsed_us([&](int r) {
        hipLaunchKernelGGL(read_regs<8>, dim3(G), dim3(512), 0, 0, buf + (size_t)(r % 20) * (MB99 / 16), pw99, out);
    });
    printf("66 + 33 MB as two dependent launches: %7.2f us (%.1f%% of 8 TB/s)\n", two, MB99 / two / 8e4);
    printf("99 MB as one launch:                  %7.2f us (%.1f%% of 8 TB/s)\n", one, MB99 / one / 8e4);
    CK(hipDeviceSynchronize());
    return 0;
}
