// Q4 LUT GEMV: Hayai's own 4-bit dictionary format ("Q4 LUT MatMul" of `hayai bench`).
//
//   y[r] = sum_c  x[2c] * lut[W[r][c] & 15]  +  x[2c+1] * lut[W[r][c] >> 4],   W: m rows of n/2 bytes
//
// Reference: cpu_lut_matmul_q4 (crates/hayai-cpu/src/matmul.rs:48-82), the OpenCL kernel
// lut_matmul_q4_v1 (crates/hayai-kernels/kernels/lut_matmul.cl:14-54, one work-item per row
// with the 16 LUT entries in __local) and its host OpenClEngine::lut_matmul_q4
// (crates/hayai-opencl/src/compute.rs:45-128).
//
// Here a wave owns a row at a time (rows grid-stride over the waves of the grid); its lanes
// walk the row's packed bytes front to back, four bytes per lane per step, so a wave's loads
// cover one contiguous 256-byte span.  Each weight byte indexes a 256-entry LDS table of
// (lut[b & 15], lut[b >> 4]) pairs: one 8-byte LDS read per two weights instead of two
// lookups.  Partial sums meet in a DPP wave reduction (hh_wave_sum).  Rows whose byte
// length is not a multiple of 4 (or x not 16-byte aligned) take the bytewise loop.
#include "common.h"

struct hh_lut_args {
    const uint8_t* w;  // m rows of n/2 packed bytes
    const float* lut;  // 16 f32 entries
    const float* x;    // n f32
    float* y;          // m f32
    uint32_t m;
    uint32_t n;
    uint32_t vec;  // 1: dword weight loads + float4 x loads are aligned
    uint32_t pad;
};

#define HH_LUT_BLOCK 256

extern "C" __global__ void __launch_bounds__(HH_LUT_BLOCK) hh_lut_gemv(const hh_lut_args a) {
    __shared__ float2 tab[256];
    for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = make_float2(a.lut[i & 15u], a.lut[i >> 4]);
    __syncthreads();
    const uint32_t lane = threadIdx.x % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / HH_WAVE);
    const uint32_t waves = gridDim.x * (HH_LUT_BLOCK / HH_WAVE);
    const uint32_t pc = a.n / 2;  // packed bytes per row
    for (uint32_t row = blockIdx.x * (HH_LUT_BLOCK / HH_WAVE) + wave; row < a.m; row += waves) {
        const uint8_t* wr = a.w + (size_t)row * pc;
        float s = 0.f;
        if (a.vec) {
            const float4* x4 = reinterpret_cast<const float4*>(a.x);
            for (uint32_t c = lane; c < pc / 4; c += HH_WAVE) {
                const uint32_t q = *reinterpret_cast<const uint32_t*>(wr + 4 * (size_t)c);
                const float4 x0 = x4[2 * c], x1 = x4[2 * c + 1];
                const float2 t0 = tab[q & 255u], t1 = tab[(q >> 8) & 255u];
                const float2 t2 = tab[(q >> 16) & 255u], t3 = tab[q >> 24];
                s += x0.x * t0.x + x0.y * t0.y;
                s += x0.z * t1.x + x0.w * t1.y;
                s += x1.x * t2.x + x1.y * t2.y;
                s += x1.z * t3.x + x1.w * t3.y;
            }
        } else {
            for (uint32_t c = lane; c < pc; c += HH_WAVE) {
                const float2 t = tab[wr[c]];
                s += a.x[2 * c] * t.x + a.x[2 * c + 1] * t.y;
            }
        }
        s = hh_wave_sum(s);
        if (lane == 0) a.y[row] = s;
    }
}
