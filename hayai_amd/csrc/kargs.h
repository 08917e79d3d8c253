// Kernel argument blocks shared by the host runtime and the gfx950 kernels.
//
// Every kernel takes exactly one of these structs by value; the host passes its address
// as the single entry of hipModuleLaunchKernel's kernelParams.  Plain C layout only.
#ifndef HH_KARGS_H
#define HH_KARGS_H

#include <stdint.h>

#define HH_TYPE_F32 0
#define HH_TYPE_F16 1
#define HH_TYPE_Q4_0 2
#define HH_TYPE_Q8_0 8
#define HH_TYPE_Q4_K 12
#define HH_TYPE_Q6_K 14
#define HH_TYPE_IQ2_XXS 16
#define HH_TYPE_IQ3_XXS 18

#define HH_ACT_SILU 0
#define HH_ACT_GELU_TANH 1

// y[m] = W[m x n] . x[n]   (one GEMV; W row-major GGUF blocks along n)
struct hh_gemv_args {
    const uint8_t* w;  // first byte of row 0
    const float* x;    // n floats
    float* y;          // m floats
    uint32_t m;
    uint32_t n;
    uint64_t row_bytes;
};

// h[m] = act(Wg . x) * (Wu . x)   (fused gate/up GEMV + SwiGLU/GELU)
struct hh_gateup_args {
    const uint8_t* wg;
    const uint8_t* wu;
    const float* x;
    float* h;
    uint32_t m;  // d_ff
    uint32_t n;  // d_model
    uint64_t row_bytes;
    int32_t act;
    int32_t pad;
};

// h[i] = act(g[i]) * u[i]
struct hh_act_args {
    const float* g;
    const float* u;
    float* h;
    uint32_t n;
    int32_t act;
};

// y = RMSNorm(x) * w over n elements (one workgroup)
struct hh_norm_args {
    const float* x;
    const float* w;
    float* y;
    uint32_t n;
    float eps;
};

// x (n f32) -> q1[n] | q2[n] int8 | scale[n/8] f32, the ring down kernels' digit form
struct hh_xd_args {
    const float* x;
    uint8_t* hx;
    uint32_t n;
    uint32_t pad;
};

// y = a + b over n elements (the residual add)
struct hh_add_args {
    const float* a;
    const float* b;
    float* y;
    uint32_t n;
    uint32_t pad;
};

// out[n] = dequant(w[...]) for n elements (the dequant probe)
struct hh_dequant_args {
    const uint8_t* w;
    float* out;
    uint64_t n;
};

// Synthetic GGUF bytes: splitmix64 stream, then f16 scale fields drawn U(lo, hi).
struct hh_synth_args {
    uint8_t* dst;
    uint64_t nbytes;     // bytes of the random stream (whole blocks)
    uint64_t seed;
    uint64_t nblocks;    // blocks whose scale fields are patched
    int32_t type;
    float lo;
    float hi;
    int32_t pad;
};

#endif
