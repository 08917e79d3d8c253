// The FFN's neighbours for layouts the ring kernels do not cover (the ring kernels fuse
// both into their own prologue / epilogue):
//   hh_rmsnorm_kernel: y = x * (1 / sqrt(mean(x^2) + eps)) * w  (rms_norm,
//                      crates/hayai-cpu/src/attention.rs:142-147)
//   hh_add_kernel:     y = a + b  (the residual add of ffn_apply,
//                      crates/hayai-core/src/hybrid_infer.rs:930-932)
// (Compiled after q4k.hip in the same translation unit: uses hh_wave_sum.)

// One workgroup of 1024 threads: strided sums of squares, a wave reduction, the 16 wave
// sums added in order from LDS, then every element scaled.
extern "C" __global__ void __launch_bounds__(1024) hh_rmsnorm_kernel(const hh_norm_args a) {
    __shared__ float red[16];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < a.n; i += 1024) ss += a.x[i] * a.x[i];
    ss = hh_wave_sum(ss);
    if (threadIdx.x % HH_WAVE == 0) red[threadIdx.x / HH_WAVE] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) tot += red[k];
    const float inv = 1.0f / sqrtf(tot / (float)a.n + a.eps);
    for (uint32_t i = threadIdx.x; i < a.n; i += 1024) a.y[i] = (a.x[i] * inv) * a.w[i];
}

extern "C" __global__ void __launch_bounds__(256) hh_add_kernel(const hh_add_args a) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.y[i] = a.a[i] + a.b[i];
}
