// Device helpers shared by the gfx950 kernels (wave64, CDNA4).
//
// All kernel sources are compiled with -ffp-contract=off: every a*b+c below is two
// rounded operations unless it is written as an explicit fmaf(), which is how the
// dequant probes reproduce the reference's unfused arithmetic bit for bit while the
// GEMV accumulations use FMA where they choose to.
#ifndef HH_KERNELS_COMMON_H
#define HH_KERNELS_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kargs.h"

#define HH_DEV __device__ __forceinline__
#define HH_WAVE 64

// IEEE binary16 bits -> f32 with the hardware converter (v_cvt_f32_f16).  For every
// non-NaN code this equals the reference's bit-manipulation decode
// (crates/hayai-model/src/gguf.rs:521-545); the dequant probe test checks all 65536.
HH_DEV float hh_f16(uint32_t bits) {
    _Float16 h;
    const uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// Byte k of a dword as float.  The compiler selects v_cvt_f32_ubyte{0..3}.
HH_DEV float hh_ub0(uint32_t v) { return (float)(v & 0xFFu); }
HH_DEV float hh_ub1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
HH_DEV float hh_ub2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
HH_DEV float hh_ub3(uint32_t v) { return (float)(v >> 24); }

// 16-byte global load of an address known to be 16-byte aligned.
HH_DEV uint4 hh_ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Little-endian u16 / u32 from a 2-byte aligned address.
HH_DEV uint32_t hh_ld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
HH_DEV uint32_t hh_ld_u32_a2(const uint8_t* p) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}

// Sum over an aligned group of TEAM lanes (TEAM <= 64) of one wave.
template <int TEAM>
HH_DEV float hh_team_sum(float v) {
#pragma unroll
    for (int off = TEAM / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, HH_WAVE);
    return v;
}

// KSIGNS_IQ2XS[i] (crates/hayai-model/src/iq2.rs:18-27) equals i | (parity(i) << 7).
HH_DEV uint32_t hh_ksign(uint32_t i7) { return i7 | ((uint32_t)(__builtin_popcount(i7) & 1) << 7); }

// SiLU(g) * u as the reference writes it (stream_infer.rs:3836-3840), or the tanh GELU
// of ffn_finish_gelu_scratch (stream_infer.rs:3889-3895).
HH_DEV float hh_act_mul(float g, float u, int act) {
    if (act == HH_ACT_GELU_TANH) {
        const float k = sqrtf(2.0f / 3.14159265358979323846f);  // f32 ops, as the reference
        float x3 = g * g * g;
        float inner = k * (g + 0.044715f * x3);
        return 0.5f * g * (1.0f + tanhf(inner)) * u;
    }
    return (g / (1.0f + expf(-g))) * u;
}

#endif
