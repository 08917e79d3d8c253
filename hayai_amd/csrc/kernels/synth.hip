// Synthetic GGUF weight streams for benchmarks and parity tests (device side).
//
// Byte j of a stream with seed s is byte (j % 8) of mix64(s + (j/8 + 1) * 0x9E3779B97F4A7C15)
// (splitmix64 at a counter), so any slice can be generated independently.  After the byte
// stream, every f16 scale field k of the format is overwritten with
// f16_rne((float)(lo + (hi - lo) * u_k)), u_k = (mix64 stream of seed ^ HH_SCALE_SALT at
// counter k) >> 11 scaled by 2^-53, in double (lo/hi are the f32 arguments widened).
// hayai_amd/synth.py is the host twin; the GPU tests compare the two byte for byte.
#include "common.h"

#define HH_GOLDEN 0x9E3779B97F4A7C15ull
#define HH_SCALE_SALT 0xD1B54A32D192ED03ull

HH_DEV uint64_t hh_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

HH_DEV uint64_t hh_synth_u64(uint64_t seed, uint64_t i) { return hh_mix64(seed + (i + 1) * HH_GOLDEN); }

// Word-granular fill; dst must be 8-byte aligned (checked on the host).
extern "C" __global__ void __launch_bounds__(256) hh_synth_bytes(const hh_synth_args a) {
    const uint64_t nwords = (a.nbytes + 7) / 8;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < nwords; i += (uint64_t)gridDim.x * 256) {
        const uint64_t v = hh_synth_u64(a.seed, i);
        if (8 * i + 8 <= a.nbytes) {
            *reinterpret_cast<uint64_t*>(a.dst + 8 * i) = v;
        } else {
            for (uint64_t j = 8 * i; j < a.nbytes; j++) a.dst[j] = (uint8_t)(v >> (8 * (j - 8 * i)));
        }
    }
}

HH_DEV uint16_t hh_synth_scale(const hh_synth_args& a, uint64_t field) {
    const double u = (double)(hh_synth_u64(a.seed ^ HH_SCALE_SALT, field) >> 11) * 0x1.0p-53;
    const double lo = (double)a.lo, hi = (double)a.hi;
    const float v = (float)(lo + (hi - lo) * u);
    const _Float16 h = (_Float16)v;  // v_cvt_f16_f32, round to nearest even
    uint16_t bits;
    __builtin_memcpy(&bits, &h, 2);
    return bits;
}

HH_DEV void hh_put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFFu);
    p[1] = (uint8_t)(v >> 8);
}

// Patch the f16 scale fields: Q4_K d (field 2b) and dmin (field 2b+1); Q4_0 / Q8_0 /
// IQ2_XXS / IQ3_XXS d (field b, at the block start); Q6_K d (field b, at byte 208).
extern "C" __global__ void __launch_bounds__(256) hh_synth_scales(const hh_synth_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= a.nblocks) return;
    switch (a.type) {
    case HH_TYPE_Q4_K:
        hh_put16(a.dst + b * 144, hh_synth_scale(a, 2 * b));
        hh_put16(a.dst + b * 144 + 2, hh_synth_scale(a, 2 * b + 1));
        break;
    case HH_TYPE_Q4_0: hh_put16(a.dst + b * 18, hh_synth_scale(a, b)); break;
    case HH_TYPE_IQ2_XXS: hh_put16(a.dst + b * 66, hh_synth_scale(a, b)); break;
    case HH_TYPE_IQ3_XXS: hh_put16(a.dst + b * 98, hh_synth_scale(a, b)); break;
    case HH_TYPE_Q8_0: hh_put16(a.dst + b * 34, hh_synth_scale(a, b)); break;
    case HH_TYPE_Q6_K: hh_put16(a.dst + b * 210 + 208, hh_synth_scale(a, b)); break;
    default: break;
    }
}
