// Dequant probes: one thread per GGUF block writes that block's f32 weights, computed with
// the reference's exact operation order and no contraction (this file is built with
// -ffp-contract=off), so the output is bit-identical to hayai-model's dequant:
//   Q4_0    (float)(q - 8) * d                                  gguf.rs:348-372
//   Q4_K    (d*sc)*q - (dmin*m)                                 q4k.rs:178-203
//   Q8_0    (float)(i8)q * d                                    gguf.rs:401-420
//   Q6_K    (d*sc)*(q - 32)                                     q6k.rs:27-57
//   IQ2_XXS ((d*(0.5+s))*0.25 * g) * (+-1)                      iq2.rs:504-523
//   IQ3_XXS ((d*(0.5+s))*0.5 * g) * (+-1)                       iq3.rs:147-173
//   F16     IEEE binary16 -> f32                                gguf.rs:521-545
// The hardware f16 converter is used for d/dmin; the F16 probe run over all 65536 codes
// is what shows it equal to the reference's bit-manipulation decode.
#include "quant.h"

HH_DEV float hh_signed_mul(float db, uint32_t g, uint32_t signs, int j) {
    const float s = ((signs >> j) & 1u) ? -1.0f : 1.0f;
    return db * (float)g * s;
}

extern "C" __global__ void __launch_bounds__(256) hh_dequant_q4_0(const hh_dequant_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t nblk = (a.n + 31) / 32;
    if (b >= nblk) return;
    const uint8_t* blk = a.w + b * 18;
    const float d = hh_f16(hh_ld_u16(blk));
    for (int j = 0; j < 16; j++) {
        const uint32_t q = blk[2 + j];
        const uint64_t i0 = b * 32 + j, i1 = b * 32 + j + 16;
        if (i0 < a.n) a.out[i0] = (float)((int)(q & 0x0Fu) - 8) * d;
        if (i1 < a.n) a.out[i1] = (float)((int)(q >> 4) - 8) * d;
    }
}

extern "C" __global__ void __launch_bounds__(256) hh_dequant_q4_k(const hh_dequant_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= a.n / 256) return;
    const uint8_t* blk = a.w + b * 144;
    uint4 h;
    __builtin_memcpy(&h, blk, 16);
    const float d = hh_f16(h.x & 0xFFFFu);
    const float mn = hh_f16(h.x >> 16);
    float* y = a.out + b * 256;
    for (uint32_t g = 0; g < 4; g++) {
        uint32_t sc0, m0, sc1, m1;
        QK4<false>::scales(h, g, sc0, m0, sc1, m1);
        const float d1 = d * (float)sc0;
        const float m1v = mn * (float)m0;
        const float d2 = d * (float)sc1;
        const float m2v = mn * (float)m1;
        const uint8_t* q = blk + 16 + 32 * g;
        for (int l = 0; l < 32; l++) y[64 * g + l] = d1 * (float)(q[l] & 0x0Fu) - m1v;
        for (int l = 0; l < 32; l++) y[64 * g + 32 + l] = d2 * (float)(q[l] >> 4) - m2v;
    }
}

extern "C" __global__ void __launch_bounds__(256) hh_dequant_q8_0(const hh_dequant_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t nblk = (a.n + 31) / 32;
    if (b >= nblk) return;
    const uint8_t* blk = a.w + b * 34;
    const float d = hh_f16(hh_ld_u16(blk));
    for (int j = 0; j < 32; j++) {
        const uint64_t i = b * 32 + j;
        if (i < a.n) a.out[i] = (float)(int8_t)blk[2 + j] * d;
    }
}

// One thread per superblock; element order and products as dequant_q6_k_block.
extern "C" __global__ void __launch_bounds__(256) hh_dequant_q6_k(const hh_dequant_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= a.n / 256) return;
    const uint8_t* blk = a.w + b * 210;
    const float d = hh_f16(hh_ld_u16(blk + 208));
    float* y = a.out + b * 256;
    for (int h = 0; h < 2; h++) {
        const uint8_t* ql = blk + 64 * h;
        const uint8_t* qh = blk + 128 + 32 * h;
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * h);
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0x0Fu) | (((qh[l] >> 0) & 3u) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0x0Fu) | (((qh[l] >> 2) & 3u) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3u) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3u) << 4)) - 32;
            y[128 * h + l] = d * (float)sc[is] * (float)q1;
            y[128 * h + l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[128 * h + l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[128 * h + l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) hh_dequant_iq2_xxs(const hh_dequant_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= a.n / 256) return;
    const uint8_t* blk = a.w + b * 66;
    const float d = hh_f16(hh_ld_u16(blk));
    float* y = a.out + b * 256;
    for (int ib = 0; ib < 8; ib++) {
        const uint32_t aux0 = hh_ld_u32_a2(blk + 2 + 8 * ib);
        const uint32_t aux1 = hh_ld_u32_a2(blk + 6 + 8 * ib);
        const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const uint64_t g = hh_iq2xxs_grid[(aux0 >> (8 * l)) & 0xFFu];
            const uint32_t signs = hh_ksign((aux1 >> (7 * l)) & 127u);
            for (int j = 0; j < 8; j++)
                y[32 * ib + 8 * l + j] = hh_signed_mul(db, (uint32_t)(g >> (8 * j)) & 0xFFu, signs, j);
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) hh_dequant_iq3_xxs(const hh_dequant_args a) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= a.n / 256) return;
    const uint8_t* blk = a.w + b * 98;
    const float d = hh_f16(hh_ld_u16(blk));
    const uint8_t* qs = blk + 2;
    float* y = a.out + b * 256;
    for (int ib = 0; ib < 8; ib++) {
        const uint32_t aux = hh_ld_u32_a2(blk + 66 + 4 * ib);
        const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            const uint32_t signs = hh_ksign((aux >> (7 * l)) & 127u);
            const uint32_t g1 = hh_iq3xxs_grid[qs[8 * ib + 2 * l]];
            const uint32_t g2 = hh_iq3xxs_grid[qs[8 * ib + 2 * l + 1]];
            for (int j = 0; j < 4; j++) {
                y[32 * ib + 8 * l + j] = hh_signed_mul(db, (g1 >> (8 * j)) & 0xFFu, signs, j);
                y[32 * ib + 8 * l + 4 + j] = hh_signed_mul(db, (g2 >> (8 * j)) & 0xFFu, signs, j + 4);
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) hh_dequant_f16(const hh_dequant_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.out[i] = hh_f16(hh_ld_u16(a.w + 2 * i));
}
