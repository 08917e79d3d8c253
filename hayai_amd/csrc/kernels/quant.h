// Per-format "unit" traits for the team GEMV kernels.
//
// A unit is the slice of one weight row that one lane owns: UNIT consecutive columns plus
// whatever block header they need.  A lane keeps the matching UNIT floats of x in
// registers for the whole kernel, so x is read once per team and the weight stream is
// the only HBM traffic.  Unit layouts (GGUF blocks, little endian):
//   Q4_K    unit = group g of a 144-byte superblock: header 16 B (d, dmin, scales[12])
//           + qs[32g .. 32g+32); 64 columns: low nibbles -> sub-block 2g, high -> 2g+1
//           (crates/hayai-model/src/q4k.rs:178-203)
//   Q4_0    unit = one 18-byte block, 32 columns (gguf.rs:348-372)
//   Q8_0    unit = one 34-byte block: d + 32 int8 codes (gguf.rs:401-420)
//   Q6_K    unit = quarter (h, is) of a 210-byte superblock: 16 columns of each of the four
//           32-column groups of half h, taken from ql[64h+16is..+16), ql[64h+32+16is..+16),
//           qh[32h+16is..+16), scales[8h+is+{0,2,4,6}] and d (q6k.rs:27-57)
//   IQ2_XXS unit = one 32-column sub-block ib of a 66-byte block: d + aux0/aux1
//           (iq2.rs:504-523)
//   IQ3_XXS unit = one 32-column sub-block ib of a 98-byte block: d + qs[8ib..8ib+8) +
//           scales/signs word ib (iq3.rs:147-173)
//   F32/F16 unit = 32 consecutive values (tests and non-quantized matrices)
//
// dot() returns the unit's contribution to the row sum in factored form, e.g. for Q4_K
// (d*sc)*sum(q*x) - (dmin*m)*sum(x): the same scale products the reference forms, applied
// once per 32 columns instead of per weight.  The dequant probes (dequant.hip) build the
// per-weight values exactly as the reference does; the GEMV is held to the FFN
// tolerance, not to bits (its summation order differs from any CPU order anyway).
#ifndef HH_KERNELS_QUANT_H
#define HH_KERNELS_QUANT_H

#include "common.h"
#include "../iq_grids.h"

__constant__ uint64_t hh_iq2xxs_grid[256] = {HH_IQ2XXS_GRID_VALUES};
__constant__ uint32_t hh_iq3xxs_grid[256] = {HH_IQ3XXS_GRID_VALUES};

// Table staging in LDS: IQ formats gather grid entries per 8 columns; LDS beats the
// scalar constant cache for per-lane divergent indices.
struct hh_tables {
    uint64_t g2[256];
    uint32_t g3[256];
};

// ------------------------------------------------------------------------ Q4_K ------
template <bool ALIGNED>
struct QK4 {
    static constexpr uint32_t UNIT = 64;
    static constexpr uint32_t BLOCK = 256;
    static constexpr uint32_t BLOCK_BYTES = 144;
    static constexpr bool TABLES = false;
    struct Data {
        uint4 h, q0, q1;
    };
    struct X {
        float v[64];
        float s0, s1;
    };

    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 144;
        const uint8_t* q = blk + 16 + (u & 3) * 32;
        Data d;
        if (ALIGNED) {
            d.h = hh_ld16(blk);
            d.q0 = hh_ld16(q);
            d.q1 = hh_ld16(q + 16);
        } else {
            __builtin_memcpy(&d.h, blk, 16);
            __builtin_memcpy(&d.q0, q, 16);
            __builtin_memcpy(&d.q1, q + 16, 16);
        }
        return d;
    }

    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 64;
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            xr.v[i] = p[i];
            s0 += xr.v[i];
        }
#pragma unroll
        for (int i = 32; i < 64; i++) {
            xr.v[i] = p[i];
            s1 += xr.v[i];
        }
        xr.s0 = s0;
        xr.s1 = s1;
    }

    // (sc, m) of sub-blocks 2g and 2g+1 from the 12 scale bytes held in h.y/h.z/h.w;
    // get_scale_min_k4, crates/hayai-model/src/q4k.rs:34-43.
    static HH_DEV void scales(const uint4& h, uint32_t g, uint32_t& sc0, uint32_t& m0, uint32_t& sc1,
                              uint32_t& m1) {
        const uint32_t sh = (g & 1u) * 16u;  // byte pair 2(g&1) of each scale word
        const uint32_t y2 = (h.y >> sh) & 0xFFFFu;  // s[j'], s[j'+1]        (j' = 2(g&1))
        const uint32_t z2 = (h.z >> sh) & 0xFFFFu;  // s[j'+4], s[j'+5]
        const uint32_t w2 = (h.w >> sh) & 0xFFFFu;  // s[j'+8], s[j'+9]
        // j < 4: sc = s[j] & 63, m = s[j+4] & 63
        const uint32_t lo_sc0 = y2 & 63u, lo_sc1 = (y2 >> 8) & 63u;
        const uint32_t lo_m0 = z2 & 63u, lo_m1 = (z2 >> 8) & 63u;
        // j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m = (s[j+4] >> 4) | (s[j] >> 6) << 4
        const uint32_t hi_sc0 = (w2 & 15u) | (((y2 >> 6) & 3u) << 4);
        const uint32_t hi_sc1 = ((w2 >> 8) & 15u) | (((y2 >> 14) & 3u) << 4);
        const uint32_t hi_m0 = ((w2 >> 4) & 15u) | (((z2 >> 6) & 3u) << 4);
        const uint32_t hi_m1 = ((w2 >> 12) & 15u) | (((z2 >> 14) & 3u) << 4);
        const bool hi = g >= 2;
        sc0 = hi ? hi_sc0 : lo_sc0;
        sc1 = hi ? hi_sc1 : lo_sc1;
        m0 = hi ? hi_m0 : lo_m0;
        m1 = hi ? hi_m1 : lo_m1;
    }

    static HH_DEV float dot(const Data& d, const X& xr, uint32_t u, const hh_tables*) {
        uint32_t sc0, m0, sc1, m1;
        scales(d.h, u & 3u, sc0, m0, sc1, m1);
        const float dd = hh_f16(d.h.x & 0xFFFFu);
        const float dm = hh_f16(d.h.x >> 16);
        const float d1 = dd * (float)sc0;
        const float m1v = dm * (float)m0;
        const float d2 = dd * (float)sc1;
        const float m2v = dm * (float)m1;
        const uint32_t qw[8] = {d.q0.x, d.q0.y, d.q0.z, d.q0.w, d.q1.x, d.q1.y, d.q1.z, d.q1.w};
        float al0 = 0.f, al1 = 0.f, ah0 = 0.f, ah1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const uint32_t l0 = qw[i] & 0x0F0F0F0Fu, h0 = qw[i] & 0xF0F0F0F0u;  // h = 16*q
            const uint32_t l1 = qw[i + 1] & 0x0F0F0F0Fu, h1 = qw[i + 1] & 0xF0F0F0F0u;
            const float* xl = xr.v + 4 * i;
            const float* xh = xr.v + 32 + 4 * i;
            al0 = fmaf(hh_ub0(l0), xl[0], al0);
            al0 = fmaf(hh_ub1(l0), xl[1], al0);
            al0 = fmaf(hh_ub2(l0), xl[2], al0);
            al0 = fmaf(hh_ub3(l0), xl[3], al0);
            al1 = fmaf(hh_ub0(l1), xl[4], al1);
            al1 = fmaf(hh_ub1(l1), xl[5], al1);
            al1 = fmaf(hh_ub2(l1), xl[6], al1);
            al1 = fmaf(hh_ub3(l1), xl[7], al1);
            ah0 = fmaf(hh_ub0(h0), xh[0], ah0);
            ah0 = fmaf(hh_ub1(h0), xh[1], ah0);
            ah0 = fmaf(hh_ub2(h0), xh[2], ah0);
            ah0 = fmaf(hh_ub3(h0), xh[3], ah0);
            ah1 = fmaf(hh_ub0(h1), xh[4], ah1);
            ah1 = fmaf(hh_ub1(h1), xh[5], ah1);
            ah1 = fmaf(hh_ub2(h1), xh[6], ah1);
            ah1 = fmaf(hh_ub3(h1), xh[7], ah1);
        }
        const float al = al0 + al1;
        const float ah = (ah0 + ah1) * 0.0625f;  // exact: undo the 16x of the high nibble
        return (d1 * al - m1v * xr.s0) + (d2 * ah - m2v * xr.s1);
    }
};

// ------------------------------------------------------------------------ Q4_0 ------
struct Q40 {
    static constexpr uint32_t UNIT = 32;
    static constexpr uint32_t BLOCK = 32;
    static constexpr uint32_t BLOCK_BYTES = 18;
    static constexpr bool TABLES = false;
    struct Data {
        uint32_t d;
        uint32_t q[4];
    };
    struct X {
        float v[32];
        float s;
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* blk = row + (size_t)u * 18;  // 2-byte aligned
        Data d;
        d.d = hh_ld_u16(blk);
#pragma unroll
        for (int i = 0; i < 4; i++) d.q[i] = hh_ld_u32_a2(blk + 2 + 4 * i);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 32;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            xr.v[i] = p[i];
            s += xr.v[i];
        }
        xr.s = s;
    }
    // d * sum((q - 8) x) = d * (sum(q x) - 8 sum(x)); low nibbles are columns 0..15,
    // high nibbles 16..31 (gguf.rs:360-368).
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables*) {
        float al = 0.f, ah = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l = d.q[i] & 0x0F0F0F0Fu, h = d.q[i] & 0xF0F0F0F0u;
            al = fmaf(hh_ub0(l), xr.v[4 * i + 0], al);
            al = fmaf(hh_ub1(l), xr.v[4 * i + 1], al);
            al = fmaf(hh_ub2(l), xr.v[4 * i + 2], al);
            al = fmaf(hh_ub3(l), xr.v[4 * i + 3], al);
            ah = fmaf(hh_ub0(h), xr.v[16 + 4 * i + 0], ah);
            ah = fmaf(hh_ub1(h), xr.v[16 + 4 * i + 1], ah);
            ah = fmaf(hh_ub2(h), xr.v[16 + 4 * i + 2], ah);
            ah = fmaf(hh_ub3(h), xr.v[16 + 4 * i + 3], ah);
        }
        return hh_f16(d.d) * ((al + ah * 0.0625f) - 8.0f * xr.s);
    }
};

// ------------------------------------------------------------------------ Q8_0 ------
struct Q80 {
    static constexpr uint32_t UNIT = 32;
    static constexpr uint32_t BLOCK = 32;
    static constexpr uint32_t BLOCK_BYTES = 34;
    static constexpr bool TABLES = false;
    struct Data {
        uint32_t d;
        uint32_t q[8];
    };
    struct X {
        float v[32];
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* blk = row + (size_t)u * 34;  // 2-byte aligned
        Data d;
        d.d = hh_ld_u16(blk);
#pragma unroll
        for (int i = 0; i < 8; i++) d.q[i] = hh_ld_u32_a2(blk + 2 + 4 * i);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 32;
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[i];
    }
    // d * sum(q x) over the block's 32 signed codes
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables*) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int32_t w = (int32_t)d.q[i];
            float& a = (i & 1) ? a1 : a0;
            a = fmaf((float)((w << 24) >> 24), xr.v[4 * i + 0], a);
            a = fmaf((float)((w << 16) >> 24), xr.v[4 * i + 1], a);
            a = fmaf((float)((w << 8) >> 24), xr.v[4 * i + 2], a);
            a = fmaf((float)(w >> 24), xr.v[4 * i + 3], a);
        }
        return hh_f16(d.d) * (a0 + a1);
    }
};

// ------------------------------------------------------------------------ Q6_K ------
struct QK6 {
    static constexpr uint32_t UNIT = 64;
    static constexpr uint32_t BLOCK = 256;
    static constexpr uint32_t BLOCK_BYTES = 210;
    static constexpr bool TABLES = false;
    struct Data {
        uint32_t la[4], lb[4], h[4];  // ql run (groups 0, 2), ql run (groups 1, 3), qh run
        uint32_t sc;                  // scales of groups 0..3 (i8 bytes)
        uint32_t d;
    };
    struct X {
        float v[64];  // 16 columns of each group, group r at v[16r..16r+16)
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* blk = row + (size_t)(u >> 2) * 210;  // 2-byte aligned
        const uint32_t hh = (u >> 1) & 1u, is = u & 1u;
        const uint8_t* qa = blk + 64 * hh + 16 * is;
        const uint8_t* qh = blk + 128 + 32 * hh + 16 * is;
        Data d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.la[i] = hh_ld_u32_a2(qa + 4 * i);
            d.lb[i] = hh_ld_u32_a2(qa + 32 + 4 * i);
            d.h[i] = hh_ld_u32_a2(qh + 4 * i);
        }
        const uint8_t* sc = blk + 192 + 8 * hh + is;
        d.sc = (uint32_t)sc[0] | ((uint32_t)sc[2] << 8) | ((uint32_t)sc[4] << 16) | ((uint32_t)sc[6] << 24);
        d.d = hh_ld_u16(blk + 208);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)(u >> 2) * 256 + 128 * ((u >> 1) & 1u) + 16 * (u & 1u);
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int l = 0; l < 16; l++) xr.v[16 * r + l] = p[32 * r + l];
    }
    // d * sum_r sc_r * sum_l (q - 32) x over the four groups (q = 4 low bits | 2 high bits)
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables*) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hb = d.h[i];
            // groups 0..3 of 4 columns: (ql low, qh bits 0-1), (ql' low, bits 2-3),
            // (ql high, bits 4-5), (ql' high, bits 6-7)
            const uint32_t q0 = (d.la[i] & 0x0F0F0F0Fu) | ((hb << 4) & 0x30303030u);
            const uint32_t q1 = (d.lb[i] & 0x0F0F0F0Fu) | ((hb << 2) & 0x30303030u);
            const uint32_t q2 = ((d.la[i] >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u);
            const uint32_t q3 = ((d.lb[i] >> 4) & 0x0F0F0F0Fu) | ((hb >> 2) & 0x30303030u);
            const uint32_t qq[4] = {q0, q1, q2, q3};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float* xv = xr.v + 16 * r + 4 * i;
                acc[r] = fmaf(hh_ub0(qq[r]) - 32.f, xv[0], acc[r]);
                acc[r] = fmaf(hh_ub1(qq[r]) - 32.f, xv[1], acc[r]);
                acc[r] = fmaf(hh_ub2(qq[r]) - 32.f, xv[2], acc[r]);
                acc[r] = fmaf(hh_ub3(qq[r]) - 32.f, xv[3], acc[r]);
            }
        }
        const int32_t sc = (int32_t)d.sc;
        const float s =
            (float)((sc << 24) >> 24) * acc[0] + (float)((sc << 16) >> 24) * acc[1] +
            (float)((sc << 8) >> 24) * acc[2] + (float)(sc >> 24) * acc[3];
        return hh_f16(d.d) * s;
    }
};

// --------------------------------------------------------------------- IQ2_XXS ------
struct QI2 {
    static constexpr uint32_t UNIT = 32;
    static constexpr uint32_t BLOCK = 256;
    static constexpr uint32_t BLOCK_BYTES = 66;
    static constexpr bool TABLES = true;
    struct Data {
        uint32_t d, a0, a1;
    };
    struct X {
        float v[32];
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 66;
        const uint8_t* q = blk + 2 + 8 * (u & 7u);
        Data d;
        d.d = hh_ld_u16(blk);
        d.a0 = hh_ld_u32_a2(q);
        d.a1 = hh_ld_u32_a2(q + 4);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 32;
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[i];
    }
    // db * sum(+-grid * x), db = d * (0.5 + aux1>>28) * 0.25 (iq2.rs:513).
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables* t) {
        const float db = hh_f16(d.d) * (0.5f + (float)(d.a1 >> 28)) * 0.25f;
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint64_t g = t->g2[(d.a0 >> (8 * l)) & 0xFFu];
            const uint32_t sg = hh_ksign((d.a1 >> (7 * l)) & 127u);
            const uint32_t glo = (uint32_t)g, ghi = (uint32_t)(g >> 32);
            const float gv[8] = {hh_ub0(glo), hh_ub1(glo), hh_ub2(glo), hh_ub3(glo),
                                 hh_ub0(ghi), hh_ub1(ghi), hh_ub2(ghi), hh_ub3(ghi)};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float xv = ((sg >> j) & 1u) ? -xr.v[8 * l + j] : xr.v[8 * l + j];
                s = fmaf(gv[j], xv, s);
            }
        }
        return db * s;
    }
};

// --------------------------------------------------------------------- IQ3_XXS ------
struct QI3 {
    static constexpr uint32_t UNIT = 32;
    static constexpr uint32_t BLOCK = 256;
    static constexpr uint32_t BLOCK_BYTES = 98;
    static constexpr bool TABLES = true;
    struct Data {
        uint32_t d, q0, q1, aux;
    };
    struct X {
        float v[32];
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 98;
        const uint32_t ib = u & 7u;
        Data d;
        d.d = hh_ld_u16(blk);
        d.q0 = hh_ld_u32_a2(blk + 2 + 8 * ib);
        d.q1 = hh_ld_u32_a2(blk + 6 + 8 * ib);
        d.aux = hh_ld_u32_a2(blk + 66 + 4 * ib);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 32;
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[i];
    }
    // db * sum(+-grid * x), db = d * (0.5 + aux>>28) * 0.5 (iq3.rs:160).
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables* t) {
        const float db = hh_f16(d.d) * (0.5f + (float)(d.aux >> 28)) * 0.5f;
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t qq = l < 2 ? d.q0 : d.q1;
            const uint32_t i1 = (qq >> (16 * (l & 1))) & 0xFFu;
            const uint32_t i2 = (qq >> (16 * (l & 1) + 8)) & 0xFFu;
            const uint32_t g1 = t->g3[i1], g2 = t->g3[i2];
            const uint32_t sg = hh_ksign((d.aux >> (7 * l)) & 127u);
            const float gv[8] = {hh_ub0(g1), hh_ub1(g1), hh_ub2(g1), hh_ub3(g1),
                                 hh_ub0(g2), hh_ub1(g2), hh_ub2(g2), hh_ub3(g2)};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float xv = ((sg >> j) & 1u) ? -xr.v[8 * l + j] : xr.v[8 * l + j];
                s = fmaf(gv[j], xv, s);
            }
        }
        return db * s;
    }
};

// -------------------------------------------------------------------- F32 / F16 -----
struct QF32 {
    static constexpr uint32_t UNIT = 32;
    static constexpr uint32_t BLOCK = 1;
    static constexpr uint32_t BLOCK_BYTES = 4;
    static constexpr bool TABLES = false;
    struct Data {
        uint4 v[8];
    };
    struct X {
        float v[32];
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* p = row + (size_t)u * 128;
        Data d;
#pragma unroll
        for (int i = 0; i < 8; i++) d.v[i] = hh_ld16(p + 16 * i);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 32;
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[i];
    }
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables*) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = fmaf(__uint_as_float(d.v[i].x), xr.v[4 * i + 0], s0);
            s1 = fmaf(__uint_as_float(d.v[i].y), xr.v[4 * i + 1], s1);
            s0 = fmaf(__uint_as_float(d.v[i].z), xr.v[4 * i + 2], s0);
            s1 = fmaf(__uint_as_float(d.v[i].w), xr.v[4 * i + 3], s1);
        }
        return s0 + s1;
    }
};

struct QF16 {
    static constexpr uint32_t UNIT = 32;
    static constexpr uint32_t BLOCK = 1;
    static constexpr uint32_t BLOCK_BYTES = 2;
    static constexpr bool TABLES = false;
    struct Data {
        uint4 v[4];
    };
    struct X {
        float v[32];
    };
    static HH_DEV Data load(const uint8_t* row, uint32_t u) {
        const uint8_t* p = row + (size_t)u * 64;
        Data d;
#pragma unroll
        for (int i = 0; i < 4; i++) d.v[i] = hh_ld16(p + 16 * i);
        return d;
    }
    static HH_DEV void load_x(const float* x, uint32_t u, X& xr) {
        const float* p = x + (size_t)u * 32;
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[i];
    }
    static HH_DEV float dot(const Data& d, const X& xr, uint32_t, const hh_tables*) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w[4] = {d.v[i].x, d.v[i].y, d.v[i].z, d.v[i].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 = fmaf(hh_f16(w[k] & 0xFFFFu), xr.v[8 * i + 2 * k], s0);
                s1 = fmaf(hh_f16(w[k] >> 16), xr.v[8 * i + 2 * k + 1], s1);
            }
        }
        return s0 + s1;
    }
};

#endif
