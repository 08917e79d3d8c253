/*
 * hayai_oracle.c -- CPU restatement of the Hayai FFN GEMV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP library: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and never
 * as the thing that is measured or shipped.  The product path (hayai_amd) does not link,
 * import or call anything here.
 *
 * Every function restates a function of the reference (aitups/hayai, Rust) and cites the
 * file:line it follows.  The reference cannot be compiled in this environment (no Rust
 * toolchain), so this is a restatement, not a build of it.
 *
 * Floating-point rules kept from the reference:
 *   - no contraction: this file is compiled with -ffp-contract=off, so a*b+c is two
 *     rounded operations exactly as in Rust (which never fuses);
 *   - std::simd f32x8 accumulators are emulated lane by lane, and `reduce_sum` is the
 *     ordered left-to-right lane sum;
 *   - per-row summation order is the Rust order (rayon only splits rows, never a row).
 *
 * Pinning (how each function is checked by tests/test_oracle.py):
 *   or_f16_to_f32        exhaustive over all 65536 codes vs numpy's IEEE conversion
 *   dequant (all types)  closed-form special cases from the reference's own tests
 *                        (Q4_K d=1,dmin=0,scales=1 -> w=nibble; Q4_0 d=0x2E66 -> (q-8)*d;
 *                        Q6_K d=1,scales=1 -> w=6-bit code-32; Q8_0 d=0x2E66 -> q*d),
 *                        the reference quantizer round trip (q4k.rs:319-350), scale
 *                        packing inverse over all 64x64 (sc,m), IQ sign parity and grid
 *                        invariants, golden fixtures in tests/golden/
 *   gemv (all types)     fp64 brute force bound, linearity in x, reference fixtures
 *   route_experts        the reference's own known-answer tests (moe_infer.rs:1039-1121)
 *   or_ffn, or_moe_token float64 compositions of the pinned dequant with numpy's exp,
 *                        under a propagated fp32 rounding bound; planted mistakes
 *                        (or_set_mutation) must fail the same checks
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "iq_grids.inc"

/* GGML type ids, crates/hayai-model/src/gguf_types.rs:6-78. */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14, OR_IQ2_XXS = 16, OR_IQ3_XXS = 18 };

/* Status codes shared with the ctypes wrapper. */
enum { OR_OK = 0, OR_EINVAL = 2 };

static int g_threads = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_num_procs();
#else
    return 1;
#endif
}

/* Planted mistakes for the tests that pin this oracle: a pin check must fail when one of
 * these is switched on (0 = none, 1 = or_ffn swaps gate and up, 2 = or_moe_token reads
 * expert ids[t] + 1 instead of ids[t], 3 = or_moe_shared swaps its gate and up). */
static int g_mutation = 0;

void or_set_mutation(int m) { g_mutation = m; }

/* ---------------------------------------------------------------- f16 ---------- */

/* IEEE binary16 -> f32 by bit manipulation; crates/hayai-model/src/gguf.rs:521-545.
 * Subnormals are normalised; Inf/NaN keep their payload (no sNaN quieting). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)((h >> 15) & 1u);
    uint32_t exp = (uint32_t)((h >> 10) & 0x1Fu);
    uint32_t mant = (uint32_t)(h & 0x3FFu);
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t m = mant;
            uint32_t e = 127 - 15 + 1;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            m &= 0x3FFu;
            bits = (sign << 31) | (e << 23) | (m << 13);
        }
    } else if (exp == 31) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void or_f16_to_f32_array(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(h[i]);
}

/* The reference's own f32 -> f16 (round half up on the dropped mantissa bits, not RNE);
 * crates/hayai-model/src/q4k.rs:46-83.  Used only by the reference quantizer below. */
uint16_t or_f32_to_f16_ref(float value) {
    uint32_t f;
    memcpy(&f, &value, 4);
    uint32_t sign = (f >> 16) & 0x8000u;
    int32_t exponent = (int32_t)((f >> 23) & 0xffu) - 127 + 15;
    uint32_t mantissa = f & 0x7fffffu;
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        uint32_t m = mantissa | 0x800000u;
        uint32_t shift = (uint32_t)(14 - exponent);
        uint32_t sm1 = shift == 0 ? 0 : shift - 1;
        m = m >> shift;
        if (mantissa & (1u << sm1)) m += 1;
        return (uint16_t)(sign | m);
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    uint32_t m = mantissa >> 13;
    if (mantissa & 0x1000u) m += 1;
    if ((m & 0x400u) == 0x400u) {
        m = 0;
        exponent += 1;
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)exponent << 10) | m);
}

static inline float f16le(const uint8_t* p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

static inline uint32_t u32le(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Ordered lane sum of an f32x8; core::simd `reduce_sum` (simd_reduce_add_ordered). */
static inline float reduce_sum8(const float a[8]) {
    float r = 0.0f;
    for (int i = 0; i < 8; i++) r = r + a[i];
    return r;
}

/* ------------------------------------------------------ shape validation ---------- */

/* Block geometry per GGML type; crates/hayai-opencl/src/compute.rs:877-907 (gemv_row_bytes). */
static int block_geom(int type, size_t* block, size_t* bytes) {
    switch (type) {
    case OR_Q4_0: *block = 32; *bytes = 18; return 1;
    case OR_Q8_0: *block = 32; *bytes = 34; return 1;
    case OR_Q4_K: *block = 256; *bytes = 144; return 1;
    case OR_Q6_K: *block = 256; *bytes = 210; return 1;
    case OR_IQ2_XXS: *block = 256; *bytes = 66; return 1;
    case OR_IQ3_XXS: *block = 256; *bytes = 98; return 1;
    case OR_F32: *block = 1; *bytes = 4; return 1;
    case OR_F16: *block = 1; *bytes = 2; return 1;
    default: return 0;
    }
}

/* Packed bytes per row for n columns into *out; OR_EINVAL for an unknown type or an n
 * that is not a block multiple (n == 0 is a valid 0-byte row); compute.rs:877-907. */
int or_row_bytes(int type, size_t n, size_t* out) {
    size_t block, bytes;
    if (!block_geom(type, &block, &bytes)) return OR_EINVAL;
    if (n % block != 0) return OR_EINVAL;
    *out = (n / block) * bytes;
    return OR_OK;
}

static size_t row_bytes_or0(int type, size_t n) {
    size_t r = 0;
    return or_row_bytes(type, n, &r) == OR_OK ? r : 0;
}

/* compute.rs:935-949 (validate_gemv_shape): m,n > 0 and n a block multiple. */
int or_validate_shape(int type, size_t m, size_t n) {
    size_t r;
    if (m == 0 || n == 0) return OR_EINVAL;
    return or_row_bytes(type, n, &r);
}

/* compute.rs:912-931 (validate_gemv_weights): buffer >= m * row_bytes (checked). */
int or_validate_weights(int type, size_t m, size_t n, size_t len) {
    size_t row;
    if (or_row_bytes(type, n, &row) != OR_OK) return OR_EINVAL;
    if (m != 0 && row > SIZE_MAX / m) return OR_EINVAL;
    if (len < m * row) return OR_EINVAL;
    return OR_OK;
}

/* --------------------------------------------------------------- dequant ---------- */

/* Q4_0 dequant; crates/hayai-model/src/gguf.rs:348-372. */
static void dequant_q4_0_block(const uint8_t* blk, float* y) {
    float d = f16le(blk);
    const uint8_t* qs = blk + 2;
    for (int j = 0; j < 16; j++) {
        int x0 = (int)(qs[j] & 0x0F) - 8;
        int x1 = (int)(qs[j] >> 4) - 8;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}

/* Q8_0 dequant: (i8 q) * d; crates/hayai-model/src/gguf.rs:401-420. */
static void dequant_q8_0_block(const uint8_t* blk, float* y) {
    float d = f16le(blk);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)blk[2 + j] * d;
}

/* Q6_K dequant; crates/hayai-model/src/q6k.rs:27-57.  Block: ql[128] | qh[64] | scales[16]
 * (i8) | d (f16).  Two halves of 128 elements; in half h, l in 0..32 gives the elements
 * l, l+32, l+64, l+96 from ql[64h+l] / ql[64h+l+32] (low, then high nibbles) and bit pairs
 * 0,2,4,6 of qh[32h+l], each minus 32, scaled by (d * scales[8h + l/16 + 0,2,4,6]). */
static void dequant_q6_k_block(const uint8_t* blk, float* y) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    float d = f16le(blk + 208);
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)(int8_t)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)(int8_t)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

/* get_scale_min_k4; crates/hayai-model/src/q4k.rs:34-43. */
void or_get_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* dequant_q4_k_block; crates/hayai-model/src/q4k.rs:178-203.
 * y = (d*sc)*q - (dmin*m), each product rounded on its own. */
static void dequant_q4_k_block(const uint8_t* blk, float* y) {
    float d = f16le(blk);
    float mn = f16le(blk + 2);
    const uint8_t* scales = blk + 4;
    const uint8_t* q = blk + 16;
    int is = 0, yo = 0;
    for (int g = 0; g < 4; g++) {
        uint8_t sc0, m0, sc1, m1;
        or_get_scale_min_k4(is, scales, &sc0, &m0);
        or_get_scale_min_k4(is + 1, scales, &sc1, &m1);
        float d1 = d * (float)sc0;
        float m1v = mn * (float)m0;
        float d2 = d * (float)sc1;
        float m2v = mn * (float)m1;
        for (int l = 0; l < 32; l++) y[yo + l] = d1 * (float)(q[l] & 0x0F) - m1v;
        yo += 32;
        for (int l = 0; l < 32; l++) y[yo + l] = d2 * (float)(q[l] >> 4) - m2v;
        yo += 32;
        q += 32;
        is += 2;
    }
}

static inline uint8_t ksign(uint32_t i7) {
    /* KSIGNS_IQ2XS[i] == i | (parity(i) << 7) (iq2.rs:18-27; checked against the table
     * values in tests/golden). */
    return (uint8_t)(i7 | ((uint32_t)(__builtin_popcount(i7) & 1) << 7));
}

/* signed_mul: (db * g) * (+-1); crates/hayai-model/src/iq2.rs:487-495. */
static inline float signed_mul(float db, uint8_t g, uint8_t signs, int j) {
    float s = (signs & (1u << j)) ? -1.0f : 1.0f;
    return db * (float)g * s;
}

/* dequant_iq2_xxs_block; crates/hayai-model/src/iq2.rs:504-523. */
static void dequant_iq2_xxs_block(const uint8_t* blk, float* y) {
    float d = f16le(blk);
    const uint8_t* qs = blk + 2;
    int yo = 0;
    for (int ib = 0; ib < 8; ib++) {
        uint32_t aux0 = u32le(qs + 8 * ib);
        uint32_t aux1 = u32le(qs + 8 * ib + 4);
        float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint64_t g = OR_IQ2XXS_GRID[(aux0 >> (8 * l)) & 0xFF];
            uint8_t signs = ksign((aux1 >> (7 * l)) & 127);
            for (int j = 0; j < 8; j++) y[yo + j] = signed_mul(db, (uint8_t)(g >> (8 * j)), signs, j);
            yo += 8;
        }
    }
}

/* dequant_iq3_xxs_block; crates/hayai-model/src/iq3.rs:147-173. */
static void dequant_iq3_xxs_block(const uint8_t* blk, float* y) {
    float d = f16le(blk);
    const uint8_t* qs = blk + 2;
    const uint8_t* ss = blk + 66;
    int yo = 0, qoff = 0;
    for (int ib = 0; ib < 8; ib++) {
        uint32_t aux = u32le(ss + 4 * ib);
        float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            uint8_t signs = ksign((aux >> (7 * l)) & 127);
            uint32_t g1 = OR_IQ3XXS_GRID[qs[qoff + 2 * l]];
            uint32_t g2 = OR_IQ3XXS_GRID[qs[qoff + 2 * l + 1]];
            for (int j = 0; j < 4; j++) {
                y[yo + j] = signed_mul(db, (uint8_t)(g1 >> (8 * j)), signs, j);
                y[yo + 4 + j] = signed_mul(db, (uint8_t)(g2 >> (8 * j)), signs, j + 4);
            }
            yo += 8;
        }
        qoff += 8;
    }
}

/* Dequantize n elements of one tensor; gguf.rs:307-346 dispatch (the supported subset).
 * Returns OR_EINVAL on a short buffer or an n the block layout cannot hold. */
int or_dequant(int type, const uint8_t* bytes, size_t len, size_t n, float* out) {
    size_t block, bb;
    if (!block_geom(type, &block, &bb)) return OR_EINVAL;
    if (type == OR_F32) {
        if (len < n * 4) return OR_EINVAL;
        memcpy(out, bytes, n * 4);
        return OR_OK;
    }
    if (type == OR_F16) {
        if (len < n * 2) return OR_EINVAL;
        for (size_t i = 0; i < n; i++) out[i] = f16le(bytes + 2 * i);
        return OR_OK;
    }
    if (type != OR_Q4_0 && type != OR_Q8_0 && n % block != 0) return OR_EINVAL; /* q4k.rs:163, iq2.rs:577, q6k.rs:12 */
    size_t nblk = (n + block - 1) / block;
    if (len < nblk * bb) return OR_EINVAL;
    float tmp[256];
    for (size_t b = 0; b < nblk; b++) {
        const uint8_t* blk = bytes + b * bb;
        switch (type) {
        case OR_Q4_0: dequant_q4_0_block(blk, tmp); break;
        case OR_Q8_0: dequant_q8_0_block(blk, tmp); break;
        case OR_Q4_K: dequant_q4_k_block(blk, tmp); break;
        case OR_Q6_K: dequant_q6_k_block(blk, tmp); break;
        case OR_IQ2_XXS: dequant_iq2_xxs_block(blk, tmp); break;
        case OR_IQ3_XXS: dequant_iq3_xxs_block(blk, tmp); break;
        }
        size_t take = n - b * block < block ? n - b * block : block; /* Q4_0 / Q8_0 tail, gguf.rs:363-368,412-416 */
        memcpy(out + b * block, tmp, take * sizeof(float));
    }
    return OR_OK;
}

/* ------------------------------------------------------------------ GEMV ---------- */

/* gemv_q4_0 with f32x8 MAC per half-block; crates/hayai-model/src/quant.rs:538-574. */
static float row_q4_0(const uint8_t* row, size_t nb, const float* x) {
    float sum = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 18;
        float d = f16le(blk);
        const uint8_t* qs = blk + 2;
        float q_lo[16], q_hi[16];
        for (int j = 0; j < 16; j++) {
            q_lo[j] = (float)((int)(qs[j] & 0x0F) - 8);
            q_hi[j] = (float)((int)(qs[j] >> 4) - 8);
        }
        const float* xb = x + b * 32;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int chunk = 0; chunk < 2; chunk++) {
            int o = chunk * 8;
            for (int l = 0; l < 8; l++) {
                /* acc += ql * d_v * xl + qh * d_v * xh  (quant.rs:566) */
                float t0 = q_lo[o + l] * d * xb[o + l];
                float t1 = q_hi[o + l] * d * xb[16 + o + l];
                acc[l] = acc[l] + (t0 + t1);
            }
        }
        sum += reduce_sum8(acc);
    }
    return sum;
}

/* gemv_q4k_sub32; crates/hayai-model/src/q4k.rs:10-32.  The "magic number" nibble to
 * float conversion there is exact, so it is a plain int -> float here. */
static inline float q4k_sub32(float d, float minv, const uint8_t* q, const float* x, int high) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int chunk = 0; chunk < 4; chunk++) {
        int o = chunk * 8;
        for (int l = 0; l < 8; l++) {
            uint8_t by = q[o + l];
            float f = (float)(high ? (by >> 4) : (by & 0x0F));
            float wv = f * d - minv;
            acc[l] = acc[l] + wv * x[o + l];
        }
    }
    return reduce_sum8(acc);
}

/* gemv_q4_k row; crates/hayai-model/src/q4k.rs:233-253. */
static float row_q4_k(const uint8_t* row, size_t nb, const float* x) {
    float sum = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 144;
        float d = f16le(blk);
        float mn = f16le(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* q = blk + 16;
        const float* xb = x + b * 256;
        int is = 0, xo = 0;
        for (int g = 0; g < 4; g++) {
            uint8_t sc0, m0, sc1, m1;
            or_get_scale_min_k4(is, scales, &sc0, &m0);
            or_get_scale_min_k4(is + 1, scales, &sc1, &m1);
            float d1 = d * (float)sc0;
            float m1v = mn * (float)m0;
            float d2 = d * (float)sc1;
            float m2v = mn * (float)m1;
            sum += q4k_sub32(d1, m1v, q, xb + xo, 0);
            xo += 32;
            sum += q4k_sub32(d2, m2v, q, xb + xo, 1);
            xo += 32;
            q += 32;
            is += 2;
        }
    }
    return sum;
}

/* gemv_q8_0 row: sum += (i8 q) * d * x, element by element in column order;
 * crates/hayai-model/src/quant.rs:598-613. */
static float row_q8_0(const uint8_t* row, size_t nb, const float* x) {
    float sum = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * 34;
        float d = f16le(blk);
        const float* xb = x + b * 32;
        for (int j = 0; j < 32; j++) sum += (float)(int8_t)blk[2 + j] * d * xb[j];
    }
    return sum;
}

/* gemv_q6_k row: dequant every block of the row, then sum += v[c] * x[c] in column order;
 * crates/hayai-model/src/q6k.rs:59-88. */
static float row_q6_k(const uint8_t* row, size_t nb, const float* x) {
    float sum = 0.0f;
    float tmp[256];
    for (size_t b = 0; b < nb; b++) {
        dequant_q6_k_block(row + b * 210, tmp);
        const float* xb = x + b * 256;
        for (int j = 0; j < 256; j++) sum += tmp[j] * xb[j];
    }
    return sum;
}

/* IQ GEMV row: dequant 256 into tmp, then scalar sum += tmp[j] * x[j];
 * crates/hayai-model/src/iq2.rs:591-626 (macro body) and iq3.rs:258-295. */
static float row_iq(const uint8_t* row, size_t nb, const float* x, int type) {
    float sum = 0.0f;
    float tmp[256];
    for (size_t b = 0; b < nb; b++) {
        if (type == OR_IQ2_XXS)
            dequant_iq2_xxs_block(row + b * 66, tmp);
        else
            dequant_iq3_xxs_block(row + b * 98, tmp);
        const float* xb = x + b * 256;
        for (int j = 0; j < 256; j++) sum += tmp[j] * xb[j];
    }
    return sum;
}

/* F32 / F16 GEMV: scalar `s += w * x` per row, the CPU reference of the reference's own
 * f32/f16 kernel tests; crates/hayai-opencl/src/compute.rs:1508-1545. */
static float row_f32(const uint8_t* row, size_t n, const float* x) {
    float s = 0.0f;
    for (size_t c = 0; c < n; c++) {
        float w;
        memcpy(&w, row + 4 * c, 4);
        s += w * x[c];
    }
    return s;
}

static float row_f16(const uint8_t* row, size_t n, const float* x) {
    float s = 0.0f;
    for (size_t c = 0; c < n; c++) s += f16le(row + 2 * c) * x[c];
    return s;
}

/* y[m] = W[m x n] . x[n] with W row-major in GGUF blocks along n; quant.rs:28-29.
 * Validation as compute.rs:912-949. */
int or_gemv(int type, size_t m, size_t n, const uint8_t* w, size_t wlen, const float* x, float* y) {
    if (or_validate_shape(type, m, n) != OR_OK) return OR_EINVAL;
    if (or_validate_weights(type, m, n, wlen) != OR_OK) return OR_EINVAL;
    size_t rb = row_bytes_or0(type, n);
    size_t block = 1, bb = 0;
    block_geom(type, &block, &bb);
    size_t nb = n / block;
    long long mm = (long long)m;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < mm; r++) {
        const uint8_t* row = w + (size_t)r * rb;
        float v;
        switch (type) {
        case OR_Q4_0: v = row_q4_0(row, nb, x); break;
        case OR_Q8_0: v = row_q8_0(row, nb, x); break;
        case OR_Q4_K: v = row_q4_k(row, nb, x); break;
        case OR_Q6_K: v = row_q6_k(row, nb, x); break;
        case OR_IQ2_XXS:
        case OR_IQ3_XXS: v = row_iq(row, nb, x, type); break;
        case OR_F32: v = row_f32(row, n, x); break;
        default: v = row_f16(row, n, x); break;
        }
        y[r] = v;
    }
    return OR_OK;
}

/* fp64 brute force: dequantize (bit-exact path above) and accumulate in double.  Used by
 * the tests to bound the fp32 GEMV, not a restatement of a reference function. */
int or_gemv_f64(int type, size_t m, size_t n, const uint8_t* w, size_t wlen, const double* x, double* y) {
    if (or_validate_shape(type, m, n) != OR_OK) return OR_EINVAL;
    if (or_validate_weights(type, m, n, wlen) != OR_OK) return OR_EINVAL;
    size_t rb = row_bytes_or0(type, n);
    float* row = (float*)malloc(n * sizeof(float));
    if (!row) return OR_EINVAL;
    for (size_t r = 0; r < m; r++) {
        or_dequant(type, w + r * rb, rb, n, row);
        double s = 0.0;
        for (size_t c = 0; c < n; c++) s += (double)row[c] * x[c];
        y[r] = s;
    }
    free(row);
    return OR_OK;
}

/* B independent GEMVs sharing W: X[B x n] -> Y[B x m].  The reference's batched entry
 * point is checked against per-batch gemv_q4_k (compute.rs:1648-1670) and its non-Q4_K
 * dispatcher runs B sequential GEMVs (orchestrator.rs:258-261). */
int or_gemv_batched(int type, size_t m, size_t n, const uint8_t* w, size_t wlen, size_t batch,
                    const float* X, float* Y) {
    for (size_t b = 0; b < batch; b++) {
        int rc = or_gemv(type, m, n, w, wlen, X + b * n, Y + b * m);
        if (rc != OR_OK) return rc;
    }
    return OR_OK;
}

/* cpu_lut_matmul_q4: nibble pairs index a 16-entry f32 LUT;
 * crates/hayai-cpu/src/matmul.rs:48-82.  sum += x0*w0 + x1*w1. */
int or_lut_matmul_q4(size_t m, size_t n, const uint8_t* wq, const float* lut, const float* x, float* y) {
    if (n % 2 != 0) return OR_EINVAL;
    size_t pc = n / 2;
    long long mm = (long long)m;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < mm; r++) {
        const uint8_t* row = wq + (size_t)r * pc;
        float sum = 0.0f;
        for (size_t c = 0; c < pc; c++) {
            uint8_t p = row[c];
            float w0 = lut[p & 0x0F];
            float w1 = lut[(p >> 4) & 0x0F];
            float x0 = x[2 * c];
            float x1 = x[2 * c + 1];
            sum += x0 * w0 + x1 * w1;
        }
        y[r] = sum;
    }
    return OR_OK;
}

/* ------------------------------------------------------------- SwiGLU / FFN ---------- */

/* SiLU(g) * u; crates/hayai-core/src/stream_infer.rs:3836-3840 (f32::exp = libm expf). */
void or_swiglu(const float* g, const float* u, float* h, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float gi = g[i];
        h[i] = (gi / (1.0f + expf(-gi))) * u[i];
    }
}

/* tanh-approximate GELU(g) * u; crates/hayai-core/src/stream_infer.rs:3889-3895. */
void or_gelu_tanh(const float* g, const float* u, float* h, size_t n) {
    const float k = sqrtf(2.0f / 3.14159265358979323846f);
    for (size_t i = 0; i < n; i++) {
        float x = g[i];
        float x3 = x * x * x;
        float inner = k * (x + 0.044715f * x3);
        h[i] = 0.5f * x * (1.0f + tanhf(inner)) * u[i];
    }
}

/* RMSNorm; rms_norm, crates/hayai-cpu/src/attention.rs:142-147: the mean square as
 * simd_mean_square (crates/hayai-cpu/src/simd_ops.rs:10-24: f32x8 lane sums of v*v, ordered
 * reduce_sum, scalar tail, / n), inv = 1 / sqrt(ms + eps), then simd_scale_mul (:28-41):
 * (x * inv) * w over whole f32x8s, x * (inv * w) on the tail. */
void or_rms_norm(const float* x, const float* w, float eps, float* y, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = acc[l] + x[i + l] * x[i + l];
    float ms = reduce_sum8(acc);
    for (; i < n; i++) ms = ms + x[i] * x[i];
    ms = ms / (float)n;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (i = 0; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) y[i + l] = (x[i + l] * inv) * w[i + l];
    for (; i < n; i++) y[i] = x[i] * (inv * w[i]);
}

/* The FFN op: gate & up GEMV -> act(gate)*up -> down GEMV;
 * ffn_begin_gate_up_scratch + ffn_finish_scratch, stream_infer.rs:3752-3864.
 * act 0 = SiLU, 1 = GELU(tanh).  h (d_ff floats) is optional scratch output. */
int or_ffn(int tg, int tu, int td, size_t d_model, size_t d_ff, const uint8_t* wg, size_t lg,
           const uint8_t* wu, size_t lu, const uint8_t* wd, size_t ld, int act, const float* x, float* y,
           float* h_out) {
    float* g = (float*)malloc(d_ff * sizeof(float));
    float* u = (float*)malloc(d_ff * sizeof(float));
    float* h = h_out ? h_out : (float*)malloc(d_ff * sizeof(float));
    int rc = OR_EINVAL;
    if (!g || !u || !h) goto out;
    if ((rc = or_gemv(tg, d_ff, d_model, wg, lg, x, g)) != OR_OK) goto out;
    if ((rc = or_gemv(tu, d_ff, d_model, wu, lu, x, u)) != OR_OK) goto out;
    if (g_mutation == 1) {
        float* t = g;
        g = u;
        u = t;
    }
    if (act == 0)
        or_swiglu(g, u, h, d_ff);
    else
        or_gelu_tanh(g, u, h, d_ff);
    rc = or_gemv(td, d_model, d_ff, wd, ld, h, y);
out:
    free(g);
    free(u);
    if (!h_out) free(h);
    return rc;
}

/* The FFN residual block of one token; ffn_apply, crates/hayai-core/src/hybrid_infer.rs:
 * 883-936: xn = rms_norm(x), y = x + FFN(xn) (x[i] += ws_down[i]). */
int or_ffn_block(int tg, int tu, int td, size_t d_model, size_t d_ff, const uint8_t* wg, size_t lg,
                 const uint8_t* wu, size_t lu, const uint8_t* wd, size_t ld, int act, const float* norm, float eps,
                 const float* x, float* y) {
    float* xn = (float*)malloc(d_model * sizeof(float));
    float* f = (float*)malloc(d_model * sizeof(float));
    if (!xn || !f) {
        free(xn);
        free(f);
        return OR_EINVAL;
    }
    or_rms_norm(x, norm, eps, xn, d_model);
    int st = or_ffn(tg, tu, td, d_model, d_ff, wg, lg, wu, lu, wd, ld, act, xn, f, NULL);
    if (st == OR_OK)
        for (size_t i = 0; i < d_model; i++) y[i] = x[i] + f[i];
    free(xn);
    free(f);
    return st;
}

/* ------------------------------------------------------------- MoE routing ---------- */

/* Stable descending sort of idx[] by key (partial_cmp, NaN compares Equal);
 * Rust `sort_by` is stable, so ties keep the earlier index first. */
static void stable_sort_desc(int* idx, int n, const float* key) {
    for (int i = 1; i < n; i++) {
        int v = idx[i];
        int j = i - 1;
        while (j >= 0 && key[v] > key[idx[j]]) {
            idx[j + 1] = idx[j];
            j--;
        }
        idx[j + 1] = v;
    }
}

/* route_experts (+ top_k_indices); crates/hayai-core/src/moe_infer.rs:852-934.
 * gating 0 = softmax over ALL experts then take the selected values, 1 = sigmoid.
 * Writes k = min(max(top_k,1), n) ids and weights; returns k (0 for n == 0). */
int or_route_experts(const float* scores, int n, const float* bias, int top_k, int n_group, int topk_group,
                     int gating, int norm_topk_prob, float routed_scaling_factor, int* ids_out, float* w_out) {
    if (n <= 0) return 0;
    float* choice = (float*)malloc(sizeof(float) * (size_t)n);
    int* top = (int*)malloc(sizeof(int) * (size_t)n);
    int ntop = 0;
    for (int i = 0; i < n; i++) choice[i] = bias ? scores[i] + bias[i] : scores[i];
    int grouped = n_group > 0 && topk_group > 0 && n % n_group == 0;
    if (grouped) {
        int gs = n / n_group;
        float* gscore = (float*)malloc(sizeof(float) * (size_t)n_group);
        int* gidx = (int*)malloc(sizeof(int) * (size_t)n_group);
        int* tmp = (int*)malloc(sizeof(int) * (size_t)gs);
        for (int g = 0; g < n_group; g++) {
            for (int j = 0; j < gs; j++) tmp[j] = g * gs + j;
            stable_sort_desc(tmp, gs, choice);
            float s = 0.0f;
            for (int j = 0; j < gs && j < 2; j++) s += choice[tmp[j]];
            gscore[g] = s;
            gidx[g] = g;
        }
        stable_sort_desc(gidx, n_group, gscore);
        int keep = topk_group < n_group ? topk_group : n_group;
        for (int t = 0; t < keep; t++)
            for (int j = 0; j < gs; j++) top[ntop++] = gidx[t] * gs + j;
        int k = top_k < 1 ? 1 : top_k;
        int lim = ntop < 1 ? 1 : ntop;
        if (k > lim) k = lim;
        stable_sort_desc(top, ntop, choice);
        if (ntop > k) ntop = k;
        free(gscore);
        free(gidx);
        free(tmp);
    } else {
        int k = top_k < n ? top_k : n;
        if (k < 1) k = 1;
        for (int i = 0; i < n; i++) top[i] = i;
        stable_sort_desc(top, n, choice);
        ntop = k;
    }
    if (gating == 1) {
        for (int t = 0; t < ntop; t++) w_out[t] = 1.0f / (1.0f + expf(-scores[top[t]]));
    } else {
        float mx = -INFINITY;
        for (int i = 0; i < n; i++) mx = fmaxf(mx, scores[i]);
        float* ex = (float*)malloc(sizeof(float) * (size_t)n);
        float sum = 0.0f;
        for (int i = 0; i < n; i++) ex[i] = expf(scores[i] - mx);
        for (int i = 0; i < n; i++) sum += ex[i];
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int t = 0; t < ntop; t++) w_out[t] = ex[top[t]] * inv;
        free(ex);
    }
    if (norm_topk_prob) {
        float s = 0.0f;
        for (int t = 0; t < ntop; t++) s += w_out[t];
        if (s > 0.0f)
            for (int t = 0; t < ntop; t++) w_out[t] /= s;
    }
    if (fabs((double)routed_scaling_factor - 1.0) > 1e-9)
        for (int t = 0; t < ntop; t++) w_out[t] *= routed_scaling_factor;
    for (int t = 0; t < ntop; t++) ids_out[t] = top[t];
    free(choice);
    free(top);
    return ntop;
}

/* One token through a routed MoE FFN; crates/hayai-core/src/moe_infer.rs:342-380
 * (per expert: gate, up, SiLU*up, down; then acc[j] += w_e * down_e[j] in top order).
 * Experts live in one buffer: expert e's gate/up/down at e*expert_stride + {g,u,d}_off.
 * acc (d_model floats) is accumulated into, as the reference accumulates into its
 * zero-initialised `acc`. */
int or_moe_token(int type, size_t d_model, size_t d_ff, const uint8_t* w, size_t expert_stride, size_t g_off,
                 size_t u_off, size_t d_off, int k, const int* ids, const float* wts, const float* x, float* acc) {
    size_t rg = row_bytes_or0(type, d_model), rd = row_bytes_or0(type, d_ff);
    float* g = (float*)malloc(d_ff * sizeof(float));
    float* u = (float*)malloc(d_ff * sizeof(float));
    float* d = (float*)malloc(d_model * sizeof(float));
    int rc = OR_OK;
    for (int t = 0; t < k && rc == OR_OK; t++) {
        size_t e = (size_t)ids[t];
        if (g_mutation == 2) e = e + 1; /* the pinning test keeps every id below the last expert */
        const uint8_t* base = w + e * expert_stride;
        rc = or_gemv(type, d_ff, d_model, base + g_off, d_ff * rg, x, g);
        if (rc == OR_OK) rc = or_gemv(type, d_ff, d_model, base + u_off, d_ff * rg, x, u);
        if (rc == OR_OK) {
            for (size_t j = 0; j < d_ff; j++) g[j] = (g[j] / (1.0f + expf(-g[j]))) * u[j];
            rc = or_gemv(type, d_model, d_ff, base + d_off, d_model * rd, g, d);
        }
        if (rc == OR_OK)
            for (size_t j = 0; j < d_model; j++) acc[j] += wts[t] * d[j];
    }
    free(g);
    free(u);
    free(d);
    return rc;
}

/* The shared expert of an MoE layer; crates/hayai-core/src/moe_infer.rs:456-493: always
 * active with weight 1, after the routed experts: g = gate_s . x, u = up_s . x,
 * g[j] = (g[j] / (1 + exp(-g[j]))) * u[j], d = down_s . g, acc[j] += d[j]. */
int or_moe_shared(int type, size_t d_model, size_t d_ff, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                  const float* x, float* acc) {
    size_t rg = row_bytes_or0(type, d_model), rd = row_bytes_or0(type, d_ff);
    float* g = (float*)malloc(d_ff * sizeof(float));
    float* u = (float*)malloc(d_ff * sizeof(float));
    float* d = (float*)malloc(d_model * sizeof(float));
    int rc = (g && u && d) ? OR_OK : OR_EINVAL;
    if (g_mutation == 3) { /* planted: the shared expert reads its up tensor as gate */
        const uint8_t* t = wg;
        wg = wu;
        wu = t;
    }
    if (rc == OR_OK) rc = or_gemv(type, d_ff, d_model, wg, d_ff * rg, x, g);
    if (rc == OR_OK) rc = or_gemv(type, d_ff, d_model, wu, d_ff * rg, x, u);
    if (rc == OR_OK) {
        for (size_t j = 0; j < d_ff; j++) g[j] = (g[j] / (1.0f + expf(-g[j]))) * u[j];
        rc = or_gemv(type, d_model, d_ff, wd, d_model * rd, g, d);
    }
    if (rc == OR_OK)
        for (size_t j = 0; j < d_model; j++) acc[j] += d[j];
    free(g);
    free(u);
    free(d);
    return rc;
}

/* ------------------------------------------------------------ quantizers ---------- */

/* quantize_q4_k_block; crates/hayai-model/src/q4k.rs:100-160 (the reference's own
 * quantizer; used to pin dequant through its round-trip test q4k.rs:319-350). */
static void quantize_q4_k_block(const float* x, uint8_t* out) {
    float scales[8], mins[8];
    uint8_t L[256];
    for (int j = 0; j < 8; j++) {
        float mn = INFINITY, mx = -INFINITY;
        for (int i = 0; i < 32; i++) {
            mn = fminf(mn, x[j * 32 + i]);
            mx = fmaxf(mx, x[j * 32 + i]);
        }
        scales[j] = (mx - mn) / 15.0f;
        mins[j] = mn;
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) max_scale = fmaxf(max_scale, scales[j]);
    for (int j = 0; j < 8; j++) max_min = fmaxf(max_min, fabsf(mins[j]));
    max_scale = fmaxf(max_scale, 1e-30f);
    max_min = fmaxf(max_min, 1e-30f);
    float d = max_scale / 63.0f;
    float dmin = max_min / 63.0f;
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        float a = roundf(scales[j] * 63.0f / max_scale);
        float b = roundf(-mins[j] * 63.0f / max_min);
        ls[j] = (uint8_t)fminf(fmaxf(a, 0.0f), 63.0f);
        lm[j] = (uint8_t)fminf(fmaxf(b, 0.0f), 63.0f);
    }
    for (int j = 0; j < 8; j++) {
        float d1 = d * (float)ls[j];
        if (d1 == 0.0f) {
            for (int i = 0; i < 32; i++) L[j * 32 + i] = 0;
            continue;
        }
        float dm = dmin * (float)lm[j];
        for (int i = 0; i < 32; i++) {
            float q = roundf((x[j * 32 + i] + dm) / d1);
            L[j * 32 + i] = (uint8_t)fminf(fmaxf(q, 0.0f), 15.0f);
        }
    }
    uint16_t hd = or_f32_to_f16_ref(d), hm = or_f32_to_f16_ref(dmin);
    out[0] = (uint8_t)(hd & 0xFF);
    out[1] = (uint8_t)(hd >> 8);
    out[2] = (uint8_t)(hm & 0xFF);
    out[3] = (uint8_t)(hm >> 8);
    uint8_t sp[12] = {0};
    for (int j = 0; j < 8; j++) {
        uint8_t sc = ls[j], m = lm[j];
        if (j < 4) {
            sp[j] = sc;
            sp[j + 4] = m;
        } else {
            sp[j + 4] = (uint8_t)((sc & 0xF) | ((m & 0xF) << 4));
            sp[j - 4] |= (uint8_t)((sc >> 4) << 6);
            sp[j] |= (uint8_t)((m >> 4) << 6);
        }
    }
    memcpy(out + 4, sp, 12);
    for (int j = 0; j < 256; j += 64) {
        int base = j / 64 * 32;
        for (int i = 0; i < 32; i++) out[16 + base + i] = (uint8_t)(L[j + i] | (L[j + i + 32] << 4));
    }
}

int or_quantize_q4_k(const float* x, size_t n, uint8_t* out) {
    if (n % 256 != 0) return OR_EINVAL;
    for (size_t b = 0; b < n / 256; b++) quantize_q4_k_block(x + b * 256, out + b * 144);
    return OR_OK;
}

/* int8 activation quantization per 32-element block (the batched path's input).  The
 * reference has no int8 activation path; this is the project's stated choice: s = amax /
 * 127, q = round_half_away(x / s) clamped to +-127, s = 0 -> q = 0.  Not a restatement;
 * pinned by closed-form tests only. */
int or_quantize_act_q8(const float* x, size_t n, int8_t* q, float* s) {
    if (n % 32 != 0) return OR_EINVAL;
    for (size_t b = 0; b < n / 32; b++) {
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[b * 32 + i]));
        float sc = amax / 127.0f;
        s[b] = sc;
        for (int i = 0; i < 32; i++) {
            float v = sc > 0.0f ? roundf(x[b * 32 + i] / sc) : 0.0f;
            v = fminf(fmaxf(v, -127.0f), 127.0f);
            q[b * 32 + i] = (int8_t)v;
        }
    }
    return OR_OK;
}

/* x -> q * s, the activation the batched int8 path computes with (q, s of
 * or_quantize_act_q8; one f32 product per element). */
static int dequant_act_q8(const float* x, size_t n, float* out) {
    int8_t* q = (int8_t*)malloc(n);
    float* s = (float*)malloc(sizeof(float) * (n / 32 + 1));
    int rc = OR_EINVAL;
    if (q && s && or_quantize_act_q8(x, n, q, s) == OR_OK) {
        for (size_t i = 0; i < n; i++) out[i] = (float)q[i] * s[i / 32];
        rc = OR_OK;
    }
    free(q);
    free(s);
    return rc;
}

/* The FFN of the batched int8 path (activations quantized to int8
 * per 32-element block): both GEMV inputs are the dequantized int8 activations, x -> q * s
 * before gate and up, h -> q * s before down; otherwise or_ffn. */
int or_ffn_q8(int tg, int tu, int td, size_t d_model, size_t d_ff, const uint8_t* wg, size_t lg,
              const uint8_t* wu, size_t lu, const uint8_t* wd, size_t ld, int act, const float* x, float* y) {
    float* xq = (float*)malloc(d_model * sizeof(float));
    float* h = (float*)malloc(d_ff * sizeof(float));
    float* hq = (float*)malloc(d_ff * sizeof(float));
    float* tmp = (float*)malloc(d_model * sizeof(float));
    int rc = OR_EINVAL;
    if (xq && h && hq && tmp && dequant_act_q8(x, d_model, xq) == OR_OK &&
        or_ffn(tg, tu, td, d_model, d_ff, wg, lg, wu, lu, wd, ld, act, xq, tmp, h) == OR_OK &&
        dequant_act_q8(h, d_ff, hq) == OR_OK)
        rc = or_gemv(td, d_model, d_ff, wd, ld, hq, y);
    free(xq);
    free(h);
    free(hq);
    free(tmp);
    return rc;
}

/* Table accessors for the tests. */
void or_iq2xxs_grid(uint64_t* out) { memcpy(out, OR_IQ2XXS_GRID, sizeof(OR_IQ2XXS_GRID)); }
void or_iq3xxs_grid(uint32_t* out) { memcpy(out, OR_IQ3XXS_GRID, sizeof(OR_IQ3XXS_GRID)); }
void or_ksigns(uint8_t* out) {
    for (uint32_t i = 0; i < 128; i++) out[i] = ksign(i);
}
