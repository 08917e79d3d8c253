// IQ2_XXS and IQ3_XXS in the ring FFN / ring GEMV kernels (q4k_ring.hip's generic bodies):
//   gate/up  hh_iq{2,3}_gu_ring_g<W1>[_n]: h = act(W_gate . x) * (W_up . x) as h digits
//   down     hh_iq{2,3}_dn_ring_d<W2>:     y = W_down . h (also the ring GEMV: x -> digits
//                                          by hh_x_digits, then this kernel)
// (dequant_iq2_xxs_block, crates/hayai-model/src/iq2.rs:504-523; dequant_iq3_xxs_block,
// iq3.rs:147-173; ggml_gemv_iq2_xxs / ggml_gemv_iq3_xxs, crates/hayai-kernels/kernels/
// ggml_gemv_q4.cl:916-961,1499-1536.)  Compiled after q6k_ring.hip in the same translation
// unit.
//
// Integer form.  A group of 32 columns (one ib32 of the reference) has one scale
// db = d * (0.5 + aux>>28) * k (k = 1/4 for IQ2_XXS, 1/2 for IQ3_XXS) and eight-element
// codebook entries with one sign byte each.  Codebook magnitudes are small positive bytes
// (8..62), so a signed entry is built per 4 bytes with no carries between bytes:
//   v = (g ^ m) + (m & 0x01010101),   m = 0xFF in every byte whose sign bit is set
// and dotted with the activation's two int8 digits (v_dot4), the int32 sums of a group
// meeting its scale once (per-32 x digits) or per granule of 8 (h digits, prefix-summed as
// in hh_ffnp_h).  Codebook and sign masks sit in LDS (the lanes' indices diverge).
//
// Unit (lane) = 64 columns = two groups = 16 qs bytes (IQ3_XXS: + 8 scale/sign bytes) of a
// 66- or 98-byte block.  Rows start 4-byte aligned (the host requires an even number of
// blocks per row), so a lane's pieces are 4-byte aligned or 2 bytes off: the lane loads the
// dwords covering them and realigns with one byte permute per dword.  An aligned piece is
// loaded from 4 bytes before it (inside its block), a misaligned one from 2 bytes before
// it, so no load runs past its block except in even blocks, which are never a row's last.

// Sign entry of ksigns(i) = i | parity(i) << 7: byte masks m (0xFF where the sign bit is set)
// and m & 0x01010101, for elements 0-3 and 4-7.
struct hh_iq_sign {
    uint32_t mlo, mhi, olo, ohi;
};
struct hh_iq2_tab {
    uint64_t grid[256];  // IQ2_XXS codebook
    hh_iq_sign sgn[128];
};
struct hh_iq3_tab {
    uint32_t grid[256];  // IQ3_XXS codebook
    hh_iq_sign sgn[128];
};

constexpr hh_iq_sign hh_sign_entry(uint32_t i) {
    uint32_t par = 0;
    for (uint32_t b = 0; b < 7; b++) par ^= (i >> b) & 1u;
    const uint32_t s = i | (par << 7);
    uint32_t m[2] = {0u, 0u};
    for (uint32_t j = 0; j < 8; j++)
        if ((s >> j) & 1u) m[j / 4] |= 0xFFu << (8 * (j % 4));
    return hh_iq_sign{m[0], m[1], m[0] & 0x01010101u, m[1] & 0x01010101u};
}
constexpr hh_iq2_tab hh_make_iq2_tab() {
    hh_iq2_tab t{{HH_IQ2XXS_GRID_VALUES}, {}};
    for (uint32_t i = 0; i < 128; i++) t.sgn[i] = hh_sign_entry(i);
    return t;
}
constexpr hh_iq3_tab hh_make_iq3_tab() {
    hh_iq3_tab t{{HH_IQ3XXS_GRID_VALUES}, {}};
    for (uint32_t i = 0; i < 128; i++) t.sgn[i] = hh_sign_entry(i);
    return t;
}

__device__ __attribute__((aligned(16))) const hh_iq2_tab hh_iq2_ring_tab = hh_make_iq2_tab();
__device__ __attribute__((aligned(16))) const hh_iq3_tab hh_iq3_ring_tab = hh_make_iq3_tab();
static_assert(sizeof(hh_iq2_tab) % 16 == 0 && sizeof(hh_iq3_tab) % 16 == 0, "tables copy in 16-byte chunks");

// (a ^ b) + c in one VALU op (the compiler does not form v_xad_u32 from the xor and add).
// The int8 dot products stay with the compiler's builtin: a DOT result read by another VALU
// op needs wait states that only the compiler's hazard tracking inserts.
HH_DEV uint32_t hh_xad(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_xad_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// A lane's x: per-32 digits of its 64 columns, the two group scales / 256.
struct hh_iq_x {
    uint32_t q1[16], q2[16];
    float s[2];
};
// A lane's h: per-8 digits of its 64 columns, prefix-sum weights (s_k - s_{k+1}) / 256 of
// the four granules of each group (s_4 = 0).
struct hh_iq_h {
    uint32_t q1[16], q2[16];
    float w[8];
};

HH_DEV void hh_iq_load_digits(const int8_t* q1, const int8_t* q2, uint32_t u, uint32_t (&d1)[16], uint32_t (&d2)[16]) {
    const uint4* a = reinterpret_cast<const uint4*>(q1 + (size_t)u * 64);
    const uint4* b = reinterpret_cast<const uint4*>(q2 + (size_t)u * 64);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        hh_unpack4(a[i], d1 + 4 * i);
        hh_unpack4(b[i], d2 + 4 * i);
    }
}
HH_DEV void hh_iq_load_x(const hh_digits_ptr& xd, uint32_t u, hh_iq_x& x) {
    hh_iq_load_digits(xd.q1, xd.q2, u, x.q1, x.q2);
    const float2 sc = reinterpret_cast<const float2*>(xd.sc)[u];
    x.s[0] = sc.x * (1.0f / 256.0f);
    x.s[1] = sc.y * (1.0f / 256.0f);
}
HH_DEV void hh_iq_load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_iq_h& h) {
    hh_iq_load_digits(q1, q2, u, h.q1, h.q2);
    const float4 s0 = reinterpret_cast<const float4*>(sc)[2 * u];
    const float4 s1 = reinterpret_cast<const float4*>(sc)[2 * u + 1];
    const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int k = 0; k < 8; k++) h.w[k] = (s[k] - ((k & 3) < 3 ? s[k + 1] : 0.f)) * (1.0f / 256.0f);
}

// One signed 8-element codebook entry against the digits of elements 8l..8l+7 of group g,
// accumulated into the group's int32 digit sums.
template <class X>
HH_DEV void hh_iq_entry(uint32_t glo, uint32_t ghi, const hh_iq_sign& m, const X& x, int g, int l, int& c1, int& c2) {
    const int vlo = (int)hh_xad(glo, m.mlo, m.olo);
    const int vhi = (int)hh_xad(ghi, m.mhi, m.ohi);
    const int i = 8 * g + 2 * l;
    // |c1| <= 32 * 62 * 127 per group, so 256 * c1 + c2 fits an int32 exactly
    c1 = __builtin_amdgcn_sdot4(vlo, (int)x.q1[i], l == 0 ? 0 : c1, false);
    c2 = __builtin_amdgcn_sdot4(vlo, (int)x.q2[i], l == 0 ? 0 : c2, false);
    c1 = __builtin_amdgcn_sdot4(vhi, (int)x.q1[i + 1], c1, false);
    c2 = __builtin_amdgcn_sdot4(vhi, (int)x.q2[i + 1], c2, false);
}

// Group g's digit sums -> f32, with the per-32 x scale or the per-8 h weights.
template <class X>
HH_DEV float hh_iq_group_t(const X& x, int g, const int (&c1)[4], const int (&c2)[4]);
template <>
HH_DEV float hh_iq_group_t<hh_iq_x>(const hh_iq_x& x, int g, const int (&c1)[4], const int (&c2)[4]) {
    return x.s[g] * (float)(c1[3] * 256 + c2[3]);
}
template <>
HH_DEV float hh_iq_group_t<hh_iq_h>(const hh_iq_h& h, int g, const int (&c1)[4], const int (&c2)[4]) {
    float t = 0.f;
#pragma unroll
    for (int l = 0; l < 4; l++) t = fmaf(h.w[4 * g + l], (float)(c1[l] * 256 + c2[l]), t);
    return t;
}

// Fixed byte offsets of a lane's pieces: `p` is the piece's offset in the row; returns the
// dword-aligned load offset and the permute selector realigning the loaded run.
HH_DEV void hh_iq_piece(uint32_t p, uint32_t& off, uint32_t& sel) {
    const bool odd = (p & 2u) != 0u;
    off = odd ? p - 2u : p - 4u;
    sel = odd ? 0x05040302u : 0x07060504u;
}

typedef uint32_t hh_v2u_a4i __attribute__((ext_vector_type(2), aligned(4)));

struct hh_ring_iq2 {
    static constexpr uint32_t UNIT = 64;
    static constexpr uint32_t BB = 66;  // block bytes: d (f16) + 8 groups x (4 codebook indices, 4 sign/scale bytes)
    static constexpr uint32_t TAB_BYTES = sizeof(hh_iq2_tab);
    struct lane_t {
        uint32_t qo, dof, sel, dsh;
    };
    struct data {
        uint32_t a[5];  // 20 bytes covering the lane's 16 qs bytes
        uint32_t d;     // the dword holding the block's d
    };
    typedef hh_iq_x xr_t;
    typedef hh_iq_h hr_t;
    static HH_DEV lane_t lane(uint32_t u) {
        const uint32_t bo = (u >> 2) * BB;
        lane_t l;
        hh_iq_piece(bo + 2u + 16u * (u & 3u), l.qo, l.sel);
        l.dof = bo & ~3u;
        l.dsh = (bo & 2u) * 8u;
        return l;
    }
    static HH_DEV void issue(const uint8_t* row, const lane_t& l, data& s) {
        const hh_v4u_a4 v = *reinterpret_cast<const hh_v4u_a4*>(row + l.qo);
        s.a[0] = v.x;
        s.a[1] = v.y;
        s.a[2] = v.z;
        s.a[3] = v.w;
        s.a[4] = *reinterpret_cast<const uint32_t*>(row + l.qo + 16);
        s.d = *reinterpret_cast<const uint32_t*>(row + l.dof);
    }
    static HH_DEV const uint4* tables() { return reinterpret_cast<const uint4*>(&hh_iq2_ring_tab); }
    static HH_DEV void load_x(const hh_digits_ptr& xd, uint32_t u, xr_t& x) { hh_iq_load_x(xd, u, x); }
    static HH_DEV void load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hr_t& h) {
        hh_iq_load_h(q1, q2, sc, u, h);
    }
    // d/8 * sum_g (2 s_g + 1) t_g  ==  sum_g d (0.5 + s_g) / 4 * t_g   (iq2.rs:513)
    template <class X>
    static HH_DEV float unit(const data& s, const lane_t& l, const X& x, const char* tab) {
        const hh_iq2_tab* t = reinterpret_cast<const hh_iq2_tab*>(tab);
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_perm(s.a[i + 1], s.a[i], l.sel);
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const uint32_t a0 = q[2 * g], a1 = q[2 * g + 1];
            int c1[4], c2[4];
            int r1 = 0, r2 = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint64_t gv = t->grid[(a0 >> (8 * k)) & 0xFFu];
                const hh_iq_sign m = t->sgn[(a1 >> (7 * k)) & 0x7Fu];
                hh_iq_entry((uint32_t)gv, (uint32_t)(gv >> 32), m, x, g, k, r1, r2);
                c1[k] = r1;
                c2[k] = r2;
            }
            acc = fmaf((float)(2u * (a1 >> 28) + 1u), hh_iq_group_t(x, g, c1, c2), acc);
        }
        return hh_f16((s.d >> l.dsh) & 0xFFFFu) * 0.125f * acc;
    }
    static HH_DEV float unit_x(const data& s, const lane_t& l, const xr_t& x, const char* tab) { return unit(s, l, x, tab); }
    static HH_DEV float unit_h(const data& s, const lane_t& l, const hr_t& h, const char* tab) { return unit(s, l, h, tab); }
};

struct hh_ring_iq3 {
    static constexpr uint32_t UNIT = 64;
    static constexpr uint32_t BB = 98;  // d (f16) + 64 codebook indices + 8 x (4 sign/scale bytes)
    static constexpr uint32_t TAB_BYTES = sizeof(hh_iq3_tab);
    struct lane_t {
        uint32_t qo, ao, dof, sel, dsh;
    };
    struct data {
        uint32_t a[5];  // 20 bytes covering the lane's 16 index bytes
        uint32_t b[3];  // 12 bytes covering its two sign/scale words
        uint32_t d;
    };
    typedef hh_iq_x xr_t;
    typedef hh_iq_h hr_t;
    static HH_DEV lane_t lane(uint32_t u) {
        const uint32_t bo = (u >> 2) * BB, j = u & 3u;
        lane_t l;
        uint32_t sel2;
        hh_iq_piece(bo + 2u + 16u * j, l.qo, l.sel);
        hh_iq_piece(bo + 66u + 8u * j, l.ao, sel2);  // same parity as the indices
        l.dof = bo & ~3u;
        l.dsh = (bo & 2u) * 8u;
        return l;
    }
    static HH_DEV void issue(const uint8_t* row, const lane_t& l, data& s) {
        const hh_v4u_a4 v = *reinterpret_cast<const hh_v4u_a4*>(row + l.qo);
        s.a[0] = v.x;
        s.a[1] = v.y;
        s.a[2] = v.z;
        s.a[3] = v.w;
        s.a[4] = *reinterpret_cast<const uint32_t*>(row + l.qo + 16);
        const hh_v2u_a4i w = *reinterpret_cast<const hh_v2u_a4i*>(row + l.ao);
        s.b[0] = w.x;
        s.b[1] = w.y;
        s.b[2] = *reinterpret_cast<const uint32_t*>(row + l.ao + 8);
        s.d = *reinterpret_cast<const uint32_t*>(row + l.dof);
    }
    static HH_DEV const uint4* tables() { return reinterpret_cast<const uint4*>(&hh_iq3_ring_tab); }
    static HH_DEV void load_x(const hh_digits_ptr& xd, uint32_t u, xr_t& x) { hh_iq_load_x(xd, u, x); }
    static HH_DEV void load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hr_t& h) {
        hh_iq_load_h(q1, q2, sc, u, h);
    }
    // d/4 * sum_g (2 s_g + 1) t_g  ==  sum_g d (0.5 + s_g) / 2 * t_g   (iq3.rs:160)
    template <class X>
    static HH_DEV float unit(const data& s, const lane_t& l, const X& x, const char* tab) {
        const hh_iq3_tab* t = reinterpret_cast<const hh_iq3_tab*>(tab);
        uint32_t q[4], aux[2];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_perm(s.a[i + 1], s.a[i], l.sel);
#pragma unroll
        for (int i = 0; i < 2; i++) aux[i] = __builtin_amdgcn_perm(s.b[i + 1], s.b[i], l.sel);
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const uint32_t ax = aux[g];
            int c1[4], c2[4];
            int r1 = 0, r2 = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                // entry k: codebook indices 2k, 2k+1 of the group (elements 8k..8k+3, 8k+4..8k+7)
                const uint32_t qq = q[2 * g + (k >> 1)] >> (16 * (k & 1));
                const uint32_t g1 = t->grid[qq & 0xFFu], g2 = t->grid[(qq >> 8) & 0xFFu];
                const hh_iq_sign m = t->sgn[(ax >> (7 * k)) & 0x7Fu];
                hh_iq_entry(g1, g2, m, x, g, k, r1, r2);
                c1[k] = r1;
                c2[k] = r2;
            }
            acc = fmaf((float)(2u * (ax >> 28) + 1u), hh_iq_group_t(x, g, c1, c2), acc);
        }
        return hh_f16((s.d >> l.dsh) & 0xFFFFu) * 0.25f * acc;
    }
    static HH_DEV float unit_x(const data& s, const lane_t& l, const xr_t& x, const char* tab) { return unit(s, l, x, tab); }
    static HH_DEV float unit_h(const data& s, const lane_t& l, const hr_t& h, const char* tab) { return unit(s, l, h, tab); }
};

// Gate/up: D rows in flight per wave (each item is 16.5 / 24.5 bytes per lane, so the ring
// is deeper than Q4_K's 48).  Down: the same.
#define HH_IQ_GU_DEPTH 6
#define HH_IQ_DN_DEPTH 6
#define HH_IQ_RING(Q, F)                                                                                      \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_##Q##_gu_ring_g1(const hh_gur_args a) {    \
        hh_gu_ring_body<F, 1, HH_IQ_GU_DEPTH, 2, false>(a);                                                  \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_##Q##_gu_ring_g1_n(const hh_gur_args a) {  \
        hh_gu_ring_body<F, 1, HH_IQ_GU_DEPTH, 2, true>(a);                                                   \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_##Q##_gu_ring_g2(const hh_gur_args a) {    \
        hh_gu_ring_body<F, 2, HH_IQ_GU_DEPTH, 2, false>(a);                                                  \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_##Q##_gu_ring_g2_n(const hh_gur_args a) {  \
        hh_gu_ring_body<F, 2, HH_IQ_GU_DEPTH, 2, true>(a);                                                   \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_##Q##_dn_ring_d1(const hh_dnr_args a) {      \
        hh_dn_ring_body<F, 1, HH_IQ_DN_DEPTH>(a);                                                            \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_##Q##_dn_ring_d2(const hh_dnr_args a) {      \
        hh_dn_ring_body<F, 2, HH_IQ_DN_DEPTH>(a);                                                            \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_##Q##_dn_ring_d4(const hh_dnr_args a) {      \
        hh_dn_ring_body<F, 4, HH_IQ_DN_DEPTH>(a);                                                            \
    }                                                                                                         \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_##Q##_dn_ring_d8(const hh_dnr_args a) {      \
        hh_dn_ring_body<F, 8, HH_IQ_DN_DEPTH>(a);                                                            \
    }
HH_IQ_RING(iq2, hh_ring_iq2)
HH_IQ_RING(iq3, hh_ring_iq3)
