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
// in hh_hd).  Codebook and sign masks sit in LDS (the lanes' indices diverge).
//
// Unit (lane) = 64 columns = two groups = 16 qs bytes (IQ3_XXS: + 8 scale/sign bytes) of a
// 66- or 98-byte block.  Rows start 4-byte aligned (the host requires an even number of
// blocks per row), so a lane's pieces are 4-byte aligned or 2 bytes off: the lane loads the
// dwords covering them and realigns with one byte permute per dword.  An aligned piece is
// loaded from 4 bytes before it (inside its block), a misaligned one from 2 bytes before
// it, so no load runs past its block except in even blocks, which are never a row's last.

// Sign entry of ksigns(i) = i | parity(i) << 7: byte masks m (0xFF where the sign bit is set)
// for elements 0-3 and 4-7; with HH_IQ_SIGN16 also m & 0x01010101 (16-byte entries: fewer
// VALU ops, more LDS traffic per codebook entry).
#ifndef HH_IQ_SIGN16
#define HH_IQ_SIGN16 0
#endif
struct hh_iq_sign {
    uint32_t mlo, mhi;
#if HH_IQ_SIGN16
    uint32_t olo, ohi;
#endif
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
#if HH_IQ_SIGN16
    return hh_iq_sign{m[0], m[1], m[0] & 0x01010101u, m[1] & 0x01010101u};
#else
    return hh_iq_sign{m[0], m[1]};
#endif
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

typedef uint32_t hh_v2u_a4i __attribute__((ext_vector_type(2), aligned(4)));

// A lane's x: per-32 digits of its NG groups (32 NG columns), the group scales / 256.
template <int NG>
struct hh_iq_x {
    uint32_t q1[8 * NG], q2[8 * NG];
    float s[NG];
};
// A lane's h: per-8 digits of its columns, prefix-sum weights (s_k - s_{k+1}) / 256 of the
// four granules of each group (s_4 = 0).
template <int NG>
struct hh_iq_h {
    uint32_t q1[8 * NG], q2[8 * NG];
    float w[4 * NG];
};

template <int NG>
HH_DEV void hh_iq_load_digits(const int8_t* q1, const int8_t* q2, uint32_t u, uint32_t (&d1)[8 * NG],
                              uint32_t (&d2)[8 * NG]) {
    const uint4* a = reinterpret_cast<const uint4*>(q1 + (size_t)u * 32 * NG);
    const uint4* b = reinterpret_cast<const uint4*>(q2 + (size_t)u * 32 * NG);
#pragma unroll
    for (int i = 0; i < 2 * NG; i++) {
        hh_unpack4(a[i], d1 + 4 * i);
        hh_unpack4(b[i], d2 + 4 * i);
    }
}
template <int NG>
HH_DEV void hh_iq_load_x(const hh_digits_ptr& xd, uint32_t u, hh_iq_x<NG>& x) {
    hh_iq_load_digits<NG>(xd.q1, xd.q2, u, x.q1, x.q2);
#pragma unroll
    for (int g = 0; g < NG; g++) x.s[g] = xd.sc[NG * u + g] * (1.0f / 256.0f);
}
// A lane's h bytes as loaded, apart from the arithmetic (as hh_hd_raw).
template <int NG>
struct hh_iq_hraw {
    uint4 a[2 * NG], b[2 * NG];
    float4 s[NG];
};
template <int NG>
HH_DEV void hh_iq_load_h_raw(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_iq_hraw<NG>& r) {
    const uint4* a = reinterpret_cast<const uint4*>(q1 + (size_t)u * 32 * NG);
    const uint4* b = reinterpret_cast<const uint4*>(q2 + (size_t)u * 32 * NG);
#pragma unroll
    for (int i = 0; i < 2 * NG; i++) {
        r.a[i] = a[i];
        r.b[i] = b[i];
    }
#pragma unroll
    for (int i = 0; i < NG; i++) r.s[i] = reinterpret_cast<const float4*>(sc)[NG * u + i];
}
template <int NG>
HH_DEV void hh_iq_make_h(const hh_iq_hraw<NG>& r, hh_iq_h<NG>& h) {
#pragma unroll
    for (int i = 0; i < 2 * NG; i++) {
        hh_unpack4(r.a[i], h.q1 + 4 * i);
        hh_unpack4(r.b[i], h.q2 + 4 * i);
    }
    float s[4 * NG];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        s[4 * i] = r.s[i].x;
        s[4 * i + 1] = r.s[i].y;
        s[4 * i + 2] = r.s[i].z;
        s[4 * i + 3] = r.s[i].w;
    }
#pragma unroll
    for (int k = 0; k < 4 * NG; k++) h.w[k] = (s[k] - ((k & 3) < 3 ? s[k + 1] : 0.f)) * (1.0f / 256.0f);
}
template <int NG>
HH_DEV void hh_iq_load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_iq_h<NG>& h) {
    hh_iq_hraw<NG> r;
    hh_iq_load_h_raw<NG>(q1, q2, sc, u, r);
    hh_iq_make_h<NG>(r, h);
}

// One signed 8-element codebook entry against the digits of elements 8l..8l+7 of group g,
// accumulated into the group's int32 digit sums.
template <class X>
HH_DEV void hh_iq_entry(uint32_t glo, uint32_t ghi, const hh_iq_sign& m, const X& x, int g, int l, int& c1, int& c2) {
#if HH_IQ_SIGN16
    const uint32_t olo = m.olo, ohi = m.ohi;
#else
    const uint32_t olo = m.mlo & 0x01010101u, ohi = m.mhi & 0x01010101u;
#endif
    const int vlo = (int)hh_xad(glo, m.mlo, olo);
    const int vhi = (int)hh_xad(ghi, m.mhi, ohi);
    const int i = 8 * g + 2 * l;
    // |c1| <= 32 * 62 * 127 per group, so 256 * c1 + c2 fits an int32 exactly
    c1 = __builtin_amdgcn_sdot4(vlo, (int)x.q1[i], l == 0 ? 0 : c1, false);
    c2 = __builtin_amdgcn_sdot4(vlo, (int)x.q2[i], l == 0 ? 0 : c2, false);
    c1 = __builtin_amdgcn_sdot4(vhi, (int)x.q1[i + 1], c1, false);
    c2 = __builtin_amdgcn_sdot4(vhi, (int)x.q2[i + 1], c2, false);
}

// Group g's digit sums -> f32, with the per-32 x scale or the per-8 h weights.
template <int NG>
HH_DEV float hh_iq_group_t(const hh_iq_x<NG>& x, int g, const int (&c1)[4], const int (&c2)[4]) {
    return x.s[g] * (float)(c1[3] * 256 + c2[3]);
}
template <int NG>
HH_DEV float hh_iq_group_t(const hh_iq_h<NG>& h, int g, const int (&c1)[4], const int (&c2)[4]) {
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

// Loads N dwords at p (4-byte aligned): dwordx4 pieces, then the tail.
template <int N>
HH_DEV void hh_iq_load_run(const uint8_t* p, uint32_t (&w)[N]) {
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        const hh_v4u_a4 v = *reinterpret_cast<const hh_v4u_a4*>(p + 4 * i);
        w[i] = v.x;
        w[i + 1] = v.y;
        w[i + 2] = v.z;
        w[i + 3] = v.w;
    }
    if constexpr (N % 4 == 1) w[N - 1] = *reinterpret_cast<const uint32_t*>(p + 4 * (N - 1));
    if constexpr (N % 4 == 3) {
        const hh_v2u_a4i v = *reinterpret_cast<const hh_v2u_a4i*>(p + 4 * (N - 3));
        w[N - 3] = v.x;
        w[N - 2] = v.y;
        w[N - 1] = *reinterpret_cast<const uint32_t*>(p + 4 * (N - 1));
    }
}

// The block's d for a lane whose unit is NG groups of a block.  NG = 2: from a dword load of
// its own.  NG = 4 (two lanes per block, the even lane first): the even lane's index run
// starts at the block or 2 bytes before it, so its first dword holds d; the odd lane takes
// that dword by DPP (quad_perm [0,0,2,2]).
template <int NG>
HH_DEV uint32_t hh_iq_block_d(uint32_t d_or_first, uint32_t dsh) {
    if constexpr (NG == 4) d_or_first = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)d_or_first, 0xA0, 0xF, 0xF, true);
    return (d_or_first >> dsh) & 0xFFFFu;
}

// Keeps a unit's table reads ahead of its arithmetic (the scheduler otherwise sinks each
// read to its use and waits on it).
#ifndef HH_IQ_PREFETCH
#define HH_IQ_PREFETCH 0
#endif
#if HH_IQ_PREFETCH
#define HH_IQ_FETCH_FENCE() __builtin_amdgcn_sched_barrier(0)
#else
#define HH_IQ_FETCH_FENCE() ((void)0)
#endif

// IQ2_XXS, NG groups (32 NG columns) per lane.
template <int NG>
struct hh_ring_iq2 {
    static constexpr uint32_t UNIT = 32 * NG;
    static constexpr uint32_t BB = 66;  // block bytes: d (f16) + 8 groups x (4 codebook indices, 4 sign/scale bytes)
    static constexpr uint32_t UPB = 8 / NG;  // units per block
    static constexpr uint32_t TAB_BYTES = sizeof(hh_iq2_tab);
    static constexpr bool DIRECT_H = true;  // down: h digits per lane, the tables by the copy wave
    static constexpr bool LANE_PARTIALS = true;
    static constexpr int RUN = 2 * NG + 1;  // dwords covering the lane's 8 NG index/sign bytes
    struct lane_t {
        uint32_t qo, dof, sel, dsh;
    };
    struct data {
        uint32_t a[RUN];
        uint32_t d;  // NG = 2: the dword holding the block's d
    };
    typedef hh_iq_x<NG> xr_t;
    typedef hh_iq_h<NG> hr_t;
    static HH_DEV lane_t lane(uint32_t u) {
        const uint32_t bo = (u / UPB) * BB;
        lane_t l;
        hh_iq_piece(bo + 2u + 8u * NG * (u % UPB), l.qo, l.sel);
        l.dof = bo & ~3u;
        l.dsh = (bo & 2u) * 8u;
        return l;
    }
    static HH_DEV void issue(const uint8_t* row, const lane_t& l, data& s) {
        hh_iq_load_run<RUN>(row + l.qo, s.a);
        if constexpr (NG == 2) s.d = *reinterpret_cast<const uint32_t*>(row + l.dof);
    }
    static HH_DEV const uint4* tables() { return reinterpret_cast<const uint4*>(&hh_iq2_ring_tab); }
    static HH_DEV void load_x(const hh_digits_ptr& xd, uint32_t u, xr_t& x) { hh_iq_load_x<NG>(xd, u, x); }
    static HH_DEV void load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hr_t& h) {
        hh_iq_load_h<NG>(q1, q2, sc, u, h);
    }
    typedef hh_iq_hraw<NG> hraw_t;
    static HH_DEV void load_h_raw(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hraw_t& r) {
        hh_iq_load_h_raw<NG>(q1, q2, sc, u, r);
    }
    static HH_DEV void make_h(const hraw_t& r, uint32_t, hr_t& h) { hh_iq_make_h<NG>(r, h); }
    // d/8 * sum_g (2 s_g + 1) t_g  ==  sum_g d (0.5 + s_g) / 4 * t_g   (iq2.rs:513)
    template <class X>
    static HH_DEV float unit(const data& s, const lane_t& l, const X& x, const char* tab) {
        const hh_iq2_tab* t = reinterpret_cast<const hh_iq2_tab*>(tab);
        const uint32_t d = hh_iq_block_d<NG>(NG == 2 ? s.d : s.a[0], l.dsh);
        uint32_t q[2 * NG];
#pragma unroll
        for (int i = 0; i < 2 * NG; i++) q[i] = __builtin_amdgcn_perm(s.a[i + 1], s.a[i], l.sel);
        uint64_t gv[4 * NG];
        hh_iq_sign m[4 * NG];
#pragma unroll
        for (int e = 0; e < 4 * NG; e++) {
            gv[e] = t->grid[(q[2 * (e >> 2)] >> (8 * (e & 3))) & 0xFFu];
            m[e] = t->sgn[(q[2 * (e >> 2) + 1] >> (7 * (e & 3))) & 0x7Fu];
        }
        HH_IQ_FETCH_FENCE();
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const uint32_t a1 = q[2 * g + 1];
            int c1[4], c2[4];
            int r1 = 0, r2 = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int e = 4 * g + k;
                hh_iq_entry((uint32_t)gv[e], (uint32_t)(gv[e] >> 32), m[e], x, g, k, r1, r2);
                c1[k] = r1;
                c2[k] = r2;
            }
            acc = fmaf((float)(2u * (a1 >> 28) + 1u), hh_iq_group_t<NG>(x, g, c1, c2), acc);
        }
        return hh_f16(d) * 0.125f * acc;
    }
    static HH_DEV float unit_x(const data& s, const lane_t& l, const xr_t& x, const char* tab) { return unit(s, l, x, tab); }
    static HH_DEV float unit_h(const data& s, const lane_t& l, const hr_t& h, const char* tab) { return unit(s, l, h, tab); }
};

// IQ3_XXS, NG groups per lane.
template <int NG>
struct hh_ring_iq3 {
    static constexpr uint32_t UNIT = 32 * NG;
    static constexpr uint32_t BB = 98;  // d (f16) + 64 codebook indices + 8 x (4 sign/scale bytes)
    static constexpr uint32_t UPB = 8 / NG;
    static constexpr uint32_t TAB_BYTES = sizeof(hh_iq3_tab);
    static constexpr bool DIRECT_H = true;  // down: h digits per lane, the tables by the copy wave
    static constexpr bool LANE_PARTIALS = true;
    static constexpr int RUN = 2 * NG + 1;  // dwords covering the 8 NG index bytes
    static constexpr int ARUN = NG + 1;     // dwords covering the NG sign/scale words
    struct lane_t {
        uint32_t qo, ao, dof, sel, dsh;
    };
    struct data {
        uint32_t a[RUN];
        uint32_t b[ARUN];
        uint32_t d;  // NG = 2
    };
    typedef hh_iq_x<NG> xr_t;
    typedef hh_iq_h<NG> hr_t;
    static HH_DEV lane_t lane(uint32_t u) {
        const uint32_t bo = (u / UPB) * BB, j = u % UPB;
        lane_t l;
        uint32_t sel2;
        hh_iq_piece(bo + 2u + 8u * NG * j, l.qo, l.sel);
        hh_iq_piece(bo + 66u + 4u * NG * j, l.ao, sel2);  // same parity as the indices
        l.dof = bo & ~3u;
        l.dsh = (bo & 2u) * 8u;
        return l;
    }
    static HH_DEV void issue(const uint8_t* row, const lane_t& l, data& s) {
        hh_iq_load_run<RUN>(row + l.qo, s.a);
        hh_iq_load_run<ARUN>(row + l.ao, s.b);
        if constexpr (NG == 2) s.d = *reinterpret_cast<const uint32_t*>(row + l.dof);
    }
    static HH_DEV const uint4* tables() { return reinterpret_cast<const uint4*>(&hh_iq3_ring_tab); }
    static HH_DEV void load_x(const hh_digits_ptr& xd, uint32_t u, xr_t& x) { hh_iq_load_x<NG>(xd, u, x); }
    static HH_DEV void load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hr_t& h) {
        hh_iq_load_h<NG>(q1, q2, sc, u, h);
    }
    typedef hh_iq_hraw<NG> hraw_t;
    static HH_DEV void load_h_raw(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hraw_t& r) {
        hh_iq_load_h_raw<NG>(q1, q2, sc, u, r);
    }
    static HH_DEV void make_h(const hraw_t& r, uint32_t, hr_t& h) { hh_iq_make_h<NG>(r, h); }
    // d/4 * sum_g (2 s_g + 1) t_g  ==  sum_g d (0.5 + s_g) / 2 * t_g   (iq3.rs:160)
    template <class X>
    static HH_DEV float unit(const data& s, const lane_t& l, const X& x, const char* tab) {
        const hh_iq3_tab* t = reinterpret_cast<const hh_iq3_tab*>(tab);
        const uint32_t d = hh_iq_block_d<NG>(NG == 2 ? s.d : s.a[0], l.dsh);
        uint32_t q[2 * NG], aux[NG];
#pragma unroll
        for (int i = 0; i < 2 * NG; i++) q[i] = __builtin_amdgcn_perm(s.a[i + 1], s.a[i], l.sel);
#pragma unroll
        for (int i = 0; i < NG; i++) aux[i] = __builtin_amdgcn_perm(s.b[i + 1], s.b[i], l.sel);
        // entry k of group g: codebook indices 2k, 2k+1 of the group (elements 8k..8k+3 and
        // 8k+4..8k+7)
        uint32_t g1[4 * NG], g2[4 * NG];
        hh_iq_sign m[4 * NG];
#pragma unroll
        for (int e = 0; e < 4 * NG; e++) {
            const int g = e >> 2, k = e & 3;
            const uint32_t qq = q[2 * g + (k >> 1)] >> (16 * (k & 1));
            g1[e] = t->grid[qq & 0xFFu];
            g2[e] = t->grid[(qq >> 8) & 0xFFu];
            m[e] = t->sgn[(aux[g] >> (7 * k)) & 0x7Fu];
        }
        HH_IQ_FETCH_FENCE();
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const uint32_t ax = aux[g];
            int c1[4], c2[4];
            int r1 = 0, r2 = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int e = 4 * g + k;
                hh_iq_entry(g1[e], g2[e], m[e], x, g, k, r1, r2);
                c1[k] = r1;
                c2[k] = r2;
            }
            acc = fmaf((float)(2u * (ax >> 28) + 1u), hh_iq_group_t<NG>(x, g, c1, c2), acc);
        }
        return hh_f16(d) * 0.25f * acc;
    }
    static HH_DEV float unit_x(const data& s, const lane_t& l, const xr_t& x, const char* tab) { return unit(s, l, x, tab); }
    static HH_DEV float unit_h(const data& s, const lane_t& l, const hr_t& h, const char* tab) { return unit(s, l, h, tab); }
};

// Rows in flight per wave.  Narrow lanes: 64 columns (16.5 / 24.5 bytes per row).  Wide
// lanes: 128 columns (33 / 49 bytes per row), which stream faster; the host picks them for
// gate/up at d_model 8192 (one wave per row) and for IQ2_XXS down projections of at least
// 8192 columns (IQ3_XXS's wide down lane does not fit the down kernel's register budget).
#ifndef HH_IQ_GU_DEPTH
#define HH_IQ_GU_DEPTH 4
#endif
#ifndef HH_IQ_DN_DEPTH
#define HH_IQ_DN_DEPTH 4
#endif
#ifndef HH_IQ_W_DEPTH
#define HH_IQ_W_DEPTH 4
#endif
#ifndef HH_IQ_WDN_DEPTH
#define HH_IQ_WDN_DEPTH 2  // the down kernels' 9-wave workgroups leave 168 VGPRs per lane
#endif
#define HH_IQ_GU(NAME, F, W1, D)                                                                               \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) NAME##_gu_ring_g##W1(HH_GUR_PARAMS) {       \
        hh_gu_ring_body<F, W1, D, 2, false>(HH_GUR_ARGS);                                                     \
    }                                                                                                          \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) NAME##_gu_ring_g##W1##_n(HH_GUR_PARAMS) {   \
        hh_gu_ring_body<F, W1, D, 2, true>(HH_GUR_ARGS);                                                      \
    }
#define HH_IQ_DN(NAME, F, W2, D)                                                                               \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) NAME##_dn_ring_d##W2(HH_DNR_PARAMS) {         \
        hh_dn_ring_body<F, W2, D>(HH_DNR_ARGS);                                                               \
    }
HH_IQ_GU(hh_iq2, hh_ring_iq2<2>, 1, HH_IQ_GU_DEPTH)
HH_IQ_GU(hh_iq2, hh_ring_iq2<2>, 2, HH_IQ_GU_DEPTH)
HH_IQ_DN(hh_iq2, hh_ring_iq2<2>, 1, HH_IQ_DN_DEPTH)
HH_IQ_DN(hh_iq2, hh_ring_iq2<2>, 2, HH_IQ_DN_DEPTH)
HH_IQ_DN(hh_iq2, hh_ring_iq2<2>, 4, HH_IQ_DN_DEPTH)
HH_IQ_DN(hh_iq2, hh_ring_iq2<2>, 8, HH_IQ_DN_DEPTH)
HH_IQ_GU(hh_iq2w, hh_ring_iq2<4>, 1, HH_IQ_W_DEPTH)
HH_IQ_DN(hh_iq2w, hh_ring_iq2<4>, 1, HH_IQ_WDN_DEPTH)
HH_IQ_DN(hh_iq2w, hh_ring_iq2<4>, 2, HH_IQ_WDN_DEPTH)
HH_IQ_DN(hh_iq2w, hh_ring_iq2<4>, 4, HH_IQ_WDN_DEPTH)
HH_IQ_GU(hh_iq3, hh_ring_iq3<2>, 1, HH_IQ_GU_DEPTH)
HH_IQ_GU(hh_iq3, hh_ring_iq3<2>, 2, HH_IQ_GU_DEPTH)
HH_IQ_DN(hh_iq3, hh_ring_iq3<2>, 1, HH_IQ_DN_DEPTH)
HH_IQ_DN(hh_iq3, hh_ring_iq3<2>, 2, HH_IQ_DN_DEPTH)
HH_IQ_DN(hh_iq3, hh_ring_iq3<2>, 4, HH_IQ_DN_DEPTH)
HH_IQ_DN(hh_iq3, hh_ring_iq3<2>, 8, HH_IQ_DN_DEPTH)
HH_IQ_GU(hh_iq3w, hh_ring_iq3<4>, 1, HH_IQ_W_DEPTH)
