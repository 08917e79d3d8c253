// The down projection of the ring FFN (q4k_ring.hip) for a Q6_K W_down: real Q4_K_M files
// keep ffn_down of many layers in Q6_K (gemv_q6_k, crates/hayai-model/src/q6k.rs:59-88;
// ggml_gemv_q6_k, crates/hayai-kernels/kernels/ggml_gemv_q4.cl:422-472).  It consumes the
// gate/up ring kernel's intermediate (h as two int8 digits per element, one scale per
// granule of 8) and has the Q4_K down kernel's shape: a team of WPT2 waves per row, lane =
// unit, a ring of D rows in flight per wave, a ninth wave copying the intermediate into LDS,
// lane partials reduced per row in a fixed order.
// (Compiled after q4k_ring.hip in the same translation unit.)
//
// Unit (lane) = quarter (h, is) of a 210-byte superblock: 16 columns of each of the four
// 32-column groups of half h (the element order of dequant_q6_k_block, q6k.rs:27-57).
// Superblocks sit at 210-byte steps, so a block is 4-byte aligned or 2 bytes off: the lane
// loads the dwords covering each 16-byte piece (4-byte aligned) and realigns them with one
// funnel shift per dword.

// A lane's pieces of one superblock, realigned: ql[64h+16is..+16), ql[64h+32+16is..+16),
// qh[32h+16is..+16), the 8 scale bytes of half h, and the dword holding d.
struct hh_q6k_raw {
    uint32_t a[5], b[5], h[5], s[3], d;
};

typedef uint32_t hh_v4u_a4 __attribute__((ext_vector_type(4), aligned(4)));

HH_DEV void hh_q6k_ld5(const uint8_t* p, uint32_t* w) {
    const hh_v4u_a4 v = *reinterpret_cast<const hh_v4u_a4*>(p);
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
    w[4] = *reinterpret_cast<const uint32_t*>(p + 16);
}

// h of one unit: the digits of its four 16-element runs, the 8 granule scales / 256 and the
// exact sums of the quantized h over each run (for the -32 offset of the codes).
struct hh_q6k_h {
    uint32_t q1[16], q2[16];
    float w[8];
    float hs[4];
};

HH_DEV void hh_q6k_load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_q6k_h& h) {
    const uint32_t e0 = (u >> 2) * 256 + 128 * ((u >> 1) & 1u) + 16 * (u & 1u);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t e = e0 + 32 * r;
        const uint4 a = *reinterpret_cast<const uint4*>(q1 + e);
        const uint4 b = *reinterpret_cast<const uint4*>(q2 + e);
        h.q1[4 * r] = a.x;
        h.q1[4 * r + 1] = a.y;
        h.q1[4 * r + 2] = a.z;
        h.q1[4 * r + 3] = a.w;
        h.q2[4 * r] = b.x;
        h.q2[4 * r + 1] = b.y;
        h.q2[4 * r + 2] = b.z;
        h.q2[4 * r + 3] = b.w;
        const float2 s = *reinterpret_cast<const float2*>(sc + e / 8);
        h.w[2 * r] = s.x * (1.0f / 256.0f);
        h.w[2 * r + 1] = s.y * (1.0f / 256.0f);
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            int a1 = __builtin_amdgcn_sdot4((int)h.q1[4 * r + 2 * k], 0x01010101, 0, false);
            a1 = __builtin_amdgcn_sdot4((int)h.q1[4 * r + 2 * k + 1], 0x01010101, a1, false);
            int a2 = __builtin_amdgcn_sdot4((int)h.q2[4 * r + 2 * k], 0x01010101, 0, false);
            a2 = __builtin_amdgcn_sdot4((int)h.q2[4 * r + 2 * k + 1], 0x01010101, a2, false);
            t = fmaf(h.w[2 * r + k], (float)(a1 * 256 + a2), t);
        }
        h.hs[r] = t;
    }
}

// Contribution of one (row, unit): d * sum_r sc_r * (sum_l q_l h_l - 32 * sum_l h_l), with the
// 6-bit codes q built per byte from the ql nibbles and the qh bit pairs.
HH_DEV float hh_q6k_unit(const hh_q6k_raw& raw, uint32_t sh, uint32_t is, const hh_q6k_h& h) {
    uint32_t la[4], lb[4], hb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        la[i] = __builtin_amdgcn_alignbit(raw.a[i + 1], raw.a[i], sh);
        lb[i] = __builtin_amdgcn_alignbit(raw.b[i + 1], raw.b[i], sh);
        hb[i] = __builtin_amdgcn_alignbit(raw.h[i + 1], raw.h[i], sh);
    }
    // scales of half h: bytes 0..7 of the realigned 8-byte run; this unit's four are
    // bytes is, is+2, is+4, is+6
    const uint32_t s0 = __builtin_amdgcn_alignbit(raw.s[1], raw.s[0], sh);
    const uint32_t s1 = __builtin_amdgcn_alignbit(raw.s[2], raw.s[1], sh);
    const uint32_t sel = is ? 0x07050301u : 0x06040200u;  // bytes (is, is+2) of s0, then of s1
    const int32_t scw = (int32_t)__builtin_amdgcn_perm(s1, s0, sel);
    const float d = hh_f16((raw.d >> sh) & 0xFFFFu);
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            int c1 = 0, c2 = 0;
#pragma unroll
            for (int i = 2 * k; i < 2 * k + 2; i++) {
                // codes of columns 4i..4i+3 of run r (q6k.rs:39-42)
                uint32_t q;
                if (r == 0) q = (la[i] & 0x0F0F0F0Fu) | ((hb[i] << 4) & 0x30303030u);
                else if (r == 1) q = (lb[i] & 0x0F0F0F0Fu) | ((hb[i] << 2) & 0x30303030u);
                else if (r == 2) q = ((la[i] >> 4) & 0x0F0F0F0Fu) | (hb[i] & 0x30303030u);
                else q = ((lb[i] >> 4) & 0x0F0F0F0Fu) | ((hb[i] >> 2) & 0x30303030u);
                c1 = __builtin_amdgcn_sdot4((int)q, (int)h.q1[4 * r + i], c1, false);
                c2 = __builtin_amdgcn_sdot4((int)q, (int)h.q2[4 * r + i], c2, false);
            }
            // |c1| <= 8 * 63 * 127, so 256 * c1 + c2 is exact in an int32
            t = fmaf(h.w[2 * r + k], (float)(c1 * 256 + c2), t);
        }
        const float sc = (float)((scw << (24 - 8 * r)) >> 24);  // i8 scale of run r
        acc = fmaf(sc, t - 32.0f * h.hs[r], acc);
    }
    return d * acc;
}

// The Q6_K down format of the generic ring body (hh_dn_ring_body, q4k_ring.hip).  Rows start
// 4-byte aligned (the host checks: an even number of superblocks per row), so the lane's
// block is 4-byte aligned or 2 bytes off (210*b mod 4) and the last block of a row (odd b)
// ends its row's reads exactly.
struct hh_ring_q6k {
    static constexpr uint32_t UNIT = 64;
    static constexpr uint32_t TAB_BYTES = 0;
    static constexpr bool DIRECT_H = false;  // down: the copy wave brings h's digits into LDS
    static constexpr bool LANE_PARTIALS = false;
    struct lane_t {
        uint32_t oa, ob, oh, os, od;  // dword-aligned offsets of the lane's pieces
        uint32_t sh, is;              // realignment (0 or 16 bits), quarter within the half
    };
    typedef hh_q6k_raw data;
    typedef hh_q6k_h hr_t;
    static HH_DEV lane_t lane(uint32_t u) {
        const uint32_t blk = (u >> 2) * 210u, hh = (u >> 1) & 1u, is = u & 1u;
        const uint32_t base = blk & ~3u;
        lane_t l;
        l.oa = base + 64u * hh + 16u * is;
        l.ob = l.oa + 32u;
        l.oh = base + 128u + 32u * hh + 16u * is;
        l.os = base + 192u + 8u * hh;
        l.od = base + 208u;
        l.sh = (blk & 2u) * 8u;
        l.is = is;
        return l;
    }
    static HH_DEV void issue(const uint8_t* row, const lane_t& l, data& s) {
        hh_q6k_ld5(row + l.oa, s.a);
        hh_q6k_ld5(row + l.ob, s.b);
        hh_q6k_ld5(row + l.oh, s.h);
        s.s[0] = *reinterpret_cast<const uint32_t*>(row + l.os);
        s.s[1] = *reinterpret_cast<const uint32_t*>(row + l.os + 4);
        s.s[2] = *reinterpret_cast<const uint32_t*>(row + l.os + 8);
        s.d = *reinterpret_cast<const uint32_t*>(row + l.od);
    }
    static HH_DEV const uint4* tables() { return nullptr; }
    static HH_DEV void load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hr_t& h) {
        hh_q6k_load_h(q1, q2, sc, u, h);
    }
    static HH_DEV float unit_h(const data& s, const lane_t& l, const hr_t& h, const char*) {
        return hh_q6k_unit(s, l.sh, l.is, h);
    }
};

// Two rows in flight per wave: deeper rings measured slower here (8B down, 4096 x 14336:
// 14.2 us at D = 2, 14.8 at 3, 15.8 at 4, 17.3 at 5).
#define HH_Q6K_DN_RING(W2)                                                                              \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_q6k_dn_ring_d##W2(HH_DNR_PARAMS) {     \
        hh_dn_ring_body<hh_ring_q6k, W2, 2>(HH_DNR_ARGS);                                               \
    }
HH_Q6K_DN_RING(1)
HH_Q6K_DN_RING(2)
HH_Q6K_DN_RING(4)
HH_Q6K_DN_RING(8)

// x -> digits for the ring GEMV (the same two-digit form the gate/up ring kernel writes for
// h): per granule of 8, scale = max|x| / 127, d1 = rint(x / scale), d2 = rint((x - d1 scale)
// * 256 / scale), both clamped to +-127.  One thread per granule.
extern "C" __global__ void __launch_bounds__(256) hh_x_digits(const hh_xd_args a) {
    const uint32_t g = blockIdx.x * 256 + threadIdx.x;
    if (g >= a.n / 8) return;
    float v[8];
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        v[k] = a.x[8 * g + k];
        amax = fmaxf(amax, fabsf(v[k]));
    }
    const float scale = amax * (1.0f / 127.0f);
    const float inv = amax > 0.f ? 127.0f / amax : 0.f;
    uint32_t q1[2] = {0u, 0u}, q2[2] = {0u, 0u};
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float d1 = fminf(fmaxf(rintf(v[k] * inv), -127.f), 127.f);
        const float r = v[k] - d1 * scale;
        const float d2 = fminf(fmaxf(rintf(r * inv * 256.0f), -127.f), 127.f);
        q1[k / 4] |= ((uint32_t)(int32_t)d1 & 0xFFu) << (8 * (k % 4));
        q2[k / 4] |= ((uint32_t)(int32_t)d2 & 0xFFu) << (8 * (k % 4));
    }
    int8_t* hq1 = reinterpret_cast<int8_t*>(a.hx);
    int8_t* hq2 = hq1 + a.n;
    float* hsc = reinterpret_cast<float*>(hq2 + a.n);
    *reinterpret_cast<uint2*>(hq1 + 8 * g) = make_uint2(q1[0], q1[1]);
    *reinterpret_cast<uint2*>(hq2 + 8 * g) = make_uint2(q2[0], q2[1]);
    hsc[g] = scale;
}
