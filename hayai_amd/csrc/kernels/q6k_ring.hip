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

template <int WPT2, int D>
HH_DEV void hh_q6k_dn_ring_body(const hh_dnr_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr uint32_t TEAM2 = WPT2 * HH_WAVE, TPW2 = HH_FFNP_CW / WPT2;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff;
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G);
    const uint32_t q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t n2 = (q1 - q0 + TPW2 - 1) / TPW2;
    const uint32_t n2p = (n2 + D - 1) / D * D;

    // the residual of the first row this thread stores, fetched now rather than on the tail
    float res0 = 0.f;
    if (a.res && tid % 32 == 31 && tid / 32 < q1 - q0) res0 = a.res[q0 + tid / 32];

    // LDS: [intermediate][lane partials: rows x TEAM2]
    const uint32_t hbytes = 2u * dff + (dff / 8u) * 4u;
    int8_t* hq1 = reinterpret_cast<int8_t*>(hh_smem);
    int8_t* hq2 = hq1 + dff;
    float* hsc = reinterpret_cast<float*>(hq2 + dff);
    float* part = reinterpret_cast<float*>(hh_smem + ((hbytes + 15u) & ~15u));

    const uint32_t lane2 = tid % TEAM2, team2 = (wave / WPT2) % TPW2;
    const bool act2 = lane2 < dff / 64;
    const uint32_t u2 = act2 ? lane2 : 0u;
    // this lane's superblock within a row and its pieces (row-relative byte offsets); rows
    // start 4-byte aligned (the host checks: an even number of superblocks per row), so the
    // block's alignment is 210*b mod 4 and the last block of a row (odd b) ends its row's
    // reads exactly
    const uint32_t blk = (u2 >> 2) * 210u, hh = (u2 >> 1) & 1u, is = u2 & 1u;
    const uint32_t sh = (blk & 2u) * 8u;  // 0 or 16 bits
    const uint32_t base = blk & ~3u;
    const uint32_t oa = base + 64u * hh + 16u * is, ob = oa + 32u, oh = base + 128u + 32u * hh + 16u * is;
    const uint32_t os = base + 192u + 8u * hh, od = base + 208u;
    const uint8_t* const wdp = a.wd;
    auto issue = [&](uint32_t k, hh_q6k_raw& s) {  // item k: row team2 + k*TPW2
        const uint32_t r = q0 + team2 + k * TPW2;
        const uint8_t* row = wdp + (size_t)(r < q1 ? r : q0) * a.rb2;
        hh_q6k_ld5(row + oa, s.a);
        hh_q6k_ld5(row + ob, s.b);
        hh_q6k_ld5(row + oh, s.h);
        s.s[0] = *reinterpret_cast<const uint32_t*>(row + os);
        s.s[1] = *reinterpret_cast<const uint32_t*>(row + os + 4);
        s.s[2] = *reinterpret_cast<const uint32_t*>(row + os + 8);
        s.d = *reinterpret_cast<const uint32_t*>(row + od);
    };

    hh_q6k_raw ring[D];
    if (wave < HH_FFNP_CW) {
#pragma unroll
        for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
    } else {
        // the intermediate -> LDS, every 16-byte chunk in flight at once
        const uint32_t chunks = hbytes / 16u;
        for (uint32_t c0 = 0; c0 < chunks; c0 += HH_WAVE) {
            if (c0 + lane < chunks)
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void*)(a.hx + (size_t)(c0 + lane) * 16),
                    (__attribute__((address_space(3))) void*)(hh_smem + (size_t)c0 * 16), 16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();  // the intermediate is in LDS (the rings stay in flight)

    if (wave < HH_FFNP_CW) {
        hh_q6k_h hr;
        hh_q6k_load_h(hq1, hq2, hsc, u2, hr);
        for (uint32_t j0 = 0; j0 < n2p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t k = j0 + (uint32_t)s;
                const uint32_t rl = team2 + k * TPW2;  // local row
                if (q0 + rl < q1) {                    // wave-uniform
                    const float v = hh_q6k_unit(ring[s], sh, is, hr);
                    part[rl * TEAM2 + lane2] = act2 ? v : 0.f;  // reduced after the loop
                }
                issue(k + D, ring[s]);
            }
        }
    }
    __syncthreads();  // lane partials are in LDS
    {
        constexpr uint32_t PER = TEAM2 / 32;
        const uint32_t nrows = q1 - q0;
        for (uint32_t rl0 = 0; rl0 < nrows; rl0 += HH_DN_BLOCK / 32) {
            const uint32_t rl = rl0 + tid / 32, seg = tid % 32;
            float s = 0.f;
            if (rl < nrows) {
                const float* p = part + rl * TEAM2 + seg * PER;
#pragma unroll
                for (uint32_t i = 0; i < PER; i++) s += p[i];
            }
            s += hh_dpp<0xB1>(s);        // quad_perm [1,0,3,2]
            s += hh_dpp<0x4E>(s);        // quad_perm [2,3,0,1]
            s += hh_dpp<0x124>(s);       // row_ror:4
            s += hh_dpp<0x128>(s);       // row_ror:8 -> each row of 16 holds its sum
            s += hh_dpp<0x142, 0xA>(s);  // row_bcast:15 -> lanes 31 and 63 hold their half's sum
            if (rl < nrows && seg == 31) a.y[q0 + rl] = a.res ? (rl0 == 0 ? res0 : a.res[q0 + rl]) + s : s;
        }
    }
}

// Two rows in flight per wave: deeper rings measured slower here (8B down, 4096 x 14336:
// 14.2 us at D = 2, 14.8 at 3, 15.8 at 4, 17.3 at 5).
#define HH_Q6K_DN_RING(W2)                                                                              \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_q6k_dn_ring_d##W2(const hh_dnr_args a) { \
        hh_q6k_dn_ring_body<W2, 2>(a);                                                                  \
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
