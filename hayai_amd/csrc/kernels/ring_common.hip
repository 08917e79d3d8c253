// Shared pieces of the batch-1 ring kernels (gfx950; q4k_ring.hip, q6k_ring.hip, iq_ring.hip,
// moe_ring.hip) and the grid barrier of the one-launch small FFN (small_ffn.hip).
// (Compiled after q4k.hip in the same translation unit; uses its digit helpers.)
//
// The intermediate h of an FFN crosses from the gate/up kernel to the down kernel as two
// int8 digits per element with one f32 scale per granule of 8 elements:
//   q1[d_ff] | q2[d_ff] int8 | scale[d_ff/8] f32,   h ~= scale * (q1 + q2/256)
// A down lane owns one 64-column unit of a row and holds that unit's digits in registers.

#define HH_RING_CW 8  // compute waves per ring workgroup

// Digits of h for one lane's down unit u (64 columns), one scale per 8-element granule.
// The granule sums of a sub-block are folded into prefix sums (Abel summation):
//   sum_k s_k * p_k = sum_k (s_k - s_{k+1}) * c_k,   c_k = p_0 + ... + p_k,  s_4 = 0,
// so each digit's dot products run as one chain per sub-block (c_k read off along the way)
// and the weights w_k = (s_k - s_{k+1}) / 256 are computed once per lane.
struct hh_hd {
    uint32_t q1lo[8], q2lo[8], q1hi[8], q2hi[8];
    float wlo[4], whi[4];  // (s_k - s_{k+1}) / 256 per granule
    float xlo, xhi;        // sums of the two sub-blocks' quantized h values
    uint32_t sel_yz, sel_w;
    bool hi_form;
};

// Sum of the quantized values of one 32-element sub-block from its digits and granule
// scales: sum_k s_k * (sum q1 + sum q2 / 256) over granule k.
HH_DEV float hh_hd_sub_sum(const uint32_t (&q1)[8], const uint32_t (&q2)[8], const float (&s)[4]) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int a1 = __builtin_amdgcn_sdot4((int)q1[2 * k], 0x01010101, 0, false);
        a1 = __builtin_amdgcn_sdot4((int)q1[2 * k + 1], 0x01010101, a1, false);
        int a2 = __builtin_amdgcn_sdot4((int)q2[2 * k], 0x01010101, 0, false);
        a2 = __builtin_amdgcn_sdot4((int)q2[2 * k + 1], 0x01010101, a2, false);
        t = fmaf(s[k], (float)(a1 * 256 + a2) * (1.0f / 256.0f), t);
    }
    return t;
}

// A lane's h bytes as loaded (digits of its 64 columns, the 8 granule scales): the loads are
// issued apart from the arithmetic, so a caller can put its weight loads between them.
struct hh_hd_raw {
    uint4 a[4], b[4];
    float4 s0, s1;
};
HH_DEV void hh_hd_load_raw(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_hd_raw& r) {
    const uint4* a = reinterpret_cast<const uint4*>(q1 + (size_t)u * 64);
    const uint4* b = reinterpret_cast<const uint4*>(q2 + (size_t)u * 64);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.a[i] = a[i];
        r.b[i] = b[i];
    }
    r.s0 = reinterpret_cast<const float4*>(sc)[2 * u];
    r.s1 = reinterpret_cast<const float4*>(sc)[2 * u + 1];
}
HH_DEV void hh_hd_make(const hh_hd_raw& r, uint32_t u, hh_hd& h) {
    hh_unpack4(r.a[0], h.q1lo);
    hh_unpack4(r.a[1], h.q1lo + 4);
    hh_unpack4(r.a[2], h.q1hi);
    hh_unpack4(r.a[3], h.q1hi + 4);
    hh_unpack4(r.b[0], h.q2lo);
    hh_unpack4(r.b[1], h.q2lo + 4);
    hh_unpack4(r.b[2], h.q2hi);
    hh_unpack4(r.b[3], h.q2hi + 4);
    const float4 s0 = r.s0, s1 = r.s1;
    const float slo[4] = {s0.x, s0.y, s0.z, s0.w}, shi[4] = {s1.x, s1.y, s1.z, s1.w};
    const float k = 1.0f / 256.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h.wlo[i] = (slo[i] - (i < 3 ? slo[i + 1] : 0.f)) * k;
        h.whi[i] = (shi[i] - (i < 3 ? shi[i + 1] : 0.f)) * k;
    }
    h.xlo = hh_hd_sub_sum(h.q1lo, h.q2lo, slo);
    h.xhi = hh_hd_sub_sum(h.q1hi, h.q2hi, shi);
    const uint32_t g = u & 3u;
    const uint32_t kk = 2u * (g & 1u);
    h.sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    h.sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    h.hi_form = g >= 2;
}
HH_DEV void hh_hd_load(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_hd& h) {
    hh_hd_raw r;
    hh_hd_load_raw(q1, q2, sc, u, r);
    hh_hd_make(r, u, h);
}

// Contribution of one (row, unit) with per-8 granule digit scales.
HH_DEV float hh_q4k_unit_h(const hh_q4k_data& d, const hh_hd& h) {
    const uint32_t qw[8] = {d.q0.x, d.q0.y, d.q0.z, d.q0.w, d.q1.x, d.q1.y, d.q1.z, d.q1.w};
    int c1l = 0, c2l = 0, c1h = 0, c2h = 0;  // prefix sums over granules (see hh_hd)
    float tlo = 0.f, thi = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {  // granule k = qs dwords 2k, 2k+1 (elements 8k..8k+7)
#pragma unroll
        for (int i = 2 * k; i < 2 * k + 2; i++) {
            const int lo = (int)(qw[i] & 0x0F0F0F0Fu);
            const int hi = (int)((qw[i] >> 4) & 0x0F0F0F0Fu);
            c1l = __builtin_amdgcn_sdot4(lo, (int)h.q1lo[i], c1l, false);
            c2l = __builtin_amdgcn_sdot4(lo, (int)h.q2lo[i], c2l, false);
            c1h = __builtin_amdgcn_sdot4(hi, (int)h.q1hi[i], c1h, false);
            c2h = __builtin_amdgcn_sdot4(hi, (int)h.q2hi[i], c2h, false);
        }
        tlo = fmaf(h.wlo[k], (float)(c1l * 256 + c2l), tlo);
        thi = fmaf(h.whi[k], (float)(c1h * 256 + c2h), thi);
    }
    const uint32_t b = __builtin_amdgcn_perm(d.h.z, d.h.y, h.sel_yz);
    const uint32_t lo = b & 0x3F3F3F3Fu;
    const uint32_t wp = __builtin_amdgcn_perm(d.h.w, d.h.w, h.sel_w);
    const uint32_t hi = (wp & 0x00000F0Fu) | ((wp >> 4) & 0x0F0F0000u) | ((b >> 2) & 0x30303030u);
    const uint32_t s = h.hi_form ? hi : lo;
    const float dd = hh_f16(d.h.x & 0xFFFFu);
    const float dm = hh_f16(d.h.x >> 16);
    const float q = hh_ub0(s) * tlo + hh_ub1(s) * thi;
    const float mn = hh_ub2(s) * h.xlo + hh_ub3(s) * h.xhi;
    return dd * q - dm * mn;
}

// Digits of x's chunk c (8 elements, 4 lanes per 32-element sub-block; the quad's lanes
// must all execute this, `has` = chunk exists).
HH_DEV void hh_x_digits_chunk(const float4& t0, const float4& t1, uint32_t c, bool has, const hh_digits_ptr& dst) {
    const float v[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
    float amax = 0.f, s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        s += v[i];
    }
    amax = hh_quad_max(amax);
    s = hh_quad_sum(s);
    const float scale = amax * (1.0f / 127.0f);
    const float inv = amax > 0.f ? 127.0f / amax : 0.f;
    uint2 o1, o2;
    hh_digits8(v, scale, inv, o1, o2);
    if (has) {
        reinterpret_cast<uint2*>(dst.q1)[c] = o1;
        reinterpret_cast<uint2*>(dst.q2)[c] = o2;
        if ((c & 3u) == 0) {
            dst.sc[c / 4] = scale;
            dst.sum[c / 4] = s;
        }
    }
}

// The grouped grid barrier of q4k.hip split into arrival and a bounded wait (one wave
// arrives, then waits; after ~2^20 sleeps the wait records the error word and gives up).
HH_DEV void hh_barrier_arrive(unsigned* bar, unsigned gen) {
    const unsigned G = gridDim.x < HH_BAR_GROUPS ? gridDim.x : HH_BAR_GROUPS;
    const unsigned g = blockIdx.x % HH_BAR_GROUPS;
    const unsigned members = (gridDim.x - g + HH_BAR_GROUPS - 1) / HH_BAR_GROUPS;
    unsigned* cnt = bar + g * HH_BAR_LINE;
    unsigned* top = bar + 2 * HH_BAR_GROUPS * HH_BAR_LINE;
    hh_barrier_gen_ready(gen);
    if (hh_atomic_add_agent(cnt, 1u) == members - 1) {
        hh_store_agent(cnt, 0u);
        if (hh_atomic_add_agent(top, 1u) == G - 1) {
            hh_store_agent(top, 0u);
            __builtin_amdgcn_s_waitcnt(0);
            for (unsigned k = 0; k < G; k++) hh_store_agent(bar + (HH_BAR_GROUPS + k) * HH_BAR_LINE, gen);
            hh_store_agent(top + 2 * HH_BAR_LINE, gen);
        }
    }
}

// Bounded wait for the release of generation gen; false (and the error word set) on timeout.
HH_DEV bool hh_barrier_wait(unsigned* bar, unsigned gen) {
    unsigned* flag = bar + (HH_BAR_GROUPS + blockIdx.x % HH_BAR_GROUPS) * HH_BAR_LINE;
    unsigned* err = bar + (2 * HH_BAR_GROUPS + 1) * HH_BAR_LINE;
    for (unsigned spins = 0; hh_load_agent(flag) != gen; spins++) {
        __builtin_amdgcn_s_sleep(2);
        if (spins > (1u << 20)) {
            hh_store_agent(err, 1u);
            return false;
        }
    }
    return true;
}
