// One persistent launch per Q4_K FFN layer at batch 1 (gfx950):
//   y = W_down . (act(W_gate . x) * (W_up . x))
// i.e. ffn_begin_gate_up_scratch + ffn_finish_scratch (crates/hayai-core/src/
// stream_infer.rs:3752-3864) as one kernel whose HBM stream never pauses between the two
// halves.  (Compiled after q4k.hip in the same translation unit; uses its digit helpers.)
//
// Grid = one workgroup per CU, all co-resident (the host checks occupancy; the dynamic LDS
// request leaves room for one workgroup per CU).  A workgroup is 8 compute waves + 1
// exchange wave.
//
// Weight stream of a compute wave: a ring of D slots, each one lane "item" (the 16-byte
// Q4_K block header + 32 qs bytes of one 64-column unit of one row).  Items are issued D
// ahead of their use, gate/up items first, then down items: the down projection's weights
// are already in flight while the gate/up tail is computed and while the workgroup waits at
// the grid barrier, so HBM keeps streaming through the phase change.  (Workgroup barriers
// on gfx950 wait for LDS only, not for outstanding global loads.)
//
//   phase 1 (gate/up): h rows in granules of 8; workgroup w owns granules
//     [w*NG/G, (w+1)*NG/G) of both W_gate and W_up; a team of WPT1 waves reads one row
//     (lane = unit, x as per-32 int8 digits in registers, as in q4k.hip).
//   exchange (wave 8, which has no weight loads outstanding, so waiting for its own stores
//     waits for nothing else): h = act(g) * u of the workgroup's rows, two int8 digits per
//     element with one scale per 8-element granule (granules never straddle workgroups),
//     stored device-coherently (sc1); arrival at the grid barrier; after the release, all
//     of h's digits are copied (sc1 loads) into LDS for the compute waves.
//   phase 2 (down): workgroup w owns output rows [w*M/G, (w+1)*M/G); a team of WPT2 waves
//     covers one row (lane = unit); partial sums per (row, wave) meet in LDS and lane r of
//     the last step writes y[row].  All sums are in a fixed order: deterministic.
//
// Grid barrier: the grouped counters / generation-tagged release flags of q4k.hip
// (hh_grid_barrier), split into arrival and wait so only the exchange wave touches them.
// The wait is bounded: after ~2^20 sleeps it records an error word and the kernel finishes
// (the host reports the error at its next synchronizing call).

#define HH_FFNP_CW 8                           // compute waves per workgroup
#define HH_FFNP_BLOCK ((HH_FFNP_CW + 1) * HH_WAVE)  // + the exchange wave

struct hh_ffnp_args {
    const uint8_t* wg;  // W_gate [d_ff][rb1]
    const uint8_t* wu;  // W_up   [d_ff][rb1]
    const uint8_t* wd;  // W_down [d_model][rb2]
    const float* x;     // d_model f32, 16-byte aligned
    float* y;           // d_model f32
    uint8_t* hx;        // exchange: q1[d_ff] | q2[d_ff] | scale[d_ff/8] f32 | sum[d_ff/8] f32
    unsigned* bar;      // HH_BAR_WORDS words of grid-barrier state
    uint64_t rb1;       // row bytes of gate/up (d_model columns)
    uint64_t rb2;       // row bytes of down (d_ff columns)
    uint32_t d_model;
    uint32_t d_ff;
    int32_t act;
};

// Digits of h for one lane's down unit u (64 columns), one scale per 8-element granule.
// The granule sums of a sub-block are folded into prefix sums (Abel summation):
//   sum_k s_k * p_k = sum_k (s_k - s_{k+1}) * c_k,   c_k = p_0 + ... + p_k,  s_4 = 0,
// so each digit's dot products run as one chain per sub-block (c_k read off along the way)
// and the weights w_k = (s_k - s_{k+1}) / 256 are computed once per lane.
struct hh_ffnp_h {
    uint32_t q1lo[8], q2lo[8], q1hi[8], q2hi[8];
    float wlo[4], whi[4];  // (s_k - s_{k+1}) / 256 per granule
    float xlo, xhi;        // sums of the two sub-blocks' quantized h values
    uint32_t sel_yz, sel_w;
    bool hi_form;
};

// Sum of the quantized values of one 32-element sub-block from its digits and granule
// scales: sum_k s_k * (sum q1 + sum q2 / 256) over granule k.
HH_DEV float hh_ffnp_sub_sum(const uint32_t (&q1)[8], const uint32_t (&q2)[8], const float (&s)[4]) {
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
struct hh_ffnp_hraw {
    uint4 a[4], b[4];
    float4 s0, s1;
};
HH_DEV void hh_ffnp_load_h_raw(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_ffnp_hraw& r) {
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
HH_DEV void hh_ffnp_make_h(const hh_ffnp_hraw& r, uint32_t u, hh_ffnp_h& h) {
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
    h.xlo = hh_ffnp_sub_sum(h.q1lo, h.q2lo, slo);
    h.xhi = hh_ffnp_sub_sum(h.q1hi, h.q2hi, shi);
    const uint32_t g = u & 3u;
    const uint32_t kk = 2u * (g & 1u);
    h.sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    h.sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    h.hi_form = g >= 2;
}
HH_DEV void hh_ffnp_load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hh_ffnp_h& h) {
    hh_ffnp_hraw r;
    hh_ffnp_load_h_raw(q1, q2, sc, u, r);
    hh_ffnp_make_h(r, u, h);
}

// Contribution of one (row, unit) with per-8 granule digit scales.
HH_DEV float hh_ffnp_unit_g8(const hh_q4k_data& d, const hh_ffnp_h& h) {
    const uint32_t qw[8] = {d.q0.x, d.q0.y, d.q0.z, d.q0.w, d.q1.x, d.q1.y, d.q1.z, d.q1.w};
    int c1l = 0, c2l = 0, c1h = 0, c2h = 0;  // prefix sums over granules (see hh_ffnp_h)
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
HH_DEV void hh_ffnp_digits_chunk(const float4& t0, const float4& t1, uint32_t c, bool has, const hh_digits_ptr& dst) {
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


template <int WPT1, int WPT2, int D, int P>
HH_DEV void hh_ffnp_body(const hh_ffnp_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr uint32_t TEAM1 = WPT1 * HH_WAVE, TPW1 = HH_FFNP_CW / WPT1;
    constexpr uint32_t TEAM2 = WPT2 * HH_WAVE, TPW2 = HH_FFNP_CW / WPT2;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const bool xw = wave == HH_FFNP_CW;  // the exchange wave
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff;
    const unsigned epoch = xw ? hh_barrier_epoch(a.bar) : 0u;  // the exchange wave's

    // phase-1 rows (granules of 8) and phase-2 rows of this workgroup
    const uint32_t NG = dff / 8;
    const uint32_t r0 = 8u * (uint32_t)(((uint64_t)w * NG) / G);
    const uint32_t r1 = 8u * (uint32_t)(((uint64_t)(w + 1) * NG) / G);
    const uint32_t RR = 2u * (r1 - r0);  // row reads: (gate, up) of each row
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G);
    const uint32_t q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t n1 = (RR + TPW1 - 1) / TPW1;
    const uint32_t n1p = (n1 + D - 1) / D * D;  // phase-1 items padded to whole rings
    const uint32_t n2 = (q1 - q0 + TPW2 - 1) / TPW2;
    const uint32_t n2p = (n2 + D - 1) / D * D;

    // LDS: [digits: x (phase 1) / h (phase 2)][gate/up row sums][down lane partials][staging]
    const uint32_t dig_bytes = max(2u * dm + (dm / 32u) * 8u, 2u * dff + (dff / 8u) * 4u);
    char* lds = hh_smem;
    hh_digits_ptr xd;
    xd.q1 = reinterpret_cast<int8_t*>(lds);
    xd.q2 = xd.q1 + dm;
    xd.sc = reinterpret_cast<float*>(xd.q2 + dm);
    xd.sum = xd.sc + dm / 32;
    int8_t* hq1 = reinterpret_cast<int8_t*>(lds);
    int8_t* hq2 = hq1 + dff;
    float* hsc = reinterpret_cast<float*>(hq2 + dff);
    float* gu = reinterpret_cast<float*>(lds + ((dig_bytes + 15u) & ~15u));  // [RR][WPT1]
    float* part = gu + ((RR * WPT1 + 3u) & ~3u);  // [local down row][TEAM2 lanes]
    uint8_t* stage = reinterpret_cast<uint8_t*>(part + (q1 - q0) * TEAM2);  // 2 x 64 B

    // lane roles (team indices from the wave index, which the compiler knows is uniform)
    const uint32_t lane1 = tid % TEAM1, team1 = (wave / WPT1) % TPW1;
    const uint32_t lane2 = tid % TEAM2, team2 = (wave / WPT2) % TPW2;
    const uint32_t U1 = dm / 64, U2 = dff / 64;
    const bool act1 = lane1 < U1, act2 = lane2 < U2;
    const uint32_t u1 = act1 ? lane1 : 0u, u2 = act2 ? lane2 : 0u;

    // The ring's loads: a wave-uniform row address (scalar registers) plus this lane's fixed
    // offsets of its unit (block header, then its 32 qs bytes).  Every decision is
    // wave-uniform, so the loads are never under divergent control flow and the wait counts
    // stay static.  Lanes past the end of a row read unit 0 (their result is discarded);
    // items that are not computed (padding of the last ring, rows past the workgroup's
    // range) re-read the start of W_down.
    const uint8_t* const wgp = a.wg;
    const uint8_t* const wup = a.wu;
    const uint8_t* const wdp = a.wd;
    const uint32_t oh1 = (u1 >> 2) * 144u, oq1 = oh1 + 16u + (u1 & 3u) * 32u;
    const uint32_t oh2 = (u2 >> 2) * 144u, oq2 = oh2 + 16u + (u2 & 3u) * 32u;
    auto load3 = [](const uint8_t* row, uint32_t oh, uint32_t oq, hh_q4k_data& s) {
        s.h = hh_ld16(row + oh);
        s.q0 = hh_ld16(row + oq);
        s.q1 = hh_ld16(row + oq + 16);
    };
    auto issue1 = [&](uint32_t j, hh_q4k_data& s) {  // phase-1 item j (a gate or up row)
        const uint32_t i = team1 + j * TPW1;
        const uint8_t* row = i < RR ? ((i & 1u) ? wup : wgp) + (size_t)(r0 + (i >> 1)) * a.rb1 : wdp;
        load3(row, oh1, oq1, s);
    };
    auto issue2 = [&](uint32_t k, hh_q4k_data& s) {  // phase-2 item k (a down row)
        const uint32_t r = q0 + team2 + k * TPW2;
        load3(r < q1 ? wdp + (size_t)r * a.rb2 : wdp, oh2, oq2, s);
    };

    // Prologue: every compute thread first loads its 8 elements of x, then (after a
    // workgroup barrier, so all of the CU's x requests are queued before any ring request)
    // the ring's first P items go out, x is quantized into per-32 digits in LDS, and only
    // then the rest of the ring: a deep ring burst at start would delay x (its requests
    // share the memory queues with every CU's ring), while a short one gets x back fast.
    hh_q4k_data ring[D];
    auto fill = [&](int s) {
        if ((uint32_t)s < n1p) issue1((uint32_t)s, ring[s]);
        else issue2((uint32_t)s - n1p, ring[s]);
    };
    const uint32_t c = tid;  // chunk of 8 elements (d_model <= 8 * 512 per pass)
    const bool has = !xw && c < dm / 8;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    float4 t0 = make_float4(0.f, 0.f, 0.f, 0.f), t1 = t0;
    if (!xw) {
        t0 = x4[2 * min(c, dm / 8 - 1)];
        t1 = x4[2 * min(c, dm / 8 - 1) + 1];
    }
    __syncthreads();
    if (!xw) {
#pragma unroll
        for (int s = 0; s < P; s++) fill(s);
        hh_ffnp_digits_chunk(t0, t1, c, has, xd);
        for (uint32_t c2 = c + HH_FFNP_CW * HH_WAVE; c2 < dm / 8; c2 += HH_FFNP_CW * HH_WAVE) {
            const float4 u0 = x4[2 * c2], u1 = x4[2 * c2 + 1];  // d_model > 4096: later passes
            hh_ffnp_digits_chunk(u0, u1, c2, true, xd);
        }
#pragma unroll
        for (int s = P; s < D; s++) fill(s);
    }
    __syncthreads();

    if (!xw) {
        hh_q4k_x xr;
        hh_q4k_load_lane_x(xd, u1, xr);
        for (uint32_t j0 = 0; j0 < n1p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t j = j0 + (uint32_t)s;
                const uint32_t i = team1 + j * TPW1;
                if (i < RR) {  // wave-uniform
                    float v = hh_q4k_unit(ring[s], xr);
                    v = hh_wave_sum(act1 ? v : 0.f);
                    if (lane == 0) gu[i * WPT1 + wave % WPT1] = v;
                }
                // the next gate/up item, or (in the last ring) a down item
                if (j + D < n1p) issue1(j + D, ring[s]);
                else issue2(j + D - n1p, ring[s]);
            }
        }
    }
    __syncthreads();  // phase-1 row sums are in LDS

    if (xw) {
        uint64_t* gq1 = reinterpret_cast<uint64_t*>(a.hx);
        uint64_t* gq2 = reinterpret_cast<uint64_t*>(a.hx + dff);
        unsigned* gsc = reinterpret_cast<unsigned*>(a.hx + 2 * (size_t)dff);
        for (uint32_t rho0 = 0; rho0 < r1 - r0; rho0 += HH_WAVE) {
            const uint32_t rho = rho0 + lane;
            const bool ok = rho < r1 - r0;  // granule-aligned: whole 8-lane groups agree
            float hv = 0.f;
            if (ok) {
                float g = 0.f, u = 0.f;
#pragma unroll
                for (int k = 0; k < WPT1; k++) {
                    g += gu[(2 * rho) * WPT1 + k];
                    u += gu[(2 * rho + 1) * WPT1 + k];
                }
                hv = hh_act_mul(g, u, a.act);
            }
            float amax = fabsf(hv);
#pragma unroll
            for (int m = 1; m < 8; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, HH_WAVE));
            const float scale = amax * (1.0f / 127.0f);
            const float inv = amax > 0.f ? 127.0f / amax : 0.f;
            const float d1 = fminf(fmaxf(rintf(hv * inv), -127.f), 127.f);
            const float rr = hv - d1 * scale;
            const float d2 = fminf(fmaxf(rintf(rr * inv * 256.0f), -127.f), 127.f);
            stage[lane] = (uint8_t)(int8_t)(int)d1;
            stage[64 + lane] = (uint8_t)(int8_t)(int)d2;
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): staged bytes visible to the wave
            __builtin_amdgcn_wave_barrier();
            if (ok && (lane & 7u) == 0) {
                const uint32_t gi = (r0 + rho) / 8;  // granule index in h
                const uint64_t v1 = *reinterpret_cast<const uint64_t*>(stage + lane);
                const uint64_t v2 = *reinterpret_cast<const uint64_t*>(stage + 64 + lane);
                __hip_atomic_store(gq1 + gi, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(gq2 + gi, v2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                hh_store_agent(gsc + gi, __float_as_uint(scale));
            }
            __builtin_amdgcn_wave_barrier();
        }
        // every h store of this wave is complete (vmcnt covers stores), then arrive and wait
        __builtin_amdgcn_s_waitcnt(0);
        int good = 1;
        if (lane == 0) {
            hh_barrier_arrive(a.bar, epoch + 1u);
            good = hh_barrier_wait(a.bar, epoch + 1u) ? 1 : 0;
        }
        good = __builtin_amdgcn_readfirstlane(good);
        if (good) {
            // all of h's digits -> LDS by global->LDS DMA, every chunk in flight at once.  Plain
            // (L2-cached) loads: no L2 holds these lines yet in this launch (they are first
            // read after the barrier, and each kernel starts with the L2s invalidated), so the
            // first workgroup of an XCD fetches them from memory and the others hit its L2.
            const uint32_t chunks = (2u * dff + (dff / 8u) * 4u) / 16u;
            for (uint32_t c0 = 0; c0 < chunks; c0 += HH_WAVE) {
                if (c0 + lane < chunks)
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void*)(a.hx + (size_t)(c0 + lane) * 16),
                        (__attribute__((address_space(3))) void*)(hq1 + (size_t)c0 * 16), 16, 0, 0);
            }
            __builtin_amdgcn_s_waitcnt(0);
        }
    }
    __syncthreads();  // h digits are in LDS

    if (!xw) {
        hh_ffnp_h hr;
        hh_ffnp_load_h(hq1, hq2, hsc, u2, hr);
        for (uint32_t j0 = 0; j0 < n2p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t k = j0 + (uint32_t)s;
                const uint32_t rl = team2 + k * TPW2;  // local row
                if (q0 + rl < q1) {                    // wave-uniform
                    const float v = hh_ffnp_unit_g8(ring[s], hr);
                    part[rl * TEAM2 + lane2] = act2 ? v : 0.f;  // reduced after the loop
                }
                issue2(k + D, ring[s]);
            }
        }
    }
    __syncthreads();  // down lane partials are in LDS
    // y[q0 + rl] = sum over the TEAM2 lane partials of row rl: 32 threads per row, each sums
    // TEAM2/32 consecutive partials, then a 32-lane DPP reduction (rows never straddle the
    // 32-lane halves of a wave; fixed order: deterministic)
    {
        constexpr uint32_t PER = TEAM2 / 32;
        const uint32_t nrows = q1 - q0;
        for (uint32_t rl0 = 0; rl0 < nrows; rl0 += HH_FFNP_BLOCK / 32) {
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
            if (rl < nrows && seg == 31) a.y[q0 + rl] = s;
        }
    }
}

// hh_q4k_ffnp_g<WPT1>_d<WPT2>: WPT1 waves per gate/up row (d_model <= 4096 * WPT1),
// WPT2 waves per down row (d_ff <= 4096 * WPT2), ring depth D, P ring items issued before x.
#define HH_FFNP(G1, G2, D, P)                                                                   \
    extern "C" __global__ void __launch_bounds__(HH_FFNP_BLOCK) hh_q4k_ffnp_g##G1##_d##G2(const hh_ffnp_args a) { \
        hh_ffnp_body<G1, G2, D, P>(a);                                                          \
    }
HH_FFNP(1, 1, 3, 1)
HH_FFNP(1, 2, 3, 1)
HH_FFNP(1, 4, 3, 1)
HH_FFNP(1, 8, 3, 1)
HH_FFNP(2, 2, 3, 1)
HH_FFNP(2, 4, 3, 1)
HH_FFNP(2, 8, 3, 1)
