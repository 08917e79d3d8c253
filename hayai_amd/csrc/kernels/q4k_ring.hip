// The Q4_K FFN at batch 1 as two streaming launches (gfx950):
//   hh_q4k_gu_ring_g<W1>:  h = act(W_gate . x) * (W_up . x), written as int8 digits
//                          (ffn_begin_gate_up_scratch, crates/hayai-core/src/
//                          stream_infer.rs:3752-3808, with the activation of :3836-3840)
//   hh_q4k_dn_ring_d<W2>:  y = W_down . h from those digits (ffn_finish_scratch, :3809-3864)
// (Compiled after ring_common.hip in the same translation unit; uses its digit helpers.)
//
// Each launch is one weight stream with nothing else on its path: a kernel boundary costs
// less than an exchange of h between the workgroups of one launch (measured: a grid barrier
// plus the exchange under a full HBM stream took ~5 us, the boundary plus the h hop ~3 us),
// so the layer is split there.  In both kernels every compute wave keeps D items
// (one 64-column Q4_K unit of one row per lane: 16-byte block header + 32 qs bytes) in
// flight, addressed by a wave-uniform row base plus fixed lane offsets, so the wait counts
// are static and HBM never waits for the math.
//
// Intermediate: q1[d_ff] | q2[d_ff] int8 | scale[d_ff/8] f32, h ~ scale * (q1 + q2/256) per
// granule of 8 rows (granules never straddle workgroups).
//
// The two bodies are generic over the weight format F (Q4_K here; Q6_K in q6k_ring.hip,
// IQ2_XXS / IQ3_XXS in iq_ring.hip).  F supplies:
//   UNIT             columns per lane unit (64 for every format)
//   TAB_BYTES        lookup tables the format keeps in static LDS (multiple of 16; 0: none),
//                    copied from tables() by the kernel
//   lane_t, lane(u)  the lane's fixed byte offsets within a row for unit u
//   data, issue()    one ring item: the lane's loads of one row
//   xr_t, load_x()   x as per-32 digits (gate/up); unit_x(): the (row, unit) contribution
//   hr_t, load_h()   h as per-8 digits (down);     unit_h(): the (row, unit) contribution
//   LANE_PARTIALS    gate/up: each lane's contribution goes to LDS and rows are summed once
//                    after the loop (formats with long per-row arithmetic), instead of a
//                    wave reduction per row
//   DIRECT_H         down: each lane loads its h digits from global memory itself

#define HH_RING_BLOCK (HH_RING_CW * HH_WAVE)
// Row assignment.  HH_RING_ILV 1 (default): workgroup w takes granules (gate/up) or rows
// (down) w, w + G, w + 2G, ..., so at any moment the whole grid reads one contiguous band of
// the matrix and sweeps it front to back; 0: a contiguous range per workgroup.  Measured on
// the 8B headline: gate/up 13.75 -> 13.02 us per launch, 719 -> 689 us per 32-layer step (down
// unchanged).
#ifndef HH_RING_ILV
#define HH_RING_ILV 1
#endif

// Phase timeline of the ring kernels, compiled in only when a separate code object is built
// with -DHH_RING_TRACE for a timeline probe (never in the library): one timestamp of the
// 100 MHz realtime counter per workgroup and phase, indexed by the layer that the weight
// pointer falls in ((w - base) / stride, both set by the probe's host side).
#ifdef HH_RING_TRACE
__device__ unsigned long long hh_ring_trace[2][64][512][8];  // [gate/up, down][layer][workgroup][phase]
__constant__ const uint8_t* hh_ring_trace_base;  // constant: scalar loads, no vector-memory wait
__constant__ unsigned long long hh_ring_trace_stride;
HH_DEV void hh_ring_mark(int kind, const uint8_t* w, int phase) {
    const long long l = (long long)((w - hh_ring_trace_base) / (long long)hh_ring_trace_stride);
    if (l >= 0 && l < 64 && blockIdx.x < 512) hh_ring_trace[kind][l][blockIdx.x][phase] = __builtin_amdgcn_s_memrealtime();
}
#define HH_RING_MARK(kind, w, phase, cond) \
    do {                                   \
        if (cond) hh_ring_mark(kind, w, phase); \
    } while (0)
#else
#define HH_RING_MARK(kind, w, phase, cond) ((void)0)
#endif

// sum of squares of 8 elements, and x * inv * weight in the reference's order
// (simd_scale_mul, crates/hayai-cpu/src/simd_ops.rs:28-41)
HH_DEV float hh_sq8(const float4& a, const float4& b) {
    return a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
}
HH_DEV void hh_norm8(float4& a, float4& b, const float4& wa, const float4& wb, float inv) {
    a.x = (a.x * inv) * wa.x;
    a.y = (a.y * inv) * wa.y;
    a.z = (a.z * inv) * wa.z;
    a.w = (a.w * inv) * wa.w;
    b.x = (b.x * inv) * wb.x;
    b.y = (b.y * inv) * wb.y;
    b.z = (b.z * inv) * wb.z;
    b.w = (b.w * inv) * wb.w;
}

struct hh_gur_args {
    const uint8_t* wg;  // W_gate [d_ff][rb1]
    const uint8_t* wu;  // W_up   [d_ff][rb1]
    const float* x;     // d_model f32, 16-byte aligned
    uint8_t* hx;        // intermediate (above)
    const float* nw;    // RMSNorm weight (d_model f32, 16-byte aligned), or null: x as given
    uint64_t rb1;       // row bytes of gate/up
    uint32_t d_model;
    uint32_t d_ff;
    int32_t act;
    float eps;          // RMSNorm epsilon (with nw)
    uint32_t grid;      // workgroups of the launch
};

struct hh_dnr_args {
    const uint8_t* wd;  // W_down [d_model][rb2]
    const uint8_t* hx;  // intermediate (above), 16-byte aligned
    float* y;           // d_model f32
    const float* res;   // residual added to y (may be y itself), or null
    uint64_t rb2;       // row bytes of down
    uint32_t d_model;
    uint32_t d_ff;
};

// The format's LDS tables: a static LDS array (its address is a compile-time constant, so
// table reads take an immediate offset), or none.
template <uint32_t N>
HH_DEV char* hh_ring_tables_lds() {
    __shared__ __attribute__((aligned(16))) char t[N];
    return t;
}
template <>
HH_DEV char* hh_ring_tables_lds<0>() {
    return nullptr;
}

struct hh_ring_q4k {
    static constexpr uint32_t UNIT = 64;
    static constexpr uint32_t TAB_BYTES = 0;
    static constexpr bool DIRECT_H = true;  // down: h digits loaded per lane (no LDS copy)
    static constexpr bool LANE_PARTIALS = false;
    struct lane_t {
        uint32_t oh, oq;  // block header, this unit's 32 qs bytes
    };
    typedef hh_q4k_data data;
    typedef hh_q4k_x xr_t;
    typedef hh_hd hr_t;
    static HH_DEV lane_t lane(uint32_t u) {
        const uint32_t oh = (u >> 2) * 144u;
        return lane_t{oh, oh + 16u + (u & 3u) * 32u};
    }
    static HH_DEV void issue(const uint8_t* row, const lane_t& l, data& s) {
        s.h = hh_ld16(row + l.oh);
        s.q0 = hh_ld16(row + l.oq);
        s.q1 = hh_ld16(row + l.oq + 16);
    }
    static HH_DEV const uint4* tables() { return nullptr; }
    static HH_DEV void load_x(const hh_digits_ptr& xd, uint32_t u, xr_t& xr) { hh_q4k_load_lane_x(xd, u, xr); }
    static HH_DEV void load_h(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hr_t& h) {
        hh_hd_load(q1, q2, sc, u, h);
    }
    typedef hh_hd_raw hraw_t;
    static HH_DEV void load_h_raw(const int8_t* q1, const int8_t* q2, const float* sc, uint32_t u, hraw_t& r) {
        hh_hd_load_raw(q1, q2, sc, u, r);
    }
    static HH_DEV void make_h(const hraw_t& r, uint32_t u, hr_t& h) { hh_hd_make(r, u, h); }
    static HH_DEV float unit_x(const data& s, const lane_t&, const xr_t& xr, const char*) { return hh_q4k_unit(s, xr); }
    static HH_DEV float unit_h(const data& s, const lane_t&, const hr_t& h, const char*) { return hh_q4k_unit_h(s, h); }
};

// Gate/up: workgroup w owns the 8-row granules w, w + G, ... of W_gate and W_up (HH_RING_ILV);
// a team of WPT1 waves reads one row (lane = unit, x as per-32 digits in registers).  After
// the last row, wave 0 applies the activation to the workgroup's rows and writes their
// digits.
template <class F, int WPT1, int D, int P, bool NORM>
HH_DEV void hh_gu_ring_body(const hh_gur_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr uint32_t TEAM1 = WPT1 * HH_WAVE, TPW1 = HH_RING_CW / WPT1;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = a.grid, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff;
    const uint32_t NG = dff / 8;
#if HH_RING_ILV
    // granules w, w + G, w + 2G, ...: every workgroup's reads spread over the whole matrix
    const uint32_t nrw = 8u * ((NG - min(w, NG) + G - 1) / G);  // the workgroup's rows
    auto row_of = [&](uint32_t rho) { return 8u * (w + (rho / 8u) * G) + rho % 8u; };
#else
    const uint32_t r0 = 8u * (uint32_t)(((uint64_t)w * NG) / G);
    const uint32_t r1 = 8u * (uint32_t)(((uint64_t)(w + 1) * NG) / G);
    const uint32_t nrw = r1 - r0;
    auto row_of = [&](uint32_t rho) { return r0 + rho; };
#endif
    const uint32_t RR = 2u * nrw;  // row reads: (gate, up) of each row
    HH_RING_MARK(0, a.wg, 0, tid == 0);
    const uint32_t n1 = (RR + TPW1 - 1) / TPW1;
    const uint32_t n1p = (n1 + D - 1) / D * D;

    // LDS: static: the format's tables; dynamic: [x digits][gate/up row sums][staging 128 B],
    // with lane partials: [x digits][partials: RR x TEAM1][row sums: RR][staging 128 B]
    constexpr bool LP = F::LANE_PARTIALS;
    char* const tabs = hh_ring_tables_lds<F::TAB_BYTES>();
    char* const lds = hh_smem;
    const uint32_t xbytes = 2u * dm + (dm / 32u) * 8u;
    hh_digits_ptr xd;
    xd.q1 = reinterpret_cast<int8_t*>(lds);
    xd.q2 = xd.q1 + dm;
    xd.sc = reinterpret_cast<float*>(xd.q2 + dm);
    xd.sum = xd.sc + dm / 32;
    float* gu = reinterpret_cast<float*>(lds + ((xbytes + 15u) & ~15u));  // [RR][WPT1] or [RR][TEAM1]
    float* rows = gu + (LP ? RR * TEAM1 : 0u);                            // [RR] (lane partials)
    uint8_t* stage = reinterpret_cast<uint8_t*>(rows + ((RR * (LP ? 1u : WPT1) + 3u) & ~3u));

    const uint32_t lane1 = tid % TEAM1, team1 = (wave / WPT1) % TPW1;
    const bool act1 = lane1 < dm / F::UNIT;
    const uint32_t u1 = act1 ? lane1 : 0u;
    const uint8_t* const wgp = a.wg;
    const uint8_t* const wup = a.wu;
    const typename F::lane_t lo = F::lane(u1);
    // item j of this team: row read i = team1 + j*TPW1 (gate and up rows interleaved); reads
    // past the workgroup's rows (ring padding) re-read the start of W_gate
    auto issue = [&](uint32_t j, typename F::data& s) {
        const uint32_t i = team1 + j * TPW1;
        const uint8_t* row = i < RR ? ((i & 1u) ? wup : wgp) + (size_t)row_of(i >> 1) * a.rb1 : wgp;
        F::issue(row, lo, s);
    };

    // the format's tables (if any) are requested first and stored to LDS with x's digits
    constexpr uint32_t TAB16 = F::TAB_BYTES / 16u;
    uint4 tab = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (TAB16 > 0) {
        static_assert(TAB16 <= HH_RING_BLOCK, "one 16-byte table chunk per thread");
        if (tid < TAB16) tab = F::tables()[tid];
    }

    // prologue: x loads first, then P ring items, x -> per-32 digits in LDS, the rest of the
    // ring (x is not queued behind a burst of weight requests)
    typename F::data ring[D];
    const uint32_t c = tid;  // chunk of 8 elements (d_model <= 8 * 512 per pass)
    const bool has = c < dm / 8;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    float4 t0 = x4[2 * min(c, dm / 8 - 1)];
    float4 t1 = x4[2 * min(c, dm / 8 - 1) + 1];
    const float4* n4 = reinterpret_cast<const float4*>(a.nw);
    float4 m0 = make_float4(1.f, 1.f, 1.f, 1.f), m1 = m0;
    if constexpr (NORM) {
        m0 = n4[2 * min(c, dm / 8 - 1)];
        m1 = n4[2 * min(c, dm / 8 - 1) + 1];
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < P; s++) issue((uint32_t)s, ring[s]);
    if constexpr (NORM) {
        // RMSNorm (rms_norm, crates/hayai-cpu/src/attention.rs:142-147, applied before the
        // FFN by ffn_apply, crates/hayai-core/src/hybrid_infer.rs:895-896): every workgroup
        // forms sum(x^2) itself (d_model floats from L2).  The GEMVs are linear in x, so x *
        // weight is quantized right away and the common factor inv = 1 / sqrt(mean + eps)
        // scales the gate and up row sums in the epilogue: no barrier on the prologue's path.
        float ss = has ? hh_sq8(t0, t1) : 0.f;
        for (uint32_t c2 = c + HH_RING_BLOCK; c2 < dm / 8; c2 += HH_RING_BLOCK) ss += hh_sq8(x4[2 * c2], x4[2 * c2 + 1]);
        ss = hh_wave_sum(ss);
        HH_RING_MARK(0, a.wg, 4, tid == 0 && ss != -1.f);                    // x arrived (wave 0)
        HH_RING_MARK(0, a.wg, 5, tid == HH_RING_BLOCK - HH_WAVE && ss != -1.f);  // x arrived (last wave)
        float* red = reinterpret_cast<float*>(stage);  // free until the epilogue
        if (lane == 0) red[wave] = ss;                   // read after the main loop's barrier
        hh_norm8(t0, t1, m0, m1, 1.f);
    }
    if constexpr (TAB16 > 0) {
        if (tid < TAB16) reinterpret_cast<uint4*>(tabs)[tid] = tab;
    }
    hh_x_digits_chunk(t0, t1, c, has, xd);
    for (uint32_t c2 = c + HH_RING_BLOCK; c2 < dm / 8; c2 += HH_RING_BLOCK) {
        float4 v0 = x4[2 * c2], v1 = x4[2 * c2 + 1];  // d_model > 4096: later passes
        if constexpr (NORM) hh_norm8(v0, v1, n4[2 * c2], n4[2 * c2 + 1], 1.f);
        hh_x_digits_chunk(v0, v1, c2, true, xd);
    }
#pragma unroll
    for (int s = P; s < D; s++) issue((uint32_t)s, ring[s]);
    __syncthreads();
    HH_RING_MARK(0, a.wg, 1, tid == 0);  // x's digits in LDS

    {
        typename F::xr_t xr;
        F::load_x(xd, u1, xr);
        auto consume = [&](uint32_t j, const typename F::data& s) {
            const uint32_t i = team1 + j * TPW1;
            if (i < RR) {  // wave-uniform
                float v = F::unit_x(s, lo, xr, tabs);
                if constexpr (LP) {
                    gu[i * TEAM1 + lane1] = act1 ? v : 0.f;  // summed after the loop
                } else {
                    v = hh_wave_sum(act1 ? v : 0.f);
                    if (lane == 0) gu[i * WPT1 + wave % WPT1] = v;
                }
                HH_RING_MARK(0, a.wg, 6, j == 0 && tid == 0 && v != -1.f);  // first item done (wave 0)
            }
        };
        // every round but the last issues the items D ahead; the last issues nothing
        uint32_t j0 = 0;
        for (; j0 + D < n1p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                consume(j0 + (uint32_t)s, ring[s]);
                issue(j0 + (uint32_t)s + D, ring[s]);
            }
        }
#pragma unroll
        for (int s = 0; s < D; s++) consume(j0 + (uint32_t)s, ring[s]);
    }
    __syncthreads();  // row sums (or lane partials) are in LDS
    HH_RING_MARK(0, a.wg, 2, tid == 0);
    if constexpr (LP) {
        // row i = the TEAM1 partials of row read i: 32 threads per row, each adding TEAM1/32
        // consecutive partials, then a 32-lane DPP reduction (fixed order: deterministic)
        constexpr uint32_t PER = TEAM1 / 32;
        for (uint32_t i0 = 0; i0 < RR; i0 += HH_RING_BLOCK / 32) {
            const uint32_t i = i0 + tid / 32, seg = tid % 32;
            float v = 0.f;
            if (i < RR) {
                const float* p = gu + i * TEAM1 + seg * PER;
#pragma unroll
                for (uint32_t k = 0; k < PER; k++) v += p[k];
            }
            v += hh_dpp<0xB1>(v);        // quad_perm [1,0,3,2]
            v += hh_dpp<0x4E>(v);        // quad_perm [2,3,0,1]
            v += hh_dpp<0x124>(v);       // row_ror:4
            v += hh_dpp<0x128>(v);       // row_ror:8 -> each row of 16 holds its sum
            v += hh_dpp<0x142, 0xA>(v);  // row_bcast:15 -> lanes 31 and 63 hold their half's sum
            if (i < RR && seg == 31) rows[i] = v;
        }
        __syncthreads();
    }

    {
        float inv = 1.f;
        if constexpr (NORM) {
            const float* red = reinterpret_cast<const float*>(stage);
            float tot = 0.f;
#pragma unroll
            for (int k = 0; k < HH_RING_CW; k++) tot += red[k];
            inv = 1.0f / sqrtf(tot / (float)dm + a.eps);
        }
        // h = act(g) * u, two int8 digits per element, one scale per granule of 8 rows: one
        // thread per row (every wave), the granule's max by DPP within its 8 lanes
        int8_t* gq1 = reinterpret_cast<int8_t*>(a.hx);
        int8_t* gq2 = gq1 + dff;
        float* gsc = reinterpret_cast<float*>(gq2 + dff);
        for (uint32_t rho0 = 0; rho0 < nrw; rho0 += HH_RING_BLOCK) {
            const uint32_t rho = rho0 + tid;
            const bool ok = rho < nrw;  // granule-aligned: whole 8-lane groups agree
            float hv = 0.f;
            if (ok) {
                float g = 0.f, u = 0.f;
                if constexpr (LP) {
                    g = rows[2 * rho];
                    u = rows[2 * rho + 1];
                } else {
#pragma unroll
                    for (int k = 0; k < WPT1; k++) {
                        g += gu[(2 * rho) * WPT1 + k];
                        u += gu[(2 * rho + 1) * WPT1 + k];
                    }
                }
                if constexpr (NORM) {
                    g *= inv;
                    u *= inv;
                }
                hv = hh_act_mul(g, u, a.act);
            }
            float amax = fabsf(hv);
            amax = fmaxf(amax, hh_dpp<0xB1>(amax));   // quad_perm [1,0,3,2]
            amax = fmaxf(amax, hh_dpp<0x4E>(amax));   // quad_perm [2,3,0,1]
            amax = fmaxf(amax, hh_dpp<0x141>(amax));  // row_half_mirror: the other quad of the 8
            const float scale = amax * (1.0f / 127.0f);
            const float rinv = amax > 0.f ? 127.0f / amax : 0.f;
            const float d1 = fminf(fmaxf(rintf(hv * rinv), -127.f), 127.f);
            const float rr = hv - d1 * scale;
            const float d2 = fminf(fmaxf(rintf(rr * rinv * 256.0f), -127.f), 127.f);
            if (ok) {
                const uint32_t r = row_of(rho);
                gq1[r] = (int8_t)(int)d1;
                gq2[r] = (int8_t)(int)d2;
                if ((lane & 7u) == 0) gsc[r / 8] = scale;
            }
        }
    }
    HH_RING_MARK(0, a.wg, 3, lane == 0);  // the last wave to get here leaves the final stamp
}

// Down: workgroup w owns output rows w, w + G, ... (HH_RING_ILV); a team of WPT2 waves covers
// one row (lane = unit).  A ninth wave copies into LDS by global->LDS DMA, at kernel start, what the
// compute waves read from there (the format's tables, the intermediate unless F::DIRECT_H),
// so neither queues behind the other's requests; lane partials meet in LDS and a 32-lane DPP
// reduction per row writes y (fixed order: deterministic).
#define HH_DN_BLOCK ((HH_RING_CW + 1) * HH_WAVE)
template <class F, int WPT2, int D>
HH_DEV void hh_dn_ring_body(const hh_dnr_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr uint32_t TEAM2 = WPT2 * HH_WAVE, TPW2 = HH_RING_CW / WPT2;
    constexpr bool DIRECT_H = F::DIRECT_H;
    constexpr bool TABLES = F::TAB_BYTES > 0;  // with direct h loads the copy wave brings only these
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff;
#if HH_RING_ILV
    // rows w, w + G, w + 2G, ...
    const uint32_t nrows = (dm - min(w, dm) + G - 1) / G;
    auto drow = [&](uint32_t rl) { return w + rl * G; };
#else
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G);
    const uint32_t q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t nrows = q1 - q0;
    auto drow = [&](uint32_t rl) { return q0 + rl; };
#endif
    const uint32_t n2 = (nrows + TPW2 - 1) / TPW2;
    const uint32_t n2p = (n2 + D - 1) / D * D;
    HH_RING_MARK(1, a.wd, 0, tid == 0);

    // the residual of the first row this thread stores, fetched now rather than on the tail
    float res0 = 0.f;
    if (a.res && tid % 32 == 31 && tid / 32 < nrows) res0 = a.res[drow(tid / 32)];

    // LDS: static: the format's tables; dynamic: [intermediate (unless DIRECT_H)][lane
    // partials: rows x TEAM2]
    char* const tabs = hh_ring_tables_lds<F::TAB_BYTES>();
    char* const lds = hh_smem;
    const uint32_t hbytes = DIRECT_H ? 0u : 2u * dff + (dff / 8u) * 4u;
    int8_t* hq1 = reinterpret_cast<int8_t*>(lds);
    int8_t* hq2 = hq1 + dff;
    float* hsc = reinterpret_cast<float*>(hq2 + dff);
    float* part = reinterpret_cast<float*>(lds + ((hbytes + 15u) & ~15u));

    const uint32_t lane2 = tid % TEAM2, team2 = (wave / WPT2) % TPW2;
    const bool act2 = lane2 < dff / F::UNIT;
    const uint32_t u2 = act2 ? lane2 : 0u;
    const uint8_t* const wdp = a.wd;
    const typename F::lane_t lo = F::lane(u2);
    auto issue = [&](uint32_t k, typename F::data& s) {  // item k: local row team2 + k*TPW2
        const uint32_t rl = team2 + k * TPW2;
        F::issue(wdp + (size_t)drow(rl < nrows ? rl : 0u) * a.rb2, lo, s);  // padding re-reads the first row
    };

    // F::DIRECT_H (Q4_K, IQ): every compute lane loads its own unit's digits of the
    // intermediate straight into registers, ahead of its ring, so a wave starts as soon as its
    // own ~160 bytes per lane arrive (no copy into LDS, no barrier before the loop; 8B down
    // 9.3 -> 9.15 us), the copy wave then bringing only the format's LDS tables (if any).
    // Otherwise (Q6_K: slower that way, its LM-head grids re-read h per
    // workgroup many times) the copy wave brings the intermediate (and the tables) into LDS.
    typename F::data ring[D];
    typename F::hr_t hr;
    if (wave < HH_RING_CW) {
        if constexpr (DIRECT_H) {
            // h's loads, then every ring item's, and only then the arithmetic on h (which
            // waits for h): no ring load is held back behind the intermediate's arrival
            typename F::hraw_t hraw;
            const int8_t* gq1 = reinterpret_cast<const int8_t*>(a.hx);
            F::load_h_raw(gq1, gq1 + dff, reinterpret_cast<const float*>(gq1 + 2 * (size_t)dff), u2, hraw);
#pragma unroll
            for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
            __builtin_amdgcn_sched_barrier(0);
            F::make_h(hraw, u2, hr);
#ifdef HH_RING_TRACE
            if constexpr (__is_same(typename F::hraw_t, hh_hd_raw)) {  // Q4_K's digit form
                const float hchk = __builtin_bit_cast(float, hraw.a[0].x ^ hraw.b[3].w) + hraw.s1.w;
                HH_RING_MARK(1, a.wd, 4, tid == 0 && hchk != -1.f);                     // h arrived (wave 0)
                HH_RING_MARK(1, a.wd, 5, tid == HH_RING_BLOCK - HH_WAVE && hchk != -1.f);  // h arrived (last wave)
            }
#endif
        } else {
#pragma unroll
            for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
        }
    } else {
        // every 16-byte chunk in flight at once (the hardware holds the wave's issue while its
        // count of outstanding loads is full)
        auto dma = [&](const uint8_t* src, char* dst, uint32_t chunks) {
            for (uint32_t c0 = 0; c0 < chunks; c0 += HH_WAVE) {
                if (c0 + lane < chunks)
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void*)(src + (size_t)(c0 + lane) * 16),
                        (__attribute__((address_space(3))) void*)(dst + (size_t)c0 * 16), 16, 0, 0);
            }
        };
        if constexpr (TABLES) dma(reinterpret_cast<const uint8_t*>(F::tables()), tabs, F::TAB_BYTES / 16u);
        if constexpr (!DIRECT_H) dma(a.hx, lds, hbytes / 16u);
        __builtin_amdgcn_s_waitcnt(0);
    }
    // the intermediate (or, with direct h loads, only the tables) is in LDS; the rings stay in flight
    if constexpr (!DIRECT_H || TABLES) __syncthreads();
    HH_RING_MARK(1, a.wd, 1, tid == 0);

    if (wave < HH_RING_CW) {
        if constexpr (!DIRECT_H) F::load_h(hq1, hq2, hsc, u2, hr);
        auto consume = [&](uint32_t k, const typename F::data& s) {
            const uint32_t rl = team2 + k * TPW2;  // local row
            if (rl < nrows) {                      // wave-uniform
                const float v = F::unit_h(s, lo, hr, tabs);
                part[rl * TEAM2 + lane2] = act2 ? v : 0.f;  // reduced after the loop
                HH_RING_MARK(1, a.wd, 6, k == 0 && tid == 0 && v != -1.f);  // first item done (wave 0)
            }
        };
        // every round but the last issues the items D ahead; the last issues nothing
        uint32_t j0 = 0;
        for (; j0 + D < n2p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                consume(j0 + (uint32_t)s, ring[s]);
                issue(j0 + (uint32_t)s + D, ring[s]);
            }
        }
#pragma unroll
        for (int s = 0; s < D; s++) consume(j0 + (uint32_t)s, ring[s]);
    }
    __syncthreads();  // lane partials are in LDS
    HH_RING_MARK(1, a.wd, 2, tid == 0);
    // y[q0 + rl] = sum over the TEAM2 lane partials of row rl: 32 threads per row, each sums
    // TEAM2/32 consecutive partials, then a 32-lane DPP reduction (rows never straddle the
    // 32-lane halves of a wave)
    {
        constexpr uint32_t PER = TEAM2 / 32;
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
            if (rl < nrows && seg == 31) a.y[drow(rl)] = a.res ? (rl0 == 0 ? res0 : a.res[drow(rl)]) + s : s;
        }
    }
    HH_RING_MARK(1, a.wd, 3, lane == 0);
}

// Ring depths (items per wave) of the Q4_K ring kernels.
#ifndef HH_Q4K_GU_RING_D
#define HH_Q4K_GU_RING_D 3
#endif
#ifndef HH_Q4K_DN_RING_D
#define HH_Q4K_DN_RING_D 2
#endif
#ifndef HH_Q4K_GU_RING_P
#define HH_Q4K_GU_RING_P 2  // gate/up ring items issued before x is quantized (1: 689 us per 8B step, 2: 687)
#endif

// The ring kernels (Q4_K here, Q6_K and IQ in their files) take hh_gur_args' / hh_dnr_args'
// fields as separate scalar parameters (the same kernel-argument layout; the host passes the
// struct's bytes), so the code object's kernel-argument preload (build flag) puts the leading
// dwords in SGPRs before the waves start instead of a scalar load at the head of every wave
// (the down kernel 9.65 -> 9.3 us per 8B layer).
// Gate/up packs what its first addresses need into the 14 dwords the preload can hold: five
// pointers, the row bytes, d_model | d_ff << 16 and the grid size (in place of the dispatch's
// own count, which would sit past them); act and eps follow.
#define HH_GUR_PARAMS                                                                             \
    const uint8_t *wg, const uint8_t *wu, const float *x, uint8_t *hx, const float *nw, uint32_t rb1, \
        uint32_t dims, uint32_t grid, int32_t act, float eps
#define HH_GUR_ARGS hh_gur_args{wg, wu, x, hx, nw, rb1, dims & 0xFFFFu, dims >> 16, act, eps, grid}
#define HH_DNR_PARAMS                                                                                 \
    const uint8_t *wd, const uint8_t *hx, float *y, const float *res, uint64_t rb2, uint32_t d_model, uint32_t d_ff
#define HH_DNR_ARGS hh_dnr_args{wd, hx, y, res, rb2, d_model, d_ff}

// _n: with the RMSNorm prologue (the FFN residual block)
#define HH_GU_RING(G1)                                                                          \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_q4k_gu_ring_g##G1(HH_GUR_PARAMS) { \
        hh_gu_ring_body<hh_ring_q4k, G1, HH_Q4K_GU_RING_D, HH_Q4K_GU_RING_P, false>(HH_GUR_ARGS);              \
    }                                                                                           \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_q4k_gu_ring_g##G1##_n(HH_GUR_PARAMS) { \
        hh_gu_ring_body<hh_ring_q4k, G1, HH_Q4K_GU_RING_D, HH_Q4K_GU_RING_P, true>(HH_GUR_ARGS);               \
    }
#define HH_DN_RING(G2)                                                                          \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_q4k_dn_ring_d##G2(HH_DNR_PARAMS) { \
        hh_dn_ring_body<hh_ring_q4k, G2, HH_Q4K_DN_RING_D>(HH_DNR_ARGS);                        \
    }
HH_GU_RING(1)
HH_GU_RING(2)
HH_DN_RING(1)
HH_DN_RING(2)
HH_DN_RING(4)
HH_DN_RING(8)
