// The MoE expert FFN of one token (decode) as two streaming launches (gfx950):
//   y = sum_s w_s * down_{e_s}(act(gate_{e_s} x) * up_{e_s} x)
// (the expert loop and combine of crates/hayai-core/src/moe_infer.rs:342-455, routed by
// route_experts :852-934).  With the routing weight folded into the intermediate,
// h'_s = w_s * act(g_s) * u_s, this is one FFN whose gate/up rows are the k selected
// experts' rows and whose down rows are the concatenation of their down rows:
// y[j] = sum over the k*d_ff columns of [down_{e_0}[j,:] | down_{e_1}[j,:] | ...] . h'.
//   hh_moe_gu_ring_u<U1>: every workgroup routes the token (one wave selects, one sums the
//     softmax, the others turn x into per-32 digits meanwhile), then streams its share of
//     the k*d_ff gathered rows of gate and up with the ring of q4k_ring.hip (64/U1 rows per
//     wave item, lane = (row, unit)), applies the activation and the weight, and writes h'
//     as granule digits.
//   hh_moe_dn_ring_d<W2>: as hh_q4k_dn_ring over the concatenated columns: a lane's unit
//     lies in slot s = unit / (d_ff/64), so its base address is expert e_s's down matrix.
// An empty slot (id -1) contributes zero and reads expert 0's bytes.  (Compiled after
// moe.hip and q4k_ring.hip in the same translation unit.)

struct hh_moe_ring_args {
    hh_moe_args m;  // experts, offsets, row bytes, ids/wts, x, y, shapes, act, routing
    uint8_t* hx;    // h' digits: q1[k*d_ff] | q2[k*d_ff] | scale[k*d_ff/8] f32
};

// Sum over the U lanes of each U-lane group of a wave (U = 16, 32 or 64), fixed order; the
// group's sum lands in its last lane.
template <int U>
HH_DEV float hh_group_sum(float s) {
    s += hh_dpp<0xB1>(s);   // quad_perm [1,0,3,2]
    s += hh_dpp<0x4E>(s);   // quad_perm [2,3,0,1]
    s += hh_dpp<0x124>(s);  // row_ror:4
    s += hh_dpp<0x128>(s);  // row_ror:8 -> every lane of a row of 16 holds the row's sum
    if (U >= 32) s += hh_dpp<0x142, 0xA>(s);  // row_bcast:15 -> lanes 31, 63: 32-lane sums
    if (U >= 64) s += hh_dpp<0x143, 0xC>(s);  // row_bcast:31 -> lane 63: the wave's sum
    return s;
}

template <int U1, int D>
HH_DEV void hh_moe_gu_ring_body(const hh_moe_ring_args& ra) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ __attribute__((aligned(16))) hh_route_lds rl;
    __shared__ int s_ids[64];
    __shared__ float s_w[64];
    const hh_moe_args& a = ra.m;
    constexpr uint32_t RPI = HH_WAVE / U1;  // row reads per wave item
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff, k = a.k;
    const uint32_t R = k * dff;  // gathered rows (of gate, and of up)
    const uint32_t NG = R / 8;
    const uint32_t r0 = 8u * (uint32_t)(((uint64_t)w * NG) / G);
    const uint32_t r1 = 8u * (uint32_t)(((uint64_t)(w + 1) * NG) / G);
    const uint32_t RR = 2u * (r1 - r0);  // row reads: (gate, up) of each row
    const uint32_t NI = (RR + RPI - 1) / RPI;
    const uint32_t n1 = (NI + HH_RING_CW - 1) / HH_RING_CW;
    const uint32_t n1p = (n1 + D - 1) / D * D;

    // LDS: [x digits][gate/up row sums][staging 128 B]
    const uint32_t xbytes = 2u * dm + (dm / 32u) * 8u;
    hh_digits_ptr xd;
    xd.q1 = reinterpret_cast<int8_t*>(hh_smem);
    xd.q2 = xd.q1 + dm;
    xd.sc = reinterpret_cast<float*>(xd.q2 + dm);
    xd.sum = xd.sc + dm / 32;
    float* gu = reinterpret_cast<float*>(hh_smem + ((xbytes + 15u) & ~15u));  // [RR]
    uint8_t* stage = reinterpret_cast<uint8_t*>(gu + ((RR + 3u) & ~3u));

    // routing: the last wave selects the experts, the one before it sums the softmax over all
    // experts meanwhile (the weights follow once both are done), the others quantize x
    __shared__ float rex[HH_MOE_MAX_E];
    __shared__ int s_sel[64];
    __shared__ float s_inv;
    __shared__ uint32_t s_kk;
    constexpr uint32_t XT = (HH_RING_CW - 2) * HH_WAVE;
    if (wave == HH_RING_CW - 1) {
        if (a.route) {
            int sel;
            const uint32_t kk = hh_route_select(a.r, 0, true, rl, &sel);
            if (lane < k) {
                s_sel[lane] = lane < kk ? sel : 0;
                s_ids[lane] = lane < kk ? hh_moe_valid(a, sel) : -1;
            }
            if (lane == 0) s_kk = kk;
        } else if (lane < k) {
            s_ids[lane] = hh_moe_valid(a, a.ids[lane]);
            s_w[lane] = a.wts[lane];
        }
    } else if (wave == HH_RING_CW - 2) {
        if (a.route && a.r.gating != 1) {
            const float inv = hh_route_softmax(a.r, 0, true, rex);
            if (lane == 0) s_inv = inv;
        }
    } else {
        hh_quantize_digits(a.x, dm, xd, tid, XT);
    }
    __syncthreads();  // expert ids and x digits are in LDS

    // lane roles: row read i = (wave + 8 * item) * RPI + rin; unit u1 of the row
    const uint32_t rin = lane / U1, u1 = lane % U1;
    const uint32_t oh = (u1 >> 2) * 144u, oq = oh + 16u + (u1 & 3u) * 32u;
    auto issue = [&](uint32_t j, hh_q4k_data& s) {
        const uint32_t i = (wave + j * HH_RING_CW) * RPI + rin;
        const uint8_t* row = a.experts;  // padding, rows past the share, empty slots: expert 0's bytes
        if (i < RR) {
            const uint32_t r = r0 + (i >> 1), slot = r / dff;
            const int e = s_ids[slot];
            if (e >= 0)
                row = a.experts + (size_t)e * a.expert_stride + ((i & 1u) ? a.up_off : a.gate_off) +
                      (size_t)(r - slot * dff) * a.rb_in;
        }
        s.h = hh_ld16(row + oh);
        s.q0 = hh_ld16(row + oq);
        s.q1 = hh_ld16(row + oq + 16);
    };
    hh_q4k_data ring[D];
#pragma unroll
    for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
    {
        hh_q4k_x xr;
        hh_q4k_load_lane_x(xd, u1, xr);
        for (uint32_t j0 = 0; j0 < n1p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t j = j0 + (uint32_t)s;
                const uint32_t ib = (wave + j * HH_RING_CW) * RPI;  // first row read of the item
                if (ib < RR) {                                       // wave-uniform
                    const float v = hh_group_sum<U1>(hh_q4k_unit(ring[s], xr));
                    const uint32_t i = ib + rin;
                    if (u1 == U1 - 1 && i < RR) gu[i] = v;
                }
                issue(j + D, ring[s]);
            }
        }
    }
    __syncthreads();  // row sums are in LDS

    if (wave == 0) {
        if (a.route) {  // the slot weights (lane r: slot r); workgroup 0 publishes ids and weights
            const uint32_t kk = s_kk;
            const float wv = hh_route_weight(a.r, rl.sc, rex, s_inv, s_sel[lane < k ? lane : 0], kk);
            if (lane < k) {
                s_w[lane] = lane < kk ? wv : 0.f;
                if (w == 0) {
                    a.ids[lane] = lane < kk ? s_sel[lane] : -1;
                    a.wts[lane] = lane < kk ? wv : 0.f;
                }
            }
            hh_wave_sync();
        }
        // h' = w_s * act(g) * u, two int8 digits per element, one scale per granule of 8
        // (granules never straddle slots: d_ff is a multiple of 8)
        int8_t* gq1 = reinterpret_cast<int8_t*>(ra.hx);
        int8_t* gq2 = gq1 + R;
        float* gsc = reinterpret_cast<float*>(gq2 + R);
        for (uint32_t rho0 = 0; rho0 < r1 - r0; rho0 += HH_WAVE) {
            const uint32_t rho = rho0 + lane;
            const bool ok = rho < r1 - r0;
            float hv = 0.f;
            if (ok) {
                const uint32_t slot = (r0 + rho) / dff;
                if (s_ids[slot] >= 0) hv = s_w[slot] * hh_act_mul(gu[2 * rho], gu[2 * rho + 1], a.act);
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
                const uint32_t r = r0 + rho;
                *reinterpret_cast<uint64_t*>(gq1 + r) = *reinterpret_cast<const uint64_t*>(stage + lane);
                *reinterpret_cast<uint64_t*>(gq2 + r) = *reinterpret_cast<const uint64_t*>(stage + 64 + lane);
                gsc[r / 8] = scale;
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

template <int WPT2, int D>
HH_DEV void hh_moe_dn_ring_body(const hh_moe_ring_args& ra) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ int s_ids[64];
    const hh_moe_args& a = ra.m;
    constexpr uint32_t TEAM2 = WPT2 * HH_WAVE, TPW2 = HH_RING_CW / WPT2;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff, k = a.k;
    const uint32_t K = k * dff;  // concatenated columns
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G);
    const uint32_t q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t n2 = (q1 - q0 + TPW2 - 1) / TPW2;
    const uint32_t n2p = (n2 + D - 1) / D * D;

    // LDS: [h' digits][lane partials: rows x TEAM2]
    const uint32_t hbytes = 2u * K + (K / 8u) * 4u;
    int8_t* hq1 = reinterpret_cast<int8_t*>(hh_smem);
    int8_t* hq2 = hq1 + K;
    float* hsc = reinterpret_cast<float*>(hq2 + K);
    float* part = reinterpret_cast<float*>(hh_smem + ((hbytes + 15u) & ~15u));

    if (tid < k) s_ids[tid] = hh_moe_valid(a, a.ids[tid]);
    __syncthreads();
    const uint32_t lane2 = tid % TEAM2, team2 = (wave / WPT2) % TPW2;
    const uint32_t ue = dff / 64;  // units per slot
    const bool act2 = lane2 < K / 64;
    const uint32_t u2 = act2 ? lane2 : 0u;
    const uint32_t slot = u2 / ue, lu = u2 - slot * ue;
    const int e = s_ids[slot];
    const uint8_t* base = a.experts + (size_t)(e >= 0 ? e : 0) * a.expert_stride + a.down_off;
    const uint32_t oh = (lu >> 2) * 144u, oq = oh + 16u + (lu & 3u) * 32u;
    auto issue = [&](uint32_t kk, hh_q4k_data& s) {  // item kk: row team2 + kk*TPW2
        const uint32_t r = q0 + team2 + kk * TPW2;
        const uint8_t* row = base + (size_t)(r < q1 ? r : q0) * a.rb_ff;
        s.h = hh_ld16(row + oh);
        s.q0 = hh_ld16(row + oq);
        s.q1 = hh_ld16(row + oq + 16);
    };

    // every compute lane loads its own unit's digits of h' from global memory, ahead of its
    // ring, and starts as soon as they arrive (no copy into LDS, no barrier before the loop)
    hh_q4k_data ring[D];
    hh_hd hr;
    if (wave < HH_RING_CW) {
        const int8_t* g1 = reinterpret_cast<const int8_t*>(ra.hx);
        hh_hd_load(g1, g1 + K, reinterpret_cast<const float*>(g1 + 2 * (size_t)K), u2, hr);  // (lu & 3 = u2 & 3)
#pragma unroll
        for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
    }

    if (wave < HH_RING_CW) {
        for (uint32_t j0 = 0; j0 < n2p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t kk = j0 + (uint32_t)s;
                const uint32_t rl = team2 + kk * TPW2;
                if (q0 + rl < q1) {
                    const float v = hh_q4k_unit_h(ring[s], hr);
                    part[rl * TEAM2 + lane2] = act2 ? v : 0.f;
                }
                issue(kk + D, ring[s]);
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
            s = hh_group_sum<32>(s);
            if (rl < nrows && seg == 31) a.y[q0 + rl] = s;
        }
    }
}

#define HH_MOE_GU_RING(U)                                                                               \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_moe_gu_ring_u##U(const hh_moe_ring_args a) { \
        hh_moe_gu_ring_body<U, 3>(a);                                                                   \
    }
#define HH_MOE_DN_RING(W2)                                                                              \
    extern "C" __global__ void __launch_bounds__(HH_DN_BLOCK) hh_moe_dn_ring_d##W2(const hh_moe_ring_args a) { \
        hh_moe_dn_ring_body<W2, 3>(a);                                                                  \
    }
HH_MOE_GU_RING(16)
HH_MOE_GU_RING(32)
HH_MOE_GU_RING(64)
HH_MOE_DN_RING(1)
HH_MOE_DN_RING(2)
HH_MOE_DN_RING(4)
HH_MOE_DN_RING(8)
