// The grouped MoE expert FFN for several tokens in the ring form (gfx950): the rows of all
// selected experts, concatenated in expert order, streamed once per call through a register
// ring, each row dotted with every token routed to its expert.  Same arithmetic and results
// as the grouped kernels of moe_group.hip (the expert loop + combine of
// crates/hayai-core/src/moe_infer.rs:342-455), with the intermediate's digits written by the
// gate/up kernel itself:
//   hh_moe_gu_gring_u<U1>: workgroup w owns 32-row granules [w*NG/G, (w+1)*NG/G) of the
//     concatenated gate/up rows (a granule never straddles experts); it stages the digits of
//     x for the pairs of its experts in LDS, streams its gate and up rows (a wave item is
//     64/U1 row groups x 2 rows, lane = (row group, 64-column unit), one x load serving a
//     lane's 2 rows), keeps every (row, pair) sum in LDS, then writes h = act(g) * u of each
//     pair as per-32 digits (hh_moe_digits layout).
//   hh_moe_dn_gring_u<U2>: the same over the concatenated down rows with each pair's h
//     digits; writes yp[pair][row] (summed per token by hh_moe_combine).
// An expert with more pairs than the LDS holds is handled in passes over pair chunks (its
// rows are streamed once per pass).  Workgroups are independent: no grid-wide exchange.
// (Compiled after moe_group.hip and moe_ring.hip: hh_moeg_args, hh_group_sum.)

struct hh_moegr_args {
    hh_moeg_args g;
    uint32_t ns;    // pairs staged per pass
    uint32_t rmax;  // rows of the largest workgroup share (LDS sums)
};

#define HH_GRING_MAX_SLOTS 64  // experts one workgroup's share can touch

// The share's experts: slot s = es - es_a is expert e[s] with pairs [lo[s], hi[s]) of
// order[]; pair[] holds the current chunk's pair ids.  Kept in LDS: a global load in the
// ring's address computation would make every refill wait for the loads in flight.
#define HH_GRING_MAX_NS 64
struct hh_gring_experts {
    int e[HH_GRING_MAX_SLOTS];
    int lo[HH_GRING_MAX_SLOTS];
    int hi[HH_GRING_MAX_SLOTS];
    int pair[HH_GRING_MAX_NS];
};

// Digits of n elements (U = n / 64 units) staged lane-interleaved, so the lanes of a wave
// read consecutive 16-byte chunks (no LDS bank conflicts): chunk k of unit u (k 0..3: the
// unit's 64 q1 bytes, 4..7: its q2 bytes) at (k * U + u) * 16, then the U float2 scales and
// the U float2 sums as in hh_moe_digits.  src: the hh_moe_digits layout (global).
// np vectors at once (vector qq from src + id[qq] * bytes, id[qq] = pair[qq] / div), every
// chunk's load in flight together.
HH_DEV void hh_gring_stage(char* dst, const uint8_t* src, const int* pair, uint32_t div, uint32_t np, uint32_t n,
                           uint32_t first, uint32_t stride) {
    const uint32_t U = n / 64u, nq = n / 16u;  // q1 chunks (= q2 chunks)
    const uint32_t per = 2u * nq + U, bytes = per * 16u;
    for (uint32_t cg = first; cg < np * per; cg += stride) {
        const uint32_t qq = cg / per, c = cg % per;
        uint32_t d = c;
        if (c < 2u * nq) {
            const uint32_t cc = c < nq ? c : c - nq, u = cc / 4u, k = cc % 4u + (c < nq ? 0u : 4u);
            d = k * U + u;
        }
        const uint32_t id = (uint32_t)pair[qq] / div;
        reinterpret_cast<uint4*>(dst + (size_t)qq * bytes)[d] = reinterpret_cast<const uint4*>(src + (size_t)id * bytes)[c];
    }
}

// hh_q4k_load_lane_x from the interleaved stage.
HH_DEV void hh_gring_load_x(const char* xs, uint32_t U, uint32_t u, hh_q4k_x& xr) {
    const uint4* b = reinterpret_cast<const uint4*>(xs);
    hh_unpack4(b[0 * U + u], xr.q1lo);
    hh_unpack4(b[1 * U + u], xr.q1lo + 4);
    hh_unpack4(b[2 * U + u], xr.q1hi);
    hh_unpack4(b[3 * U + u], xr.q1hi + 4);
    hh_unpack4(b[4 * U + u], xr.q2lo);
    hh_unpack4(b[5 * U + u], xr.q2lo + 4);
    hh_unpack4(b[6 * U + u], xr.q2hi);
    hh_unpack4(b[7 * U + u], xr.q2hi + 4);
    const float2 sc = reinterpret_cast<const float2*>(xs + (size_t)U * 128u)[u];
    const float2 sm = reinterpret_cast<const float2*>(xs + (size_t)U * 136u)[u];
    xr.slo = sc.x * (1.0f / 256.0f);
    xr.shi = sc.y * (1.0f / 256.0f);
    xr.xlo = sm.x;
    xr.xhi = sm.y;
    const uint32_t g = u & 3u;
    const uint32_t kk = 2u * (g & 1u);
    xr.sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    xr.sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    xr.hi_form = g >= 2;
}

// The slot (expert of the share) of local row rl: boundaries between the share's experts are
// (s + 1) * rows_per_expert - off, s < ns_e - 1 (a uniform loop over at most a few).
HH_DEV uint32_t hh_gring_slot(uint32_t rl, uint32_t off, uint32_t per, uint32_t ns_e) {
    uint32_t s = 0;
    while (s + 1 < ns_e && rl + off >= (s + 1) * per) s++;
    return s;
}

#define HH_GRING_M 2  // rows per lane per wave item (one x load serves them)

template <int U1, int D>
HH_DEV void hh_moe_gu_gring_body(const hh_moegr_args& ra) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ hh_gring_experts ex;
    const hh_moeg_args& a = ra.g;
    constexpr uint32_t RPI = HH_WAVE / U1;        // row groups per wave item
    constexpr uint32_t IR = RPI * HH_GRING_M;     // row reads per wave item
    const uint32_t tid = threadIdx.x, lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff, NS = ra.ns, RM = ra.rmax;
    const uint32_t na = (uint32_t)a.elist[a.n_experts];
    const uint32_t NG = na * (dff / 32u);
    const uint32_t r0 = 32u * (uint32_t)(((uint64_t)w * NG) / G);
    const uint32_t r1 = 32u * (uint32_t)(((uint64_t)(w + 1) * NG) / G);
    if (r0 >= r1) return;  // whole workgroup
    const uint32_t RR = 2u * (r1 - r0);
    const uint32_t NI = (RR + IR - 1) / IR;
    const uint32_t n1 = (NI + HH_FFNP_CW - 1) / HH_FFNP_CW;
    const uint32_t n1p = (n1 + D - 1) / D * D;
    const uint32_t es_a = r0 / dff, ns_e = (r1 - 1) / dff - es_a + 1;
    const uint32_t off = r0 - es_a * dff;  // local row 0 is row `off` of the share's first expert
    if (tid < ns_e) {
        const int e = a.elist[es_a + tid];
        ex.e[tid] = e;
        ex.lo[tid] = a.estart[e];
        ex.hi[tid] = a.estart[e + 1];
    }
    __syncthreads();
    const int P_a = ex.lo[0], P_b = ex.hi[ns_e - 1];

    // LDS: [NS pairs' x digits, interleaved][sums: rows x NS x (gate, up)][h: NS x RM]
    const uint32_t xbytes = (uint32_t)hh_digits_bytes_dev(dm), UX = dm / 64u;
    char* xs = hh_smem;
    float* sums = reinterpret_cast<float*>(hh_smem + (size_t)NS * xbytes);
    float* hl = sums + (size_t)RM * NS * 2u;

    const uint32_t rin = lane / U1, u1 = lane % U1;
    const bool act = u1 < UX;
    const uint32_t uu = act ? u1 : 0u;
    const uint32_t oh = (uu >> 2) * 144u, oq = oh + 16u + (uu & 3u) * 32u;
    struct Item {
        hh_q4k_data d[HH_GRING_M];
    };
    auto issue = [&](uint32_t j, Item& it) {
        const uint32_t ib = (wave + j * HH_FFNP_CW) * IR;
        const uint32_t slot = hh_gring_slot(ib >> 1, off, dff, ns_e);
        const uint8_t* ebase = a.experts + (size_t)ex.e[slot] * a.expert_stride;
        const uint32_t lrow0 = off + (ib >> 1) - slot * dff;  // expert-local row of the item's first row
#pragma unroll
        for (int m = 0; m < HH_GRING_M; m++) {
            const uint32_t i = ib + rin + RPI * (uint32_t)m;
            const uint8_t* row = i < RR ? ebase + ((i & 1u) ? a.up_off : a.gate_off) +
                                              (size_t)(lrow0 + ((i - ib) >> 1)) * a.rb_in
                                        : a.experts;  // padding
            it.d[m].h = hh_ld16(row + oh);
            it.d[m].q0 = hh_ld16(row + oq);
            it.d[m].q1 = hh_ld16(row + oq + 16);
        }
    };

    for (int c0 = P_a; c0 < P_b; c0 += (int)NS) {
        const int c1 = min(c0 + (int)NS, P_b);
        // the chunk's pair ids, then their x digits -> LDS (token t = pair / k)
        // the ring's first items go out first (they need only the expert ids), then the
        // chunk's pair ids and their x digits -> LDS (token t = pair / k)
        Item ring[D];
#pragma unroll
        for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
        if (tid < (uint32_t)(c1 - c0)) ex.pair[tid] = a.order[c0 + (int)tid];
        __syncthreads();
        hh_gring_stage(xs, a.xq, ex.pair, a.k, (uint32_t)(c1 - c0), dm, tid, blockDim.x);
        __syncthreads();  // the chunk's digits are in LDS

        for (uint32_t j0 = 0; j0 < n1p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t j = j0 + (uint32_t)s;
                const uint32_t ib = (wave + j * HH_FFNP_CW) * IR;  // the item's first row read
                if (ib < RR) {                                      // wave-uniform
                    // the item's rows lie in one expert (IR / 2 <= 4 rows of a 32-row granule)
                    const uint32_t slot = hh_gring_slot(ib >> 1, off, dff, ns_e);
                    const int qlo = max(ex.lo[slot], c0), qhi = min(ex.hi[slot], c1);
                    for (int q = qlo; q < qhi; q++) {
                        hh_q4k_x xr;
                        hh_gring_load_x(xs + (size_t)(q - c0) * xbytes, UX, uu, xr);
#pragma unroll
                        for (int m = 0; m < HH_GRING_M; m++) {
                            const uint32_t i = ib + rin + RPI * (uint32_t)m;
                            const float v = hh_group_sum<U1>(act ? hh_q4k_unit(ring[s].d[m], xr) : 0.f);
                            if (u1 == U1 - 1 && i < RR) sums[((i >> 1) * NS + (uint32_t)(q - c0)) * 2u + (i & 1u)] = v;
                        }
                    }
                }
                issue(j + D, ring[s]);
            }
        }
        __syncthreads();  // every (row, pair) sum is in LDS

        // h = act(g) * u per (pair, row of its expert)
        for (uint32_t idx = tid; idx < (r1 - r0) * NS; idx += blockDim.x) {
            const uint32_t rl = idx / NS, qq = idx % NS;
            const uint32_t slot = hh_gring_slot(rl, off, dff, ns_e);
            const int q = c0 + (int)qq;
            if (q < c1 && q >= ex.lo[slot] && q < ex.hi[slot])
                hl[qq * RM + rl] = hh_act_mul(sums[(rl * NS + qq) * 2u], sums[(rl * NS + qq) * 2u + 1u], a.act);
        }
        __syncthreads();
        // each pair's rows of this share -> per-32 digits of its intermediate
        const size_t hbytes = hh_digits_bytes_dev(dff);
        for (int q = c0; q < c1; q++) {
            uint32_t slot = 0;
            while (slot + 1 < ns_e && q >= ex.hi[slot]) slot++;
            const uint32_t eb = (es_a + slot) * dff;  // first concatenated row of the expert
            const uint32_t ra0 = max(r0, eb), rb0 = min(r1, eb + dff);
            const uint32_t jr = ra0 - eb;  // first local row (a multiple of 32)
            const hh_digits_ptr hd = hh_moe_digits((char*)a.hq + (size_t)ex.pair[q - c0] * hbytes, dff);
            const hh_digits_ptr dst{hd.q1 + jr, hd.q2 + jr, hd.sc + jr / 32u, hd.sum + jr / 32u};
            hh_quantize_digits(hl + (size_t)(q - c0) * RM + (ra0 - r0), rb0 - ra0, dst);
        }
        __syncthreads();  // LDS is reused by the next chunk
    }
}

template <int U2, int D>
HH_DEV void hh_moe_dn_gring_body(const hh_moegr_args& ra) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ hh_gring_experts ex;
    const hh_moeg_args& a = ra.g;
    constexpr uint32_t RPI = HH_WAVE / U2;     // row groups per wave item
    constexpr uint32_t IR = RPI * HH_GRING_M;  // rows per wave item
    const uint32_t tid = threadIdx.x, lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, dff = a.d_ff, NS = ra.ns;
    const uint32_t na = (uint32_t)a.elist[a.n_experts];
    const uint32_t NG = na * (dm / 8u);  // 8-row granules (never straddle experts)
    const uint32_t r0 = 8u * (uint32_t)(((uint64_t)w * NG) / G);
    const uint32_t r1 = 8u * (uint32_t)(((uint64_t)(w + 1) * NG) / G);
    if (r0 >= r1) return;
    const uint32_t NR = r1 - r0;
    const uint32_t NI = (NR + IR - 1) / IR;
    const uint32_t n2 = (NI + HH_FFNP_CW - 1) / HH_FFNP_CW;
    const uint32_t n2p = (n2 + D - 1) / D * D;
    const uint32_t es_a = r0 / dm, ns_e = (r1 - 1) / dm - es_a + 1;
    const uint32_t off = r0 - es_a * dm;
    if (tid < ns_e) {
        const int e = a.elist[es_a + tid];
        ex.e[tid] = e;
        ex.lo[tid] = a.estart[e];
        ex.hi[tid] = a.estart[e + 1];
    }
    __syncthreads();
    const int P_a = ex.lo[0], P_b = ex.hi[ns_e - 1];

    const uint32_t hbytes = (uint32_t)hh_digits_bytes_dev(dff), UH = dff / 64u;
    char* hs = hh_smem;  // [NS pairs' h digits, interleaved]
    const uint32_t rin = lane / U2, u2 = lane % U2;
    const bool act = u2 < UH;
    const uint32_t uu = act ? u2 : 0u;
    const uint32_t oh = (uu >> 2) * 144u, oq = oh + 16u + (uu & 3u) * 32u;
    struct Item {
        hh_q4k_data d[HH_GRING_M];
    };
    auto issue = [&](uint32_t j, Item& it) {
        const uint32_t ib = (wave + j * HH_FFNP_CW) * IR;
        const uint32_t slot = hh_gring_slot(ib, off, dm, ns_e);
        const uint8_t* ebase = a.experts + (size_t)ex.e[slot] * a.expert_stride + a.down_off;
        const uint32_t lrow0 = off + ib - slot * dm;
#pragma unroll
        for (int m = 0; m < HH_GRING_M; m++) {
            const uint32_t i = ib + rin + RPI * (uint32_t)m;
            const uint8_t* row = i < NR ? ebase + (size_t)(lrow0 + (i - ib)) * a.rb_ff : a.experts;
            it.d[m].h = hh_ld16(row + oh);
            it.d[m].q0 = hh_ld16(row + oq);
            it.d[m].q1 = hh_ld16(row + oq + 16);
        }
    };

    for (int c0 = P_a; c0 < P_b; c0 += (int)NS) {
        const int c1 = min(c0 + (int)NS, P_b);
        Item ring[D];
#pragma unroll
        for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
        if (tid < (uint32_t)(c1 - c0)) ex.pair[tid] = a.order[c0 + (int)tid];
        __syncthreads();
        hh_gring_stage(hs, a.hq, ex.pair, 1u, (uint32_t)(c1 - c0), dff, tid, blockDim.x);
        __syncthreads();  // the chunk's h digits are in LDS

        for (uint32_t j0 = 0; j0 < n2p; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t j = j0 + (uint32_t)s;
                const uint32_t ib = (wave + j * HH_FFNP_CW) * IR;
                if (ib < NR) {  // wave-uniform; the item's rows lie in one 8-row granule
                    const uint32_t slot = hh_gring_slot(ib, off, dm, ns_e);
                    const int qlo = max(ex.lo[slot], c0), qhi = min(ex.hi[slot], c1);
                    const uint32_t lrow0 = off + ib - slot * dm;
                    for (int q = qlo; q < qhi; q++) {
                        hh_q4k_x hr;
                        hh_gring_load_x(hs + (size_t)(q - c0) * hbytes, UH, uu, hr);
                        float* yq = a.yp + (size_t)ex.pair[q - c0] * dm + lrow0;
#pragma unroll
                        for (int m = 0; m < HH_GRING_M; m++) {
                            const uint32_t i = ib + rin + RPI * (uint32_t)m;
                            const float v = hh_group_sum<U2>(act ? hh_q4k_unit(ring[s].d[m], hr) : 0.f);
                            if (u2 == U2 - 1 && i < NR) yq[i - ib] = v;
                        }
                    }
                }
                issue(j + D, ring[s]);
            }
        }
        __syncthreads();  // LDS is reused by the next chunk
    }
}

#define HH_MOE_GRING(U)                                                                                   \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_moe_gu_gring_u##U(const hh_moegr_args a) { \
        hh_moe_gu_gring_body<U, 3>(a);                                                                    \
    }                                                                                                     \
    extern "C" __global__ void __launch_bounds__(HH_RING_BLOCK) hh_moe_dn_gring_u##U(const hh_moegr_args a) { \
        hh_moe_dn_gring_body<U, 3>(a);                                                                    \
    }
HH_MOE_GRING(16)
HH_MOE_GRING(32)
HH_MOE_GRING(64)
