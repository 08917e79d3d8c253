// Team GEMV and fused gate/up(+SwiGLU) kernels for gfx950.
//
// Work decomposition (replaces ggml_gemv_* of crates/hayai-kernels/kernels/ggml_gemv_q4.cl,
// which ran one work-item per row, or 32 lanes per row with a serial LDS reduce):
//   - A TEAM of lanes (16..1024, a sub-wave, a wave or a whole workgroup) owns one output
//     row at a time.  Lane l owns units l, l+TEAM, ... (UPL units) of every row and keeps
//     their x slice in registers for the kernel's lifetime.
//   - Teams walk rows grid-stride, R rows per step, issuing all R rows' unit loads before
//     any math so each lane has R independent 16-byte loads in flight.
//   - Consecutive lanes own consecutive units, so a wave's loads of one row cover one
//     contiguous byte range of the packed tensor (coalesced; every byte fetched once).
//   - The team sum is a butterfly over lanes (every lane ends with the total), plus one LDS
//     step across waves when TEAM > 64.  Lane r stores row r of the step: plain stores,
//     deterministic order, no atomics.
#include "quant.h"

template <class Q>
HH_DEV void hh_stage_tables(hh_tables* t) {
    if constexpr (Q::TABLES) {
        for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
            t->g2[i] = hh_iq2xxs_grid[i];
            t->g3[i] = hh_iq3xxs_grid[i];
        }
        __syncthreads();
    }
}

// Reduce R per-lane partials over the team; afterwards every lane of the team holds all R
// totals.  TEAM <= 64: butterfly.  TEAM > 64: butterfly per wave, per-wave sums through
// LDS, then every lane adds them up (broadcast LDS reads, same order in every lane).
template <int TEAM, int R>
HH_DEV void hh_team_reduce(float (&acc)[R], float* red) {
    if constexpr (TEAM <= HH_WAVE) {
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = hh_team_sum<TEAM>(acc[r]);
    } else {
        constexpr int NW = TEAM / HH_WAVE;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = hh_team_sum<HH_WAVE>(acc[r]);
        const uint32_t wave = threadIdx.x / HH_WAVE, lane = threadIdx.x % HH_WAVE;
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) red[wave * R + r] = acc[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) s += red[w * R + r];
            acc[r] = s;
        }
        __syncthreads();  // red is rewritten by the next step
    }
}

template <int R>
HH_DEV float hh_pick(const float (&acc)[R], uint32_t i) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; r++)
        if ((uint32_t)r == i) v = acc[r];
    return v;
}

// Teams of up to one wave share a 256-thread workgroup (no barriers in their row loop).
// A team wider than a wave IS the workgroup: its reduction uses workgroup barriers and a
// per-wave LDS slot array, so no other team may live in the same workgroup.
template <int TEAM>
struct hh_geom {
    static constexpr int BLOCK = TEAM > HH_WAVE ? TEAM : 256;
    static constexpr int TPB = BLOCK / TEAM;  // teams per workgroup
    static_assert(TEAM <= HH_WAVE || TPB == 1, "multi-wave teams own their workgroup");
};

template <class Q, int TEAM, int UPL, int R>
HH_DEV void hh_gemv_body(const hh_gemv_args& a) {
    using G = hh_geom<TEAM>;
    __shared__ hh_tables tabs;
    __shared__ float red[(TEAM > HH_WAVE ? TEAM / HH_WAVE : 1) * R];
    hh_stage_tables<Q>(&tabs);

    const uint32_t lane = threadIdx.x % TEAM;
    const uint32_t team = blockIdx.x * G::TPB + threadIdx.x / TEAM;
    const uint32_t nteams = gridDim.x * G::TPB;
    const uint32_t P = a.n / Q::UNIT;

    typename Q::X xr[UPL];
    bool act[UPL];
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        const uint32_t u = lane + k * TEAM;
        act[k] = u < P;
        if (act[k]) Q::load_x(a.x, u, xr[k]);
    }

    for (uint32_t row0 = team * R; row0 < a.m; row0 += nteams * R) {
        typename Q::Data dat[UPL][R];
#pragma unroll
        for (int k = 0; k < UPL; k++)
#pragma unroll
            for (int r = 0; r < R; r++)
                if (act[k] && row0 + r < a.m)
                    dat[k][r] = Q::load(a.w + (size_t)(row0 + r) * a.row_bytes, lane + k * TEAM);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
        for (int k = 0; k < UPL; k++)
#pragma unroll
            for (int r = 0; r < R; r++)
                if (act[k] && row0 + r < a.m) acc[r] += Q::dot(dat[k][r], xr[k], lane + k * TEAM, &tabs);
        hh_team_reduce<TEAM, R>(acc, red);
        if (lane < (uint32_t)R && row0 + lane < a.m) a.y[row0 + lane] = hh_pick<R>(acc, lane);
    }
}

template <class Q, int TEAM, int UPL, int R>
HH_DEV void hh_gateup_body(const hh_gateup_args& a) {
    using G = hh_geom<TEAM>;
    __shared__ hh_tables tabs;
    __shared__ float red[(TEAM > HH_WAVE ? TEAM / HH_WAVE : 1) * 2 * R];
    hh_stage_tables<Q>(&tabs);

    const uint32_t lane = threadIdx.x % TEAM;
    const uint32_t team = blockIdx.x * G::TPB + threadIdx.x / TEAM;
    const uint32_t nteams = gridDim.x * G::TPB;
    const uint32_t P = a.n / Q::UNIT;

    typename Q::X xr[UPL];
    bool act[UPL];
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        const uint32_t u = lane + k * TEAM;
        act[k] = u < P;
        if (act[k]) Q::load_x(a.x, u, xr[k]);
    }

    for (uint32_t row0 = team * R; row0 < a.m; row0 += nteams * R) {
        typename Q::Data dg[UPL][R], du[UPL][R];
#pragma unroll
        for (int k = 0; k < UPL; k++)
#pragma unroll
            for (int r = 0; r < R; r++)
                if (act[k] && row0 + r < a.m) {
                    const size_t off = (size_t)(row0 + r) * a.row_bytes;
                    dg[k][r] = Q::load(a.wg + off, lane + k * TEAM);
                    du[k][r] = Q::load(a.wu + off, lane + k * TEAM);
                }
        float acc[2 * R];
#pragma unroll
        for (int r = 0; r < 2 * R; r++) acc[r] = 0.f;
#pragma unroll
        for (int k = 0; k < UPL; k++)
#pragma unroll
            for (int r = 0; r < R; r++)
                if (act[k] && row0 + r < a.m) {
                    acc[r] += Q::dot(dg[k][r], xr[k], lane + k * TEAM, &tabs);
                    acc[R + r] += Q::dot(du[k][r], xr[k], lane + k * TEAM, &tabs);
                }
        hh_team_reduce<TEAM, 2 * R>(acc, red);
        if (lane < (uint32_t)R && row0 + lane < a.m) {
            const float g = hh_pick<2 * R>(acc, lane);
            const float u = hh_pick<2 * R>(acc, R + lane);
            a.h[row0 + lane] = hh_act_mul(g, u, a.act);
        }
    }
}

// Instantiations: kernel names are hh_gemv_<fmt>_t<TEAM>_u<UPL> and
// hh_gateup_<fmt>_t<TEAM>_u<UPL>; the host picks the smallest TEAM*UPL covering the row's
// unit count.  R (rows per step) is 4 for a plain GEMV and 2 for gate/up (4 rows' loads),
// halved when a lane owns two units.  Teams stop at 512 lanes: a 1024-thread workgroup
// caps a lane at 128 VGPRs, which spills the x slice.
#define HH_GEMV_KERNEL(NAME, Q, TEAM, UPL)                                              \
    extern "C" __global__ void __launch_bounds__(hh_geom<TEAM>::BLOCK)                 \
        hh_gemv_##NAME##_t##TEAM##_u##UPL(const hh_gemv_args a) {                       \
        hh_gemv_body<Q, TEAM, UPL, (UPL == 1 ? 4 : 2)>(a);                              \
    }
#define HH_GATEUP_KERNEL(NAME, Q, TEAM, UPL)                                            \
    extern "C" __global__ void __launch_bounds__(hh_geom<TEAM>::BLOCK)                 \
        hh_gateup_##NAME##_t##TEAM##_u##UPL(const hh_gateup_args a) {                   \
        hh_gateup_body<Q, TEAM, UPL, (UPL == 1 ? 2 : 1)>(a);                            \
    }
#define HH_TEAMS(X, NAME, Q)                                                            \
    X(NAME, Q, 16, 1)                                                                   \
    X(NAME, Q, 32, 1)                                                                   \
    X(NAME, Q, 64, 1)                                                                   \
    X(NAME, Q, 128, 1)                                                                  \
    X(NAME, Q, 256, 1)                                                                  \
    X(NAME, Q, 512, 1)                                                                  \
    X(NAME, Q, 512, 2)

HH_TEAMS(HH_GEMV_KERNEL, q4_k, QK4<true>)
HH_TEAMS(HH_GEMV_KERNEL, q4_k_unaligned, QK4<false>)
HH_TEAMS(HH_GEMV_KERNEL, q4_0, Q40)
HH_TEAMS(HH_GEMV_KERNEL, iq2_xxs, QI2)
HH_TEAMS(HH_GEMV_KERNEL, iq3_xxs, QI3)
HH_TEAMS(HH_GEMV_KERNEL, q8_0, Q80)
HH_TEAMS(HH_GEMV_KERNEL, q6_k, QK6)
HH_TEAMS(HH_GEMV_KERNEL, f32, QF32)
HH_TEAMS(HH_GEMV_KERNEL, f16, QF16)

HH_TEAMS(HH_GATEUP_KERNEL, q4_k, QK4<true>)
HH_TEAMS(HH_GATEUP_KERNEL, q4_k_unaligned, QK4<false>)
HH_TEAMS(HH_GATEUP_KERNEL, q4_0, Q40)
HH_TEAMS(HH_GATEUP_KERNEL, iq2_xxs, QI2)
HH_TEAMS(HH_GATEUP_KERNEL, iq3_xxs, QI3)
HH_TEAMS(HH_GATEUP_KERNEL, q8_0, Q80)
HH_TEAMS(HH_GATEUP_KERNEL, q6_k, QK6)

// Element-wise act(g) * u, for FFNs whose gate and up formats differ (unfused path).
extern "C" __global__ void __launch_bounds__(256) hh_act_mul_kernel(const hh_act_args a) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.h[i] = hh_act_mul(a.g[i], a.u[i], a.act);
}

// Scalar-column GEMV for F32/F16 rows whose width is not a multiple of 32 or whose start
// is not 16-byte aligned: one wave per row, lanes stride the columns.
template <int FMT>
HH_DEV void hh_gemv_plain_body(const hh_gemv_args& a) {
    const uint32_t lane = threadIdx.x % HH_WAVE;
    const uint32_t wave = blockIdx.x * 4 + threadIdx.x / HH_WAVE;
    const uint32_t nw = gridDim.x * 4;
    for (uint32_t row = wave; row < a.m; row += nw) {
        const uint8_t* p = a.w + (size_t)row * a.row_bytes;
        float s = 0.f;
        for (uint32_t c = lane; c < a.n; c += HH_WAVE) {
            float w;
            if (FMT == HH_TYPE_F32) {
                uint32_t b;
                __builtin_memcpy(&b, p + 4 * (size_t)c, 4);
                w = __uint_as_float(b);
            } else {
                w = hh_f16(hh_ld_u16(p + 2 * (size_t)c));
            }
            s = fmaf(w, a.x[c], s);
        }
        s = hh_team_sum<HH_WAVE>(s);
        if (lane == 0) a.y[row] = s;
    }
}
extern "C" __global__ void __launch_bounds__(256) hh_gemv_f32_plain(const hh_gemv_args a) {
    hh_gemv_plain_body<HH_TYPE_F32>(a);
}
extern "C" __global__ void __launch_bounds__(256) hh_gemv_f16_plain(const hh_gemv_args a) {
    hh_gemv_plain_body<HH_TYPE_F16>(a);
}
