// Q4_K GEMV and fused gate/up(+act) kernels for gfx950: the FFN hot path at batch 1.
//
// Layout and arithmetic:
//   - Workgroup = 8 waves.  A team of WPT waves (64*WPT lanes) owns one output row at a
//     time; lane l owns "unit" l of the row: Q4_K group g = l & 3 of superblock l >> 2, i.e.
//     qs[32g, 32g+32) (low nibbles = sub-block 2g, high nibbles = sub-block 2g+1) plus the
//     16-byte block header (d, dmin, scales[12]); crates/hayai-model/src/q4k.rs:178-203.
//   - x never leaves the chip after the prologue: the workgroup turns x into two int8 digits
//     per element, x ~= s * (q1 + q2/256) with s = amax/127 per 32-element sub-block (error
//     <= s/512), stored in LDS with the per-sub-block scale and exact f32 sum.  Each lane then
//     holds its unit's 64 x 2 digits in 32 VGPRs.
//   - Per weight dword (8 nibbles): one AND (low nibbles), shift+AND (high nibbles) and four
//     v_dot4_i32_i8 (nibbles x digit 1, nibbles x digit 2, for both sub-blocks) -- integer
//     sums, exact.  Per (row, group): the sub-block sums are scaled once in f32:
//       d*sc*s*(sum1 + sum2/256) - dmin*m*sum(x)     (factored form of (d*sc)*q - dmin*m)
//   - Loads are double-buffered in registers: row step k+1's 16-byte loads are in flight
//     while step k is computed.  Consecutive lanes read consecutive 32-byte qs chunks, so
//     each wave reads whole rows front to back.
//   - Team sums: DPP butterfly/broadcast within the wave (v_add_f32_dpp, row_bcast15/31),
//     then an LDS step across the team's waves when WPT > 1.
//   - Each workgroup owns a contiguous row range; row steps are uniform across the
//     workgroup (barriers in the multi-wave reduction stay convergent).
#include "quant.h"

#define HH_Q4K_WAVES 8
#define HH_Q4K_BLOCK (HH_Q4K_WAVES * HH_WAVE)

struct hh_q4k_args {
    const uint8_t* w0;  // the matrix (GEMV) or W_gate (gate/up)
    const uint8_t* w1;  // W_up (gate/up only)
    const float* x;     // n floats, 16-byte aligned
    float* y;           // m floats (y, or h for gate/up)
    uint32_t m;
    uint32_t n;
    uint64_t row_bytes;
    int32_t act;
    int32_t pad;
};

template <int CTRL, int ROW_MASK = 0xF>
HH_DEV float hh_dpp(float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, true));
}

// Sum over the 64 lanes of a wave; the total is returned to every lane (wave-uniform).
HH_DEV float hh_wave_sum(float v) {
    v += hh_dpp<0xB1>(v);        // quad_perm [1,0,3,2]
    v += hh_dpp<0x4E>(v);        // quad_perm [2,3,0,1]
    v += hh_dpp<0x124>(v);       // row_ror:4
    v += hh_dpp<0x128>(v);       // row_ror:8  -> each row of 16 holds its row sum
    v += hh_dpp<0x142, 0xA>(v);  // row_bcast:15 -> rows 1,3 add rows 0,2
    v += hh_dpp<0x143, 0xC>(v);  // row_bcast:31 -> rows 2,3 add row 1: lane 63 = total
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// LDS layout (dynamic): q1[n] int8 | q2[n] int8 | scale[n/32] f32 | sum[n/32] f32 | red[]
struct hh_xdig {
    const int8_t* q1;
    const int8_t* q2;
    const float* sc;
    const float* sum;
    float* red;
};

// Prologue: x -> digits in LDS, one 32-element sub-block per thread.
HH_DEV hh_xdig hh_q4k_stage_x(const float* __restrict__ x, uint32_t n, char* smem) {
    int8_t* q1 = reinterpret_cast<int8_t*>(smem);
    int8_t* q2 = q1 + n;
    float* sc = reinterpret_cast<float*>(q2 + n);
    float* sm = sc + n / 32;
    for (uint32_t sb = threadIdx.x; sb < n / 32; sb += HH_Q4K_BLOCK) {
        const float4* p = reinterpret_cast<const float4*>(x + (size_t)sb * 32);
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 t = p[i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
        float amax = 0.f, s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            amax = fmaxf(amax, fabsf(v[i]));
            s += v[i];
        }
        const float scale = amax * (1.0f / 127.0f);
        const float inv = amax > 0.f ? 127.0f / amax : 0.f;
        uint32_t d1[8], d2[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t p1 = 0, p2 = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float xv = v[4 * i + k];
                const float a = fminf(fmaxf(rintf(xv * inv), -127.f), 127.f);
                const float r = xv - a * scale;
                const float b = fminf(fmaxf(rintf(r * inv * 256.0f), -127.f), 127.f);
                p1 |= ((uint32_t)(int)a & 0xFFu) << (8 * k);
                p2 |= ((uint32_t)(int)b & 0xFFu) << (8 * k);
            }
            d1[i] = p1;
            d2[i] = p2;
        }
        uint4* o1 = reinterpret_cast<uint4*>(q1 + (size_t)sb * 32);
        uint4* o2 = reinterpret_cast<uint4*>(q2 + (size_t)sb * 32);
        o1[0] = make_uint4(d1[0], d1[1], d1[2], d1[3]);
        o1[1] = make_uint4(d1[4], d1[5], d1[6], d1[7]);
        o2[0] = make_uint4(d2[0], d2[1], d2[2], d2[3]);
        o2[1] = make_uint4(d2[4], d2[5], d2[6], d2[7]);
        sc[sb] = scale;
        sm[sb] = s;
    }
    hh_xdig xd{q1, q2, sc, sm, sm + n / 32};
    return xd;
}

// A lane's x digits for its unit u (64 columns): lo = sub-block 2u, hi = 2u+1.
struct hh_q4k_x {
    uint32_t q1lo[8], q2lo[8], q1hi[8], q2hi[8];
    float slo, shi;  // digit scales / 256 (applied to 256*sum1 + sum2)
    float xlo, xhi;  // exact f32 sums of the two sub-blocks
    uint32_t sel_yz, sel_w;  // v_perm selectors picking this lane's scale bytes
    bool hi_form;            // groups 2,3 use the 6-bit split encoding
};

HH_DEV void hh_q4k_load_lane_x(const hh_xdig& xd, uint32_t u, hh_q4k_x& xr) {
    const uint4* a = reinterpret_cast<const uint4*>(xd.q1 + (size_t)u * 64);
    const uint4* b = reinterpret_cast<const uint4*>(xd.q2 + (size_t)u * 64);
    uint4 t;
    t = a[0]; xr.q1lo[0] = t.x; xr.q1lo[1] = t.y; xr.q1lo[2] = t.z; xr.q1lo[3] = t.w;
    t = a[1]; xr.q1lo[4] = t.x; xr.q1lo[5] = t.y; xr.q1lo[6] = t.z; xr.q1lo[7] = t.w;
    t = a[2]; xr.q1hi[0] = t.x; xr.q1hi[1] = t.y; xr.q1hi[2] = t.z; xr.q1hi[3] = t.w;
    t = a[3]; xr.q1hi[4] = t.x; xr.q1hi[5] = t.y; xr.q1hi[6] = t.z; xr.q1hi[7] = t.w;
    t = b[0]; xr.q2lo[0] = t.x; xr.q2lo[1] = t.y; xr.q2lo[2] = t.z; xr.q2lo[3] = t.w;
    t = b[1]; xr.q2lo[4] = t.x; xr.q2lo[5] = t.y; xr.q2lo[6] = t.z; xr.q2lo[7] = t.w;
    t = b[2]; xr.q2hi[0] = t.x; xr.q2hi[1] = t.y; xr.q2hi[2] = t.z; xr.q2hi[3] = t.w;
    t = b[3]; xr.q2hi[4] = t.x; xr.q2hi[5] = t.y; xr.q2hi[6] = t.z; xr.q2hi[7] = t.w;
    xr.slo = xd.sc[2 * u] * (1.0f / 256.0f);
    xr.shi = xd.sc[2 * u + 1] * (1.0f / 256.0f);
    xr.xlo = xd.sum[2 * u];
    xr.xhi = xd.sum[2 * u + 1];
    const uint32_t g = u & 3u;
    const uint32_t kk = 2u * (g & 1u);  // byte pair of each scale word this group uses
    // perm(src0 = z-word, src1 = y-word): bytes [y_kk, y_kk+1, z_kk, z_kk+1]
    xr.sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    // perm(w, w): bytes [w_kk, w_kk+1, w_kk, w_kk+1]
    xr.sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    xr.hi_form = g >= 2;
}

// Packed [sc0, sc1, m0, m1] of sub-blocks 2g, 2g+1 (get_scale_min_k4, q4k.rs:34-43):
//   j < 4 : sc = s[j] & 63, m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m = (s[j+4] >> 4) | (s[j] >> 6) << 4
HH_DEV uint32_t hh_q4k_scales_packed(const uint4& h, const hh_q4k_x& xr) {
    const uint32_t b = __builtin_amdgcn_perm(h.z, h.y, xr.sel_yz);  // [s_j, s_j+1, s_j+4, s_j+5] (lo form)
    const uint32_t lo = b & 0x3F3F3F3Fu;
    const uint32_t wp = __builtin_amdgcn_perm(h.w, h.w, xr.sel_w);  // [s_j+4, s_j+5, s_j+4, s_j+5] (hi form)
    const uint32_t hi = (wp & 0x00000F0Fu) | ((wp >> 4) & 0x0F0F0000u) | ((b >> 2) & 0x30303030u);
    return xr.hi_form ? hi : lo;
}

struct hh_q4k_data {
    uint4 h, q0, q1;
};

template <bool ACTIVE>
HH_DEV void hh_q4k_load(const uint8_t* row, uint32_t u, hh_q4k_data& d) {
    const uint8_t* blk = row + (size_t)(u >> 2) * 144;
    const uint8_t* q = blk + 16 + (u & 3u) * 32;
    d.h = hh_ld16(blk);
    d.q0 = hh_ld16(q);
    d.q1 = hh_ld16(q + 16);
}

// Contribution of one (row, unit) to the row sum.
HH_DEV float hh_q4k_unit(const hh_q4k_data& d, const hh_q4k_x& xr) {
    const uint32_t qw[8] = {d.q0.x, d.q0.y, d.q0.z, d.q0.w, d.q1.x, d.q1.y, d.q1.z, d.q1.w};
    int a1l = 0, a2l = 0, a1h = 0, a2h = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int lo = (int)(qw[i] & 0x0F0F0F0Fu);
        const int hi = (int)((qw[i] >> 4) & 0x0F0F0F0Fu);
        a1l = __builtin_amdgcn_sdot4(lo, (int)xr.q1lo[i], a1l, false);
        a2l = __builtin_amdgcn_sdot4(lo, (int)xr.q2lo[i], a2l, false);
        a1h = __builtin_amdgcn_sdot4(hi, (int)xr.q1hi[i], a1h, false);
        a2h = __builtin_amdgcn_sdot4(hi, (int)xr.q2hi[i], a2h, false);
    }
    // |a1| <= 32*15*127, so 256*a1 + a2 fits an int32 exactly
    const float tlo = (float)(a1l * 256 + a2l);
    const float thi = (float)(a1h * 256 + a2h);
    const uint32_t s = hh_q4k_scales_packed(d.h, xr);
    const float dd = hh_f16(d.h.x & 0xFFFFu);
    const float dm = hh_f16(d.h.x >> 16);
    const float q = hh_ub0(s) * (xr.slo * tlo) + hh_ub1(s) * (xr.shi * thi);
    const float mn = hh_ub2(s) * xr.xlo + hh_ub3(s) * xr.xhi;
    return dd * q - dm * mn;
}

// Row loop of one team.  NV = values per row (1 = GEMV, 2 = gate/up), R rows per step.
template <int WPT, int R, bool GATEUP>
HH_DEV void hh_q4k_body(const hh_q4k_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr int TEAM = WPT * HH_WAVE;
    constexpr int TPW = HH_Q4K_WAVES / WPT;  // teams per workgroup
    constexpr int NV = GATEUP ? 2 : 1;
    const hh_xdig xd = hh_q4k_stage_x(a.x, a.n, hh_smem);
    __syncthreads();

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % TEAM;
    const uint32_t team = tid / TEAM;
    const uint32_t wave = tid / HH_WAVE;
    const uint32_t P = a.n / 64;
    const bool act = lane < P;
    hh_q4k_x xr;
    if (act) hh_q4k_load_lane_x(xd, lane, xr);

    // contiguous row range of this workgroup
    const uint32_t r0 = (uint32_t)(((uint64_t)blockIdx.x * a.m) / gridDim.x);
    const uint32_t r1 = (uint32_t)(((uint64_t)(blockIdx.x + 1) * a.m) / gridDim.x);
    constexpr uint32_t ROWS_PER_STEP = TPW * R;
    const uint32_t nsteps = (r1 - r0 + ROWS_PER_STEP - 1) / ROWS_PER_STEP;

    auto row_of = [&](uint32_t k, int r) -> uint32_t { return r0 + k * ROWS_PER_STEP + team * R + r; };
    auto load_step = [&](uint32_t k, hh_q4k_data (&buf)[NV][R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = row_of(k, r);
            if (act && row < r1) {
                hh_q4k_load<true>(a.w0 + (size_t)row * a.row_bytes, lane, buf[0][r]);
                if constexpr (GATEUP) hh_q4k_load<true>(a.w1 + (size_t)row * a.row_bytes, lane, buf[NV - 1][r]);
            }
        }
    };
    auto compute_step = [&](uint32_t k, const hh_q4k_data (&buf)[NV][R]) {
        float v[NV * R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const bool ok = act && row_of(k, r) < r1;
#pragma unroll
            for (int j = 0; j < NV; j++) v[j * R + r] = ok ? hh_q4k_unit(buf[j][r], xr) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NV * R; i++) v[i] = hh_wave_sum(v[i]);
        if constexpr (WPT > 1) {
            float* red = xd.red;
            if ((tid % HH_WAVE) == 0) {
#pragma unroll
                for (int i = 0; i < NV * R; i++) red[wave * (NV * R) + i] = v[i];
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NV * R; i++) {
                float s = 0.f;
#pragma unroll
                for (int w = 0; w < WPT; w++) s += red[(team * WPT + w) * (NV * R) + i];
                v[i] = s;
            }
            __syncthreads();
        }
        if (lane < (uint32_t)R) {
            float val = v[0], val2 = v[NV * R - 1];
#pragma unroll
            for (int r = 0; r < R; r++)
                if ((uint32_t)r == lane) {
                    val = v[r];
                    val2 = v[(NV - 1) * R + r];
                }
            const uint32_t row = row_of(k, (int)lane);
            if (row < r1) a.y[row] = GATEUP ? hh_act_mul(val, val2, a.act) : val;
        }
    };

    hh_q4k_data A[NV][R], B[NV][R];
    if (nsteps > 0) load_step(0, A);
    for (uint32_t k = 0; k < nsteps; k += 2) {
        if (k + 1 < nsteps) load_step(k + 1, B);
        compute_step(k, A);
        if (k + 1 >= nsteps) break;
        if (k + 2 < nsteps) load_step(k + 2, A);
        compute_step(k + 1, B);
    }
}

#define HH_Q4K_KERNELS(WPT, R)                                                                     \
    extern "C" __global__ void __launch_bounds__(HH_Q4K_BLOCK) hh_q4k_gemv_w##WPT(const hh_q4k_args a) { \
        hh_q4k_body<WPT, R, false>(a);                                                             \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(HH_Q4K_BLOCK)                                     \
        hh_q4k_gateup_w##WPT(const hh_q4k_args a) {                                                \
        hh_q4k_body<WPT, (R > 1 ? R / 2 : 1), true>(a);                                           \
    }

HH_Q4K_KERNELS(1, 2)
HH_Q4K_KERNELS(2, 2)
HH_Q4K_KERNELS(4, 2)
HH_Q4K_KERNELS(8, 2)
