// Q4_K GEMV and fused gate/up(+act) kernels for gfx950: the FFN hot path at batch 1.
//
// Layout and arithmetic:
//   - Workgroup = 8 waves.  A team of WPT waves (64*WPT lanes) owns one output row at a
//     time; lane l owns "unit" l of the row: Q4_K group g = l & 3 of superblock l >> 2, i.e.
//     qs[32g, 32g+32) (low nibbles = sub-block 2g, high nibbles = sub-block 2g+1) plus the
//     16-byte block header (d, dmin, scales[12]); crates/hayai-model/src/q4k.rs:178-203.
//   - x enters as two int8 digits per element, x ~= s * (q1 + q2/256) with s = amax/127 per
//     32-element sub-block (error <= s/512), plus the per-sub-block scale and exact f32 sum.
//     Either the workgroup builds them from f32 x in LDS (4 lanes per sub-block), or they
//     come pre-built from global memory: the fused gate/up kernel writes the digits of h for
//     the down projection.  Each lane holds its unit's 64 x 2 digits in 32 VGPRs.
//   - Per weight dword (8 nibbles): one AND (low nibbles), shift+AND (high nibbles) and four
//     v_dot4_i32_i8 (nibbles x digit 1, nibbles x digit 2, for both sub-blocks) -- integer
//     sums, exact.  Per (row, group): the sub-block sums are scaled once in f32:
//       d*sc*s*(sum1 + sum2/256) - dmin*m*sum(x)     (factored form of (d*sc)*q - dmin*m)
//   - Loads are double-buffered in registers: row step k+1's 16-byte loads are in flight
//     while step k is computed, and step 0 is issued before the x prologue.  Consecutive
//     lanes read consecutive 32-byte qs chunks, so a wave reads its rows front to back.
//     Row base addresses are wave-uniform (scalar registers).
//   - Team sums: DPP butterfly/broadcast within the wave (v_add_f32_dpp, row_bcast15/31),
//     then an LDS step across the team's waves when WPT > 1.
//   - Each workgroup owns a contiguous row range (32-row aligned for gate/up, so it can
//     quantize its own slice of h); row steps are uniform across the workgroup, so the
//     barriers of the multi-wave reduction stay convergent.
#include "quant.h"

#define HH_Q4K_WAVES 8
#define HH_Q4K_BLOCK (HH_Q4K_WAVES * HH_WAVE)

// Pre-quantized activation digits in global memory (layout of the h workspace):
// q1[n] int8 | q2[n] int8 | scale[n/32] f32 | sum[n/32] f32
struct hh_digits_ptr {
    int8_t* q1;
    int8_t* q2;
    float* sc;
    float* sum;
};

struct hh_q4k_args {
    const uint8_t* w0;  // the matrix (GEMV) or W_gate (gate/up)
    const uint8_t* w1;  // W_up (gate/up only)
    const float* x;     // n floats, 16-byte aligned (f32 input mode)
    float* y;           // m floats (y, or h for gate/up)
    hh_digits_ptr xq;   // digits of x (digit input mode)
    hh_digits_ptr hq;   // gate/up: where to write the digits of h (q1 == NULL: skip)
    uint32_t m;
    uint32_t n;
    uint64_t row_bytes;
    int32_t act;
    uint32_t hrows;  // gate/up: LDS rows reserved for h (max rows of one workgroup)
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

// Quad (4 consecutive lanes) reductions.
HH_DEV float hh_quad_sum(float v) {
    v += hh_dpp<0xB1>(v);
    v += hh_dpp<0x4E>(v);
    return v;
}
HH_DEV float hh_quad_max(float v) {
    v = fmaxf(v, hh_dpp<0xB1>(v));
    v = fmaxf(v, hh_dpp<0x4E>(v));
    return v;
}

// Digits of 8 consecutive elements of one sub-block (scale s = amax/127, inv = 127/amax).
HH_DEV void hh_digits8(const float (&v)[8], float scale, float inv, uint2& o1, uint2& o2) {
    uint32_t p1[2] = {0, 0}, p2[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float a = fminf(fmaxf(rintf(v[i] * inv), -127.f), 127.f);
        const float r = v[i] - a * scale;
        const float b = fminf(fmaxf(rintf(r * inv * 256.0f), -127.f), 127.f);
        p1[i / 4] |= ((uint32_t)(int)a & 0xFFu) << (8 * (i % 4));
        p2[i / 4] |= ((uint32_t)(int)b & 0xFFu) << (8 * (i % 4));
    }
    o1 = make_uint2(p1[0], p1[1]);
    o2 = make_uint2(p2[0], p2[1]);
}

// Device-coherent (agent scope) 32/64-bit accesses: they go to the device coherence point
// (sc1), so data written by one XCD is seen by another without flushing any L2.
HH_DEV void hh_store_coherent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Quantize n f32 values (n % 32 == 0) into digits: 4 lanes per 32-element sub-block,
// chunk c = 8 elements.  Threads first, first + stride, ... take chunks (by default the
// whole workgroup; quads stay whole because first and stride are multiples of 4 and n/8
// is a multiple of 4).  COHERENT: write with
// device-coherent stores (the digits are read by other workgroups in the same launch).
template <bool COHERENT = false>
HH_DEV void hh_quantize_digits(const float* src, uint32_t n, const hh_digits_ptr& dst, uint32_t first = threadIdx.x,
                               uint32_t stride = blockDim.x) {
    for (uint32_t c = first; c < n / 8; c += stride) {
        const float4 t0 = reinterpret_cast<const float4*>(src)[2 * c];
        const float4 t1 = reinterpret_cast<const float4*>(src)[2 * c + 1];
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
        if constexpr (COHERENT) {
            uint32_t* q1 = reinterpret_cast<uint32_t*>(dst.q1) + 2 * c;
            uint32_t* q2 = reinterpret_cast<uint32_t*>(dst.q2) + 2 * c;
            hh_store_coherent(q1, o1.x);
            hh_store_coherent(q1 + 1, o1.y);
            hh_store_coherent(q2, o2.x);
            hh_store_coherent(q2 + 1, o2.y);
            if ((c & 3u) == 0) {
                hh_store_coherent(reinterpret_cast<uint32_t*>(dst.sc) + c / 4, __float_as_uint(scale));
                hh_store_coherent(reinterpret_cast<uint32_t*>(dst.sum) + c / 4, __float_as_uint(s));
            }
        } else {
            reinterpret_cast<uint2*>(dst.q1)[c] = o1;
            reinterpret_cast<uint2*>(dst.q2)[c] = o2;
            if ((c & 3u) == 0) {
                dst.sc[c / 4] = scale;
                dst.sum[c / 4] = s;
            }
        }
    }
}

// A lane's x digits for its unit u (64 columns): lo = sub-block 2u, hi = 2u+1.
struct hh_q4k_x {
    uint32_t q1lo[8], q2lo[8], q1hi[8], q2hi[8];
    float slo, shi;  // digit scales / 256 (applied to 256*sum1 + sum2)
    float xlo, xhi;  // exact f32 sums of the two sub-blocks
    uint32_t sel_yz, sel_w;  // v_perm selectors picking this lane's scale bytes
    bool hi_form;            // groups 2,3 use the 6-bit split encoding
};

HH_DEV void hh_unpack4(const uint4& t, uint32_t* d) {
    d[0] = t.x;
    d[1] = t.y;
    d[2] = t.z;
    d[3] = t.w;
}

// Works for digits in LDS or in global memory (generic address space).
HH_DEV void hh_q4k_load_lane_x(const hh_digits_ptr& xd, uint32_t u, hh_q4k_x& xr) {
    const uint4* a = reinterpret_cast<const uint4*>(xd.q1 + (size_t)u * 64);
    const uint4* b = reinterpret_cast<const uint4*>(xd.q2 + (size_t)u * 64);
    hh_unpack4(a[0], xr.q1lo);
    hh_unpack4(a[1], xr.q1lo + 4);
    hh_unpack4(a[2], xr.q1hi);
    hh_unpack4(a[3], xr.q1hi + 4);
    hh_unpack4(b[0], xr.q2lo);
    hh_unpack4(b[1], xr.q2lo + 4);
    hh_unpack4(b[2], xr.q2hi);
    hh_unpack4(b[3], xr.q2hi + 4);
    const float2 sc = reinterpret_cast<const float2*>(xd.sc)[u];
    const float2 sm = reinterpret_cast<const float2*>(xd.sum)[u];
    xr.slo = sc.x * (1.0f / 256.0f);
    xr.shi = sc.y * (1.0f / 256.0f);
    xr.xlo = sm.x;
    xr.xhi = sm.y;
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

// One kernel body for all variants.
//   WPT     waves per team (row width up to 64*WPT units)
//   R       rows per team step
//   GATEUP  two matrices, output act(gate)*up (and optionally the digits of that output)
//   XDIG    x arrives as pre-built digits (a.xq) instead of f32 (a.x)
template <int WPT, int R, bool GATEUP, bool XDIG>
HH_DEV void hh_q4k_body(const hh_q4k_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr int TEAM = WPT * HH_WAVE;
    constexpr int TPW = HH_Q4K_WAVES / WPT;  // teams per workgroup
    constexpr int NV = GATEUP ? 2 : 1;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % TEAM;
    const uint32_t team = __builtin_amdgcn_readfirstlane(tid / TEAM);  // wave-uniform
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t P = a.n / 64;
    const bool act = lane < P;

    // Contiguous row range of this workgroup.  When gate/up also emits the digits of h it
    // splits 32-row sub-blocks, so each workgroup owns whole sub-blocks of h.
    uint32_t r0, r1;
    if (GATEUP && a.hq.q1 != nullptr) {
        const uint32_t S = (a.m + 31) / 32;
        r0 = 32u * (uint32_t)(((uint64_t)blockIdx.x * S) / gridDim.x);
        r1 = min(a.m, 32u * (uint32_t)(((uint64_t)(blockIdx.x + 1) * S) / gridDim.x));
    } else {
        r0 = (uint32_t)(((uint64_t)blockIdx.x * a.m) / gridDim.x);
        r1 = (uint32_t)(((uint64_t)(blockIdx.x + 1) * a.m) / gridDim.x);
    }
    constexpr uint32_t ROWS_PER_STEP = TPW * R;
    const uint32_t nsteps = (r1 - r0 + ROWS_PER_STEP - 1) / ROWS_PER_STEP;

    // LDS: [x digits (f32 input mode)] [h rows (gate/up)] [team reduction slots]
    char* lds = hh_smem;
    hh_digits_ptr xd = a.xq;
    if constexpr (!XDIG) {
        xd.q1 = reinterpret_cast<int8_t*>(lds);
        xd.q2 = xd.q1 + a.n;
        xd.sc = reinterpret_cast<float*>(xd.q2 + a.n);
        xd.sum = xd.sc + a.n / 32;
        lds = reinterpret_cast<char*>(xd.sum + a.n / 32);
    }
    float* hl = reinterpret_cast<float*>(lds);  // gate/up: h of rows [r0, r1)
    float* red = hl + (GATEUP ? a.hrows : 0);

    hh_q4k_x xr;
    auto row_of = [&](uint32_t k, int r) -> uint32_t { return r0 + k * ROWS_PER_STEP + team * R + r; };
    auto load_step = [&](uint32_t k, hh_q4k_data (&buf)[NV][R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = row_of(k, r);
            if (row < r1) {
                const size_t off = (size_t)row * a.row_bytes;  // scalar
                if (act) {
                    hh_q4k_load(a.w0 + off, lane, buf[0][r]);
                    if constexpr (GATEUP) hh_q4k_load(a.w1 + off, lane, buf[NV - 1][r]);
                }
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
            if (row < r1) {
                const float out = GATEUP ? hh_act_mul(val, val2, a.act) : val;
                a.y[row] = out;
                if constexpr (GATEUP) hl[row - r0] = out;
            }
        }
    };

    // The first row step's weights do not depend on x: put them in flight before the
    // x prologue so HBM latency overlaps the digit conversion.
    hh_q4k_data A[NV][R], B[NV][R];
    if (nsteps > 0) load_step(0, A);
    if constexpr (!XDIG) {
        hh_quantize_digits(a.x, a.n, xd);
        __syncthreads();
    }
    if (act) hh_q4k_load_lane_x(xd, lane, xr);

    for (uint32_t k = 0; k < nsteps; k += 2) {
        if (k + 1 < nsteps) load_step(k + 1, B);
        compute_step(k, A);
        if (k + 1 >= nsteps) break;
        if (k + 2 < nsteps) load_step(k + 2, A);
        compute_step(k + 1, B);
    }

    if constexpr (GATEUP) {
        // Digits of this workgroup's slice of h for the down projection.
        if (a.hq.q1 != nullptr && r1 > r0) {
            __syncthreads();
            const hh_digits_ptr dst{a.hq.q1 + r0, a.hq.q2 + r0, a.hq.sc + r0 / 32, a.hq.sum + r0 / 32};
            hh_quantize_digits(hl, r1 - r0, dst);
        }
    }
}

// Kernel names: hh_q4k_{gemv,gemvq,gateup}_w<WPT>.  WPT = waves per team (row width up to
// 64*WPT units); gemvq takes x as pre-built digits.  Rows per team step: 2 for a GEMV,
// 1 for gate/up (two matrices), which measured best on MI355X.
#define HH_Q4K_KERNEL(KIND, GU, XD, WPT, R)                                                  \
    extern "C" __global__ void __launch_bounds__(HH_Q4K_BLOCK) hh_q4k_##KIND##_w##WPT(const hh_q4k_args a) { \
        hh_q4k_body<WPT, R, GU, XD>(a);                                                      \
    }
#define HH_Q4K_WPT(WPT)                          \
    HH_Q4K_KERNEL(gemv, false, false, WPT, 2)    \
    HH_Q4K_KERNEL(gemvq, false, true, WPT, 2)    \
    HH_Q4K_KERNEL(gateup, true, false, WPT, 1)

HH_Q4K_WPT(1)
HH_Q4K_WPT(2)
HH_Q4K_WPT(4)
HH_Q4K_WPT(8)

// ----------------------------------------------------------------------------------------
// Grid-wide barrier of the persistent launches (small_ffn.hip, small_stack.hip, the grouped
// MoE kernels).
//
// All workgroups are co-resident (the host sizes the grid from the occupancy API), so a
// grid barrier is safe; it is still bounded: a wait that exceeds ~2^20 sleeps gives up,
// records the failure in the error word and the kernel finishes (the host reports that
// error, sticky, at its next synchronizing call and then clears the barrier state).
//
// Barrier state (hh_bar_*, one 128-byte line each so arrivals and polls spread over memory
// channels instead of serializing on one address):
//   line g      (g < 16)  arrival counter of group g = workgroups with blockIdx % 16 == g
//   line 16 + g           release flag of group g (holds the generation of the last release)
//   line 32               arrival counter of groups
//   line 33               error word
//   line 34               epoch: the generation of the last release
//   line 35               stack epoch: the last tag of the FFN-stack exchange (small_stack.hip)
// A launch's generation is the epoch plus one, read by every workgroup before it arrives.
// The last arriver of a group resets its group counter and counts the group; the last
// group resets that counter and writes the generation into every release flag and into
// the epoch.  Counters therefore return to zero at every release and flags need no reset.
// The epoch changes only at a release, which needs every workgroup's arrival, so all
// workgroups of a launch read the same value: the one the previous launch on this state
// released (launches on one stream do not overlap).  No argument changes between
// launches, so a captured graph replays them as they are.  Data that crosses workgroups
// (and XCDs) goes through device-coherent stores and loads, ordered by s_waitcnt before
// the arrival and by the barrier.
#define HH_BAR_GROUPS 16
#define HH_BAR_LINE 32  // u32 words per 128-byte line
#define HH_BAR_WORDS (HH_BAR_LINE * (2 * HH_BAR_GROUPS + 4))
#define HH_BAR_STACK_EPOCH ((2 * HH_BAR_GROUPS + 3) * HH_BAR_LINE)

HH_DEV unsigned hh_atomic_add_agent(unsigned* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
HH_DEV void hh_store_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
HH_DEV unsigned hh_load_agent(unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The epoch as this launch starts; its generation is the epoch plus one.  Read at the
// start of the kernel by every thread of a wave (one request per wave), so the wait for it
// falls on the wait before the arrival instead of stalling the wave's first loads.
HH_DEV unsigned hh_barrier_epoch(unsigned* bar) { return hh_load_agent(bar + (2 * HH_BAR_GROUPS + 2) * HH_BAR_LINE); }

// The epoch load behind gen has returned before any later memory operation is issued: an
// arrival that overtook it could complete a release whose epoch store the load then sees.
HH_DEV void hh_barrier_gen_ready(unsigned gen) { asm volatile("" ::"v"(gen) : "memory"); }

