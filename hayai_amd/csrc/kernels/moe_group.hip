// The MoE expert FFN for several tokens as a grouped gather-GEMV (gfx950): every selected
// expert's weights are read once per call for all the tokens routed to it, instead of once
// per (token, expert) pair.  Same results as the expert loop + combine of
// crates/hayai-core/src/moe_infer.rs:342-455 (y[t] = sum over slots s of
// w[t][s] * down_e(act(gate_e x_t) * up_e x_t), e = ids[t][s]):
//   hh_moe_prep:         (token, slot) pairs p = t * k + s grouped by expert, in p order
//                        within an expert, the active experts in ascending order, with one
//                        record per active expert (hh_moeg_args::rec); and every token's x as
//                        int8 digits (hh_moe_route_prep: the routing too)
//   hh_moe_gu_grp_t<TM>: grid.y = active expert; every row of gate and up is read once and
//                        dotted with each of the expert's tokens: h[p][row] = act(g) * u
//   hh_moe_hdigits:      h as digits, by pair
//   hh_moe_dn_grp_t<TM>: grid.y = active expert; every down row read once: yp[p][row]
//   hh_moe_combine:      y[t][row] = sum over valid slots, in slot order, of w[t][s] * yp[t*k+s][row]
// (Compiled after moe.hip in the same translation unit: hh_moe_digits and the Q4_K digit dot
// products of q4k.hip.)

struct hh_moeg_args {
    const uint8_t* experts;  // expert packs, expert e at e * expert_stride
    uint64_t expert_stride;
    uint64_t gate_off, up_off, down_off;
    uint64_t rb_in, rb_ff;   // row bytes of gate/up (d_model columns) and down (d_ff columns)
    const int32_t* ids;      // [T][k]
    const float* wts;        // [T][k]
    const float* x;          // [T][d_model]
    float* h;                // [T * k][d_ff], by pair
    float* yp;               // [T * k][d_model], by pair
    float* y;                // [T][d_model]
    int32_t* order;          // [T * k] pairs grouped by expert
    int32_t* rec;            // [min(E, T * k)][8]: per active expert y (ascending): the expert,
                             // its first position in order, its pair count, its first
                             // HH_MOEG_NS pairs; expert -1 past the active ones
    uint8_t* xq;             // [T] digit forms of x (hh_moe_digits layout, d_model elements)
    uint8_t* hq;             // [T * k] digit forms of h (d_ff elements)
    uint32_t T, k, d_model, d_ff, n_experts;
    int32_t act;
};

#define HH_MOEG_MAX_E 512     // experts the grouping kernel handles
#define HH_MOEG_MAX_P 4096    // (token, slot) pairs
#define HH_MOEG_GU_RPT 2      // rows per team, loads issued together (gate/up: 2 matrices)
#define HH_MOEG_DN_RPT 4
#define HH_MOEG_NS 4          // tokens whose digits a workgroup stages in LDS at a time
#define HH_MOEG_REC 8         // ints per expert record (3 + HH_MOEG_NS, padded to 32 bytes)
#define HH_MOEG_STAGE (HH_MOEG_NS * (2 * 4096 + (4096 / 32) * 8))  // d_model, d_ff <= 4096

// bytes of the digit form of n elements (q1, q2, scale and sum per 32), as hh_moe_digits lays
// it out; a multiple of 16 for n % 64 == 0
HH_DEV size_t hh_digits_bytes_dev(uint32_t n) { return 2u * (size_t)n + (size_t)(n / 32u) * 8u; }

// Sum over a team of TEAM (16, 32, 64) lanes by DPP row operations; the total is valid in
// the team's last lane (TEAM - 1).
template <int TEAM>
HH_DEV float hh_moeg_team_sum(float v) {
    v += hh_dpp<0xB1>(v);  // quad_perm [1,0,3,2]
    v += hh_dpp<0x4E>(v);  // quad_perm [2,3,0,1]
    v += hh_dpp<0x124>(v);  // row_ror:4
    v += hh_dpp<0x128>(v);  // row_ror:8 -> every lane of a row of 16 holds its sum
    if constexpr (TEAM >= 32) v += hh_dpp<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3 hold 32-lane sums
    if constexpr (TEAM >= 64) v += hh_dpp<0x143, 0xC>(v);  // row_bcast:31 -> lane 63 holds the total
    return v;
}

HH_DEV int hh_moeg_valid(const hh_moeg_args& a, int e) { return (e < 0 || (uint32_t)e >= a.n_experts) ? -1 : e; }

// Workgroup 0 groups the pairs; workgroup 1 + t turns token t's x into digits (global, read
// by every expert's gate/up workgroups from L2).  Grouping: pair p's position is its expert's
// start plus the number of earlier pairs with the same expert (its rank); an expert's start
// is the sum of the counts of the experts before it.  The starts (and the list of active
// experts) come from one exclusive scan over the counts; a rank is a few popcounts of the
// expert's bitmask of pairs (built with atomicOr: order-free), or, when the masks would not
// fit LDS, a count over the earlier pairs.  Every result is a pure function of ids.
#define HH_MOEG_MASK_WORDS 4096  // LDS words for the per-expert pair bitmasks

// Exclusive scan over the workgroup of (a, b) pairs, one pair per thread (256 threads):
// returns the sums of the pairs of lower threads; *ta, *tb get the totals.
HH_DEV int2 hh_moeg_scan256(int a, int b, int* ta, int* tb) {
    __shared__ int ws[2][4];
    const uint32_t tid = threadIdx.x, lane = tid % 64, w = tid / 64;
    int ia = a, ib = b;  // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int xa = __shfl_up(ia, d, 64), xb = __shfl_up(ib, d, 64);
        if ((int)lane >= d) {
            ia += xa;
            ib += xb;
        }
    }
    if (lane == 63) {
        ws[0][w] = ia;
        ws[1][w] = ib;
    }
    __syncthreads();
    int oa = 0, ob = 0, sa = 0, sb = 0;
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        if (k < w) {
            oa += ws[0][k];
            ob += ws[1][k];
        }
        sa += ws[0][k];
        sb += ws[1][k];
    }
    *ta = sa;
    *tb = sb;
    return make_int2(oa + ia - a, ob + ib - b);
}

// The grouping, by one workgroup of 256 threads.  Each active expert's record carries what
// its gate/up and down workgroups need before their first loads (one scalar load of 32 bytes
// instead of a chain of dependent reads).
HH_DEV void hh_moeg_group(const hh_moeg_args& a) {
    __shared__ int cnt[HH_MOEG_MAX_E];
    __shared__ int first[HH_MOEG_MAX_E];
    __shared__ int apos[HH_MOEG_MAX_E];  // an active expert's position in ascending order
    __shared__ int pid[HH_MOEG_MAX_P];
    __shared__ uint32_t mask[HH_MOEG_MASK_WORDS];
    const uint32_t tid = threadIdx.x;
    const uint32_t E = a.n_experts, P = a.T * a.k;
    const uint32_t PW = (P + 31) / 32;                     // mask words per expert
    const bool masks = (size_t)E * PW <= HH_MOEG_MASK_WORDS;  // else: count earlier pairs
    for (uint32_t e = tid; e < E; e += 256) cnt[e] = 0;
    if (masks)
        for (uint32_t i = tid; i < E * PW; i += 256) mask[i] = 0u;
    for (uint32_t p = tid; p < P; p += 256) pid[p] = hh_moeg_valid(a, a.ids[p]);
    __syncthreads();
    for (uint32_t p = tid; p < P; p += 256) {
        const int e = pid[p];
        if (e < 0) continue;
        atomicAdd(&cnt[e], 1);  // counts and masks only: order-free
        if (masks) atomicOr(&mask[(uint32_t)e * PW + p / 32], 1u << (p % 32));
    }
    __syncthreads();
    // starts and active-expert positions: each thread owns experts 2 tid and 2 tid + 1
    // (E <= HH_MOEG_MAX_E = 512)
    {
        const uint32_t e0 = 2 * tid, e1 = e0 + 1;
        const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
        int tot, tot_a;
        const int2 ex = hh_moeg_scan256(c0 + c1, (c0 > 0) + (c1 > 0), &tot, &tot_a);
        if (e0 < E) {
            first[e0] = ex.x;
            if (c0) {
                int* r = a.rec + (size_t)ex.y * HH_MOEG_REC;
                r[0] = (int)e0;
                r[1] = ex.x;
                r[2] = c0;
                apos[e0] = ex.y;
            }
        }
        if (e1 < E) {
            first[e1] = ex.x + c0;
            if (c1) {
                const int y = ex.y + (c0 > 0);
                int* r = a.rec + (size_t)y * HH_MOEG_REC;
                r[0] = (int)e1;
                r[1] = ex.x + c0;
                r[2] = c1;
                apos[e1] = y;
            }
        }
        // the records past the active experts, up to the grid's min(E, P) rows
        for (uint32_t y = (uint32_t)tot_a + tid; y < min(E, P); y += 256) a.rec[(size_t)y * HH_MOEG_REC] = -1;
    }
    __syncthreads();
    for (uint32_t p = tid; p < P; p += 256) {
        const int e = pid[p];
        if (e < 0) continue;
        int r = 0;
        if (masks) {
            const uint32_t* m = mask + (uint32_t)e * PW;
            for (uint32_t wi = 0; wi < p / 32; wi++) r += __popc(m[wi]);
            r += __popc(m[p / 32] & ((1u << (p % 32)) - 1u));
        } else {
            for (uint32_t q = 0; q < p; q++) r += pid[q] == e;
        }
        a.order[first[e] + r] = (int)p;
        if (r < HH_MOEG_NS) a.rec[(size_t)apos[e] * HH_MOEG_REC + 3 + r] = (int)p;
    }
}

// Token t's x -> digits (global, read by every expert's gate/up workgroups from L2).
HH_DEV void hh_moeg_x_digits(const hh_moeg_args& a, uint32_t t) {
    hh_quantize_digits(a.x + (size_t)t * a.d_model, a.d_model,
                       hh_moe_digits((char*)a.xq + t * hh_digits_bytes_dev(a.d_model), a.d_model));
}

extern "C" __global__ void __launch_bounds__(256) hh_moe_prep(const hh_moeg_args a) {
    if (blockIdx.x > 0) {
        hh_moeg_x_digits(a, blockIdx.x - 1);
        return;
    }
    hh_moeg_group(a);
}

// Routing and hh_moe_prep in one launch: workgroups 0 .. R-1 route four tokens each (one per
// wave, as hh_moe_route), workgroups R .. R+T-1 turn token t's x into digits.  A routing
// workgroup publishes its ids (device-scope fence) and counts itself on a device counter;
// the last one to arrive fences again, groups every pair (hh_moeg_group) and resets the
// counter for the next launch.  No workgroup waits for another, so the launch needs no
// co-residency and is captured into graphs as it is.
struct hh_moeg_rp_args {
    hh_route_args r;
    hh_moeg_args g;
    unsigned* arrivals;  // one word, 0 between launches
};
extern "C" __global__ void __launch_bounds__(HH_MOE_BLOCK) hh_moe_route_prep(const hh_moeg_rp_args a) {
    const uint32_t R = (a.r.T + HH_MOE_BLOCK / HH_WAVE - 1) / (HH_MOE_BLOCK / HH_WAVE);
    if (blockIdx.x >= R) {
        hh_moeg_x_digits(a.g, blockIdx.x - R);
        return;
    }
    {
        __shared__ __attribute__((aligned(16))) hh_route_lds lds[HH_MOE_BLOCK / HH_WAVE];
        const uint32_t lane = threadIdx.x % HH_WAVE, w = threadIdx.x / HH_WAVE;
        const uint32_t t = blockIdx.x * (HH_MOE_BLOCK / HH_WAVE) + w;
        int id;
        float wv;
        const uint32_t kk = hh_route_token(a.r, t, t < a.r.T, lds[w], &id, &wv);
        if (t < a.r.T && lane < a.r.k_out) {
            a.r.ids[(size_t)t * a.r.k_out + lane] = lane < kk ? id : -1;
            a.r.wts[(size_t)t * a.r.k_out + lane] = lane < kk ? wv : 0.f;
        }
    }
    __shared__ int last;
    __threadfence();  // this workgroup's ids are visible device-wide before it counts itself
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(a.arrivals, 1u) == R - 1u;
    __syncthreads();
    if (!last) return;
    __threadfence();  // every workgroup's ids are visible to this one
    hh_moeg_group(a.g);
    if (threadIdx.x == 0) __hip_atomic_store(a.arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// h (f32, by pair) -> digits, one workgroup per pair.
extern "C" __global__ void __launch_bounds__(256) hh_moe_hdigits(const hh_moeg_args a) {
    const uint32_t p = blockIdx.x;
    if (hh_moeg_valid(a, a.ids[p]) < 0) return;
    hh_quantize_digits(a.h + (size_t)p * a.d_ff, a.d_ff,
                       hh_moe_digits((char*)a.hq + p * hh_digits_bytes_dev(a.d_ff), a.d_ff));
}

// The digit forms of the expert's tokens (or pairs) i0 .. i0 + n - 1 -> LDS, 16 bytes per
// thread per step (the forms are a multiple of 16 bytes); ends with a workgroup barrier.
HH_DEV void hh_moeg_stage(uint8_t* lds, const uint8_t* src, const int32_t* order, int p0, int i0, int n,
                          uint32_t k_div, size_t bytes) {
    const uint32_t per = (uint32_t)(bytes / 16);
    for (uint32_t c = threadIdx.x; c < (uint32_t)n * per; c += blockDim.x) {
        const uint32_t i = c / per, o = c % per;
        const uint32_t p = (uint32_t)order[p0 + i0 + (int)i], id = k_div ? p / k_div : p;
        reinterpret_cast<uint4*>(lds + i * bytes)[o] = reinterpret_cast<const uint4*>(src + id * bytes)[o];
    }
    __syncthreads();
}

// The first batch's token forms (pairs from the expert's record) requested ahead of a
// workgroup's weight loads, by global->LDS DMA (no registers held): 64 consecutive 16-byte chunks of the stage per instruction, wave w
// taking chunk runs w, w + 4, ...  Vector loads complete in order, so once at most the weight
// loads issued after them are outstanding the forms are in LDS (hh_moeg_stage_wait); a form
// loaded after the weights, as hh_moeg_stage does, waits for all of them.
HH_DEV void hh_moeg_stage_dma(uint8_t* lds, const uint8_t* src, const int (&first)[HH_MOEG_NS], int n, uint32_t k_div,
                              size_t bytes) {
    static_assert(HH_MOEG_NS == 4, "the pair select below");
    const uint32_t per = (uint32_t)(bytes / 16), tot = (uint32_t)n * per;
    const uint32_t wave = threadIdx.x / HH_WAVE, lane = threadIdx.x % HH_WAVE;
    for (uint32_t c0 = wave * HH_WAVE; c0 < tot; c0 += 4u * HH_WAVE) {  // 4 waves per workgroup
        const uint32_t c = c0 + lane;
        if (c < tot) {
            const uint32_t i = c / per, o = c % per;
            const int f = i == 0 ? first[0] : i == 1 ? first[1] : i == 2 ? first[2] : first[3];
            const uint32_t p = (uint32_t)f, id = k_div ? p / k_div : p;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + id * bytes + o * 16u),
                                             (__attribute__((address_space(3))) void*)(lds + (size_t)c0 * 16u), 16, 0, 0);
        }
    }
    // the weight loads that follow stay after these copies in the instruction stream
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
// after the weight loads: the DMA of hh_moeg_stage_dma has landed (at most NW loads newer than
// it outstanding), then every wave's part is visible
template <int NW>
HH_DEV void hh_moeg_stage_wait() {
    __builtin_amdgcn_s_waitcnt((NW & 15) | ((NW >> 4) << 14) | (7 << 4) | (15 << 8));
    __syncthreads();
}

// Gate/up: a team of TEAM lanes per row (lane = 64-column unit, d_model <= 64 * TEAM); each
// team takes HH_MOEG_GU_RPT rows with all their loads in flight, then dots them with every token
// of the expert (the lane's slice of the token's digits, staged in LDS HH_MOEG_NS tokens at a
// time: every team reads them, so from L2 each would be read TPB times).
template <int TEAM>
HH_DEV void hh_moe_gu_grp_body(const hh_moeg_args& a) {
    __shared__ __attribute__((aligned(16))) uint8_t stage[HH_MOEG_STAGE];
    const int* const rc = a.rec + (size_t)blockIdx.y * HH_MOEG_REC;
    const int e = rc[0];
    if (e < 0) return;  // grid.y covers the most experts a call can select
    const int p0 = rc[1], np = rc[2];
    const int first[HH_MOEG_NS] = {rc[3], rc[4], rc[5], rc[6]};
    const uint32_t dm = a.d_model, df = a.d_ff, P = dm / 64;
    const size_t xbytes = hh_digits_bytes_dev(dm);
    constexpr uint32_t TPB = 256 / TEAM;
    const uint32_t l = threadIdx.x % TEAM, team = threadIdx.x / TEAM;
    const uint32_t rows_per_block = TPB * HH_MOEG_GU_RPT;
    const uint32_t j0 = blockIdx.x * rows_per_block + team * HH_MOEG_GU_RPT;
    const uint8_t* pack = a.experts + (size_t)e * a.expert_stride;
    const bool act = l < P;
    const uint32_t u = act ? l : 0u;
    hh_moeg_stage_dma(stage, a.xq, first, min(HH_MOEG_NS, np), a.k, xbytes);
    hh_q4k_data g[HH_MOEG_GU_RPT], up[HH_MOEG_GU_RPT];
#pragma unroll
    for (int r = 0; r < HH_MOEG_GU_RPT; r++) {
        const uint32_t j = min(j0 + r, df - 1);
        hh_q4k_load(pack + a.gate_off + (size_t)j * a.rb_in, u, g[r]);
        hh_q4k_load(pack + a.up_off + (size_t)j * a.rb_in, u, up[r]);
    }
    for (int i0 = 0; i0 < np; i0 += HH_MOEG_NS) {
        const int n = min(HH_MOEG_NS, np - i0);
        if (i0 == 0) {
            hh_moeg_stage_wait<3 * 2 * HH_MOEG_GU_RPT>();  // three loads per (row, matrix)
        } else {
            __syncthreads();  // the previous tokens' digits are consumed
            hh_moeg_stage(stage, a.xq, a.order, p0, i0, n, a.k, xbytes);
        }
        for (int i = 0; i < n; i++) {
            const uint32_t p = (uint32_t)a.order[p0 + i0 + i];
            hh_q4k_x xr;
            hh_q4k_load_lane_x(hh_moe_digits((char*)stage + i * xbytes, dm), u, xr);
            // every lane computes (a lane past the row's units holds unit 0's data and
            // contributes zero): no branch, so the rows' dot and DPP chains interleave
            float gt[HH_MOEG_GU_RPT], ut[HH_MOEG_GU_RPT];
#pragma unroll
            for (int r = 0; r < HH_MOEG_GU_RPT; r++) {
                const float gx = hh_q4k_unit(g[r], xr), ux = hh_q4k_unit(up[r], xr);
                gt[r] = act ? gx : 0.f;
                ut[r] = act ? ux : 0.f;
            }
#pragma unroll
            for (int r = 0; r < HH_MOEG_GU_RPT; r++) {
                gt[r] = hh_moeg_team_sum<TEAM>(gt[r]);
                ut[r] = hh_moeg_team_sum<TEAM>(ut[r]);
            }
#pragma unroll
            for (int r = 0; r < HH_MOEG_GU_RPT; r++)
                if (l == TEAM - 1 && j0 + r < df) a.h[(size_t)p * df + j0 + r] = hh_act_mul(gt[r], ut[r], a.act);
        }
    }
}

// Down: the same with the expert's pairs' h (d_ff columns) and d_model rows -> yp[p][row].
template <int TEAM>
HH_DEV void hh_moe_dn_grp_body(const hh_moeg_args& a) {
    __shared__ __attribute__((aligned(16))) uint8_t stage[HH_MOEG_STAGE];
    const int* const rc = a.rec + (size_t)blockIdx.y * HH_MOEG_REC;
    const int e = rc[0];
    if (e < 0) return;
    const int p0 = rc[1], np = rc[2];
    const int first[HH_MOEG_NS] = {rc[3], rc[4], rc[5], rc[6]};
    const uint32_t dm = a.d_model, df = a.d_ff, P = df / 64;
    const size_t hbytes = hh_digits_bytes_dev(df);
    constexpr uint32_t TPB = 256 / TEAM;
    const uint32_t l = threadIdx.x % TEAM, team = threadIdx.x / TEAM;
    const uint32_t rows_per_block = TPB * HH_MOEG_DN_RPT;
    const uint32_t j0 = blockIdx.x * rows_per_block + team * HH_MOEG_DN_RPT;
    const uint8_t* pack = a.experts + (size_t)e * a.expert_stride;
    const bool act = l < P;
    const uint32_t u = act ? l : 0u;
    hh_moeg_stage_dma(stage, a.hq, first, min(HH_MOEG_NS, np), 0u, hbytes);
    hh_q4k_data w[HH_MOEG_DN_RPT];
#pragma unroll
    for (int r = 0; r < HH_MOEG_DN_RPT; r++) hh_q4k_load(pack + a.down_off + (size_t)min(j0 + r, dm - 1) * a.rb_ff, u, w[r]);
    for (int i0 = 0; i0 < np; i0 += HH_MOEG_NS) {
        const int n = min(HH_MOEG_NS, np - i0);
        if (i0 == 0) {
            hh_moeg_stage_wait<3 * HH_MOEG_DN_RPT>();
        } else {
            __syncthreads();
            hh_moeg_stage(stage, a.hq, a.order, p0, i0, n, 0u, hbytes);
        }
        for (int i = 0; i < n; i++) {
            const uint32_t p = (uint32_t)a.order[p0 + i0 + i];
            hh_q4k_x hr;
            hh_q4k_load_lane_x(hh_moe_digits((char*)stage + i * hbytes, df), u, hr);
            float dt[HH_MOEG_DN_RPT];
#pragma unroll
            for (int r = 0; r < HH_MOEG_DN_RPT; r++) {
                const float dx = hh_q4k_unit(w[r], hr);
                dt[r] = act ? dx : 0.f;
            }
#pragma unroll
            for (int r = 0; r < HH_MOEG_DN_RPT; r++) dt[r] = hh_moeg_team_sum<TEAM>(dt[r]);
#pragma unroll
            for (int r = 0; r < HH_MOEG_DN_RPT; r++)
                if (l == TEAM - 1 && j0 + r < dm) a.yp[(size_t)p * dm + j0 + r] = dt[r];
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) hh_moe_combine(const hh_moeg_args a) {
    const uint32_t j = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (j >= a.d_model) return;
    float acc = 0.f;
    for (uint32_t s = 0; s < a.k; s++) {
        const uint32_t p = t * a.k + s;
        if (hh_moeg_valid(a, a.ids[p]) >= 0) acc += a.wts[p] * a.yp[(size_t)p * a.d_model + j];
    }
    a.y[(size_t)t * a.d_model + j] = acc;
}

// gate/up held to 128 VGPRs: four of its 4-wave workgroups per CU (the LDS stage allows four)
#define HH_MOEG_KERNELS(TEAM)                                                                          \
    extern "C" __global__ void __launch_bounds__(256, 4) hh_moe_gu_grp_t##TEAM(const hh_moeg_args a) {  \
        hh_moe_gu_grp_body<TEAM>(a);                                                                   \
    }                                                                                                  \
    extern "C" __global__ void __launch_bounds__(256) hh_moe_dn_grp_t##TEAM(const hh_moeg_args a) {     \
        hh_moe_dn_grp_body<TEAM>(a);                                                                   \
    }
HH_MOEG_KERNELS(16)
HH_MOEG_KERNELS(32)
HH_MOEG_KERNELS(64)
