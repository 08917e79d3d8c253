// MoE expert routing and the grouped expert FFN (gfx950).
//
// Routing follows route_experts + top_k_indices (crates/hayai-core/src/moe_infer.rs:852-934):
// choice = score (+ e_score_correction_bias); optional grouped selection (group score = sum
// of its top-2 choice values, keep the topk_group best groups, candidates listed group by
// group in rank order); top_k by a stable descending sort of the choice values; weights =
// sigmoid(score) or the softmax over ALL experts' raw scores taken at the selected experts;
// optional renormalisation over the top_k; routed scaling.  One wave routes one token with
// the scores in registers (up to 8 per lane, E <= 512): the stable sort is k rounds of a
// wave-wide argmax ordered by (choice desc, candidate position asc), which yields exactly
// the first k entries of the stable sort.  The softmax denominator is summed sequentially
// in expert order, as the reference's iterator sum is.
//
// Expert FFN (the expert loop + combine of moe_infer.rs:342-455): for token t and its k
// selected experts, y[t] = sum_s w[t][s] * down_e(act(gate_e x) * up_e x), e = ids[t][s].
//   hh_moe_gateup_t<TEAM> (grid.y = token): optionally routes the token first (wave 0, into
//     LDS; workgroup 0 also publishes ids / weights for the down kernel), then rows
//     r < k*d_ff: row r % d_ff of expert ids[t][r / d_ff] -> h[t][r].
//   hh_moe_down_t<TEAM>: a workgroup owns a few output rows; its teams take (row, slot)
//     pairs, and the partial dots meet in LDS, where each row adds w[t][s] * dot_s in slot
//     order.
// Both use the Q4_K int8-digit dot products of q4k.hip with a team of TEAM lanes (16, 32 or
// 64) per row: expert rows are short (e.g. 2048 or 768 columns), so several rows share a
// wave.  Lane l of a team owns units l, l + TEAM, ... of the row; x (or h) is converted to
// digits in LDS once per workgroup.  (Compiled after q4k.hip in the same translation unit.)

#define HH_MOE_BLOCK 256
#define HH_MOE_MAX_E 512
#define HH_MOE_EPL (HH_MOE_MAX_E / HH_WAVE)  // experts per lane

struct hh_route_args {
    const float* logits;  // [T][E]
    const float* bias;    // [E] or null
    int32_t* ids;         // [T][k_out]
    float* wts;           // [T][k_out]
    uint32_t T, E, top_k, k_out;  // k_out = slots per token in ids / wts (= top_k)
    uint32_t n_group, topk_group;
    int32_t gating, norm;
    float scale;
    uint32_t pad;
};

// Per-wave LDS scratch of the routing.
struct hh_route_lds {
    float sc[HH_MOE_MAX_E];  // raw scores
    float ex[HH_MOE_MAX_E];  // choice values (grouped pass), then exp(score - max)
    float gscore[64];
    int grank[64];
    int group_of_rank[64];
};

// Key of a candidate in the order of the stable descending sort (value desc, position asc):
// order-preserving bits of the value (+0 for -0, which compares equal to it), then the
// complemented position.  0 marks "no candidate" and is below every candidate's key.
HH_DEV uint64_t hh_route_key(float v, int p) {
    uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)~(uint32_t)p;
}

template <int CTRL, int ROW_MASK = 0xF>
HH_DEV uint64_t hh_dpp_u64(uint64_t v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xF, true);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Maximum over the wave's 64 lanes, returned to every lane (DPP within rows of 16, row
// broadcasts into lane 63, then readlane).  Lanes a DPP step does not write see 0.
HH_DEV uint64_t hh_wave_max_u64(uint64_t k) {
    uint64_t o;
    o = hh_dpp_u64<0xB1>(k);  // quad_perm [1,0,3,2]
    k = o > k ? o : k;
    o = hh_dpp_u64<0x4E>(k);  // quad_perm [2,3,0,1]
    k = o > k ? o : k;
    o = hh_dpp_u64<0x124>(k);  // row_ror:4
    k = o > k ? o : k;
    o = hh_dpp_u64<0x128>(k);  // row_ror:8
    k = o > k ? o : k;
    o = hh_dpp_u64<0x142, 0xA>(k);  // row_bcast:15
    k = o > k ? o : k;
    o = hh_dpp_u64<0x143, 0xC>(k);  // row_bcast:31
    k = o > k ? o : k;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

HH_DEV float hh_wave_max_f(float v) {
    v = fmaxf(v, hh_dpp<0xB1>(v));
    v = fmaxf(v, hh_dpp<0x4E>(v));
    v = fmaxf(v, hh_dpp<0x124>(v));
    v = fmaxf(v, hh_dpp<0x128>(v));
    // row broadcasts leave 0 in the lanes they do not write: only combine the written ones
    const uint32_t lane = threadIdx.x % HH_WAVE;
    const float b15 = hh_dpp<0x142, 0xA>(v);
    if ((lane >> 4) & 1u) v = fmaxf(v, b15);
    const float b31 = hh_dpp<0x143, 0xC>(v);
    if (lane >= 32) v = fmaxf(v, b31);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// LDS written by other lanes of this wave is read after this point.
HH_DEV void hh_wave_sync() {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
}

// Routing of token t by one wave, in three steps that hh_route_token runs back to back and
// the one-token MoE kernel runs on two waves at once:
//   hh_route_select_n:  the selection; lane r < kk gets the expert of slot r (return kk);
//   hh_route_softmax_n: exp(score - max) of every expert into ex[], returns 1/sum (the sum
//                       sequential in expert order, as the reference's iterator sum);
//   hh_route_weight:    slot weights (softmax or sigmoid), renormalisation, scaling.
// EPL = experts per lane held in registers (E <= 64 * EPL); every EPL gives the same
// selections and bit-identical weights (the same operations in the same order on the same
// candidates; lanes' extra slots only ever hold non-candidates).
template <int EPL>
HH_DEV uint32_t hh_route_select_n(const hh_route_args& a, uint32_t t, bool valid, hh_route_lds& L, int* id) {
    const uint32_t lane = threadIdx.x % HH_WAVE;
    const uint32_t E = a.E;
    float sc[EPL], ch[EPL];
    int pos[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const uint32_t e = lane + HH_WAVE * i;
        const bool in = e < E;
        const float s = (in && valid) ? a.logits[(size_t)t * E + e] : 0.f;
        sc[i] = s;
        ch[i] = in ? (a.bias ? s + a.bias[e] : s) : -INFINITY;
        pos[i] = in ? (int)e : -1;
        if (in) {
            L.sc[e] = s;
            L.ex[e] = ch[i];
        }
    }
    hh_wave_sync();
    const bool grouped = a.n_group > 0 && a.topk_group > 0 && E % a.n_group == 0;
    uint32_t kk;
    if (grouped) {
        const uint32_t G = a.n_group, gs = E / G;
        if (lane < G) {
            float m1 = -INFINITY, m2 = -INFINITY;  // the two largest choice values of the group
            for (uint32_t j = 0; j < gs; j++) {
                const float v = L.ex[lane * gs + j];
                if (v > m1) {
                    m2 = m1;
                    m1 = v;
                } else if (v > m2) {
                    m2 = v;
                }
            }
            L.gscore[lane] = gs >= 2 ? m1 + m2 : m1;
        }
        hh_wave_sync();
        if (lane < G) {
            const float v = L.gscore[lane];
            int rank = 0;
            for (uint32_t g = 0; g < G; g++) {
                const float u = L.gscore[g];
                rank += (u > v || (u == v && g < lane)) ? 1 : 0;
            }
            L.grank[lane] = rank;
            L.group_of_rank[rank] = (int)lane;
        }
        hh_wave_sync();
        const uint32_t keep = a.topk_group < G ? a.topk_group : G;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const uint32_t e = lane + HH_WAVE * i;
            if (e < E) {
                const uint32_t g = e / gs;
                const int rank = L.grank[g];
                pos[i] = (uint32_t)rank < keep ? rank * (int)gs + (int)(e - g * gs) : -1;
            }
        }
        const uint32_t ncand = keep * gs > 0 ? keep * gs : 1;
        kk = a.top_k < 1 ? 1 : a.top_k;
        kk = kk < ncand ? kk : ncand;
    } else {
        kk = a.top_k < E ? a.top_k : E;
        if (kk < 1) kk = 1;
    }

    // k rounds of wave argmax over the candidates' keys (every round has a candidate: kk
    // never exceeds their number).  Candidate position -> expert: e = p (ungrouped) or
    // e = group_of_rank[p / gs] * gs + p % gs (grouped).
    const uint32_t gsz = grouped ? E / a.n_group : E;
    int sel = 0;
    for (uint32_t r = 0; r < kk; r++) {
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const uint64_t key = pos[i] >= 0 ? hh_route_key(ch[i], pos[i]) : 0ull;
            best = key > best ? key : best;
        }
        best = hh_wave_max_u64(best);
        const int p = best ? (int)~(uint32_t)best : 0;
        const int be = grouped ? L.group_of_rank[p / (int)gsz] * (int)gsz + p % (int)gsz : p;
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if ((int)(lane + HH_WAVE * i) == be) pos[i] = -1;
        if (lane == r) sel = be;
    }
    *id = sel;
    return kk;
}

template <int EPL>
HH_DEV float hh_route_softmax_n(const hh_route_args& a, uint32_t t, bool valid, float* ex) {
    const uint32_t lane = threadIdx.x % HH_WAVE;
    const uint32_t E = a.E;
    float sc[EPL];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const uint32_t e = lane + HH_WAVE * i;
        sc[i] = (e < E && valid) ? a.logits[(size_t)t * E + e] : 0.f;
        if (e < E) mx = fmaxf(mx, sc[i]);
    }
    mx = hh_wave_max_f(mx);
    hh_wave_sync();  // (ex may be the selection's scratch, done with by now)
#pragma unroll
    for (int i = 0; i < EPL; i++)
        if (lane + HH_WAVE * i < E) ex[lane + HH_WAVE * i] = expf(sc[i] - mx);
    hh_wave_sync();
    // sequential sum in expert order (every lane computes it; the loads are broadcasts)
    float sum = 0.f;
    uint32_t e = 0;
#pragma unroll 8
    for (; e + 4 <= E; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(&ex[e]);
        sum += v.x;
        sum += v.y;
        sum += v.z;
        sum += v.w;
    }
    for (; e < E; e++) sum += ex[e];
    return sum > 0.f ? 1.0f / sum : 0.f;
}

// Lane r < kk: the weight of slot r (expert sel); sc = raw scores, ex / inv from
// hh_route_softmax_n (unused for sigmoid gating).
HH_DEV float hh_route_weight(const hh_route_args& a, const float* sc, const float* ex, float inv, int sel,
                             uint32_t kk) {
    const uint32_t lane = threadIdx.x % HH_WAVE;
    float wv = 0.f;
    if (a.gating == 1) {
        if (lane < kk) wv = 1.0f / (1.0f + expf(-sc[sel]));
    } else {
        if (lane < kk) wv = ex[sel] * inv;
    }
    if (a.norm) {
        float s = 0.f;
        for (uint32_t r = 0; r < kk; r++)  // in selection order
            s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wv), (int)r));
        if (s > 0.f) wv = wv / s;
    }
    if (fabsf(a.scale - 1.0f) > 1e-9f) wv = wv * a.scale;
    return wv;
}

template <int EPL>
HH_DEV uint32_t hh_route_token_n(const hh_route_args& a, uint32_t t, bool valid, hh_route_lds& L, int* id, float* w) {
    int sel;
    const uint32_t kk = hh_route_select_n<EPL>(a, t, valid, L, &sel);
    const float inv = a.gating == 1 ? 0.f : hh_route_softmax_n<EPL>(a, t, valid, L.ex);
    *id = sel;
    *w = hh_route_weight(a, L.sc, L.ex, inv, sel, kk);
    return kk;
}

HH_DEV uint32_t hh_route_select(const hh_route_args& a, uint32_t t, bool valid, hh_route_lds& L, int* id) {
    if (a.E <= 64) return hh_route_select_n<1>(a, t, valid, L, id);
    if (a.E <= 128) return hh_route_select_n<2>(a, t, valid, L, id);
    if (a.E <= 256) return hh_route_select_n<4>(a, t, valid, L, id);
    return hh_route_select_n<HH_MOE_EPL>(a, t, valid, L, id);
}

HH_DEV float hh_route_softmax(const hh_route_args& a, uint32_t t, bool valid, float* ex) {
    if (a.E <= 64) return hh_route_softmax_n<1>(a, t, valid, ex);
    if (a.E <= 128) return hh_route_softmax_n<2>(a, t, valid, ex);
    if (a.E <= 256) return hh_route_softmax_n<4>(a, t, valid, ex);
    return hh_route_softmax_n<HH_MOE_EPL>(a, t, valid, ex);
}

HH_DEV uint32_t hh_route_token(const hh_route_args& a, uint32_t t, bool valid, hh_route_lds& L, int* id, float* w) {
    if (a.E <= 64) return hh_route_token_n<1>(a, t, valid, L, id, w);
    if (a.E <= 128) return hh_route_token_n<2>(a, t, valid, L, id, w);
    if (a.E <= 256) return hh_route_token_n<4>(a, t, valid, L, id, w);
    return hh_route_token_n<HH_MOE_EPL>(a, t, valid, L, id, w);
}

extern "C" __global__ void __launch_bounds__(HH_MOE_BLOCK) hh_moe_route(const hh_route_args a) {
    __shared__ __attribute__((aligned(16))) hh_route_lds lds[HH_MOE_BLOCK / HH_WAVE];
    const uint32_t lane = threadIdx.x % HH_WAVE, w = threadIdx.x / HH_WAVE;
    const uint32_t t = blockIdx.x * (HH_MOE_BLOCK / HH_WAVE) + w;
    int id;
    float wv;
    const uint32_t kk = hh_route_token(a, t, t < a.T, lds[w], &id, &wv);
    // Slots past the selected count (fewer candidates than top_k) hold id -1, weight 0.
    if (t < a.T && lane < a.k_out) {
        a.ids[(size_t)t * a.k_out + lane] = lane < kk ? id : -1;
        a.wts[(size_t)t * a.k_out + lane] = lane < kk ? wv : 0.f;
    }
}

// ---------------------------------------------------------------- expert FFN ----------

struct hh_moe_args {
    const uint8_t* experts;  // expert packs, expert e at e * expert_stride
    uint64_t expert_stride;
    uint64_t gate_off, up_off, down_off;  // tensor offsets inside a pack
    uint64_t rb_in, rb_ff;                // row bytes of gate/up (d_model cols) and down (d_ff cols)
    int32_t* ids;                         // [T][k] (written by the gate/up kernel when it routes)
    float* wts;                           // [T][k]
    const float* x;                       // [T][d_model]
    float* h;                             // [T][k][d_ff]
    float* y;                             // [T][d_model]
    uint32_t d_model, d_ff, k, n_experts;
    int32_t act;
    uint32_t route;                       // gate/up: route the token first (with r)
    hh_route_args r;
};

// Digit layout of n elements at the start of LDS.
HH_DEV hh_digits_ptr hh_moe_digits(char* lds, uint32_t n) {
    hh_digits_ptr d;
    d.q1 = reinterpret_cast<int8_t*>(lds);
    d.q2 = d.q1 + n;
    d.sc = reinterpret_cast<float*>(d.q2 + n);
    d.sum = d.sc + n / 32;
    return d;
}

// Dot of one Q4_K row (units u = l, l + TEAM, ... < P) with digits xd at unit offset u0.
template <int TEAM>
HH_DEV float hh_moe_row_dot(const uint8_t* row, const hh_digits_ptr& xd, uint32_t u0, uint32_t P, uint32_t l) {
    float acc = 0.f;
    for (uint32_t u = l; u < P; u += TEAM) {
        hh_q4k_data dw;
        hh_q4k_load(row, u, dw);
        hh_q4k_x xr;
        hh_q4k_load_lane_x(xd, u0 + u, xr);
        acc += hh_q4k_unit(dw, xr);
    }
    return hh_team_sum<TEAM>(acc);
}

// An expert id, or -1 for an empty slot.  Ids outside [0, n_experts) are treated as empty
// (they never address memory outside the expert buffer).
HH_DEV int hh_moe_valid(const hh_moe_args& a, int e) { return (e < 0 || (uint32_t)e >= a.n_experts) ? -1 : e; }

template <int TEAM>
HH_DEV void hh_moe_gateup_body(const hh_moe_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ __attribute__((aligned(16))) hh_route_lds rl;
    __shared__ int s_ids[64];
    const uint32_t t = blockIdx.y;
    if (a.route) {
        if (threadIdx.x < HH_WAVE) {
            int id;
            float wv;
            const uint32_t kk = hh_route_token(a.r, t, true, rl, &id, &wv);
            const uint32_t lane = threadIdx.x;
            if (lane < a.k) {
                s_ids[lane] = lane < kk ? id : -1;
                if (blockIdx.x == 0) {
                    a.ids[(size_t)t * a.k + lane] = lane < kk ? id : -1;
                    a.wts[(size_t)t * a.k + lane] = lane < kk ? wv : 0.f;
                }
            }
        }
    } else if (threadIdx.x < a.k) {
        s_ids[threadIdx.x] = a.ids[(size_t)t * a.k + threadIdx.x];
    }
    const hh_digits_ptr xd = hh_moe_digits(hh_smem, a.d_model);
    hh_quantize_digits(a.x + (size_t)t * a.d_model, a.d_model, xd);
    __syncthreads();
    const uint32_t P = a.d_model / 64;
    const uint32_t l = threadIdx.x % TEAM;
    const uint32_t tpb = HH_MOE_BLOCK / TEAM;
    const uint32_t team = blockIdx.x * tpb + threadIdx.x / TEAM;
    const uint32_t nteams = gridDim.x * tpb;
    const uint32_t R = a.k * a.d_ff;
    for (uint32_t r = team; r < R; r += nteams) {
        const uint32_t s = r / a.d_ff, j = r - s * a.d_ff;
        const int e = hh_moe_valid(a, s_ids[s]);  // uniform across the team
        float hv = 0.f;
        if (e >= 0) {
            const uint8_t* pack = a.experts + (size_t)e * a.expert_stride;
            const float g = hh_moe_row_dot<TEAM>(pack + a.gate_off + (size_t)j * a.rb_in, xd, 0, P, l);
            const float u = hh_moe_row_dot<TEAM>(pack + a.up_off + (size_t)j * a.rb_in, xd, 0, P, l);
            hv = hh_act_mul(g, u, a.act);
        }
        if (l == 0) a.h[(size_t)t * R + r] = hv;
    }
}

#define HH_MOE_DOWN_ROWS 4  // output rows per workgroup (x k slots = its (row, slot) items)

template <int TEAM>
HH_DEV void hh_moe_down_body(const hh_moe_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ float part[HH_MOE_DOWN_ROWS][64];
    __shared__ int s_ids[64];
    __shared__ float s_w[64];
    const uint32_t t = blockIdx.y;
    if (threadIdx.x < a.k) {
        s_ids[threadIdx.x] = hh_moe_valid(a, a.ids[(size_t)t * a.k + threadIdx.x]);
        s_w[threadIdx.x] = a.wts[(size_t)t * a.k + threadIdx.x];
    }
    const uint32_t nh = a.k * a.d_ff;  // all k intermediate vectors of the token, back to back
    const hh_digits_ptr hd = hh_moe_digits(hh_smem, nh);
    hh_quantize_digits(a.h + (size_t)t * nh, nh, hd);
    __syncthreads();
    const uint32_t P = a.d_ff / 64;
    const uint32_t l = threadIdx.x % TEAM;
    const uint32_t tpb = HH_MOE_BLOCK / TEAM;
    const uint32_t team = threadIdx.x / TEAM;
    const uint32_t j0 = blockIdx.x * HH_MOE_DOWN_ROWS;
    const uint32_t items = HH_MOE_DOWN_ROWS * a.k;
    for (uint32_t it = team; it < items; it += tpb) {
        const uint32_t rl = it / a.k, s = it - rl * a.k, j = j0 + rl;
        const int e = s_ids[s];
        float d = 0.f;
        if (e >= 0 && j < a.d_model) {
            const uint8_t* pack = a.experts + (size_t)e * a.expert_stride;
            d = hh_moe_row_dot<TEAM>(pack + a.down_off + (size_t)j * a.rb_ff, hd, s * P, P, l);
        }
        if (l == 0) part[rl][s] = d;
    }
    __syncthreads();
    if (threadIdx.x < HH_MOE_DOWN_ROWS && j0 + threadIdx.x < a.d_model) {
        float acc = 0.f;
        for (uint32_t s = 0; s < a.k; s++)
            if (s_ids[s] >= 0) acc += s_w[s] * part[threadIdx.x][s];
        a.y[(size_t)t * a.d_model + j0 + threadIdx.x] = acc;
    }
}

#define HH_MOE_KERNELS(TEAM)                                                                           \
    extern "C" __global__ void __launch_bounds__(HH_MOE_BLOCK) hh_moe_gateup_t##TEAM(const hh_moe_args a) { \
        hh_moe_gateup_body<TEAM>(a);                                                                   \
    }                                                                                                  \
    extern "C" __global__ void __launch_bounds__(HH_MOE_BLOCK) hh_moe_down_t##TEAM(const hh_moe_args a) { \
        hh_moe_down_body<TEAM>(a);                                                                     \
    }
HH_MOE_KERNELS(16)
HH_MOE_KERNELS(32)
HH_MOE_KERNELS(64)
