// Consecutive FFN residual blocks of one token in one persistent launch (gfx950), for small
// Q4_0 / Q8_0 layers (SmolLM2-135M: d_model 576, d_ff 1536, 1.5 MB per layer):
//   x_{l+1} = x_l + W_down,l . (act(W_gate,l . n_l) * (W_up,l . n_l)),
//   n_l = x_l * (1 / sqrt(mean(x_l^2) + eps)) * norm_l,
// the ffn_apply of crates/hayai-core/src/hybrid_infer.rs:883-936 (rms_norm of
// crates/hayai-cpu/src/attention.rs:142-147; the FFN of stream_infer.rs:3752-3864) applied
// layer after layer, y = x_L.
//
// A layer this small is latency bound: its weights stream in well under a microsecond, but
// two cross-workgroup exchanges (x -> every workgroup, h -> every workgroup) sit on its
// dependency chain.  One launch runs every layer, so
//   - weights (and norm vectors) do not depend on x: each compute thread keeps a register
//     ring of K layers and requests layer l+K's rows as soon as layer l has consumed them;
//   - the exchanges carry their own validity: every element of h and of x is published as
//     one 64-bit word (f32 bits | tag << 32) by a single device-coherent store, and readers
//     poll the words until every tag is the one of this layer.  No barrier, flag or
//     counter round trip: one store-to-load hop per exchange;
//   - the polling is done by a fifth wave (the exchange wave), so no compute wave's
//     in-order load counter ever waits behind a poll, and no poll behind a weight load.
//
// Tags: the launch reads the stack epoch E (a word of the grid-barrier state) before it
// publishes anything; layer l publishes h with tag E+l+1 and x_{l+1} with tag E+l+1.
// Workgroup 0 stores E+L once it has seen every workgroup's h of layer 0 (so every
// workgroup has read E).  Tags therefore never repeat on a word between writes, and the
// kernel's arguments do not change between launches (graph-capturable).
//
// Single exchange buffers suffice because every workgroup owns at least one gate/up row and
// one down row (grid <= min(d_model, d_ff)): a workgroup overwrites h of layer l only after
// it has every x_{l+1} row, each published after its producer read all of h of layer l; the
// same holds for x with the roles swapped.
//
// Waits are bounded: a poll that exceeds ~2^20 sleeps records the error word, and every
// wave of the workgroup leaves at the next workgroup barrier; the other workgroups then time
// out the same way.  (Compiled after small_ffn.hip: the grid-barrier state layout.)

#define HH_SSTK_CW 4                               // compute waves
#define HH_SSTK_BLOCK ((HH_SSTK_CW + 1) * HH_WAVE)  // + the exchange wave
#define HH_SSTK_MAX 2048                           // d_model, d_ff <= 64 blocks of 32

struct hh_sstk_args {
    const uint8_t* pack;  // layer 0's pack; layer l at pack + l * stride
    const float* norm;    // layer 0's norm; layer l at norm + l * norm_stride
    const float* x;       // x_0
    float* y;             // x_L (may be x)
    uint64_t* hx;         // d_ff tagged words of h
    uint64_t* xx;         // d_model tagged words of x_l (l >= 1)
    uint64_t* spare;      // 16 words (one 128-byte line) per workgroup: stores without a target
    unsigned* bar;        // grid-barrier state (the stack epoch word, the error word)
    uint64_t stride;
    uint64_t off_g, off_u, off_d;
    uint64_t rb_in, rb_ff;  // row bytes of gate/up (d_model columns) and down (d_ff columns)
    uint32_t norm_stride;   // floats
    uint32_t d_model, d_ff, n_layers;
    float eps;
    int32_t act;
};

#ifdef HH_SSTK_TRACE
// Timeline build only: s_memrealtime (100 MHz) per workgroup, layer and event.
__device__ uint64_t hh_sstk_trace[256][64][8];
#define HH_SSTK_MARK(ev, cond) \
    do { if ((cond) && w < 256 && l < 64) hh_sstk_trace[w][l][ev] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define HH_SSTK_MARK(ev, cond) do { } while (0)
#endif

HH_DEV uint64_t hh_sstk_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
HH_DEV void hh_sstk_publish(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The exchange wave gathers n tagged words (element lane + 64 j in t[j]); false on timeout.
// Every poll requests all NJ words at once (indices past n re-read word n-1, so the loads
// are unconditional and never wait for one another), until one poll finds every tag.  A
// word that carries the tag keeps it until this wave has finished: its producer writes it
// again only for the next layer, which needs this workgroup's own next publication.
template <int NJ>
HH_DEV bool hh_sstk_gather(const uint64_t* src, uint32_t n, uint32_t tag, uint64_t (&t)[NJ], uint32_t lane) {
#pragma unroll
    for (int j = 0; j < NJ; j++) t[j] = hh_sstk_load(src + min(lane + 64u * j, n - 1u));
    for (uint32_t spins = 0;; spins++) {
        bool stale = false;
#pragma unroll
        for (int j = 0; j < NJ; j++) stale |= (uint32_t)(t[j] >> 32) != tag;
        if (__ballot(stale) == 0) return true;  // wave-uniform
        if (spins > (1u << 20)) return false;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < NJ; j++) t[j] = hh_sstk_load(src + min(lane + 64u * j, n - 1u));
    }
}
HH_DEV float hh_sstk_value(uint64_t t) { return __uint_as_float((uint32_t)t); }

// Sum over an aligned team of TEAM lanes (16, 32 or 64) by DPP: every lane of the team's
// last row of 16 lanes holds the team's sum (hh_sstk_result_row).
template <int TEAM>
HH_DEV float hh_sstk_team_sum(float v) {
    v += hh_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += hh_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += hh_dpp<0x124>(v);  // row_ror:4
    v += hh_dpp<0x128>(v);  // row_ror:8: every lane holds its row's sum
    if (TEAM >= 32) v += hh_dpp<0x142, 0xA>(v);  // row_bcast:15: rows 1, 3 add rows 0, 2
    if (TEAM >= 64) v += hh_dpp<0x143, 0xC>(v);  // row_bcast:31: row 3 adds rows 0 + 1
    return v;
}
template <int TEAM>
HH_DEV bool hh_sstk_result_row(uint32_t lane) {
    const uint32_t row = (lane >> 4) & 3u;
    return TEAM == 16 ? true : (TEAM == 32 ? (row & 1u) != 0 : row == 3u);
}

// Q: the block format; TEAM1 / TEAM2 lanes per gate/up / down row (one block per lane); at
// most R rows per team and phase; K layers of weights in flight per compute thread.  A
// compute wave's memory operations in flight (R * 5 row loads and R * 3 stores per layer,
// times K) stay well under the 63 its counter tracks.
template <class Q, int TEAM1, int TEAM2, int R, int K>
HH_DEV void hh_sstk_body(const hh_sstk_args& a) {
    __shared__ float xraw[2][HH_SSTK_MAX];  // x_l by layer parity (the residual reads it late)
    __shared__ float xn[HH_SSTK_MAX];       // n_l
    __shared__ float hs[HH_SSTK_MAX];       // h_l
    __shared__ int s_bad;
    constexpr uint32_t TPB1 = (HH_SSTK_CW * HH_WAVE) / TEAM1, TPB2 = (HH_SSTK_CW * HH_WAVE) / TEAM2;
    constexpr int NJX = TEAM1 / 2;  // x words per exchange lane (d_model <= 32 * TEAM1)
    constexpr int NJH = TEAM2 / 2;  // h words per exchange lane (d_ff <= 32 * TEAM2)
    const uint32_t tid = threadIdx.x, lane = tid % HH_WAVE;
    const bool xw = __builtin_amdgcn_readfirstlane(tid / HH_WAVE) == HH_SSTK_CW;
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, df = a.d_ff, L = a.n_layers;
    const uint32_t r0 = (uint32_t)(((uint64_t)w * df) / G), r1 = (uint32_t)(((uint64_t)(w + 1) * df) / G);
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G), q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t l1 = tid % TEAM1, t1 = tid / TEAM1, l2 = tid % TEAM2, t2 = tid / TEAM2;
    const bool a1 = l1 < dm / Q::UNIT, a2 = l2 < df / Q::UNIT;
    unsigned* epoch_word = a.bar + HH_BAR_STACK_EPOCH;
    unsigned* err_word = a.bar + (2 * HH_BAR_GROUPS + 1) * HH_BAR_LINE;
    const uint32_t E = hh_load_agent(epoch_word);
    // The exchange wave's read of E completes before this workgroup publishes anything (the
    // compute threads' publishes depend on E through their tags).
    if (xw) hh_barrier_gen_ready(E);
    if (tid == 0) s_bad = 0;

    if (xw) {
        // The exchange wave: x_l (the input, or the previous layer's published rows), its
        // RMSNorm n_l into LDS; then h_l.  Two workgroup barriers per layer, paired with the
        // compute waves' below.  It holds norm_l (element lane + 64 j), requested a layer
        // ahead.
        float nv[NJX];
        auto load_norm = [&](uint32_t l) {
            const float* src = a.norm + (size_t)l * a.norm_stride;
#pragma unroll
            for (int j = 0; j < NJX; j++) nv[j] = src[min(lane + 64u * j, dm - 1u)];
        };
        load_norm(0);
        __syncthreads();  // s_bad
        for (uint32_t l = 0; l < L; l++) {
            const uint32_t p = l & 1u;
            bool ok = true;
            float xv[NJX];
            if (l == 0) {
#pragma unroll
                for (int j = 0; j < NJX; j++) xv[j] = a.x[min(lane + 64u * j, dm - 1u)];
            } else {
                uint64_t t[NJX];
                ok = hh_sstk_gather<NJX>(a.xx, dm, E + l, t, lane);
#pragma unroll
                for (int j = 0; j < NJX; j++) xv[j] = hh_sstk_value(t[j]);
            }
            HH_SSTK_MARK(0, lane == 0);
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NJX; j++) ss += lane + 64u * j < dm ? xv[j] * xv[j] : 0.f;
            ss = hh_wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)dm + a.eps);
#pragma unroll
            for (int j = 0; j < NJX; j++) {
                const uint32_t i = lane + 64u * j;
                if (i < dm) {
                    xraw[p][i] = xv[j];
                    xn[i] = (xv[j] * inv) * nv[j];
                }
            }
            if (l + 1 < L) load_norm(l + 1);
            if (!ok && lane == 0) {
                s_bad = 1;
                hh_store_agent(err_word, 1u);
            }
            __syncthreads();  // A: x_l and n_l are in LDS
            if (s_bad) return;
            {
                uint64_t t[NJH];
                ok = hh_sstk_gather<NJH>(a.hx, df, E + l + 1u, t, lane);
                HH_SSTK_MARK(1, lane == 0);
#pragma unroll
                for (int j = 0; j < NJH; j++)
                    if (lane + 64u * j < df) hs[lane + 64u * j] = hh_sstk_value(t[j]);
            }
            if (lane == 0) {
                if (ok && l == 0 && w == 0) hh_store_agent(epoch_word, E + L);
                if (!ok) {
                    s_bad = 1;
                    hh_store_agent(err_word, 1u);
                }
            }
            __syncthreads();  // B: h_l is in LDS
            if (s_bad) return;
        }
        return;
    }

    // The compute waves: a register ring of K layers' gate/up and down rows, each slot
    // refilled as soon as its layer has consumed it (with layer l+K, or the last layer again
    // near the end).  Every load and store is issued by every compute wave in the same order
    // whatever the shape (lanes and teams without work read row r0 / q0 and unit 0, and store
    // to the workgroup's own spare line), so the wait counts are static and a wait for slot
    // s never waits for the loads issued after it.
    typename Q::Data dg[K][R], du[K][R], dd[K][R];
    const uint32_t u1 = a1 ? l1 : 0u, u2 = a2 ? l2 : 0u;
    const bool res1 = hh_sstk_result_row<TEAM1>(lane), res2 = hh_sstk_result_row<TEAM2>(lane);
    uint64_t* const spare = a.spare + 16u * w;
    auto issue_gu = [&](uint32_t l, int s) {
        const uint8_t* base = a.pack + (size_t)l * a.stride;
#pragma unroll
        for (int k = 0; k < R; k++) {
            const uint32_t row = r0 + t1 + k * TPB1;
            const uint32_t rr = row < r1 ? row : r0;
            dg[s][k] = Q::load(base + a.off_g + (size_t)rr * a.rb_in, u1);
            du[s][k] = Q::load(base + a.off_u + (size_t)rr * a.rb_in, u1);
        }
    };
    auto issue_dn = [&](uint32_t l, int s) {
        const uint8_t* base = a.pack + (size_t)l * a.stride + a.off_d;
#pragma unroll
        for (int k = 0; k < R; k++) {
            const uint32_t row = q0 + t2 + k * TPB2;
            dd[s][k] = Q::load(base + (size_t)(row < q1 ? row : q0) * a.rb_ff, u2);
        }
    };
#pragma unroll
    for (int s = 0; s < K; s++) {
        const uint32_t ls = min((uint32_t)s, L - 1u);
        issue_gu(ls, s);
        issue_dn(ls, s);
    }
    __syncthreads();  // s_bad

    // One layer on ring slot s (a constant after unrolling); false when the workgroup must
    // leave (an exchange timed out).
    auto layer = [&](uint32_t l, int s) -> bool {
        const uint32_t p = l & 1u;
        const uint32_t next = min(l + K, L - 1u);
        __syncthreads();  // A
        HH_SSTK_MARK(2, tid == 0);
        if (s_bad) return false;
        {
            typename Q::X xr;
            Q::load_x(xn, u1, xr);
#pragma unroll
            for (int k = 0; k < R; k++) {
                const uint32_t row = r0 + t1 + k * TPB1;
                const float g = hh_sstk_team_sum<TEAM1>(a1 ? Q::dot(dg[s][k], xr, u1, nullptr) : 0.f);
                const float u = hh_sstk_team_sum<TEAM1>(a1 ? Q::dot(du[s][k], xr, u1, nullptr) : 0.f);
                hh_sstk_publish(res1 && row < r1 ? a.hx + row : spare, hh_act_mul(g, u, a.act), E + l + 1u);
            }
        }
        HH_SSTK_MARK(3, tid == 0);
        issue_gu(next, s);
        __syncthreads();  // B
        HH_SSTK_MARK(4, tid == 0);
        if (s_bad) return false;
        {
            typename Q::X hr;
            Q::load_x(hs, u2, hr);
#pragma unroll
            for (int k = 0; k < R; k++) {
                const uint32_t row = q0 + t2 + k * TPB2;
                const bool own = res2 && row < q1;
                const float v = hh_sstk_team_sum<TEAM2>(a2 ? Q::dot(dd[s][k], hr, u2, nullptr) : 0.f);
                const float yv = xraw[p][row < q1 ? row : q0] + v;
                hh_sstk_publish(own ? a.xx + row : spare, yv, E + l + 1u);
                float* yd = (own && l + 1 == L) ? a.y + row : reinterpret_cast<float*>(spare + 1);
                *yd = yv;
            }
        }
        HH_SSTK_MARK(5, tid == 0);
        issue_dn(next, s);
        return true;
    };
    // Whole rings of K layers, then the last L % K: no exit inside the unrolled ring, so its
    // wait counts stay exact.
    uint32_t l0 = 0;
    for (; l0 + K <= L; l0 += K) {
#pragma unroll
        for (int s = 0; s < K; s++)
            if (!layer(l0 + (uint32_t)s, s)) return;
    }
#pragma unroll
    for (int s = 0; s < K - 1; s++)
        if (l0 + (uint32_t)s < L && !layer(l0 + (uint32_t)s, s)) return;
}

#define HH_SSTK(NAME, Q, T1, T2, R, K)                                                                    \
    extern "C" __global__ void __launch_bounds__(HH_SSTK_BLOCK)                                           \
        hh_sstk_##NAME##_t##T1##_##T2##_r##R(const hh_sstk_args a) {                                      \
        hh_sstk_body<Q, T1, T2, R, K>(a);                                                                 \
    }
#define HH_SSTK_TEAMS(NAME, Q, R, K) \
    HH_SSTK(NAME, Q, 16, 16, R, K)   \
    HH_SSTK(NAME, Q, 16, 32, R, K)   \
    HH_SSTK(NAME, Q, 16, 64, R, K)   \
    HH_SSTK(NAME, Q, 32, 16, R, K)   \
    HH_SSTK(NAME, Q, 32, 32, R, K)   \
    HH_SSTK(NAME, Q, 32, 64, R, K)   \
    HH_SSTK(NAME, Q, 64, 16, R, K)   \
    HH_SSTK(NAME, Q, 64, 32, R, K)   \
    HH_SSTK(NAME, Q, 64, 64, R, K)
HH_SSTK_TEAMS(q4_0, Q40, 1, 4)
HH_SSTK_TEAMS(q4_0, Q40, 2, 3)
HH_SSTK_TEAMS(q4_0, Q40, 3, 2)
HH_SSTK_TEAMS(q4_0, Q40, 4, 2)
HH_SSTK_TEAMS(q8_0, Q80, 1, 2)
HH_SSTK_TEAMS(q8_0, Q80, 2, 2)
