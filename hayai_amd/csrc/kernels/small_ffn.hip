// The FFN of a small model in one launch (gfx950): SmolLM2-135M's layer (d_model 576, d_ff
// 1536, Q4_0) moves 1.5 MB, so two launches spend most of their time
// waiting for their first weight loads.  Here every workgroup requests its gate/up rows, its
// down rows and its x slice at once, computes its rows of h = act(W_gate . x) * (W_up . x)
// (stream_infer.rs:3752-3808, 3836-3840), publishes them, meets the other workgroups at a
// grid barrier (one workgroup per CU: all resident; bounded wait, error word on timeout) and
// finishes its rows of y = W_down . h (:3809-3864) with the down weights already in
// registers.  Teams of TEAM1 / TEAM2 lanes per row (lane = block unit, as the team kernels of
// gemv.hip), at most two rows per team and phase.
// (Compiled after ring_common.hip in the same translation unit: the grid barrier.)

struct hh_sffn_args {
    const uint8_t* wg;
    const uint8_t* wu;
    const uint8_t* wd;
    const float* x;
    float* y;
    float* h;        // d_ff f32, written with device-scope stores before the barrier
    unsigned* bar;   // grid-barrier state (HH_BAR_WORDS words)
    uint64_t rb_in;  // row bytes of gate/up (d_model columns) and down (d_ff columns)
    uint64_t rb_ff;
    uint32_t d_model, d_ff;
    int32_t act;
    uint32_t grid;   // workgroups of the launch
};

// The kernels take what their first loads need as 14 scalar dwords, all preloaded into SGPRs
// (the host passes the raw bytes): W_gate, x, y, h and the barrier state as pointers, W_up and
// W_down as signed byte offsets from W_gate, d_model | d_ff << 16 and the grid size; act
// follows.  Row bytes follow from the shape and the format.
template <class Q, int TEAM1, int TEAM2>
HH_DEV void hh_sffn_body(const hh_sffn_args& a) {
    __shared__ int s_good;
    constexpr uint32_t TPB1 = 256 / TEAM1, TPB2 = 256 / TEAM2;
    const uint32_t tid = threadIdx.x, G = a.grid, w = blockIdx.x;
    const uint32_t dm = a.d_model, df = a.d_ff;
    const uint32_t r0 = (uint32_t)(((uint64_t)w * df) / G), r1 = (uint32_t)(((uint64_t)(w + 1) * df) / G);
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G), q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t l1 = tid % TEAM1, t1 = tid / TEAM1, l2 = tid % TEAM2, t2 = tid / TEAM2;
    const bool a1 = l1 < dm / Q::UNIT, a2 = l2 < df / Q::UNIT;

    // the barrier epoch, then every load of the launch: gate/up rows, down rows, the x slice
    const unsigned epoch = hh_barrier_epoch(a.bar);
    typename Q::Data dg[2], du[2], dd[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t row = r0 + t1 + k * TPB1;
        if (a1 && row < r1) {
            dg[k] = Q::load(a.wg + (size_t)row * a.rb_in, l1);
            du[k] = Q::load(a.wu + (size_t)row * a.rb_in, l1);
        }
        const uint32_t row2 = q0 + t2 + k * TPB2;
        if (a2 && row2 < q1) dd[k] = Q::load(a.wd + (size_t)row2 * a.rb_ff, l2);
    }
    typename Q::X xr;
    if (a1) Q::load_x(a.x, l1, xr);

#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t row = r0 + t1 + k * TPB1;
        const bool on = a1 && row < r1;
        const float g = hh_team_sum<TEAM1>(on ? Q::dot(dg[k], xr, l1, nullptr) : 0.f);
        const float u = hh_team_sum<TEAM1>(on ? Q::dot(du[k], xr, l1, nullptr) : 0.f);
        if (l1 == 0 && row < r1) hh_store_agent(reinterpret_cast<unsigned*>(a.h + row), __float_as_uint(hh_act_mul(g, u, a.act)));
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's h stores are complete
    __syncthreads();
    if (tid == 0) {
        hh_barrier_arrive(a.bar, epoch + 1u);
        s_good = hh_barrier_wait(a.bar, epoch + 1u) ? 1 : 0;
    }
    __syncthreads();
    if (!s_good) return;  // timed out: the error word is set, y is not written

    // h: plain loads (no cache of this launch holds its lines: h is first read here, and each
    // launch starts with the caches invalidated)
    typename Q::X hr;
    if (a2) Q::load_x(a.h, l2, hr);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t row = q0 + t2 + k * TPB2;
        const bool on = a2 && row < q1;
        const float v = hh_team_sum<TEAM2>(on ? Q::dot(dd[k], hr, l2, nullptr) : 0.f);
        if (l2 == 0 && row < q1) a.y[row] = v;
    }
}

#define HH_SFFN(NAME, Q, T1, T2)                                                                        \
    extern "C" __global__ void __launch_bounds__(256) hh_sffn_##NAME##_t##T1##_##T2(                   \
        const uint8_t* wg, const float* x, float* y, float* h, unsigned* bar, int32_t du, int32_t dd,    \
        uint32_t dims, uint32_t grid, int32_t act) {                                                     \
        const uint32_t dm = dims & 0xFFFFu, df = dims >> 16;                                             \
        hh_sffn_body<Q, T1, T2>(hh_sffn_args{wg, wg + du, wg + dd, x, y, h, bar,                         \
                                             (uint64_t)(dm / Q::BLOCK) * Q::BLOCK_BYTES,                 \
                                             (uint64_t)(df / Q::BLOCK) * Q::BLOCK_BYTES, dm, df, act, grid}); \
    }
#define HH_SFFN_TEAMS(NAME, Q)  \
    HH_SFFN(NAME, Q, 16, 16)    \
    HH_SFFN(NAME, Q, 16, 32)    \
    HH_SFFN(NAME, Q, 16, 64)    \
    HH_SFFN(NAME, Q, 32, 16)    \
    HH_SFFN(NAME, Q, 32, 32)    \
    HH_SFFN(NAME, Q, 32, 64)    \
    HH_SFFN(NAME, Q, 64, 16)    \
    HH_SFFN(NAME, Q, 64, 32)    \
    HH_SFFN(NAME, Q, 64, 64)
HH_SFFN_TEAMS(q4_0, Q40)
HH_SFFN_TEAMS(q8_0, Q80)
