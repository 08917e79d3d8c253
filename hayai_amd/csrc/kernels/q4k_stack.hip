// Consecutive Q4_K FFN residual blocks of one token in one persistent launch (gfx950), for
// layers whose down share fits a CU's LDS (the Llama-3-8B shape: d_model 4096, d_ff 14336):
//   x_{l+1} = x_l + W_down,l . (act(W_gate,l . n_l) * (W_up,l . n_l)),
//   n_l = x_l * (1 / sqrt(mean(x_l^2) + eps)) * norm_l,
// the ffn_apply of crates/hayai-core/src/hybrid_infer.rs:883-936 (rms_norm of
// crates/hayai-cpu/src/attention.rs:142-147; the FFN of stream_infer.rs:3752-3864) applied
// layer after layer, y = x_L.
//
// Why one launch: a layer's 99 MB stream in one launch is ~17.5 us at best and two launches
// ~19.7 us, because every launch and every dependent hop (x -> gate/up, h -> down) leaves HBM
// idle for a few microseconds.  Here the weight stream never waits for a dependency: the
// weights do not depend on x, so
//   - the gate/up ring (the ring kernels' register ring: one 64-column unit of one row per
//     lane and item, D items per wave) runs on from one layer into the next: while a layer
//     exchanges h, computes down and exchanges x, the next layer's first D items per wave
//     are already in flight;
//   - each workgroup's share of W_down (its d_model/G rows, contiguous in the pack) is copied
//     into LDS by a DMA wave (global -> LDS, no registers) while gate/up streams, and the
//     next layer's share as soon as down has read this one, so down itself reads no HBM and
//     the x exchange overlaps that copy;
//   - exchanges carry their own validity (small_stack.hip): every word is published by one
//     device-coherent 64-bit store with a tag in its top bits, and readers poll until every
//     tag is this layer's.  h travels as its int8 digits: per 8-row granule three words of
//     48 payload bits (q1[8] | q2[8] | bf16 scale) and a 16-bit tag; x as f32 words with a
//     32-bit tag.
//
// Waves: 8 compute waves (gate/up ring, the h epilogue, down from LDS, y), HH_QSTK_XW
// exchange waves (gather x -> digits of x * norm in LDS; gather h -> LDS) and one DMA wave.
// Each kind has its own load counter, so no wait for a poll waits behind a weight load or
// the other way round.  Four workgroup barriers per layer:
//   A: x_l's digits (and the residual rows, sum(x_l^2)) in LDS
//   B: gate/up row sums in LDS          (gate/up loop done)
//   C: h_l's digits and W_down,l's share in LDS
//   E: down's row partials in LDS       (W_down,l's share and h_l free again)
// then y = residual + partials is published as x_{l+1}.
//
// Digits of h: scale = amax/127 of the granule rounded up to a bf16 (so the LDS copy is
// exact and every |digit| <= 127), q1 = rint(h/scale), q2 = rint((h - q1 scale) 256/scale);
// the down dot is the ring kernels' (prefix-summed granule partials, v_dot4).
//
// Tags: the launch reads its epoch E (a word of the grid-barrier state that only this kernel
// advances, by the layer count per launch) before it publishes anything;
// layer l publishes h_l and x_{l+1} with tag 2(E + l) + 1 (odd: the zeroed buffers never
// match; the h words keep its low 16 bits, which still differ from the previous write's).
// Workgroup 0 stores E + L once it has seen every workgroup's h of layer 0.  Single exchange
// buffers suffice: a workgroup overwrites its h words of layer l+1 only after it has all of
// x_{l+1}, each row published after its producer read all of h_l; the same holds for x.
//
// Waits are bounded (~2^20 polls, or earlier once another workgroup has recorded the error
// word): the wave records the error word, every wave of the workgroup leaves after the next
// workgroup barrier, and the other workgroups time out the same way.
// (Compiled after q4k_ffn.hip and small_stack.hip: digit helpers, grid-barrier state.)

#define HH_QSTK_CW 8  // compute waves
#define HH_QSTK_XW 3  // exchange waves
#define HH_QSTK_WAVES (HH_QSTK_CW + HH_QSTK_XW + 1)
#define HH_QSTK_BLOCK (HH_QSTK_WAVES * HH_WAVE)
#define HH_QSTK_GT 14  // h words per exchange thread and gather pass
#define HH_QSTK_NXW ((4096 / HH_QSTK_XW + 32 + 63) / 64)  // x words per exchange lane (d_model <= 4096)
// Exchange buffers are padded so that every lane's gather loads stay inside them without
// clamping: h to a whole number of passes, x by one wave's reach past d_model.
#define HH_QSTK_HPAD(w) (((w) + HH_QSTK_XW * 64 * HH_QSTK_GT - 1) / (HH_QSTK_XW * 64 * HH_QSTK_GT) * (HH_QSTK_XW * 64 * HH_QSTK_GT))
#define HH_QSTK_XPAD(n) ((n) + 64 * HH_QSTK_NXW)

struct hh_qstk_args {
    const uint8_t* pack;  // layer 0's pack; layer l at pack + l * stride
    const float* norm;    // layer 0's norm; layer l at norm + l * norm_stride
    const float* x;       // x_0, 16-byte aligned
    float* y;             // x_L (may be x)
    uint64_t* hx;         // 3 * d_ff / 8 words: h granules (padded: HH_QSTK_HPAD)
    uint64_t* xx;         // d_model words: x_{l+1} (padded: HH_QSTK_XPAD)
    unsigned* bar;        // grid-barrier state (the stack epoch word, the error word)
    uint64_t stride;
    uint64_t off_g, off_u, off_d;
    uint64_t rb1, rb2;      // row bytes of gate/up (d_model columns) and down (d_ff columns)
    uint32_t norm_stride;   // floats
    uint32_t d_model, d_ff, n_layers;
    uint32_t lds_wd, lds_hx;  // LDS bytes of the W_down share and of the x / h digit region
    float eps;
    int32_t act;
};

#define HH_BAR_QSTK_EPOCH (HH_BAR_STACK_EPOCH + 1)

#ifdef HH_QSTK_TRACE
// Timeline build only: s_memrealtime (100 MHz) per workgroup, layer and event: 0 compute
// waves pass A, 1 end the gate/up loop, 2 pass B, 3 pass C, 4 pass E; 5 exchange waves have
// h_l, 6 have x_{l+1}; 7 the DMA wave's share has landed; 8 the compute waves end down, 9
// have h's digits in registers (csrc/trace/q4k_stack_timeline.cpp reads them).
__device__ uint64_t hh_qstk_trace[256][64][10];
#define HH_QSTK_MARK(ev, cond) \
    do { if ((cond) && w < 256 && l < 64) hh_qstk_trace[w][l][ev] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define HH_QSTK_MARK(ev, cond) do { } while (0)
#endif

// The workgroup's failure flag, a static LDS word (a ds_read: reading it never waits for the
// wave's outstanding global loads), read after a barrier.
HH_DEV int* hh_qstk_flag() {
    __shared__ int f;
    return &f;
}
HH_DEV int hh_qstk_bad(const int*) { return *hh_qstk_flag(); }

// A workgroup barrier for the DMA wave: no release fence, so its global->LDS copies stay in
// flight across it (an acquire keeps later LDS reads after it).
HH_DEV void hh_qstk_barrier_nowait() {
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

HH_DEV uint64_t hh_qstk_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
HH_DEV void hh_qstk_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// amax / 127 rounded up to a bf16 (positive, finite inputs)
HH_DEV float hh_qstk_scale(float amax) {
    uint32_t b = __float_as_uint(amax * (1.0f / 127.0f));
    if (b & 0xFFFFu) b = (b & 0xFFFF0000u) + 0x10000u;
    return __uint_as_float(b);
}

// The h digits of a lane's down unit u (64 columns = granules 8u..8u+7) with bf16 granule
// scales: hh_ffnp_load_h's fields, the scales widened from bf16.
HH_DEV void hh_qstk_load_h(const int8_t* q1, const int8_t* q2, const uint16_t* sc16, uint32_t u, hh_ffnp_h& h) {
    const uint4* a = reinterpret_cast<const uint4*>(q1 + (size_t)u * 64);
    const uint4* b = reinterpret_cast<const uint4*>(q2 + (size_t)u * 64);
    hh_unpack4(a[0], h.q1lo);
    hh_unpack4(a[1], h.q1lo + 4);
    hh_unpack4(a[2], h.q1hi);
    hh_unpack4(a[3], h.q1hi + 4);
    hh_unpack4(b[0], h.q2lo);
    hh_unpack4(b[1], h.q2lo + 4);
    hh_unpack4(b[2], h.q2hi);
    hh_unpack4(b[3], h.q2hi + 4);
    const uint4 s = reinterpret_cast<const uint4*>(sc16)[u];
    const float slo[4] = {__uint_as_float(s.x << 16), __uint_as_float(s.x & 0xFFFF0000u), __uint_as_float(s.y << 16),
                          __uint_as_float(s.y & 0xFFFF0000u)};
    const float shi[4] = {__uint_as_float(s.z << 16), __uint_as_float(s.z & 0xFFFF0000u), __uint_as_float(s.w << 16),
                          __uint_as_float(s.w & 0xFFFF0000u)};
    const float k = 1.0f / 256.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h.wlo[i] = (slo[i] - (i < 3 ? slo[i + 1] : 0.f)) * k;
        h.whi[i] = (shi[i] - (i < 3 ? shi[i + 1] : 0.f)) * k;
    }
    h.xlo = hh_ffnp_sub_sum(h.q1lo, h.q2lo, slo);
    h.xhi = hh_ffnp_sub_sum(h.q1hi, h.q2hi, shi);
    const uint32_t g = u & 3u;
    const uint32_t kk = 2u * (g & 1u);
    h.sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    h.sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    h.hi_form = g >= 2;
}

// WPT2 compute waves per down row (d_ff <= 4096 * WPT2), ring depth D, at most T 1 KB copies
// of the DMA wave in flight; one wave per gate/up row (d_model <= 4096), at most 16 down rows
// per workgroup.
template <int WPT2, int D, int T>
HH_DEV void hh_qstk_body(const hh_qstk_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    constexpr uint32_t TPW1 = HH_QSTK_CW;  // gate/up teams (one wave each)
    constexpr uint32_t TEAM2 = WPT2 * HH_WAVE, TPW2 = HH_QSTK_CW / WPT2;
    constexpr uint32_t XT = HH_QSTK_XW * HH_WAVE;  // exchange threads
    const uint32_t tid = threadIdx.x, lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t dm = a.d_model, df = a.d_ff, L = a.n_layers;
    const uint32_t NG = df / 8;
    const uint32_t r0 = 8u * (uint32_t)(((uint64_t)w * NG) / G), r1 = 8u * (uint32_t)(((uint64_t)(w + 1) * NG) / G);
    const uint32_t RR = 2u * (r1 - r0);  // row reads: (gate, up) of each row
    const uint32_t q0 = (uint32_t)(((uint64_t)w * dm) / G), q1 = (uint32_t)(((uint64_t)(w + 1) * dm) / G);
    const uint32_t nrow = q1 - q0;
    const uint32_t n1 = (RR + TPW1 - 1) / TPW1;
    const uint32_t n1p = (n1 + D - 1) / D * D;
    const uint32_t nrow_max = (dm + G - 1) / G;

    // LDS (dynamic): [W_down share][x digits | h digits][gate/up row sums][down partials]
    // [sum(x^2) per exchange wave][residual rows x 2]; the failure flag is static
    char* const wdl = hh_smem;
    char* const hxl = hh_smem + a.lds_wd;
    hh_digits_ptr xd;
    xd.q1 = reinterpret_cast<int8_t*>(hxl);
    xd.q2 = xd.q1 + dm;
    xd.sc = reinterpret_cast<float*>(xd.q2 + dm);
    xd.sum = xd.sc + dm / 32;
    int8_t* const hq1 = reinterpret_cast<int8_t*>(hxl);
    int8_t* const hq2 = hq1 + df;
    uint16_t* const hsc = reinterpret_cast<uint16_t*>(hq2 + df);
    float* const gu = reinterpret_cast<float*>(hxl + a.lds_hx);                          // [RR]
    float* const part = gu + ((2u * 8u * ((NG + G - 1) / G) + 3u) & ~3u);                // [nrow][WPT2]
    float* const red = part + ((nrow_max * WPT2 + 3u) & ~3u);                            // [XW]
    float* const xres = red + ((HH_QSTK_XW + 3u) & ~3u);                                 // [2][nrow_max]
    int* const s_bad = hh_qstk_flag();

    unsigned* const epoch_word = a.bar + HH_BAR_QSTK_EPOCH;
    unsigned* const err_word = a.bar + (2 * HH_BAR_GROUPS + 1) * HH_BAR_LINE;
    const uint32_t E = hh_load_agent(epoch_word);
    if (tid == 0) *s_bad = 0;

    if (wave < HH_QSTK_CW) {
        // ---------------------------------------------------------------- compute waves
        const uint32_t team1 = wave;
        const bool act1 = lane < dm / 64u;
        const uint32_t u1 = act1 ? lane : 0u;
        const uint32_t oh1 = (u1 >> 2) * 144u, oq1 = oh1 + 16u + (u1 & 3u) * 32u;
        const uint32_t team2 = wave / WPT2, lane2 = tid % TEAM2;
        const bool act2 = lane2 < df / 64u;
        const uint32_t u2 = act2 ? lane2 : 0u;
        const uint32_t oh2 = (u2 >> 2) * 144u, oq2 = oh2 + 16u + (u2 & 3u) * 32u;
        // gate/up item j of layer ll: row read i = team1 + j * TPW1 (gate and up rows
        // interleaved); padding items and layers past the last re-read an earlier row
        auto issue = [&](uint32_t ll, uint32_t j, hh_q4k_data& s) {
            const uint8_t* base = a.pack + (size_t)min(ll, L - 1u) * a.stride;
            const uint32_t i = team1 + j * TPW1;
            const uint32_t ii = i < RR ? i : 0u;
            const uint8_t* row = base + ((ii & 1u) ? a.off_u : a.off_g) + (size_t)(r0 + (ii >> 1)) * a.rb1;
            s.h = hh_ld16(row + oh1);
            s.q0 = hh_ld16(row + oq1);
            s.q1 = hh_ld16(row + oq1 + 16);
        };
        hh_q4k_data ring[D];
#pragma unroll
        for (int s = 0; s < D; s++) issue(0u, (uint32_t)s, ring[s]);
        __syncthreads();  // P: the flag is initialized

        for (uint32_t l = 0; l < L; l++) {
            const uint32_t tag = 2u * (E + l) + 1u;
            __syncthreads();  // A: x_l's digits are in LDS
            if (hh_qstk_bad(s_bad)) return;
            HH_QSTK_MARK(0, tid == 0);
            {
                hh_q4k_x xr;
                hh_q4k_load_lane_x(xd, u1, xr);
                for (uint32_t j0 = 0; j0 < n1p; j0 += D) {
#pragma unroll
                    for (int s = 0; s < D; s++) {
                        const uint32_t j = j0 + (uint32_t)s;
                        const uint32_t i = team1 + j * TPW1;
                        if (i < RR) {  // wave-uniform
                            float v = hh_q4k_unit(ring[s], xr);
                            v = hh_wave_sum(act1 ? v : 0.f);
                            if (lane == 0) gu[i] = v;
                        }
                        const uint32_t jn = j + D;  // the next item: this layer's, or the next layer's
                        const bool same = jn < n1p;
                        issue(same ? l : l + 1u, same ? jn : jn - n1p, ring[s]);
                    }
                }
            }
            HH_QSTK_MARK(1, lane == 0);  // the last wave to finish leaves the stamp
            __syncthreads();  // B: row sums are in LDS
            HH_QSTK_MARK(2, tid == 0);
            {
                // h = act(g) * u of the workgroup's rows, one thread per row; digits per
                // granule of 8 (the granule's max by DPP); the granule's first lane publishes
                // its three words
                float tot = 0.f;
#pragma unroll
                for (int k = 0; k < HH_QSTK_XW; k++) tot += red[k];
                const float inv = 1.0f / sqrtf(tot / (float)dm + a.eps);
                for (uint32_t rho0 = 0; rho0 < r1 - r0; rho0 += HH_QSTK_CW * HH_WAVE) {
                    const uint32_t rho = rho0 + tid;
                    const bool ok = rho < r1 - r0;  // granule-aligned: whole 8-lane groups agree
                    float hv = 0.f;
                    if (ok) hv = hh_act_mul(gu[2 * rho] * inv, gu[2 * rho + 1] * inv, a.act);
                    float amax = fabsf(hv);
                    amax = fmaxf(amax, hh_dpp<0xB1>(amax));   // quad_perm [1,0,3,2]
                    amax = fmaxf(amax, hh_dpp<0x4E>(amax));   // quad_perm [2,3,0,1]
                    amax = fmaxf(amax, hh_dpp<0x141>(amax));  // row_half_mirror: the other quad of the 8
                    const float scale = hh_qstk_scale(amax);
                    const float rinv = amax > 0.f ? 1.0f / scale : 0.f;
                    const float d1 = fminf(fmaxf(rintf(hv * rinv), -127.f), 127.f);
                    const float rr = hv - d1 * scale;
                    const float d2 = fminf(fmaxf(rintf(rr * rinv * 256.0f), -127.f), 127.f);
                    const uint32_t p = ((uint32_t)(int)d1 & 0xFFu) | (((uint32_t)(int)d2 & 0xFFu) << 8);
                    uint64_t Q1 = p & 0xFFu, Q2 = p >> 8;
#pragma unroll
                    for (int k = 1; k < 8; k++) {
                        const uint32_t pk = (uint32_t)__shfl((int)p, (int)(lane + (uint32_t)k), HH_WAVE);
                        Q1 |= (uint64_t)(pk & 0xFFu) << (8 * k);
                        Q2 |= (uint64_t)(pk >> 8) << (8 * k);
                    }
                    if (ok && (lane & 7u) == 0) {
                        const uint32_t g = (r0 + rho) / 8u;
                        const uint64_t TG = (uint64_t)(tag & 0xFFFFu) << 48;
                        const uint64_t S = __float_as_uint(scale) >> 16;
                        hh_qstk_store(a.hx + 3u * g, (Q1 & 0xFFFFFFFFFFFFull) | TG);
                        hh_qstk_store(a.hx + 3u * g + 1u, (Q1 >> 48) | ((Q2 & 0xFFFFFFFFull) << 16) | TG);
                        hh_qstk_store(a.hx + 3u * g + 2u, (Q2 >> 32) | (S << 32) | TG);
                    }
                }
            }
            __syncthreads();  // C: h_l and W_down,l's share are in LDS
            if (hh_qstk_bad(s_bad)) return;
            HH_QSTK_MARK(3, tid == 0);
            {
                // the team's rows (at most RPT) two at a time: their LDS reads issued together,
                // then the dots, then the wave sums of all of them (independent DPP chains)
                hh_ffnp_h hr;
                hh_qstk_load_h(hq1, hq2, hsc, u2, hr);
                HH_QSTK_MARK(9, lane == 0);  // h digits in registers
                constexpr int RPT = 16 / (int)TPW2;
                float v[RPT];
#pragma unroll
                for (int k0 = 0; k0 < RPT; k0 += 2) {
                    hh_q4k_data dd[2];
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const uint32_t rl = min(team2 + (uint32_t)(k0 + k) * TPW2, nrow - 1u);
                        const char* rowp = wdl + (size_t)rl * a.rb2;
                        dd[k].h = *reinterpret_cast<const uint4*>(rowp + oh2);
                        dd[k].q0 = *reinterpret_cast<const uint4*>(rowp + oq2);
                        dd[k].q1 = *reinterpret_cast<const uint4*>(rowp + oq2 + 16);
                    }
#pragma unroll
                    for (int k = 0; k < 2; k++) v[k0 + k] = act2 ? hh_ffnp_unit_g8(dd[k], hr) : 0.f;
                }
#pragma unroll
                for (int k = 0; k < RPT; k++) v[k] = hh_wave_sum(v[k]);
                if (lane == 0) {
#pragma unroll
                    for (int k = 0; k < RPT; k++) {
                        const uint32_t rl = team2 + (uint32_t)k * TPW2;
                        if (rl < nrow) part[rl * WPT2 + wave % WPT2] = v[k];
                    }
                }
            }
            HH_QSTK_MARK(8, lane == 0);  // the last compute wave to end down leaves the stamp
            __syncthreads();  // E: down partials are in LDS
            HH_QSTK_MARK(4, tid == 0);
            if (tid < nrow) {
                float s = 0.f;
#pragma unroll
                for (int k = 0; k < WPT2; k++) s += part[tid * WPT2 + k];
                const float yv = xres[(l & 1u) * nrow_max + tid] + s;
                hh_qstk_store(a.xx + q0 + tid, ((uint64_t)tag << 32) | __float_as_uint(yv));
                if (l + 1u == L) a.y[q0 + tid] = yv;
            }
        }
        return;
    }

    if (wave == HH_QSTK_CW + HH_QSTK_XW) {
        // ---------------------------------------------------------------- the DMA wave
        // W_down,l's share (rows q0..q1, contiguous) -> LDS, 1 KB per instruction, every
        // chunk in flight at once (the load counter bounds the issue)
        const uint32_t bytes = nrow * (uint32_t)a.rb2;
        auto dma = [&](uint32_t l) {
            const uint8_t* src = a.pack + (size_t)l * a.stride + a.off_d + (size_t)q0 * a.rb2;
            for (uint32_t c0 = 0; c0 < bytes; c0 += 1024u) {
                const uint32_t off = c0 + lane * 16u;
                if (off < bytes)
                    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + off),
                                                     (__attribute__((address_space(3))) void*)(wdl + c0), 16, 0, 0);
                // at most T copies in flight: a deep burst would queue every exchange's
                // requests behind it
                if constexpr (T < 63) __builtin_amdgcn_s_waitcnt(((T >> 4) << 14) | 0x0F70 | (T & 15));
            }
        };
        dma(0u);
        hh_qstk_barrier_nowait();  // P
        for (uint32_t l = 0; l < L; l++) {
            hh_qstk_barrier_nowait();  // A (the copy stays in flight)
            if (hh_qstk_bad(s_bad)) return;
            hh_qstk_barrier_nowait();  // B
            __builtin_amdgcn_s_waitcnt(0);  // W_down,l's share has landed in LDS
            HH_QSTK_MARK(7, lane == 0);
            __syncthreads();                // C
            if (hh_qstk_bad(s_bad)) return;
            __syncthreads();  // E: down has read the share
            if (l + 1u < L) dma(l + 1u);
        }
        return;
    }

    // -------------------------------------------------------------------- exchange waves
    const uint32_t xt = tid - HH_QSTK_CW * HH_WAVE;  // 0 .. XT-1
    const uint32_t xw = wave - HH_QSTK_CW;
    // Bounded poll of tagged words: ok stays true while no wait timed out; a wait also ends
    // early once another workgroup has recorded the error word.
    auto bad_now = [&](uint32_t spins) -> bool {
        if (spins > (1u << 20)) return true;
        if ((spins & 255u) == 255u && hh_load_agent(err_word) != 0u) return true;
        return false;
    };
    // x_l (l == 0: the input; else the published words) -> digits of x * norm_l in LDS,
    // the residual rows, this wave's sum(x^2).  Exchange wave xw owns the elements
    // [s0, s1) (a multiple of 32 long): its lanes read consecutive words (one instruction
    // covers 64 words, 8 cache lines), stage the values in LDS (xraw, beside the digits) and
    // then form the digits of their own 8-element chunks; only this wave reads what it
    // staged, so a wave barrier orders it.
    const uint32_t SX = ((dm + HH_QSTK_XW * 32u - 1u) / (HH_QSTK_XW * 32u)) * 32u;
    const uint32_t s0 = min(xw * SX, dm), s1 = min(s0 + SX, dm);
    float* const xraw = reinterpret_cast<float*>(hxl + ((2u * dm + (dm / 32u) * 8u + 15u) & ~15u));
    auto take_x = [&](uint32_t l) -> bool {
        const uint32_t tag = 2u * (E + l - 1u) + 1u;  // published by layer l - 1
        const float4* n4 = reinterpret_cast<const float4*>(a.norm + (size_t)l * a.norm_stride);
        bool ok = true;
        constexpr int NXW = HH_QSTK_NXW;
        constexpr int NCI = (NXW * 64 / 8 + 63) / 64;              // 8-element chunks per lane
        float4 nw[NCI][2];  // norm_l of this lane's chunks, requested before x
#pragma unroll
        for (int i = 0; i < NCI; i++) {
            const uint32_t c = s0 / 8u + lane + 64u * (uint32_t)i;
            const uint32_t cc = c < s1 / 8u ? c : s0 / 8u;
            nw[i][0] = n4[2 * cc];
            nw[i][1] = n4[2 * cc + 1];
        }
        if (l == 0) {
            for (uint32_t e = s0 + lane; e < s1; e += HH_WAVE) xraw[e] = a.x[e];
        } else {
            uint64_t t[NXW];
            const uint64_t* xb = a.xx + s0 + lane;
#pragma unroll
            for (int k = 0; k < NXW; k++) t[k] = hh_qstk_load(xb + 64u * (uint32_t)k);
            for (uint32_t spins = 0;; spins++) {
                bool stale = false;
#pragma unroll
                for (int k = 0; k < NXW; k++) stale |= s0 + lane + 64u * (uint32_t)k < s1 && (uint32_t)(t[k] >> 32) != tag;
                if (__ballot(stale) == 0) break;  // wave-uniform
                if (bad_now(spins)) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int k = 0; k < NXW; k++)
                    if ((uint32_t)(t[k] >> 32) != tag) t[k] = hh_qstk_load(xb + 64u * (uint32_t)k);
            }
#pragma unroll
            for (int k = 0; k < NXW; k++) {
                const uint32_t e = s0 + lane + 64u * (uint32_t)k;
                if (e < s1) xraw[e] = __uint_as_float((uint32_t)t[k]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the staged values are in LDS
        __builtin_amdgcn_wave_barrier();
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NCI; i++) {
            const uint32_t c = s0 / 8u + lane + 64u * (uint32_t)i;
            const bool has = c < s1 / 8u;
            const uint32_t cc = has ? c : s0 / 8u;
            float4 v0 = reinterpret_cast<const float4*>(xraw)[2 * cc];
            float4 v1 = reinterpret_cast<const float4*>(xraw)[2 * cc + 1];
            if (has) {
                ss += hh_sq8(v0, v1);
                if (8u * c + 8u > q0 && 8u * c < q1) {
                    const float xs[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const uint32_t r = 8u * c + (uint32_t)e;
                        if (r >= q0 && r < q1) xres[(l & 1u) * nrow_max + (r - q0)] = xs[e];
                    }
                }
            }
            hh_norm8(v0, v1, nw[i][0], nw[i][1], 1.f);
            hh_ffnp_digits_chunk(v0, v1, c, has, xd);  // every quad lane executes it
        }
        ss = hh_wave_sum(ss);
        if (lane == 0) red[xw] = ss;
        return ok;
    };
    // h_l's words -> digits in LDS (granule g: q1 at 8g, q2 at d_ff + 8g, bf16 scale at g).
    // Lanes read consecutive words (word j = 3g + e); each word's payload goes straight to
    // its place: e = 0: q1[0..5]; e = 1: q1[6..7], q2[0..3]; e = 2: q2[4..7], the scale.
    auto take_h = [&](uint32_t l) -> bool {
        const uint32_t tag16 = (2u * (E + l) + 1u) & 0xFFFFu;
        const uint32_t W = 3u * NG;
        bool ok = true;
        for (uint32_t jb = 0; jb < W; jb += XT * HH_QSTK_GT) {
            uint64_t t[HH_QSTK_GT];
            const uint64_t* hb = a.hx + jb + xt;
#pragma unroll
            for (int k = 0; k < HH_QSTK_GT; k++) t[k] = hh_qstk_load(hb + (uint32_t)k * XT);
            for (uint32_t spins = 0;; spins++) {
                bool stale = false;
#pragma unroll
                for (int k = 0; k < HH_QSTK_GT; k++) stale |= jb + xt + (uint32_t)k * XT < W && (uint32_t)(t[k] >> 48) != tag16;
                if (__ballot(stale) == 0) break;
                if (bad_now(spins)) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int k = 0; k < HH_QSTK_GT; k++)
                    if ((uint32_t)(t[k] >> 48) != tag16) t[k] = hh_qstk_load(hb + (uint32_t)k * XT);
            }
#pragma unroll
            for (int k = 0; k < HH_QSTK_GT; k++) {
                const uint32_t j = jb + xt + (uint32_t)k * XT;
                if (j < W) {
                    const uint32_t g = j / 3u, e = j - 3u * g;
                    const uint32_t lo = (uint32_t)t[k], mid = (uint32_t)(t[k] >> 32) & 0xFFFFu;
                    if (e == 0u) {
                        *reinterpret_cast<uint32_t*>(hq1 + 8u * g) = lo;
                        *reinterpret_cast<uint16_t*>(hq1 + 8u * g + 4u) = (uint16_t)mid;
                    } else if (e == 1u) {
                        *reinterpret_cast<uint16_t*>(hq1 + 8u * g + 6u) = (uint16_t)lo;
                        *reinterpret_cast<uint16_t*>(hq2 + 8u * g) = (uint16_t)(lo >> 16);
                        *reinterpret_cast<uint16_t*>(hq2 + 8u * g + 2u) = (uint16_t)mid;
                    } else {
                        *reinterpret_cast<uint32_t*>(hq2 + 8u * g + 4u) = lo;
                        hsc[g] = (uint16_t)mid;
                    }
                }
            }
        }
        return ok;
    };

    bool ok = take_x(0u);
    if (!ok && lane == 0) {
        *s_bad = 1;
        hh_store_agent(err_word, 1u);
    }
    __syncthreads();  // P
    for (uint32_t l = 0; l < L; l++) {
        __syncthreads();  // A
        if (hh_qstk_bad(s_bad)) return;
        __syncthreads();  // B: the compute waves have read x's digits; the region takes h
        ok = take_h(l);
        HH_QSTK_MARK(5, lane == 0);
        if (lane == 0) {
            if (!ok) {
                *s_bad = 1;
                hh_store_agent(err_word, 1u);
            }
        }
        __syncthreads();  // C
        if (hh_qstk_bad(s_bad)) return;
        if (l == 0 && w == 0 && tid == HH_QSTK_CW * HH_WAVE) hh_store_agent(epoch_word, E + L);
        __syncthreads();  // E: down has read h; the region takes x_{l+1}'s digits
        if (l + 1u < L) {
            ok = take_x(l + 1u);
            HH_QSTK_MARK(6, lane == 0);
            if (!ok && lane == 0) {
                *s_bad = 1;
                hh_store_agent(err_word, 1u);
            }
        }
    }
}

#define HH_QSTK(G2, D, T)                                                                            \
    extern "C" __global__ void __launch_bounds__(HH_QSTK_BLOCK) hh_q4k_stk_d##G2##_r##D##_t##T(const hh_qstk_args a) { \
        hh_qstk_body<G2, D, T>(a);                                                                   \
    }
HH_QSTK(2, 3, 24)
HH_QSTK(4, 3, 24)
