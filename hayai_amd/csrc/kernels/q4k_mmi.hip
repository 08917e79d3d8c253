// Batched Q4_K for 16..64 tokens per pass with int8 activations (gfx950):
//   hh_mmi_prep              tokens [b][n] f32 -> token stages (below): per 32-element block of
//                            each token s = amax / 127, q = round_half_away(x / s) clamped to
//                            +-127 (the batched path's activation quantization), zero-padded
//                            to 16 * TT tokens
//   hh_q4k_mmi_t<TT>_d<D>    Y[b][m] = W . X from those stages (ggml_gemv_batched_q4_k,
//                            crates/hayai-opencl/src/compute.rs:179-257;
//                            execute_quant_gemv_batched, crates/hayai-core/src/
//                            orchestrator.rs:240-269)
//   hh_q4k_mmi_gu_t<TT>_d<D> h = act(W_gate . X) * (W_up . X) (prefill_batched's gate/up and
//                            SiLU * up, crates/hayai-core/src/prefill_wave.rs:569-584, fused),
//                            quantized the same way and written as the token stages of the
//                            down projection
// (Compiled after mm_common.hip: its vector types, the f16 weight decode hh_mm_scq and the
// coherent partial-sum helpers.)
//
// Arithmetic.  A Q4_K weight is d sc_j q - dmin m_j for sub-block j (32 columns) and a token
// element s_tj xq, so one output is
//   sum_sb [ d * sum_j s_tj P_j  -  dmin * sum_j m_j u_tj ],  P_j = sum_k (sc_j q_k) xq_k,
//   u_tj = s_tj * sum_k xq_k.
// P_j is one v_mfma_f32_16x16x32_f16 per sub-block with A = sc_j q (integers <= 945, exact in
// f16) and B = xq (integers in [-127, 127], exact in f16): every product is an integer below
// 2^17 and every sum of 32 below 2^22, so the f32 result is exact, the same integer the int8
// matrix cores would produce, but with the 6-bit sub-block scale already inside (an int8
// operand cannot hold sc * q).  So each sub-block costs one FMA per output (P_j * s_tj) where
// the int8 form costs a convert, a multiply and an FMA (d sc_j s_tj differs per row, token
// and sub-block), and the superblock's d is applied once.  The min term is two
// v_mfma_f32_16x16x4f32 per superblock (A = -dmin m_j, B = u_tj), accumulated straight into
// the output tile.  Lane l holds output rows 4 (l/16) .. +3 of token l % 16.
//
// Token stage of one (superblock, 16-token tile), 9216 bytes; stage (sb, tt) at
// (sb * TT + tt) * 9216:
//   [0, 8192)      B fragments: sub-block j, lane l: 8 f16 at (64 j + l) * 16, the values xq
//                  of token l % 16 at superblock elements 32 j + 8 (l / 16) + e, e = 0..7
//   [8192, 8704)   s_tj f32 at (8 t + j) * 4
//   [8704, 9216)   u_tj f32 at (16 j + t) * 4
// Weights: lane (quarter c, row r) holds, for each 32-byte qs group g, bytes 8c .. 8c + 7:
// the low nibbles are elements 8c .. 8c + 7 of sub-block 2g, the high nibbles those of
// sub-block 2g + 1 (q4k.rs:178-203): the A fragment of either sub-block in the stage's order.
//
// Work split: a workgroup is 4 compute waves owning 4 consecutive 16-row units (64 rows)
// over a chunk of superblocks, plus one copy wave.  Each compute wave streams its unit's
// superblocks through a register ring of D items (per tile: the 16-byte block header and four
// 8-byte qs pieces at fixed lane offsets, so wait counts are static).  The copy wave brings the
// chunk's token stages into an LDS ring of R superblock slots by global->LDS DMA; when the
// chunk is longer than R, every superblock ends at a workgroup barrier after which the copy
// wave refills the slot just consumed (only the copy wave issues DMA, so the compute waves'
// wait counts never include it).  Gate/up takes whole rows (one chunk): its 4 units are 64
// rows, two 32-row blocks of h, so the workgroup quantizes its h itself (the pair of units of
// a block exchange their maxima and sums through LDS).  Chunks of one row group (GEMM and
// down) meet in a workspace; the last workgroup to arrive adds them in chunk order
// (deterministic).

#define HH_MMI_STAGE 9216u
#define HH_MMI_WAVES 4  // units (16 rows each) per workgroup
#define HH_MMI_LDS 147456u  // the stage ring's bytes at most

struct hh_mmi_prep_args {
    const float* x;  // [b][n] f32
    uint8_t* xs;     // [n / 256][tt] stages
    uint32_t n;
    uint32_t b;      // valid tokens
    uint32_t tt;     // 16-token tiles
    uint32_t pad;
};

// A team of 32 lanes per (token, 32-element block), one element per lane: amax and the sum
// of the quantized values by cross-lane reductions; lanes 8c then store quarter c's 8 f16.
// Tokens past b are written as zeros.
extern "C" __global__ void __launch_bounds__(256) hh_mmi_prep(const hh_mmi_prep_args a) {
    const uint32_t nb = a.n / 32;
    const uint32_t blk = blockIdx.x * 8u + threadIdx.x / 32u;  // (token, block) index
    const uint32_t e = threadIdx.x % 32u;
    if (blk >= 16u * a.tt * nb) return;  // whole 32-lane teams exit together
    const uint32_t t = blk / nb, k = blk % nb;
    const uint32_t sb = k / 8, j = k % 8, t16 = t % 16;
    uint8_t* st = a.xs + ((size_t)sb * a.tt + t / 16) * HH_MMI_STAGE;
    const float v = t < a.b ? a.x[(size_t)t * a.n + 32u * k + e] : 0.f;
    float amax = fabsf(v);
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float s = amax / 127.0f;
    float q = s > 0.f ? roundf(v / s) : 0.f;
    q = fminf(fmaxf(q, -127.f), 127.f);
    int sum = (int)q;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) sum += __shfl_xor(sum, m, 32);
    // f16 of q; lanes 2i hold elements 2i | 2i + 1 << 16, lanes 8c gather their quarter
    const uint32_t hb = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q);
    uint32_t w = (e & 1u) ? hb << 16 : hb;
    w |= __shfl_xor(w, 1, 32);
    const uint32_t w1 = __shfl_down(w, 2, 32), w2 = __shfl_down(w, 4, 32), w3 = __shfl_down(w, 6, 32);
    if ((e & 7u) == 0)
        *reinterpret_cast<uint4*>(st + (size_t)(j * 64u + (e / 8u) * 16u + t16) * 16u) = make_uint4(w, w1, w2, w3);
    if (e == 0) {
        *reinterpret_cast<float*>(st + 8192u + (t16 * 8u + j) * 4u) = s;
        *reinterpret_cast<float*>(st + 8704u + (j * 16u + t16) * 4u) = s * (float)sum;
    }
}

struct hh_mmi_args {
    const uint8_t* w0;  // GEMM: W; FFN: W_gate   [m][row_bytes]
    const uint8_t* w1;  // FFN: W_up
    const uint8_t* xs;  // token stages of the input [n / 256][TT]
    float* y;           // GEMM: Y [b][m]
    uint8_t* hs;        // FFN: token stages of h [m / 256][TT]
    float* part;        // kc > 1: [groups][kc][4 waves][TT * 4][64 lanes] partial sums
    unsigned* cnt;      // kc > 1: arrival counter per row group (zero between launches)
    uint64_t row_bytes;
    uint32_t m;         // rows (FFN: d_ff, a multiple of 256)
    uint32_t n;         // columns (multiple of 256)
    uint32_t b;         // valid tokens (<= 16 * TT)
    uint32_t kc;        // superblock chunks = workgroups per row group (FFN: 1)
    uint32_t sbc;       // superblocks per chunk
    int32_t act;
};

// -dmin * m_j of a lane's row for sub-blocks c and c + 4 (get_scale_min_k4, q4k.rs:34-43):
// the A operand of the min-term MFMA.
struct hh_mmi_head {
    float nm0, nm1;
};
HH_DEV uint32_t hh_byte(uint32_t v, uint32_t i) { return (v >> (8 * i)) & 0xFFu; }
HH_DEV void hh_mmi_mins(const uint4& h, uint32_t c, hh_mmi_head& t) {
    const float dmin = hh_f16(h.x >> 16);
    const uint32_t q[3] = {h.y, h.z, h.w};  // the 12 scale bytes
    auto qb = [&](uint32_t i) { return hh_byte(q[i >> 2], i & 3u); };
    // sub-block c < 4: m = q[c + 4] & 63; sub-block c + 4: (q[c + 8] >> 4) | ((q[c + 4] >> 6) << 4)
    const uint32_t b4 = qb(c + 4u), b8 = qb(c + 8u);
    t.nm0 = -dmin * (float)(b4 & 63u);
    t.nm1 = -dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4));
}

// A workgroup barrier for LDS traffic only: each wave waits for its own LDS accesses, not for
// its weight loads in flight (__syncthreads() would also wait for those).
HH_DEV void hh_mmi_lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited for
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt immediate for vmcnt <= n (expcnt and lgkmcnt not waited for)
constexpr int hh_mmi_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int NT, int TT, int D, bool REFILL>
HH_DEV void hh_mmi_body(const hh_mmi_args& a) {
    constexpr uint32_t NCW = HH_MMI_WAVES;  // compute waves; wave NCW copies
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];  // the stage ring
    __shared__ float xch[2][HH_MMI_WAVES][TT * 16];                  // gate/up: h block exchange
    __shared__ int last_flag;
    constexpr uint32_t SBT = HH_MMI_STAGE * TT;  // one superblock's stages: a ring slot
    constexpr uint32_t R = HH_MMI_LDS / SBT < 16 ? HH_MMI_LDS / SBT : 16;
    constexpr uint32_t CHUNKS = SBT / 1024u;     // 1 KB DMA instructions per slot
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t nsb = a.n / 256;
    const uint32_t grp = blockIdx.x / a.kc, kci = blockIdx.x % a.kc;
    const uint32_t sb0 = kci * a.sbc;
    const uint32_t ns = min(a.sbc, nsb - sb0);  // superblocks of this chunk (>= 1)
    const uint32_t nsp = (ns + D - 1) / D * D;  // padded to whole ring rounds: items past ns add nothing
    char* const slots = hh_smem;

    if (wave == NCW) {
        // copy wave: superblock k of the chunk (clamped to the last) -> its slot
        auto copy = [&](uint32_t k, uint32_t slot) {
            const uint8_t* src = a.xs + (size_t)(sb0 + min(k, ns - 1u)) * SBT + lane * 16u;
            char* dst = slots + (size_t)slot * SBT;
#pragma unroll
            for (uint32_t i = 0; i < CHUNKS; i++)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + i * 1024u),
                                                 (__attribute__((address_space(3))) void*)(dst + i * 1024u), 16, 0, 0);
        };
        if constexpr (REFILL) {
            // Slots 0 .. R-1 first; then after each item k every compute wave is done with
            // slot k % R, which takes superblock k + R (past the chunk: a copy of its last
            // superblock into a slot nobody reads again, so every step issues the same
            // copies).  Before that barrier the slot of item k + 1 has landed: every copy but
            // the last R - 2 slots' is complete.
            for (uint32_t k = 0; k < R; k++) copy(k, k);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            hh_mmi_lds_barrier();                // the first slots are in LDS
            for (uint32_t k = 0; k < nsp; k++) {
                constexpr int later = (int)((R - 2) * CHUNKS) < 63 ? (int)((R - 2) * CHUNKS) : 63;
                __builtin_amdgcn_s_waitcnt(hh_mmi_vmcnt(later));
                hh_mmi_lds_barrier();
                copy(k + R, k % R);
            }
        } else {
            // the whole chunk fits the ring
            for (uint32_t k = 0; k < ns; k++) copy(k, k);
            __builtin_amdgcn_s_waitcnt(0x0F70);
            hh_mmi_lds_barrier();
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }

    // compute waves: unit us of the group
    const uint32_t c = lane >> 4, r16 = lane & 15u;
    const uint32_t nu = (a.m + 15) / 16;
    const uint32_t us = min(wave, NCW - 1u);
    const uint32_t u0 = grp * HH_MMI_WAVES + us;
    const bool live = wave < NCW && u0 < nu;  // waves past the last unit repeat it, store nothing
    const uint32_t unit = min(u0, nu - 1);
    const uint32_t row = min(unit * 16 + r16, a.m - 1);
    const size_t lofs = (size_t)row * a.row_bytes + (size_t)sb0 * 144;
    const uint8_t* const p0 = a.w0 + lofs;
    const uint8_t* const p1 = (NT == 2 ? a.w1 : a.w0) + lofs;
    struct Item {
        uint4 h;
        uint2 q[4];
    };
    hh_f4 acc[NT][TT];
#pragma unroll
    for (int q = 0; q < NT; q++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[q][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};

    if (wave < NCW) {
        Item ring[D][NT];
        auto issue = [&](uint32_t k, Item* it) {  // items past the chunk re-read its last superblock
            const uint32_t off = min(k, ns - 1u) * 144u;
#pragma unroll
            for (int q = 0; q < NT; q++) {
                const uint8_t* p = (q ? p1 : p0) + off;
                it[q].h = hh_ld16(p);
#pragma unroll
                for (int g = 0; g < 4; g++) it[q].q[g] = *reinterpret_cast<const uint2*>(p + 16u + 32u * g + 8u * c);
            }
        };
#pragma unroll
        for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
        hh_mmi_lds_barrier();  // the first slots are in LDS

#pragma unroll 1
        for (uint32_t k0 = 0; k0 < nsp; k0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const uint32_t k = k0 + (uint32_t)s;
                const bool valid = k < ns;
                const char* st = slots + (size_t)(min(k, ns - 1u) % R) * SBT;  // padded items: any valid slot
                // the item's A operands (sc_j q for the 8 sub-blocks), d and dmin of the lane's
                // four output rows, -dmin m_j of sub-blocks c and c + 4; then the ring slot is
                // refilled at once
                hh_h8 wa[NT][8];
                float d4[NT][4];
                hh_mmi_head hd[NT];
#pragma unroll
                for (int q = 0; q < NT; q++) {
                    uint4 h = ring[s][q].h;
                    if (!valid) h.x = 0u;  // d = dmin = 0
                    const uint32_t sc03 = h.y & 0x3F3F3F3Fu;
                    const uint32_t sc47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const uint32_t b = (uint32_t)(j & 3);
                        const uint32_t sel = b | (4u << 8) | (b << 16) | (4u << 24);
                        const hh_h2 s1024 = hh_h2_bits(__builtin_amdgcn_perm(0x64646464u, j < 4 ? sc03 : sc47, sel));
                        const hh_h2 sc2 = s1024 - hh_h2{(_Float16)1024.0f, (_Float16)1024.0f};
                        const hh_h2 nb2 = sc2 * hh_h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
                        const uint2 p = ring[s][q].q[j >> 1];
                        const uint32_t lo = (j & 1) ? (p.x >> 4) & 0x0F0F0F0Fu : p.x & 0x0F0F0F0Fu;
                        const uint32_t hi = (j & 1) ? (p.y >> 4) & 0x0F0F0F0Fu : p.y & 0x0F0F0F0Fu;
                        hh_h2 r[4];
                        hh_mm_scq(lo, sc2, nb2, r);
                        hh_mm_scq(hi, sc2, nb2, r + 2);
                        wa[q][j] = hh_h8{r[0].x, r[0].y, r[1].x, r[1].y, r[2].x, r[2].y, r[3].x, r[3].y};
                    }
                    const float d = hh_f16(h.x & 0xFFFFu);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        d4[q][i] = __builtin_bit_cast(
                            float, __builtin_amdgcn_ds_bpermute((int)((c * 4u + (uint32_t)i) * 4u), __builtin_bit_cast(int, d)));
                    hh_mmi_mins(h, c, hd[q]);
                }
                __builtin_amdgcn_sched_barrier(0);
                issue(k + D, ring[s]);
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    const char* sg = st + tt * HH_MMI_STAGE;
                    const float4 sa = *reinterpret_cast<const float4*>(sg + 8192u + r16 * 32u);
                    const float4 sb = *reinterpret_cast<const float4*>(sg + 8192u + r16 * 32u + 16u);
                    const float sj[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
                    const float u0v = *reinterpret_cast<const float*>(sg + 8704u + (c * 16u + r16) * 4u);
                    const float u1v = *reinterpret_cast<const float*>(sg + 8704u + ((c + 4u) * 16u + r16) * 4u);
                    hh_f4 ps[NT];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const hh_h8 xb = *reinterpret_cast<const hh_h8*>(sg + ((uint32_t)j * 64u + lane) * 16u);
#pragma unroll
                        for (int q = 0; q < NT; q++) {
                            const hh_f4 pj = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[q][j], xb, hh_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            if (j == 0) {
#pragma unroll
                                for (int i = 0; i < 4; i++) ps[q][i] = pj[i] * sj[0];
                            } else {
#pragma unroll
                                for (int i = 0; i < 4; i++) ps[q][i] = fmaf(pj[i], sj[j], ps[q][i]);
                            }
                        }
                    }
#pragma unroll
                    for (int q = 0; q < NT; q++) {
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[q][tt][i] = fmaf(d4[q][i], ps[q][i], acc[q][tt][i]);
                        acc[q][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(hd[q].nm0, u0v, acc[q][tt], 0, 0, 0);
                        acc[q][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(hd[q].nm1, u1v, acc[q][tt], 0, 0, 0);
                    }
                }
                if constexpr (REFILL) hh_mmi_lds_barrier();  // done with this item's slot
            }
        }
    }

    // C lane (quarter c, token r16): acc[q][tt][i] is row R0 + 4c + i of token 16 tt + r16
    const uint32_t R0 = unit * 16;
    if constexpr (NT == 2) {
        // h of the unit's rows; per token the max |h| and the sum of the quantized values over
        // each 32-row block, the pair of units of a block meeting through LDS (every wave,
        // the copy wave included, passes both barriers)
        float hv[TT][4];
        int qi[TT][4];
        float am[TT];
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            am[tt] = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                hv[tt][i] = hh_act_mul(acc[0][tt][i], acc[1][tt][i], a.act);
                am[tt] = fmaxf(am[tt], fabsf(hv[tt][i]));
            }
            am[tt] = fmaxf(am[tt], __shfl_xor(am[tt], 16, HH_WAVE));
            am[tt] = fmaxf(am[tt], __shfl_xor(am[tt], 32, HH_WAVE));
        }
        const uint32_t wv = us;
        if (wave < NCW && c == 0)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) xch[0][wv][tt * 16 + r16] = am[tt];
        __syncthreads();
        float sc[TT];
        int xsum[TT];
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            sc[tt] = fmaxf(am[tt], xch[0][wv ^ 1u][tt * 16 + r16]) / 127.0f;
            xsum[tt] = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float q = sc[tt] > 0.f ? roundf(hv[tt][i] / sc[tt]) : 0.f;
                q = fminf(fmaxf(q, -127.f), 127.f);
                qi[tt][i] = (int)q;
                xsum[tt] += qi[tt][i];
            }
            xsum[tt] += __shfl_xor(xsum[tt], 16, HH_WAVE);
            xsum[tt] += __shfl_xor(xsum[tt], 32, HH_WAVE);
        }
        if (wave < NCW && c == 0)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) xch[1][wv][tt * 16 + r16] = (float)xsum[tt];
        __syncthreads();
        if (!live) return;
        // stage (sbd, tt) of the down projection: this unit is half `half` of sub-block jd;
        // lanes of even quarters gather the next quarter's four rows and store 8 consecutive
        // rows of one token (one 16-byte fragment piece)
        const uint32_t sbd = R0 / 256, jd = (R0 % 256) / 32, half = (R0 / 16) & 1u;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            uint8_t* st = a.hs + ((size_t)sbd * TT + tt) * HH_MMI_STAGE;
            auto f16b = [](int v) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v); };
            const uint32_t w0 = f16b(qi[tt][0]) | (f16b(qi[tt][1]) << 16);
            const uint32_t w1 = f16b(qi[tt][2]) | (f16b(qi[tt][3]) << 16);
            const uint32_t x0 = __shfl_xor(w0, 16, HH_WAVE), x1 = __shfl_xor(w1, 16, HH_WAVE);
            if ((c & 1u) == 0)
                *reinterpret_cast<uint4*>(st + (size_t)(jd * 64u + (2u * half + c / 2u) * 16u + r16) * 16u) =
                    make_uint4(w0, w1, x0, x1);
            if (half == 0 && c == 0) {
                const float xs = (float)(xsum[tt] + (int)xch[1][wv ^ 1u][tt * 16 + r16]);
                *reinterpret_cast<float*>(st + 8192u + (r16 * 8u + jd) * 4u) = sc[tt];
                *reinterpret_cast<float*>(st + 8704u + (jd * 16u + r16) * 4u) = sc[tt] * xs;
            }
        }
    } else {
        // partials [wave][tile][i][lane]: every store and load instruction covers 256
        // contiguous bytes
        if (a.kc > 1) {
            constexpr uint32_t PT = TT * 4u * HH_WAVE;
            const uint32_t wv = us;
            float* my = a.part + (((size_t)grp * a.kc + kci) * HH_MMI_WAVES + wv) * PT + lane;
            if (wave < NCW)
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) hh_store_coherent_f(my + (tt * 4 + i) * HH_WAVE, acc[0][tt][i]);
            __builtin_amdgcn_s_waitcnt(0);  // partial stores complete before the arrival
            __syncthreads();
            if (tid == 0) {
                const unsigned old = __hip_atomic_fetch_add(a.cnt + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int last = old == a.kc - 1;
                if (last) __hip_atomic_store(a.cnt + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_flag = last;
            }
            __syncthreads();
            if (!last_flag || wave >= NCW) return;
            // the last to arrive adds all chunks' partials in chunk order
#pragma unroll
            for (int tt = 0; tt < TT; tt++) acc[0][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};
            for (uint32_t k = 0; k < a.kc; k++) {
                const float* p = a.part + (((size_t)grp * a.kc + k) * HH_MMI_WAVES + wv) * PT + lane;
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[0][tt][i] += hh_load_coherent_f(p + (tt * 4 + i) * HH_WAVE);
            }
        }
        if (!live) return;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const uint32_t tok = tt * 16u + r16;
            if (tok >= a.b) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t R = R0 + 4u * c + (uint32_t)i;
                if (R < a.m) a.y[(size_t)tok * a.m + R] = acc[0][tt][i];
            }
        }
    }
}

#define HH_MMI_BLOCK ((HH_MMI_WAVES + 1) * HH_WAVE)
#define HH_MMI_K(NAME, NT, TT, D, RF)                                                          \
    extern "C" __global__ void __launch_bounds__(HH_MMI_BLOCK) NAME(const hh_mmi_args a) { \
        hh_mmi_body<NT, TT, D, RF>(a);                                                      \
    }
// GEMM / down: tiles 1..4, ring depth 2 or 4, stages whole (_w) or refilled (_r).  Gate/up
// (two tiles per item) keeps ring depth 2: at depth 4 the compiler no longer keeps the ring
// in place and waits for every load at the head of each round; three token tiles run as four
// (their register allocation spills).
#define HH_MMI_GEMM(TT)                                  \
    HH_MMI_K(hh_q4k_mmi_t##TT##_d2_w, 1, TT, 2, false) \
    HH_MMI_K(hh_q4k_mmi_t##TT##_d4_w, 1, TT, 4, false) \
    HH_MMI_K(hh_q4k_mmi_t##TT##_d2_r, 1, TT, 2, true)  \
    HH_MMI_K(hh_q4k_mmi_t##TT##_d4_r, 1, TT, 4, true)
HH_MMI_GEMM(1)
HH_MMI_GEMM(2)
HH_MMI_GEMM(3)
HH_MMI_GEMM(4)
HH_MMI_K(hh_q4k_mmi_gu_t1_d2_w, 2, 1, 2, false)
HH_MMI_K(hh_q4k_mmi_gu_t1_d2_r, 2, 1, 2, true)
HH_MMI_K(hh_q4k_mmi_gu_t2_d2_w, 2, 2, 2, false)
HH_MMI_K(hh_q4k_mmi_gu_t2_d2_r, 2, 2, 2, true)
HH_MMI_K(hh_q4k_mmi_gu_t4_d2_w, 2, 4, 2, false)
HH_MMI_K(hh_q4k_mmi_gu_t4_d2_r, 2, 4, 2, true)
