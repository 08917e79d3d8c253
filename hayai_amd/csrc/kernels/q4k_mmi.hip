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
// (Compiled after mm_common.hip: its vector types and the
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
//                  of token l % 16 at superblock elements 32 j + 8 (l / 16) + e, e in the
//                  order 0 2 1 3 4 6 5 7 (the order the weight decode produces)
//   [8192, 8704)   s_tj f32 at (8 t + j) * 4
//   [8704, 9216)   u_tj f32 at (16 j + t) * 4
// The A fragment of sub-blocks 2g (low nibbles) and 2g + 1 (high nibbles) is, for lane
// (quarter c, row r), bytes 8c .. 8c + 7 of the row's 32-byte qs group g (q4k.rs:178-203), in
// the stage's element order.
//
// Work split: a workgroup is 8 compute waves, two per 16-row unit (4 consecutive units, 64
// rows), over a chunk of superblocks, plus a wave that copies the token stages; the wave of half h takes sub-blocks 4h .. 4h + 3 of every
// superblock (the split below).  Each wave streams its unit's superblocks through a register
// ring of D items (per item and matrix the 16-byte block header and 16 bytes of qs at fixed
// lane offsets, so wait counts are static).  The chunk's token stages sit in an LDS ring of R
// superblock slots, copied there by global->LDS DMA; when the chunk is longer than R they
// stream through in rounds of R / 2 superblocks, one barrier per round (below).  Gate/up takes whole rows (one
// chunk): its 4 units are 64 rows, two 32-row blocks of h, so the workgroup quantizes its h
// itself (the pair of units of a block exchange their maxima and sums through LDS).  Chunks of
// one row group (GEMM and down) meet in a workspace; the last workgroup to arrive adds them in
// chunk order (deterministic).  Against one compute wave per unit (8-byte qs loads, a barrier
// per superblock): 64 tokens 3.16 -> 2.52 ms per 32 8B layers, 17 tokens 1.98 -> 1.90; the
// compute waves copying the stages themselves instead of the ninth wave: 2-3% slower.

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
    // f16 of q; lanes e with bit 1 clear hold elements e | e + 2 << 16, lanes 8c gather their
    // quarter as the pairs (0, 2) (1, 3) (4, 6) (5, 7): the weight fragments' element order
    const uint32_t hb = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q);
    uint32_t w = (e & 2u) ? hb << 16 : hb;
    w |= __shfl_xor(w, 2, 32);
    const uint32_t w1 = __shfl_down(w, 1, 32), w2 = __shfl_down(w, 4, 32), w3 = __shfl_down(w, 5, 32);
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

// Two waves per 16-row unit (two per SIMD), wave half h taking sub-blocks 4h .. 4h + 3 of every
// superblock: per item and matrix one 16-byte header load and one 16-byte qs load per lane (the
// lane's row r16 = l % 16, bytes 64h + 16c .. + 15 of its qs, c = l / 16: 16-byte loads stream
// such 16-row tiles at ~4.6-5 TB/s where 8-byte pieces reach ~3.3-3.6), which two lane swaps
// turn into the A fragments of the four sub-blocks (below).  The halves' sums meet in LDS at
// the end, half 0 adding half 1's (a fixed order), and half 0 runs the epilogue.
//
// The swaps: lane group c holds X_c = qs bytes 64h + 16c .. + 7 and Y_c = the next 8; the
// fragment of sub-blocks 4h, 4h + 1 (qs group 2h) wants bytes 64h + 8c .. + 7 in group c,
// i.e. (X_0, Y_0, X_1, Y_1) over the four groups, and that of sub-blocks 4h + 2, 4h + 3 (qs
// group 2h + 1) wants (X_2, Y_2, X_3, Y_3).  v_permlane16_swap(X, Y) exchanges X's odd
// 16-lane rows with Y's even rows: X = (X_0, Y_0, X_2, Y_2), Y = (X_1, Y_1, X_3, Y_3); then
// v_permlane32_swap(X, Y) exchanges X's upper half with Y's lower half: X = (X_0, Y_0, X_1,
// Y_1), Y = (X_2, Y_2, X_3, Y_3).  Two swaps per dword pair, four per 16 bytes.
template <int NT, int TT, int D, bool REFILL>
HH_DEV void hh_mmi_body(const hh_mmi_args& a) {
    constexpr uint32_t NU = HH_MMI_WAVES;  // units per workgroup
    constexpr uint32_t NCW = 2 * NU;       // compute waves, two per unit; wave NCW copies the stages
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];  // the stage ring
    __shared__ float xch[2][NU][TT * 16];                            // gate/up: h block exchange
    __shared__ int last_flag;
    constexpr uint32_t SBT = HH_MMI_STAGE * TT;
    constexpr uint32_t R = HH_MMI_LDS / SBT < 16 ? HH_MMI_LDS / SBT : 16;
    constexpr uint32_t CHUNKS = SBT / 1024u;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t nsb = a.n / 256;
    const uint32_t grp = blockIdx.x / a.kc, kci = blockIdx.x % a.kc;
    const uint32_t sb0 = kci * a.sbc;
    const uint32_t ns = min(a.sbc, nsb - sb0);
    // Stages stream through the ring in rounds of P items (half the ring): at the end of round r
    // the waves meet, after which the copy wave puts items rP + R .. rP + P - 1 + R into the
    // slots the round used; those land while round r + 1 runs on the other half.  Compute waves
    // cover DP items per loop body (a multiple of D and P), so the barriers sit at fixed places.
    constexpr uint32_t P = REFILL ? (R / 2 < 1 ? 1 : R / 2) : D;
    constexpr uint32_t DP = (D % P == 0) ? D : (P % D == 0 ? P : D * P);
    const uint32_t nsp = (ns + DP - 1) / DP * DP;
    char* const slots = hh_smem;

    if (wave == NCW) {
        // superblock k (clamped to the chunk's last) -> a slot; only this wave issues DMA, so
        // the compute waves' wait counts never include it
        auto copy = [&](uint32_t k, uint32_t slot) {
            const uint8_t* src = a.xs + (size_t)(sb0 + min(k, ns - 1u)) * SBT + lane * 16u;
            char* dst = slots + (size_t)slot * SBT;
#pragma unroll
            for (uint32_t i = 0; i < CHUNKS; i++)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + i * 1024u),
                                                 (__attribute__((address_space(3))) void*)(dst + i * 1024u), 16, 0, 0);
        };
        if constexpr (REFILL) {
            // the first round's slots, then the rest of the ring (landing during the first
            // round); at the barrier closing each round every copy issued so far has landed,
            // so the next round's slots are in LDS when it starts
            for (uint32_t k = 0; k < P; k++) copy(k, k);
            __builtin_amdgcn_s_waitcnt(0x0F70);
            hh_mmi_lds_barrier();
            for (uint32_t k = P; k < R; k++) copy(k, k);
            for (uint32_t k0 = 0; k0 < nsp; k0 += P) {
                __builtin_amdgcn_s_waitcnt(0x0F70);
                hh_mmi_lds_barrier();
                for (uint32_t k = k0; k < k0 + P; k++) copy(k + R, k % R);
            }
        } else {
            for (uint32_t k = 0; k < ns; k++) copy(k, k);
            __builtin_amdgcn_s_waitcnt(0x0F70);
            hh_mmi_lds_barrier();
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // every copy has landed before the ring is reused
    }

    const uint32_t c = lane >> 4, r16 = lane & 15u;
    const uint32_t nu = (a.m + 15) / 16;
    const uint32_t us = wave % NU;           // the copy wave: unit 0, half 0, owns nothing
    const uint32_t half = (wave / NU) & 1u;
    const bool own = wave < NU;  // half 0: owns the unit's outputs
    const uint32_t u0 = grp * NU + us;
    const bool live = own && u0 < nu;
    const uint32_t unit = min(u0, nu - 1);
    const uint32_t row = min(unit * 16 + r16, a.m - 1);
    const size_t lofs = (size_t)row * a.row_bytes + (size_t)sb0 * 144;
    const uint8_t* const p0 = a.w0 + lofs;
    const uint8_t* const p1 = (NT == 2 ? a.w1 : a.w0) + lofs;
    struct Item {
        uint4 h;
        uint4 q;
    };
    hh_f4 acc[NT][TT];
#pragma unroll
    for (int q = 0; q < NT; q++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[q][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};

    if (wave < NCW) {
        // the decode's constants in registers: a gfx9 VOP3 instruction takes no literal, so
        // held this way (two masks in SGPRs, the f16 exponent bits in a VGPR: one scalar operand
        // per instruction) each (v & mask) | magic is one v_and_or_b32
        uint32_t mlo, mhi, magic;
        asm volatile("s_mov_b32 %0, 0x000F000F" : "=s"(mlo));
        asm volatile("s_mov_b32 %0, 0x00F000F0" : "=s"(mhi));
        asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
        Item ring[D][NT];
        const uint32_t qofs = 16u + 64u * half + 16u * c;
        auto issue = [&](uint32_t k, Item* it) {
            const uint32_t off = min(k, ns - 1u) * 144u;
#pragma unroll
            for (int q = 0; q < NT; q++) {
                const uint8_t* p = (q ? p1 : p0) + off;
                it[q].h = hh_ld16(p);
                it[q].q = hh_ld16(p + qofs);
            }
        };
#pragma unroll
        for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
        hh_mmi_lds_barrier();  // the first round's stages are in LDS

#pragma unroll 1
        for (uint32_t k0 = 0; k0 < nsp; k0 += DP) {
#pragma unroll
            for (int s = 0; s < (int)DP; s++) {
                const uint32_t k = k0 + (uint32_t)s;
                const bool valid = k < ns;
                Item* const cur = ring[s % D];
                const char* st = slots + (size_t)(min(k, ns - 1u) % R) * SBT;
                hh_h8 wa[NT][4];
                float d4[NT][4];
                float nm[NT];
#pragma unroll
                for (int q = 0; q < NT; q++) {
                    uint4 h = cur[q].h;
                    if (!valid) h.x = 0u;
                    const uint4 w = cur[q].q;
                    const auto s0 = __builtin_amdgcn_permlane16_swap(w.x, w.z, false, false);
                    const auto s1 = __builtin_amdgcn_permlane16_swap(w.y, w.w, false, false);
                    const auto t0 = __builtin_amdgcn_permlane32_swap(s0[0], s0[1], false, false);
                    const auto t1 = __builtin_amdgcn_permlane32_swap(s1[0], s1[1], false, false);
                    const uint2 g[2] = {make_uint2(t0[0], t1[0]), make_uint2(t0[1], t1[1])};
                    const uint32_t sch = half ? (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u) : h.y & 0x3F3F3F3Fu;
                    // sub-blocks 2pr (low nibbles) and 2pr + 1 (high nibbles) of the half from
                    // qs dwords g[pr]: (v & 0x000F000F) | 0x64006400 is the f16 pair (1024 + n)
                    // of bytes 0 and 2, with mask 0x00F000F0 (1024 + 16 n); the pair's scales
                    // (sc_a, sc_b / 16) and offsets (-1024 sc_a, -64 sc_b) make one FMA per two
                    // weights give n sc exactly.  Elements come in the order 0 2 1 3 4 6 5 7 of
                    // the lane's eight (the stage stores B in the same order).
#pragma unroll
                    for (int pr = 0; pr < 2; pr++) {
                        const uint32_t sel = (2u * pr) | (4u << 8) | ((2u * pr + 1u) << 16) | (4u << 24);
                        const hh_h2 s1024 = hh_h2_bits(__builtin_amdgcn_perm(0x64646464u, sch, sel));
                        const hh_h2 scab = s1024 - hh_h2{(_Float16)1024.0f, (_Float16)1024.0f};
                        const hh_h2 mult = scab * hh_h2{(_Float16)1.0f, (_Float16)0.0625f};
                        const hh_h2 off = mult * hh_h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
                        const hh_h2 ma = hh_h2{mult.x, mult.x}, oa = hh_h2{off.x, off.x};
                        const hh_h2 mb = hh_h2{mult.y, mult.y}, ob = hh_h2{off.y, off.y};
                        const uint2 pq = g[pr];
                        const uint32_t v[4] = {pq.x, pq.x >> 8, pq.y, pq.y >> 8};
                        hh_h2 ra[4], rb[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            ra[i] = __builtin_elementwise_fma(hh_h2_bits((v[i] & mlo) | magic), ma, oa);
                            rb[i] = __builtin_elementwise_fma(hh_h2_bits((v[i] & mhi) | magic), mb, ob);
                        }
                        wa[q][2 * pr] = hh_h8{ra[0].x, ra[0].y, ra[1].x, ra[1].y, ra[2].x, ra[2].y, ra[3].x, ra[3].y};
                        wa[q][2 * pr + 1] = hh_h8{rb[0].x, rb[0].y, rb[1].x, rb[1].y, rb[2].x, rb[2].y, rb[3].x, rb[3].y};
                    }
                    const float d = hh_f16(h.x & 0xFFFFu);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        d4[q][i] = __builtin_bit_cast(
                            float, __builtin_amdgcn_ds_bpermute((int)((c * 4u + (uint32_t)i) * 4u), __builtin_bit_cast(int, d)));
                    hh_mmi_head hd;
                    hh_mmi_mins(h, c, hd);
                    nm[q] = half ? hd.nm1 : hd.nm0;  // -dmin m_j of sub-block 4 half + c
                }
                __builtin_amdgcn_sched_barrier(0);
                issue(k + D, cur);
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    const char* sg = st + tt * HH_MMI_STAGE;
                    const float4 sa = *reinterpret_cast<const float4*>(sg + 8192u + r16 * 32u + 16u * half);
                    const float sj[4] = {sa.x, sa.y, sa.z, sa.w};
                    const float uv = *reinterpret_cast<const float*>(sg + 8704u + ((4u * half + c) * 16u + r16) * 4u);
                    hh_f4 ps[NT];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const hh_h8 xb = *reinterpret_cast<const hh_h8*>(sg + ((4u * half + (uint32_t)jj) * 64u + lane) * 16u);
#pragma unroll
                        for (int q = 0; q < NT; q++) {
                            const hh_f4 pj = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[q][jj], xb, hh_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            if (jj == 0) {
#pragma unroll
                                for (int i = 0; i < 4; i++) ps[q][i] = pj[i] * sj[0];
                            } else {
#pragma unroll
                                for (int i = 0; i < 4; i++) ps[q][i] = fmaf(pj[i], sj[jj], ps[q][i]);
                            }
                        }
                    }
#pragma unroll
                    for (int q = 0; q < NT; q++) {
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[q][tt][i] = fmaf(d4[q][i], ps[q][i], acc[q][tt][i]);
                        acc[q][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(nm[q], uv, acc[q][tt], 0, 0, 0);
                    }
                }
                if constexpr (REFILL) {
                    if (((uint32_t)s + 1) % P == 0) hh_mmi_lds_barrier();  // the round's slots are free
                }
            }
        }
    }

    // the halves meet: the ring is free once every wave (the copy wave after its last copy
    // landed) has passed this barrier
    __syncthreads();
    float* const xs2 = reinterpret_cast<float*>(slots) + (size_t)us * (NT * TT * 4u * HH_WAVE) + lane;
    if (wave < NCW && half == 1u) {
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int i = 0; i < 4; i++) xs2[((q * TT + tt) * 4 + i) * HH_WAVE] = acc[q][tt][i];
    }
    __syncthreads();
    if (own) {
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[q][tt][i] += xs2[((q * TT + tt) * 4 + i) * HH_WAVE];
    }

    const uint32_t R0 = unit * 16;
    if constexpr (NT == 2) {
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
        if (own && c == 0)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) xch[0][us][tt * 16 + r16] = am[tt];
        __syncthreads();
        float sc[TT];
        int xsum[TT];
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            sc[tt] = fmaxf(am[tt], xch[0][us ^ 1u][tt * 16 + r16]) / 127.0f;
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
        if (own && c == 0)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) xch[1][us][tt * 16 + r16] = (float)xsum[tt];
        __syncthreads();
        if (!live) return;
        const uint32_t sbd = R0 / 256, jd = (R0 % 256) / 32, hf = (R0 / 16) & 1u;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            uint8_t* st = a.hs + ((size_t)sbd * TT + tt) * HH_MMI_STAGE;
            auto f16b = [](int v) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v); };
            const uint32_t w0 = f16b(qi[tt][0]) | (f16b(qi[tt][2]) << 16);  // rows in the order 0 2 1 3
            const uint32_t w1 = f16b(qi[tt][1]) | (f16b(qi[tt][3]) << 16);
            const uint32_t x0 = __shfl_xor(w0, 16, HH_WAVE), x1 = __shfl_xor(w1, 16, HH_WAVE);
            if ((c & 1u) == 0)
                *reinterpret_cast<uint4*>(st + (size_t)(jd * 64u + (2u * hf + c / 2u) * 16u + r16) * 16u) =
                    make_uint4(w0, w1, x0, x1);
            if (hf == 0 && c == 0) {
                const float xsv = (float)(xsum[tt] + (int)xch[1][us ^ 1u][tt * 16 + r16]);
                *reinterpret_cast<float*>(st + 8192u + (r16 * 8u + jd) * 4u) = sc[tt];
                *reinterpret_cast<float*>(st + 8704u + (jd * 16u + r16) * 4u) = sc[tt] * xsv;
            }
        }
    } else {
        if (a.kc > 1) {
            constexpr uint32_t PT = TT * 4u * HH_WAVE;
            float* my = a.part + (((size_t)grp * a.kc + kci) * NU + us) * PT + lane;
            if (own)
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) hh_store_coherent_f(my + (tt * 4 + i) * HH_WAVE, acc[0][tt][i]);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0) {
                const unsigned old = __hip_atomic_fetch_add(a.cnt + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int last = old == a.kc - 1;
                if (last) __hip_atomic_store(a.cnt + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_flag = last;
            }
            __syncthreads();
            if (!last_flag || !own) return;
#pragma unroll
            for (int tt = 0; tt < TT; tt++) acc[0][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};
            for (uint32_t k = 0; k < a.kc; k++) {
                const float* p = a.part + (((size_t)grp * a.kc + k) * NU + us) * PT + lane;
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
                const uint32_t Rr = R0 + 4u * c + (uint32_t)i;
                if (Rr < a.m) a.y[(size_t)tok * a.m + Rr] = acc[0][tt][i];
            }
        }
    }
}

// GEMM / down: tiles 1..4, ring depth 2 or 4, stages whole (_w) or streamed in rounds (_r).
// Gate/up (two matrices per item) keeps ring depth 2 (depth 4 measured slower at 64 tokens:
// 2.73 vs 2.55 ms per 32 layers); three token tiles run as four.
#define HH_MMI_BLOCK ((2 * HH_MMI_WAVES + 1) * HH_WAVE)
#define HH_MMI_K(NAME, NT, TT, D, RF)                                                          \
    extern "C" __global__ void __launch_bounds__(HH_MMI_BLOCK) NAME(const hh_mmi_args a) { \
        hh_mmi_body<NT, TT, D, RF>(a);                                                      \
    }
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
