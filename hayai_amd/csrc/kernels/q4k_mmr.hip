// Batched Q4_K on the matrix cores as one weight stream per launch (gfx950), for up to 16
// tokens (one 16-token tile):
//   hh_q4k_mmr_gu_s<S>  FFN gate/up + act: h = act(W_gate . X) * (W_up . X), written as the
//                       token stages of the down projection (prefill_batched's gate/up and
//                       host SiLU*up, crates/hayai-core/src/prefill_wave.rs:569-584, fused)
//   hh_q4k_mmr_dn_s<S>  Y = W_down . H from those stages (prefill_wave.rs:579-584)
//   hh_q4k_mmr_s<S>     Y = W . X (ggml_gemv_batched_q4_k, crates/hayai-opencl/src/
//                       compute.rs:179-257)
// (Compiled after mm_common.hip: the same MFMA arithmetic, tile decode and token-stage layout;
// hh_mm_prep writes the token stages of X once per call.)
//
// Token stages.  X enters as hi + lo f16 halves (the 17 KB stages of mm_common.hip: f32-level
// accuracy; a single f16 rounding of the FFN input costs up to ~2e-3 of relative output
// error).  h enters the down projection as one f16 per element plus hi/lo sums (9 KB stages:
// [0, 8192) operands, [8192, 8704) sums hi, [8704, 9216) sums lo); its rounding costs at most
// ~2.5e-4 of the output and halves the down projection's MFMAs and staging.
//
// Work split: rows in 16-row units (FFN: the gate tile and the up tile of the same 16
// rows), superblocks in chunks of S.  A workgroup owns nw units of one chunk: it copies the
// chunk's S token stages into LDS by DMA and waits for them before its first weight request
// (a burst of weight requests would queue the copy behind it), then each of its nw waves
// streams its unit's S superblocks through a ring of D items in flight.  An item is the
// lane's 48 bytes of each tile (block header + 32 qs bytes) at a wave-uniform base plus fixed
// lane offsets, so wait counts are static and nothing stands between the weight stream and
// the MFMAs.  The MFMAs take the tokens as A and the weights as B, so each D lane holds four
// tokens of its own weight row and the superblock's d and dmin apply lane by lane; each
// weight operand is decoded right before its MFMA step (hh_mmr_wstep).
// The chunks of one row group meet in a workspace: each workgroup writes its partial sums
// with device-coherent stores, and the last to arrive (per-row-group counter, reset by it)
// adds them in chunk order, so results do not depend on arrival order.
// Token slots b..15 of the stages are zero (hh_mm_prep) or whatever the gate/up kernel
// computed for them: an MFMA output depends only on its own token, so they stay in outputs
// that are never stored.

struct hh_mmr_args {
    const uint8_t* w0;  // GEMM: W; FFN: W_gate   [m][row_bytes]
    const uint8_t* w1;  // FFN: W_up
    const uint8_t* xop; // token stages of the input [n/256]
    float* y;           // GEMM: [b][m] f32
    uint8_t* hop;       // FFN: h as single-f16 token stages [m/256]
    float* part;        // kc > 1: [groups][kc][nw][tiles * 4 rows][64 lanes] partial sums
    unsigned* cnt;      // kc > 1: arrival counter per row group (zero between launches)
    uint64_t row_bytes;
    uint32_t m;         // rows (FFN: d_ff, a multiple of 256)
    uint32_t n;         // columns (multiple of 256)
    uint32_t b;         // valid tokens, 1..16
    uint32_t nw;        // units (= waves) per workgroup, 1..8
    uint32_t kc;        // superblock chunks = workgroups per row group
    int32_t act;
};

#define HH_MMR_MAX_WAVES 8
#define HH_MMR_STAGE_HI 9216u  // single-f16 stage: operands, sums hi, sums lo

// Superblock header of this lane's row, decoded for its group c: the sub-block scales as
// (sc, -1024 sc) f16 pairs for the low nibbles and (sc / 16, -64 sc) for the high ones (see
// hh_mmr_wstep), the mins as the B operand of the min MFMA, d and dmin (q4k.rs:34-43).
struct hh_mmr_head {
    hh_h2 sl, sh, nl, nh;
    hh_h4 amin;
    float d, dmin;
};
HH_DEV void hh_mmr_head_decode(const uint4& h, uint32_t c, hh_mmr_head& t) {
    const uint32_t kk = 2u * (c & 1u);
    const uint32_t sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    const uint32_t sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    const uint32_t b = __builtin_amdgcn_perm(h.z, h.y, sel_yz);
    const uint32_t lo = b & 0x3F3F3F3Fu;
    const uint32_t wp = __builtin_amdgcn_perm(h.w, h.w, sel_w);
    const uint32_t hi = (wp & 0x00000F0Fu) | ((wp >> 4) & 0x0F0F0000u) | ((b >> 2) & 0x30303030u);
    const uint32_t s = c >= 2 ? hi : lo;
    const float sc_lo = hh_ub0(s), sc_hi = hh_ub1(s);
    t.d = hh_f16(h.x & 0xFFFFu);
    t.dmin = hh_f16(h.x >> 16);
    const _Float16 mlo = (_Float16)(-hh_ub2(s));
    const _Float16 mhi = (_Float16)(-hh_ub3(s));
    t.amin = hh_h4{mlo, mlo, mhi, mhi};
    t.sl = hh_h2{(_Float16)sc_lo, (_Float16)sc_lo};
    t.sh = hh_h2{(_Float16)(0.0625f * sc_hi), (_Float16)(0.0625f * sc_hi)};
    t.nl = hh_h2{(_Float16)(-1024.0f * sc_lo), (_Float16)(-1024.0f * sc_lo)};
    t.nh = hh_h2{(_Float16)(-64.0f * sc_hi), (_Float16)(-64.0f * sc_hi)};
}

// Weight operand of MFMA step s: s < 4 takes the low nibbles of qs dwords 2s, 2s+1 of this
// lane's group, s >= 4 the high nibbles of dwords 2(s-4), 2(s-4)+1; each weight becomes sc * q,
// exact in f16.  (v & 0x000F000F) | 0x64006400 is the f16 pair (1024 + q) of bytes 0 and 2 of
// v, with mask 0x00F000F0 (1024 + 16 q): one v_and_or_b32 (masks and exponent bits held in
// registers: a gfx9 VOP3 instruction takes no literal) and one packed FMA per two weights;
// the elements come in the order 0 2 1 3 4 6 5 7 of the lane's eight (the token stages hold B
// in that order).
struct hh_mmr_consts {
    uint32_t mlo, mhi, magic;
};
template <int S_>
HH_DEV hh_h8 hh_mmr_wstep(const uint4& q0, const uint4& q1, const hh_mmr_head& t, const hh_mmr_consts& k) {
    constexpr int s4 = S_ & 3;
    const uint32_t w0 = s4 == 0 ? q0.x : s4 == 1 ? q0.z : s4 == 2 ? q1.x : q1.z;
    const uint32_t w1 = s4 == 0 ? q0.y : s4 == 1 ? q0.w : s4 == 2 ? q1.y : q1.w;
    const uint32_t v[4] = {w0, w0 >> 8, w1, w1 >> 8};
    const uint32_t mask = S_ < 4 ? k.mlo : k.mhi;
    const hh_h2 m = S_ < 4 ? t.sl : t.sh, o = S_ < 4 ? t.nl : t.nh;
    hh_h2 r[4];
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = __builtin_elementwise_fma(hh_h2_bits((v[i] & mask) | k.magic), m, o);
    return hh_h8{r[0].x, r[0].y, r[1].x, r[1].y, r[2].x, r[2].y, r[3].x, r[3].y};
}

// FFN: NT = 2 tiles per unit (gate, up); GEMM: 1.  LO: the input stages carry lo halves
// (17 KB stages) or not (9 KB).  S superblocks per chunk, D ring items in flight per wave,
// refilled RB at a time (RB consecutive superblocks of each row per request burst: longer
// runs per DRAM page than one 144-byte block).
template <bool FFN, bool LO, int S, int D, int RB>
HH_DEV void hh_mmr_body(const hh_mmr_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];  // S token stages [+ FFN tiles]
    __shared__ int last_flag;
    constexpr int NT = FFN ? 2 : 1;
    constexpr uint32_t SB = LO ? HH_MM_STAGE : HH_MMR_STAGE_HI;  // stage bytes
    constexpr uint32_t SUMS = LO ? 16384u : 8192u;               // offset of the sums
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t nthr = a.nw * HH_WAVE;
    const uint32_t nsb = a.n / 256;
    const uint32_t grp = blockIdx.x / a.kc, kci = blockIdx.x % a.kc;
    const uint32_t sb0 = kci * S;
    const uint32_t ns = min((uint32_t)S, nsb - sb0);  // superblocks of this chunk (>= 1)
    const uint32_t nu = (a.m + 15) / 16;
    // waves past the last unit repeat it (in-bounds reads) and store nothing
    const bool live = grp * a.nw + wave < nu;
    const uint32_t unit = min(grp * a.nw + wave, nu - 1);
    const uint32_t c = lane >> 4, r16 = lane & 15u;
    const uint32_t row = min(unit * 16 + r16, a.m - 1);
    const size_t lofs = (size_t)row * a.row_bytes + (size_t)sb0 * 144;
    const uint8_t* const p0 = a.w0 + lofs;
    const uint8_t* const p1 = (FFN ? a.w1 : a.w0) + lofs;
    const uint32_t qo = 16u + 32u * c;
    uint8_t* const stages = reinterpret_cast<uint8_t*>(hh_smem);

    // item j: superblock sb0 + j of this wave's unit; items past the chunk re-read item 0
    hh_mm_wq ring[D][NT];
    auto issue = [&](int j, hh_mm_wq* w) {
        const uint32_t off = ((uint32_t)j < ns ? (uint32_t)j : 0u) * 144u;
        w[0].h = hh_ld16(p0 + off);
        w[0].q0 = hh_ld16(p0 + off + qo);
        w[0].q1 = hh_ld16(p0 + off + qo + 16);
        if constexpr (FFN) {
            w[1].h = hh_ld16(p1 + off);
            w[1].q0 = hh_ld16(p1 + off + qo);
            w[1].q1 = hh_ld16(p1 + off + qo + 16);
        }
    };
    constexpr int D0 = D < S ? D : S;
    hh_mmr_consts kc;
    asm volatile("s_mov_b32 %0, 0x000F000F" : "=s"(kc.mlo));
    asm volatile("s_mov_b32 %0, 0x00F000F0" : "=s"(kc.mhi));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kc.magic));

    // the chunk's stages -> LDS (SB / 16 = 17 * 64 or 9 * 64 chunks of 16 bytes per stage),
    // complete before the first weight request; then the ring
    {
        const uint8_t* src = a.xop + (size_t)sb0 * SB;
        const uint32_t chunks = ns * (SB / 16u);
        for (uint32_t c0 = wave * HH_WAVE; c0 < chunks; c0 += nthr)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + (size_t)(c0 + lane) * 16),
                                             (__attribute__((address_space(3))) void*)(stages + (size_t)c0 * 16), 16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
#pragma unroll
    for (int s = 0; s < D0; s++) issue(s, ring[s]);
    __syncthreads();  // the chunk's token stages are in LDS

    hh_f4 acc[NT];
#pragma unroll
    for (int q = 0; q < NT; q++) acc[q] = hh_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < S; j++) {
        hh_mmr_head hd[NT];
        uint4 qa[NT], qb[NT];
#pragma unroll
        for (int q = 0; q < NT; q++) {
            hh_mmr_head_decode(ring[j % D][q].h, c, hd[q]);
            qa[q] = ring[j % D][q].q0;
            qb[q] = ring[j % D][q].q1;
        }
        static_assert(D % RB == 0, "refill batches must divide the ring");
        if ((j + 1) % RB == 0) {
#pragma unroll
            for (int k = j + 1 - RB + D; k <= j + D; k++)
                if (k < S) issue(k, ring[k % D]);
        }
        // items past a short last chunk add nothing: their weights and token stage repeat
        // item 0's (finite values, scaled by zero)
        uint32_t jst = (uint32_t)j;
        if (j > 0) {
            jst = (uint32_t)j < ns ? (uint32_t)j : 0u;
            const float keep = (uint32_t)j < ns ? 1.f : 0.f;
#pragma unroll
            for (int q = 0; q < NT; q++) {
                hd[q].d *= keep;
                hd[q].dmin *= keep;
            }
        }
        const uint8_t* st = stages + jst * SB;
        // all token fragments of the item are requested at once, ahead of the decode
        constexpr int NF = LO ? 16 : 8;
        hh_h8 xf[NF];
#pragma unroll
        for (int i = 0; i < NF; i++) xf[i] = *reinterpret_cast<const hh_h8*>(st + (i >> 3) * 8192 + ((i & 7) * 64 + lane) * 16);
        const hh_h4 shi = *reinterpret_cast<const hh_h4*>(st + SUMS + lane * 8);
        const hh_h4 slo = *reinterpret_cast<const hh_h4*>(st + SUMS + 512 + lane * 8);
        __builtin_amdgcn_sched_barrier(0);
        const hh_f4 z = hh_f4{0.f, 0.f, 0.f, 0.f};
        hh_f4 ah[NT], al[NT], am[NT];
#pragma unroll
        for (int q = 0; q < NT; q++) {
            ah[q] = z;
            al[q] = z;
        }
#define HH_MMR_STEP(SS)                                                                     \
    _Pragma("unroll") for (int q = 0; q < NT; q++) {                                         \
        const hh_h8 w = hh_mmr_wstep<SS>(qa[q], qb[q], hd[q], kc);                           \
        ah[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[SS], w, ah[q], 0, 0, 0);           \
        if constexpr (LO) al[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[8 + ((SS) & 7)], w, al[q], 0, 0, 0); \
    }
        HH_MMR_STEP(0)
        HH_MMR_STEP(1)
        HH_MMR_STEP(2)
        HH_MMR_STEP(3)
        HH_MMR_STEP(4)
        HH_MMR_STEP(5)
        HH_MMR_STEP(6)
        HH_MMR_STEP(7)
#undef HH_MMR_STEP
#pragma unroll
        for (int q = 0; q < NT; q++) {
            am[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(shi, hd[q].amin, z, 0, 0, 0);
            am[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(slo, hd[q].amin, am[q], 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[q][r] = fmaf(hd[q].d, LO ? ah[q][r] + al[q][r] : ah[q][r], acc[q][r]);
                acc[q][r] = fmaf(hd[q].dmin, am[q][r], acc[q][r]);
            }
    }

    // Partials are laid out [tile][r][lane] so every store and load instruction covers 256
    // contiguous bytes.
    if (a.kc > 1) {
        constexpr uint32_t PT = NT * 4u * HH_WAVE;
        float* my = a.part + (((size_t)grp * a.kc + kci) * a.nw + wave) * PT + lane;
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) hh_store_coherent_f(my + (q * 4 + r) * HH_WAVE, acc[q][r]);
        __builtin_amdgcn_s_waitcnt(0);  // partial stores complete before the arrival
        __syncthreads();
        if (tid == 0) {
            const unsigned old = __hip_atomic_fetch_add(a.cnt + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == a.kc - 1;
            if (last) __hip_atomic_store(a.cnt + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = last;
        }
        __syncthreads();
        if (!last_flag) return;
        // the last to arrive adds all chunks' partials in chunk order, 8 chunks' loads at a time
        // (chunks past kc repeat the last one and add zero)
#pragma unroll
        for (int q = 0; q < NT; q++) acc[q] = hh_f4{0.f, 0.f, 0.f, 0.f};
        for (uint32_t k0 = 0; k0 < a.kc; k0 += 8) {
            float v[8][NT * 4];
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const uint32_t k = min(k0 + (uint32_t)kk, a.kc - 1);
                const float* p = a.part + (((size_t)grp * a.kc + k) * a.nw + wave) * PT + lane;
#pragma unroll
                for (int i = 0; i < NT * 4; i++) v[kk][i] = hh_load_coherent_f(p + i * HH_WAVE);
            }
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const bool use = k0 + (uint32_t)kk < a.kc;
#pragma unroll
                for (int q = 0; q < NT; q++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[q][r] += use ? v[kk][q * 4 + r] : 0.f;
            }
        }
    }
    if (!live) return;

    // D lane (row r16, quarter c): acc[q][r] is token 4c + r of row R = unit * 16 + r16
    const uint32_t R0 = unit * 16, R = R0 + r16;
    if constexpr (FFN) {
        // h -> single-f16 token stages of the down projection (n = m).  The wave transposes
        // its 16 x 16 tile through LDS (its own 512 bytes past the stages) so that lanes 0..31
        // each write one 16-byte chunk: 8 consecutive rows of one token.
        _Float16* tp = reinterpret_cast<_Float16*>(stages + (size_t)S * SB + wave * 512u);
        float hsum[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float h = hh_act_mul(acc[0][r], acc[1][r], a.act);
            hsum[r] = h;
            tp[(4 * c + (uint32_t)r) * 16 + r16] = (_Float16)h;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile is in LDS
        __builtin_amdgcn_wave_barrier();
        if (lane < 32) {
            const uint32_t run = lane >> 4, tok = lane & 15u;
            const hh_h8 c8 = *reinterpret_cast<const hh_h8*>(tp + tok * 16 + 8 * run);
            const hh_h8 chunk = __builtin_shufflevector(c8, c8, 0, 2, 1, 3, 4, 6, 5, 7);  // the stage order
            uint8_t* st = a.hop + (size_t)(R0 / 256) * HH_MMR_STAGE_HI;
            *reinterpret_cast<hh_h8*>(st + hh_mm_elem_off(tok, (R0 & 255u) + 8 * run)) = chunk;
        }
        // the unit's 16 rows are one half-sub-block of h: per token, their f32 sum (over the
        // 16 lanes of the quarter) feeds the down projection's min term as hi + lo
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) hsum[r] += __shfl_xor(hsum[r], m, HH_WAVE);
        if (r16 == 0) {
            uint8_t* ss = a.hop + (size_t)(R0 / 256) * HH_MMR_STAGE_HI;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                _Float16 hi, lo;
                hh_split_f16(hsum[r], hi, lo);
                const uint32_t off = hh_mm_sum_off(4 * c + (uint32_t)r, (R0 & 255u) / 16) - 16384u + 8192u;
                *reinterpret_cast<_Float16*>(ss + off) = hi;
                *reinterpret_cast<_Float16*>(ss + 512 + off) = lo;
            }
        }
    } else {
        if (R < a.m) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = 4 * c + (uint32_t)r;
                if (tok < a.b) a.y[(size_t)tok * a.m + R] = acc[0][r];
            }
        }
    }
}

#define HH_MMR_BLOCK (HH_MMR_MAX_WAVES * HH_WAVE)
#define HH_MMR_GU(S)                                                                                   \
    extern "C" __global__ void __launch_bounds__(HH_MMR_BLOCK) hh_q4k_mmr_gu_s##S(const hh_mmr_args a) { \
        hh_mmr_body<true, true, S, (S < 3 ? S : 3), 1>(a);                                                              \
    }
#define HH_MMR_GEMM(S)                                                                                 \
    extern "C" __global__ void __launch_bounds__(HH_MMR_BLOCK) hh_q4k_mmr_s##S(const hh_mmr_args a) {    \
        hh_mmr_body<false, true, S, (S < 6 ? S : 6), 1>(a);                                               \
    }
#define HH_MMR_DN(S)                                                                                   \
    extern "C" __global__ void __launch_bounds__(HH_MMR_BLOCK) hh_q4k_mmr_dn_s##S(const hh_mmr_args a) { \
        hh_mmr_body<false, false, S, (S < 4 ? S : 4), (S < 4 ? 1 : 2)>(a);                                              \
    }
HH_MMR_GU(2)
HH_MMR_GU(4)
HH_MMR_GU(7)
HH_MMR_GU(8)
HH_MMR_GEMM(2)
HH_MMR_GEMM(4)
HH_MMR_GEMM(7)
HH_MMR_GEMM(8)
HH_MMR_DN(2)
HH_MMR_DN(4)
HH_MMR_DN(7)
HH_MMR_DN(8)
HH_MMR_DN(14)
HH_MMR_DN(16)
