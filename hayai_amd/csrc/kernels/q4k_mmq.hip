// Batched Q4_K on the int8 matrix cores (gfx950), 16 to 64 tokens per pass:
//   hh_mmq_prep              tokens [b][n] f32 -> int8 token stages (per 32-element block
//                            of each token: s = amax / 127, q = round_half_away(x / s)
//                            clamped to +-127, the activation quantization of the batched
//                            path), zero-padded to 16 * TT tokens
//   hh_q4k_mmq_s<S>_t<TT>    Y[b][m] = W . X from those stages (ggml_gemv_batched_q4_k,
//                            crates/hayai-opencl/src/compute.rs:179-257;
//                            execute_quant_gemv_batched, crates/hayai-core/src/
//                            orchestrator.rs:240-269)
//   hh_q4k_mmq_gu_s<S>_t<TT> H[b][m] = act(W_gate . X) * (W_up . X) (prefill_batched's
//                            gate/up and SiLU * up, crates/hayai-core/src/prefill_wave.rs:
//                            569-584, fused)
// (Compiled after mm_common.hip: shares its vector types and coherent partial-sum helpers.)
//
// Arithmetic.  A Q4_K weight is d * sc_j * q - dmin * m_j for sub-block j (32 columns) and a
// token element is s_tj * xq (its block's scale), so one output is
//   sum_j d sc_j s_tj (sum_k q xq)  -  sum_j dmin m_j (s_tj sum_k xq).
// The inner sums sum_k q * xq are exact int32 products of v_mfma_i32_16x16x32_i8 (one
// instruction per sub-block: K = 32 columns, q in 0..15, xq in -127..127); each is scaled in
// f32 by d sc_j s_tj.  The min term is one f32 MFMA (v_mfma_f32_16x16x4f32) per four
// sub-blocks: A = s_tj sum xq per (token, sub-block) from the stage, B = -dmin m_j per
// (sub-block, row).  The MFMAs take the tokens as A and the weights as B, so each C lane holds
// four tokens of one weight row (lane % 16): the row's scales apply lane by lane.
//
// Token stage of one superblock for tp = 16 * TT tokens (320 * tp bytes):
//   [0, 256 tp)        xq: 8 bytes per (sub-block j, quarter c, token t) at ((4 j + c) tp + t) * 8,
//                      the columns 32 j + 8 c .. + 7 of token t (one MFMA A fragment per lane:
//                      a wave's 64 lanes read 512 contiguous bytes)
//   [256 tp, 288 tp)   s_tj at (j tp + t) * 4
//   [288 tp, 320 tp)   s_tj * sum_k xq at (j tp + t) * 4
// Weights: a lane (quarter c, row r) holds, for each of the superblock's four 32-byte qs
// groups g, bytes 8 c .. 8 c + 7 of group g: the low nibbles are columns 8 c .. + 7 of
// sub-block 2 g, the high nibbles those of sub-block 2 g + 1 (q4k.rs:178-203), i.e. the MFMA
// B fragment of either sub-block with the k order of the token stage.
//
// Work split (as q4k_mmr.hip): rows in 16-row units, superblocks in chunks of S; a workgroup
// owns nw units of one chunk, copies the chunk's S stages into LDS by DMA before its first
// weight request, and each wave streams its unit's S superblocks through a ring of D items
// (per tile: the 16-byte block header + four 8-byte qs pieces).  Chunks of one row group
// meet in a workspace; the last workgroup to arrive adds them in chunk order (deterministic).

typedef int hh_i4 __attribute__((ext_vector_type(4)));

#define HH_MMQ_MAX_WAVES 8
#define HH_MMQ_BLOCK (HH_MMQ_MAX_WAVES * HH_WAVE)

struct hh_mmq_prep_args {
    const float* x;  // [b][n] f32, 16-byte aligned rows
    uint8_t* xs;     // [n / 256] stages of 320 * tp bytes
    uint32_t n;
    uint32_t b;      // valid tokens
    uint32_t tp;     // padded tokens (multiple of 16)
    uint32_t pad;
};

// A team of 32 lanes per (token, 32-element block), one element per lane: amax and the sum
// of the quantized values by cross-lane reductions; eight lanes then write their quarter's
// 8 bytes as one store.  Tokens past b are written as zeros.
extern "C" __global__ void __launch_bounds__(256) hh_mmq_prep(const hh_mmq_prep_args a) {
    const uint32_t nb = a.n / 32;
    const uint32_t blk = blockIdx.x * 8u + threadIdx.x / 32u;  // (token, block) index
    const uint32_t e = threadIdx.x % 32u;                      // element within the block
    if (blk >= a.tp * nb) return;                               // whole 32-lane teams exit together
    const uint32_t t = blk / nb, k = blk % nb;
    const uint32_t sb = k / 8, j = k % 8;
    uint8_t* st = a.xs + (size_t)sb * 320u * a.tp;
    const float v = t < a.b ? a.x[(size_t)t * a.n + 32u * k + e] : 0.f;
    float amax = fabsf(v);
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float s = amax / 127.0f;
    float q = s > 0.f ? roundf(v / s) : 0.f;
    q = fminf(fmaxf(q, -127.f), 127.f);
    const int qi = (int)q;
    int sum = qi;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) sum += __shfl_xor(sum, m, 32);
    // gather the quarter's 8 bytes (elements 8c .. 8c + 7) into lane 8c
    const uint32_t byte = (uint32_t)qi & 0xFFu;
    uint32_t w = byte << (8 * (e & 3u));
    w |= __shfl_xor(w, 1, 32);
    w |= __shfl_xor(w, 2, 32);  // lanes 4i.. hold the dword of elements 4i .. 4i + 3
    const uint32_t hi = __shfl_down(w, 4, 32);
    if ((e & 7u) == 0) {
        const uint32_t c = e / 8u;
        *reinterpret_cast<uint2*>(st + ((size_t)(4u * j + c) * a.tp + t) * 8u) = make_uint2(w, hi);
    }
    if (e == 0) {
        *reinterpret_cast<float*>(st + 256u * a.tp + ((size_t)j * a.tp + t) * 4u) = s;
        *reinterpret_cast<float*>(st + 288u * a.tp + ((size_t)j * a.tp + t) * 4u) = s * (float)sum;
    }
}

struct hh_mmq_args {
    const uint8_t* w0;  // GEMM: W; FFN: W_gate   [m][row_bytes]
    const uint8_t* w1;  // FFN: W_up
    const uint8_t* xs;  // token stages [n / 256]
    float* y;           // GEMM: Y [b][m]; FFN: H [b][m]
    float* part;        // kc > 1: [groups][kc][nw][NT * TT * 4][64 lanes] partial sums
    unsigned* cnt;      // kc > 1: arrival counter per row group (zero between launches)
    uint64_t row_bytes;
    uint32_t m;         // rows
    uint32_t n;         // columns (multiple of 256)
    uint32_t b;         // valid tokens (<= 16 * TT)
    uint32_t nw;        // units (= waves) per workgroup, 1..8
    uint32_t kc;        // superblock chunks = workgroups per row group
    int32_t act;
};

// -dmin * m_j of a lane's row for sub-blocks c and c + 4 (get_scale_min_k4, q4k.rs:34-43):
// the B operand of the min-term MFMA.
struct hh_mmq_head {
    float nm0, nm1;
};
HH_DEV uint32_t hh_byte(uint32_t v, uint32_t i) { return (v >> (8 * i)) & 0xFFu; }
HH_DEV void hh_mmq_mins(const uint4& h, uint32_t c, hh_mmq_head& t) {
    const float dmin = hh_f16(h.x >> 16);
    const uint32_t q[3] = {h.y, h.z, h.w};  // the 12 scale bytes
    auto qb = [&](uint32_t i) { return hh_byte(q[i >> 2], i & 3u); };
    // sub-block c < 4: m = q[c + 4] & 63; sub-block c + 4: (q[c + 8] >> 4) | ((q[c + 4] >> 6) << 4)
    const uint32_t b4 = qb(c + 4u), b8 = qb(c + 8u);
    t.nm0 = -dmin * (float)(b4 & 63u);
    t.nm1 = -dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4));
}

// d * sc_j of sub-block j (a constant after unrolling) from a block header.
HH_DEV float hh_mmq_dsc(const uint4& h, uint32_t j) {
    const uint32_t q[3] = {h.y, h.z, h.w};
    auto qb = [&](uint32_t i) { return hh_byte(q[i >> 2], i & 3u); };
    const uint32_t sc = j < 4 ? (qb(j) & 63u) : ((qb(j + 4) & 0xFu) | ((qb(j - 4) >> 6) << 4));
    return hh_f16(h.x & 0xFFFFu) * (float)sc;
}

template <int NT, int TT, int S, int D>
HH_DEV void hh_mmq_body(const hh_mmq_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];  // S token stages
    __shared__ int last_flag;
    constexpr uint32_t TP = 16u * TT;
    constexpr uint32_t SB = 320u * TP;
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
    const uint8_t* const p1 = (NT == 2 ? a.w1 : a.w0) + lofs;
    uint8_t* const stages = reinterpret_cast<uint8_t*>(hh_smem);

    struct Item {
        uint4 h;
        uint2 q[4];
    };
    Item ring[D][NT];
    auto issue = [&](uint32_t jj, Item* it) {  // items past the chunk re-read item 0
        const uint32_t off = (jj < ns ? jj : 0u) * 144u;
#pragma unroll
        for (int q = 0; q < NT; q++) {
            const uint8_t* p = (q ? p1 : p0) + off;
            it[q].h = hh_ld16(p);
#pragma unroll
            for (int g = 0; g < 4; g++) it[q].q[g] = *reinterpret_cast<const uint2*>(p + 16u + 32u * g + 8u * c);
        }
    };
    static_assert(S % D == 0, "the ring depth divides the chunk");

    // the chunk's stages -> LDS (SB / 16 chunks of 16 bytes per stage), complete before the
    // first weight request; then the ring
    {
        const uint8_t* src = a.xs + (size_t)sb0 * SB;
        const uint32_t chunks = ns * (SB / 16u);
        for (uint32_t c0 = wave * HH_WAVE; c0 < chunks; c0 += nthr)
            if (c0 + lane < chunks)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + (size_t)(c0 + lane) * 16),
                                                 (__attribute__((address_space(3))) void*)(stages + (size_t)c0 * 16), 16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
#pragma unroll
    for (int s = 0; s < D; s++) issue((uint32_t)s, ring[s]);
    __syncthreads();  // the chunk's token stages are in LDS

    hh_f4 acc[NT][TT];
#pragma unroll
    for (int q = 0; q < NT; q++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[q][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};
    const hh_i4 zi = hh_i4{0, 0, 0, 0};

#pragma unroll 1
    for (uint32_t j0 = 0; j0 < (uint32_t)S; j0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const uint32_t j = j0 + (uint32_t)s;
            // items past a short last chunk add nothing: their d and dmin read as zero (their
            // stage repeats item 0's)
            const bool valid = j < ns;
            const uint8_t* st = stages + (valid ? j : 0u) * SB;
            // the item's B fragments of the eight sub-blocks, their scales d * sc_j and the
            // mins, decoded straight from the ring slot, which is then refilled at once (the
            // last D refills of a chunk re-read its first item from the cache: no branch)
            long w[NT][8];
            float dsc[NT][8];
            hh_mmq_head hd[NT];
#pragma unroll
            for (int q = 0; q < NT; q++) {
                uint4 h = ring[s][q].h;
                if (!valid) h.x = 0u;
#pragma unroll
                for (int sj = 0; sj < 8; sj++) {
                    const uint2 p = ring[s][q].q[sj >> 1];
                    const uint32_t lo = (sj & 1) ? (p.x >> 4) & 0x0F0F0F0Fu : p.x & 0x0F0F0F0Fu;
                    const uint32_t hi = (sj & 1) ? (p.y >> 4) & 0x0F0F0F0Fu : p.y & 0x0F0F0F0Fu;
                    w[q][sj] = (long)(((uint64_t)hi << 32) | lo);
                    dsc[q][sj] = hh_mmq_dsc(h, (uint32_t)sj);
                }
                hh_mmq_mins(h, c, hd[q]);
            }
            __builtin_amdgcn_sched_barrier(0);
            issue(j + D, ring[s]);
            const float* ms = reinterpret_cast<const float*>(st + 288u * TP);
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                // min term: A = s_tj * sum xq (token r16 of tile tt, sub-blocks c and c + 4)
                const float am0 = ms[c * TP + tt * 16 + r16];
                const float am1 = ms[(c + 4u) * TP + tt * 16 + r16];
#pragma unroll
                for (int q = 0; q < NT; q++) {
                    acc[q][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, hd[q].nm0, acc[q][tt], 0, 0, 0);
                    acc[q][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, hd[q].nm1, acc[q][tt], 0, 0, 0);
                }
                // main term, software-pipelined: the MFMAs of sub-block sj are issued before the
                // f32 scaling of sub-block sj - 1 (d sc_j s_tj per output)
                hh_i4 cc[NT];
                float4 sp = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int sj = 0; sj <= 8; sj++) {
                    hh_i4 cn[NT];
                    float4 sn = sp;
                    if (sj < 8) {
                        const long xa =
                            *reinterpret_cast<const long*>(st + ((size_t)(4u * sj + c) * TP + tt * 16 + r16) * 8u);
                        sn = *reinterpret_cast<const float4*>(st + 256u * TP + ((uint32_t)sj * TP + tt * 16 + 4u * c) * 4u);
#pragma unroll
                        for (int q = 0; q < NT; q++) cn[q] = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, w[q][sj], zi, 0, 0, 0);
                    }
                    if (sj > 0) {
#pragma unroll
                        for (int q = 0; q < NT; q++) {
                            const float f = dsc[q][sj - 1];
                            acc[q][tt][0] = fmaf((float)cc[q][0], f * sp.x, acc[q][tt][0]);
                            acc[q][tt][1] = fmaf((float)cc[q][1], f * sp.y, acc[q][tt][1]);
                            acc[q][tt][2] = fmaf((float)cc[q][2], f * sp.z, acc[q][tt][2]);
                            acc[q][tt][3] = fmaf((float)cc[q][3], f * sp.w, acc[q][tt][3]);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    if (sj < 8) {
#pragma unroll
                        for (int q = 0; q < NT; q++) cc[q] = cn[q];
                        sp = sn;
                    }
                }
            }
        }
    }

    // partials [tile][r][lane]: every store and load instruction covers 256 contiguous bytes
    if (a.kc > 1) {
        constexpr uint32_t PT = NT * TT * 4u * HH_WAVE;
        float* my = a.part + (((size_t)grp * a.kc + kci) * a.nw + wave) * PT + lane;
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) hh_store_coherent_f(my + ((q * TT + tt) * 4 + r) * HH_WAVE, acc[q][tt][r]);
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
        // the last to arrive adds all chunks' partials in chunk order
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) acc[q][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};
        for (uint32_t k = 0; k < a.kc; k++) {
            const float* p = a.part + (((size_t)grp * a.kc + k) * a.nw + wave) * PT + lane;
#pragma unroll
            for (int q = 0; q < NT; q++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[q][tt][r] += hh_load_coherent_f(p + ((q * TT + tt) * 4 + r) * HH_WAVE);
        }
    }
    if (!live) return;

    // C lane (quarter c, row r16): acc[q][tt][r] is token 16 tt + 4 c + r of row R
    const uint32_t R = unit * 16 + r16;
    if (R >= a.m) return;
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t tok = tt * 16u + 4u * c + (uint32_t)r;
            if (tok < a.b) {
                const float v = NT == 2 ? hh_act_mul(acc[0][tt][r], acc[NT - 1][tt][r], a.act) : acc[0][tt][r];
                a.y[(size_t)tok * a.m + R] = v;
            }
        }
}

#define HH_MMQ(S, TT, DG, DF)                                                                             \
    extern "C" __global__ void __launch_bounds__(HH_MMQ_BLOCK) hh_q4k_mmq_s##S##_t##TT(const hh_mmq_args a) { \
        hh_mmq_body<1, TT, S, DG>(a);                                                                     \
    }                                                                                                     \
    extern "C" __global__ void __launch_bounds__(HH_MMQ_BLOCK) hh_q4k_mmq_gu_s##S##_t##TT(const hh_mmq_args a) { \
        hh_mmq_body<2, TT, S, DF>(a);                                                                     \
    }
// S: superblocks per chunk (LDS holds S stages of 320 * 16 TT bytes); the ring depths (GEMM,
// gate/up) divide S
HH_MMQ(2, 1, 2, 2)
HH_MMQ(4, 1, 4, 4)
HH_MMQ(7, 1, 7, 7)
HH_MMQ(8, 1, 8, 4)
HH_MMQ(14, 1, 7, 7)
HH_MMQ(16, 1, 8, 4)
HH_MMQ(2, 2, 2, 2)
HH_MMQ(4, 2, 4, 4)
HH_MMQ(7, 2, 7, 7)
HH_MMQ(8, 2, 8, 4)
HH_MMQ(14, 2, 7, 7)
HH_MMQ(2, 3, 2, 2)
HH_MMQ(4, 3, 4, 2)
HH_MMQ(7, 3, 7, 7)
HH_MMQ(8, 3, 4, 2)
HH_MMQ(2, 4, 2, 2)
HH_MMQ(4, 4, 4, 2)
HH_MMQ(6, 4, 6, 2)
HH_MMQ(7, 4, 7, 7)
