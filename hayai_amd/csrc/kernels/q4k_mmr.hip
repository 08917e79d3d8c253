// Batched Q4_K on the matrix cores as one weight stream per launch (gfx950), for up to 16
// tokens (one 16-token tile):
//   hh_q4k_mmr_gu_s<S>  FFN gate/up + act: h = act(W_gate . X) * (W_up . X), written as
//                       token stages of the down projection (prefill_batched's gate/up and
//                       host SiLU*up, crates/hayai-core/src/prefill_wave.rs:569-584, fused)
//   hh_q4k_mmr_dn_s<S>  Y = W_down . H from those stages (prefill_wave.rs:579-584)
//   hh_q4k_mmr_s<S>     Y = W . X from f32 tokens (ggml_gemv_batched_q4_k,
//                       crates/hayai-opencl/src/compute.rs:179-257)
// (Compiled after q4k_mm.hip: the same MFMA arithmetic, tile decode and token-stage layout.)
//
// Work split: rows in 16-row units (FFN: the gate tile and the up tile of the same 16
// rows), superblocks in chunks of S.  A workgroup owns nw units of one chunk.  It builds the
// chunk's S token stages in LDS once (S x 17 KB: from f32 tokens, or copied by LDS DMA from
// stages in global memory), then each of its nw waves streams its own unit's S superblocks
// through a ring of D items in flight.  An item is the lane's 48 bytes of each tile (block
// header + 32 qs bytes, the operands of hh_mm_decode) at a wave-uniform base plus fixed
// lane offsets, so wait counts are static and no barrier or exchange stands between the
// weight stream and the MFMAs.
// The chunks of one row group meet in a workspace: each workgroup writes its partial sums
// with device-coherent stores, and the last to arrive (per-row-group counter, reset by it)
// adds them in chunk order, so results do not depend on arrival order.
// Token columns b..15 of the stages are never initialised: an MFMA output column depends
// only on its own B column, so whatever they hold stays in outputs that are never stored.

struct hh_mmr_args {
    const uint8_t* w0;  // GEMM: W; FFN: W_gate   [m][row_bytes]
    const uint8_t* w1;  // FFN: W_up
    const void* x;      // f32 tokens [b][n], or token stages [n/256] (down projection)
    float* y;           // GEMM: [b][m] f32
    uint8_t* hop;       // FFN: h as token stages [m/256]
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
#define HH_MMR_XROUNDS 5  // token-staging jobs per thread kept in registers ahead of the ring

// One staging job: token t, half-sub-block hs (16 elements) of the chunk, from 4 float4 of
// f32 tokens into hi/lo f16 operands and the half's sum (as hh_mm_prep).
HH_DEV void hh_mmr_stage_job(uint8_t* stages, uint32_t t, uint32_t hs, const float4* v) {
    uint8_t* st = stages + (hs / 16u) * HH_MM_STAGE;
    const uint32_t h = hs % 16u;
    const float e[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                         v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
    float s = 0.f;
#pragma unroll
    for (int half8 = 0; half8 < 2; half8++) {
        hh_h8 hi, lo;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            _Float16 vh, vl;
            hh_split_f16(e[8 * half8 + k], vh, vl);
            hi[k] = vh;
            lo[k] = vl;
            s += e[8 * half8 + k];
        }
        const uint32_t off = hh_mm_elem_off(t, h * 16 + 8 * half8);
        *reinterpret_cast<hh_h8*>(st + off) = hi;
        *reinterpret_cast<hh_h8*>(st + 8192 + off) = lo;
    }
    _Float16 sh, sl;
    hh_split_f16(s, sh, sl);
    const uint32_t so = hh_mm_sum_off(t, h);
    *reinterpret_cast<_Float16*>(st + so) = sh;
    *reinterpret_cast<_Float16*>(st + 512 + so) = sl;
}

HH_DEV void hh_mmr_load_job(const float* x, uint32_t n, uint32_t sb0, uint32_t per_tok, uint32_t job, float4* v,
                            uint32_t& t, uint32_t& hs) {
    t = job / per_tok;
    hs = job % per_tok;
    const float4* src = reinterpret_cast<const float4*>(x + (size_t)t * n + (size_t)sb0 * 256 + (size_t)hs * 16);
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] = src[q];
}

// FFN: NT = 2 tiles per unit (gate, up); GEMM: 1.  XF32: tokens arrive as f32 (else as
// stages in global memory).  S superblocks per chunk, D ring items in flight per wave, P of
// them issued before the f32 tokens are converted.
template <bool FFN, bool XF32, int S, int D, int P>
HH_DEV void hh_mmr_body(const hh_mmr_args& a) {
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];  // S token stages
    __shared__ int last_flag;
    constexpr int NT = FFN ? 2 : 1;
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

    if constexpr (XF32) {
        // f32 tokens: the first HH_MMR_XROUNDS jobs per thread are loaded before any weight
        // request (surplus threads repeat the last job: identical bytes to the same place)
        const float* x = reinterpret_cast<const float*>(a.x);
        const uint32_t per_tok = ns * 16u;
        const uint32_t jobs = a.b * per_tok;
        float4 xv[HH_MMR_XROUNDS][4];
        uint32_t jt[HH_MMR_XROUNDS], jh[HH_MMR_XROUNDS];
#pragma unroll
        for (int k = 0; k < HH_MMR_XROUNDS; k++)
            hh_mmr_load_job(x, a.n, sb0, per_tok, min(tid + (uint32_t)k * nthr, jobs - 1), xv[k], jt[k], jh[k]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < (P < D0 ? P : D0); s++) issue(s, ring[s]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < HH_MMR_XROUNDS; k++) hh_mmr_stage_job(stages, jt[k], jh[k], xv[k]);
        for (uint32_t job = tid + HH_MMR_XROUNDS * nthr; job < jobs; job += nthr) {  // few waves only
            float4 v[4];
            uint32_t t, hs;
            hh_mmr_load_job(x, a.n, sb0, per_tok, job, v, t, hs);
            hh_mmr_stage_job(stages, t, hs, v);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = (P < D0 ? P : D0); s < D0; s++) issue(s, ring[s]);
    } else {
        // stages in global memory: LDS DMA of the chunk (17 * 64 chunks of 16 bytes per
        // stage), then the ring; the DMA is complete once at most the ring's loads remain
        const uint8_t* src = reinterpret_cast<const uint8_t*>(a.x) + (size_t)sb0 * HH_MM_STAGE;
        const uint32_t chunks = ns * (HH_MM_STAGE / 16u);
        for (uint32_t c0 = wave * HH_WAVE; c0 < chunks; c0 += nthr)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + (size_t)(c0 + lane) * 16),
                                             (__attribute__((address_space(3))) void*)(stages + (size_t)c0 * 16), 16, 0, 0);
#pragma unroll
        for (int s = 0; s < D0; s++) issue(s, ring[s]);
        constexpr uint32_t pend = (uint32_t)(D0 * NT * 3);  // vmcnt: only ring loads may remain
        static_assert(pend < 64, "ring loads exceed the vmcnt range");
        __builtin_amdgcn_s_waitcnt((pend & 0xFu) | (0x7u << 4) | (0xFu << 8) | ((pend >> 4) << 14));
    }
    __syncthreads();  // the chunk's token stages are in LDS

    hh_f4 acc[NT];
#pragma unroll
    for (int q = 0; q < NT; q++) acc[q] = hh_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < S; j++) {
        hh_mm_tile t[NT];
#pragma unroll
        for (int q = 0; q < NT; q++) hh_mm_decode(ring[j % D][q].h, ring[j % D][q].q0, ring[j % D][q].q1, c, lane, t[q]);
        if (j + D < S) issue(j + D, ring[j % D]);
        // items past a short last chunk add nothing: their weights and token stage repeat
        // item 0's (finite values, scaled by zero)
        uint32_t jst = (uint32_t)j;
        if (j > 0) {
            jst = (uint32_t)j < ns ? (uint32_t)j : 0u;
            const float keep = (uint32_t)j < ns ? 1.f : 0.f;
#pragma unroll
            for (int q = 0; q < NT; q++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    t[q].d4[r] *= keep;
                    t[q].dmin4[r] *= keep;
                }
        }
        const uint8_t* st = stages + jst * HH_MM_STAGE;
        const hh_f4 z = hh_f4{0.f, 0.f, 0.f, 0.f};
        hh_f4 sq[NT], sm[NT];
#pragma unroll
        for (int q = 0; q < NT; q++) sq[q] = z;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const hh_h8 xh = *reinterpret_cast<const hh_h8*>(st + (s * 64 + lane) * 16);
#pragma unroll
            for (int q = 0; q < NT; q++) sq[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(t[q].a[s], xh, sq[q], 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const hh_h8 xl = *reinterpret_cast<const hh_h8*>(st + 8192 + (s * 64 + lane) * 16);
#pragma unroll
            for (int q = 0; q < NT; q++) sq[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(t[q].a[s], xl, sq[q], 0, 0, 0);
        }
        const hh_h4 shi = *reinterpret_cast<const hh_h4*>(st + 16384 + lane * 8);
        const hh_h4 slo = *reinterpret_cast<const hh_h4*>(st + 16896 + lane * 8);
#pragma unroll
        for (int q = 0; q < NT; q++) {
            sm[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(t[q].amin, shi, z, 0, 0, 0);
            sm[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(t[q].amin, slo, sm[q], 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < NT; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[q][r] = fmaf(t[q].d4[r], sq[q][r], acc[q][r]);
                acc[q][r] = fmaf(t[q].dmin4[r], sm[q][r], acc[q][r]);
            }
    }

    // D lane (token r16, quarter c) holds rows 4c..4c+3 of its unit.  Partials are laid out
    // [tile][row r][lane] so every store and load instruction covers 256 contiguous bytes.
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

    const uint32_t rbase = unit * 16 + 4 * c;
    if constexpr (FFN) {
        // h of rows rbase..rbase+3, token r16 -> the down projection's token stages (n = m).
        // Lanes c and c^1 swap their rows, so each holds the 8-row run 8(c/2).. of its token and
        // writes one 16-byte chunk of it: the hi halves (c even) or the lo halves (c odd).
        float h[4];
        float hsum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            h[r] = hh_act_mul(acc[0][r], acc[1][r], a.act);
            hsum += h[r];
        }
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; r++) o[r] = __shfl_xor(h[r], 16, HH_WAVE);
        const bool odd = (c & 1u) != 0;
        hh_h8 run;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float first = odd ? o[r] : h[r];  // rows 8p + r
            const float second = odd ? h[r] : o[r];  // rows 8p + 4 + r
            _Float16 hi0, lo0, hi1, lo1;
            hh_split_f16(first, hi0, lo0);
            hh_split_f16(second, hi1, lo1);
            run[r] = odd ? lo0 : hi0;
            run[4 + r] = odd ? lo1 : hi1;
        }
        const uint32_t e0 = unit * 16 + 8 * (c >> 1);  // first row of the run
        uint8_t* st = a.hop + (size_t)(e0 / 256) * HH_MM_STAGE;
        *reinterpret_cast<hh_h8*>(st + (odd ? 8192u : 0u) + hh_mm_elem_off(r16, e0 & 255u)) = run;
        // the unit's 16 rows are one half-sub-block of h: their sum feeds the min term
        hsum += __shfl_xor(hsum, 16, HH_WAVE);
        hsum += __shfl_xor(hsum, 32, HH_WAVE);
        if (c == 0) {
            _Float16 hi, lo;
            hh_split_f16(hsum, hi, lo);
            uint8_t* ss = a.hop + (size_t)(unit * 16 / 256) * HH_MM_STAGE;
            const uint32_t off = hh_mm_sum_off(r16, (unit * 16 & 255u) / 16);
            *reinterpret_cast<_Float16*>(ss + off) = hi;
            *reinterpret_cast<_Float16*>(ss + 512 + off) = lo;
        }
    } else {
        if (r16 < a.b) {
            float* yp = a.y + (size_t)r16 * a.m + rbase;
            if (rbase + 4 <= a.m && ((uintptr_t)yp & 15u) == 0) {
                *reinterpret_cast<float4*>(yp) = make_float4(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (rbase + r < a.m) yp[r] = acc[0][r];
            }
        }
    }
}

#define HH_MMR_BLOCK (HH_MMR_MAX_WAVES * HH_WAVE)
#define HH_MMR_KERNELS(S)                                                                               \
    extern "C" __global__ void __launch_bounds__(HH_MMR_BLOCK) hh_q4k_mmr_gu_s##S(const hh_mmr_args a) { \
        hh_mmr_body<true, true, S, 4, 2>(a);                                                            \
    }                                                                                                   \
    extern "C" __global__ void __launch_bounds__(HH_MMR_BLOCK) hh_q4k_mmr_dn_s##S(const hh_mmr_args a) { \
        hh_mmr_body<false, false, S, S, S>(a);                                                          \
    }                                                                                                   \
    extern "C" __global__ void __launch_bounds__(HH_MMR_BLOCK) hh_q4k_mmr_s##S(const hh_mmr_args a) {    \
        hh_mmr_body<false, true, S, S, 4>(a);                                                           \
    }
HH_MMR_KERNELS(2)
HH_MMR_KERNELS(4)
HH_MMR_KERNELS(7)
HH_MMR_KERNELS(8)
