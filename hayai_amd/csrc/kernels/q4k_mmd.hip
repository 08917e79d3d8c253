// Batched Q4_K on the int8 matrix cores with the weights staged through LDS by DMA, up to 16
// tokens per pass:
//   hh_q4k_mmd_gu_k<KR>   H[b][m] = act(W_gate . X) * (W_up . X) (prefill_batched's gate/up and
//                         SiLU * up, crates/hayai-core/src/prefill_wave.rs:569-584, fused)
//   hh_q4k_mmd_k<KR>      Y[b][m] = W . X (ggml_gemv_batched_q4_k, crates/hayai-opencl/src/
//                         compute.rs:179-257; execute_quant_gemv_batched, crates/hayai-core/src/
//                         orchestrator.rs:240-269)
// from the int8 token stages hh_mmq_prep writes (q4k_mmq.hip: the same arithmetic per
// superblock, the same stage layout).
//
// Access pattern.  A q4k_mmq wave reads its MFMA B fragments straight from memory: every load
// instruction touches 16 rows x 32 bytes, which streams at 2-2.7 TB/s.  Here a step is 16 rows
// (of each of the NT matrices) x SU superblocks; its bytes travel as row runs of SU * 144
// consecutive bytes into an LDS ring slot by global_load_lds (16 bytes per lane: a load
// instruction covers 1 KB of row bytes), and the fragments are read from LDS.  Slot rows are
// SU * 144 + 16 bytes apart (the 16-byte pad puts the 16 rows of a fragment read on different
// banks).
//
// Work split (stream-K).  Steps are ordered (K-range r of KR superblocks, row tile t, step s of
// the range); workgroup w (one per CU, sixteen waves) takes steps [w S / G, (w + 1) S / G).
// Wave v computes sub-blocks 4 (v / 8) .. + 3 of item v % 8 = (matrix % NT, superblock / NT)
// of each step and accumulates while the steps stay in one (r, t) segment.  At a segment's end
// the waves' sums meet in LDS (in wave order).  A tile that one segment covers is written at
// once (with the activation for gate/up); every other segment stores a partial under its first
// K-step, and after the workgroup's last step adds its length to the tile's counter: the
// workgroup that completes the count adds the tile's partials in K order (deterministic) and
// writes the result.  The token stages of a K-range (KR x 5 KB) are copied into LDS once: a
// workgroup's steps span at most two ranges.
//
// Waits.  Waves 0..7 issue the copies, the same number each per step (IPU; the last block of a
// slot is clamped so it ends inside the slot, surplus lanes rewriting bytes that other lanes
// also write), so "step i has landed" is vmcnt <= (RING - 2) * IPU on those waves followed by
// a barrier (step i - 1's slot is refilled right after it).
//
// Status: correct (held to the quantized-activation oracle) but slower than the f16 kernels
// of q4k_mmr.hip at 16 tokens, so the engine uses it only when asked (HAYAI_HIP_MMD=1).  8B
// FFN layer, 16 tokens (rocprofv3): gate/up 23.3 us, down 19.2 us (+ two 4.6 us token preps)
// against 24.5 + 13.2 us (+ one 4.8 us prep) on the f16 kernels.  Probe builds: without the
// arithmetic the same structure streams the layer in 18.4 + 15.8 us (with an 8-slot ring and
// no token stages, 19.2 + 17.4 us: not a matter of bytes in flight); without the weight
// copies it computes in 19.5 + 16.1 us.  The arithmetic is the cost: each 32-column
// sub-block's int32 tile needs cvt + mul + fma per output (d sc_j s_tj differs per row,
// token and sub-block), about 107 VALU instructions per wave and half-superblock, where the
// f16 form applies d once per superblock.

#define HH_MMD_MAX_SEG 32
#define HH_MMD_WAVES 16

struct hh_mmd_args {
    const uint8_t* w0;  // GEMM: W; FFN: W_gate   [m][row_bytes]
    const uint8_t* w1;  // FFN: W_up (GEMM: = w0)
    const uint8_t* xs;  // token stages [n / 256][320 * 16]
    float* y;           // GEMM: Y [b][m]; FFN: H [b][m]
    float* part;        // [tiles][n / (256 SU)][NT * 256] partial sums
    unsigned* cnt;      // [tiles] K-steps done (zero between launches)
    uint64_t row_bytes;
    uint32_t m;         // rows
    uint32_t n;         // columns (multiple of 256 KR)
    uint32_t b;         // valid tokens (<= 16)
    uint32_t tiles;     // (m + 15) / 16
    int32_t act;
    uint32_t pad;
};

// s_waitcnt immediate for vmcnt <= n (expcnt and lgkmcnt not waited for)
constexpr int hh_vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// 16 bytes per lane global -> LDS at lds + 16 * lane (lds wave-uniform).  Issued from inline
// assembly so that the compiler does not track it: with the builtin it waits for every copy in
// flight (vmcnt(0)) before any LDS read, which would drain the ring at every step; the kernel
// waits for its copies itself.  (M0 holds the LDS address; one wait state before its use.)
// No other code of these kernels uses M0, so nothing needs it preserved across the statement.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
HH_DEV void hh_dma16(const void* src, const char* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

// A workgroup barrier for LDS traffic only.  __syncthreads() also orders global memory, so
// after a global store it waits for vmcnt(0), i.e. for every copy in flight; here each wave
// waits for its own LDS accesses (lgkmcnt(0)) and the copies stay in flight.
HH_DEV void hh_lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited for
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One wave's share of a step: sub-blocks 4 H .. 4 H + 3 of one superblock of one 16-row tile
// (wrow: the lane's row in the slot), tokens' stage st.  Min term: the f32 MFMA over the four
// lane groups c, i.e. sub-block c + 4 H; main term: one int8 MFMA per sub-block, its int32
// sums scaled by d sc_j s_tj (the MFMA of sub-block j issued before the scaling of j - 1).
template <int H, uint32_t TP>
HH_DEV void hh_mmd_item(const char* wrow, const char* st, uint32_t c, uint32_t r16, hh_f4& acc) {
    const hh_i4 zi = hh_i4{0, 0, 0, 0};
    const uint4 h = *reinterpret_cast<const uint4*>(wrow);
    uint2 qp[2];
#pragma unroll
    for (int g = 0; g < 2; g++) qp[g] = *reinterpret_cast<const uint2*>(wrow + 16u + 32u * (2 * H + g) + 8u * c);
    long wv[4];
    float dsc[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint2 pp = qp[k >> 1];
        const uint32_t lo = (k & 1) ? (pp.x >> 4) & 0x0F0F0F0Fu : pp.x & 0x0F0F0F0Fu;
        const uint32_t hi = (k & 1) ? (pp.y >> 4) & 0x0F0F0F0Fu : pp.y & 0x0F0F0F0Fu;
        wv[k] = (long)(((uint64_t)hi << 32) | lo);
        dsc[k] = hh_mmq_dsc(h, (uint32_t)(4 * H + k));
    }
    hh_mmq_head hd;
    hh_mmq_mins(h, c, hd);
    const float* ms = reinterpret_cast<const float*>(st + 288u * TP);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ms[(c + 4u * H) * TP + r16], H ? hd.nm1 : hd.nm0, acc, 0, 0, 0);
    hh_i4 cc = zi;
    float4 sp = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k <= 4; k++) {
        const uint32_t sj = (uint32_t)(4 * H + k);
        hh_i4 cn = zi;
        float4 sn = sp;
        if (k < 4) {
            const long xa = *reinterpret_cast<const long*>(st + ((4u * sj + c) * TP + r16) * 8u);
            sn = *reinterpret_cast<const float4*>(st + 256u * TP + (sj * TP + 4u * c) * 4u);
            cn = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, wv[k], zi, 0, 0, 0);
        }
        if (k > 0) {
            const float f = dsc[k - 1];
            acc[0] = fmaf((float)cc[0], f * sp.x, acc[0]);
            acc[1] = fmaf((float)cc[1], f * sp.y, acc[1]);
            acc[2] = fmaf((float)cc[2], f * sp.z, acc[2]);
            acc[3] = fmaf((float)cc[3], f * sp.w, acc[3]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (k < 4) {
            cc = cn;
            sp = sn;
        }
    }
}

template <int NT, int SU, int KR, int RING>
HH_DEV void hh_mmd_body(const hh_mmd_args& a) {
    constexpr uint32_t TP = 16u, SB = 320u * TP;          // tokens per tile, stage bytes per superblock
    constexpr uint32_t GR = SU * 9u + 1u;                 // 16-byte granules per slot row (+ pad)
    constexpr uint32_t PITCH = GR * 16u, ROWS = NT * 16u, SLOT = ROWS * PITCH;
    constexpr uint32_t P = ROWS * GR, IPU = (P + 511u) / 512u;
    constexpr uint32_t AB = KR * SB, SPR = KR / SU;
    static_assert(NT * SU == 8, "one (matrix, superblock) item per wave and step");
    static_assert(KR % SU == 0 && (AB / 16u) % 512u == 0, "K-range layout");
    static_assert((RING - 2) * IPU <= 63, "vmcnt range");
    static_assert(SLOT >= HH_MMD_WAVES * 256u * 4u, "a slot holds the segment reduction");
    static_assert(RING >= 2, "ring depth");
    extern __shared__ __attribute__((aligned(16))) char hh_smem[];
    __shared__ uint32_t seg_t[HH_MMD_MAX_SEG], seg_len[HH_MMD_MAX_SEG];
    __shared__ uint32_t s_nseg;
    __shared__ int s_last;

    const uint32_t tid = threadIdx.x, lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t nsb = a.n / 256u, nr = nsb / KR, KS = nsb / SU, tiles = a.tiles;
    const uint32_t per_r = tiles * SPR, S = nr * per_r;
    const uint32_t x0 = (uint32_t)(((uint64_t)w * S) / G), x1 = (uint32_t)(((uint64_t)(w + 1) * S) / G);
    if (x0 >= x1) return;  // the whole workgroup
    const uint32_t nst = x1 - x0;
    const uint32_t r0 = x0 / per_r, r1 = (x1 - 1u) / per_r;  // r1 <= r0 + 1 (host)
    char* const A0 = hh_smem;
    char* const ring = hh_smem + (nr > 1u ? 2u : 1u) * AB;
    if (tid == 0) s_nseg = 0;

    auto decode = [&](uint32_t x, uint32_t& r, uint32_t& t, uint32_t& s) {
        r = x / per_r;
        const uint32_t rem = x - r * per_r;
        t = rem / SPR;
        s = rem - t * SPR;
    };
    // step x0 + min(i, nst - 1) -> slot i % RING (steps past the end repeat the last one into a
    // slot nobody reads again)
    auto issue = [&](uint32_t i) {
        uint32_t r, t, s;
        decode(x0 + min(i, nst - 1u), r, t, s);
        const size_t cofs = (size_t)(r * KR + s * SU) * 144u;
        char* const dst = ring + (i % RING) * SLOT;
#pragma unroll
        for (uint32_t k = 0; k < IPU; k++) {
            const uint32_t blk = min(k * 512u + wave * 64u, P - 64u);
            const uint32_t p = blk + lane;
            const uint32_t l = p / GR, col = p - l * GR;
            const uint32_t row = min(t * 16u + (l & 15u), a.m - 1u);
            const uint8_t* src = (l >= 16u ? a.w1 : a.w0) + (size_t)row * a.row_bytes + cofs +
                                 (col < SU * 9u ? col : 0u) * 16u;
            hh_dma16(src, dst + blk * 16u);
        }
    };
    // K-step k of tile t opens a segment: a K-range's first step or a workgroup's first step
    auto seg_first = [&](uint32_t t, uint32_t k) {
        const uint32_t r = k / SPR, s = k - r * SPR;
        if (s == 0) return true;
        const uint32_t x = (r * tiles + t) * SPR + s;
        const uint64_t wf = ((uint64_t)x * G + S - 1u) / S;  // first workgroup starting at or after x
        return wf < G && (uint32_t)((wf * S) / G) == x;
    };

    // the K-ranges' token stages, then the ring.  Only waves 0..7 copy (IPU instructions per
    // step each), so a copier's wait for a step is a fixed count.
    const bool copier = wave < 8u;
    if (copier) {
        for (uint32_t k = 0; k <= r1 - r0; k++) {
            const uint8_t* src = a.xs + (size_t)(r0 + k) * AB;
            char* const dst = A0 + k * AB;
            for (uint32_t c0 = wave * 64u; c0 < AB / 16u; c0 += 512u)
                hh_dma16(src + (size_t)(c0 + lane) * 16u, dst + c0 * 16u);
        }
#pragma unroll
        for (uint32_t i = 0; i + 1u < (uint32_t)RING; i++) issue(i);

    }

    // wave v: item v % 8 = (matrix, superblock of the step), sub-blocks 4 (v / 8) .. + 3
    const uint32_t item = wave % 8u, half = wave / 8u;
    const uint32_t q = item % NT, sbl = item / NT;
    const uint32_t c = lane >> 4, r16 = lane & 15u;
    hh_f4 acc = hh_f4{0.f, 0.f, 0.f, 0.f};
    uint32_t seg_i0 = 0;

#pragma unroll 1
    for (uint32_t i = 0; i < nst; i++) {
        if (copier) __builtin_amdgcn_s_waitcnt(hh_vmcnt_imm((RING - 2) * IPU));
        hh_lds_barrier();  // step i's slot (and the stages) have landed; step i - 1's slot is free
        if (copier) issue(i + (uint32_t)RING - 1u);  // into slot (i - 1) % RING

        uint32_t r, t, s;
        decode(x0 + i, r, t, s);
        const char* const slot = ring + (i % RING) * SLOT;
        const char* const wrow = slot + (q * 16u + r16) * PITCH + sbl * 144u;
        const char* const st = A0 + (r - r0) * AB + (s * SU + sbl) * SB;
        if (half == 0u)
            hh_mmd_item<0, TP>(wrow, st, c, r16, acc);
        else
            hh_mmd_item<1, TP>(wrow, st, c, r16, acc);
        bool end = i + 1u == nst;
        if (!end) {
            uint32_t r2, t2, s2;
            decode(x0 + i + 1u, r2, t2, s2);
            end = r2 != r || t2 != t;
        }
        if (end) {  // workgroup-uniform: the waves' sums meet in the slot just read
            hh_lds_barrier();
            float* const red = reinterpret_cast<float*>(const_cast<char*>(slot));
#pragma unroll
            for (int rr = 0; rr < 4; rr++) red[(wave * 4u + (uint32_t)rr) * HH_WAVE + lane] = acc[rr];
            hh_lds_barrier();
            // the sum of matrix qq over the waves holding it, in wave order
            auto wsum = [&](uint32_t qq, uint32_t rr, uint32_t ln) {
                float v = 0.f;
#pragma unroll
                for (uint32_t hf = 0; hf < 2u; hf++)
#pragma unroll
                    for (uint32_t sb = 0; sb < (uint32_t)SU; sb++)
                        v += red[((hf * 8u + sb * NT + qq) * 4u + rr) * HH_WAVE + ln];
                return v;
            };
            const uint32_t s_first = s + seg_i0 - i, len = i - seg_i0 + 1u;
            // C lane (quarter cq, row rq): value rr is token 4 cq + rr of row 16 t + rq
            if (nr == 1u && len == SPR) {  // the whole tile: the result
                if (tid < 256u) {
                    const uint32_t rr = tid / HH_WAVE, ln = tid % HH_WAVE;
                    const float g = wsum(0u, rr, ln);
                    const uint32_t tok = 4u * (ln >> 4) + rr, row = t * 16u + (ln & 15u);
                    if (tok < a.b && row < a.m)
                        a.y[(size_t)tok * a.m + row] = NT == 2 ? hh_act_mul(g, wsum(NT - 1u, rr, ln), a.act) : g;
                }
            } else {  // a partial under the segment's first K-step
                if (tid < NT * 256u) {
                    const uint32_t qq = tid / 256u, rr = (tid / HH_WAVE) % 4u, ln = tid % HH_WAVE;
                    hh_store_coherent_f(a.part + ((size_t)t * KS + r * SPR + s_first) * (NT * 256u) + tid, wsum(qq, rr, ln));
                }
                if (tid == 0) {
                    seg_t[s_nseg] = t;
                    seg_len[s_nseg] = len;
                    s_nseg = s_nseg + 1u;
                }
            }
            acc = hh_f4{0.f, 0.f, 0.f, 0.f};
            seg_i0 = i + 1u;
            // the next step's barrier comes before this slot is refilled
        }
    }

    // publish the partial segments (one thread each, all at once); the workgroup that
    // completes a tile adds its partials in K order
    __builtin_amdgcn_s_waitcnt(0);  // partial stores complete (and the surplus copies)
    __syncthreads();
    const uint32_t nseg = s_nseg;
    if (tid < nseg) {
        const uint32_t t = seg_t[tid], len = seg_len[tid];
        const unsigned old = __hip_atomic_fetch_add(a.cnt + t, len, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + len == KS;
        if (last) __hip_atomic_store(a.cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        seg_len[tid] = last ? 1u : 0u;
    }
    __syncthreads();
    for (uint32_t e = tid / 256u; e < nseg; e += HH_MMD_WAVES / 4u) {  // 256 threads per tile
        if (seg_len[e] == 0u) continue;
        const uint32_t t = seg_t[e], o = tid % 256u;
        float v[NT];
#pragma unroll
        for (int qq = 0; qq < NT; qq++) v[qq] = 0.f;
        for (uint32_t k = 0; k < KS; k++) {
            if (!seg_first(t, k)) continue;
            const float* p = a.part + ((size_t)t * KS + k) * (NT * 256u) + o;
#pragma unroll
            for (int qq = 0; qq < NT; qq++) v[qq] += hh_load_coherent_f(p + qq * 256u);
        }
        const uint32_t rr = o / HH_WAVE, ln = o % HH_WAVE;
        const uint32_t tok = 4u * (ln >> 4) + rr, row = t * 16u + (ln & 15u);
        if (tok < a.b && row < a.m) a.y[(size_t)tok * a.m + row] = NT == 2 ? hh_act_mul(v[0], v[NT - 1], a.act) : v[0];
    }
}

// <NT, SU, KR, RING>: LDS = (one K-range's stages, or two when the row spans several) + RING
// slots: gate/up 80 KB + 4 x 18.5 KB; the GEMM (down) 2 x 40 KB + 4 x 18.3 KB
extern "C" __global__ void __launch_bounds__(HH_MMD_WAVES * 64) hh_q4k_mmd_gu_k16(const hh_mmd_args a) { hh_mmd_body<2, 4, 16, 4>(a); }
extern "C" __global__ void __launch_bounds__(HH_MMD_WAVES * 64) hh_q4k_mmd_gu_k8(const hh_mmd_args a) { hh_mmd_body<2, 4, 8, 4>(a); }
extern "C" __global__ void __launch_bounds__(HH_MMD_WAVES * 64) hh_q4k_mmd_k8(const hh_mmd_args a) { hh_mmd_body<1, 8, 8, 4>(a); }
