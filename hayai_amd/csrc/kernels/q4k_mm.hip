// Batched Q4_K GEMM on MFMA (gfx950): Y[b][r] = W[r] . X[b] for 2 <= B <= 64 tokens, and
// the batched FFN gate/up(+act) half.  The reference's batched kernel
// (ggml_gemv_q4.cl:349-419, host compute.rs:179-257) re-reads each weight row per token;
// here every weight is read and decoded once per launch and multiplied by all tokens on
// the matrix cores.
//
// Arithmetic (per Q4_K superblock of one row, 8 sub-blocks of 32 elements):
//   sum_k w_k x_k = d * sum_k (sc_k q_k) x_k  -  dmin * sum_sb m_sb * (sum of x over sb)
//   - sc*q is an integer <= 63*15 = 945, exact in f16.  It is built from the nibbles with
//     one v_perm_b32 (bytes -> f16 1024+q) and one packed FMA ((1024+q)*sc - 1024*sc,
//     exact because the FMA rounds only its exact result) per two weights.
//   - x enters as two f16 values, hi = f16(x) and lo = f16(x - hi), so hi + lo carries x
//     to ~2^-22 relative.  v_mfma_f32_16x16x32_f16 accumulates sum_k (sc q)_k (hi_k + lo_k)
//     per superblock in f32 (two MFMAs per step); the superblock's d (f32, exact) scales
//     that partial into the running sum.
//   - The min term: v_mfma_f32_16x16x16_f16 with A = -m (integers, exact) and B = the f32
//     sums of x over 16-element halves of each sub-block, again as hi + lo f16; dmin (f32)
//     scales it per superblock.
//   A single f16 rounding of x alone gives ~3e-4 relative output error, which compounds to
//   ~2e-3 through gate/up -> act -> down; with the hi/lo split the error is that of f32
//   accumulation (~1e-6).
//
// MFMA mapping:
//   - A = weights (16 rows x 32 k), B = tokens (32 k x 16 tokens), D = 16 x 16.  Lane l: A
//     row l%16, B token l%16; lane quarter c = l/16 supplies k-slots 8c..8c+7 (16x16x32) or
//     4c..4c+3 (16x16x16); D holds rows 4c..4c+3 of token l%16.
//   - The k order inside a superblock is free (weights are real values by then): quarter c
//     owns Q4_K group c (qs bytes 32c..32c+31).  Step s < 4 takes the low nibbles of bytes
//     32c+8s..+8 (elements 64c+8s+e), step s >= 4 the high nibbles (elements 64c+32+8(s-4)+e).
//
// Token operands ("stages"): the prep kernel (and the FFN gate/up epilogue, for the down
// projection) write tokens in MFMA operand order, one contiguous 17 KB stage per (16-token
// tile tt, superblock sb):
//   [0, 8192)       hi: step s, lane l (= 16c + token j), 8 halves    -> (64 s + l) * 16 B
//   [8192, 16384)   lo: same
//   [16384, 16896)  half-sub-block sums hi: lane l, 4 halves e (half 4c + e) -> 8 l B
//   [16896, 17408)  sums lo: same
// Stage (tt, sb) starts at (tt * nsb + sb) * 17408.
//
// Work split: a workgroup is 4 waves; wave w owns row pair 4*g + w (two 16-row tiles: two
// consecutive row tiles, or in FFN mode the gate and up tile of the same 16 rows) over the
// workgroup's superblock range.  The 4 waves consume the same stages, which are loaded once
// per workgroup into double-buffered LDS (coalesced 16-byte loads of one contiguous block).
// When rows are few the superblock range is split over ksg workgroups: each writes its
// partial sums to a workspace with device-coherent stores and the last one to arrive (a
// per-row-group counter, reset by that workgroup) adds the partials in k order, so results
// do not depend on arrival order.
#include "quant.h"

typedef _Float16 hh_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 hh_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 hh_h8 __attribute__((ext_vector_type(8)));
typedef float hh_f4 __attribute__((ext_vector_type(4)));

#define HH_MM_WAVES 4
#define HH_MM_BLOCK (HH_MM_WAVES * HH_WAVE)
#define HH_MM_STAGE 17408u  // bytes of one (token tile, superblock) stage
#define HH_MM_STAGE_CHUNKS (HH_MM_STAGE / 16u)

struct hh_mm_args {
    const uint8_t* w0;  // GEMM: the matrix; FFN: W_gate
    const uint8_t* w1;  // FFN: W_up
    const uint8_t* xop; // token stages of the input ([TT][n/256] stages)
    float* y;           // GEMM: [b][m] f32
    uint8_t* hop;       // FFN: act(gate)*up written as token stages of an n = m input
    float* part;        // ksg > 1: [groups][ksg][2 tiles][T][64 rows] partial sums
    unsigned* cnt;      // ksg > 1: arrival counter per row group (zero between launches)
    uint32_t m;         // rows (FFN: rows of gate = rows of up = d_ff)
    uint32_t n;         // columns (multiple of 256)
    uint32_t b;         // valid tokens (<= T)
    uint32_t ksg;       // workgroups splitting the superblocks of one row group
    uint64_t row_bytes;
    int32_t act;
    uint32_t pad;
};

HH_DEV hh_h2 hh_h2_bits(uint32_t v) { return __builtin_bit_cast(hh_h2, v); }

// 8 nibbles (one qs dword, low or high nibbles already isolated as bytes) -> 4 f16 pairs
// of sc*q, exact.
HH_DEV void hh_mm_scq(uint32_t nib, hh_h2 sc2, hh_h2 nb2, hh_h2* out) {
    const uint32_t magic = 0x64646464u;  // f16 0x64qq = 1024 + qq for qq < 16
    const hh_h2 p0 = hh_h2_bits(__builtin_amdgcn_perm(magic, nib, 0x04010400u));
    const hh_h2 p1 = hh_h2_bits(__builtin_amdgcn_perm(magic, nib, 0x04030402u));
    out[0] = __builtin_elementwise_fma(p0, sc2, nb2);
    out[1] = __builtin_elementwise_fma(p1, sc2, nb2);
}

struct hh_mm_tile {
    hh_h8 a[8];      // A operands of the 8 MFMA steps
    hh_h4 amin;      // -m of sub-blocks 2c, 2c, 2c+1, 2c+1
    float d4[4];     // d of the 4 D rows this lane holds
    float dmin4[4];  // dmin of those rows
};

// Decode this lane's part (row l%16, group c) of one superblock into MFMA operands.
HH_DEV void hh_mm_decode(const uint4& h, const uint4& q0, const uint4& q1, uint32_t c, uint32_t lane,
                         hh_mm_tile& t) {
    // [sc(2c), sc(2c+1), m(2c), m(2c+1)] from the 12 scale bytes (q4k.rs:34-43)
    const uint32_t kk = 2u * (c & 1u);
    const uint32_t sel_yz = kk | ((kk + 1u) << 8) | ((kk + 4u) << 16) | ((kk + 5u) << 24);
    const uint32_t sel_w = kk | ((kk + 1u) << 8) | (kk << 16) | ((kk + 1u) << 24);
    const uint32_t b = __builtin_amdgcn_perm(h.z, h.y, sel_yz);
    const uint32_t lo = b & 0x3F3F3F3Fu;
    const uint32_t wp = __builtin_amdgcn_perm(h.w, h.w, sel_w);
    const uint32_t hi = (wp & 0x00000F0Fu) | ((wp >> 4) & 0x0F0F0000u) | ((b >> 2) & 0x30303030u);
    const uint32_t s = c >= 2 ? hi : lo;
    const float sc_lo = hh_ub0(s), sc_hi = hh_ub1(s);
    const float d = hh_f16(h.x & 0xFFFFu);
    const float dmin = hh_f16(h.x >> 16);
    const _Float16 mlo = (_Float16)(-hh_ub2(s));
    const _Float16 mhi = (_Float16)(-hh_ub3(s));
    t.amin = hh_h4{mlo, mlo, mhi, mhi};
    const hh_h2 sl = hh_h2{(_Float16)sc_lo, (_Float16)sc_lo};
    const hh_h2 sh = hh_h2{(_Float16)sc_hi, (_Float16)sc_hi};
    const hh_h2 nl = hh_h2{(_Float16)(-1024.0f * sc_lo), (_Float16)(-1024.0f * sc_lo)};
    const hh_h2 nh = hh_h2{(_Float16)(-1024.0f * sc_hi), (_Float16)(-1024.0f * sc_hi)};
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
        hh_h2 l[4], u[4];
        hh_mm_scq(qw[2 * s4] & 0x0F0F0F0Fu, sl, nl, l);
        hh_mm_scq(qw[2 * s4 + 1] & 0x0F0F0F0Fu, sl, nl, l + 2);
        hh_mm_scq((qw[2 * s4] >> 4) & 0x0F0F0F0Fu, sh, nh, u);
        hh_mm_scq((qw[2 * s4 + 1] >> 4) & 0x0F0F0F0Fu, sh, nh, u + 2);
        t.a[s4] = hh_h8{l[0].x, l[0].y, l[1].x, l[1].y, l[2].x, l[2].y, l[3].x, l[3].y};
        t.a[4 + s4] = hh_h8{u[0].x, u[0].y, u[1].x, u[1].y, u[2].x, u[2].y, u[3].x, u[3].y};
    }
    // d, dmin of D rows 4c'..4c'+3 (c' = this lane's quarter) live in lanes 4c'+i of quarter 0
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int src = (int)((lane >> 4) * 4 + i);
        t.d4[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src * 4, __builtin_bit_cast(int, d)));
        t.dmin4[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src * 4, __builtin_bit_cast(int, dmin)));
    }
}

struct hh_mm_wq {
    uint4 h, q0, q1;
};

HH_DEV void hh_mm_load(const uint8_t* row, uint32_t sb, uint32_t c, hh_mm_wq& w) {
    const uint8_t* blk = row + (size_t)sb * 144;
    w.h = hh_ld16(blk);
    w.q0 = hh_ld16(blk + 16 + 32 * c);
    w.q1 = hh_ld16(blk + 32 + 32 * c);
}

// f32 -> hi + lo f16 pair
HH_DEV void hh_split_f16(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Byte offsets, inside its stage, of token j's element e (0..255 of the superblock) and of
// half-sub-block h (0..15).
HH_DEV uint32_t hh_mm_elem_off(uint32_t j, uint32_t e) {
    const uint32_t c = e >> 6, f = e & 63u;
    const uint32_t s = f < 32 ? (f >> 3) : 4 + ((f - 32) >> 3);
    return (s * 64 + c * 16 + j) * 16 + (f & 7u) * 2;
}
HH_DEV uint32_t hh_mm_sum_off(uint32_t j, uint32_t h) { return 16384u + ((h >> 2) * 16 + j) * 8 + (h & 3u) * 2; }

HH_DEV void hh_store_coherent_f(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
HH_DEV float hh_load_coherent_f(const float* p) {
    return __uint_as_float(__hip_atomic_load(const_cast<uint32_t*>(reinterpret_cast<const uint32_t*>(p)),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// One stage in flight between global memory and LDS: 5 x 16 bytes per thread.  Loads are
// unconditional (index clamped; the surplus of the 5th chunk re-reads the last one), because a
// load under a branch joins into a copy that waits for it at once.
// (A native vector type: copies of HIP's uint4 class lower to memcpy through private memory.)
typedef uint32_t hh_v4u __attribute__((ext_vector_type(4)));
struct hh_mm_pre {
    hh_v4u v0, v1, v2, v3, v4;
};

template <int TT>
HH_DEV void hh_mm_fetch(const hh_mm_args& a, uint32_t g0, uint32_t nsb, uint32_t tid, uint32_t i, hh_mm_pre& p) {
    const uint32_t sb = g0 + i / TT, tt = i % TT;
    const hh_v4u* src = reinterpret_cast<const hh_v4u*>(a.xop + ((size_t)tt * nsb + sb) * HH_MM_STAGE);
    p.v0 = src[tid];
    p.v1 = src[tid + 256];
    p.v2 = src[tid + 512];
    p.v3 = src[tid + 768];
    p.v4 = src[min(tid + 1024, HH_MM_STAGE_CHUNKS - 1)];
}

// Registers -> one LDS stage buffer (surplus threads rewrite the last chunk with its value).
HH_DEV void hh_mm_commit(uint8_t* buf, uint32_t tid, const hh_mm_pre& p) {
    hh_v4u* dst = reinterpret_cast<hh_v4u*>(buf);
    dst[tid] = p.v0;
    dst[tid + 256] = p.v1;
    dst[tid + 512] = p.v2;
    dst[tid + 768] = p.v3;
    dst[min(tid + 1024, HH_MM_STAGE_CHUNKS - 1)] = p.v4;
}

template <int TT, bool FFN>
HH_DEV void hh_mm_body(const hh_mm_args& a) {
    __shared__ __attribute__((aligned(16))) uint8_t xs_lds[2][HH_MM_STAGE];
    __shared__ int last_flag;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % HH_WAVE;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / HH_WAVE);
    const uint32_t grp = blockIdx.x / a.ksg;  // row group (4 row pairs)
    const uint32_t kg = blockIdx.x % a.ksg;   // superblock group
    const uint32_t nsb = a.n / 256;
    const uint32_t g0 = (uint32_t)(((uint64_t)kg * nsb) / a.ksg);
    const uint32_t g1 = (uint32_t)(((uint64_t)(kg + 1) * nsb) / a.ksg);
    const uint32_t c = lane >> 4;
    const uint32_t r16 = lane & 15u;
    const uint32_t rp = grp * HH_MM_WAVES + wave;  // this wave's row pair

    // Rows of the two tiles at this lane (A layout).  Rows past m are clamped to a valid
    // row for loading; their outputs are never stored.
    const uint32_t base0 = FFN ? 16u * rp : 32u * rp;
    const uint32_t base1 = FFN ? 16u * rp : 32u * rp + 16u;
    const uint32_t row0 = min(base0 + r16, a.m - 1);
    const uint32_t row1 = min(base1 + r16, a.m - 1);
    const uint8_t* p0 = a.w0 + (size_t)row0 * a.row_bytes;
    const uint8_t* p1 = (FFN ? a.w1 : a.w0) + (size_t)row1 * a.row_bytes;

    hh_f4 acc[2][TT];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[t][tt] = hh_f4{0.f, 0.f, 0.f, 0.f};

    // Stage pipeline over (sb, tt) in order; stage i of this workgroup is buffer i % 2.
    const uint32_t nst = (g1 - g0) * TT;
    hh_mm_pre pre;
    hh_mm_wq w0, w1;
    if (nst > 0) {
        hh_mm_load(p0, g0, c, w0);
        hh_mm_load(p1, g0, c, w1);
        hh_mm_fetch<TT>(a, g0, nsb, tid, 0, pre);
        hh_mm_commit(xs_lds[0], tid, pre);
        hh_mm_fetch<TT>(a, g0, nsb, tid, min(1u, nst - 1), pre);
    }
    __syncthreads();
    uint32_t i = 0;
    for (uint32_t sb = g0; sb < g1; sb++) {
        hh_mm_tile t0, t1;
        hh_mm_decode(w0.h, w0.q0, w0.q1, c, lane, t0);
        hh_mm_decode(w1.h, w1.q0, w1.q1, c, lane, t1);
        // next superblock's weights (the last iteration re-reads its own: no branch)
        const uint32_t sn = min(sb + 1, g1 - 1);
        hh_mm_load(p0, sn, c, w0);
        hh_mm_load(p1, sn, c, w1);
#pragma unroll
        for (int tt = 0; tt < TT; tt++, i++) {
            const uint8_t* st = xs_lds[i & 1u];
            const hh_f4 z = hh_f4{0.f, 0.f, 0.f, 0.f};
            hh_f4 q0 = z, q1 = z;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const hh_h8 xh = *reinterpret_cast<const hh_h8*>(st + (s * 64 + lane) * 16);
                q0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(t0.a[s], xh, q0, 0, 0, 0);
                q1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(t1.a[s], xh, q1, 0, 0, 0);
            }
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const hh_h8 xl = *reinterpret_cast<const hh_h8*>(st + 8192 + (s * 64 + lane) * 16);
                q0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(t0.a[s], xl, q0, 0, 0, 0);
                q1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(t1.a[s], xl, q1, 0, 0, 0);
            }
            const hh_h4 shi = *reinterpret_cast<const hh_h4*>(st + 16384 + lane * 8);
            const hh_h4 slo = *reinterpret_cast<const hh_h4*>(st + 16896 + lane * 8);
            hh_f4 m0 = __builtin_amdgcn_mfma_f32_16x16x16f16(t0.amin, shi, z, 0, 0, 0);
            hh_f4 m1 = __builtin_amdgcn_mfma_f32_16x16x16f16(t1.amin, shi, z, 0, 0, 0);
            m0 = __builtin_amdgcn_mfma_f32_16x16x16f16(t0.amin, slo, m0, 0, 0, 0);
            m1 = __builtin_amdgcn_mfma_f32_16x16x16f16(t1.amin, slo, m1, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[0][tt][r] = fmaf(t0.d4[r], q0[r], acc[0][tt][r]);
                acc[1][tt][r] = fmaf(t1.d4[r], q1[r], acc[1][tt][r]);
                acc[0][tt][r] = fmaf(t0.dmin4[r], m0[r], acc[0][tt][r]);
                acc[1][tt][r] = fmaf(t1.dmin4[r], m1[r], acc[1][tt][r]);
            }
            // Next stage: its registers go to the other buffer (free since the barrier
            // that ended stage i-1), then the stage after it is fetched.  After the last
            // stage this writes a buffer nobody reads again.
            hh_mm_commit(xs_lds[(i + 1) & 1u], tid, pre);
            hh_mm_fetch<TT>(a, g0, nsb, tid, min(i + 2, nst - 1), pre);
            __syncthreads();
        }
    }

    // Partial sums across superblock groups: publish, the last arrival adds them in order.
    const uint32_t T = 16u * TT;
    const uint32_t grows = HH_MM_WAVES * 16u;  // rows of one tile plane of a group
    if (a.ksg > 1) {
        // part[k][t][tok][row in group]: D lane (j, c) holds rows 4c..4c+3 of token j
        const uint32_t lrow = wave * 16 + 4 * c;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                float* p = a.part + ((((size_t)grp * a.ksg + kg) * 2 + t) * T + tt * 16 + r16) * grows + lrow;
#pragma unroll
                for (int r = 0; r < 4; r++) hh_store_coherent_f(p + r, acc[t][tt][r]);
            }
        __builtin_amdgcn_s_waitcnt(0);  // partial stores complete before the arrival (vmcnt covers stores)
        __syncthreads();
        if (tid == 0) {
            const unsigned old = __hip_atomic_fetch_add(a.cnt + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == a.ksg - 1;
            if (last) __hip_atomic_store(a.cnt + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = last;
        }
        __syncthreads();
        if (!last_flag) return;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                hh_f4 s = hh_f4{0.f, 0.f, 0.f, 0.f};
                for (uint32_t k = 0; k < a.ksg; k++) {
                    const float* p = a.part + ((((size_t)grp * a.ksg + k) * 2 + t) * T + tt * 16 + r16) * grows + lrow;
#pragma unroll
                    for (int r = 0; r < 4; r++) s[r] += hh_load_coherent_f(p + r);
                }
                acc[t][tt] = s;
            }
    }

    if constexpr (FFN) {
        // h rows 16rp + 4c + r of token tt*16 + j -> token stages of the down projection
        // (n = m), hi/lo, and the sum over this row pair's 16 rows (one half-sub-block).
        const uint32_t nsb_h = a.m / 256;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            float hsum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t row = base0 + 4 * c + r;
                const float h = row < a.m ? hh_act_mul(acc[0][tt][r], acc[1][tt][r], a.act) : 0.f;
                hsum += h;
                if (row < a.m) {
                    _Float16 hi, lo;
                    hh_split_f16(h, hi, lo);
                    uint8_t* st = a.hop + ((size_t)tt * nsb_h + row / 256) * HH_MM_STAGE;
                    const uint32_t off = hh_mm_elem_off(r16, row & 255u);
                    *reinterpret_cast<_Float16*>(st + off) = hi;
                    *reinterpret_cast<_Float16*>(st + 8192 + off) = lo;
                }
            }
            hsum += __shfl_xor(hsum, 16, HH_WAVE);
            hsum += __shfl_xor(hsum, 32, HH_WAVE);
            if (c == 0 && base0 + 16 <= a.m) {
                _Float16 hi, lo;
                hh_split_f16(hsum, hi, lo);
                uint8_t* st = a.hop + ((size_t)tt * nsb_h + base0 / 256) * HH_MM_STAGE;
                const uint32_t off = hh_mm_sum_off(r16, (base0 & 255u) / 16);
                *reinterpret_cast<_Float16*>(st + off) = hi;
                *reinterpret_cast<_Float16*>(st + 512 + off) = lo;
            }
        }
        return;
    }

#pragma unroll
    for (int t = 0; t < 2; t++) {
        const uint32_t row = (t == 0 ? base0 : base1) + 4 * c;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const uint32_t tok = (uint32_t)tt * 16 + r16;
            if (tok >= a.b) continue;
            float* yp = a.y + (size_t)tok * a.m + row;
            if (row + 4 <= a.m && ((uintptr_t)yp & 15u) == 0) {
                *reinterpret_cast<float4*>(yp) = make_float4(acc[t][tt][0], acc[t][tt][1], acc[t][tt][2], acc[t][tt][3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (row + r < a.m) yp[r] = acc[t][tt][r];
            }
        }
    }
}

// hh_q4k_mm_t<TT>: GEMM; hh_q4k_mm_gateup_t<TT>: FFN gate/up + act into token stages.
#define HH_MM_KERNELS(TT)                                                                              \
    extern "C" __global__ void __launch_bounds__(HH_MM_BLOCK) hh_q4k_mm_t##TT(const hh_mm_args a) {    \
        hh_mm_body<TT, false>(a);                                                                      \
    }                                                                                                  \
    extern "C" __global__ void __launch_bounds__(HH_MM_BLOCK) hh_q4k_mm_gateup_t##TT(const hh_mm_args a) { \
        hh_mm_body<TT, true>(a);                                                                       \
    }
HH_MM_KERNELS(1)
HH_MM_KERNELS(2)
HH_MM_KERNELS(4)

// Tokens [b][n] f32 -> token stages for T = 16 * TT token slots (padded tokens are zero).
// One thread per 16 consecutive elements of one token (one half-sub-block).
struct hh_mm_prep_args {
    const float* x;  // [b][n] f32
    uint8_t* xop;    // [TT][n/256] stages
    uint32_t b, n, T, pad;
};

extern "C" __global__ void __launch_bounds__(256) hh_mm_prep(const hh_mm_prep_args a) {
    const uint32_t chunks = a.n / 16;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)a.T * chunks) return;
    const uint32_t t = (uint32_t)(i / chunks), ch = (uint32_t)(i % chunks);
    const uint32_t tt = t / 16, j = t % 16, sb = ch / 16, h = ch % 16;
    uint8_t* st = a.xop + ((size_t)tt * (a.n / 256) + sb) * HH_MM_STAGE;
    float e[16];
    if (t < a.b) {
        const float4* src = reinterpret_cast<const float4*>(a.x + (size_t)t * a.n + (size_t)ch * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = src[q];
            e[4 * q] = v.x;
            e[4 * q + 1] = v.y;
            e[4 * q + 2] = v.z;
            e[4 * q + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) e[k] = 0.f;
    }
    // 16 consecutive elements = two runs of 8 that share an MFMA step: one 16-byte store each
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
        const uint32_t off = hh_mm_elem_off(j, h * 16 + 8 * half8);
        *reinterpret_cast<hh_h8*>(st + off) = hi;
        *reinterpret_cast<hh_h8*>(st + 8192 + off) = lo;
    }
    _Float16 sh, sl;
    hh_split_f16(s, sh, sl);
    const uint32_t so = hh_mm_sum_off(j, h);
    *reinterpret_cast<_Float16*>(st + so) = sh;
    *reinterpret_cast<_Float16*>(st + 512 + so) = sl;
}
