// Shared pieces of the f16 batched Q4_K MFMA kernels (q4k_mmr.hip): the token-stage layout
// and the kernel that writes token stages (the weight decode is in q4k_mmr.hip).
// The reference's batched kernel (ggml_gemv_q4.cl:349-419, host compute.rs:179-257)
// re-reads each weight row per token; the batched kernels read and decode every weight
// once per launch and multiply it by all tokens on the matrix cores.
//
// Arithmetic (per Q4_K superblock of one row, 8 sub-blocks of 32 elements):
//   sum_k w_k x_k = d * sum_k (sc_k q_k) x_k  -  dmin * sum_sb m_sb * (sum of x over sb)
//   - sc*q is an integer <= 63*15 = 945, exact in f16.  It is built from the nibbles with
//     one v_and_or_b32 (two nibbles -> the f16 pair 1024+q, or 1024+16q for high nibbles)
//     and one packed FMA ((1024+q)*sc - 1024*sc, or (1024+16q)*sc/16 - 64*sc, exact because
//     the FMA rounds only its exact result) per two weights.
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
//   - A = tokens (16 tokens x 32 k), B = weights (32 k x 16 rows), D = 16 x 16.  Lane l: A
//     token l%16, B row l%16; lane quarter c = l/16 supplies k-slots 8c..8c+7 (16x16x32) or
//     4c..4c+3 (16x16x16); D holds tokens 4c..4c+3 of row l%16.
//   - The k order inside a superblock is free (weights are real values by then): quarter c
//     owns Q4_K group c (qs bytes 32c..32c+31).  Step s < 4 takes the low nibbles of bytes
//     32c+8s..+8 (elements 64c+8s+e), step s >= 4 the high nibbles (elements 64c+32+8(s-4)+e),
//     e in the order 0 2 1 3 4 6 5 7 (the order the decode produces).
//
// Token operands ("stages"): the prep kernel (and the FFN gate/up epilogue, for the down
// projection) write tokens in MFMA operand order, one contiguous 17 KB stage per (16-token
// tile tt, superblock sb):
//   [0, 8192)       hi: step s, lane l (= 16c + token j), 8 halves    -> (64 s + l) * 16 B
//                   (elements e in the order 0 2 1 3 4 6 5 7)
//   [8192, 16384)   lo: same
//   [16384, 16896)  half-sub-block sums hi: lane l, 4 halves e (half 4c + e) -> 8 l B
//   [16896, 17408)  sums lo: same
// Stage (tt, sb) starts at (tt * nsb + sb) * 17408.
//
typedef _Float16 hh_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 hh_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 hh_h8 __attribute__((ext_vector_type(8)));
typedef float hh_f4 __attribute__((ext_vector_type(4)));

#define HH_MM_STAGE 17408u  // bytes of one (token tile, superblock) stage

HH_DEV hh_h2 hh_h2_bits(uint32_t v) { return __builtin_bit_cast(hh_h2, v); }

struct hh_mm_wq {
    uint4 h, q0, q1;
};

// f32 -> hi + lo f16 pair
HH_DEV void hh_split_f16(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Byte offsets, inside its stage, of token j's run of 8 elements starting at e (a multiple of
// 8, 0..248 of the superblock; the run is stored in the order above) and of half-sub-block h
// (0..15).
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
            const int pos = (k & 4) | ((k & 1) << 1) | ((k >> 1) & 1);  // the order 0 2 1 3 4 6 5 7
            hi[pos] = vh;
            lo[pos] = vl;
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
