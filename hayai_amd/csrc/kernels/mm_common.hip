// Shared pieces of the f16 batched Q4_K MFMA kernels (q4k_mmr.hip): the superblock decode
// into MFMA operands, the token-stage layout, and the kernel that writes token stages.
// The reference's batched kernel (ggml_gemv_q4.cl:349-419, host compute.rs:179-257)
// re-reads each weight row per token; the batched kernels read and decode every weight
// once per launch and multiply it by all tokens on the matrix cores.
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
typedef _Float16 hh_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 hh_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 hh_h8 __attribute__((ext_vector_type(8)));
typedef float hh_f4 __attribute__((ext_vector_type(4)));

#define HH_MM_STAGE 17408u  // bytes of one (token tile, superblock) stage

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
