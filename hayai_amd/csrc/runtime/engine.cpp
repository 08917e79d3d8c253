// HIP runtime of the FFN engine: device bring-up, code-object loading, validation,
// workspaces and kernel dispatch.  The extern "C" surface is in capi.cpp.
#include "engine.h"

#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>

// gfx950 code object embedded by blob.S (.incbin of the --genco output).
extern "C" const unsigned char hh_kernels_blob[];
extern "C" const unsigned char hh_kernels_blob_end[];

namespace hh {

static thread_local std::string g_last_error;

const std::string& last_error() { return g_last_error; }

hh_status fail(hh_status st, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

hh_status hip_fail(hipError_t err, const char* what) {
    return fail(err == hipErrorOutOfMemory ? HH_ERR_OUT_OF_MEMORY : HH_ERR_RUNTIME, "%s: %s (%d)", what,
                hipGetErrorString(err), (int)err);
}

// Formats with kernels here; block geometry from compute.rs:877-907.
static const Format kFormats[] = {
    {HH_TYPE_F32, "f32", 1, 4, 32, false},
    {HH_TYPE_F16, "f16", 1, 2, 32, false},
    {HH_TYPE_Q4_0, "q4_0", 32, 18, 32, true},
    {HH_TYPE_Q4_K, "q4_k", 256, 144, 64, true},
    {HH_TYPE_IQ2_XXS, "iq2_xxs", 256, 66, 32, true},
    {HH_TYPE_IQ3_XXS, "iq3_xxs", 256, 98, 32, true},
    {HH_TYPE_Q8_0, "q8_0", 32, 34, 32, true},
    {HH_TYPE_Q6_K, "q6_k", 256, 210, 64, true},
};

const Format* format_of(int t) {
    for (const Format& f : kFormats)
        if (f.type == t) return &f;
    return nullptr;
}

const TeamCfg kTeamCfgs[] = {{16, 1}, {32, 1}, {64, 1}, {128, 1}, {256, 1}, {512, 1}, {512, 2}};
const int kNumTeamCfgs = (int)(sizeof kTeamCfgs / sizeof kTeamCfgs[0]);

hh_status row_bytes(int t, size_t n, size_t* out) {
    const Format* f = format_of(t);
    if (!f) return fail(HH_ERR_KERNEL_MISSING, "no GEMV kernel for GGML type %d", t);
    if (n % f->block != 0)
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: n=%zu is not a valid column count for this layout", f->name,
                    n);
    *out = (n / f->block) * f->bytes;
    return HH_OK;
}

// validate_gemv_shape, compute.rs:935-949.
hh_status validate_shape(int t, size_t m, size_t n) {
    const Format* f = format_of(t);
    if (!f) return fail(HH_ERR_KERNEL_MISSING, "no GEMV kernel for GGML type %d", t);
    if (m == 0 || n == 0) return fail(HH_ERR_INVALID, "ggml_gemv_%s: empty shape m=%zu n=%zu", f->name, m, n);
    size_t rb;
    return row_bytes(t, n, &rb);
}

// validate_gemv_weights, compute.rs:912-931.
hh_status validate_weights(int t, size_t m, size_t n, size_t len) {
    size_t rb;
    HH_TRY(row_bytes(t, n, &rb));
    const Format* f = format_of(t);
    if (m != 0 && rb > SIZE_MAX / m)
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: weight size overflow for %zux%zu", f->name, m, n);
    if (len < m * rb)
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: weight buffer %zu B < %zu B required for %zux%zu", f->name,
                    len, m * rb, m, n);
    return HH_OK;
}

// Pick the smallest instantiated team covering `units` lane units of a row.
static const TeamCfg* pick_team(size_t units) {
    for (int i = 0; i < kNumTeamCfgs; i++)
        if ((size_t)kTeamCfgs[i].team * kTeamCfgs[i].upl >= units) return &kTeamCfgs[i];
    return nullptr;
}

// Workgroup size of a team kernel; must equal hh_geom<TEAM>::BLOCK in gemv.hip.
static int block_of(int team) { return team > 64 ? team : 256; }

}  // namespace hh

using namespace hh;

hh_status hh_engine::select() {
    hipError_t err = hipSetDevice(device);
    if (err != hipSuccess) return hip_fail(err, "hipSetDevice");
    return HH_OK;
}

hh_status hh_engine::kernel(const std::string& name, hipFunction_t* out) {
    auto it = fns.find(name);
    if (it != fns.end()) {
        *out = it->second;
        return HH_OK;
    }
    hipFunction_t f = nullptr;
    hipError_t err = hipModuleGetFunction(&f, module, name.c_str());
    if (err != hipSuccess || !f)
        return fail(HH_ERR_KERNEL_MISSING, "kernel %s missing from the gfx950 code object", name.c_str());
    fns[name] = f;
    *out = f;
    return HH_OK;
}

int hh_engine::resident_blocks(const std::string& name, int block) {
    if (blocks_per_cu_override > 0) return blocks_per_cu_override;
    auto it = blocks_per_cu.find(name);
    if (it != blocks_per_cu.end()) return it->second;
    hipFunction_t f;
    int nb = 1;
    if (kernel(name, &f) == HH_OK) {
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, block, 0) != hipSuccess || nb < 1) nb = 1;
    }
    blocks_per_cu[name] = nb;
    return nb;
}

void hh_engine::free_retired() {
    if (ws_retired.empty()) return;
    (void)hipStreamSynchronize(stream);
    for (void* p : ws_retired) (void)hipFree(p);
    ws_retired.clear();
}

hh_status hh_engine::no_capture(const char* what) const {
    if (capturing) return fail(HH_ERR_INVALID, "%s cannot be captured into a graph", what);
    return HH_OK;
}

hh_status hh_engine::grow(void** p, size_t* cap, size_t need) {
    if (need <= *cap && *p) return HH_OK;
    if (capturing)
        return fail(HH_ERR_INVALID,
                    "a workspace would grow during graph capture: run the sequence once before capturing it");
    if (*p) {
        if (live_graphs > 0) {
            // a graph may name this allocation in its kernels' arguments: keep it alive
            ws_retired.push_back(*p);
        } else {
            hipError_t e1 = hipStreamSynchronize(stream);
            if (e1 != hipSuccess) return hip_fail(e1, "hipStreamSynchronize");
            (void)hipFree(*p);
        }
        *p = nullptr;
        *cap = 0;
    }
    size_t sz = std::max<size_t>(need, 256);
    hipError_t err = hipMalloc(p, sz);
    if (err != hipSuccess) return hip_fail(err, "hipMalloc(workspace)");
    *cap = sz;
    return HH_OK;
}

// Kernel argument block of q4k.hip (same layout).
struct hh_digits_ptr {
    int8_t* q1;
    int8_t* q2;
    float* sc;
    float* sum;
};
struct hh_q4k_args {
    const uint8_t* w0;
    const uint8_t* w1;
    const float* x;
    float* y;
    hh_digits_ptr xq;
    hh_digits_ptr hq;
    uint32_t m;
    uint32_t n;
    uint64_t row_bytes;
    int32_t act;
    uint32_t hrows;
};

// Digit layout of an n-element activation in one buffer (see q4k.hip).
static hh_digits_ptr digits_at(void* base, size_t n) {
    int8_t* q1 = (int8_t*)base;
    int8_t* q2 = q1 + n;
    float* sc = (float*)(q2 + n);
    return hh_digits_ptr{q1, q2, sc, sc + n / 32};
}

size_t hh_digits_bytes(size_t n) { return 2 * n + (n / 32) * 8; }

hh_status hh_engine::enqueue_q4k(size_t m, size_t n, const uint8_t* w0, const uint8_t* w1, const float* x, float* y,
                                 int act, bool gateup, const void* xdigits, void* hdigits) {
    const size_t units = n / 64;
    const size_t rb = (n / 256) * 144;
    if (q4k_generic || units == 0 || units > 512 || ((uintptr_t)w0 & 15u) || (gateup && ((uintptr_t)w1 & 15u)) ||
        (!xdigits && ((uintptr_t)x & 15u)) || (hdigits && (m % 256 != 0)))
        return HH_ERR_UNSUPPORTED_DEVICE;
    int wpt = 1;
    while ((size_t)wpt * 64 < units) wpt *= 2;
    const int waves = 8, tpw = waves / wpt;
    const int rows_per_team_step = gateup ? 1 : 2;
    const char* kind = gateup ? "hh_q4k_gateup_w" : (xdigits ? "hh_q4k_gemvq_w" : "hh_q4k_gemv_w");
    const std::string name = std::string(kind) + std::to_string(wpt);
    hipFunction_t fn;
    HH_TRY(kernel(name, &fn));
    // Occupancy with the largest LDS this kernel asks for (gate/up h rows bounded below).
    const size_t xbytes = xdigits ? 0 : hh_digits_bytes(n);
    const size_t red_bytes = (size_t)waves * 4 * sizeof(float);
    int occ = blocks_per_cu_override;
    if (occ <= 0) {
        auto it = blocks_per_cu.find(name);
        if (it != blocks_per_cu.end()) {
            occ = it->second;
        } else {
            const size_t probe = xbytes + red_bytes + (gateup ? 64 * sizeof(float) : 0);
            if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, waves * 64, probe) != hipSuccess ||
                occ < 1)
                occ = 1;
            blocks_per_cu[name] = occ;
        }
    }
    const size_t cap = (size_t)props.multiProcessorCount * occ;
    size_t grid;
    uint32_t hrows = 0;
    if (gateup && hdigits) {
        const size_t S = (m + 31) / 32;  // 32-row sub-blocks of h
        grid = std::max<size_t>(1, std::min(S, cap));
        hrows = (uint32_t)(32 * ((S + grid - 1) / grid));
    } else {
        const size_t rows_per_wg_step = (size_t)tpw * rows_per_team_step;
        grid = std::max<size_t>(1, std::min((m + rows_per_wg_step - 1) / rows_per_wg_step, cap));
        if (gateup) hrows = (uint32_t)((m + grid - 1) / grid + 3) & ~3u;
    }
    const size_t smem = xbytes + (size_t)hrows * sizeof(float) + red_bytes;
    hh_q4k_args a{w0, w1, x, y, hh_digits_ptr{}, hh_digits_ptr{}, (uint32_t)m, (uint32_t)n, (uint64_t)rb, act, hrows};
    if (xdigits) a.xq = digits_at(const_cast<void*>(xdigits), n);
    if (hdigits) a.hq = digits_at(hdigits, m);
    void* params[] = {&a};
    hipError_t err = hipModuleLaunchKernel(fn, (uint32_t)grid, 1, 1, waves * 64, 1, 1, (unsigned)smem, stream, params,
                                           nullptr);
    if (err != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel(q4k)");
    return HH_OK;
}

// Must match struct hh_lut_args in kernels/lut.hip.
struct LutArgs {
    const uint8_t* w;
    const float* lut;
    const float* x;
    float* y;
    uint32_t m, n, vec, pad;
};

hh_status hh_engine::enqueue_lut(size_t m, size_t n, const uint8_t* w, const float* lut, const float* x, float* y) {
    if (m > UINT32_MAX || n > UINT32_MAX) return fail(HH_ERR_INVALID, "lut_matmul_q4: %zux%zu exceeds 32-bit sizes", m, n);
    hipFunction_t f;
    HH_TRY(kernel("hh_lut_gemv", &f));
    const size_t pc = n / 2;
    // dword weight loads need every row start 4-aligned; float4 x loads need x 16-aligned.
    const bool vec = pc % 4 == 0 && ((uintptr_t)w & 3u) == 0 && ((uintptr_t)x & 15u) == 0;
    LutArgs a{w, lut, x, y, (uint32_t)m, (uint32_t)n, vec ? 1u : 0u, 0u};
    const size_t cap = (size_t)props.multiProcessorCount * 8;
    const size_t grid = std::max<size_t>(1, std::min(cap, (m + 3) / 4));
    return launch(f, (uint32_t)grid, 256, a);
}

hh_status hh_engine::enqueue_gemv(int type, size_t m, size_t n, const uint8_t* w, const float* x, float* y,
                                  void* xq_ws) {
    const Format* f = format_of(type);
    if (!f) return fail(HH_ERR_KERNEL_MISSING, "no GEMV kernel for GGML type %d", type);
    size_t rb;
    HH_TRY(row_bytes(type, n, &rb));
    if (((uintptr_t)x & 3u) || ((uintptr_t)y & 3u))
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: activations must be 4-byte aligned", f->name);
    hh_gemv_args a{w, x, y, (uint32_t)m, (uint32_t)n, (uint64_t)rb};
    if (m > UINT32_MAX / 2 || n > UINT32_MAX / 2)
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: shape %zux%zu too large", f->name, m, n);

    if (type != HH_TYPE_Q4_K && type != HH_TYPE_F32 && ((uintptr_t)w & 1u))
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: weight address must be 2-byte aligned", f->name);
    const bool aligned16 = (((uintptr_t)w & 15u) == 0) && (rb % 16 == 0);
    if (type == HH_TYPE_Q4_K && aligned16) {
        hh_status st = enqueue_q4k(m, n, w, nullptr, x, y, 0, false, nullptr, nullptr);
        if (st != HH_ERR_UNSUPPORTED_DEVICE) return st;
    }
    if (type == HH_TYPE_Q6_K || type == HH_TYPE_IQ2_XXS || type == HH_TYPE_IQ3_XXS) {
        hh_status st = enqueue_ring_gemv(type, m, n, w, x, y, xq_ws);
        if (st != HH_ERR_UNSUPPORTED_DEVICE) return st;
    }
    std::string name;
    int team = 0, upl = 1;
    if ((type == HH_TYPE_F32 || type == HH_TYPE_F16) && (n % 32 != 0 || !aligned16)) {
        name = type == HH_TYPE_F32 ? "hh_gemv_f32_plain" : "hh_gemv_f16_plain";
        hipFunction_t fn;
        HH_TRY(kernel(name, &fn));
        uint32_t grid = (uint32_t)std::min<size_t>((m + 3) / 4, (size_t)props.multiProcessorCount * 8);
        return launch(fn, std::max<uint32_t>(grid, 1), 256, a);
    }
    const TeamCfg* tc = pick_team(n / f->unit);
    if (!tc)
        return fail(HH_ERR_INVALID, "ggml_gemv_%s: row of %zu columns is wider than the widest team", f->name, n);
    team = tc->team;
    upl = tc->upl;
    std::string stem = f->name;
    if (type == HH_TYPE_Q4_K && !aligned16) stem += "_unaligned";
    name = "hh_gemv_" + stem + "_t" + std::to_string(team) + "_u" + std::to_string(upl);
    hipFunction_t fn;
    HH_TRY(kernel(name, &fn));
    const int block = block_of(team);
    const int tpb = block / team;
    const int rows_per_step = upl == 1 ? 4 : 2;
    const size_t teams = (m + rows_per_step - 1) / rows_per_step;
    const size_t need = (teams + tpb - 1) / tpb;
    const size_t cap = (size_t)props.multiProcessorCount * resident_blocks(name, block);
    const uint32_t grid = (uint32_t)std::max<size_t>(1, std::min(need, cap));
    return launch(fn, grid, (uint32_t)block, a);
}

hh_status hh_engine::enqueue_gateup(int tg, int tu, size_t d_ff, size_t d_model, const uint8_t* wg,
                                    const uint8_t* wu, const float* x, float* h, int act, float* gu_ws) {
    const Format* f = format_of(tg);
    if (!f || !format_of(tu)) return fail(HH_ERR_KERNEL_MISSING, "no GEMV kernel for GGML type %d/%d", tg, tu);
    size_t rb;
    HH_TRY(row_bytes(tg, d_model, &rb));
    if (tg == HH_TYPE_Q4_K && tu == HH_TYPE_Q4_K) {
        hh_status st = enqueue_q4k(d_ff, d_model, wg, wu, x, h, act, true, nullptr, nullptr);
        if (st != HH_ERR_UNSUPPORTED_DEVICE) return st;
    }
    if (tg == tu && f->fused_gateup) {
        if (tg != HH_TYPE_Q4_K && (((uintptr_t)wg | (uintptr_t)wu) & 1u))
            return fail(HH_ERR_INVALID, "ffn gate/up %s: weight address must be 2-byte aligned", f->name);
        const TeamCfg* tc = pick_team(d_model / f->unit);
        if (!tc) return fail(HH_ERR_INVALID, "ffn: d_model=%zu wider than the widest team", d_model);
        const bool aligned16 = (((uintptr_t)wg & 15u) == 0) && (((uintptr_t)wu & 15u) == 0) && (rb % 16 == 0);
        std::string stem = f->name;
        if (tg == HH_TYPE_Q4_K && !aligned16) stem += "_unaligned";
        std::string name = "hh_gateup_" + stem + "_t" + std::to_string(tc->team) + "_u" + std::to_string(tc->upl);
        hipFunction_t fn;
        HH_TRY(kernel(name, &fn));
        const int block = block_of(tc->team);
        const int tpb = block / tc->team;
        const int rows_per_step = tc->upl == 1 ? 2 : 1;
        const size_t teams = (d_ff + rows_per_step - 1) / rows_per_step;
        const size_t need = (teams + tpb - 1) / tpb;
        const size_t cap = (size_t)props.multiProcessorCount * resident_blocks(name, block);
        hh_gateup_args a{wg, wu, x, h, (uint32_t)d_ff, (uint32_t)d_model, (uint64_t)rb, act, 0};
        return launch(fn, (uint32_t)std::max<size_t>(1, std::min(need, cap)), (uint32_t)block, a);
    }
    // Unfused: gate and up in their own formats, then act(g) * u.
    float *g = gu_ws, *u = gu_ws ? gu_ws + d_ff : nullptr;
    void* xq = gu_ws ? (void*)(gu_ws + 2 * d_ff) : nullptr;
    if (!gu_ws) {
        HH_TRY(grow(&ws_g, &ws_g_cap, d_ff * sizeof(float)));
        HH_TRY(grow(&ws_u, &ws_u_cap, d_ff * sizeof(float)));
        g = (float*)ws_g;
        u = (float*)ws_u;
    }
    HH_TRY(enqueue_gemv(tg, d_ff, d_model, wg, x, g, xq));
    HH_TRY(enqueue_gemv(tu, d_ff, d_model, wu, x, u, xq));
    hipFunction_t fn;
    HH_TRY(kernel("hh_act_mul_kernel", &fn));
    hh_act_args a{(const float*)g, (const float*)u, h, (uint32_t)d_ff, act};
    return launch(fn, (uint32_t)((d_ff + 255) / 256), 256, a);
}

// Grid-barrier state (q4k.hip): 16 arrival-counter lines, 16 release-flag lines, the group
// counter, the error word, the barrier epoch and the FFN-stack epoch, 128 bytes each.
constexpr size_t kBarLine = 128;
constexpr size_t kBarBytes = kBarLine * (2 * 16 + 4);
constexpr size_t kBarEpochOffset = kBarLine * (2 * 16 + 2);  // the epochs survive an error reset
constexpr size_t kBarErrOffset = kBarLine * (2 * 16 + 1);
// the grouped MoE's routing-arrival counter (hh_moe_route_prep): word 4 of the last line
constexpr size_t kBarMoeArrivalsOffset = kBarLine * (2 * 16 + 3) + 4 * 4;

// Must match struct hh_gur_args / hh_dnr_args in kernels/q4k_ring.hip.
struct GurArgs {  // the ring gate/up kernels' scalar parameters (HH_GUR_PARAMS, q4k_ring.hip)
    const uint8_t* wg;
    const uint8_t* wu;
    const float* x;
    uint8_t* hx;
    const float* nw;
    uint32_t rb1;
    uint32_t dims;  // d_model | d_ff << 16
    uint32_t grid;
    int32_t act;
    float eps;
};
struct DnrArgs {
    const uint8_t* wd;
    const uint8_t* hx;
    float* y;
    const float* res;
    uint64_t rb2;
    uint32_t d_model, d_ff;
};

// The ring kernels' grid: `per_cu` workgroups per CU when the occupancy allows it.
static size_t ring_grid(int occ, int per_cu, size_t cus) { return cus * (size_t)std::max(1, std::min(occ, per_cu)); }

// Weight formats of the ring kernels (kernels/q4k_ring.hip, q6k_ring.hip, iq_ring.hip):
// kernel stem, block bytes, the static LDS tables the kernels keep, whether a gate/up
// kernel exists.  Formats whose blocks are not a multiple of 4 bytes need an even number of
// blocks per row, so that rows start 4-byte aligned.
struct RingFmt {
    int type;
    const char* stem;
    uint32_t block_bytes;
    uint32_t tab_bytes;
    bool gate_up;
    bool lane_partials;  // the gate/up kernel keeps every lane's row contribution in LDS
    bool wide_gu;        // 128-column lanes for gate/up at d_model 8192 (kernel stem + "w")
    bool wide_dn;        // 128-column lanes for down rows of at least 8192 columns
    bool direct_h;       // down: lanes load h's digits themselves (no LDS copy of h)
};
static const RingFmt kRingFmts[] = {
    {HH_TYPE_Q4_K, "q4k", 144, 0, true, false, false, false, true},
    {HH_TYPE_Q6_K, "q6k", 210, 0, false, false, false, false, false},
    {HH_TYPE_IQ2_XXS, "iq2", 66, 3072, true, true, true, true, true},
    {HH_TYPE_IQ3_XXS, "iq3", 98, 2048, true, true, true, false, true},
};
static const RingFmt* ring_fmt(int type) {
    for (const RingFmt& f : kRingFmts)
        if (f.type == type) return &f;
    return nullptr;
}
// Columns per row the ring kernels accept for a format: whole 256-column blocks, 4-byte
// aligned rows, at most 32768 (digits in LDS).
static bool ring_cols_ok(const RingFmt* f, size_t n) {
    return f && n % 256 == 0 && (f->block_bytes % 4 == 0 || n % 512 == 0) && n <= 32768;
}

bool hh_engine::ring_ok(const hh_ffn_desc* d, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                        const float* x) const {
    const size_t dm = d->d_model, df = d->d_ff;
    const RingFmt* fg = ring_fmt(d->type_gate);
    const RingFmt* fd = ring_fmt(d->type_down);
    // gate and up share the gate/up kernel's format; any ring format for down (h's digits
    // are the same for all of them)
    return ring && !q4k_generic && fg && fg->gate_up && d->type_up == d->type_gate && ring_cols_ok(fg, dm) &&
           dm <= 8192 && ring_cols_ok(fd, df) &&
           ((((uintptr_t)wg | (uintptr_t)wu | (uintptr_t)wd | (uintptr_t)x) & 15u) == 0);
}

hh_status hh_engine::enqueue_ring_gu(const hh_ffn_desc* d, const uint8_t* wg, const uint8_t* wu,
                                     const float* x, const float* norm, float eps, uint8_t* hx) {
    const size_t dm = d->d_model, df = d->d_ff;
    const RingFmt* f = ring_fmt(d->type_gate);
    if (!f || !f->gate_up) return fail(HH_ERR_INVALID, "ring gate/up: no kernel for GGML type %d", d->type_gate);
    const bool wide = f->wide_gu && dm == 8192;  // one wave of 128-column lanes per row
    const int w1 = wide || dm <= 4096 ? 1 : 2;
    const std::string name =
        std::string("hh_") + f->stem + (wide ? "w" : "") + "_gu_ring_g" + std::to_string(w1) + (norm ? "_n" : "");
    hipFunction_t fn;
    HH_TRY(kernel(name, &fn));
    const int block = 8 * 64;
    const size_t cus = (size_t)props.multiProcessorCount;
    // LDS: x digits + gate/up row sums (or lane partials and row sums) + 128 B staging (the
    // kernel's layout), sized for a grid of g workgroups (the largest row range of any)
    auto smem_for = [&](size_t g) {
        const size_t rr_max = 2 * 8 * ((df / 8 + g - 1) / g);
        const size_t sums = f->lane_partials ? rr_max * (size_t)w1 * 64 + ((rr_max + 3) & ~size_t(3))
                                             : ((rr_max * w1 + 3) & ~size_t(3));
        return (((2 * dm + (dm / 32) * 8) + 15) & ~size_t(15)) + sums * 4 + 128;
    };
    // ring_gu_per_cu workgroups per CU where that many fit with their LDS, else one
    auto occupancy = [&](size_t smem) {
        const std::string key = name + ":" + std::to_string(smem);
        auto it = blocks_per_cu.find(key);
        if (it != blocks_per_cu.end()) return it->second;
        int occ = 0;
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, block, smem) != hipSuccess) occ = 1;
        blocks_per_cu[key] = occ;
        return occ;
    };
    size_t grid = cus, smem = smem_for(cus);
    if (ring_gu_per_cu > 1) {
        const size_t g2 = ring_grid(ring_gu_per_cu, ring_gu_per_cu, cus), s2 = smem_for(g2);
        const int occ = occupancy(s2);
        if (occ > 1) {
            grid = ring_grid(occ, ring_gu_per_cu, cus);
            smem = smem_for(grid);
        }
    }
    if (!hx) {
        HH_TRY(grow(&ws_hq, &ws_hq_cap, hh::ring_digits_bytes(df)));
        hx = (uint8_t*)ws_hq;
    }
    GurArgs a{wg, wu, x, hx, norm, (uint32_t)((dm / 256) * f->block_bytes), (uint32_t)(dm | (df << 16)), (uint32_t)grid,
              d->act, eps};
    // the argument block as raw kernel-argument bytes: the Q4_K kernels take its fields as
    // separate scalar parameters (same layout), so their leading dwords can be preloaded
    size_t asz = sizeof a;
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &a, HIP_LAUNCH_PARAM_BUFFER_SIZE, &asz, HIP_LAUNCH_PARAM_END};
    hipError_t err = hipModuleLaunchKernel(fn, (uint32_t)grid, 1, 1, block, 1, 1, (unsigned)smem, stream, nullptr, cfg);
    if (err != hipSuccess) return hip_fail(err, "launch(ring gate/up)");
    return HH_OK;
}

hh_status hh_engine::enqueue_ring_dn(const hh_ffn_desc* d, const uint8_t* wd, float* y, const float* res) {
    return launch_dn_ring(d->type_down, d->d_model, d->d_ff, wd, (const uint8_t*)ws_hq, y, res);
}

// The ring down kernel over m rows of n columns (any ring format) from digits `hx`.  Each
// workgroup keeps the digits and its rows' lane partials in LDS: the grid is at least one
// workgroup per CU and large enough that every workgroup's rows fit.
hh_status hh_engine::launch_dn_ring(int type, size_t m, size_t n, const uint8_t* w, const uint8_t* hx, float* y,
                                    const float* res) {
    const RingFmt* f = ring_fmt(type);
    if (!f) return fail(HH_ERR_INVALID, "ring down: no kernel for GGML type %d", type);
    const bool wide = f->wide_dn && n >= 8192;
    const size_t units = n / (wide ? 128 : 64);  // lane units per row
    int w2 = 1;
    while ((size_t)w2 * 64 < units) w2 *= 2;
    const std::string name = std::string("hh_") + f->stem + (wide ? "w" : "") + "_dn_ring_d" + std::to_string(w2);
    hipFunction_t fn;
    HH_TRY(kernel(name, &fn));
    const int block = 9 * 64;  // 8 compute waves + the wave that copies into LDS
    const size_t cus = (size_t)props.multiProcessorCount;
    const size_t lds = (size_t)props.sharedMemPerBlock - f->tab_bytes;  // the tables are static LDS
    // the intermediate's copy in LDS (formats whose lanes do not load it themselves)
    const size_t hb = f->direct_h ? 0 : ((2 * n + (n / 8) * 4) + 15) & ~size_t(15);
    const size_t per_row = (size_t)w2 * 64 * 4;
    if (hb + per_row > lds) return HH_ERR_UNSUPPORTED_DEVICE;
    const size_t rows_fit = (lds - hb) / per_row;
    int occ = 0;
    auto it = blocks_per_cu.find(name);
    if (it != blocks_per_cu.end()) {
        occ = it->second;
    } else {
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, block, hb + per_row) != hipSuccess) occ = 1;
        blocks_per_cu[name] = occ;
    }
    const size_t grid = std::max(ring_grid(occ, ring_dn_per_cu, cus), (m + rows_fit - 1) / rows_fit);
    const size_t rows_max = (m + grid - 1) / grid;
    const size_t smem = hb + rows_max * per_row;
    DnrArgs a{w, hx, y, res, (uint64_t)((n / 256) * f->block_bytes), (uint32_t)m, (uint32_t)n};
    size_t asz = sizeof a;  // raw argument bytes, as for the gate/up kernel
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &a, HIP_LAUNCH_PARAM_BUFFER_SIZE, &asz, HIP_LAUNCH_PARAM_END};
    hipError_t err = hipModuleLaunchKernel(fn, (uint32_t)grid, 1, 1, block, 1, 1, (unsigned)smem, stream, nullptr, cfg);
    if (err != hipSuccess) return hip_fail(err, "launch(ring down)");
    return HH_OK;
}

// x -> the ring down kernels' digit form (q1 | q2 | one scale per 8), then a ring down kernel
// as a GEMV: the LM head of Q4_K_M files (output.weight in Q6_K), and every IQ2_XXS /
// IQ3_XXS GEMV of a shape the ring kernels take.
hh_status hh_engine::enqueue_ring_gemv(int type, size_t m, size_t n, const uint8_t* w, const float* x, float* y,
                                       void* xq_ws) {
    if (!ring || !ring_cols_ok(ring_fmt(type), n) || m > UINT32_MAX / 2 || (((uintptr_t)w | (uintptr_t)x) & 15u))
        return HH_ERR_UNSUPPORTED_DEVICE;
    if (!xq_ws) {
        HH_TRY(grow(&ws_xq, &ws_xq_cap, hh::ring_digits_bytes(n)));
        xq_ws = ws_xq;
    }
    hipFunction_t fn;
    HH_TRY(kernel("hh_x_digits", &fn));
    hh_xd_args xa{x, (uint8_t*)xq_ws, (uint32_t)n, 0u};
    HH_TRY(launch(fn, (uint32_t)((n / 8 + 255) / 256), 256, xa));
    return launch_dn_ring(type, m, n, w, (const uint8_t*)xq_ws, y, nullptr);
}

hh_status hh_engine::check_device_error() {
    unsigned flag = 0;
    HH_TRY_HIP(hipStreamSynchronize(stream), "hipStreamSynchronize");
    HH_TRY_HIP(hipMemcpy(&flag, (char*)grid_sync + kBarErrOffset, sizeof flag, hipMemcpyDeviceToHost),
               "hipMemcpy(err)");
    if (flag) {
        // Counters, flags and the error word back to zero; the epochs keep counting, so no
        // tag or generation of the failed launch can be taken for a later one's.  The stack
        // exchange words go back to tag 0, which no launch uses.
        HH_TRY_HIP(hipMemset(grid_sync, 0, kBarEpochOffset), "hipMemset(grid_sync)");
        if (ws_stk) HH_TRY_HIP(hipMemset(ws_stk, 0, ws_stk_cap), "hipMemset(stack exchange)");
        return fail(HH_ERR_RUNTIME, "grid-wide exchange timed out (workgroups not co-resident)");
    }
    return HH_OK;
}

static bool same_ffn(const hh_ffn_desc* a, const hh_ffn_desc* b) {
    return a->type_gate == b->type_gate && a->type_up == b->type_up && a->type_down == b->type_down &&
           a->act == b->act && a->d_model == b->d_model && a->d_ff == b->d_ff;
}

hh_status hh_engine::enqueue_ffn_begin(const hh_ffn_desc* d, const uint8_t* pack, const float* x,
                                       const float* norm, float eps) {
    ffn_stage_valid = false;
    HH_TRY(grow(&ws_h, &ws_h_cap, d->d_ff * sizeof(float)));
    const uint8_t* wg = pack + d->gate_off;
    const uint8_t* wu = pack + d->up_off;
    bool digits = false;
    hh_status st = HH_ERR_UNSUPPORTED_DEVICE;
    if (ring_ok(d, wg, wu, pack + d->down_off, x) && ((uintptr_t)norm & 15u) == 0) {
        // the ring kernels: gate/up writes h's granule digits, the finish step reads them
        // (with norm: the RMSNorm rides in gate/up's prologue and epilogue)
        HH_TRY(enqueue_ring_gu(d, wg, wu, x, norm, eps));
        ffn_stage = *d;
        ffn_stage_digits = false;
        ffn_stage_ring = true;
        ffn_stage_valid = true;
        ffn_calls += 2;
        return HH_OK;
    }
    if (norm) {
        // other layouts: RMSNorm as its own kernel, then the plain begin step on its output
        HH_TRY(grow(&ws_xn, &ws_xn_cap, d->d_model * sizeof(float)));
        hipFunction_t fn;
        HH_TRY(kernel("hh_rmsnorm_kernel", &fn));
        hh_norm_args na{x, norm, (float*)ws_xn, (uint32_t)d->d_model, eps};
        HH_TRY(launch(fn, 1, 1024, na));
        x = (const float*)ws_xn;
    }
    if (d->type_gate == HH_TYPE_Q4_K && d->type_up == HH_TYPE_Q4_K && d->type_down == HH_TYPE_Q4_K) {
        // Gate/up writes h and its int8 digits; the down projection consumes the digits.
        HH_TRY(grow(&ws_hq, &ws_hq_cap, hh_digits_bytes(d->d_ff)));
        st = enqueue_q4k(d->d_ff, d->d_model, wg, wu, x, (float*)ws_h, d->act, true, nullptr, ws_hq);
        digits = st == HH_OK;
    }
    if (st == HH_ERR_UNSUPPORTED_DEVICE)
        st = enqueue_gateup(d->type_gate, d->type_up, d->d_ff, d->d_model, wg, wu, x, (float*)ws_h, d->act);
    if (st != HH_OK) return st;
    ffn_stage = *d;
    ffn_stage_digits = digits;
    ffn_stage_ring = false;
    ffn_stage_valid = true;
    ffn_calls += 2;
    return HH_OK;
}

hh_status hh_engine::enqueue_ffn_finish(const hh_ffn_desc* d, const uint8_t* pack, float* y, const float* res) {
    if (!ffn_stage_valid || !same_ffn(d, &ffn_stage))
        return fail(HH_ERR_INVALID, "ffn finish: no gate/up of this FFN shape is pending (call the begin step first)");
    ffn_stage_valid = false;
    const uint8_t* wd = pack + d->down_off;
    if (ffn_stage_ring) {  // the ring down kernel adds the residual as it stores y
        const hh_status st = enqueue_ring_dn(d, wd, y, res);
        if (st == HH_OK) ffn_calls += 1;
        return st;
    }
    float* out = y;
    if (res) {
        HH_TRY(grow(&ws_f, &ws_f_cap, d->d_model * sizeof(float)));
        out = (float*)ws_f;
    }
    hh_status st = HH_ERR_UNSUPPORTED_DEVICE;
    if (ffn_stage_digits) st = enqueue_q4k(d->d_model, d->d_ff, wd, nullptr, nullptr, out, 0, false, ws_hq, nullptr);
    if (st == HH_ERR_UNSUPPORTED_DEVICE) st = enqueue_gemv(d->type_down, d->d_model, d->d_ff, wd, (const float*)ws_h, out);
    if (st != HH_OK) return st;
    ffn_calls += 1;
    if (!res) return HH_OK;
    hipFunction_t fn;
    HH_TRY(kernel("hh_add_kernel", &fn));
    hh_add_args aa{res, (const float*)ws_f, y, (uint32_t)d->d_model, 0u};
    return launch(fn, (uint32_t)((d->d_model + 255) / 256), 256, aa);
}

hh_status hh_engine::enqueue_ffn(const hh_ffn_desc* d, const uint8_t* pack, const float* x, float* y) {
    if (ring_ok(d, pack + d->gate_off, pack + d->up_off, pack + d->down_off, x)) {
        HH_TRY(enqueue_ring_gu(d, pack + d->gate_off, pack + d->up_off, x));
        HH_TRY(enqueue_ring_dn(d, pack + d->down_off, y));
        ffn_stage_valid = false;
        ffn_calls += 3;
        return HH_OK;
    }
    if (d->type_gate == d->type_up && d->type_up == d->type_down &&
        (d->type_gate == HH_TYPE_Q4_0 || d->type_gate == HH_TYPE_Q8_0)) {
        const hh_status sst = enqueue_small_ffn(d, pack + d->gate_off, pack + d->up_off, pack + d->down_off, x, y);
        if (sst == HH_OK) {
            ffn_stage_valid = false;
            ffn_calls += 3;
            return HH_OK;
        }
        if (sst != HH_ERR_UNSUPPORTED_DEVICE) return sst;
    }
    HH_TRY(enqueue_ffn_begin(d, pack, x));
    return enqueue_ffn_finish(d, pack, y);
}

// The FFN op with every intermediate in the device's fixed scratch array instead of the
// engine's workspaces (hh_ffn_dev_noalloc): nothing here allocates.  The ring layouts keep
// h's digits in the scratch; the others run the two-step form (gate/up + activation into an
// f32 h, then the down GEMV) with h, the unfused form's gate and up outputs and a Q6_K
// GEMV's x digits in the scratch.  The one-launch forms (persistent Q4_K, small Q4_0/Q8_0),
// whose grid barriers keep per-launch state, are not used.
hh_status hh_engine::enqueue_ffn_noalloc(const hh_ffn_desc* d, const uint8_t* pack, const float* x, float* y) {
    if (!noalloc_ws)
        return fail(HH_ERR_RUNTIME, "ffn_dev_noalloc: no scratch array on device %d (%s)", device,
                    noalloc_error.c_str());
    const size_t dm = d->d_model, df = d->d_ff;
    if (df > HH_NOALLOC_MAX_D_FF)
        return fail(HH_ERR_INVALID, "ffn_dev_noalloc: d_ff=%zu exceeds the scratch limit of %u", df,
                    (unsigned)HH_NOALLOC_MAX_D_FF);
    uint8_t* ws = (uint8_t*)noalloc_ws;
    const uint8_t* wg = pack + d->gate_off;
    const uint8_t* wu = pack + d->up_off;
    const uint8_t* wd = pack + d->down_off;
    if (ring_ok(d, wg, wu, wd, x)) {
        HH_TRY(enqueue_ring_gu(d, wg, wu, x, nullptr, 0.f, ws));
        HH_TRY(launch_dn_ring(d->type_down, dm, df, wd, ws, y, nullptr));
        ffn_calls += 3;
        return HH_OK;
    }
    // [h: df f32][g: df f32][u: df f32][x digits of the widest ring GEMV]
    const size_t widest = std::min<size_t>(std::max(dm, df), 32768);
    const size_t need = 3 * df * sizeof(float) + hh::ring_digits_bytes(widest);
    if (need > HH_NOALLOC_SCRATCH_BYTES)
        return fail(HH_ERR_INVALID, "ffn_dev_noalloc: d_model=%zu, d_ff=%zu need %zu bytes of scratch, more than %u",
                    dm, df, need, (unsigned)HH_NOALLOC_SCRATCH_BYTES);
    float* h = (float*)ws;
    float* gu = h + df;
    HH_TRY(enqueue_gateup(d->type_gate, d->type_up, df, dm, wg, wu, x, h, d->act, gu));
    HH_TRY(enqueue_gemv(d->type_down, dm, df, wd, h, y, (void*)(gu + 2 * df)));
    ffn_calls += 3;
    return HH_OK;
}

// Must match struct hh_sffn_args in kernels/small_ffn.hip.
struct SffnArgs {  // the small FFN kernels' scalar parameters (small_ffn.hip)
    const uint8_t* wg;
    const float* x;
    float* y;
    float* h;
    unsigned* bar;
    int32_t du, dd;  // W_up, W_down - W_gate in bytes
    uint32_t dims;   // d_model | d_ff << 16
    uint32_t grid;
    int32_t act;
};

// A small Q4_0 / Q8_0 FFN in one launch (small_ffn.hip): every workgroup's rows fit its teams
// (at most two rows per team and phase), one workgroup per CU, a grid barrier between gate/up
// and down.
hh_status hh_engine::enqueue_small_ffn(const hh_ffn_desc* d, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                                       const float* x, float* y) {
    const size_t dm = d->d_model, df = d->d_ff, G = (size_t)props.multiProcessorCount;
    auto team_of = [](size_t units) { return units <= 16 ? 16 : (units <= 32 ? 32 : 64); };
    const int t1 = team_of(dm / 32), t2 = team_of(df / 32);
    if (!small_ffn || dm % 32 || df % 32 || dm / 32 > 64 || df / 32 > 64 ||
        (df + G - 1) / G > 2 * (256 / (size_t)t1) || (dm + G - 1) / G > 2 * (256 / (size_t)t2) ||
        (((uintptr_t)wg | (uintptr_t)wu | (uintptr_t)wd) & 1u) || ((uintptr_t)x & 3u) || ((uintptr_t)y & 3u))
        return HH_ERR_UNSUPPORTED_DEVICE;
    const std::string name = std::string("hh_sffn_") + (d->type_gate == HH_TYPE_Q4_0 ? "q4_0" : "q8_0") + "_t" +
                             std::to_string(t1) + "_" + std::to_string(t2);
    hipFunction_t fn;
    HH_TRY(kernel(name, &fn));
    HH_TRY(grow(&ws_h, &ws_h_cap, df * sizeof(float)));
    size_t rin, rff;
    HH_TRY(row_bytes(d->type_gate, dm, &rin));
    HH_TRY(row_bytes(d->type_down, df, &rff));
    const int64_t du = (int64_t)(wu - wg), dd = (int64_t)(wd - wg);
    if (du != (int32_t)du || dd != (int32_t)dd) return HH_ERR_UNSUPPORTED_DEVICE;
    (void)rin;
    (void)rff;
    SffnArgs a{wg, x, y, (float*)ws_h, (unsigned*)grid_sync, (int32_t)du, (int32_t)dd, (uint32_t)(dm | (df << 16)),
               (uint32_t)G, d->act};
    size_t asz = sizeof a;  // raw argument bytes (the kernel takes the fields as scalar parameters)
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &a, HIP_LAUNCH_PARAM_BUFFER_SIZE, &asz, HIP_LAUNCH_PARAM_END};
    hipError_t err = hipModuleLaunchKernel(fn, (uint32_t)G, 1, 1, 256, 1, 1, 0, stream, nullptr, cfg);
    if (err != hipSuccess) return hip_fail(err, "launch(small ffn)");
    return HH_OK;
}

// Must match struct hh_sstk_args in kernels/small_stack.hip.
struct SstkArgs {
    const uint8_t* pack;
    const float* norm;
    const float* x;
    float* y;
    uint64_t* hx;
    uint64_t* xx;
    uint64_t* spare;
    unsigned* bar;
    uint64_t stride, off_g, off_u, off_d, rb_in, rb_ff;
    uint32_t norm_stride, d_model, d_ff, n_layers;
    float eps;
    int32_t act;
};

// Consecutive small Q4_0 / Q8_0 FFN residual blocks in one persistent launch
// (small_stack.hip): one workgroup per CU (every one resident: the exchange polls), 4
// compute waves + the exchange wave, at most two rows per team and phase, every workgroup
// with a gate/up row and a down row.
hh_status hh_engine::enqueue_small_stack(const hh_ffn_desc* d, const uint8_t* pack, size_t stride, size_t n_layers,
                                         const float* norm, size_t norm_stride, float eps, const float* x, float* y) {
    const size_t dm = d->d_model, df = d->d_ff;
    const size_t cus = (size_t)props.multiProcessorCount;
    const size_t G = std::min({stack_grid > 0 ? std::min((size_t)stack_grid, cus) : cus, dm, df});
    auto team_of = [](size_t units) { return units <= 16 ? 16 : (units <= 32 ? 32 : 64); };
    const int t1 = team_of(dm / 32), t2 = team_of(df / 32);
    // rows per team and phase (instantiated: 1..4 for Q4_0, 1..2 for Q8_0)
    const size_t rows1 = (df + G - 1) / G, rows2 = (dm + G - 1) / G;
    const size_t tpb1 = 256 / (size_t)t1, tpb2 = 256 / (size_t)t2;
    const size_t R = std::max((rows1 + tpb1 - 1) / tpb1, (rows2 + tpb2 - 1) / tpb2);
    const size_t r_max = d->type_gate == HH_TYPE_Q4_0 ? 4 : 2;
    if (!small_stack || !(d->type_gate == d->type_up && d->type_up == d->type_down) ||
        (d->type_gate != HH_TYPE_Q4_0 && d->type_gate != HH_TYPE_Q8_0) || dm % 32 || df % 32 || dm / 32 > 64 ||
        df / 32 > 64 || n_layers > 0xFFFFu || norm_stride > 0xFFFFFFFFu || R > r_max ||
        ((uintptr_t)pack | d->gate_off | d->up_off | d->down_off | stride) & 1u || ((uintptr_t)x & 3u) ||
        ((uintptr_t)y & 3u) || ((uintptr_t)norm & 3u))
        return HH_ERR_UNSUPPORTED_DEVICE;
    const std::string name = std::string("hh_sstk_") + (d->type_gate == HH_TYPE_Q4_0 ? "q4_0" : "q8_0") + "_t" +
                             std::to_string(t1) + "_" + std::to_string(t2) + "_r" + std::to_string(R);
    hipFunction_t fn;
    HH_TRY(kernel(name, &fn));
    const size_t need = (df + dm + 16 * G) * sizeof(uint64_t);  // h, x, a spare line per workgroup
    if (ws_stk_cap < need) {
        HH_TRY(grow(&ws_stk, &ws_stk_cap, need));
        HH_TRY_HIP(hipMemset(ws_stk, 0, ws_stk_cap), "hipMemset(stack exchange)");
    }
    size_t rin, rff;
    HH_TRY(row_bytes(d->type_gate, dm, &rin));
    HH_TRY(row_bytes(d->type_down, df, &rff));
    SstkArgs a{pack, norm, x, y, (uint64_t*)ws_stk, (uint64_t*)ws_stk + df, (uint64_t*)ws_stk + df + dm, (unsigned*)grid_sync, (uint64_t)stride,
               (uint64_t)d->gate_off, (uint64_t)d->up_off, (uint64_t)d->down_off, (uint64_t)rin, (uint64_t)rff,
               (uint32_t)norm_stride, (uint32_t)dm, (uint32_t)df, (uint32_t)n_layers, eps, d->act};
    void* params[] = {&a};
    hipError_t err = hipModuleLaunchKernel(fn, (uint32_t)G, 1, 1, 5 * 64, 1, 1, 0, stream, params, nullptr);
    if (err != hipSuccess) return hip_fail(err, "launch(small ffn stack)");
    return HH_OK;
}

hh_status hh_engine::enqueue_ffn_block_stack(const hh_ffn_desc* d, const uint8_t* pack, size_t stride,
                                             size_t n_layers, const float* norm, size_t norm_stride, float eps,
                                             const float* x, float* y) {
    if (n_layers == 0) return HH_OK;
    hh_status st = enqueue_small_stack(d, pack, stride, n_layers, norm, norm_stride, eps, x, y);
    if (st == HH_OK) {
        ffn_stage_valid = false;
        ffn_calls += 3 * n_layers;
        return HH_OK;
    }
    if (st != HH_ERR_UNSUPPORTED_DEVICE) return st;
    for (size_t l = 0; l < n_layers; l++)
        HH_TRY(enqueue_ffn_block(d, pack + l * stride, l == 0 ? x : y, norm + l * norm_stride, eps, y));
    return HH_OK;
}

// The FFN residual block of one token: y = x + FFN(RMSNorm(x)) (ffn_apply,
// crates/hayai-core/src/hybrid_infer.rs:883-936, with rms_norm of
// crates/hayai-cpu/src/attention.rs:142-147).  The ring kernels fuse both neighbours: gate/up
// normalizes x while quantizing it, down adds the residual as it stores y.  Other layouts
// run RMSNorm, the FFN and the residual add as three steps.  y may be x.
hh_status hh_engine::enqueue_ffn_block(const hh_ffn_desc* d, const uint8_t* pack, const float* x, const float* norm,
                                       float eps, float* y) {
    const uint8_t* wg = pack + d->gate_off;
    const uint8_t* wu = pack + d->up_off;
    const uint8_t* wd = pack + d->down_off;
    if (ring_ok(d, wg, wu, wd, x) && ((uintptr_t)norm & 15u) == 0) {
        HH_TRY(enqueue_ring_gu(d, wg, wu, x, norm, eps));
        HH_TRY(enqueue_ring_dn(d, wd, y, x));
        ffn_stage_valid = false;
        ffn_calls += 3;
        return HH_OK;
    }
    const size_t dm = d->d_model;
    HH_TRY(grow(&ws_xn, &ws_xn_cap, dm * sizeof(float)));
    HH_TRY(grow(&ws_f, &ws_f_cap, dm * sizeof(float)));
    hipFunction_t fn;
    HH_TRY(kernel("hh_rmsnorm_kernel", &fn));
    hh_norm_args na{x, norm, (float*)ws_xn, (uint32_t)dm, eps};
    HH_TRY(launch(fn, 1, 1024, na));
    HH_TRY(enqueue_ffn(d, pack, (const float*)ws_xn, (float*)ws_f));
    HH_TRY(kernel("hh_add_kernel", &fn));
    hh_add_args aa{x, (const float*)ws_f, y, (uint32_t)dm, 0u};
    return launch(fn, (uint32_t)((dm + 255) / 256), 256, aa);
}

// ---------------------------------------------------------------- batched (MFMA) ------

// Kernel argument block of hh_mm_prep (mm_common.hip, same layout).
struct hh_mm_prep_args {
    const float* x;
    void* xop;
    uint32_t b, n, T, pad;
};
constexpr size_t kMmMaxTokens = 64;  // tokens per MFMA launch (4 tiles of 16)
constexpr size_t kMmStage = 17408;   // bytes of one (16-token tile, superblock) operand stage

static size_t mm_stage_bytes(size_t n, size_t tt) { return tt * (n / 256) * kMmStage; }

hh_status hh_engine::enqueue_mm_prep(const float* x, size_t b, size_t n, size_t tt) {
    HH_TRY(grow(&ws_xop, &ws_xop_cap, mm_stage_bytes(n, tt)));
    hipFunction_t fn;
    HH_TRY(kernel("hh_mm_prep", &fn));
    const size_t T = 16 * tt;
    hh_mm_prep_args a{x, ws_xop, (uint32_t)b, (uint32_t)n, (uint32_t)T, 0};
    const size_t threads = T * (n / 16);
    return launch(fn, (uint32_t)((threads + 255) / 256), 256, a);
}

// Kernel argument block of q4k_mmr.hip (same layout).
struct hh_mmr_args {
    const uint8_t* w0;
    const uint8_t* w1;
    const void* xop;
    float* y;
    void* hop;
    float* part;
    unsigned* cnt;
    uint64_t row_bytes;
    uint32_t m, n, b, nw, kc;
    int32_t act;
};
constexpr size_t kMmrMaxTokens = 16;
constexpr size_t kMmrStageHi = 9216;     // single-f16 token stage (the down projection's h)
constexpr size_t kMmrTileLds = 8 * 512;  // gate/up: per-wave 512-byte transposition tile after the stages

static size_t mmr_stage_bytes(int kind) { return kind == hh_engine::MMR_DN ? kMmrStageHi : kMmStage; }

// Work split of a weight-stream launch over nu 16-row units and nsb superblocks: chunks of
// S superblocks (their token stages in LDS) and nw units (one wave each) per workgroup.  A
// CU holds res = min(LDS / stages, 8 / nw) workgroups at once (the kernels need more than
// 128 VGPRs: at most two waves per SIMD); its stream rate is taken as proportional to its
// resident waves (up to 8), plus a fixed start-up cost of about two items per round (stage
// copy, first-data latency).  Ties go to the split that fills more of the CU slots, then to
// longer chunks (fewer partial sums).
struct mmr_plan {
    int S = 0;
    uint32_t nw = 0, kc = 0, groups = 0;
};
static mmr_plan plan_mmr(int kind, size_t nu, size_t nsb, size_t cus, size_t lds) {
    static const int gu_s[] = {8, 7, 4, 2}, dn_s[] = {16, 14, 8, 7, 4, 2};
    const int* ss = kind == hh_engine::MMR_DN ? dn_s : gu_s;
    const size_t nss = kind == hh_engine::MMR_DN ? 6 : 4;
    const size_t sb = mmr_stage_bytes(kind), extra = (kind == hh_engine::MMR_GU ? kMmrTileLds : 0) + 64;
    mmr_plan best;
    double best_cost = 1e300, best_fill = 0;
    for (size_t si = 0; si < nss; si++) {
        const int S = ss[si];
        if (S > 2 && (size_t)S > nsb) continue;
        const size_t kc = (nsb + S - 1) / S;
        const size_t by_lds = lds / ((size_t)S * sb + extra);
        if (by_lds == 0) continue;
        for (size_t nw = 8; nw >= 1; nw--) {
            const size_t groups = (nu + nw - 1) / nw;
            const size_t wgs = groups * kc;
            const size_t res = std::min(by_lds, 8 / nw);
            const size_t rounds = (wgs + cus * res - 1) / (cus * res);
            const double cost = (double)rounds * ((double)(res * nw * S) / (double)std::min<size_t>(nw * res, 8) + 2.0);
            const double fill = (double)wgs / (double)(rounds * cus * res);
            if (cost < best_cost - 1e-9 || (cost < best_cost + 1e-9 && fill > best_fill + 1e-9)) {
                best_cost = cost;
                best_fill = fill;
                best.S = S;
                best.nw = (uint32_t)nw;
                best.kc = (uint32_t)kc;
                best.groups = (uint32_t)groups;
            }
        }
    }
    return best;
}

bool hh_engine::mmr_ok(size_t m, size_t n, size_t b, const void* w0, const void* w1, const void* x) const {
    return mmr && !q4k_generic && b >= 1 && b <= kMmrMaxTokens && m >= 1 && n >= 256 && n % 256 == 0 &&
           m <= 0x7FFFFFFFu && n <= 0x7FFFFFFFu && ((((uintptr_t)w0 | (uintptr_t)w1 | (uintptr_t)x) & 15u) == 0);
}

hh_status hh_engine::enqueue_q4k_mmr(int kind, size_t m, size_t n, const uint8_t* w0, const uint8_t* w1, const void* x,
                                     size_t b, float* y, int act) {
    if (!mmr_ok(m, n, b, w0, kind == MMR_GU ? w1 : w0, x) || (kind == MMR_GU && m % 256 != 0))
        return HH_ERR_UNSUPPORTED_DEVICE;
    const size_t nsb = n / 256, nu = (m + 15) / 16;
    const mmr_plan pl = plan_mmr(kind, nu, nsb, (size_t)props.multiProcessorCount, (size_t)props.sharedMemPerBlock);
    if (pl.S == 0) return HH_ERR_UNSUPPORTED_DEVICE;
    const size_t smem = (size_t)pl.S * mmr_stage_bytes(kind) + (kind == MMR_GU ? kMmrTileLds : 0);
    const size_t nt = kind == MMR_GU ? 2 : 1;
    if (pl.kc > 1) {
        HH_TRY(grow(&ws_part, &ws_part_cap, (size_t)pl.groups * pl.kc * pl.nw * nt * 256 * sizeof(float)));
        if (ws_cnt_cap < pl.groups * sizeof(unsigned)) {
            HH_TRY(grow(&ws_cnt, &ws_cnt_cap, pl.groups * sizeof(unsigned)));
            HH_TRY_HIP(hipMemsetAsync(ws_cnt, 0, ws_cnt_cap, stream), "hipMemsetAsync(counters)");
        }
    }
    // the input's token stages: f32 tokens are staged once per call (hi + lo halves); the down
    // projection reads the gate/up kernel's single-f16 stages of h
    const void* xop = x;
    if (kind != MMR_DN) {
        HH_TRY(enqueue_mm_prep((const float*)x, b, n, 1));
        xop = ws_xop;
    }
    if (kind == MMR_GU) HH_TRY(grow(&ws_hop, &ws_hop_cap, (m / 256) * kMmrStageHi));
    static const char* kinds[] = {"hh_q4k_mmr_s", "hh_q4k_mmr_gu_s", "hh_q4k_mmr_dn_s"};
    hipFunction_t fn;
    HH_TRY(kernel(std::string(kinds[kind]) + std::to_string(pl.S), &fn));
    hh_mmr_args a{};
    a.w0 = w0;
    a.w1 = kind == MMR_GU ? w1 : w0;
    a.xop = xop;
    a.y = y;
    a.hop = ws_hop;
    a.part = (float*)ws_part;
    a.cnt = (unsigned*)ws_cnt;
    a.row_bytes = (uint64_t)(nsb * 144);
    a.m = (uint32_t)m;
    a.n = (uint32_t)n;
    a.b = (uint32_t)b;
    a.nw = pl.nw;
    a.kc = pl.kc;
    a.act = act;
    void* params[] = {&a};
    hipError_t err = hipModuleLaunchKernel(fn, pl.groups * pl.kc, 1, 1, pl.nw * 64, 1, 1, (unsigned)smem, stream,
                                           params, nullptr);
    if (err != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel(q4k_mmr)");
    return HH_OK;
}

// ---- batched Q4_K with int8 activations (q4k_mmi.hip) ----

// Batched Q4_K with int8 activations (q4k_mmi.hip) from 17 tokens on: at 16 the f16
// weight-stream kernels (q4k_mmr.hip) are faster on the MI355X (8B FFN, 32 layers: 1.26 ms
// f16 vs 1.50 ms int8).
constexpr size_t kMmqMinTokens = 17, kMmqMaxTokens = 64;

bool hh_engine::mmq_ok(size_t m, size_t n, size_t b, const void* w0, const void* w1, const void* x) const {
    return mmq && !q4k_generic && b >= std::min(mmi_min, kMmqMinTokens) && b >= 2 && b <= kMmqMaxTokens && m >= 1 &&
           m <= 0xFFFFFFFFu && n >= 256 && n % 256 == 0 && n <= 0xFFFFFFFFu &&
           ((((uintptr_t)w0 | (uintptr_t)w1 | (uintptr_t)x) & 15u) == 0);
}

// Must match struct hh_mmi_prep_args / hh_mmi_args in kernels/q4k_mmi.hip.
struct MmiPrepArgs {
    const float* x;
    uint8_t* xs;
    uint32_t n, b, tt, pad;
};
struct MmiArgs {
    const uint8_t* w0;
    const uint8_t* w1;
    const uint8_t* xs;
    float* y;
    uint8_t* hs;
    float* part;
    unsigned* cnt;
    uint64_t row_bytes;
    uint32_t m, n, b, kc, sbc;
    int32_t act;
};
constexpr size_t kMmiStage = 9216, kMmiWaves = 4, kMmiLds = 147456;
// 16-token tiles of a pass: an FFN's three token tiles run as four (its gate/up kernel is
// instantiated for 1, 2 and 4), and its prep, gate/up and down agree on the count
static size_t mmi_tiles(bool ffn, size_t b) {
    const size_t tt = (b + 15) / 16;
    return ffn && tt == 3 ? 4 : tt;
}

hh_status hh_engine::enqueue_mmi_prep(const float* x, size_t b, size_t n, size_t tt, void* xs) {
    hipFunction_t fn;
    HH_TRY(kernel("hh_mmi_prep", &fn));
    MmiPrepArgs a{x, (uint8_t*)xs, (uint32_t)n, (uint32_t)b, (uint32_t)tt, 0u};
    const size_t teams = 16 * tt * (n / 32);  // one 32-lane team per (token, block), 8 per workgroup
    return launch(fn, (uint32_t)((teams + 7) / 8), 256, a);
}

// Workgroups of 4 units (64 rows), two waves per unit, + a copy wave.  FFN gate/up: whole rows
// (one chunk), so the workgroup quantizes its own rows of h; GEMM / down: the superblocks split
// into chunks so that the grid fills the CUs once, the chunks' partial sums added by the last
// workgroup of a group.
hh_status hh_engine::enqueue_q4k_mmi(bool ffn, size_t m, size_t n, const uint8_t* w0, const uint8_t* w1,
                                     const void* xs, size_t b, float* y, void* hs, int act, size_t tiles) {
    const size_t tt = tiles ? tiles : mmi_tiles(ffn, b), nsb = n / 256, nu = (m + 15) / 16;
    const size_t groups = (nu + kMmiWaves - 1) / kMmiWaves;
    size_t kc = 1, sbc = nsb;
    if (!ffn) {
        const size_t cus = (size_t)props.multiProcessorCount;
        kc = std::max<size_t>(1, std::min(nsb, (cus + groups / 2) / groups));
        sbc = (nsb + kc - 1) / kc;
        kc = (nsb + sbc - 1) / sbc;
    }
    const size_t slot = kMmiStage * tt, ring = std::min<size_t>(16, kMmiLds / slot);
    const bool refill = sbc > ring;  // the chunk's stages stream through the LDS ring
    const int D = ffn ? 2 : mmi_d == 2 || mmi_d == 4 ? mmi_d : (sbc % 4 == 0 ? 4 : 2);
    if (kc > 1) {
        HH_TRY(grow(&ws_part, &ws_part_cap, groups * kc * kMmiWaves * tt * 4 * 64 * sizeof(float)));
        if (ws_cnt_cap < groups * sizeof(unsigned)) {
            HH_TRY(grow(&ws_cnt, &ws_cnt_cap, groups * sizeof(unsigned)));
            HH_TRY_HIP(hipMemsetAsync(ws_cnt, 0, ws_cnt_cap, stream), "hipMemsetAsync(counters)");
        }
    }
    hipFunction_t fn;
    HH_TRY(kernel(std::string(ffn ? "hh_q4k_mmi_gu_t" : "hh_q4k_mmi_t") + std::to_string(tt) + "_d" + std::to_string(D) +
                      (refill ? "_r" : "_w"),
                  &fn));
    MmiArgs a{};
    a.w0 = w0;
    a.w1 = ffn ? w1 : w0;
    a.xs = (const uint8_t*)xs;
    a.y = y;
    a.hs = (uint8_t*)hs;
    a.part = (float*)ws_part;
    a.cnt = (unsigned*)ws_cnt;
    a.row_bytes = (uint64_t)(nsb * 144);
    a.m = (uint32_t)m;
    a.n = (uint32_t)n;
    a.b = (uint32_t)b;
    a.kc = (uint32_t)kc;
    a.sbc = (uint32_t)sbc;
    a.act = act;
    const size_t smem = (refill ? ring : sbc) * slot;
    void* params[] = {&a};
    hipError_t err = hipModuleLaunchKernel(fn, (unsigned)(groups * kc), 1, 1, (unsigned)((2 * kMmiWaves + 1) * 64), 1, 1,
                                           (unsigned)smem, stream, params, nullptr);
    if (err != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel(q4k_mmi)");
    return HH_OK;
}

hh_status hh_engine::enqueue_gemv_batched(int type, size_t m, size_t n, const uint8_t* w, const float* x, size_t batch,
                                          float* y) {
    if (batch == 0) return HH_OK;
    const bool mfma = type == HH_TYPE_Q4_K && batch >= 2 && !q4k_generic && ((uintptr_t)w & 15u) == 0 &&
                      ((uintptr_t)x & 15u) == 0 && m <= 0xFFFFFFFFu && n <= 0xFFFFFFFFu;
    if (!mfma) {
        for (size_t b = 0; b < batch; b++) HH_TRY(enqueue_gemv(type, m, n, w, x + b * n, y + b * m));
        return HH_OK;
    }
    for (size_t b0 = 0; b0 < batch; b0 += kMmMaxTokens) {
        const size_t nb = std::min(kMmMaxTokens, batch - b0);
        if (nb == 1) {
            HH_TRY(enqueue_gemv(type, m, n, w, x + b0 * n, y + b0 * m));
            continue;
        }
        if (nb >= mmi_min && mmq_ok(m, n, nb, w, w, x + b0 * n)) {
            // int8 activations on the f16 matrix cores
            const size_t tt = (nb + 15) / 16;
            HH_TRY(grow(&ws_xop, &ws_xop_cap, (n / 256) * tt * kMmiStage));
            HH_TRY(enqueue_mmi_prep(x + b0 * n, nb, n, tt, ws_xop));
            HH_TRY(enqueue_q4k_mmi(false, m, n, w, nullptr, ws_xop, nb, y + b0 * m, nullptr, 0));
            continue;
        }
        if (nb <= kMmrMaxTokens && mmr_ok(m, n, nb, w, w, x + b0 * n)) {
            HH_TRY(enqueue_q4k_mmr(MMR_GEMM, m, n, w, nullptr, x + b0 * n, nb, y + b0 * m, 0));
            continue;
        }
        for (size_t b = b0; b < b0 + nb; b++) HH_TRY(enqueue_gemv(type, m, n, w, x + b * n, y + b * m));
    }
    return HH_OK;
}

hh_status hh_engine::enqueue_ffn_batched(const hh_ffn_desc* d, const uint8_t* pack, const float* x, size_t batch,
                                         float* y) {
    if (batch == 0) return HH_OK;
    const size_t dm = d->d_model, df = d->d_ff;
    const uint8_t* wg = pack + d->gate_off;
    const uint8_t* wu = pack + d->up_off;
    const uint8_t* wd = pack + d->down_off;
    const bool mfma = d->type_gate == HH_TYPE_Q4_K && d->type_up == HH_TYPE_Q4_K && d->type_down == HH_TYPE_Q4_K &&
                      batch >= 2 && !q4k_generic && (((uintptr_t)wg | (uintptr_t)wu | (uintptr_t)wd | (uintptr_t)x) & 15u) == 0;
    // Q4_K_M layers (Q4_K gate/up, Q6_K down): gate and up for all tokens as weight-stream MFMA
    // GEMMs, the activation over [batch][d_ff], then the Q6_K ring GEMV per token.
    const bool q4km = d->type_gate == HH_TYPE_Q4_K && d->type_up == HH_TYPE_Q4_K && d->type_down == HH_TYPE_Q6_K &&
                      batch >= 4 && batch <= kMmrMaxTokens && df % 512 == 0 && !capturing &&
                      mmr_ok(df, dm, batch, wg, wg, x) && mmr_ok(df, dm, batch, wu, wu, x) &&
                      (((uintptr_t)wd | (uintptr_t)x) & 15u) == 0;
    if (q4km) {
        HH_TRY(grow(&ws_g, &ws_g_cap, batch * df * sizeof(float)));
        HH_TRY(grow(&ws_u, &ws_u_cap, batch * df * sizeof(float)));
        HH_TRY(grow(&ws_h, &ws_h_cap, batch * df * sizeof(float)));
        HH_TRY(enqueue_q4k_mmr(MMR_GEMM, df, dm, wg, nullptr, x, batch, (float*)ws_g, 0));
        HH_TRY(enqueue_q4k_mmr(MMR_GEMM, df, dm, wu, nullptr, x, batch, (float*)ws_u, 0));
        hipFunction_t fn;
        HH_TRY(kernel("hh_act_mul_kernel", &fn));
        hh_act_args aa{(const float*)ws_g, (const float*)ws_u, (float*)ws_h, (uint32_t)(batch * df), d->act};
        HH_TRY(launch(fn, (uint32_t)((batch * df + 255) / 256), 256, aa));
        for (size_t b = 0; b < batch; b++) {
            const hh_status st = enqueue_ring_gemv(HH_TYPE_Q6_K, dm, df, wd, (const float*)ws_h + b * df, y + b * dm);
            if (st == HH_ERR_UNSUPPORTED_DEVICE)
                HH_TRY(enqueue_gemv(HH_TYPE_Q6_K, dm, df, wd, (const float*)ws_h + b * df, y + b * dm));
            else if (st != HH_OK)
                return st;
        }
        ffn_stage_valid = false;
        ffn_calls += 3 * batch;
        return HH_OK;
    }
    if (!mfma) {
        for (size_t b = 0; b < batch; b++) HH_TRY(enqueue_ffn(d, pack, x + b * dm, y + b * dm));
        return HH_OK;
    }
    for (size_t b0 = 0; b0 < batch; b0 += kMmMaxTokens) {
        const size_t nb = std::min(kMmMaxTokens, batch - b0);
        if (nb == 1) {
            HH_TRY(enqueue_ffn(d, pack, x + b0 * dm, y + b0 * dm));
            continue;
        }
        if (nb >= mmi_min && df % 256 == 0 && mmq_ok(df, dm, nb, wg, wu, x + b0 * dm) &&
            mmq_ok(dm, df, nb, wd, wd, wd)) {
            // int8 activations on the f16 matrix cores: x -> stages, gate/up + act -> h stages
            // (quantized in the gate/up kernel), down
            const size_t tt = mmi_tiles(true, nb);
            HH_TRY(grow(&ws_xop, &ws_xop_cap, (dm / 256) * tt * kMmiStage));
            HH_TRY(grow(&ws_hop, &ws_hop_cap, (df / 256) * tt * kMmiStage));
            HH_TRY(enqueue_mmi_prep(x + b0 * dm, nb, dm, tt, ws_xop));
            HH_TRY(enqueue_q4k_mmi(true, df, dm, wg, wu, ws_xop, nb, nullptr, ws_hop, d->act));
            HH_TRY(enqueue_q4k_mmi(false, dm, df, wd, nullptr, ws_hop, nb, y + b0 * dm, nullptr, 0, tt));
            ffn_stage_valid = false;
            ffn_calls += 3 * nb;
            continue;
        }
        if (nb <= kMmrMaxTokens && df % 256 == 0 && mmr_ok(df, dm, nb, wg, wu, x + b0 * dm) &&
            mmr_ok(dm, df, nb, wd, wd, wd)) {
            HH_TRY(enqueue_q4k_mmr(MMR_GU, df, dm, wg, wu, x + b0 * dm, nb, nullptr, d->act));
            HH_TRY(enqueue_q4k_mmr(MMR_DN, dm, df, wd, nullptr, ws_hop, nb, y + b0 * dm, 0));
            ffn_calls += 3 * nb;
            continue;
        }
        for (size_t b = b0; b < b0 + nb; b++) HH_TRY(enqueue_ffn(d, pack, x + b * dm, y + b * dm));
    }
    return HH_OK;
}

// ---------------------------------------------------------------- MoE ----------------

// Kernel argument blocks of moe.hip (same layout).
struct hh_route_args {
    const float* logits;
    const float* bias;
    int32_t* ids;
    float* wts;
    uint32_t T, E, top_k, k_out;
    uint32_t n_group, topk_group;
    int32_t gating, norm;
    float scale;
    uint32_t pad;
};
struct hh_moe_args {
    const uint8_t* experts;
    uint64_t expert_stride;
    uint64_t gate_off, up_off, down_off;
    uint64_t rb_in, rb_ff;
    int32_t* ids;
    float* wts;
    const float* x;
    float* h;
    float* y;
    uint32_t d_model, d_ff, k, n_experts;
    int32_t act;
    uint32_t route;
    hh_route_args r;
};
constexpr int kMoeBlock = 256;
constexpr size_t kLdsBytes = 160 * 1024;  // LDS per workgroup on gfx950
constexpr size_t kMoeDownRows = 4;  // output rows per down workgroup (moe.hip)
constexpr size_t kMoegGuRows = 2, kMoegDnRows = 4;  // grouped MoE rows per team (HH_MOEG_*_RPT, moe_group.hip)
constexpr size_t kMoegRecInts = 8;                   // ints per grouped-MoE expert record (HH_MOEG_REC)

static int moe_team(size_t units) { return units <= 16 ? 16 : (units <= 32 ? 32 : 64); }

static hh_route_args route_args(const hh_moe_desc* d, const float* logits, const float* bias, size_t T, int32_t* ids,
                                float* wts) {
    return hh_route_args{logits, bias, ids, wts, (uint32_t)T, (uint32_t)d->n_experts, (uint32_t)d->top_k,
                         (uint32_t)d->top_k, (uint32_t)d->n_group, (uint32_t)d->topk_group, d->gating,
                         d->norm_topk_prob, d->routed_scaling_factor, 0};
}

hh_status hh_engine::enqueue_moe_route(const hh_moe_desc* d, const float* logits, const float* bias, size_t T,
                                       int32_t* ids, float* wts) {
    if (T == 0) return HH_OK;
    hipFunction_t fn;
    HH_TRY(kernel("hh_moe_route", &fn));
    const hh_route_args a = route_args(d, logits, bias, T, ids, wts);
    return launch(fn, (uint32_t)((T + 3) / 4), kMoeBlock, a);
}

hh_status hh_engine::enqueue_moe_ffn(const hh_moe_desc* d, const uint8_t* experts, const float* x, size_t T,
                                     int32_t* ids, float* wts, float* y, const float* logits, const float* bias) {
    if (T == 0) return HH_OK;
    const size_t k = d->top_k, dm = d->d_model, df = d->d_ff;
    HH_TRY(grow(&ws_moe_h, &ws_moe_h_cap, T * k * df * sizeof(float)));
    hh_moe_args a{};
    a.experts = experts;
    a.expert_stride = d->expert_stride;
    a.gate_off = d->gate_off;
    a.up_off = d->up_off;
    a.down_off = d->down_off;
    a.rb_in = (dm / 256) * 144;
    a.rb_ff = (df / 256) * 144;
    a.ids = ids;
    a.wts = wts;
    a.x = x;
    a.h = (float*)ws_moe_h;
    a.y = y;
    a.d_model = (uint32_t)dm;
    a.d_ff = (uint32_t)df;
    a.k = (uint32_t)k;
    a.n_experts = (uint32_t)d->n_experts;
    a.act = d->act;
    a.route = logits != nullptr;
    if (logits) a.r = route_args(d, logits, bias, T, ids, wts);
    // One token (decode): the ring kernels (moe_ring.hip), when the shape allows them.
    const size_t K = k * df, uin = dm / 64;
    if (T == 1 && ring && (uin == 16 || uin == 32 || uin == 64) && df % 256 == 0 && K / 64 <= 512 &&
        ((d->expert_stride | d->gate_off | d->up_off | d->down_off | (uintptr_t)experts | (uintptr_t)x) & 15u) == 0) {
        HH_TRY(grow(&ws_moe_hx, &ws_moe_hx_cap, 2 * K + (K / 8) * 4 + 16));
        struct {
            hh_moe_args m;
            uint8_t* hx;
        } ra{a, (uint8_t*)ws_moe_hx};
        void* rparams[] = {&ra};
        const size_t cus = (size_t)props.multiProcessorCount;
        {
            const std::string name = "hh_moe_gu_ring_u" + std::to_string(uin);
            hipFunction_t fn;
            HH_TRY(kernel(name, &fn));
            const size_t rr_max = 2 * 8 * ((K / 8 + cus - 1) / cus);
            const size_t smem = (((2 * dm + (dm / 32) * 8) + 15) & ~size_t(15)) + ((rr_max + 3) & ~size_t(3)) * 4 + 128;
            HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)cus, 1, 1, 8 * 64, 1, 1, (unsigned)smem, stream, rparams,
                                             nullptr),
                       "launch(moe ring gate/up)");
        }
        {
            int w2 = 1;
            while ((size_t)w2 * 64 < K / 64) w2 *= 2;
            const std::string name = "hh_moe_dn_ring_d" + std::to_string(w2);
            hipFunction_t fn;
            HH_TRY(kernel(name, &fn));
            const size_t rows_max = (dm + cus - 1) / cus;
            const size_t smem = (((2 * K + (K / 8) * 4) + 15) & ~size_t(15)) + rows_max * (size_t)w2 * 64 * 4;
            if (smem > props.sharedMemPerBlock) return fail(HH_ERR_INVALID, "moe: expert intermediate too large");
            HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)cus, 1, 1, 9 * 64, 1, 1, (unsigned)smem, stream, rparams,
                                             nullptr),
                       "launch(moe ring down)");
        }
        ffn_calls += 3;
        return HH_OK;
    }
    // Several tokens: the grouped gather-GEMV (moe_group.hip), every selected expert read once.
    const size_t P = T * k, E = d->n_experts;
    if (moe_grouped && P <= 4096 && E <= 512 && dm / 64 <= 64 && df / 64 <= 64 &&
        ((d->expert_stride | d->gate_off | d->up_off | d->down_off | (uintptr_t)experts | (uintptr_t)x) & 15u) == 0) {
        HH_TRY(grow(&ws_moe_yp, &ws_moe_yp_cap, P * dm * sizeof(float)));
        const size_t gy = std::min(E, P);  // grid rows of the grouped kernels: the most active experts
        HH_TRY(grow(&ws_moe_grp, &ws_moe_grp_cap, (P + gy * kMoegRecInts) * sizeof(int32_t)));
        const size_t xqb = hh_digits_bytes(dm), hqb = hh_digits_bytes(df);
        HH_TRY(grow(&ws_moe_q, &ws_moe_q_cap, T * xqb + P * hqb));
        struct {
            const uint8_t* experts;
            uint64_t expert_stride, gate_off, up_off, down_off, rb_in, rb_ff;
            const int32_t* ids;
            const float* wts;
            const float* x;
            float *h, *yp, *y;
            int32_t *order, *rec;
            uint8_t *xq, *hq;
            uint32_t T, k, d_model, d_ff, n_experts;
            int32_t act;
        } g{experts, d->expert_stride, d->gate_off, d->up_off, d->down_off, a.rb_in, a.rb_ff, ids, wts, x,
            (float*)ws_moe_h, (float*)ws_moe_yp, y, (int32_t*)ws_moe_grp + gy * kMoegRecInts,
            (int32_t*)ws_moe_grp, (uint8_t*)ws_moe_q, (uint8_t*)ws_moe_q + T * xqb, (uint32_t)T,
            (uint32_t)k, (uint32_t)dm, (uint32_t)df, (uint32_t)E, d->act};
        hipFunction_t fn;
        if (logits) {
            // routing, grouping and x's digits in one launch (hh_moe_route_prep): the last
            // routing workgroup to finish groups the pairs; its arrival counter is a word of
            // the grid-barrier state that every launch leaves at zero
            struct {
                hh_route_args r;
                decltype(g) m;
                unsigned* arrivals;
            } rp{route_args(d, logits, bias, T, ids, wts), g, (unsigned*)((char*)grid_sync + kBarMoeArrivalsOffset)};
            HH_TRY(kernel("hh_moe_route_prep", &fn));
            void* rpp[] = {&rp};
            HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)((T + 3) / 4 + T), 1, 1, kMoeBlock, 1, 1, 0, stream, rpp,
                                             nullptr),
                       "launch(moe route + prep)");
        } else {
            HH_TRY(kernel("hh_moe_prep", &fn));
            HH_TRY(launch(fn, (uint32_t)(1 + T), 256, g));
        }
        {
            const int team = moe_team(dm / 64);
            const size_t rows = (size_t)(kMoeBlock / team) * kMoegGuRows;
            HH_TRY(kernel("hh_moe_gu_grp_t" + std::to_string(team), &fn));
            void* gp[] = {&g};
            HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)((df + rows - 1) / rows), (uint32_t)gy, 1, kMoeBlock, 1, 1, 0, stream,
                                             gp, nullptr),
                       "launch(moe grouped gate/up)");
        }
        HH_TRY(kernel("hh_moe_hdigits", &fn));
        HH_TRY(launch(fn, (uint32_t)P, 256, g));
        {
            const int team = moe_team(df / 64);
            const size_t rows = (size_t)(kMoeBlock / team) * kMoegDnRows;
            HH_TRY(kernel("hh_moe_dn_grp_t" + std::to_string(team), &fn));
            void* gp[] = {&g};
            HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)((dm + rows - 1) / rows), (uint32_t)gy, 1, kMoeBlock, 1, 1, 0, stream,
                                             gp, nullptr),
                       "launch(moe grouped down)");
        }
        HH_TRY(kernel("hh_moe_combine", &fn));
        {
            void* gp[] = {&g};
            HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)((dm + 255) / 256), (uint32_t)T, 1, 256, 1, 1, 0, stream, gp,
                                             nullptr),
                       "launch(moe combine)");
        }
        ffn_calls += 3 * T;
        return HH_OK;
    }
    const size_t cap = std::max<size_t>(1, ((size_t)props.multiProcessorCount * 2 + T - 1) / T);
    void* params[] = {&a};
    {
        const int team = moe_team(dm / 64);
        const size_t tpb = kMoeBlock / team;
        const size_t gx = std::max<size_t>(1, std::min((k * df + tpb - 1) / tpb, cap));
        const std::string name = "hh_moe_gateup_t" + std::to_string(team);
        hipFunction_t fn;
        HH_TRY(kernel(name, &fn));
        HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)gx, (uint32_t)T, 1, kMoeBlock, 1, 1,
                                         (unsigned)hh_digits_bytes(dm), stream, params, nullptr),
                   "launch(moe gate/up)");
    }
    {
        const int team = moe_team(df / 64);
        const size_t gx = (dm + kMoeDownRows - 1) / kMoeDownRows;
        const std::string name = "hh_moe_down_t" + std::to_string(team);
        hipFunction_t fn;
        HH_TRY(kernel(name, &fn));
        HH_TRY_HIP(hipModuleLaunchKernel(fn, (uint32_t)gx, (uint32_t)T, 1, kMoeBlock, 1, 1,
                                         (unsigned)hh_digits_bytes(k * df), stream, params, nullptr),
                   "launch(moe down)");
    }
    ffn_calls += 3 * T;
    return HH_OK;
}

// The shared expert (DeepSeek-style, crates/hayai-core/src/moe_infer.rs:456-493): an FFN of
// d_model x shared_d_ff added with weight 1 after the routed experts' sum (acc[j] += d[j],
// then the caller's x += acc).  One token: the ring kernels, the down kernel adding its output
// to y as it stores (y = y + down).  Several tokens: the batched FFN in passes of at most 16
// tokens (the f16 weight-stream MFMA kernels, f32-level accuracy: no int8 activations here),
// into a workspace, then y += it.
hh_status hh_engine::enqueue_moe_shared(const hh_moe_desc* d, const uint8_t* experts, const float* x, size_t T,
                                        float* y) {
    if (d->shared_d_ff == 0 || T == 0) return HH_OK;
    if (T * d->d_model > 0xFFFFFFFFu) return fail(HH_ERR_INVALID, "moe: %zu tokens too many for the shared expert", T);
    const hh_ffn_desc s{d->type, d->type, d->type, d->act, d->d_model, d->shared_d_ff,
                        d->shared_gate_off, d->shared_up_off, d->shared_down_off};
    const size_t dm = d->d_model;
    if (T == 1 && ring_ok(&s, experts + s.gate_off, experts + s.up_off, experts + s.down_off, x)) {
        HH_TRY(enqueue_ring_gu(&s, experts + s.gate_off, experts + s.up_off, x));
        HH_TRY(enqueue_ring_dn(&s, experts + s.down_off, y, y));
        ffn_calls += 3;
        return HH_OK;
    }
    HH_TRY(grow(&ws_f, &ws_f_cap, T * dm * sizeof(float)));
    for (size_t b0 = 0; b0 < T; b0 += kMmrMaxTokens) {
        const size_t nb = std::min(kMmrMaxTokens, T - b0);
        HH_TRY(enqueue_ffn_batched(&s, experts, x + b0 * dm, nb, (float*)ws_f + b0 * dm));
    }
    hipFunction_t fn;
    HH_TRY(kernel("hh_add_kernel", &fn));
    hh_add_args aa{y, (const float*)ws_f, y, (uint32_t)(T * dm), 0u};
    return launch(fn, (uint32_t)((T * dm + 255) / 256), 256, aa);
}

// ---------------------------------------------------------------- bring-up -----------

static std::vector<std::string> required_kernels() {
    std::vector<std::string> k;
    const char* gemv_fmts[] = {"q4_k", "q4_k_unaligned", "q4_0", "iq2_xxs", "iq3_xxs", "q8_0", "q6_k", "f32", "f16"};
    const char* gateup_fmts[] = {"q4_k", "q4_k_unaligned", "q4_0", "iq2_xxs", "iq3_xxs", "q8_0", "q6_k"};
    for (int i = 0; i < kNumTeamCfgs; i++) {
        std::string suf = "_t" + std::to_string(kTeamCfgs[i].team) + "_u" + std::to_string(kTeamCfgs[i].upl);
        for (const char* f : gemv_fmts) k.push_back(std::string("hh_gemv_") + f + suf);
        for (const char* f : gateup_fmts) k.push_back(std::string("hh_gateup_") + f + suf);
    }
    for (const char* s : {"hh_gemv_f32_plain", "hh_gemv_f16_plain", "hh_act_mul_kernel", "hh_dequant_q4_0",
                          "hh_dequant_q4_k", "hh_dequant_iq2_xxs", "hh_dequant_iq3_xxs", "hh_dequant_q8_0",
                          "hh_dequant_q6_k", "hh_dequant_f16",
                          "hh_synth_bytes", "hh_synth_scales"})
        k.push_back(s);
    for (int w : {1, 2, 4, 8})
        for (const char* kind : {"hh_q4k_gemv_w", "hh_q4k_gemvq_w", "hh_q4k_gateup_w"})
            k.push_back(std::string(kind) + std::to_string(w));
    k.push_back("hh_mm_prep");
    for (int S : {2, 4, 7, 8})
        for (const char* kind : {"hh_q4k_mmr_s", "hh_q4k_mmr_gu_s"}) k.push_back(std::string(kind) + std::to_string(S));
    for (int S : {2, 4, 7, 8, 14, 16}) k.push_back("hh_q4k_mmr_dn_s" + std::to_string(S));
    k.push_back("hh_mmi_prep");
    for (int t = 1; t <= 4; t++)
        for (const char* f : {"_d2_w", "_d4_w", "_d2_r", "_d4_r"}) k.push_back("hh_q4k_mmi_t" + std::to_string(t) + f);
    for (const char* f : {"t1_d2_w", "t1_d2_r", "t2_d2_w", "t2_d2_r", "t4_d2_w", "t4_d2_r"})
        k.push_back(std::string("hh_q4k_mmi_gu_") + f);
    k.push_back("hh_lut_gemv");
    for (const char* f : {"gu_ring_g1", "gu_ring_g2", "gu_ring_g1_n", "gu_ring_g2_n", "dn_ring_d1", "dn_ring_d2", "dn_ring_d4", "dn_ring_d8"})
        k.push_back(std::string("hh_q4k_") + f);
    for (int w : {1, 2, 4, 8}) k.push_back("hh_q6k_dn_ring_d" + std::to_string(w));
    for (const char* f : {"iq2", "iq3"}) {
        for (int w : {1, 2, 4, 8}) k.push_back(std::string("hh_") + f + "_dn_ring_d" + std::to_string(w));
        for (int w : {1, 2})
            for (const char* n : {"", "_n"}) k.push_back(std::string("hh_") + f + "_gu_ring_g" + std::to_string(w) + n);
        for (const char* n : {"", "_n"}) k.push_back(std::string("hh_") + f + "w_gu_ring_g1" + n);
    }
    for (int w : {1, 2, 4}) k.push_back("hh_iq2w_dn_ring_d" + std::to_string(w));
    for (const char* f : {"gu_ring_u16", "gu_ring_u32", "gu_ring_u64", "dn_ring_d1", "dn_ring_d2", "dn_ring_d4",
                          "dn_ring_d8"})
        k.push_back(std::string("hh_moe_") + f);
    k.push_back("hh_moe_route");
    for (const char* fmt : {"q4_0", "q8_0"})
        for (int t1 : {16, 32, 64})
            for (int t2 : {16, 32, 64})
                k.push_back(std::string("hh_sffn_") + fmt + "_t" + std::to_string(t1) + "_" + std::to_string(t2));
    for (const char* f : {"hh_moe_prep", "hh_moe_route_prep", "hh_moe_hdigits", "hh_moe_combine", "hh_moe_gu_grp_t16", "hh_moe_gu_grp_t32", "hh_moe_gu_grp_t64",
                          "hh_moe_dn_grp_t16", "hh_moe_dn_grp_t32", "hh_moe_dn_grp_t64"})
        k.push_back(f);
    k.push_back("hh_rmsnorm_kernel");
    k.push_back("hh_x_digits");
    k.push_back("hh_add_kernel");
    for (int t : {16, 32, 64})
        for (const char* kind : {"hh_moe_gateup_t", "hh_moe_down_t"}) k.push_back(std::string(kind) + std::to_string(t));
    return k;
}

hh_status engine_create(int device, hh_engine** out) {
    *out = nullptr;
    int count = 0;
    hipError_t err = hipGetDeviceCount(&count);
    if (err != hipSuccess || count == 0) return fail(HH_ERR_NO_DEVICE, "no HIP device found");
    if (device < 0 || device >= count) return fail(HH_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, count);
    hh_engine* e = new hh_engine();
    e->device = device;
    auto bail = [&](hh_status st) {
        if (e->grid_sync) (void)hipFree(e->grid_sync);
        if (e->stream) (void)hipStreamDestroy(e->stream);
        if (e->copy_stream) (void)hipStreamDestroy(e->copy_stream);
    if (e->copy_stream2) (void)hipStreamDestroy(e->copy_stream2);
        if (e->module) (void)hipModuleUnload(e->module);
        delete e;
        return st;
    };
    if (hh_status st = e->select(); st != HH_OK) return bail(st);
    err = hipGetDeviceProperties(&e->props, device);
    if (err != hipSuccess) return bail(hip_fail(err, "hipGetDeviceProperties"));
    if (strncmp(e->props.gcnArchName, "gfx950", 6) != 0)
        return bail(fail(HH_ERR_UNSUPPORTED_DEVICE, "device %d is %s; this build targets gfx950 (MI355X) only",
                         device, e->props.gcnArchName));
    const char* path = getenv("HAYAI_HIP_CODE_OBJECT");
    if (path && *path)
        err = hipModuleLoad(&e->module, path);
    else
        err = hipModuleLoadData(&e->module, hh_kernels_blob);
    if (err != hipSuccess) return bail(hip_fail(err, "hipModuleLoad(gfx950 code object)"));
    err = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
    if (err != hipSuccess) return bail(hip_fail(err, "hipStreamCreate(compute)"));
    err = hipStreamCreateWithFlags(&e->copy_stream, hipStreamNonBlocking);
    if (err != hipSuccess) return bail(hip_fail(err, "hipStreamCreate(copy)"));
    err = hipStreamCreateWithFlags(&e->copy_stream2, hipStreamNonBlocking);
    if (err != hipSuccess) return bail(hip_fail(err, "hipStreamCreate(copy 2)"));
    for (const std::string& k : required_kernels()) {
        hipFunction_t f;
        if (hh_status st = e->kernel(k, &f); st != HH_OK) return bail(st);
    }
    {
        // the no-allocation entry point's scratch array: its address on this device, once
        void* p = nullptr;
        if (noalloc_scratch(device, &p) == HH_OK)
            e->noalloc_ws = p;
        else
            e->noalloc_error = last_error();
    }
    if (const char* b = getenv("HAYAI_HIP_BLOCKS_PER_CU")) e->blocks_per_cu_override = atoi(b);
    if (const char* g = getenv("HAYAI_HIP_Q4K_GENERIC")) e->q4k_generic = atoi(g) != 0;
    if (const char* f = getenv("HAYAI_HIP_RING")) e->ring = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_MOE_GROUPED")) e->moe_grouped = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_SMALL_FFN")) e->small_ffn = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_SMALL_STACK")) e->small_stack = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_STACK_GRID")) e->stack_grid = atoi(f);
    if (const char* f = getenv("HAYAI_HIP_MMQ")) e->mmq = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_DMA_SPLIT")) e->dma_split = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_RING_GU_PER_CU")) e->ring_gu_per_cu = std::max(1, atoi(f));
    if (const char* f = getenv("HAYAI_HIP_RING_DN_PER_CU")) e->ring_dn_per_cu = std::max(1, atoi(f));
    if (const char* f = getenv("HAYAI_HIP_MMR")) e->mmr = atoi(f) != 0;
    if (const char* f = getenv("HAYAI_HIP_MMI_MIN")) e->mmi_min = (size_t)std::max(2, atoi(f));
    if (const char* f = getenv("HAYAI_HIP_MMI_D")) e->mmi_d = atoi(f);
    err = hipMalloc(&e->grid_sync, kBarBytes);
    if (err == hipSuccess) err = hipMemset(e->grid_sync, 0, kBarBytes);
    if (err != hipSuccess) return bail(hip_fail(err, "hipMalloc(grid_sync)"));

    *out = e;
    return HH_OK;
}

void engine_destroy(hh_engine* e) {
    if (!e) return;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    if (e->copy_stream) (void)hipStreamSynchronize(e->copy_stream);
    if (e->copy_stream2) (void)hipStreamSynchronize(e->copy_stream2);
    for (void* p : {e->ws_x, e->ws_y, e->ws_h, e->ws_g, e->ws_u, e->ws_w, e->ws_hq, e->ws_xop, e->ws_hop, e->ws_part,
                    e->ws_cnt, e->ws_moe_h, e->ws_moe_ids, e->ws_moe_w, e->ws_moe_hx, e->ws_xn, e->ws_f, e->ws_xq, e->ws_moe_yp, e->ws_moe_grp, e->ws_moe_q, e->ws_stk, e->grid_sync})
        if (p) (void)hipFree(p);
    for (void* p : e->ws_retired) (void)hipFree(p);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    if (e->copy_stream) (void)hipStreamDestroy(e->copy_stream);
    if (e->copy_stream2) (void)hipStreamDestroy(e->copy_stream2);
    if (e->module) (void)hipModuleUnload(e->module);
    delete e;
}
