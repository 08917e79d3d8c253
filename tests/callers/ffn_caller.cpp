// A C++ caller of the C ABI (include/hayai_hip.h) that replays the reference's own call
// sequences for the FFN of a streamed decode, as its Rust code would drive a hayai-hip
// crate.  Test infrastructure: run by tests/test_gpu_callers.py on a GPU; it links the
// CPU oracle only to check results.
//
// Per layer, following crates/hayai-core/src/stream_infer.rs:
//   prefetch (:1665-1722): keep n_slots - 1 layers staged ahead: prepare_host_write +
//     host_slot (hh_streamer_host_slot), fill the layer pack, dma_ffn_slices_mapped (one
//     hh_streamer_dma per FFN region);
//   ffn_begin_gate_up_scratch (:3752-3808), ffn_finish_scratch (:3809-3864) in the three
//   forms the reference and its replacement take:
//     A. sync_gemv_from_scratch: ggml_gemv_dispatch_bound of gate and up on the bound
//        mirror (hh_gemv_bound), SiLU * up on the host, the same for down;
//     B. begin_gemv_from_scratch + PendingGemv::wait (hh_gemv_begin, hh_pending_wait,
//        hh_pending_destroy), SiLU on the host, down the same way;
//     C. the fused replacement seam: hh_ffn_begin_dev + hh_ffn_finish_dev on the mirror.
// A and B run the same GEMV kernels: bit-identical.  All three are checked against the
// oracle FFN (max |y - ref| / max |ref| <= 1e-3).  Then the error contract: a finish with
// nothing pending, a kernel-less type, binding an unstaged layer.
//
// usage: hh_ffn_caller <ggml_type> <d_model> <d_ff> <layers>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "hayai_hip.h"

extern "C" int or_ffn(int tg, int tu, int td, size_t d_model, size_t d_ff, const uint8_t* wg, size_t lg,
                      const uint8_t* wu, size_t lu, const uint8_t* wd, size_t ld, int act, const float* x, float* y,
                      float* h_out);
extern "C" void or_set_threads(int n);

static int g_fail = 0;

#define CHECK(call)                                                                                   \
    do {                                                                                              \
        hh_status _s = (call);                                                                        \
        if (_s != HH_OK) {                                                                            \
            fprintf(stderr, "[caller] %s failed: %s (%s)\n", #call, hh_status_name(_s), hh_last_error()); \
            exit(2);                                                                                  \
        }                                                                                             \
    } while (0)

static void expect(bool ok, const char* what) {
    printf("[caller] %-58s %s\n", what, ok ? "ok" : "FAILED");
    fflush(stdout);
    if (!ok) g_fail = 1;
}

static float rel_err(const std::vector<float>& y, const std::vector<float>& r) {
    float num = 0.f, den = 0.f;
    for (size_t i = 0; i < y.size(); i++) {
        num = std::fmax(num, std::fabs(y[i] - r[i]));
        den = std::fmax(den, std::fabs(r[i]));
    }
    return den > 0.f ? num / den : num;
}

static void silu_mul(std::vector<float>& g, const std::vector<float>& u) {
    for (size_t i = 0; i < g.size(); i++) g[i] = (g[i] / (1.0f + std::exp(-g[i]))) * u[i];
}

int main(int argc, char** argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s <ggml_type> <d_model> <d_ff> <layers>\n", argv[0]);
        return 2;
    }
    const int t = atoi(argv[1]);
    const size_t dm = strtoul(argv[2], nullptr, 10), df = strtoul(argv[3], nullptr, 10);
    const size_t L = strtoul(argv[4], nullptr, 10);
    or_set_threads(8);
    hh_engine* e = nullptr;
    CHECK(hh_engine_create(0, &e));
    size_t rg = 0, rd = 0;
    CHECK(hh_row_bytes(t, dm, &rg));
    CHECK(hh_row_bytes(t, df, &rd));
    // LayerPackLayout of an FFN-only pack: gate, up, down back to back, 256-byte aligned
    auto up256 = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t gate_off = 0, up_off = up256(df * rg), down_off = up_off + up256(df * rg);
    const size_t total = down_off + up256(dm * rd);
    const hh_ffn_desc desc{t, t, t, HH_ACT_SILU, dm, df, gate_off, up_off, down_off};

    // the model image on the host (the bytes a GGUF layer pack would hold), made on the
    // device by the seeded generator and read back
    const size_t blk = (t == HH_TYPE_Q4_0 || t == HH_TYPE_Q8_0) ? 32 : 256;
    std::vector<std::vector<uint8_t>> image(L, std::vector<uint8_t>(total, 0));
    {
        hh_buf* tmp = nullptr;
        CHECK(hh_buf_alloc(e, total, HH_BUF_DEVICE, &tmp));
        for (size_t l = 0; l < L; l++) {
            CHECK(hh_buf_fill(e, tmp, 0, 0, total));
            CHECK(hh_synth_weights_dev(e, t, tmp, gate_off, df * dm / blk, 1000 + 3 * l, 1e-3f, 1e-2f));
            CHECK(hh_synth_weights_dev(e, t, tmp, up_off, df * dm / blk, 1001 + 3 * l, 1e-3f, 1e-2f));
            CHECK(hh_synth_weights_dev(e, t, tmp, down_off, dm * df / blk, 1002 + 3 * l, 1e-3f, 1e-2f));
            CHECK(hh_buf_read(e, tmp, 0, image[l].data(), total));
        }
        hh_buf_free(tmp);
    }
    std::vector<std::vector<float>> xs(L, std::vector<float>(dm));
    uint64_t z = 0x243F6A8885A308D3ull;
    for (auto& x : xs)
        for (float& v : x) {  // uniform(-1, 1) from splitmix64
            z += 0x9E3779B97F4A7C15ull;
            uint64_t q = z;
            q = (q ^ (q >> 30)) * 0xBF58476D1CE4E5B9ull;
            q = (q ^ (q >> 27)) * 0x94D049BB133111EBull;
            q ^= q >> 31;
            v = (float)((double)(q >> 11) * 0x1.0p-53 * 2.0 - 1.0);
        }

    const size_t n_slots = 2;
    hh_streamer* st = nullptr;
    CHECK(hh_streamer_create(e, total, 1, n_slots, &st));
    hh_buf *xb = nullptr, *yb = nullptr;
    CHECK(hh_buf_alloc(e, dm * 4, HH_BUF_DEVICE, &xb));
    CHECK(hh_buf_alloc(e, dm * 4, HH_BUF_DEVICE, &yb));

    auto stage = [&](size_t l) {
        void* host = nullptr;
        CHECK(hh_streamer_host_slot(st, l, &host));  // waits for the DMA still reading the slot
        memcpy(host, image[l].data(), total);
        CHECK(hh_streamer_dma(st, l, gate_off, df * rg));
        CHECK(hh_streamer_dma(st, l, up_off, df * rg));
        CHECK(hh_streamer_dma(st, l, down_off, dm * rd));
    };
    size_t next = 0;
    float worst = 0.f;
    bool ab_equal = true;
    for (size_t l = 0; l < L; l++) {
        while (next < L && next < l + n_slots - 1 + 1) stage(next++);  // n_slots - 1 ahead
        hh_buf* mirror = nullptr;
        size_t off = 0;
        CHECK(hh_streamer_bind(st, l, &mirror, &off));
        size_t woff = 0;
        CHECK(hh_streamer_weight_offset(st, l, 0, &woff));
        if (woff != off) expect(false, "weight_offset agrees with bind");
        std::vector<float> ref(dm);
        or_ffn(t, t, t, dm, df, image[l].data() + gate_off, df * rg, image[l].data() + up_off, df * rg,
               image[l].data() + down_off, dm * rd, HH_ACT_SILU, xs[l].data(), ref.data(), nullptr);
        // A: sync_gemv_from_scratch (ggml_gemv_dispatch_bound) for gate, up, down
        std::vector<float> g(df), u(df), ya(dm), yb_(dm), yc(dm);
        CHECK(hh_gemv_bound(e, t, df, dm, mirror, off + gate_off, xs[l].data(), g.data()));
        CHECK(hh_gemv_bound(e, t, df, dm, mirror, off + up_off, xs[l].data(), u.data()));
        silu_mul(g, u);
        CHECK(hh_gemv_bound(e, t, dm, df, mirror, off + down_off, g.data(), ya.data()));
        // B: begin_gemv_from_scratch + PendingGemv::wait
        hh_pending *pg = nullptr, *pu = nullptr, *pd = nullptr;
        CHECK(hh_gemv_begin(e, t, df, dm, mirror, off + gate_off, xs[l].data(), &pg));
        CHECK(hh_gemv_begin(e, t, df, dm, mirror, off + up_off, xs[l].data(), &pu));
        CHECK(hh_pending_wait(pg, g.data(), df));
        CHECK(hh_pending_wait(pu, u.data(), df));
        hh_pending_destroy(pg);
        hh_pending_destroy(pu);
        silu_mul(g, u);
        CHECK(hh_gemv_begin(e, t, dm, df, mirror, off + down_off, g.data(), &pd));
        CHECK(hh_pending_wait(pd, yb_.data(), dm));
        hh_pending_destroy(pd);
        // C: the fused seam on the same mirror
        CHECK(hh_buf_write(e, xb, 0, xs[l].data(), dm * 4));
        CHECK(hh_ffn_begin_dev(e, &desc, mirror, off, xb, 0));
        CHECK(hh_ffn_finish_dev(e, &desc, mirror, off, yb, 0));
        CHECK(hh_buf_read(e, yb, 0, yc.data(), dm * 4));
        ab_equal = ab_equal && memcmp(ya.data(), yb_.data(), dm * 4) == 0;
        const float ea = rel_err(ya, ref), eb = rel_err(yb_, ref), ec = rel_err(yc, ref);
        printf("[caller] layer %zu rel_err bound %.3e async %.3e fused %.3e\n", l, ea, eb, ec);
        worst = std::fmax(worst, std::fmax(ea, std::fmax(eb, ec)));
    }
    expect(ab_equal, "bound and async GEMV paths bit-identical");
    expect(worst <= 1e-3f, "every path within 1e-3 of the oracle FFN");
    expect(hh_engine_ffn_calls(e) >= 9 * L, "ffn_calls counted every FFN GEMV");

    // the error contract (compute.rs:877-949; orchestrator.rs:403-409; hetero_scratch.rs:853-908)
    {
        hh_buf* mirror = nullptr;
        size_t off = 0;
        CHECK(hh_streamer_bind(st, L - 1, &mirror, &off));
        expect(hh_ffn_finish_dev(e, &desc, mirror, off, yb, 0) == HH_ERR_INVALID,
               "finish with no gate/up pending -> HH_ERR_INVALID");
        std::vector<float> x(256), y(4);
        std::vector<uint8_t> w(1024);
        expect(hh_gemv(e, 3, 4, 256, w.data(), w.size(), x.data(), y.data()) == HH_ERR_KERNEL_MISSING,
               "GEMV of a type with no kernel -> HH_ERR_KERNEL_MISSING");
        expect(hh_gemv(e, HH_TYPE_Q4_0, 4, 250, w.data(), w.size(), x.data(), y.data()) == HH_ERR_INVALID,
               "n not a block multiple -> HH_ERR_INVALID");
        expect(hh_streamer_bind(st, L + 5, &mirror, &off) == HH_ERR_INVALID, "bind of an unstaged layer -> HH_ERR_INVALID");
    }
    CHECK(hh_engine_sync(e));
    hh_buf_free(xb);
    hh_buf_free(yb);
    hh_streamer_destroy(st);
    hh_engine_destroy(e);
    printf("[caller] %s\n", g_fail ? "FAILED" : "all ok");
    return g_fail;
}
