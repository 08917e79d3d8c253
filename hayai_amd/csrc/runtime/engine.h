// Internal C++ runtime of the HIP FFN engine (not part of the ABI).
//
// Engine is the MI355X counterpart of the reference's OpenClEngine
// (crates/hayai-opencl/src/context.rs:23-69): one device, its loaded gfx950 code object,
// a compute stream and a copy stream, and persistent activation workspaces that grow on
// demand (GemvSyncWorkspace, compute.rs:8-17).
#ifndef HH_RUNTIME_ENGINE_H
#define HH_RUNTIME_ENGINE_H

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/hayai_hip.h"
#include "../kargs.h"

namespace hh {

// Thread-local last error.
hh_status fail(hh_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
const std::string& last_error();
hh_status hip_fail(hipError_t err, const char* what);

#define HH_TRY_HIP(call, what)                        \
    do {                                              \
        hipError_t _e = (call);                       \
        if (_e != hipSuccess) return hh::hip_fail(_e, what); \
    } while (0)

#define HH_TRY(call)                  \
    do {                              \
        hh_status _s = (call);        \
        if (_s != HH_OK) return _s;   \
    } while (0)

// Block geometry of a GGML format with a kernel here (compute.rs:877-907).
struct Format {
    int type;
    const char* name;   // kernel-name stem
    uint32_t block;     // elements per block
    uint32_t bytes;     // bytes per block
    uint32_t unit;      // columns per lane unit of the team kernels
    bool fused_gateup;  // has a fused gate/up kernel
};
const Format* format_of(int ggml_type);
hh_status row_bytes(int ggml_type, size_t n, size_t* out);
hh_status validate_shape(int ggml_type, size_t m, size_t n);
hh_status validate_weights(int ggml_type, size_t m, size_t n, size_t len);

// Bytes of the ring kernels' digit form of an n-element activation (q1[n] | q2[n] | one
// f32 scale per 8 elements, + 16 bytes of slack for the kernels' vector tail).
inline size_t ring_digits_bytes(size_t n) { return 2 * n + (n / 8) * 4 + 16; }

// The device address of noalloc.hip's fixed scratch array on `device` (which must be the
// current device): looked up once per device and kept.
hh_status noalloc_scratch(int device, void** out);

// Team configurations instantiated in gemv.hip, in selection order.
struct TeamCfg {
    int team;
    int upl;
};
extern const TeamCfg kTeamCfgs[];
extern const int kNumTeamCfgs;

}  // namespace hh

struct hh_buf {
    hh_engine* engine;
    void* ptr;  // device pointer, or pinned host pointer (also device-accessible)
    size_t size;
    int kind;
};

struct hh_event {
    hipEvent_t ev;
    int device;
};

struct hh_engine {
    int device = 0;
    hipDeviceProp_t props{};
    hipModule_t module = nullptr;
    hipStream_t stream = nullptr;       // compute stream (default priority)
    hipStream_t copy_stream = nullptr;  // side stream for host<->device DMA
    hipStream_t copy_stream2 = nullptr; // second DMA stream: large streamer copies split in two
    bool dma_split = true;              // HAYAI_HIP_DMA_SPLIT=0: one copy stream per DMA
    std::unordered_map<std::string, hipFunction_t> fns;
    std::unordered_map<std::string, int> blocks_per_cu;  // occupancy per kernel
    std::atomic<uint64_t> ffn_calls{0};
    std::mutex ws_mutex;  // guards the workspaces below (the reference's sync_ws Mutex)
    // Growable device workspaces: x / y for host-activation calls, the FFN intermediate,
    // separate gate/up outputs for the unfused path, staged host weights for hh_gemv.
    void* ws_x = nullptr;
    size_t ws_x_cap = 0;
    void* ws_y = nullptr;
    size_t ws_y_cap = 0;
    void* ws_h = nullptr;
    size_t ws_h_cap = 0;
    void* ws_g = nullptr;
    size_t ws_g_cap = 0;
    void* ws_u = nullptr;
    size_t ws_u_cap = 0;
    void* ws_w = nullptr;
    size_t ws_w_cap = 0;
    void* ws_hq = nullptr;  // int8 digits of the FFN intermediate (gate/up -> down)
    size_t ws_hq_cap = 0;
    void* ws_xn = nullptr;  // FFN block (generic formats): RMSNorm(x), then the FFN output
    size_t ws_xn_cap = 0;
    void* ws_f = nullptr;
    size_t ws_f_cap = 0;
    void* ws_xq = nullptr;  // GEMV activations as ring digits (Q6_K ring GEMV)
    size_t ws_xq_cap = 0;
    // Batched (MFMA) path: tokens as MFMA operand stages (f16 hi/lo pairs + 16-element
    // sums), the FFN intermediate in the same form, split-K partials and their per-row-group
    // arrival counters.
    void* ws_xop = nullptr;
    size_t ws_xop_cap = 0;
    void* ws_hop = nullptr;
    size_t ws_hop_cap = 0;
    void* ws_part = nullptr;
    size_t ws_part_cap = 0;
    void* ws_cnt = nullptr;  // zeroed when allocated; every launch leaves it zero
    size_t ws_cnt_cap = 0;
    // MoE: expert intermediates [T][k][d_ff], ids and weights of hh_moe_dev.
    void* ws_moe_h = nullptr;
    size_t ws_moe_h_cap = 0;
    void* ws_moe_hx = nullptr;  // digits of the weighted expert intermediate (one-token MoE)
    size_t ws_moe_hx_cap = 0;
    void* ws_moe_ids = nullptr;
    size_t ws_moe_ids_cap = 0;
    void* ws_moe_w = nullptr;
    size_t ws_moe_w_cap = 0;
    void* ws_moe_yp = nullptr;   // grouped MoE: per-pair down outputs [T*k][d_model]
    size_t ws_moe_yp_cap = 0;
    void* ws_moe_grp = nullptr;  // grouped MoE: the active experts' records, the pairs grouped by expert
    size_t ws_moe_grp_cap = 0;
    void* ws_moe_q = nullptr;    // grouped MoE: x digits per token, h digits per pair
    size_t ws_moe_q_cap = 0;
    void* ws_stk = nullptr;     // FFN-stack exchange: tagged words of h (d_ff) then x (d_model); zeroed
    size_t ws_stk_cap = 0;      // when allocated and after a device error
    void* grid_sync = nullptr;  // grid-barrier state (counters, flags, error word, epochs)
    hh_ffn_desc ffn_stage{};    // FFN whose gate/up output is pending in ws_h (/ws_hq)
    bool ffn_stage_valid = false;
    bool ffn_stage_digits = false;  // ws_hq holds the digits of ws_h
    bool ffn_stage_ring = false;    // ws_hq holds the ring kernels' granule digits of h
    bool ring = true;           // HAYAI_HIP_RING=0: skip the two-launch ring Q4_K FFN
    bool moe_grouped = true;    // HAYAI_HIP_MOE_GROUPED=0: several-token MoE per (token, expert)
    bool small_ffn = true;      // HAYAI_HIP_SMALL_FFN=0: small Q4_0/Q8_0 FFNs as two launches
    int ring_gu_per_cu = 1;     // HAYAI_HIP_RING_GU_PER_CU: ring gate/up workgroups per CU
    int ring_dn_per_cu = 1;     // HAYAI_HIP_RING_DN_PER_CU: ring down workgroups per CU
    bool mmr = true;            // HAYAI_HIP_MMR=0: batched Q4_K (<= 16 tokens) one token at a time
    bool mmq = true;            // HAYAI_HIP_MMQ=0: batched Q4_K (>= 17 tokens) one token at a time, no int8
    size_t mmi_min = 17;        // HAYAI_HIP_MMI_MIN: fewest tokens per pass on the int8 kernels (>= 2)
    int mmi_d = 0;              // HAYAI_HIP_MMI_D: ring depth of the int8 f16-MFMA kernels (0: chosen)
    int blocks_per_cu_override = 0;  // HAYAI_HIP_BLOCKS_PER_CU
    bool q4k_generic = false;        // HAYAI_HIP_Q4K_GENERIC=1: skip the int8-digit Q4_K kernels

    hh_status select();  // hipSetDevice(device)
    // Between hh_graph_begin and hh_graph_end the compute stream is being captured into a
    // HIP graph: nothing may allocate, synchronize, or bake per-launch state into a kernel.
    bool capturing = false;
    // Instantiated graphs of this engine still alive.  Their kernels hold workspace
    // addresses, so while any exists a workspace that grows keeps its old allocation here
    // (freed when the last graph is destroyed, or with the engine) instead of freeing it.
    int live_graphs = 0;
    std::vector<void*> ws_retired;
    void free_retired();
    hh_status no_capture(const char* what) const;
    // hh_ffn_dev_noalloc: this device's fixed scratch array (noalloc.hip), resolved when the
    // engine is created; null when that failed (the reason in noalloc_error).
    void* noalloc_ws = nullptr;
    std::string noalloc_error;
    hh_status enqueue_ffn_noalloc(const hh_ffn_desc* d, const uint8_t* pack, const float* x, float* y);
    hh_status kernel(const std::string& name, hipFunction_t* out);
    int resident_blocks(const std::string& name, int block);
    template <class A>
    hh_status launch(hipFunction_t f, uint32_t grid, uint32_t block, const A& args) {
        void* params[] = {const_cast<A*>(&args)};
        hipError_t err = hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, stream, params, nullptr);
        if (err != hipSuccess) return hh::hip_fail(err, "hipModuleLaunchKernel");
        return HH_OK;
    }
    hh_status grow(void** p, size_t* cap, size_t need);

    // Enqueue one GEMV y = W . x on the compute stream (all pointers device-visible).
    // xq_ws: room for a Q6_K GEMV's x digits (hh_ring_digits_bytes(n)); null: ws_xq.
    hh_status enqueue_gemv(int type, size_t m, size_t n, const uint8_t* w, const float* x, float* y,
                           void* xq_ws = nullptr);
    // Enqueue the fused or unfused gate/up + activation into h.
    // gu_ws: room for the unfused form's gate and up outputs (2 * d_ff floats, then the
    // GEMVs' x digits); null: ws_g / ws_u (/ ws_xq).
    hh_status enqueue_gateup(int type_g, int type_u, size_t d_ff, size_t d_model, const uint8_t* wg,
                             const uint8_t* wu, const float* x, float* h, int act, float* gu_ws = nullptr);
    hh_status enqueue_ffn(const hh_ffn_desc* d, const uint8_t* pack, const float* x, float* y);
    hh_status enqueue_small_ffn(const hh_ffn_desc* d, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                                const float* x, float* y);
    hh_status enqueue_ffn_block(const hh_ffn_desc* d, const uint8_t* pack, const float* x, const float* norm,
                                float eps, float* y);
    // n_layers consecutive FFN residual blocks (layer l's pack at pack + l * stride, its norm
    // at norm + l * norm_stride floats); y = x_L, y may be x.  Small Q4_0 / Q8_0 layers run
    // in one persistent launch (small_stack.hip), others as one block per layer.
    hh_status enqueue_ffn_block_stack(const hh_ffn_desc* d, const uint8_t* pack, size_t stride, size_t n_layers,
                                      const float* norm, size_t norm_stride, float eps, const float* x, float* y);
    hh_status enqueue_small_stack(const hh_ffn_desc* d, const uint8_t* pack, size_t stride, size_t n_layers,
                                  const float* norm, size_t norm_stride, float eps, const float* x, float* y);
    bool small_stack = true;  // HAYAI_HIP_SMALL_STACK=0: FFN stacks as one block per layer
    int stack_grid = 0;       // HAYAI_HIP_STACK_GRID: workgroups of the persistent stack (0: one per CU)
    // The two halves of enqueue_ffn's two-launch path: gate/up(+act) into the engine's FFN
    // intermediate, then the down projection of that intermediate.
    // With norm: the begin step of the FFN residual block (x is RMSNorm'ed first); with res:
    // the finish step adds the residual (y = res + down; y may be res).
    hh_status enqueue_ffn_begin(const hh_ffn_desc* d, const uint8_t* pack, const float* x,
                                const float* norm = nullptr, float eps = 0.f);
    hh_status enqueue_ffn_finish(const hh_ffn_desc* d, const uint8_t* pack, float* y, const float* res = nullptr);
    // Q4_K batch-1 kernels (q4k.hip); returns HH_ERR_UNSUPPORTED_DEVICE when the shape or
    // alignment needs the generic kernels instead (the caller then falls back).  xdigits:
    // x given as int8 digits (then x is unused); hdigits: gate/up also writes h's digits.
    hh_status enqueue_q4k(size_t m, size_t n, const uint8_t* w0, const uint8_t* w1, const float* x, float* y,
                          int act, bool gateup, const void* xdigits, void* hdigits);
    bool ring_ok(const hh_ffn_desc* d, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd, const float* x) const;
    // Ring gate/up (Q4_K, IQ2_XXS, IQ3_XXS); hx: where h's digits go
    // (hh_ring_digits_bytes(d_ff)); null: ws_hq.
    hh_status enqueue_ring_gu(const hh_ffn_desc* d, const uint8_t* wg, const uint8_t* wu, const float* x,
                              const float* norm = nullptr, float eps = 0.f, uint8_t* hx = nullptr);
    hh_status enqueue_ring_dn(const hh_ffn_desc* d, const uint8_t* wd, float* y, const float* res = nullptr);
    // Ring down kernel of GGML type `type` (Q4_K, Q6_K, IQ2_XXS, IQ3_XXS) over digits hx.
    hh_status launch_dn_ring(int type, size_t m, size_t n, const uint8_t* w, const uint8_t* hx, float* y,
                             const float* res);
    hh_status enqueue_ring_gemv(int type, size_t m, size_t n, const uint8_t* w, const float* x, float* y,
                                void* xq_ws = nullptr);
    // Batched GEMV Y[b][m] = W . X[b] (x, y device pointers, row-major by token).  Q4_K with
    // 2 <= batch uses the MFMA kernels in chunks of up to 64 tokens; other formats (and
    // batch 1) run one GEMV per token, as the reference's orchestrator does
    // (orchestrator.rs:258-260).
    hh_status enqueue_gemv_batched(int type, size_t m, size_t n, const uint8_t* w, const float* x, size_t batch,
                                   float* y);
    // Batched FFN: per token y[b] = FFN(x[b]); all-Q4_K FFNs run gate/up and down on MFMA.
    hh_status enqueue_ffn_batched(const hh_ffn_desc* d, const uint8_t* pack, const float* x, size_t batch, float* y);
    // Tokens [b][n] f32 -> operand stages in ws_xop for 16 * tt token slots.
    hh_status enqueue_mm_prep(const float* x, size_t b, size_t n, size_t tt);
    // Weight-stream MFMA launch for 1..16 tokens (q4k_mmr.hip).  kind: MMR_GEMM (w0, f32 x,
    // y), MMR_GU (w0 = gate, w1 = up, f32 x, act; h stages into ws_hop) or MMR_DN (w0, x =
    // token stages, y).  HH_ERR_UNSUPPORTED_DEVICE when shape or alignment does not fit.
    enum { MMR_GEMM = 0, MMR_GU = 1, MMR_DN = 2 };
    bool mmr_ok(size_t m, size_t n, size_t b, const void* w0, const void* w1, const void* x) const;
    // batched Q4_K with int8 activations (q4k_mmi.hip) applies: 17..64 tokens (HAYAI_HIP_MMI_MIN
    // lowers the bound), shapes of whole superblocks, 16-byte aligned pointers
    bool mmq_ok(size_t m, size_t n, size_t b, const void* w0, const void* w1, const void* x) const;
    // int8 activations on the f16 matrix cores (q4k_mmi.hip): tokens [b][n] f32 -> stages
    // (9216 bytes per superblock and 16-token tile), then GEMM (y) or FFN gate/up (h stages)
    hh_status enqueue_mmi_prep(const float* x, size_t b, size_t n, size_t tt, void* xs);
    // tiles: 16-token tiles of the stages (0: from b)
    hh_status enqueue_q4k_mmi(bool ffn, size_t m, size_t n, const uint8_t* w0, const uint8_t* w1, const void* xs,
                              size_t b, float* y, void* hs, int act, size_t tiles = 0);
    hh_status enqueue_q4k_mmr(int kind, size_t m, size_t n, const uint8_t* w0, const uint8_t* w1, const void* x,
                              size_t b, float* y, int act);
    // MoE routing of T tokens (device pointers) and the grouped expert FFN.
    hh_status enqueue_moe_route(const hh_moe_desc* d, const float* logits, const float* bias, size_t T,
                                int32_t* ids, float* wts);
    // With logits, the gate/up kernel routes each token first and writes ids / wts itself.
    hh_status enqueue_moe_ffn(const hh_moe_desc* d, const uint8_t* experts, const float* x, size_t T,
                              int32_t* ids, float* wts, float* y, const float* logits = nullptr,
                              const float* bias = nullptr);
    // The shared expert of an MoE layer (moe_infer.rs:456-493), after the routed experts:
    // y[t] += FFN_shared(x[t]).  Nothing when the descriptor has none.
    hh_status enqueue_moe_shared(const hh_moe_desc* d, const uint8_t* experts, const float* x, size_t T, float* y);
    // Q4 LUT GEMV (hayai's 4-bit dictionary format): W m rows of n/2 bytes, lut 16 f32.
    hh_status enqueue_lut(size_t m, size_t n, const uint8_t* w, const float* lut, const float* x, float* y);
    // Reports (and clears) a grid-barrier timeout recorded by a fused kernel.  Syncs.
    hh_status check_device_error();
};

#endif
