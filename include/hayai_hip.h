/*
 * hayai_hip.h -- C ABI of the MI355X (gfx950) FFN GEMV engine.
 *
 * This is the drop-in boundary for Hayai's FFN hot path.  Every entry point replaces a
 * method of the reference's OpenCL device runtime (crates/hayai-opencl) or the FFN seam
 * in crates/hayai-core that calls it; the comment on each declaration names the reference
 * interface (file:line, paths relative to the reference repository root).  Plain C types
 * only: pointers, sizes, integers.  A Rust `hayai-hip` crate binds this header with an
 * `extern "C"` block that declares these functions and mirrors the structs field by field.
 *
 * Conventions
 *   - Every function returns hh_status (0 = HH_OK).  On failure a message is stored in a
 *     thread-local buffer that hh_last_error() returns (valid until the next failing call
 *     on the same thread).
 *   - Weights are unmodified GGUF bytes in a device buffer, addressed by byte offset
 *     (the reference's GgmlWeightBind::Device + weight_off, compute.rs:21-27,388-461).
 *     GEMV shape: y[m] = W[m x n] . x[n], W row-major with GGUF blocks along n
 *     (crates/hayai-model/src/quant.rs:28-29).
 *   - Shapes are validated before any launch exactly as compute.rs:877-949 does
 *     (m, n > 0; n a multiple of the format's block; weight bytes >= m * row_bytes).
 *   - A format with no kernel is a hard HH_ERR_KERNEL_MISSING, never a CPU fallback
 *     (orchestrator.rs:72-98,403-409).  There is no CPU compute path in this library.
 *   - An engine is externally synchronised (one compute stream + one copy stream), like
 *     the reference's orchestrator behind a Mutex (orchestrator.rs:65-68).
 *   - Functions with host x/y pointers block until y is written (the reference's
 *     blocking enqueue_read_buffer).  Functions suffixed _dev take device buffers for
 *     activations too and only enqueue on the engine's compute stream.
 */
#ifndef HAYAI_HIP_H
#define HAYAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HH_ABI_VERSION 1

/* Status codes.  OpenClError::{NoDeviceFound, ClError, UnsupportedPlatformVersion}
 * (crates/hayai-opencl/src/context.rs:13-21) map to NO_DEVICE, RUNTIME and
 * UNSUPPORTED_DEVICE; shape/size rejections (compute.rs:912-949) to INVALID. */
typedef enum hh_status {
    HH_OK = 0,
    HH_ERR_NO_DEVICE = 1,
    HH_ERR_INVALID = 2,
    HH_ERR_KERNEL_MISSING = 3,
    HH_ERR_RUNTIME = 4,
    HH_ERR_OUT_OF_MEMORY = 5,
    HH_ERR_UNSUPPORTED_DEVICE = 6,
    HH_ERR_IO = 7,        /* file could not be opened or read (GgufError::Io / short file) */
    HH_ERR_NOT_FOUND = 8  /* no such tensor or metadata key (GgufError::MissingTensor) */
} hh_status;

/* GGML type ids (crates/hayai-model/src/gguf_types.rs:6-78) with a kernel here. */
enum {
    HH_TYPE_F32 = 0,
    HH_TYPE_F16 = 1,
    HH_TYPE_Q4_0 = 2,
    HH_TYPE_Q8_0 = 8,
    HH_TYPE_Q4_K = 12,
    HH_TYPE_Q6_K = 14,
    HH_TYPE_IQ2_XXS = 16,
    HH_TYPE_IQ3_XXS = 18
};

/* FFN activation: SiLU(gate)*up (stream_infer.rs:3836-3840) or tanh-GELU(gate)*up
 * (ffn_finish_gelu_scratch, stream_infer.rs:3889-3895). */
enum { HH_ACT_SILU = 0, HH_ACT_GELU_TANH = 1 };

/* Buffer kinds: device HBM, or pinned host memory from hipHostMalloc (replaces the
 * CL_MEM_ALLOC_HOST_PTR / SVM host slots of crates/hayai-opencl/src/memory.rs:72-147). */
enum { HH_BUF_DEVICE = 0, HH_BUF_PINNED_HOST = 1 };

typedef struct hh_engine hh_engine;   /* OpenClEngine, context.rs:23-69 */
typedef struct hh_buf hh_buf;         /* cl_mem Buffer<u8> / PinnedHostBuffer */
typedef struct hh_pending hh_pending; /* PendingGemv, async_gemv.rs:15-57 */
typedef struct hh_event hh_event;     /* timing event on the compute stream */

typedef struct hh_device_info {
    char name[256];       /* marketing name */
    char arch[64];        /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int device_index;
    int compute_units;
    int wavefront_size;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;
    size_t total_mem;
    size_t lds_per_block;
    size_t l2_bytes;
} hh_device_info;

/* ------------------------------------------------------------------ errors / info --- */

int hh_abi_version(void);
const char* hh_last_error(void);
/* Name of a status code ("HH_ERR_INVALID", ...). */
const char* hh_status_name(hh_status st);

/* Packed bytes per row of n columns (compute.rs:877-907, gemv_row_bytes).
 * HH_ERR_INVALID when n is not a block multiple; HH_ERR_KERNEL_MISSING for a type
 * with no kernel here. */
hh_status hh_row_bytes(int ggml_type, size_t n, size_t* out);

/* Pre-launch validation, callable without a device (compute.rs:912-949):
 * validate_gemv_shape and validate_gemv_weights. */
hh_status hh_validate_gemv_shape(int ggml_type, size_t m, size_t n);
hh_status hh_validate_gemv_weights(int ggml_type, size_t m, size_t n, size_t weights_len);

/* ------------------------------------------------------------------ engine ---------- */

/* Number of HIP devices (discover_opencl_devices, crates/hayai-opencl/src/device.rs:86-184). */
hh_status hh_device_count(int* count);

/* Bring up one device: select it, load the gfx950 code object (embedded in this library,
 * or the file named by HAYAI_HIP_CODE_OBJECT) with hipModuleLoadData/hipModuleLoad,
 * resolve every kernel, create the compute and copy streams.  Fails with
 * HH_ERR_UNSUPPORTED_DEVICE on a non-gfx950 device and HH_ERR_KERNEL_MISSING if a kernel
 * is absent from the code object.  Replaces OpenClEngine::init_device
 * (crates/hayai-opencl/src/context.rs:106-232). */
hh_status hh_engine_create(int device, hh_engine** out);
void hh_engine_destroy(hh_engine* e);
hh_status hh_engine_info(const hh_engine* e, hh_device_info* out);
/* Wait for all work on both engine streams. */
hh_status hh_engine_sync(hh_engine* e);
/* Count of FFN GEMVs dispatched (the ffn_calls counter, context.rs:64-65). */
uint64_t hh_engine_ffn_calls(const hh_engine* e);

/* ------------------------------------------------------------------ buffers --------- */

/* Allocate a device (HH_BUF_DEVICE) or pinned host (HH_BUF_PINNED_HOST) buffer.
 * Buffer::create (compute.rs) / PinnedHostBuffer::new (memory.rs:72-147). */
hh_status hh_buf_alloc(hh_engine* e, size_t bytes, int kind, hh_buf** out);
void hh_buf_free(hh_buf* b);
size_t hh_buf_size(const hh_buf* b);
int hh_buf_kind(const hh_buf* b);
/* Host address of a pinned buffer (NULL for device buffers). */
void* hh_buf_host_ptr(hh_buf* b);
/* Blocking host <-> buffer copies (enqueue_write_buffer / enqueue_read_buffer with
 * CL_BLOCKING).  Ordered after all work already queued on the compute stream. */
hh_status hh_buf_write(hh_engine* e, hh_buf* dst, size_t dst_off, const void* src, size_t bytes);
hh_status hh_buf_read(hh_engine* e, const hh_buf* src, size_t src_off, void* dst, size_t bytes);
/* Buffer-to-buffer copy (device or pinned), enqueued on the compute stream. */
hh_status hh_buf_copy(hh_engine* e, hh_buf* dst, size_t dst_off, const hh_buf* src, size_t src_off, size_t bytes);
/* Device fill with a byte value (enqueued on the compute stream). */
hh_status hh_buf_fill(hh_engine* e, hh_buf* dst, size_t off, uint8_t value, size_t bytes);

/* ------------------------------------------------------------------ GEMV ------------ */

/* ggml_gemv_dispatch (crates/hayai-opencl/src/compute.rs:281-383): host weights are
 * uploaded into a persistent engine workspace, then GEMV, then blocking readback. */
hh_status hh_gemv(hh_engine* e, int ggml_type, size_t m, size_t n, const uint8_t* weights,
                  size_t weights_len, const float* x, float* y);

/* ggml_gemv_dispatch_bound (compute.rs:388-461): weights resident in a device buffer at
 * byte offset w_off; x uploaded, y read back (blocking). */
hh_status hh_gemv_bound(hh_engine* e, int ggml_type, size_t m, size_t n, const hh_buf* w,
                        size_t w_off, const float* x, float* y);

/* ggml_gemv_async_from_device (crates/hayai-opencl/src/async_gemv.rs:90-196): enqueue
 * and return a pending handle that owns its activation buffers. */
hh_status hh_gemv_begin(hh_engine* e, int ggml_type, size_t m, size_t n, const hh_buf* w,
                        size_t w_off, const float* x, hh_pending** out);
/* PendingGemv::wait (async_gemv.rs:27-46): block, copy the m outputs into y. */
hh_status hh_pending_wait(hh_pending* p, float* y, size_t m);
/* Drop for PendingGemv (async_gemv.rs:48-57): waits for the kernel, then frees. */
void hh_pending_destroy(hh_pending* p);

/* ggml_gemv_batched_q4_k (crates/hayai-opencl/src/compute.rs:179-257) generalised to every
 * type, as execute_quant_gemv_batched does (crates/hayai-core/src/orchestrator.rs:240-269):
 * outputs[b*m + r] = W[r] . inputs[b*n .. b*n+n) for b < batch.  Host weights and
 * activations, blocking.  Q4_K with batch >= 2 runs on the matrix cores in passes of up to
 * 64 tokens; other types loop over tokens.  Precision of the Q4_K passes:
 *   - passes of 2..16 tokens: f32 activations (as f16 hi + lo pairs), f32 accumulation:
 *     within ~1e-6 of the f32 product;
 *   - passes of 17..64 tokens: each token's activations are first quantized to int8 per
 *     32-element block (s = max|x| / 127, q = round-half-away(x / s), clamped to +-127)
 *     and multiplied exactly (integer products with the weights' sc * q on the matrix
 *     cores); the
 *     result differs from the f32 product by that quantization: measured 0.7-1.9% of
 *     max|y| per token on N(0,1) activations (the tests bound it at 4%).
 * Set HAYAI_HIP_MMQ=0 in the environment before creating the engine to keep f32
 * activations for every batch size (17..64 tokens then run one token at a time);
 * HAYAI_HIP_MMI_MIN=16 moves passes of 16 tokens onto the int8 form. */
hh_status hh_gemv_batched(hh_engine* e, int ggml_type, size_t m, size_t n, const uint8_t* weights,
                          size_t weights_len, const float* inputs, float* outputs, size_t batch);
/* Same with device buffers (weights at w_off; x: batch*n floats, y: batch*m floats);
 * enqueue only. */
hh_status hh_gemv_batched_dev(hh_engine* e, int ggml_type, size_t m, size_t n, const hh_buf* w, size_t w_off,
                              const hh_buf* x, size_t x_off, size_t batch, hh_buf* y, size_t y_off);

/* Device-resident GEMV: x and y are device buffers (byte offsets), enqueue only. */
hh_status hh_gemv_dev(hh_engine* e, int ggml_type, size_t m, size_t n, const hh_buf* w,
                      size_t w_off, const hh_buf* x, size_t x_off, hh_buf* y, size_t y_off);

/* Q4 LUT MatMul, Hayai's own 4-bit dictionary format: weights_q4 holds m rows of n/2
 * bytes (low nibble = even column, high nibble = odd column), each nibble an index into
 * the 16-entry f32 `lut`; y[r] = sum_c x[2c]*lut[lo] + x[2c+1]*lut[hi].
 * OpenClEngine::lut_matmul_q4 (crates/hayai-opencl/src/compute.rs:45-128), kernel
 * lut_matmul_q4_v1 (crates/hayai-kernels/kernels/lut_matmul.cl:14-54), CPU twin
 * cpu_lut_matmul_q4 (crates/hayai-cpu/src/matmul.rs:48-82).  The reference's assertions
 * (n even, weights_q4.len() == m*n/2) become HH_ERR_INVALID.  Host arrays, blocking. */
hh_status hh_lut_gemv(hh_engine* e, size_t m, size_t n, const uint8_t* weights_q4, size_t weights_len,
                      const float* lut, const float* x, float* y);
/* Same with device buffers (lut: 16 floats at lut_off; f32 offsets 4-byte aligned);
 * enqueue only. */
hh_status hh_lut_gemv_dev(hh_engine* e, size_t m, size_t n, const hh_buf* w, size_t w_off, const hh_buf* lut,
                          size_t lut_off, const hh_buf* x, size_t x_off, hh_buf* y, size_t y_off);

/* Dequant probe: n weights of a packed tensor at (w, w_off) -> f32 at (out, out_off),
 * bit-identical to hayai-model's dequant (gguf.rs:348-372, q4k.rs:162-203,
 * iq2.rs:504-523, iq3.rs:147-173; F16: gguf.rs:521-545).  Enqueue only. */
hh_status hh_dequant_dev(hh_engine* e, int ggml_type, const hh_buf* w, size_t w_off, size_t n,
                         hh_buf* out, size_t out_off);

/* ------------------------------------------------------------------ FFN ------------- */

/* One FFN op of a layer pack: gate/up/down descriptors with byte offsets into the pack
 * (LayerPackLayout gate_off/up_off/down_off, crates/hayai-model/src/gguf_stream.rs:1416-1444;
 * QuantMatrix nrows/ncols/ggml_type, quant.rs:31-54). */
typedef struct hh_ffn_desc {
    int type_gate;
    int type_up;
    int type_down;
    int act; /* HH_ACT_* */
    size_t d_model;
    size_t d_ff;
    size_t gate_off;
    size_t up_off;
    size_t down_off;
} hh_ffn_desc;

/* ffn_begin_gate_up_scratch + ffn_finish_scratch (crates/hayai-core/src/stream_infer.rs:
 * 3752-3864) as one call: y = W_down . (act(W_gate . x) * (W_up . x)).  Gate/up and the
 * activation run as one fused kernel when gate and up share a format, then down.
 * Host x / y, blocking. */
hh_status hh_ffn(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                 const float* x, float* y);
/* Same with device activations (x: d_model floats, y: d_model floats); enqueue only.
 * The d_ff intermediate lives in an engine workspace. */
hh_status hh_ffn_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                     const hh_buf* x, size_t x_off, hh_buf* y, size_t y_off);

/* No counterpart in the reference.  For callers that cannot allocate device memory at call
 * time (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * hh_ffn_dev with the d_ff intermediate in a fixed per-GPU scratch array of
 * HH_NOALLOC_SCRATCH_BYTES (held by each GPU the library runs on until the process ends)
 * instead of the engine's growable workspaces; it calls no hipMalloc/hipFree.  Same kernels
 * and results as hh_ffn_dev's two-launch forms (the ring kernels for Q4_K and Q4_K_M layers,
 * gate/up + down otherwise).  Limits: d_ff <= HH_NOALLOC_MAX_D_FF, and for layouts other
 * than Q4_K / Q4_K_M 12 * d_ff + 2.5 * min(max(d_model, d_ff), 32768) bytes must fit the
 * array; HH_ERR_INVALID otherwise.  All calls on one GPU share the array: calls that overlap
 * on one GPU (two engines, or two threads) race.  Enqueue only. */
#define HH_NOALLOC_SCRATCH_BYTES (512u * 1024u)
#define HH_NOALLOC_MAX_D_FF 32768u
hh_status hh_ffn_dev_noalloc(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                             const hh_buf* x, size_t x_off, hh_buf* y, size_t y_off);

/* The FFN residual block of one token (ffn_apply, crates/hayai-core/src/hybrid_infer.rs:
 * 883-936): y = x + FFN(RMSNorm(x)), RMSNorm as rms_norm (crates/hayai-cpu/src/attention.rs:
 * 142-147): x * (1 / sqrt(mean(x^2) + eps)) * norm.  norm: d_model floats; y may be x (the
 * reference updates x in place).  All-Q4_K and Q4_K_M layers fuse the norm into gate/up and
 * the residual into down; other layouts run norm, FFN and add as separate kernels.
 * Device buffers, enqueue only. */
hh_status hh_ffn_block_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                           const hh_buf* norm, size_t norm_off, float eps, const hh_buf* x, size_t x_off, hh_buf* y,
                           size_t y_off);

/* n_layers FFN residual blocks of one token back to back: x_{l+1} = x_l + FFN_l(RMSNorm(x_l)
 * with norm_l), y = x_{n_layers}; layer l's pack at pack_off + l * layer_stride bytes, its
 * norm at norm_off + l * norm_stride * 4 bytes (norm_stride in floats; 0 reuses one vector).
 * y may be x.  No counterpart in the reference: its decode loop calls ffn_apply
 * (hybrid_infer.rs:883-936) once per layer with attention between.  This entry point is for
 * callers that run FFN blocks with no other op between them (FFN-only layer stacks, the
 * chained-layer benchmark): small all-Q4_0 / all-Q8_0 layers (d_model, d_ff <= 2048) run
 * every layer in one persistent launch that requests each layer's weights ahead of the
 * activation exchanges; other layouts run hh_ffn_block_dev per layer.  Results match
 * hh_ffn_block_dev applied layer by layer to f32 rounding (sums in another order).
 * HH_ERR_INVALID for n_layers 0 or ranges outside the buffers.  Enqueue only. */
hh_status hh_ffn_block_stack_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                                 size_t layer_stride, size_t n_layers, const hh_buf* norm, size_t norm_off,
                                 size_t norm_stride, float eps, const hh_buf* x, size_t x_off, hh_buf* y,
                                 size_t y_off);

/* The FFN op for `batch` tokens (x, y: batch rows of d_model floats): the batched-prefill
 * form of the op (prefill_wave.rs:577-584 drives execute_quant_gemv_batched for FFN
 * matrices).  All-Q4_K FFNs run gate/up(+act) and down on the matrix cores with the
 * precision hh_gemv_batched states: passes of 17..64 tokens quantize x, and then h, to
 * int8 per 32-element block, which moves the FFN output by 3-13% of max|y| per token on
 * N(0,1) inputs (h is heavy-tailed; the tests bound it at 25%); passes of 2..16 tokens stay
 * within 1e-3 of the f32 FFN (h enters down as f16).  Other formats run the single-token op
 * per token.  _dev: device buffers, enqueue only; without: host x / y, blocking. */
hh_status hh_ffn_batched_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                             const hh_buf* x, size_t x_off, size_t batch, hh_buf* y, size_t y_off);
hh_status hh_ffn_batched(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                         const float* x, float* y, size_t batch);

/* hh_ffn_dev as the reference's two calls (the same kernels hh_ffn_dev runs in its
 * two-launch form).  hh_ffn_begin_dev: ffn_begin_gate_up_scratch (stream_infer.rs:3752-3808)
 * -- gate/up and the activation into the engine's FFN intermediate.  hh_ffn_finish_dev:
 * ffn_finish_scratch (stream_infer.rs:3809-3864) -- the down projection of the
 * intermediate left by the last begin of the same FFN shape; HH_ERR_INVALID when none is
 * pending (a finish consumes it).  Enqueue only. */
hh_status hh_ffn_begin_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                           const hh_buf* x, size_t x_off);
hh_status hh_ffn_finish_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, hh_buf* y,
                            size_t y_off);

/* hh_ffn_block_dev as the reference's ffn_apply runs it (crates/hayai-core/src/
 * hybrid_infer.rs:883-938): hh_ffn_block_begin_dev = rms_norm(x, norm, eps) (:895-896)
 * followed by ffn_begin_gate_up_scratch (:906-918); hh_ffn_block_finish_dev =
 * ffn_finish_scratch (:919-930) followed by the residual add x[i] += ws_down[i] (:933-935),
 * here y = res + down (y may be res).  Same kernels as hh_ffn_block_dev; the same pending
 * rule as hh_ffn_begin_dev / hh_ffn_finish_dev.  Enqueue only. */
hh_status hh_ffn_block_begin_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                                 const hh_buf* norm, size_t norm_off, float eps, const hh_buf* x, size_t x_off);
hh_status hh_ffn_block_finish_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                                  const hh_buf* res, size_t res_off, hh_buf* y, size_t y_off);

/* The first half of the FFN op: ffn_begin_gate_up_scratch (stream_infer.rs:3752-3806)
 * fused with the activation of ffn_finish_scratch (:3836-3840):
 * h[d_ff] = act(W_gate . x) * (W_up . x), one kernel when gate and up share a format.
 * Enqueue only; x holds d_model floats, h receives d_ff floats. */
hh_status hh_gateup_dev(hh_engine* e, int type_gate, int type_up, size_t d_ff, size_t d_model, const hh_buf* wg,
                        size_t wg_off, const hh_buf* wu, size_t wu_off, const hh_buf* x, size_t x_off, hh_buf* h,
                        size_t h_off, int act);

/* ------------------------------------------------------------------ MoE ------------- */

/* The routed experts of one MoE layer: MoeMeta (crates/hayai-core/src/exec_plan.rs:244-271)
 * plus the resident expert layout of moe_infer.rs:330-339 (expert e's pack at
 * e * expert_stride; its gate/up/down tensors at fixed offsets inside the pack). */
typedef struct hh_moe_desc {
    int type;             /* GGML type of every expert tensor; the MoE kernels take HH_TYPE_Q4_K */
    int act;              /* HH_ACT_* */
    size_t d_model;       /* expert input and output width */
    size_t d_ff;          /* expert intermediate width */
    size_t n_experts;     /* expert_count, 1..512 */
    size_t top_k;         /* experts per token, 1..64 */
    size_t expert_stride; /* bytes between consecutive expert packs (multiple of 16) */
    size_t gate_off, up_off, down_off;
    size_t n_group;       /* grouped routing: number of groups (0 = off, <= 64) */
    size_t topk_group;    /* groups kept */
    int gating;           /* 0 softmax over all experts, 1 sigmoid */
    int norm_topk_prob;   /* renormalise the top_k weights */
    float routed_scaling_factor;
    /* Shared expert (DeepSeek-style, moe_infer.rs:456-493): always active with weight 1 and
     * added after the routed experts, y[t] += down_s(act(gate_s . x[t]) * (up_s . x[t])),
     * its tensors (of `type`, shared_d_ff wide) at these byte offsets from experts_off.
     * shared_d_ff 0: no shared expert (shared_*_off unused). */
    size_t shared_d_ff;
    size_t shared_gate_off, shared_up_off, shared_down_off;
} hh_moe_desc;

/* route_experts + top_k_indices (crates/hayai-core/src/moe_infer.rs:852-934) for T tokens:
 * logits [T][n_experts] f32 (+ optional e_score_correction_bias [n_experts], NULL for none)
 * -> ids [T][top_k] int32 and weights [T][top_k] f32.  Ids are exactly the reference's; the
 * weights use the device expf (within a few ulp of libm).  Slots past the number selected
 * (fewer candidates than top_k) hold id -1 and weight 0.  _dev: device buffers, enqueue
 * only; without: host arrays, blocking. */
hh_status hh_route_experts_dev(hh_engine* e, const hh_moe_desc* d, const hh_buf* logits, size_t logits_off,
                               const hh_buf* bias, size_t bias_off, size_t T, hh_buf* ids, size_t ids_off,
                               hh_buf* weights, size_t weights_off);
hh_status hh_route_experts(hh_engine* e, const hh_moe_desc* d, const float* logits, const float* bias, size_t T,
                           int32_t* ids, float* weights);

/* The routed-expert FFN and combine of moe_infer.rs:342-455 for T tokens:
 * y[t] = sum_s weights[t][s] * down_e(act(gate_e x[t]) * up_e x[t]), e = ids[t][s], in slot
 * order, then the shared expert's output (when the descriptor has one, :456-493).  Ids
 * outside [0, n_experts) (the -1 of an empty slot) contribute nothing.  Experts live in one
 * device buffer at experts_off.  Enqueue only. */
hh_status hh_moe_ffn_dev(hh_engine* e, const hh_moe_desc* d, const hh_buf* experts, size_t experts_off,
                         const hh_buf* x, size_t x_off, size_t T, const hh_buf* ids, size_t ids_off,
                         const hh_buf* weights, size_t weights_off, hh_buf* y, size_t y_off);

/* Routing and the expert FFN in one call (ids and weights stay in engine workspaces). */
hh_status hh_moe_dev(hh_engine* e, const hh_moe_desc* d, const hh_buf* experts, size_t experts_off,
                     const hh_buf* logits, size_t logits_off, const hh_buf* bias, size_t bias_off,
                     const hh_buf* x, size_t x_off, size_t T, hh_buf* y, size_t y_off);

/* ------------------------------------------------------------------ streaming ------- */

/* Pinned-host ping-pong weight streaming: StreamingScratch
 * (crates/hayai-opencl/src/hetero_scratch.rs:48-71) with PinnedHostBuffer host slots
 * (crates/hayai-opencl/src/memory.rs:72-147) and a device mirror per slot.  n_slots slots
 * (at least 2 = classic ping-pong) of block_k * layer_bytes; layer L lives in slot
 * (L / block_k) % n_slots at offset (L % block_k) * layer_bytes (slot_for / weight_offset,
 * hetero_scratch.rs:565-571,915-925).  DMAs run on the engine's copy stream with
 * hipMemcpyAsync; the FFN kernels read the mirror on the compute stream; events order the
 * two, so DMA of layer L+1 overlaps the FFN of layer L. */
typedef struct hh_streamer hh_streamer;

/* StreamingScratch::allocate_for_pool (hetero_scratch.rs:87-236), pinned-host path:
 * block_k 0 is taken as 1 and n_slots below 2 as 2, as the reference does. */
hh_status hh_streamer_create(hh_engine* e, size_t layer_bytes, size_t block_k, size_t n_slots, hh_streamer** out);
/* Waits for both engine streams, then frees slots, mirrors and events. */
void hh_streamer_destroy(hh_streamer* s);
/* slot_for (hetero_scratch.rs:565-571). */
hh_status hh_streamer_slot_for(const hh_streamer* s, size_t layer, size_t* slot);
/* weight_offset (hetero_scratch.rs:915-925): byte offset of a tensor of `layer` inside the
 * mirror that hh_streamer_bind returns. */
hh_status hh_streamer_weight_offset(const hh_streamer* s, size_t layer, size_t tensor_off, size_t* off);
/* prepare_host_write + host_slot (hetero_scratch.rs:611-656): the pinned host address of
 * `layer`'s region (layer_bytes writable bytes), after any DMA still reading that slot has
 * completed. */
hh_status hh_streamer_host_slot(hh_streamer* s, size_t layer, void** host_ptr);
/* dma_ffn_keep_mapped / dma_ffn_slices_mapped (hetero_scratch.rs:678-849): enqueue the copy
 * of bytes [off, off+len) of `layer`'s host region into its mirror on the copy stream.  The
 * copy first waits for all work already enqueued on the compute stream (the FFN of the layer
 * that held the slot before).  Marks the slot as staged for `layer`'s block. */
hh_status hh_streamer_dma(hh_streamer* s, size_t layer, size_t off, size_t len);
/* weight_bind (hetero_scratch.rs:853-908): the device mirror holding `layer` (owned by the
 * streamer; never pass it to hh_buf_free) and the layer's byte offset in it; the compute
 * stream waits for the slot's last DMA, so FFN calls enqueued after this read the new bytes.
 * HH_ERR_INVALID when the slot's last DMA was for another block. */
hh_status hh_streamer_bind(hh_streamer* s, size_t layer, hh_buf** mirror, size_t* layer_off);

/* ------------------------------------------------------------------ timing ---------- */

hh_status hh_event_create(hh_engine* e, hh_event** out);
void hh_event_destroy(hh_event* ev);
/* Record on the engine's compute stream (the stream every kernel here runs on). */
hh_status hh_event_record(hh_engine* e, hh_event* ev);
hh_status hh_event_elapsed_ms(hh_event* start, hh_event* stop, float* ms);

/* ------------------------------------------------------------------ graphs ---------- */

/* No counterpart in the reference (its OpenCL queue replays nothing): capture a fixed
 * sequence of enqueue-only (*_dev) calls on the engine's compute stream into a HIP graph and
 * replay it, for decode loops whose launches are the same every token (one graph launch
 * instead of one dispatch per kernel).  Between hh_graph_begin and hh_graph_end only *_dev
 * calls may be made, and none may need a larger workspace than an earlier call did (run the
 * sequence once eagerly first); calls whose kernels carry per-launch state (the persistent
 * one-launch FFN form, batched and MoE FFNs) are refused or routed to graph-safe kernels.
 * A replay reads and writes the buffers the captured calls named, with their contents at
 * replay time. */
typedef struct hh_graph hh_graph;
hh_status hh_graph_begin(hh_engine* e);
/* Ends the capture (also after a refused call) and instantiates the graph. */
hh_status hh_graph_end(hh_engine* e, hh_graph** out);
/* Enqueue one replay on the engine's compute stream. */
hh_status hh_graph_launch(hh_graph* g);
void hh_graph_destroy(hh_graph* g);

/* ------------------------------------------------------------------ synthetic data -- */

/* Fill n_blocks GGUF blocks of ggml_type at (dst, off) with the seeded synthetic stream
 * (splitmix64 bytes, then every f16 scale field drawn U(lo, hi) and rounded to nearest
 * even).  Enqueue only.  The byte recipe is specified in hayai_amd/synth.py, which
 * generates the same bytes on the host.  Benchmark harness input, the analogue of the
 * reference's bench_* helpers (async_gemv.rs:309-428). */
hh_status hh_synth_weights_dev(hh_engine* e, int ggml_type, hh_buf* dst, size_t off, size_t n_blocks,
                               uint64_t seed, float lo, float hi);

/* ------------------------------------------------------------------ GGUF catalog ------
 * The model file side of the path: GgufCatalog's header parse (crates/hayai-model/src/
 * gguf.rs:25-127, gguf_stream.rs:34-192) and load_layer_pack_into (gguf_stream.rs:451-638),
 * reading through io_uring in one batch per layer (weight_io.rs:14-105,351-470; positioned
 * reads when io_uring is refused or HAYAI_FORCE_FILE_IO=1).  Host memory only: the
 * destination is typically a pinned streaming slot (hh_streamer_host_slot).  Malformed
 * files are HH_ERR_INVALID (bad magic or version, more than 4 dims, a zero dim, duplicate
 * names, unknown types, alignment not a power of two, size overflow), unreadable or short
 * ones HH_ERR_IO, missing tensors and keys HH_ERR_NOT_FOUND. */
typedef struct hh_gguf hh_gguf;

typedef struct hh_gguf_info {
    uint32_t version;      /* 1..4 */
    uint32_t io_uring;     /* 1: reads go through io_uring */
    uint32_t o_direct;     /* 1: reads bypass the page cache (HAYAI_O_DIRECT set, O_DIRECT open
                            * accepted, no fallback to page-cache reads yet) */
    uint32_t pad;
    uint64_t alignment;    /* general.alignment (default 32) */
    uint64_t data_offset;  /* absolute offset of the tensor data section */
    uint64_t header_bytes; /* bytes of header + directory */
    uint64_t n_tensors;
    uint64_t n_metadata;
    uint64_t file_size;
} hh_gguf_info;

typedef struct hh_gguf_tensor {
    const char* name;     /* owned by the catalog until hh_gguf_close */
    uint32_t n_dims;
    uint32_t type;        /* GGML type id */
    uint64_t dims[4];     /* ne0 (columns) first; unused dims are 1 */
    uint64_t offset;      /* relative to the data section */
    uint64_t abs_offset;  /* data_offset + offset */
    uint64_t nbytes;      /* tensor_nbytes (gguf.rs:240-284) */
} hh_gguf_tensor;

/* LayerPackLayout (gguf_stream.rs:1416-1432) plus each region's matrix shape and type.
 * Slots: 0 attn_q, 1 attn_k, 2 attn_v, 3 attn_output, 4 ffn_gate, 5 ffn_up, 6 ffn_down,
 * 7 attn_gate.  Regions are back to back in slot order (no padding); an absent optional
 * tensor (attn_v, ffn_gate, attn_gate) has length 0. */
typedef struct hh_layer_pack {
    size_t off[8];
    size_t len[8];
    uint32_t type[8];
    uint64_t cols[8];
    uint64_t rows[8];
    size_t total;
    int32_t fused_gate_up; /* gate and up are the two row halves of one fused tensor */
    int32_t pad;
} hh_layer_pack;

hh_status hh_gguf_open(const char* path, hh_gguf** out);
void hh_gguf_close(hh_gguf* g);
hh_status hh_gguf_header(const hh_gguf* g, hh_gguf_info* out);
hh_status hh_gguf_tensor_at(const hh_gguf* g, uint64_t index, hh_gguf_tensor* out);
/* GgufCatalog::tensor (gguf.rs:176-182) */
hh_status hh_gguf_find(const hh_gguf* g, const char* name, hh_gguf_tensor* out);
/* meta_u32 / as_u64 / meta_f32 / meta_str (gguf.rs:160-174, gguf_types.rs:100-135) */
hh_status hh_gguf_meta_u32(const hh_gguf* g, const char* key, uint32_t* out);
hh_status hh_gguf_meta_u64(const hh_gguf* g, const char* key, uint64_t* out);
hh_status hh_gguf_meta_f32(const hh_gguf* g, const char* key, float* out);
hh_status hh_gguf_meta_str(const hh_gguf* g, const char* key, const char** out, size_t* len);
/* tensor_nbytes (gguf.rs:240-284) for a type and shape */
hh_status hh_tensor_nbytes(uint32_t type, const uint64_t* dims, uint32_t n_dims, uint64_t* out);
/* The layout load_layer_pack_into would produce for `layer`, without reading. */
hh_status hh_gguf_layer_pack(const hh_gguf* g, size_t layer, hh_layer_pack* out);
/* load_layer_pack_into: the layer's tensors into dst[0, total), one batch of reads. */
hh_status hh_gguf_load_layer_pack(hh_gguf* g, size_t layer, void* dst, size_t dst_len, hh_layer_pack* out);
/* read_tensor_into (gguf_stream.rs:266-290): one whole tensor into dst. */
hh_status hh_gguf_read_tensor(hh_gguf* g, const char* name, void* dst, size_t dst_len);

#ifdef __cplusplus
}
#endif

#endif /* HAYAI_HIP_H */
