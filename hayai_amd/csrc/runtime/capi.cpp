// extern "C" surface declared in include/hayai_hip.h.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

#include "engine.h"

namespace hh {
const std::string& last_error();
}
hh_status engine_create(int device, hh_engine** out);
void engine_destroy(hh_engine* e);

using namespace hh;

#define HH_NOT_NULL(p, what) \
    if (!(p)) return fail(HH_ERR_INVALID, "%s is NULL", what)

// [off, off + bytes) must lie inside the buffer.
static hh_status check_range(const hh_buf* b, size_t off, size_t bytes, const char* what) {
    if (!b) return fail(HH_ERR_INVALID, "%s: buffer is NULL", what);
    if (off > b->size || bytes > b->size - off)
        return fail(HH_ERR_INVALID, "%s: range [%zu, +%zu) outside a %zu-byte buffer", what, off, bytes, b->size);
    return HH_OK;
}

static hh_status check_engine(hh_engine* e, const hh_buf* b, const char* what) {
    if (b && b->engine != e) return fail(HH_ERR_INVALID, "%s: buffer belongs to another engine", what);
    return HH_OK;
}

struct hh_pending {
    hh_engine* engine;
    void* dx;
    void* dy;
    size_t m;
    hipEvent_t done;
    bool waited;
};

extern "C" {

int hh_abi_version(void) { return HH_ABI_VERSION; }

const char* hh_last_error(void) { return last_error().c_str(); }

const char* hh_status_name(hh_status st) {
    switch (st) {
    case HH_OK: return "HH_OK";
    case HH_ERR_NO_DEVICE: return "HH_ERR_NO_DEVICE";
    case HH_ERR_INVALID: return "HH_ERR_INVALID";
    case HH_ERR_KERNEL_MISSING: return "HH_ERR_KERNEL_MISSING";
    case HH_ERR_RUNTIME: return "HH_ERR_RUNTIME";
    case HH_ERR_OUT_OF_MEMORY: return "HH_ERR_OUT_OF_MEMORY";
    case HH_ERR_UNSUPPORTED_DEVICE: return "HH_ERR_UNSUPPORTED_DEVICE";
    case HH_ERR_IO: return "HH_ERR_IO";
    case HH_ERR_NOT_FOUND: return "HH_ERR_NOT_FOUND";
    }
    return "HH_ERR_UNKNOWN";
}

hh_status hh_row_bytes(int t, size_t n, size_t* out) {
    HH_NOT_NULL(out, "out");
    return row_bytes(t, n, out);
}

hh_status hh_validate_gemv_shape(int t, size_t m, size_t n) { return validate_shape(t, m, n); }

hh_status hh_validate_gemv_weights(int t, size_t m, size_t n, size_t len) { return validate_weights(t, m, n, len); }

hh_status hh_device_count(int* count) {
    HH_NOT_NULL(count, "count");
    *count = 0;
    hipError_t err = hipGetDeviceCount(count);
    if (err == hipErrorNoDevice) {
        *count = 0;
        return HH_OK;
    }
    if (err != hipSuccess) return hip_fail(err, "hipGetDeviceCount");
    return HH_OK;
}

hh_status hh_engine_create(int device, hh_engine** out) {
    HH_NOT_NULL(out, "out");
    try {
        return engine_create(device, out);
    } catch (const std::bad_alloc&) {
        return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
}

void hh_engine_destroy(hh_engine* e) { engine_destroy(e); }

hh_status hh_engine_info(const hh_engine* e, hh_device_info* out) {
    HH_NOT_NULL(e, "engine");
    HH_NOT_NULL(out, "out");
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s", e->props.name);
    snprintf(out->arch, sizeof out->arch, "%s", e->props.gcnArchName);
    out->device_index = e->device;
    out->compute_units = e->props.multiProcessorCount;
    out->wavefront_size = e->props.warpSize;
    out->clock_khz = e->props.clockRate;
    out->memory_clock_khz = e->props.memoryClockRate;
    out->memory_bus_width = e->props.memoryBusWidth;
    out->total_mem = e->props.totalGlobalMem;
    out->lds_per_block = e->props.sharedMemPerBlock;
    out->l2_bytes = (size_t)e->props.l2CacheSize;
    return HH_OK;
}

hh_status hh_engine_sync(hh_engine* e) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->select());
    HH_TRY_HIP(hipStreamSynchronize(e->stream), "hipStreamSynchronize(compute)");
    HH_TRY_HIP(hipStreamSynchronize(e->copy_stream), "hipStreamSynchronize(copy)");
    return e->check_device_error();
}

uint64_t hh_engine_ffn_calls(const hh_engine* e) { return e ? e->ffn_calls.load() : 0; }

// ---------------------------------------------------------------- buffers ------------

hh_status hh_buf_alloc(hh_engine* e, size_t bytes, int kind, hh_buf** out) {
    HH_NOT_NULL(e, "engine");
    HH_NOT_NULL(out, "out");
    *out = nullptr;
    if (kind != HH_BUF_DEVICE && kind != HH_BUF_PINNED_HOST) return fail(HH_ERR_INVALID, "unknown buffer kind %d", kind);
    HH_TRY(e->select());
    void* p = nullptr;
    const size_t sz = std::max<size_t>(bytes, 1);
    if (kind == HH_BUF_DEVICE) {
        HH_TRY_HIP(hipMalloc(&p, sz), "hipMalloc");
    } else {
        HH_TRY_HIP(hipHostMalloc(&p, sz, hipHostMallocDefault), "hipHostMalloc");
    }
    hh_buf* b = new (std::nothrow) hh_buf{e, p, bytes, kind};
    if (!b) {
        if (kind == HH_BUF_DEVICE)
            (void)hipFree(p);
        else
            (void)hipHostFree(p);
        return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    *out = b;
    return HH_OK;
}

void hh_buf_free(hh_buf* b) {
    if (!b) return;
    (void)hipSetDevice(b->engine->device);
    // Work queued on the engine may still read the buffer.
    (void)hipStreamSynchronize(b->engine->stream);
    (void)hipStreamSynchronize(b->engine->copy_stream);
    if (b->kind == HH_BUF_DEVICE)
        (void)hipFree(b->ptr);
    else
        (void)hipHostFree(b->ptr);
    delete b;
}

size_t hh_buf_size(const hh_buf* b) { return b ? b->size : 0; }

int hh_buf_kind(const hh_buf* b) { return b ? b->kind : -1; }

void* hh_buf_host_ptr(hh_buf* b) { return (b && b->kind == HH_BUF_PINNED_HOST) ? b->ptr : nullptr; }

hh_status hh_buf_write(hh_engine* e, hh_buf* dst, size_t off, const void* src, size_t bytes) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("buf_write"));
    HH_TRY(check_engine(e, dst, "hh_buf_write"));
    HH_TRY(check_range(dst, off, bytes, "hh_buf_write"));
    if (bytes == 0) return HH_OK;
    HH_NOT_NULL(src, "src");
    HH_TRY(e->select());
    HH_TRY_HIP(hipMemcpyAsync((char*)dst->ptr + off, src, bytes, hipMemcpyDefault, e->stream), "hipMemcpyAsync(H2D)");
    HH_TRY_HIP(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return HH_OK;
}

hh_status hh_buf_read(hh_engine* e, const hh_buf* src, size_t off, void* dst, size_t bytes) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("buf_read"));
    HH_TRY(check_engine(e, src, "hh_buf_read"));
    HH_TRY(check_range(src, off, bytes, "hh_buf_read"));
    if (bytes == 0) return HH_OK;
    HH_NOT_NULL(dst, "dst");
    HH_TRY(e->select());
    HH_TRY_HIP(hipMemcpyAsync(dst, (const char*)src->ptr + off, bytes, hipMemcpyDefault, e->stream),
               "hipMemcpyAsync(D2H)");
    return e->check_device_error();  // syncs the stream
}

hh_status hh_buf_copy(hh_engine* e, hh_buf* dst, size_t dst_off, const hh_buf* src, size_t src_off, size_t bytes) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("buf_copy"));
    HH_TRY(check_engine(e, dst, "hh_buf_copy"));
    HH_TRY(check_engine(e, src, "hh_buf_copy"));
    HH_TRY(check_range(dst, dst_off, bytes, "hh_buf_copy dst"));
    HH_TRY(check_range(src, src_off, bytes, "hh_buf_copy src"));
    if (bytes == 0) return HH_OK;
    HH_TRY(e->select());
    HH_TRY_HIP(hipMemcpyAsync((char*)dst->ptr + dst_off, (const char*)src->ptr + src_off, bytes, hipMemcpyDefault,
                              e->stream),
               "hipMemcpyAsync(copy)");
    return HH_OK;
}

hh_status hh_buf_fill(hh_engine* e, hh_buf* dst, size_t off, uint8_t value, size_t bytes) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("buf_fill"));
    HH_TRY(check_engine(e, dst, "hh_buf_fill"));
    HH_TRY(check_range(dst, off, bytes, "hh_buf_fill"));
    if (bytes == 0) return HH_OK;
    HH_TRY(e->select());
    HH_TRY_HIP(hipMemsetAsync((char*)dst->ptr + off, value, bytes, e->stream), "hipMemsetAsync");
    return HH_OK;
}

// ---------------------------------------------------------------- GEMV ---------------

hh_status hh_gemv_dev(hh_engine* e, int t, size_t m, size_t n, const hh_buf* w, size_t w_off, const hh_buf* x,
                      size_t x_off, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_shape(t, m, n));
    size_t rb;
    HH_TRY(row_bytes(t, n, &rb));
    HH_TRY(check_engine(e, w, "weights"));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(w, w_off, m * rb, "weights"));
    HH_TRY(check_range(x, x_off, n * sizeof(float), "x"));
    HH_TRY(check_range(y, y_off, m * sizeof(float), "y"));
    HH_TRY(e->select());
    e->ffn_calls++;
    return e->enqueue_gemv(t, m, n, (const uint8_t*)w->ptr + w_off, (const float*)((const char*)x->ptr + x_off),
                           (float*)((char*)y->ptr + y_off));
}

static hh_status gemv_host_io(hh_engine* e, int t, size_t m, size_t n, const uint8_t* wdev, const float* x, float* y) {
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    HH_TRY(e->grow(&e->ws_x, &e->ws_x_cap, n * sizeof(float)));
    HH_TRY(e->grow(&e->ws_y, &e->ws_y_cap, m * sizeof(float)));
    HH_TRY_HIP(hipMemcpyAsync(e->ws_x, x, n * sizeof(float), hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(x)");
    e->ffn_calls++;
    HH_TRY(e->enqueue_gemv(t, m, n, wdev, (const float*)e->ws_x, (float*)e->ws_y));
    HH_TRY_HIP(hipMemcpyAsync(y, e->ws_y, m * sizeof(float), hipMemcpyDeviceToHost, e->stream), "hipMemcpyAsync(y)");
    HH_TRY_HIP(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return HH_OK;
}

hh_status hh_gemv_bound(hh_engine* e, int t, size_t m, size_t n, const hh_buf* w, size_t w_off, const float* x,
                        float* y) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_shape(t, m, n));
    size_t rb;
    HH_TRY(row_bytes(t, n, &rb));
    HH_TRY(check_engine(e, w, "weights"));
    HH_TRY(check_range(w, w_off, m * rb, "weights"));
    HH_NOT_NULL(x, "x");
    HH_NOT_NULL(y, "y");
    HH_TRY(e->select());
    return gemv_host_io(e, t, m, n, (const uint8_t*)w->ptr + w_off, x, y);
}

hh_status hh_gemv(hh_engine* e, int t, size_t m, size_t n, const uint8_t* weights, size_t weights_len,
                  const float* x, float* y) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_shape(t, m, n));
    HH_TRY(validate_weights(t, m, n, weights_len));
    HH_NOT_NULL(weights, "weights");
    HH_NOT_NULL(x, "x");
    HH_NOT_NULL(y, "y");
    size_t rb;
    HH_TRY(row_bytes(t, n, &rb));
    HH_TRY(e->select());
    {
        std::lock_guard<std::mutex> lk(e->ws_mutex);
        HH_TRY(e->grow(&e->ws_w, &e->ws_w_cap, m * rb));
        HH_TRY_HIP(hipMemcpyAsync(e->ws_w, weights, m * rb, hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(w)");
    }
    return gemv_host_io(e, t, m, n, (const uint8_t*)e->ws_w, x, y);
}

static hh_status batch_bytes(size_t batch, size_t len, size_t* out) {
    if (len != 0 && batch > SIZE_MAX / (len * sizeof(float))) return fail(HH_ERR_INVALID, "batch size overflow");
    *out = batch * len * sizeof(float);
    return HH_OK;
}

hh_status hh_gemv_batched(hh_engine* e, int t, size_t m, size_t n, const uint8_t* weights, size_t weights_len,
                          const float* inputs, float* outputs, size_t batch) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_shape(t, m, n));
    HH_TRY(validate_weights(t, m, n, weights_len));
    size_t xb, yb, rb;
    HH_TRY(batch_bytes(batch, n, &xb));
    HH_TRY(batch_bytes(batch, m, &yb));
    HH_TRY(row_bytes(t, n, &rb));
    if (batch == 0) return HH_OK;
    HH_NOT_NULL(weights, "weights");
    HH_NOT_NULL(inputs, "inputs");
    HH_NOT_NULL(outputs, "outputs");
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    HH_TRY(e->grow(&e->ws_w, &e->ws_w_cap, m * rb));
    HH_TRY(e->grow(&e->ws_x, &e->ws_x_cap, xb));
    HH_TRY(e->grow(&e->ws_y, &e->ws_y_cap, yb));
    HH_TRY_HIP(hipMemcpyAsync(e->ws_w, weights, m * rb, hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(w)");
    HH_TRY_HIP(hipMemcpyAsync(e->ws_x, inputs, xb, hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(x)");
    HH_TRY(e->enqueue_gemv_batched(t, m, n, (const uint8_t*)e->ws_w, (const float*)e->ws_x, batch, (float*)e->ws_y));
    HH_TRY_HIP(hipMemcpyAsync(outputs, e->ws_y, yb, hipMemcpyDeviceToHost, e->stream), "hipMemcpyAsync(y)");
    return e->check_device_error();
}

hh_status hh_gemv_batched_dev(hh_engine* e, int t, size_t m, size_t n, const hh_buf* w, size_t w_off, const hh_buf* x,
                              size_t x_off, size_t batch, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("gemv_batched_dev"));
    HH_TRY(validate_shape(t, m, n));
    size_t xb, yb, rb;
    HH_TRY(batch_bytes(batch, n, &xb));
    HH_TRY(batch_bytes(batch, m, &yb));
    HH_TRY(row_bytes(t, n, &rb));
    HH_TRY(check_engine(e, w, "weights"));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(w, w_off, m * rb, "weights"));
    HH_TRY(check_range(x, x_off, xb, "x"));
    HH_TRY(check_range(y, y_off, yb, "y"));
    if (((x_off | y_off) & 3u) != 0) return fail(HH_ERR_INVALID, "gemv_batched: x/y offsets must be 4-byte aligned");
    if (batch == 0) return HH_OK;
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_gemv_batched(t, m, n, (const uint8_t*)w->ptr + w_off, (const float*)((const char*)x->ptr + x_off),
                                   batch, (float*)((char*)y->ptr + y_off));
}

hh_status hh_gemv_begin(hh_engine* e, int t, size_t m, size_t n, const hh_buf* w, size_t w_off, const float* x,
                        hh_pending** out) {
    HH_NOT_NULL(e, "engine");
    HH_NOT_NULL(out, "out");
    *out = nullptr;
    HH_TRY(validate_shape(t, m, n));
    size_t rb;
    HH_TRY(row_bytes(t, n, &rb));
    HH_TRY(check_engine(e, w, "weights"));
    HH_TRY(check_range(w, w_off, m * rb, "weights"));
    HH_NOT_NULL(x, "x");
    HH_TRY(e->select());
    hh_pending* p = new (std::nothrow) hh_pending{e, nullptr, nullptr, m, nullptr, false};
    if (!p) return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
    auto bail = [&](hh_status st) {
        if (p->dx) (void)hipFree(p->dx);
        if (p->dy) (void)hipFree(p->dy);
        if (p->done) (void)hipEventDestroy(p->done);
        delete p;
        return st;
    };
    hipError_t err = hipMalloc(&p->dx, n * sizeof(float));
    if (err == hipSuccess) err = hipMalloc(&p->dy, m * sizeof(float));
    if (err == hipSuccess) err = hipEventCreateWithFlags(&p->done, hipEventDisableTiming);
    if (err == hipSuccess) err = hipMemcpyAsync(p->dx, x, n * sizeof(float), hipMemcpyHostToDevice, e->stream);
    if (err != hipSuccess) return bail(hip_fail(err, "hh_gemv_begin"));
    e->ffn_calls++;
    hh_status st = e->enqueue_gemv(t, m, n, (const uint8_t*)w->ptr + w_off, (const float*)p->dx, (float*)p->dy);
    if (st != HH_OK) {
        (void)hipStreamSynchronize(e->stream);
        return bail(st);
    }
    err = hipEventRecord(p->done, e->stream);
    if (err != hipSuccess) {
        (void)hipStreamSynchronize(e->stream);
        return bail(hip_fail(err, "hipEventRecord"));
    }
    *out = p;
    return HH_OK;
}

hh_status hh_pending_wait(hh_pending* p, float* y, size_t m) {
    HH_NOT_NULL(p, "pending");
    HH_NOT_NULL(y, "y");
    if (m < p->m) return fail(HH_ERR_INVALID, "hh_pending_wait: output holds %zu < %zu floats", m, p->m);
    HH_TRY(p->engine->select());
    HH_TRY_HIP(hipEventSynchronize(p->done), "hipEventSynchronize");
    p->waited = true;
    HH_TRY_HIP(hipMemcpy(y, p->dy, p->m * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy(y)");
    return HH_OK;
}

void hh_pending_destroy(hh_pending* p) {
    if (!p) return;
    (void)hipSetDevice(p->engine->device);
    (void)hipEventSynchronize(p->done);  // never free buffers a queued kernel still uses
    (void)hipFree(p->dx);
    (void)hipFree(p->dy);
    (void)hipEventDestroy(p->done);
    delete p;
}

// ---------------------------------------------------------------- Q4 LUT GEMV ------

// The reference asserts these (compute.rs:54-58, matmul.rs:61-66); here they are status codes.
static hh_status lut_shape(size_t m, size_t n) {
    if (m == 0 || n == 0) return fail(HH_ERR_INVALID, "lut_matmul_q4: empty shape m=%zu n=%zu", m, n);
    if (n % 2 != 0) return fail(HH_ERR_INVALID, "lut_matmul_q4: N must be even for packed Q4 weights (n=%zu)", n);
    if (m > SIZE_MAX / (n / 2)) return fail(HH_ERR_INVALID, "lut_matmul_q4: weight size overflow");
    return HH_OK;
}

hh_status hh_lut_gemv(hh_engine* e, size_t m, size_t n, const uint8_t* weights_q4, size_t weights_len,
                      const float* lut, const float* x, float* y) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(lut_shape(m, n));
    HH_NOT_NULL(weights_q4, "weights_q4");
    HH_NOT_NULL(lut, "lut");
    HH_NOT_NULL(x, "x");
    HH_NOT_NULL(y, "y");
    const size_t wb = m * (n / 2);
    if (weights_len != wb)
        return fail(HH_ERR_INVALID, "lut_matmul_q4: weights_q4 has %zu bytes, expected m*n/2 = %zu", weights_len, wb);
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    // one staging buffer: [lut 64 B][x n*4 B][weights], x 16-byte aligned
    const size_t xo = 64, wo = xo + ((n * sizeof(float) + 255) / 256) * 256;
    HH_TRY(e->grow(&e->ws_w, &e->ws_w_cap, wo + wb));
    HH_TRY(e->grow(&e->ws_y, &e->ws_y_cap, m * sizeof(float)));
    char* base = (char*)e->ws_w;
    HH_TRY_HIP(hipMemcpyAsync(base, lut, 16 * sizeof(float), hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(lut)");
    HH_TRY_HIP(hipMemcpyAsync(base + xo, x, n * sizeof(float), hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(x)");
    HH_TRY_HIP(hipMemcpyAsync(base + wo, weights_q4, wb, hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(w)");
    HH_TRY(e->enqueue_lut(m, n, (const uint8_t*)(base + wo), (const float*)base, (const float*)(base + xo),
                          (float*)e->ws_y));
    HH_TRY_HIP(hipMemcpyAsync(y, e->ws_y, m * sizeof(float), hipMemcpyDeviceToHost, e->stream), "hipMemcpyAsync(y)");
    HH_TRY_HIP(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return HH_OK;
}

hh_status hh_lut_gemv_dev(hh_engine* e, size_t m, size_t n, const hh_buf* w, size_t w_off, const hh_buf* lut,
                          size_t lut_off, const hh_buf* x, size_t x_off, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(lut_shape(m, n));
    HH_TRY(check_engine(e, w, "weights"));
    HH_TRY(check_engine(e, lut, "lut"));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(w, w_off, m * (n / 2), "weights"));
    HH_TRY(check_range(lut, lut_off, 16 * sizeof(float), "lut"));
    HH_TRY(check_range(x, x_off, n * sizeof(float), "x"));
    HH_TRY(check_range(y, y_off, m * sizeof(float), "y"));
    if (lut_off % 4 || x_off % 4 || y_off % 4) return fail(HH_ERR_INVALID, "lut_matmul_q4: f32 offsets must be 4-byte aligned");
    HH_TRY(e->select());
    return e->enqueue_lut(m, n, (const uint8_t*)w->ptr + w_off, (const float*)((const char*)lut->ptr + lut_off),
                          (const float*)((const char*)x->ptr + x_off), (float*)((char*)y->ptr + y_off));
}

hh_status hh_dequant_dev(hh_engine* e, int t, const hh_buf* w, size_t w_off, size_t n, hh_buf* out, size_t out_off) {
    HH_NOT_NULL(e, "engine");
    const Format* f = format_of(t);
    if (!f || t == HH_TYPE_F32) return fail(HH_ERR_KERNEL_MISSING, "no dequant kernel for GGML type %d", t);
    if (t != HH_TYPE_Q4_0 && t != HH_TYPE_Q8_0 && n % f->block != 0)
        return fail(HH_ERR_INVALID, "dequant_%s: n=%zu not a multiple of %u", f->name, n, f->block);
    const size_t nblk = (n + f->block - 1) / f->block;
    HH_TRY(check_engine(e, w, "weights"));
    HH_TRY(check_engine(e, out, "out"));
    HH_TRY(check_range(w, w_off, nblk * f->bytes, "weights"));
    HH_TRY(check_range(out, out_off, n * sizeof(float), "out"));
    if ((w_off & 1u) || (out_off & 3u)) return fail(HH_ERR_INVALID, "dequant_%s: misaligned offsets", f->name);
    if (n == 0) return HH_OK;
    HH_TRY(e->select());
    hipFunction_t fn;
    HH_TRY(e->kernel(std::string("hh_dequant_") + f->name, &fn));
    hh_dequant_args a{(const uint8_t*)w->ptr + w_off, (float*)((char*)out->ptr + out_off), (uint64_t)n};
    const size_t threads = t == HH_TYPE_F16 ? n : nblk;
    return e->launch(fn, (uint32_t)((threads + 255) / 256), 256, a);
}

// ---------------------------------------------------------------- FFN ----------------

static hh_status validate_ffn(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off) {
    HH_NOT_NULL(d, "desc");
    if (d->act != HH_ACT_SILU && d->act != HH_ACT_GELU_TANH) return fail(HH_ERR_INVALID, "ffn: unknown act %d", d->act);
    HH_TRY(validate_shape(d->type_gate, d->d_ff, d->d_model));
    HH_TRY(validate_shape(d->type_up, d->d_ff, d->d_model));
    HH_TRY(validate_shape(d->type_down, d->d_model, d->d_ff));
    size_t rg, ru, rd;
    HH_TRY(row_bytes(d->type_gate, d->d_model, &rg));
    HH_TRY(row_bytes(d->type_up, d->d_model, &ru));
    HH_TRY(row_bytes(d->type_down, d->d_ff, &rd));
    HH_TRY(check_engine(e, pack, "pack"));
    if (pack_off > pack->size) return fail(HH_ERR_INVALID, "ffn: pack offset outside the buffer");
    HH_TRY(check_range(pack, pack_off + d->gate_off, d->d_ff * rg, "ffn gate"));
    HH_TRY(check_range(pack, pack_off + d->up_off, d->d_ff * ru, "ffn up"));
    HH_TRY(check_range(pack, pack_off + d->down_off, d->d_model * rd, "ffn down"));
    return HH_OK;
}

hh_status hh_ffn_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, const hh_buf* x,
                     size_t x_off, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(x, x_off, d->d_model * sizeof(float), "x"));
    HH_TRY(check_range(y, y_off, d->d_model * sizeof(float), "y"));
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn(d, (const uint8_t*)pack->ptr + pack_off, (const float*)((const char*)x->ptr + x_off),
                          (float*)((char*)y->ptr + y_off));
}

hh_status hh_ffn_dev_noalloc(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                             const hh_buf* x, size_t x_off, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(x, x_off, d->d_model * sizeof(float), "x"));
    HH_TRY(check_range(y, y_off, d->d_model * sizeof(float), "y"));
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_noalloc(d, (const uint8_t*)pack->ptr + pack_off,
                                  (const float*)((const char*)x->ptr + x_off), (float*)((char*)y->ptr + y_off));
}

hh_status hh_ffn_block_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                           const hh_buf* norm, size_t norm_off, float eps, const hh_buf* x, size_t x_off, hh_buf* y,
                           size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, norm, "norm"));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(norm, norm_off, d->d_model * sizeof(float), "norm"));
    HH_TRY(check_range(x, x_off, d->d_model * sizeof(float), "x"));
    HH_TRY(check_range(y, y_off, d->d_model * sizeof(float), "y"));
    if (((norm_off | x_off | y_off) & 3u) != 0)
        return fail(HH_ERR_INVALID, "ffn_block: norm/x/y offsets must be 4-byte aligned");
    if (!(eps >= 0.f) || eps > 1.f) return fail(HH_ERR_INVALID, "ffn_block: eps=%g outside [0, 1]", (double)eps);
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_block(d, (const uint8_t*)pack->ptr + pack_off,
                                (const float*)((const char*)x->ptr + x_off),
                                (const float*)((const char*)norm->ptr + norm_off), eps,
                                (float*)((char*)y->ptr + y_off));
}

hh_status hh_ffn_block_stack_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                                 size_t layer_stride, size_t n_layers, const hh_buf* norm, size_t norm_off,
                                 size_t norm_stride, float eps, const hh_buf* x, size_t x_off, hh_buf* y,
                                 size_t y_off) {
    HH_NOT_NULL(e, "engine");
    if (n_layers == 0) return fail(HH_ERR_INVALID, "ffn_block_stack: n_layers must be at least 1");
    size_t last_pack, last_norm;
    if (__builtin_mul_overflow(n_layers - 1, layer_stride, &last_pack) ||
        __builtin_add_overflow(last_pack, pack_off, &last_pack) ||
        __builtin_mul_overflow(n_layers - 1, norm_stride, &last_norm) ||
        __builtin_mul_overflow(last_norm, sizeof(float), &last_norm) ||
        __builtin_add_overflow(last_norm, norm_off, &last_norm))
        return fail(HH_ERR_INVALID, "ffn_block_stack: layer offsets overflow");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(validate_ffn(e, d, pack, last_pack));  // layers lie between the first and the last
    HH_TRY(check_engine(e, norm, "norm"));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(norm, norm_off, d->d_model * sizeof(float), "norm"));
    HH_TRY(check_range(norm, last_norm, d->d_model * sizeof(float), "norm"));
    HH_TRY(check_range(x, x_off, d->d_model * sizeof(float), "x"));
    HH_TRY(check_range(y, y_off, d->d_model * sizeof(float), "y"));
    if (((norm_off | x_off | y_off) & 3u) != 0)
        return fail(HH_ERR_INVALID, "ffn_block_stack: norm/x/y offsets must be 4-byte aligned");
    if (!(eps >= 0.f) || eps > 1.f)
        return fail(HH_ERR_INVALID, "ffn_block_stack: eps=%g outside [0, 1]", (double)eps);
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_block_stack(d, (const uint8_t*)pack->ptr + pack_off, layer_stride, n_layers,
                                      (const float*)((const char*)norm->ptr + norm_off), norm_stride, eps,
                                      (const float*)((const char*)x->ptr + x_off), (float*)((char*)y->ptr + y_off));
}

hh_status hh_ffn_batched_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, const hh_buf* x,
                             size_t x_off, size_t batch, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("ffn_batched_dev"));
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    size_t xb;
    HH_TRY(batch_bytes(batch, d->d_model, &xb));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(x, x_off, xb, "x"));
    HH_TRY(check_range(y, y_off, xb, "y"));
    if (((x_off | y_off) & 3u) != 0) return fail(HH_ERR_INVALID, "ffn_batched: x/y offsets must be 4-byte aligned");
    if (batch == 0) return HH_OK;
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_batched(d, (const uint8_t*)pack->ptr + pack_off, (const float*)((const char*)x->ptr + x_off),
                                  batch, (float*)((char*)y->ptr + y_off));
}

hh_status hh_ffn_batched(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, const float* x,
                         float* y, size_t batch) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    size_t xb;
    HH_TRY(batch_bytes(batch, d->d_model, &xb));
    if (batch == 0) return HH_OK;
    HH_NOT_NULL(x, "x");
    HH_NOT_NULL(y, "y");
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    HH_TRY(e->grow(&e->ws_x, &e->ws_x_cap, xb));
    HH_TRY(e->grow(&e->ws_y, &e->ws_y_cap, xb));
    HH_TRY_HIP(hipMemcpyAsync(e->ws_x, x, xb, hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(x)");
    HH_TRY(e->enqueue_ffn_batched(d, (const uint8_t*)pack->ptr + pack_off, (const float*)e->ws_x, batch,
                                  (float*)e->ws_y));
    HH_TRY_HIP(hipMemcpyAsync(y, e->ws_y, xb, hipMemcpyDeviceToHost, e->stream), "hipMemcpyAsync(y)");
    return e->check_device_error();
}

hh_status hh_ffn_begin_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, const hh_buf* x,
                           size_t x_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_range(x, x_off, d->d_model * sizeof(float), "x"));
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_begin(d, (const uint8_t*)pack->ptr + pack_off, (const float*)((const char*)x->ptr + x_off));
}

hh_status hh_ffn_finish_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, hh_buf* y,
                            size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(y, y_off, d->d_model * sizeof(float), "y"));
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_finish(d, (const uint8_t*)pack->ptr + pack_off, (float*)((char*)y->ptr + y_off));
}

hh_status hh_ffn_block_begin_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                                 const hh_buf* norm, size_t norm_off, float eps, const hh_buf* x, size_t x_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, norm, "norm"));
    HH_TRY(check_engine(e, x, "x"));
    HH_TRY(check_range(norm, norm_off, d->d_model * sizeof(float), "norm"));
    HH_TRY(check_range(x, x_off, d->d_model * sizeof(float), "x"));
    if (((norm_off | x_off) & 3u) != 0) return fail(HH_ERR_INVALID, "ffn_block_begin: norm/x offsets must be 4-byte aligned");
    if (!(eps >= 0.f) || eps > 1.f) return fail(HH_ERR_INVALID, "ffn_block_begin: eps=%g outside [0, 1]", (double)eps);
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_begin(d, (const uint8_t*)pack->ptr + pack_off, (const float*)((const char*)x->ptr + x_off),
                                (const float*)((const char*)norm->ptr + norm_off), eps);
}

hh_status hh_ffn_block_finish_dev(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off,
                                  const hh_buf* res, size_t res_off, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_TRY(check_engine(e, res, "res"));
    HH_TRY(check_engine(e, y, "y"));
    HH_TRY(check_range(res, res_off, d->d_model * sizeof(float), "res"));
    HH_TRY(check_range(y, y_off, d->d_model * sizeof(float), "y"));
    if (((res_off | y_off) & 3u) != 0) return fail(HH_ERR_INVALID, "ffn_block_finish: res/y offsets must be 4-byte aligned");
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    return e->enqueue_ffn_finish(d, (const uint8_t*)pack->ptr + pack_off, (float*)((char*)y->ptr + y_off),
                                 (const float*)((const char*)res->ptr + res_off));
}

hh_status hh_ffn(hh_engine* e, const hh_ffn_desc* d, const hh_buf* pack, size_t pack_off, const float* x, float* y) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_ffn(e, d, pack, pack_off));
    HH_NOT_NULL(x, "x");
    HH_NOT_NULL(y, "y");
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    HH_TRY(e->grow(&e->ws_x, &e->ws_x_cap, d->d_model * sizeof(float)));
    HH_TRY(e->grow(&e->ws_y, &e->ws_y_cap, d->d_model * sizeof(float)));
    HH_TRY_HIP(hipMemcpyAsync(e->ws_x, x, d->d_model * sizeof(float), hipMemcpyHostToDevice, e->stream),
               "hipMemcpyAsync(x)");
    HH_TRY(e->enqueue_ffn(d, (const uint8_t*)pack->ptr + pack_off, (const float*)e->ws_x, (float*)e->ws_y));
    HH_TRY_HIP(hipMemcpyAsync(y, e->ws_y, d->d_model * sizeof(float), hipMemcpyDeviceToHost, e->stream),
               "hipMemcpyAsync(y)");
    return e->check_device_error();
}

hh_status hh_gateup_dev(hh_engine* e, int tg, int tu, size_t d_ff, size_t d_model, const hh_buf* wg, size_t wg_off,
                        const hh_buf* wu, size_t wu_off, const hh_buf* x, size_t x_off, hh_buf* h, size_t h_off,
                        int act) {
    HH_NOT_NULL(e, "engine");
    if (act != HH_ACT_SILU && act != HH_ACT_GELU_TANH) return fail(HH_ERR_INVALID, "gateup: unknown act %d", act);
    HH_TRY(validate_shape(tg, d_ff, d_model));
    HH_TRY(validate_shape(tu, d_ff, d_model));
    size_t rg, ru;
    HH_TRY(row_bytes(tg, d_model, &rg));
    HH_TRY(row_bytes(tu, d_model, &ru));
    for (const hh_buf* b : {wg, wu, (const hh_buf*)x, (const hh_buf*)h}) HH_TRY(check_engine(e, b, "gateup"));
    HH_TRY(check_range(wg, wg_off, d_ff * rg, "gate"));
    HH_TRY(check_range(wu, wu_off, d_ff * ru, "up"));
    HH_TRY(check_range(x, x_off, d_model * sizeof(float), "x"));
    HH_TRY(check_range(h, h_off, d_ff * sizeof(float), "h"));
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    e->ffn_calls += 2;
    return e->enqueue_gateup(tg, tu, d_ff, d_model, (const uint8_t*)wg->ptr + wg_off, (const uint8_t*)wu->ptr + wu_off,
                             (const float*)((const char*)x->ptr + x_off), (float*)((char*)h->ptr + h_off), act);
}

// ---------------------------------------------------------------- MoE ----------------

static hh_status validate_moe_desc(const hh_moe_desc* d) {
    HH_NOT_NULL(d, "moe desc");
    if (d->type != HH_TYPE_Q4_K)
        return fail(HH_ERR_KERNEL_MISSING, "moe: experts of GGML type %d have no MoE kernel (Q4_K only)", d->type);
    if (d->act != HH_ACT_SILU && d->act != HH_ACT_GELU_TANH) return fail(HH_ERR_INVALID, "moe: unknown act %d", d->act);
    if (d->n_experts < 1 || d->n_experts > 512)
        return fail(HH_ERR_INVALID, "moe: n_experts=%zu outside 1..512", d->n_experts);
    if (d->top_k < 1 || d->top_k > 64) return fail(HH_ERR_INVALID, "moe: top_k=%zu outside 1..64", d->top_k);
    if (d->n_group > 64) return fail(HH_ERR_INVALID, "moe: n_group=%zu > 64", d->n_group);
    return HH_OK;
}

static hh_status validate_moe_experts(hh_engine* e, const hh_moe_desc* d, const hh_buf* experts, size_t off) {
    HH_TRY(validate_shape(d->type, d->d_ff, d->d_model));
    HH_TRY(validate_shape(d->type, d->d_model, d->d_ff));
    size_t rin, rff;
    HH_TRY(row_bytes(d->type, d->d_model, &rin));
    HH_TRY(row_bytes(d->type, d->d_ff, &rff));
    // LDS of the expert kernels holds the digits of x (d_model) and of the k intermediates
    const size_t lds_in = 2 * d->d_model + d->d_model / 4, lds_ff = 2 * d->top_k * d->d_ff + d->top_k * d->d_ff / 4;
    if (lds_in > 65536 || lds_ff > 65536)
        return fail(HH_ERR_INVALID, "moe: d_model=%zu / top_k*d_ff=%zu too large for the expert kernels", d->d_model,
                    d->top_k * d->d_ff);
    HH_TRY(check_engine(e, experts, "experts"));
    const size_t pack_end = std::max({d->gate_off + d->d_ff * rin, d->up_off + d->d_ff * rin,
                                      d->down_off + d->d_model * rff});
    if (d->expert_stride != 0 && d->n_experts - 1 > (SIZE_MAX - pack_end) / d->expert_stride)
        return fail(HH_ERR_INVALID, "moe: expert layout overflows");
    HH_TRY(check_range(experts, off, (d->n_experts - 1) * d->expert_stride + pack_end, "moe experts"));
    if (((uintptr_t)experts->ptr + off) % 16 || d->expert_stride % 16 || d->gate_off % 16 || d->up_off % 16 ||
        d->down_off % 16)
        return fail(HH_ERR_INVALID, "moe: expert packs and tensor offsets must be 16-byte aligned");
    if (d->shared_d_ff) {  // the shared expert: an FFN of d_model x shared_d_ff in the same buffer
        HH_TRY(validate_shape(d->type, d->shared_d_ff, d->d_model));
        HH_TRY(validate_shape(d->type, d->d_model, d->shared_d_ff));
        size_t rsf;
        HH_TRY(row_bytes(d->type, d->shared_d_ff, &rsf));
        const size_t g = d->shared_d_ff * rin, dn = d->d_model * rsf;
        if (d->shared_gate_off > SIZE_MAX - g || d->shared_up_off > SIZE_MAX - g || d->shared_down_off > SIZE_MAX - dn)
            return fail(HH_ERR_INVALID, "moe: shared expert layout overflows");
        HH_TRY(check_range(experts, off, std::max({d->shared_gate_off + g, d->shared_up_off + g, d->shared_down_off + dn}),
                           "moe shared expert"));
    }
    return HH_OK;
}

hh_status hh_route_experts_dev(hh_engine* e, const hh_moe_desc* d, const hh_buf* logits, size_t logits_off,
                               const hh_buf* bias, size_t bias_off, size_t T, hh_buf* ids, size_t ids_off,
                               hh_buf* weights, size_t weights_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("route_experts_dev"));
    HH_TRY(validate_moe_desc(d));
    size_t lb = 0, kb = 0;
    HH_TRY(batch_bytes(T, d->n_experts, &lb));
    HH_TRY(batch_bytes(T, d->top_k, &kb));
    HH_TRY(check_engine(e, logits, "logits"));
    HH_TRY(check_engine(e, ids, "ids"));
    HH_TRY(check_engine(e, weights, "weights"));
    HH_TRY(check_range(logits, logits_off, lb, "logits"));
    HH_TRY(check_range(ids, ids_off, kb, "ids"));
    HH_TRY(check_range(weights, weights_off, kb, "weights"));
    if (bias) {
        HH_TRY(check_engine(e, bias, "bias"));
        HH_TRY(check_range(bias, bias_off, d->n_experts * sizeof(float), "bias"));
    }
    if ((logits_off | ids_off | weights_off | bias_off) & 3u)
        return fail(HH_ERR_INVALID, "route_experts: offsets must be 4-byte aligned");
    if (T == 0) return HH_OK;
    HH_TRY(e->select());
    return e->enqueue_moe_route(d, (const float*)((const char*)logits->ptr + logits_off),
                                bias ? (const float*)((const char*)bias->ptr + bias_off) : nullptr, T,
                                (int32_t*)((char*)ids->ptr + ids_off), (float*)((char*)weights->ptr + weights_off));
}

hh_status hh_route_experts(hh_engine* e, const hh_moe_desc* d, const float* logits, const float* bias, size_t T,
                           int32_t* ids, float* weights) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(validate_moe_desc(d));
    size_t lb = 0, kb = 0;
    HH_TRY(batch_bytes(T, d->n_experts, &lb));
    HH_TRY(batch_bytes(T, d->top_k, &kb));
    if (T == 0) return HH_OK;
    HH_NOT_NULL(logits, "logits");
    HH_NOT_NULL(ids, "ids");
    HH_NOT_NULL(weights, "weights");
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    // x workspace: logits then bias; y workspace: ids then weights
    const size_t bb = bias ? d->n_experts * sizeof(float) : 0;
    HH_TRY(e->grow(&e->ws_x, &e->ws_x_cap, lb + bb));
    HH_TRY(e->grow(&e->ws_y, &e->ws_y_cap, 2 * kb));
    HH_TRY_HIP(hipMemcpyAsync(e->ws_x, logits, lb, hipMemcpyHostToDevice, e->stream), "hipMemcpyAsync(logits)");
    if (bias)
        HH_TRY_HIP(hipMemcpyAsync((char*)e->ws_x + lb, bias, bb, hipMemcpyHostToDevice, e->stream),
                   "hipMemcpyAsync(bias)");
    HH_TRY(e->enqueue_moe_route(d, (const float*)e->ws_x, bias ? (const float*)((char*)e->ws_x + lb) : nullptr, T,
                                (int32_t*)e->ws_y, (float*)((char*)e->ws_y + kb)));
    HH_TRY_HIP(hipMemcpyAsync(ids, e->ws_y, kb, hipMemcpyDeviceToHost, e->stream), "hipMemcpyAsync(ids)");
    HH_TRY_HIP(hipMemcpyAsync(weights, (char*)e->ws_y + kb, kb, hipMemcpyDeviceToHost, e->stream),
               "hipMemcpyAsync(weights)");
    return e->check_device_error();
}

hh_status hh_moe_ffn_dev(hh_engine* e, const hh_moe_desc* d, const hh_buf* experts, size_t experts_off,
                         const hh_buf* x, size_t x_off, size_t T, const hh_buf* ids, size_t ids_off,
                         const hh_buf* weights, size_t weights_off, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("moe_ffn_dev"));
    HH_TRY(validate_moe_desc(d));
    HH_TRY(validate_moe_experts(e, d, experts, experts_off));
    size_t xb = 0, kb = 0;
    HH_TRY(batch_bytes(T, d->d_model, &xb));
    HH_TRY(batch_bytes(T, d->top_k, &kb));
    for (const hh_buf* b : {x, ids, weights, (const hh_buf*)y}) HH_TRY(check_engine(e, b, "moe"));
    HH_TRY(check_range(x, x_off, xb, "x"));
    HH_TRY(check_range(y, y_off, xb, "y"));
    HH_TRY(check_range(ids, ids_off, kb, "ids"));
    HH_TRY(check_range(weights, weights_off, kb, "weights"));
    if ((x_off & 15u) || ((y_off | ids_off | weights_off) & 3u))
        return fail(HH_ERR_INVALID, "moe_ffn: x offset must be 16-byte aligned, y/ids/weights 4-byte");
    if (T == 0) return HH_OK;
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    const uint8_t* ex = (const uint8_t*)experts->ptr + experts_off;
    const float* xp = (const float*)((const char*)x->ptr + x_off);
    float* yp = (float*)((char*)y->ptr + y_off);
    HH_TRY(e->enqueue_moe_ffn(d, ex, xp, T, (int32_t*)((char*)ids->ptr + ids_off),
                              (float*)((char*)weights->ptr + weights_off), yp));
    return e->enqueue_moe_shared(d, ex, xp, T, yp);
}

hh_status hh_moe_dev(hh_engine* e, const hh_moe_desc* d, const hh_buf* experts, size_t experts_off,
                     const hh_buf* logits, size_t logits_off, const hh_buf* bias, size_t bias_off, const hh_buf* x,
                     size_t x_off, size_t T, hh_buf* y, size_t y_off) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->no_capture("moe_dev"));
    HH_TRY(validate_moe_desc(d));
    HH_TRY(validate_moe_experts(e, d, experts, experts_off));
    size_t xb = 0, kb = 0, lb = 0;
    HH_TRY(batch_bytes(T, d->d_model, &xb));
    HH_TRY(batch_bytes(T, d->top_k, &kb));
    HH_TRY(batch_bytes(T, d->n_experts, &lb));
    for (const hh_buf* b : {logits, x, (const hh_buf*)y}) HH_TRY(check_engine(e, b, "moe"));
    HH_TRY(check_range(logits, logits_off, lb, "logits"));
    HH_TRY(check_range(x, x_off, xb, "x"));
    HH_TRY(check_range(y, y_off, xb, "y"));
    if (bias) {
        HH_TRY(check_engine(e, bias, "bias"));
        HH_TRY(check_range(bias, bias_off, d->n_experts * sizeof(float), "bias"));
    }
    if ((x_off & 15u) || ((y_off | logits_off | bias_off) & 3u))
        return fail(HH_ERR_INVALID, "moe: x offset must be 16-byte aligned, y/logits/bias 4-byte");
    if (T == 0) return HH_OK;
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    HH_TRY(e->grow(&e->ws_moe_ids, &e->ws_moe_ids_cap, kb));
    HH_TRY(e->grow(&e->ws_moe_w, &e->ws_moe_w_cap, kb));
    // routing runs inside the gate/up kernel
    const uint8_t* ex = (const uint8_t*)experts->ptr + experts_off;
    const float* xp = (const float*)((const char*)x->ptr + x_off);
    float* yp = (float*)((char*)y->ptr + y_off);
    HH_TRY(e->enqueue_moe_ffn(d, ex, xp, T, (int32_t*)e->ws_moe_ids, (float*)e->ws_moe_w, yp,
                              (const float*)((const char*)logits->ptr + logits_off),
                              bias ? (const float*)((const char*)bias->ptr + bias_off) : nullptr));
    return e->enqueue_moe_shared(d, ex, xp, T, yp);
}

// ---------------------------------------------------------------- events -------------

hh_status hh_event_create(hh_engine* e, hh_event** out) {
    HH_NOT_NULL(e, "engine");
    HH_NOT_NULL(out, "out");
    HH_TRY(e->select());
    hh_event* ev = new (std::nothrow) hh_event{nullptr, e->device};
    if (!ev) return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
    hipError_t err = hipEventCreate(&ev->ev);
    if (err != hipSuccess) {
        delete ev;
        return hip_fail(err, "hipEventCreate");
    }
    *out = ev;
    return HH_OK;
}

void hh_event_destroy(hh_event* ev) {
    if (!ev) return;
    (void)hipSetDevice(ev->device);
    (void)hipEventDestroy(ev->ev);
    delete ev;
}

hh_status hh_event_record(hh_engine* e, hh_event* ev) {
    HH_NOT_NULL(e, "engine");
    HH_NOT_NULL(ev, "event");
    HH_TRY(e->select());
    HH_TRY_HIP(hipEventRecord(ev->ev, e->stream), "hipEventRecord");
    return HH_OK;
}

hh_status hh_event_elapsed_ms(hh_event* a, hh_event* b, float* ms) {
    HH_NOT_NULL(a, "start");
    HH_NOT_NULL(b, "stop");
    HH_NOT_NULL(ms, "ms");
    HH_TRY_HIP(hipEventSynchronize(b->ev), "hipEventSynchronize");
    HH_TRY_HIP(hipEventElapsedTime(ms, a->ev, b->ev), "hipEventElapsedTime");
    return HH_OK;
}

// ---------------------------------------------------------------- graphs -------------

struct hh_graph {
    hh_engine* engine;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

hh_status hh_graph_begin(hh_engine* e) {
    HH_NOT_NULL(e, "engine");
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    if (e->capturing) return fail(HH_ERR_INVALID, "graph_begin: a capture is already open on this engine");
    HH_TRY_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    e->capturing = true;
    return HH_OK;
}

hh_status hh_graph_end(hh_engine* e, hh_graph** out) {
    HH_NOT_NULL(e, "engine");
    HH_NOT_NULL(out, "out");
    *out = nullptr;
    HH_TRY(e->select());
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    if (!e->capturing) return fail(HH_ERR_INVALID, "graph_end: no capture is open on this engine");
    e->capturing = false;
    hipGraph_t g = nullptr;
    HH_TRY_HIP(hipStreamEndCapture(e->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    hipError_t err = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_fail(err, "hipGraphInstantiate");
    }
    hh_graph* h = new (std::nothrow) hh_graph{e, g, x};
    if (!h) {
        (void)hipGraphExecDestroy(x);
        (void)hipGraphDestroy(g);
        return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
    }
    e->live_graphs++;
    *out = h;
    return HH_OK;
}

hh_status hh_graph_launch(hh_graph* g) {
    HH_NOT_NULL(g, "graph");
    HH_TRY(g->engine->select());
    std::lock_guard<std::mutex> lk(g->engine->ws_mutex);
    if (g->engine->capturing) return fail(HH_ERR_INVALID, "graph_launch: the engine's stream is being captured");
    HH_TRY_HIP(hipGraphLaunch(g->exec, g->engine->stream), "hipGraphLaunch");
    return HH_OK;
}

void hh_graph_destroy(hh_graph* g) {
    if (!g) return;
    hh_engine* e = g->engine;
    (void)e->select();
    std::lock_guard<std::mutex> lk(e->ws_mutex);
    // a replay may still be running on the stream
    (void)hipStreamSynchronize(e->stream);
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
    if (--e->live_graphs == 0) e->free_retired();
}

// ---------------------------------------------------------------- synthetic data -----

hh_status hh_synth_weights_dev(hh_engine* e, int t, hh_buf* dst, size_t off, size_t n_blocks, uint64_t seed, float lo,
                               float hi) {
    HH_NOT_NULL(e, "engine");
    const Format* f = format_of(t);
    if (!f) return fail(HH_ERR_KERNEL_MISSING, "no synthetic generator for GGML type %d", t);
    const size_t bytes = n_blocks * f->bytes;
    HH_TRY(check_engine(e, dst, "dst"));
    HH_TRY(check_range(dst, off, bytes, "synth"));
    if (off & 7u) return fail(HH_ERR_INVALID, "synth: offset must be 8-byte aligned");
    if (bytes == 0) return HH_OK;
    HH_TRY(e->select());
    hipFunction_t fb, fs;
    HH_TRY(e->kernel("hh_synth_bytes", &fb));
    HH_TRY(e->kernel("hh_synth_scales", &fs));
    hh_synth_args a{(uint8_t*)dst->ptr + off, (uint64_t)bytes, seed, (uint64_t)n_blocks, t, lo, hi, 0};
    const size_t words = (bytes + 7) / 8;
    const uint32_t grid = (uint32_t)std::min<size_t>((words + 255) / 256, 65536);
    HH_TRY(e->launch(fb, grid, 256, a));
    if (t == HH_TYPE_F32 || t == HH_TYPE_F16) return HH_OK;
    return e->launch(fs, (uint32_t)((n_blocks + 255) / 256), 256, a);
}

}  // extern "C"
