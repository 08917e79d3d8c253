// Pinned-host ping-pong weight streaming: the MI355X counterpart of the reference's
// StreamingScratch (crates/hayai-opencl/src/hetero_scratch.rs:48-71,87-236,565-571,611-656,
// 781-849,853-925) with PinnedHostBuffer slots (crates/hayai-opencl/src/memory.rs:72-147).
//
// n_slots host slots (hipHostMalloc, page-locked) and n_slots device mirrors (hipMalloc), each
// block_k * layer_bytes.  Layer L lives in slot (L / block_k) % n_slots at byte offset
// (L % block_k) * layer_bytes.  A caller (the layer loader) fills a host slot, the DMA of the
// layer's regions runs on the engine's copy stream (hipMemcpyAsync), and the FFN kernels read
// the device mirror on the compute stream.  Ordering is by events, never by host waits on the
// hot path:
//   - a DMA into a mirror slot waits (hipStreamWaitEvent on the copy stream) for everything
//     the compute stream had been given when the DMA was issued -- in particular the FFN of
//     the layer that occupied the slot before;
//   - binding layer L for compute makes the compute stream wait for the last DMA into L's slot;
//   - handing out a host slot for writing waits (host side) until no DMA still reads it
//     (prepare_host_write, hetero_scratch.rs:626-656).
#include <cstring>
#include <new>
#include <vector>

#include "engine.h"

using namespace hh;

struct hh_streamer {
    hh_engine* engine = nullptr;
    size_t layer_bytes = 0;
    size_t block_k = 1;
    size_t n_slots = 0;
    size_t slot_bytes = 0;
    std::vector<void*> host;      // pinned host slots
    std::vector<hh_buf*> mirror;  // device mirror slots (owned)
    std::vector<hipEvent_t> dma_done;   // per slot: last DMA into the mirror completed
    std::vector<bool> dma_pending;      // per slot: dma_done was recorded and not yet waited on the host
    std::vector<long long> staged;      // per slot: block id whose DMA was issued last (-1 none)
    hipEvent_t tail = nullptr;          // re-recorded on the compute stream before each DMA
    hipEvent_t half = nullptr;          // re-recorded on the second copy stream after its half
};

static void streamer_free(hh_streamer* s) {
    if (!s) return;
    if (s->engine) {
        (void)hipSetDevice(s->engine->device);
        (void)hipStreamSynchronize(s->engine->copy_stream);
        (void)hipStreamSynchronize(s->engine->copy_stream2);
        (void)hipStreamSynchronize(s->engine->stream);
    }
    for (hipEvent_t ev : s->dma_done)
        if (ev) (void)hipEventDestroy(ev);
    if (s->tail) (void)hipEventDestroy(s->tail);
    if (s->half) (void)hipEventDestroy(s->half);
    for (void* p : s->host)
        if (p) (void)hipHostFree(p);
    for (hh_buf* b : s->mirror)
        if (b) {
            if (b->ptr) (void)hipFree(b->ptr);
            delete b;
        }
    delete s;
}

static hh_status check_layer(const hh_streamer* s, size_t layer, size_t* slot, size_t* in_slot) {
    if (!s) return fail(HH_ERR_INVALID, "streamer is NULL");
    *slot = (layer / s->block_k) % s->n_slots;
    *in_slot = (layer % s->block_k) * s->layer_bytes;
    return HH_OK;
}

extern "C" {

hh_status hh_streamer_create(hh_engine* e, size_t layer_bytes, size_t block_k, size_t n_slots, hh_streamer** out) {
    if (!out) return fail(HH_ERR_INVALID, "out is NULL");
    *out = nullptr;
    if (!e) return fail(HH_ERR_INVALID, "engine is NULL");
    if (layer_bytes == 0) return fail(HH_ERR_INVALID, "streamer: layer_bytes is 0");
    if (block_k == 0) block_k = 1;       // k_chunk.max(1), hetero_scratch.rs:94
    if (n_slots < 2) n_slots = 2;        // n_slots.max(2), hetero_scratch.rs:95
    if (layer_bytes > SIZE_MAX / block_k) return fail(HH_ERR_INVALID, "streamer: slot size overflow");
    HH_TRY(e->select());
    hh_streamer* s = new (std::nothrow) hh_streamer();
    if (!s) return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
    s->engine = e;
    s->layer_bytes = layer_bytes;
    s->block_k = block_k;
    s->n_slots = n_slots;
    s->slot_bytes = layer_bytes * block_k;
    s->host.assign(n_slots, nullptr);
    s->mirror.assign(n_slots, nullptr);
    s->dma_done.assign(n_slots, nullptr);
    s->dma_pending.assign(n_slots, false);
    s->staged.assign(n_slots, -1);
    if (hipError_t err = hipEventCreateWithFlags(&s->half, hipEventDisableTiming); err != hipSuccess) {
        streamer_free(s);
        return hip_fail(err, "hipEventCreate(streamer)");
    }
    if (hipError_t err = hipEventCreateWithFlags(&s->tail, hipEventDisableTiming); err != hipSuccess) {
        streamer_free(s);
        return hip_fail(err, "hipEventCreate(streamer)");
    }
    for (size_t i = 0; i < n_slots; i++) {
        hipError_t err = hipHostMalloc(&s->host[i], s->slot_bytes, hipHostMallocDefault);
        if (err != hipSuccess) {
            streamer_free(s);
            return hip_fail(err, "hipHostMalloc(streamer slot)");
        }
        void* d = nullptr;
        err = hipMalloc(&d, s->slot_bytes);
        if (err != hipSuccess) {
            streamer_free(s);
            return hip_fail(err, "hipMalloc(streamer mirror)");
        }
        s->mirror[i] = new (std::nothrow) hh_buf{e, d, s->slot_bytes, HH_BUF_DEVICE};
        if (!s->mirror[i]) {
            (void)hipFree(d);
            streamer_free(s);
            return fail(HH_ERR_OUT_OF_MEMORY, "host allocation failed");
        }
        err = hipEventCreateWithFlags(&s->dma_done[i], hipEventDisableTiming);
        if (err != hipSuccess) {
            streamer_free(s);
            return hip_fail(err, "hipEventCreate(streamer)");
        }
    }
    *out = s;
    return HH_OK;
}

void hh_streamer_destroy(hh_streamer* s) { streamer_free(s); }

hh_status hh_streamer_slot_for(const hh_streamer* s, size_t layer, size_t* slot) {
    if (!slot) return fail(HH_ERR_INVALID, "slot is NULL");
    size_t in_slot = 0;
    return check_layer(s, layer, slot, &in_slot);
}

hh_status hh_streamer_weight_offset(const hh_streamer* s, size_t layer, size_t tensor_off, size_t* off) {
    if (!off) return fail(HH_ERR_INVALID, "off is NULL");
    size_t slot = 0, in_slot = 0;
    HH_TRY(check_layer(s, layer, &slot, &in_slot));
    *off = in_slot + tensor_off;
    return HH_OK;
}

hh_status hh_streamer_host_slot(hh_streamer* s, size_t layer, void** host_ptr) {
    if (!host_ptr) return fail(HH_ERR_INVALID, "host_ptr is NULL");
    *host_ptr = nullptr;
    size_t slot = 0, in_slot = 0;
    HH_TRY(check_layer(s, layer, &slot, &in_slot));
    HH_TRY(s->engine->select());
    if (s->dma_pending[slot]) {
        // never overwrite host bytes a DMA is still reading (wait_dma, hetero_scratch.rs:611-624)
        HH_TRY_HIP(hipEventSynchronize(s->dma_done[slot]), "hipEventSynchronize(streamer dma)");
        s->dma_pending[slot] = false;
    }
    *host_ptr = (char*)s->host[slot] + in_slot;
    return HH_OK;
}

hh_status hh_streamer_dma(hh_streamer* s, size_t layer, size_t off, size_t len) {
    size_t slot = 0, in_slot = 0;
    HH_TRY(check_layer(s, layer, &slot, &in_slot));
    if (off > s->layer_bytes || len > s->layer_bytes - off)
        return fail(HH_ERR_INVALID, "streamer dma: range [%zu, +%zu) outside a %zu-byte layer", off, len,
                    s->layer_bytes);
    hh_engine* e = s->engine;
    HH_TRY(e->select());
    const long long block = (long long)(layer / s->block_k);
    if (len > 0) {
        // The mirror slot may still be read by compute work enqueued earlier (the layer that
        // held this slot before): the copy stream waits for the compute stream's tail.
        // (A wait binds to the event's most recent record at the time of the wait.)
        HH_TRY_HIP(hipEventRecord(s->tail, e->stream), "hipEventRecord(streamer tail)");
        HH_TRY_HIP(hipStreamWaitEvent(e->copy_stream, s->tail, 0), "hipStreamWaitEvent(streamer dma)");
        const size_t at = in_slot + off;
        // copies of 32 MB and more go out as two halves on two copy streams (two DMA engines
        // pulling over the host link); the first stream waits for the second's half before
        // the slot's completion event, so dma_done covers both
        const size_t first = (e->dma_split && len >= ((size_t)32 << 20)) ? (len / 2) & ~(size_t)4095 : len;
        HH_TRY_HIP(hipMemcpyAsync((char*)s->mirror[slot]->ptr + at, (const char*)s->host[slot] + at, first,
                                  hipMemcpyHostToDevice, e->copy_stream),
                   "hipMemcpyAsync(streamer dma)");
        if (first < len) {
            HH_TRY_HIP(hipStreamWaitEvent(e->copy_stream2, s->tail, 0), "hipStreamWaitEvent(streamer dma 2)");
            HH_TRY_HIP(hipMemcpyAsync((char*)s->mirror[slot]->ptr + at + first, (const char*)s->host[slot] + at + first,
                                      len - first, hipMemcpyHostToDevice, e->copy_stream2),
                       "hipMemcpyAsync(streamer dma 2)");
            HH_TRY_HIP(hipEventRecord(s->half, e->copy_stream2), "hipEventRecord(streamer half)");
            HH_TRY_HIP(hipStreamWaitEvent(e->copy_stream, s->half, 0), "hipStreamWaitEvent(streamer half)");
        }
    }
    HH_TRY_HIP(hipEventRecord(s->dma_done[slot], e->copy_stream), "hipEventRecord(streamer dma)");
    s->dma_pending[slot] = true;
    s->staged[slot] = block;
    return HH_OK;
}

hh_status hh_streamer_bind(hh_streamer* s, size_t layer, hh_buf** mirror, size_t* layer_off) {
    if (!mirror || !layer_off) return fail(HH_ERR_INVALID, "mirror / layer_off is NULL");
    size_t slot = 0, in_slot = 0;
    HH_TRY(check_layer(s, layer, &slot, &in_slot));
    const long long block = (long long)(layer / s->block_k);
    if (s->staged[slot] != block)
        return fail(HH_ERR_INVALID, "streamer bind: layer %zu is not staged (slot %zu holds block %lld)", layer, slot,
                    s->staged[slot]);
    hh_engine* e = s->engine;
    HH_TRY(e->select());
    HH_TRY_HIP(hipStreamWaitEvent(e->stream, s->dma_done[slot], 0), "hipStreamWaitEvent(streamer bind)");
    *mirror = s->mirror[slot];
    *layer_off = in_slot;
    return HH_OK;
}

}  // extern "C"
