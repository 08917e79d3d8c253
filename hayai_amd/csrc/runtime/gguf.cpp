// GGUF catalog and layer-pack loader on the host (C ABI in include/hayai_hip.h).
//
// Replaces the reference's GgufCatalog header parse and load_layer_pack_into
// (crates/hayai-model/src/gguf.rs:25-127,240-284,547-680; gguf_stream.rs:34-192,381-397,
// 451-638) and its weight reader (crates/hayai-io/src/weight_io.rs:14-105,235-470): the
// header is parsed from a growing prefix of the file, a layer's tensors are laid out back
// to back in pack order and read with one batch of io_uring reads (plain pread where
// io_uring is unavailable or HAYAI_FORCE_FILE_IO is set).  Nothing here touches the GPU:
// the destination is any host buffer, typically a pinned streaming slot.
#include <fcntl.h>
#include <linux/io_uring.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/hayai_hip.h"
#include "engine.h"

namespace hh {

// ------------------------------------------------------------------- weight reader ------

struct IoReq {
    uint64_t offset;  // absolute file offset
    size_t start;     // destination range [start, end)
    size_t end;
};

// io_uring through its raw system calls (no liburing): one submission ring of 256 entries,
// reads submitted in batches and every completion reaped before the next batch.
struct Uring {
    int fd = -1;
    void* sq_ptr = MAP_FAILED;
    void* cq_ptr = MAP_FAILED;
    size_t sq_sz = 0, cq_sz = 0, sqes_sz = 0;
    io_uring_sqe* sqes = (io_uring_sqe*)MAP_FAILED;
    unsigned *sq_head = nullptr, *sq_tail = nullptr, *sq_mask = nullptr, *sq_array = nullptr;
    unsigned *cq_head = nullptr, *cq_tail = nullptr, *cq_mask = nullptr;
    io_uring_cqe* cqes = nullptr;
    unsigned entries = 0;
    bool broken = false;
    // IORING_ASYNC_CANCEL_ANY (Linux 5.19 uapi; older kernels reject the request, which is
    // harmless here) and the user_data tag of that cancel request's own completion.
    static constexpr uint32_t kCancelAny = 1u << 2;
    static constexpr uint64_t kCancelTag = ~(uint64_t)0;

    bool setup(unsigned n) {
        io_uring_params p;
        memset(&p, 0, sizeof p);
        fd = (int)syscall(__NR_io_uring_setup, n, &p);
        if (fd < 0) return false;
        entries = p.sq_entries;
        sq_sz = p.sq_off.array + p.sq_entries * sizeof(unsigned);
        cq_sz = p.cq_off.cqes + p.cq_entries * sizeof(io_uring_cqe);
        const bool single = (p.features & IORING_FEAT_SINGLE_MMAP) != 0;
        if (single) sq_sz = cq_sz = std::max(sq_sz, cq_sz);
        sq_ptr = mmap(nullptr, sq_sz, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_SQ_RING);
        if (sq_ptr == MAP_FAILED) return false;
        cq_ptr = single ? sq_ptr
                        : mmap(nullptr, cq_sz, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_CQ_RING);
        if (cq_ptr == MAP_FAILED) return false;
        sqes_sz = p.sq_entries * sizeof(io_uring_sqe);
        sqes = (io_uring_sqe*)mmap(nullptr, sqes_sz, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd,
                                   IORING_OFF_SQES);
        if (sqes == MAP_FAILED) return false;
        char* sq = (char*)sq_ptr;
        char* cq = (char*)cq_ptr;
        sq_head = (unsigned*)(sq + p.sq_off.head);
        sq_tail = (unsigned*)(sq + p.sq_off.tail);
        sq_mask = (unsigned*)(sq + p.sq_off.ring_mask);
        sq_array = (unsigned*)(sq + p.sq_off.array);
        cq_head = (unsigned*)(cq + p.cq_off.head);
        cq_tail = (unsigned*)(cq + p.cq_off.tail);
        cq_mask = (unsigned*)(cq + p.cq_off.ring_mask);
        cqes = (io_uring_cqe*)(cq + p.cq_off.cqes);
        return true;
    }

    ~Uring() {
        if (sqes != MAP_FAILED) munmap(sqes, sqes_sz);
        if (cq_ptr != MAP_FAILED && cq_ptr != sq_ptr) munmap(cq_ptr, cq_sz);
        if (sq_ptr != MAP_FAILED) munmap(sq_ptr, sq_sz);
        if (fd >= 0) close(fd);
    }

    // Waits for `outstanding` submitted requests to complete, dropping their results.  When
    // waiting itself fails, asks the kernel to cancel everything in flight on the ring
    // (IORING_ASYNC_CANCEL_ANY) and waits again; false if that fails too.
    bool drain(unsigned outstanding) {
        int failures = 0;
        bool cancel_queued = false;
        while (outstanding > 0) {
            const unsigned submit = cancel_queued ? 1u : 0u;
            const int rc = (int)syscall(__NR_io_uring_enter, fd, submit, 1u, IORING_ENTER_GETEVENTS, nullptr, 0);
            if (rc < 0) {
                if (errno == EINTR || errno == EAGAIN || errno == EBUSY) continue;
                if (++failures > 4) return false;
                if (!cancel_queued) {
                    // entries queued but never submitted are dropped from the ring (no
                    // SQPOLL here: the kernel reads the tail only inside io_uring_enter), so
                    // the cancel request is the next entry the kernel sees
                    unsigned tail = __atomic_load_n(sq_head, __ATOMIC_ACQUIRE);
                    const unsigned idx = tail & *sq_mask;
                    io_uring_sqe* e = &sqes[idx];
                    memset(e, 0, sizeof *e);
                    e->opcode = IORING_OP_ASYNC_CANCEL;
                    e->fd = -1;
                    e->cancel_flags = kCancelAny;
                    e->user_data = kCancelTag;
                    sq_array[idx] = idx;
                    __atomic_store_n(sq_tail, tail + 1, __ATOMIC_RELEASE);
                    cancel_queued = true;
                }
                continue;
            }
            if (cancel_queued && rc > 0) cancel_queued = false;  // the cancel request went in
            unsigned head = __atomic_load_n(cq_head, __ATOMIC_RELAXED);
            const unsigned ctail = __atomic_load_n(cq_tail, __ATOMIC_ACQUIRE);
            while (head != ctail) {
                if (cqes[head & *cq_mask].user_data != kCancelTag && outstanding > 0) outstanding--;
                head++;
            }
            __atomic_store_n(cq_head, head, __ATOMIC_RELEASE);
        }
        return true;
    }

    // Reads `n` requests (each at most 1 GiB) into dst; 0 or -errno.  Every submitted entry
    // is completed and reaped before returning, also on error, so no request outlives the
    // call.
    int read_batch(int file, char* dst, const IoReq* reqs, size_t n, bool async, std::string* why) {
        size_t done = 0;
        int err = 0;
        while (done < n) {
            const unsigned batch = (unsigned)std::min<size_t>(n - done, entries);
            unsigned tail = __atomic_load_n(sq_tail, __ATOMIC_RELAXED);
            for (unsigned i = 0; i < batch; i++) {
                const IoReq& r = reqs[done + i];
                const unsigned idx = tail & *sq_mask;
                io_uring_sqe* e = &sqes[idx];
                memset(e, 0, sizeof *e);
                e->opcode = IORING_OP_READ;
                e->fd = file;
                e->addr = (uint64_t)(uintptr_t)(dst + r.start);
                e->len = (uint32_t)(r.end - r.start);
                e->off = r.offset;
                e->user_data = done + i;
                // large pieces go to the kernel's worker threads, so several cores copy
                // page-cache pages at once instead of the submitting thread alone
                if (async) e->flags = IOSQE_ASYNC;
                sq_array[idx] = idx;
                tail++;
            }
            __atomic_store_n(sq_tail, tail, __ATOMIC_RELEASE);
            unsigned submitted = 0, reaped = 0;
            while (reaped < batch) {
                const int rc = (int)syscall(__NR_io_uring_enter, fd, batch - submitted, batch - reaped,
                                            IORING_ENTER_GETEVENTS, nullptr, 0);
                if (rc < 0) {
                    if (errno == EINTR || errno == EAGAIN || errno == EBUSY) continue;
                    const int e = errno;
                    // Requests already submitted may still be copying into dst on the
                    // kernel's worker threads: wait for every one of them before returning,
                    // so none outlives the call.  The ring is then dropped by the caller
                    // (pread from then on).  Entries never submitted never run.
                    broken = true;
                    *why = "io_uring_enter failed";
                    if (!drain(submitted - reaped)) *why = "io_uring_enter failed; in-flight reads not confirmed";
                    return -e;
                }
                submitted += (unsigned)rc;
                unsigned head = __atomic_load_n(cq_head, __ATOMIC_RELAXED);
                const unsigned ctail = __atomic_load_n(cq_tail, __ATOMIC_ACQUIRE);
                while (head != ctail) {
                    const io_uring_cqe& c = cqes[head & *cq_mask];
                    const size_t k = (size_t)c.user_data;
                    if (!err) {
                        if (k < done || k >= done + batch) {
                            err = -EIO;
                            *why = "unexpected io_uring completion";
                        } else if (c.res < 0) {
                            err = c.res;
                            *why = "io_uring read failed";
                        } else if ((size_t)c.res != reqs[k].end - reqs[k].start) {
                            err = -EIO;
                            *why = "short read (file shorter than its tensor directory)";
                        }
                    }
                    head++;
                    reaped++;
                }
                __atomic_store_n(cq_head, head, __ATOMIC_RELEASE);
            }
            if (err) return err;
            done += batch;
        }
        return 0;
    }
};

struct WeightIo {
    int fd = -1;
    uint64_t size = 0;
    Uring* ring = nullptr;  // null: pread
    // io_uring piece size (HAYAI_IO_CHUNK_KB; 0: whole runs).  Page-cache reads of a 182 MB
    // layer pack on the MI355X host: whole runs 21 GB/s (one core copying), 1 MiB pieces
    // 55 GB/s, 256 KiB pieces 63 GB/s.
    size_t chunk = (size_t)256 << 10;
    std::string path;
    // HAYAI_O_DIRECT (iouring_reader.rs:36-50, weight_io.rs:243-263,329-405): a second
    // descriptor opened with O_DIRECT, so reads bypass the page cache (cold reads from the
    // device itself).  Direct reads need offsets, lengths and buffers aligned to the logical
    // block size: each run is read as its 4096-aligned cover into an aligned bounce buffer
    // and copied out.  A run whose cover crosses an unaligned end of file, or a failed
    // direct read, switches the catalog to page-cache reads for good, as the reference does.
    static constexpr uint64_t kDirectAlign = 4096;
    int dfd = -1;
    void* bounce = nullptr;
    size_t bounce_cap = 0;

    ~WeightIo() {
        delete ring;
        if (fd >= 0) close(fd);
        drop_direct();
    }

    void drop_direct() {
        if (dfd >= 0) close(dfd);
        dfd = -1;
        free(bounce);
        bounce = nullptr;
        bounce_cap = 0;
    }

    // One run [off, off + len) -> dst through O_DIRECT; false (nothing written to dst) when
    // the run cannot be served that way.
    bool read_direct(uint64_t off, char* dst, size_t len) {
        const uint64_t a0 = off & ~(kDirectAlign - 1);
        const uint64_t a1 = (off + len + kDirectAlign - 1) & ~(kDirectAlign - 1);
        if (a1 > size) return false;  // the cover would cross an unaligned end of file
        const size_t n = (size_t)(a1 - a0);
        if (n > bounce_cap) {
            free(bounce);
            bounce = nullptr;
            bounce_cap = 0;
            if (posix_memalign(&bounce, kDirectAlign, n) != 0) {
                bounce = nullptr;
                return false;
            }
            bounce_cap = n;
        }
        char* b = (char*)bounce;
        const size_t piece = ring && chunk ? chunk : ((size_t)1 << 30);  // chunk is a multiple of 4096
        if (ring && piece % kDirectAlign == 0) {
            std::vector<IoReq> pieces;
            for (size_t s = 0; s < n; s += piece) pieces.push_back({a0 + s, s, std::min(n, s + piece)});
            std::string why;
            if (ring->read_batch(dfd, b, pieces.data(), pieces.size(), pieces.size() > 1, &why) != 0) {
                if (ring->broken) {
                    delete ring;
                    ring = nullptr;
                }
                return false;
            }
        } else {
            size_t done = 0;
            while (done < n) {
                const ssize_t r = pread(dfd, b + done, std::min<size_t>(n - done, (size_t)1 << 30), (off_t)(a0 + done));
                if (r < 0 && errno == EINTR) continue;
                if (r <= 0 || ((size_t)r % kDirectAlign != 0 && done + (size_t)r < n)) return false;
                done += (size_t)r;
            }
        }
        memcpy(dst, b + (off - a0), len);
        return true;
    }

    hh_status open_file(const char* p) {
        path = p;
        fd = ::open(p, O_RDONLY | O_CLOEXEC);
        if (fd < 0) return fail(HH_ERR_IO, "gguf: cannot open %s: %s", p, strerror(errno));
        struct stat st;
        if (fstat(fd, &st) != 0) return fail(HH_ERR_IO, "gguf: fstat %s: %s", p, strerror(errno));
        size = (uint64_t)st.st_size;
        if (const char* c = getenv("HAYAI_IO_CHUNK_KB")) chunk = (size_t)std::max(0, atoi(c)) << 10;
        if (getenv("HAYAI_O_DIRECT")) {
            dfd = ::open(p, O_RDONLY | O_CLOEXEC | O_DIRECT);  // refused (tmpfs...): page cache
            if (dfd < 0) dfd = -1;
        }
        const char* force = getenv("HAYAI_FORCE_FILE_IO");
        if (!(force && *force && strcmp(force, "0") != 0)) {
            ring = new (std::nothrow) Uring;
            if (ring && !ring->setup(256)) {
                delete ring;  // io_uring refused here (seccomp, sysctl): positioned reads
                ring = nullptr;
            }
        }
        return HH_OK;
    }

    hh_status read_at(uint64_t off, void* buf, size_t len) {
        size_t done = 0;
        while (done < len) {
            const ssize_t n = pread(fd, (char*)buf + done, std::min<size_t>(len - done, (size_t)1 << 30),
                                    (off_t)(off + done));
            if (n < 0) {
                if (errno == EINTR) continue;
                return fail(HH_ERR_IO, "gguf: read %s at %llu: %s", path.c_str(), (unsigned long long)(off + done),
                            strerror(errno));
            }
            if (n == 0)
                return fail(HH_ERR_IO, "gguf: short read of %s at %llu (file is %llu bytes)", path.c_str(),
                            (unsigned long long)(off + done), (unsigned long long)size);
            done += (size_t)n;
        }
        return HH_OK;
    }

    // read_many_at (weight_io.rs:26-49,51-85): ranges inside dst and disjoint; runs
    // contiguous in both the file and dst coalesce into one read; io_uring submits them all.
    hh_status read_many(void* dst, size_t dst_len, std::vector<IoReq> reqs) {
        for (const IoReq& r : reqs)
            if (r.start > r.end || r.end > dst_len)
                return fail(HH_ERR_INVALID, "io range %zu..%zu out of bounds for buffer of %zu", r.start, r.end,
                            dst_len);
        std::vector<IoReq> order = reqs;
        std::sort(order.begin(), order.end(), [](const IoReq& a, const IoReq& b) { return a.start < b.start; });
        for (size_t i = 1; i < order.size(); i++)
            if (order[i - 1].end > order[i].start) return fail(HH_ERR_INVALID, "overlapping io ranges");
        std::vector<IoReq> whole;  // runs contiguous in the file and in dst, coalesced
        for (size_t i = 0; i < reqs.size();) {
            size_t j = i;
            while (j + 1 < reqs.size() && reqs[j].offset + (reqs[j].end - reqs[j].start) == reqs[j + 1].offset &&
                   reqs[j].end == reqs[j + 1].start)
                j++;
            whole.push_back({reqs[i].offset, reqs[i].start, reqs[j].end});
            i = j + 1;
        }
        for (const IoReq& r : whole)
            if (r.offset > size || r.end - r.start > size - r.offset)
                return fail(HH_ERR_IO, "gguf: read of %zu bytes at %llu past the end of %s (%llu bytes)",
                            r.end - r.start, (unsigned long long)r.offset, path.c_str(), (unsigned long long)size);
        size_t first = 0;  // runs before this one were read directly
        while (dfd >= 0 && first < whole.size()) {
            const IoReq& r = whole[first];
            if (r.end > r.start && !read_direct(r.offset, (char*)dst + r.start, r.end - r.start)) {
                drop_direct();  // page-cache reads from now on (weight_io.rs:388-400)
                break;
            }
            first++;
        }
        std::vector<IoReq> runs;
        const size_t piece = ring && chunk ? chunk : (size_t)1 << 30;
        for (size_t i = first; i < whole.size(); i++) {
            // split into pieces of at most `piece` bytes (one read returns at most ~2 GiB;
            // io_uring reads large runs as parallel pieces)
            for (size_t s = whole[i].start; s < whole[i].end; s += piece)
                runs.push_back({whole[i].offset + (s - whole[i].start), s, std::min(whole[i].end, s + piece)});
        }
        if (runs.empty()) return HH_OK;
        if (ring) {
            std::string why;
            const int rc = ring->read_batch(fd, (char*)dst, runs.data(), runs.size(), chunk != 0 && runs.size() > 1, &why);
            if (rc != 0) {
                if (ring->broken) {
                    delete ring;
                    ring = nullptr;
                }
                return fail(HH_ERR_IO, "gguf: %s on %s: %s", why.c_str(), path.c_str(), strerror(-rc));
            }
            return HH_OK;
        }
        for (const IoReq& r : runs) HH_TRY(read_at(r.offset, (char*)dst + r.start, r.end - r.start));
        return HH_OK;
    }
};

// ------------------------------------------------------------------- header parse -------

enum : uint32_t { MV_U8, MV_I8, MV_U16, MV_I16, MV_U32, MV_I32, MV_F32, MV_BOOL, MV_STR, MV_ARR, MV_U64, MV_I64, MV_F64 };

// A metadata value as read (MetadataValue, gguf_types.rs:82-98); arrays keep their element
// type and length (their items are validated but not kept).
struct MetaValue {
    uint32_t type = 0;
    uint64_t u = 0;  // unsigned scalars and bool
    int64_t i = 0;   // signed scalars
    double f = 0;    // f32 / f64
    std::string s;
    uint32_t elem = 0;
    uint64_t len = 0;
};

struct TensorRec {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t nbytes = 0;
};

enum class Parse { ok, truncated, bad };

// Strings of the file as String::from_utf8_lossy makes them (gguf.rs:620-626): every maximal
// prefix of an invalid UTF-8 sequence becomes one U+FFFD, so names and keys compare as the
// reference's do.
static std::string utf8_lossy(const uint8_t* p, size_t n) {
    std::string out;
    out.reserve(n);
    size_t i = 0;
    while (i < n) {
        const uint8_t c = p[i];
        if (c < 0x80) {
            out.push_back((char)c);
            i++;
            continue;
        }
        size_t need = 0;
        uint8_t lo = 0x80, hi = 0xBF;  // range of the second byte
        if (c >= 0xC2 && c <= 0xDF) {
            need = 1;
        } else if (c >= 0xE0 && c <= 0xEF) {
            need = 2;
            if (c == 0xE0) lo = 0xA0;
            if (c == 0xED) hi = 0x9F;
        } else if (c >= 0xF0 && c <= 0xF4) {
            need = 3;
            if (c == 0xF0) lo = 0x90;
            if (c == 0xF4) hi = 0x8F;
        }
        size_t k = 1;  // bytes of the sequence seen to be valid so far
        bool ok = need > 0;
        for (size_t j = 1; ok && j <= need; j++) {
            if (i + j >= n) {
                ok = false;
                break;
            }
            const uint8_t b = p[i + j];
            const uint8_t l = j == 1 ? lo : 0x80, h = j == 1 ? hi : 0xBF;
            if (b < l || b > h) {
                ok = false;
                break;
            }
            k++;
        }
        if (ok) {
            out.append((const char*)p + i, need + 1);
            i += need + 1;
        } else {
            out.append("\xEF\xBF\xBD");
            i += k;
        }
    }
    return out;
}

struct Reader {
    const uint8_t* p;
    size_t len, pos = 0;
    std::string err;
    bool trunc = false;

    bool need(size_t n, const char* what) {
        if (n <= len - pos) return true;
        if (err.empty()) err = std::string("truncated: ") + what;
        trunc = true;
        return false;
    }
    template <class T>
    bool get(T* v, const char* what) {
        if (!need(sizeof(T), what)) return false;
        memcpy(v, p + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool str(std::string* s, const char* what) {
        uint64_t n;
        if (!get(&n, what)) return false;
        if (!need((size_t)n, what)) return false;
        *s = utf8_lossy(p + pos, (size_t)n);
        pos += (size_t)n;
        return true;
    }
    bool bad(const std::string& m) {
        if (err.empty()) err = m;
        return false;
    }
    // read_value (gguf.rs:633-676): nested arrays up to depth 32, lengths bounded by the bytes
    // left (each element takes at least one byte)
    bool value(uint32_t ty, int depth, MetaValue* out) {
        if (depth > 32) {
            trunc = false;
            return bad("metadata array nesting too deep");
        }
        MetaValue v;
        v.type = ty;
        switch (ty) {
            case MV_U8: { uint8_t x; if (!get(&x, "metadata")) return false; v.u = x; break; }
            case MV_I8: { int8_t x; if (!get(&x, "metadata")) return false; v.i = x; break; }
            case MV_U16: { uint16_t x; if (!get(&x, "metadata")) return false; v.u = x; break; }
            case MV_I16: { int16_t x; if (!get(&x, "metadata")) return false; v.i = x; break; }
            case MV_U32: { uint32_t x; if (!get(&x, "metadata")) return false; v.u = x; break; }
            case MV_I32: { int32_t x; if (!get(&x, "metadata")) return false; v.i = x; break; }
            case MV_F32: { float x; if (!get(&x, "metadata")) return false; v.f = x; break; }
            case MV_BOOL: { uint8_t x; if (!get(&x, "metadata")) return false; v.u = x != 0; break; }
            case MV_STR: if (!str(&v.s, "metadata string")) return false; break;
            case MV_ARR: {
                uint32_t et;
                uint64_t n;
                if (!get(&et, "metadata array") || !get(&n, "metadata array")) return false;
                if (n > (uint64_t)(len - pos)) {
                    trunc = true;
                    return bad("truncated: metadata array length");
                }
                v.elem = et;
                v.len = n;
                for (uint64_t k = 0; k < n; k++) {
                    MetaValue item;
                    if (!value(et, depth + 1, &item)) return false;
                }
                break;
            }
            case MV_U64: { uint64_t x; if (!get(&x, "metadata")) return false; v.u = x; break; }
            case MV_I64: { int64_t x; if (!get(&x, "metadata")) return false; v.i = x; break; }
            case MV_F64: { double x; if (!get(&x, "metadata")) return false; v.f = x; break; }
            default: {
                char m[64];
                snprintf(m, sizeof m, "unknown metadata type %u", ty);
                return bad(m);
            }
        }
        if (out) *out = std::move(v);
        return true;
    }
};

// MetadataValue::as_u64 / as_u32 / as_f32 (gguf_types.rs:100-128)
static bool as_u64(const MetaValue& v, uint64_t* out) {
    switch (v.type) {
        case MV_U64: case MV_U32: *out = v.u; return true;
        case MV_I64: case MV_I32: if (v.i < 0) return false; *out = (uint64_t)v.i; return true;
        default: return false;
    }
}
static bool as_u32(const MetaValue& v, uint32_t* out) {
    switch (v.type) {
        case MV_U32: case MV_U16: case MV_U8: *out = (uint32_t)v.u; return true;
        case MV_U64: if (v.u > UINT32_MAX) return false; *out = (uint32_t)v.u; return true;
        case MV_I32: case MV_I64: if (v.i < 0 || v.i > (int64_t)UINT32_MAX) return false; *out = (uint32_t)v.i; return true;
        default: return false;
    }
}

// Block geometry per GGML type (tensor_nbytes, gguf.rs:240-284); false: no size rule.
static bool type_geom(uint32_t t, uint64_t* block, uint64_t* bytes) {
    struct G { uint32_t t; uint64_t block, bytes; };
    static const G g[] = {
        {0, 1, 4},     {1, 1, 2},     {30, 1, 2},    {28, 1, 8},    {27, 1, 8},    {24, 1, 1},
        {25, 1, 2},    {26, 1, 4},    {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},
        {8, 32, 34},   {9, 32, 36},   {20, 32, 18},  {10, 256, 84}, {11, 256, 110}, {12, 256, 144},
        {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74}, {22, 256, 82},
        {18, 256, 98}, {21, 256, 110}, {19, 256, 50}, {29, 256, 56}, {23, 256, 136}, {34, 256, 54},
        {35, 256, 66},
    };
    for (const G& x : g)
        if (x.t == t) {
            *block = x.block;
            *bytes = x.bytes;
            return true;
        }
    return false;
}

// tensor_nbytes with checked arithmetic: element product, ceil(n / block) * block bytes.
static hh_status nbytes_of(uint32_t type, const uint64_t* dims, uint32_t n_dims, const char* name, uint64_t* out) {
    uint64_t n = 1;
    for (uint32_t k = 0; k < n_dims; k++) {
        if (dims[k] != 0 && n > UINT64_MAX / dims[k]) return fail(HH_ERR_INVALID, "tensor %s element count overflow", name);
        n *= dims[k];
    }
    uint64_t block, bytes;
    if (!type_geom(type, &block, &bytes))
        return fail(HH_ERR_KERNEL_MISSING, "tensor %s has unsupported GGML type %u", name, type);
    const uint64_t nb = n / block + (n % block != 0);
    if (nb > UINT64_MAX / bytes) return fail(HH_ERR_INVALID, "tensor %s byte size overflow", name);
    *out = nb * bytes;
    return HH_OK;
}

}  // namespace hh

using namespace hh;

struct hh_gguf {
    WeightIo io;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    size_t header_bytes = 0;
    std::unordered_map<std::string, MetaValue> meta;
    std::vector<TensorRec> tensors;
    std::unordered_map<std::string, size_t> index;
};

// parse_header_bytes (gguf.rs:25-127) over a prefix of the file.
static Parse parse_header(const uint8_t* data, size_t len, hh_gguf* g, std::string* why) {
    Reader r{data, len, 0, std::string(), false};
    uint32_t magic;
    auto done = [&](bool ok) {
        *why = r.err;
        return ok ? Parse::ok : (r.trunc ? Parse::truncated : Parse::bad);
    };
    if (!r.get(&magic, "magic")) return done(false);
    if (magic != 0x46554747u) return r.bad("invalid GGUF magic"), done(false);
    if (!r.get(&g->version, "version")) return done(false);
    if (g->version < 1 || g->version > 4) {
        char m[64];
        snprintf(m, sizeof m, "unsupported GGUF version %u", g->version);
        return r.bad(m), done(false);
    }
    uint64_t n_tensors, n_kv;
    if (!r.get(&n_tensors, "tensor count") || !r.get(&n_kv, "metadata count")) return done(false);
    const uint64_t remaining = len - r.pos;
    // counts bounded by the bytes left (gguf.rs:38-48); a longer prefix may still hold them
    if (n_kv > remaining / 8 + 1) {
        r.trunc = true;
        return r.bad("truncated: metadata count exceeds file size"), done(false);
    }
    if (n_tensors > remaining / 8 + 1) {
        r.trunc = true;
        return r.bad("truncated: tensor count exceeds file size"), done(false);
    }
    g->meta.clear();
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key;
        uint32_t ty;
        MetaValue v;
        if (!r.str(&key, "metadata key") || !r.get(&ty, "metadata type") || !r.value(ty, 0, &v)) return done(false);
        g->meta[key] = std::move(v);  // a repeated key keeps the last value (HashMap::insert)
    }
    g->tensors.clear();
    g->index.clear();
    for (uint64_t k = 0; k < n_tensors; k++) {
        TensorRec t;
        if (!r.str(&t.name, "tensor name") || !r.get(&t.n_dims, "tensor dims")) return done(false);
        if (t.n_dims > 4) return r.bad("tensor " + t.name + " has " + std::to_string(t.n_dims) + " dims"), done(false);
        for (uint32_t d = 0; d < t.n_dims; d++) {
            if (!r.get(&t.dims[d], "tensor dims")) return done(false);
            if (t.dims[d] == 0) return r.bad("tensor " + t.name + " has a zero dimension"), done(false);
        }
        if (!r.get(&t.type, "tensor type") || !r.get(&t.offset, "tensor offset")) return done(false);
        if (nbytes_of(t.type, t.dims, t.n_dims, t.name.c_str(), &t.nbytes) != HH_OK)
            return r.bad(last_error()), done(false);
        if (!g->index.emplace(t.name, (size_t)k).second)
            return r.bad("duplicate tensor name " + t.name), done(false);
        g->tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    auto it = g->meta.find("general.alignment");
    if (it != g->meta.end()) {
        uint64_t a;
        if (as_u64(it->second, &a)) align = a;
    }
    if (align == 0 || (align & (align - 1)) != 0)
        return r.bad("invalid general.alignment " + std::to_string(align) + " (must be a non-zero power of two)"),
               done(false);
    g->alignment = align;
    const uint64_t pos = r.pos, rem = pos % align;
    if (rem && pos > UINT64_MAX - (align - rem)) return r.bad("alignment overflow"), done(false);
    g->data_offset = rem ? pos + (align - rem) : pos;
    for (const TensorRec& t : g->tensors) {
        if (t.offset > UINT64_MAX - g->data_offset) return r.bad("tensor " + t.name + " absolute offset overflow"), done(false);
        if (t.nbytes > UINT64_MAX - (g->data_offset + t.offset))
            return r.bad("tensor " + t.name + " byte range overflow"), done(false);
    }
    g->header_bytes = r.pos;
    return done(true);
}

extern "C" {

hh_status hh_gguf_open(const char* path, hh_gguf** out) {
    if (!out) return fail(HH_ERR_INVALID, "hh_gguf_open: out is null");
    *out = nullptr;
    if (!path) return fail(HH_ERR_INVALID, "hh_gguf_open: path is null");
    hh_gguf* g = new (std::nothrow) hh_gguf;
    if (!g) return fail(HH_ERR_OUT_OF_MEMORY, "hh_gguf_open: allocation failed");
    hh_status st = g->io.open_file(path);
    if (st != HH_OK) {
        delete g;
        return st;
    }
    // parse_header_from_start (gguf_stream.rs:159-192): a prefix that doubles until the
    // directory fits, up to 64 MiB or the file's length
    const uint64_t cap = std::min<uint64_t>(g->io.size, (uint64_t)64 << 20);
    size_t size = (size_t)std::min<uint64_t>(cap, (uint64_t)1 << 20);
    std::vector<uint8_t> buf;
    for (;;) {
        buf.resize(size);
        st = g->io.read_at(0, buf.data(), size);
        if (st != HH_OK) break;
        std::string why;
        const Parse p = parse_header(buf.data(), size, g, &why);
        if (p == Parse::ok) {
            *out = g;
            return HH_OK;
        }
        if (p == Parse::truncated && size < cap) {
            size = (size_t)std::min<uint64_t>(cap, (uint64_t)size * 2);
            continue;
        }
        st = fail(p == Parse::truncated ? HH_ERR_IO : HH_ERR_INVALID, "gguf %s: %s", path, why.c_str());
        break;
    }
    delete g;
    return st;
}

void hh_gguf_close(hh_gguf* g) { delete g; }

hh_status hh_gguf_header(const hh_gguf* g, hh_gguf_info* out) {
    if (!g || !out) return fail(HH_ERR_INVALID, "hh_gguf_header: null argument");
    out->version = g->version;
    out->io_uring = g->io.ring != nullptr;
    out->o_direct = g->io.dfd >= 0;
    out->alignment = g->alignment;
    out->data_offset = g->data_offset;
    out->header_bytes = g->header_bytes;
    out->n_tensors = g->tensors.size();
    out->n_metadata = g->meta.size();
    out->file_size = g->io.size;
    return HH_OK;
}

static void fill_tensor(const hh_gguf* g, const TensorRec& t, hh_gguf_tensor* out) {
    out->name = t.name.c_str();
    out->n_dims = t.n_dims;
    out->type = t.type;
    for (int k = 0; k < 4; k++) out->dims[k] = t.dims[k];
    out->offset = t.offset;
    out->abs_offset = g->data_offset + t.offset;
    out->nbytes = t.nbytes;
}

hh_status hh_gguf_tensor_at(const hh_gguf* g, uint64_t i, hh_gguf_tensor* out) {
    if (!g || !out) return fail(HH_ERR_INVALID, "hh_gguf_tensor_at: null argument");
    if (i >= g->tensors.size()) return fail(HH_ERR_INVALID, "tensor index %llu of %zu", (unsigned long long)i, g->tensors.size());
    fill_tensor(g, g->tensors[i], out);
    return HH_OK;
}

hh_status hh_gguf_find(const hh_gguf* g, const char* name, hh_gguf_tensor* out) {
    if (!g || !name || !out) return fail(HH_ERR_INVALID, "hh_gguf_find: null argument");
    auto it = g->index.find(name);
    if (it == g->index.end()) return fail(HH_ERR_NOT_FOUND, "missing tensor %s", name);
    fill_tensor(g, g->tensors[it->second], out);
    return HH_OK;
}

static const MetaValue* meta_of(const hh_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

hh_status hh_gguf_meta_u64(const hh_gguf* g, const char* key, uint64_t* out) {
    const MetaValue* v = meta_of(g, key);
    if (!v || !out || !as_u64(*v, out)) return fail(HH_ERR_NOT_FOUND, "no unsigned metadata value %s", key ? key : "(null)");
    return HH_OK;
}

hh_status hh_gguf_meta_u32(const hh_gguf* g, const char* key, uint32_t* out) {
    const MetaValue* v = meta_of(g, key);
    if (!v || !out || !as_u32(*v, out)) return fail(HH_ERR_NOT_FOUND, "no u32 metadata value %s", key ? key : "(null)");
    return HH_OK;
}

hh_status hh_gguf_meta_f32(const hh_gguf* g, const char* key, float* out) {
    const MetaValue* v = meta_of(g, key);
    if (!v || !out || (v->type != MV_F32 && v->type != MV_F64))
        return fail(HH_ERR_NOT_FOUND, "no float metadata value %s", key ? key : "(null)");
    *out = (float)v->f;
    return HH_OK;
}

hh_status hh_gguf_meta_str(const hh_gguf* g, const char* key, const char** out, size_t* len) {
    const MetaValue* v = meta_of(g, key);
    if (!v || !out || !len || v->type != MV_STR)
        return fail(HH_ERR_NOT_FOUND, "no string metadata value %s", key ? key : "(null)");
    *out = v->s.data();
    *len = v->s.size();
    return HH_OK;
}

hh_status hh_tensor_nbytes(uint32_t type, const uint64_t* dims, uint32_t n_dims, uint64_t* out) {
    if (!out || (n_dims && !dims) || n_dims > 4) return fail(HH_ERR_INVALID, "hh_tensor_nbytes: bad arguments");
    return nbytes_of(type, dims, n_dims, "(query)", out);
}

// The layer pack layout of load_layer_pack_into (gguf_stream.rs:451-638): attn_q, attn_k,
// attn_v, attn_output, ffn_gate, ffn_up, ffn_down and an optional attn_gate, back to back in
// that order.  A fused gate/up tensor (ffn_gate_up, or Phi-3's ffn_up with twice down's
// columns as rows; gguf_stream.rs:381-397) is read once in the gate slot and split in rows;
// a layer without attn_v (V = K) or without ffn_gate (ungated FFN) gets a zero-length region;
// any other missing tensor is an error.
static hh_status pack_layout(const hh_gguf* g, size_t layer, hh_layer_pack* out, std::vector<IoReq>* reqs) {
    static const char* kNames[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    memset(out, 0, sizeof *out);
    auto find = [&](const std::string& n) -> const TensorRec* {
        auto it = g->index.find(n);
        return it == g->index.end() ? nullptr : &g->tensors[it->second];
    };
    const std::string pre = "blk." + std::to_string(layer) + ".";
    const TensorRec* fused = nullptr;
    if (!find(pre + "ffn_gate.weight")) {
        fused = find(pre + "ffn_gate_up.weight");
        if (!fused) {
            const TensorRec* up = find(pre + "ffn_up.weight");
            const TensorRec* dn = find(pre + "ffn_down.weight");
            const uint64_t up_rows = up && up->n_dims >= 2 ? up->dims[1] : 1;
            if (up && dn && dn->dims[0] > 0 && up_rows == 2 * dn->dims[0]) fused = up;
        }
    }
    out->fused_gate_up = fused != nullptr;
    size_t off = 0;
    auto place = [&](int slot, const TensorRec& t) {
        out->off[slot] = off;
        out->len[slot] = (size_t)t.nbytes;
        out->type[slot] = t.type;
        out->cols[slot] = t.dims[0];
        out->rows[slot] = t.n_dims >= 2 ? t.dims[1] : 1;
        if (reqs) reqs->push_back({g->data_offset + t.offset, off, off + (size_t)t.nbytes});
        off += (size_t)t.nbytes;
    };
    for (int i = 0; i < 7; i++) {
        if (i == 5 && fused) continue;  // up is the second half of the fused tensor
        if (i == 4 && fused) {
            const uint64_t rows = fused->n_dims >= 2 ? fused->dims[1] : 1;
            place(4, *fused);
            out->len[4] = out->len[5] = (size_t)fused->nbytes / 2;
            out->off[5] = out->off[4] + out->len[4];
            out->rows[4] = out->rows[5] = rows / 2;
            out->cols[5] = out->cols[4];
            out->type[5] = out->type[4];
            continue;
        }
        const TensorRec* t = find(pre + kNames[i] + ".weight");
        if (t) {
            place(i, *t);
        } else if (i == 2 || i == 4) {
            out->off[i] = off;  // V = K layer / ungated FFN: nothing to read
        } else {
            return fail(HH_ERR_NOT_FOUND, "missing tensor %s%s.weight", pre.c_str(), kNames[i]);
        }
    }
    if (const TensorRec* t = find(pre + "attn_gate.weight")) place(7, *t);
    out->total = off;
    return HH_OK;
}

hh_status hh_gguf_layer_pack(const hh_gguf* g, size_t layer, hh_layer_pack* out) {
    if (!g || !out) return fail(HH_ERR_INVALID, "hh_gguf_layer_pack: null argument");
    return pack_layout(g, layer, out, nullptr);
}

hh_status hh_gguf_load_layer_pack(hh_gguf* g, size_t layer, void* dst, size_t dst_len, hh_layer_pack* out) {
    if (!g || !out || (!dst && dst_len)) return fail(HH_ERR_INVALID, "hh_gguf_load_layer_pack: null argument");
    std::vector<IoReq> reqs;
    HH_TRY(pack_layout(g, layer, out, &reqs));
    if (out->total > dst_len)
        return fail(HH_ERR_INVALID, "layer %zu pack of %zu B exceeds the destination's %zu B", layer, out->total, dst_len);
    return g->io.read_many(dst, dst_len, std::move(reqs));
}

hh_status hh_gguf_read_tensor(hh_gguf* g, const char* name, void* dst, size_t dst_len) {
    if (!g || !name || (!dst && dst_len)) return fail(HH_ERR_INVALID, "hh_gguf_read_tensor: null argument");
    auto it = g->index.find(name);
    if (it == g->index.end()) return fail(HH_ERR_NOT_FOUND, "missing tensor %s", name);
    const TensorRec& t = g->tensors[it->second];
    if (t.nbytes > dst_len) return fail(HH_ERR_INVALID, "tensor %s of %llu B exceeds the destination's %zu B", name,
                                        (unsigned long long)t.nbytes, dst_len);
    return g->io.read_many(dst, dst_len, {{g->data_offset + t.offset, 0, (size_t)t.nbytes}});
}

}  // extern "C"
