// Host-only driver for the GGUF catalog under AddressSanitizer + UndefinedBehaviorSanitizer
// (built with g++ by tests/test_gguf_sanitizer.py together with runtime/gguf.cpp; no GPU code
// and no HIP runtime).  For every file named on the command line: open it, walk the tensor
// directory, the metadata accessors and the layer-pack layouts of layers 0 and 1, read each
// tensor of at most 1 MiB (through io_uring, or positioned reads with HAYAI_FORCE_FILE_IO=1)
// and close it.  Prints "opened N rejected M".
#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

#include "hayai_hip.h"
#include "../../hayai_amd/csrc/runtime/engine.h"

// The library's error sink (capi.cpp in the full build): keep the last message.
namespace hh {
static std::string g_last;
hh_status fail(hh_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last = buf;
    return st;
}
const std::string& last_error() { return g_last; }
}  // namespace hh

int main(int argc, char** argv) {
    int opened = 0, rejected = 0;
    std::vector<unsigned char> buf;
    for (int i = 1; i < argc; i++) {
        hh_gguf* g = nullptr;
        if (hh_gguf_open(argv[i], &g) != HH_OK) {
            rejected++;
            continue;
        }
        opened++;
        hh_gguf_info info{};
        if (hh_gguf_header(g, &info) == HH_OK) {
            for (uint64_t t = 0; t < info.n_tensors; t++) {
                hh_gguf_tensor ti{};
                if (hh_gguf_tensor_at(g, t, &ti) != HH_OK) continue;
                hh_gguf_tensor tf{};
                hh_gguf_find(g, ti.name, &tf);
                if (ti.nbytes <= (1u << 20)) {
                    buf.assign(ti.nbytes ? ti.nbytes : 1, 0);
                    hh_gguf_read_tensor(g, ti.name, buf.data(), buf.size());
                }
            }
            uint32_t u32;
            uint64_t u64;
            float f32;
            const char* s;
            size_t n;
            for (size_t layer = 0; layer < 2; layer++) {
                hh_layer_pack lp{};
                hh_gguf_layer_pack(g, layer, &lp);
            }
            for (const char* key : {"general.architecture", "n", "arr", "s", "missing"}) {
                hh_gguf_meta_u32(g, key, &u32);
                hh_gguf_meta_u64(g, key, &u64);
                hh_gguf_meta_f32(g, key, &f32);
                hh_gguf_meta_str(g, key, &s, &n);
            }
        }
        hh_gguf_close(g);
    }
    printf("opened %d rejected %d\n", opened, rejected);
    return 0;
}
