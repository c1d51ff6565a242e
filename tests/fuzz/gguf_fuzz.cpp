// gguf_fuzz.cpp — mutation fuzzer of the GGUF reader's host-only entry
// points (vx_gguf_open and every query), built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_gguf_sanitized.py. Test
// infrastructure: it links vx_gguf.cpp and vx_layout.cpp alone and supplies
// the error-reporting functions and vx_device_info that libvortx_hip.so
// defines in vx_host.cpp, so no code object or GPU is needed.
//
// usage: gguf_fuzz <seed.gguf> <iterations> <rng seed> <scratch file>
// Each iteration mutates the seed (byte flips, 8-byte overwrites with
// boundary values, truncation, insertion, duplication of a span), writes it
// to the scratch file, opens it and, when it opens, walks the header, every
// tensor (by index and by name) and every key (by index, by name, every
// string element). A sanitizer report aborts the run; exit 0 otherwise.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "vortx_gguf.h"
#include "vx_internal.hpp"

namespace vx {
static thread_local std::string g_msg;
int fail(int status, const char* msg) {
    g_msg = msg ? msg : "";
    return status;
}
int fail_hip(int, const char* what) {
    g_msg = what ? what : "";
    return VX_ERR_HIP;
}
void clear_error() { g_msg.clear(); }
}  // namespace vx

// vx_gguf_upload (never called here) asks the context for its device
extern "C" int vx_device_info(vx_ctx, int*, int*) { return VX_ERR_INVALID; }

static void walk(vx_gguf f) {
    vx_gguf_header h{};
    if (vx_gguf_get_header(f, &h) != VX_OK) std::abort();
    for (uint64_t i = 0; i < h.n_tensors; ++i) {
        vx_gguf_tensor t{};
        if (vx_gguf_tensor_info(f, i, &t) != VX_OK) std::abort();
        uint64_t j = ~0ull;
        if (vx_gguf_find_tensor(f, t.name, &j) != VX_OK) std::abort();
        if (t.size_known && t.nbytes) {
            // touch the first and last data byte inside the mapping
            volatile uint8_t s = ((const uint8_t*)t.data)[0];
            s = ((const uint8_t*)t.data)[t.nbytes - 1];
            (void)s;
        }
        vx_qweight q{};
        (void)vx_gguf_qweight(f, i, (const void*)0x1000, &q);
        vx_cview v{};
        (void)vx_gguf_view(f, i, (const void*)0x1000, &v);
    }
    for (uint64_t i = 0; i < h.n_kv; ++i) {
        vx_gguf_kv kv{};
        if (vx_gguf_kv_info(f, i, &kv) != VX_OK) std::abort();
        uint64_t j = ~0ull;
        if (vx_gguf_find_key(f, kv.key, &j) != VX_OK) std::abort();
        if (kv.nbytes) {
            volatile uint8_t s = ((const uint8_t*)kv.data)[kv.nbytes - 1];
            (void)s;
        }
        if (kv.elem_type == VX_GGUF_STRING) {
            const uint64_t n = kv.type == VX_GGUF_ARRAY ? kv.count : 1;
            for (uint64_t e = 0; e < n && e < 64; ++e) {
                const char* str = nullptr;
                uint64_t len = 0;
                if (vx_gguf_kv_string(f, i, e, &str, &len) != VX_OK) std::abort();
                if (len) {
                    volatile char c = str[len - 1];
                    (void)c;
                }
            }
        }
    }
}

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s seed.gguf iterations rng-seed scratch\n", argv[0]);
        return 2;
    }
    FILE* in = std::fopen(argv[1], "rb");
    if (!in) return 2;
    std::vector<uint8_t> seed;
    for (int c; (c = std::fgetc(in)) != EOF;) seed.push_back((uint8_t)c);
    std::fclose(in);
    const long iters = std::atol(argv[2]);
    std::mt19937_64 rng(std::strtoull(argv[3], nullptr, 10));
    const uint64_t specials[] = {0, 1, 2, 3, 4, 7, 8, 31, 32, 0x7F, 0xFF, 0x7FFFFFFF, 0x80000000u, 0xFFFFFFFFu,
                                 0xFFFFFFFFFFFFFFFFull, 0x8000000000000000ull, 0x100000000ull, 1ull << 40};
    long opened = 0;
    for (long it = 0; it < iters; ++it) {
        std::vector<uint8_t> d = seed;
        const int nmut = 1 + (int)(rng() % 4);
        for (int m = 0; m < nmut && !d.empty(); ++m) {
            const uint64_t pos = rng() % d.size();
            switch (rng() % 6) {
            case 0: d[pos] ^= (uint8_t)(1u << (rng() % 8)); break;
            case 1: d[pos] = (uint8_t)rng(); break;
            case 2: {  // 8-byte boundary value
                const uint64_t v = specials[rng() % (sizeof specials / sizeof specials[0])];
                for (int b = 0; b < 8 && pos + b < d.size(); ++b) d[pos + b] = (uint8_t)(v >> (8 * b));
                break;
            }
            case 3: d.resize(pos); break;  // truncate
            case 4: d.insert(d.begin() + (long)pos, (size_t)(1 + rng() % 16), (uint8_t)rng()); break;
            default: {  // duplicate a span
                const uint64_t len = 1 + rng() % 64, src = rng() % d.size();
                std::vector<uint8_t> span(d.begin() + (long)src, d.begin() + (long)std::min<uint64_t>(d.size(), src + len));
                d.insert(d.begin() + (long)pos, span.begin(), span.end());
            }
            }
        }
        FILE* out = std::fopen(argv[4], "wb");
        if (!out) return 2;
        if (!d.empty() && std::fwrite(d.data(), 1, d.size(), out) != d.size()) return 2;
        std::fclose(out);
        vx_gguf f = nullptr;
        if (vx_gguf_open(argv[4], &f) == VX_OK) {
            ++opened;
            walk(f);
            if (vx_gguf_close(f) != VX_OK) std::abort();
        }
    }
    std::printf("gguf_fuzz: %ld iterations, %ld opened\n", iters, opened);
    return 0;
}
