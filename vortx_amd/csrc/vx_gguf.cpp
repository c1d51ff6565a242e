// vx_gguf.cpp — GGUF model-file reader behind include/vortx_gguf.h.
//
// The file is mapped read-only once; parsing walks it with a bounds-checked
// cursor (every length and count is checked against the bytes left before
// anything is reserved or read), so a truncated or corrupt file fails with
// VX_ERR_FORMAT instead of reading past the mapping. Tensor data is never
// copied on the host except through the pinned staging of vx_gguf_upload.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "vortx_gguf.h"
#include "vx_internal.hpp"

namespace {

using vx::fail;

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint32_t kMaxDims = 4;
constexpr int kMaxArrayDepth = 8;
constexpr uint64_t kMaxKeyLen = 65535;

struct Cursor {
    const uint8_t* base;
    uint64_t size;
    uint64_t pos;

    uint64_t left() const { return size - pos; }
    bool take(uint64_t n, const uint8_t** at) {
        if (n > left()) return false;
        *at = base + pos;
        pos += n;
        return true;
    }
    bool u32(uint32_t* v) {
        const uint8_t* at;
        if (!take(4, &at)) return false;
        std::memcpy(v, at, 4);
        return true;
    }
    bool u64(uint64_t* v) {
        const uint8_t* at;
        if (!take(8, &at)) return false;
        std::memcpy(v, at, 8);
        return true;
    }
    bool str(const uint8_t** s, uint64_t* len) { return u64(len) && take(*len, s); }
};

// Size of a fixed-size value type, 0 for string / array / unknown.
uint64_t fixed_size(uint32_t t) {
    switch (t) {
    case VX_GGUF_UINT8: case VX_GGUF_INT8: case VX_GGUF_BOOL: return 1;
    case VX_GGUF_UINT16: case VX_GGUF_INT16: return 2;
    case VX_GGUF_UINT32: case VX_GGUF_INT32: case VX_GGUF_FLOAT32: return 4;
    case VX_GGUF_UINT64: case VX_GGUF_INT64: case VX_GGUF_FLOAT64: return 8;
    default: return 0;
    }
}

// ggml type -> (elements, bytes) per block; false for types without a size here.
bool type_size(uint32_t t, uint32_t* be, uint32_t* bb) {
    struct S { uint32_t e, b; };
    static const S table[] = {
        {1, 4},     // 0  F32
        {1, 2},     // 1  F16
        {32, 18},   // 2  Q4_0
        {32, 20},   // 3  Q4_1
        {0, 0},     // 4  (removed)
        {0, 0},     // 5  (removed)
        {32, 22},   // 6  Q5_0
        {32, 24},   // 7  Q5_1
        {32, 34},   // 8  Q8_0
        {32, 36},   // 9  Q8_1
        {256, 84},  // 10 Q2_K
        {256, 110}, // 11 Q3_K
        {256, 144}, // 12 Q4_K
        {256, 176}, // 13 Q5_K
        {256, 210}, // 14 Q6_K
        {256, 292}, // 15 Q8_K
        {0, 0},     // 16 IQ2_XXS
        {0, 0},     // 17 IQ2_XS
        {0, 0},     // 18 IQ3_XXS
        {0, 0},     // 19 IQ1_S
        {32, 18},   // 20 IQ4_NL
        {0, 0},     // 21 IQ3_S
        {0, 0},     // 22 IQ2_S
        {256, 136}, // 23 IQ4_XS
        {1, 1},     // 24 I8
        {1, 2},     // 25 I16
        {1, 4},     // 26 I32
        {1, 8},     // 27 I64
        {1, 8},     // 28 F64
        {0, 0},     // 29 IQ1_M
        {1, 2},     // 30 BF16
    };
    if (t >= sizeof(table) / sizeof(table[0]) || table[t].e == 0) return false;
    *be = table[t].e;
    *bb = table[t].b;
    return true;
}

struct Kv {
    std::string key;
    uint32_t type = 0, elem_type = 0;
    uint64_t count = 1;
    uint64_t value_pos = 0;          // file offset of the value (after the array header for arrays)
    uint64_t nbytes = 0;             // bytes at value_pos for fixed-size payloads
    std::vector<uint64_t> str_pos;   // strings: file offset of each element's u64 length
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0, type = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
    bool size_known = false;
};

}  // namespace

struct vx_gguf_file {
    int fd = -1;  // kept open: vx_gguf_upload reads tensor data with pread
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    vx_gguf_header hdr{};
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, uint64_t> kv_index, tensor_index;

    ~vx_gguf_file() {
        if (map) munmap((void*)map, size);
        if (fd >= 0) close(fd);
    }
};

namespace {

int bad(const std::string& m) { return fail(VX_ERR_FORMAT, m.c_str()); }

// Skips (and, at depth 0, records) one value of type t.
int read_value(Cursor& c, uint32_t t, int depth, Kv* rec) {
    const uint64_t fs = fixed_size(t);
    const uint8_t* at;
    if (fs) {
        if (rec) {
            rec->value_pos = c.pos;
            rec->nbytes = fs;
        }
        return c.take(fs, &at) ? VX_OK : bad("metadata value runs past the end of the file");
    }
    if (t == VX_GGUF_STRING) {
        const uint64_t p = c.pos;
        uint64_t len;
        if (!c.str(&at, &len)) return bad("metadata string runs past the end of the file");
        if (rec) rec->str_pos.push_back(p);
        return VX_OK;
    }
    if (t != VX_GGUF_ARRAY) return bad("unknown metadata value type " + std::to_string(t));
    if (depth >= kMaxArrayDepth) return bad("metadata arrays nested too deeply");
    uint32_t et;
    uint64_t n;
    if (!c.u32(&et) || !c.u64(&n)) return bad("metadata array header runs past the end of the file");
    const uint64_t efs = fixed_size(et);
    if (rec) {
        rec->elem_type = et;
        rec->count = n;
        rec->value_pos = c.pos;
    }
    if (efs) {
        if (n > c.left() / efs) return bad("metadata array runs past the end of the file");
        if (rec) rec->nbytes = n * efs;
        c.pos += n * efs;
        return VX_OK;
    }
    if (et != VX_GGUF_STRING && et != VX_GGUF_ARRAY) return bad("unknown metadata array element type " + std::to_string(et));
    // each element needs at least 8 (string length) or 12 (array header) bytes
    if (n > c.left() / (et == VX_GGUF_STRING ? 8u : 12u)) return bad("metadata array runs past the end of the file");
    if (rec && et == VX_GGUF_STRING) rec->str_pos.reserve(n);
    for (uint64_t i = 0; i < n; ++i) {
        if (et == VX_GGUF_STRING) {
            const uint64_t p = c.pos;
            uint64_t len;
            if (!c.str(&at, &len)) return bad("metadata string runs past the end of the file");
            if (rec) rec->str_pos.push_back(p);
        } else {
            int s = read_value(c, VX_GGUF_ARRAY, depth + 1, nullptr);
            if (s) return s;
        }
    }
    return VX_OK;
}

int parse(vx_gguf_file* f) {
    Cursor c{f->map, f->size, 0};
    uint32_t magic, version;
    if (!c.u32(&magic) || magic != kMagic) return bad("not a GGUF file (magic)");
    if (!c.u32(&version)) return bad("truncated header");
    if (version == 1) return fail(VX_ERR_UNSUPPORTED, "GGUF version 1 (32-bit counts) is not supported");
    if (version != 2 && version != 3) {
        if ((version & 0xFFFFu) == 0) return fail(VX_ERR_UNSUPPORTED, "big-endian GGUF is not supported");
        return bad("unknown GGUF version " + std::to_string(version));
    }
    uint64_t nt, nkv;
    if (!c.u64(&nt) || !c.u64(&nkv)) return bad("truncated header");
    // a key-value pair takes >= 14 bytes (key length, 1 key byte, type, 1 value byte);
    // a tensor info >= 29 (name length, n_dims, one ne, type, offset)
    if (nkv > c.left() / 14) return bad("metadata count exceeds the file size");
    if (nt > c.left() / 29) return bad("tensor count exceeds the file size");
    f->hdr.version = version;
    f->hdr.n_tensors = nt;
    f->hdr.n_kv = nkv;
    f->kv.reserve(nkv);
    const uint8_t* s;
    uint64_t len;
    for (uint64_t i = 0; i < nkv; ++i) {
        Kv kv;
        if (!c.str(&s, &len)) return bad("metadata key runs past the end of the file");
        if (len == 0 || len > kMaxKeyLen) return bad("metadata key length out of range");
        // keys are handed out NUL-terminated: an embedded NUL could never be
        // looked up by name (the specification asks for ASCII keys)
        if (std::memchr(s, 0, len)) return bad("metadata key holds a NUL byte");
        kv.key.assign((const char*)s, len);
        if (!c.u32(&kv.type)) return bad("metadata type runs past the end of the file");
        kv.elem_type = kv.type;
        int st = read_value(c, kv.type, 0, &kv);
        if (st) return st;
        if (!f->kv_index.emplace(kv.key, i).second) return bad("duplicate metadata key '" + kv.key + "'");
        f->kv.push_back(std::move(kv));
    }
    uint64_t alignment = kDefaultAlignment;
    auto it = f->kv_index.find("general.alignment");
    if (it != f->kv_index.end()) {
        const Kv& a = f->kv[it->second];
        if (a.type != VX_GGUF_UINT32) return bad("general.alignment is not a uint32");
        uint32_t v;
        std::memcpy(&v, f->map + a.value_pos, 4);
        if (v == 0 || (v & (v - 1))) return bad("general.alignment is not a power of two");
        alignment = v;
    }
    f->hdr.alignment = alignment;
    f->tensors.reserve(nt);
    for (uint64_t i = 0; i < nt; ++i) {
        Tensor t;
        if (!c.str(&s, &len)) return bad("tensor name runs past the end of the file");
        if (std::memchr(s, 0, len)) return bad("tensor name holds a NUL byte");
        t.name.assign((const char*)s, len);
        if (!c.u32(&t.n_dims)) return bad("tensor info runs past the end of the file");
        if (t.n_dims < 1 || t.n_dims > kMaxDims) return bad("tensor '" + t.name + "' has n_dims outside 1..4");
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            if (!c.u64(&t.ne[d])) return bad("tensor info runs past the end of the file");
            if (t.ne[d] > (uint64_t)INT64_MAX) return bad("tensor '" + t.name + "' has a negative dimension");
            if (t.ne[d] && elems > (uint64_t)INT64_MAX / t.ne[d]) return bad("tensor '" + t.name + "' element count overflows");
            elems *= t.ne[d];
        }
        if (!c.u32(&t.type) || !c.u64(&t.offset)) return bad("tensor info runs past the end of the file");
        if (t.offset % alignment) return bad("tensor '" + t.name + "' offset is not a multiple of the alignment");
        uint32_t be, bb;
        if (type_size(t.type, &be, &bb)) {
            if (t.ne[0] % be) return bad("tensor '" + t.name + "' ne[0] is not a multiple of its block size");
            // bytes per row; for one-element "blocks" (F32, I64, ...) bb alone can
            // carry ne[0] < 2^63 past 2^64
            if (t.ne[0] / be > UINT64_MAX / bb) return bad("tensor '" + t.name + "' byte size overflows");
            uint64_t n = t.ne[0] / be * bb;
            for (uint32_t d = 1; d < t.n_dims; ++d) {
                if (t.ne[d] && n > UINT64_MAX / t.ne[d]) return bad("tensor '" + t.name + "' byte size overflows");
                n *= t.ne[d];
            }
            t.nbytes = n;
            t.size_known = true;
        }
        if (!f->tensor_index.emplace(t.name, i).second) return bad("duplicate tensor name '" + t.name + "'");
        f->tensors.push_back(std::move(t));
    }
    // data section: the next multiple of the alignment
    uint64_t data = c.pos + (alignment - c.pos % alignment) % alignment;
    if (data < c.pos) return bad("data offset overflows");
    f->hdr.data_offset = data;
    f->hdr.data_size = data <= f->size ? f->size - data : 0;
    f->hdr.file_size = f->size;
    for (const Tensor& t : f->tensors) {
        if (t.offset > f->hdr.data_size || t.nbytes > f->hdr.data_size - t.offset)
            return bad("tensor '" + t.name + "' data runs past the end of the file");
    }
    return VX_OK;
}

bool get_file(vx_gguf f, int* status) {
    if (!f) {
        *status = fail(VX_ERR_INVALID, "null GGUF handle");
        return false;
    }
    return true;
}

// ------------------------------------------------------------- upload
// File bytes -> device memory. Up to kUploadWorkers host threads each own
// every kUploadWorkers-th chunk of the range, two pinned staging buffers and
// a stream of their own: a worker preads chunk i into one buffer while the
// DMA of its previous chunk drains from the other. pread copies from the
// page cache without faulting in the mapping, and several readers keep the
// host-to-device link busy (one reader alone tops out near half the link).
// The worker streams first wait for everything already queued on the
// caller's stream, and the call returns once every copy has completed.
constexpr int kUploadWorkers = 2;
constexpr uint64_t kUploadChunk = 16ull << 20;

struct UploadWorker {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    void* buf[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    int status = VX_OK;
    int hip_error = 0;
    std::string msg;

    int hip_fail(hipError_t e, const char* what) {
        status = VX_ERR_HIP;
        hip_error = (int)e;
        msg = std::string(what) + ": " + hipGetErrorString(e);
        return status;
    }
    int setup(uint64_t bytes, hipEvent_t after) {
        hipError_t e;
        if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
        if ((e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking)) != hipSuccess)
            return hip_fail(e, "hipStreamCreateWithFlags");
        if ((e = hipStreamWaitEvent(stream, after, 0)) != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
        for (int b = 0; b < 2; ++b) {
            if ((e = hipHostMalloc(&buf[b], bytes, hipHostMallocDefault)) != hipSuccess)
                return hip_fail(e, "hipHostMalloc (upload staging)");
            if ((e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming)) != hipSuccess)
                return hip_fail(e, "hipEventCreateWithFlags");
        }
        return VX_OK;
    }
    // Runs on the worker thread: chunks first, first + step, ... of [0, n).
    void run(int fd, uint64_t file_pos, uint64_t n, uint8_t* dst, uint64_t first, uint64_t step) {
        uint64_t k = 0;
        for (uint64_t c = first; c * kUploadChunk < n && status == VX_OK; c += step, ++k) {
            const int b = (int)(k & 1);
            const uint64_t at = c * kUploadChunk, len = n - at < kUploadChunk ? n - at : kUploadChunk;
            hipError_t e;
            if (pending[b]) {
                if ((e = hipEventSynchronize(ev[b])) != hipSuccess) return (void)hip_fail(e, "hipEventSynchronize");
                pending[b] = false;
            }
            for (uint64_t got = 0; got < len;) {
                const ssize_t r = pread(fd, (uint8_t*)buf[b] + got, len - got, (off_t)(file_pos + at + got));
                if (r < 0 && errno == EINTR) continue;
                if (r <= 0) {
                    status = VX_ERR_IO;
                    msg = std::string("reading the GGUF file: ") + (r < 0 ? std::strerror(errno) : "unexpected end of file");
                    return;
                }
                got += (uint64_t)r;
            }
            if ((e = hipMemcpyAsync(dst + at, buf[b], len, hipMemcpyHostToDevice, stream)) != hipSuccess)
                return (void)hip_fail(e, "hipMemcpyAsync (upload)");
            if ((e = hipEventRecord(ev[b], stream)) != hipSuccess) return (void)hip_fail(e, "hipEventRecord");
            pending[b] = true;
        }
    }
    // Waits for the copies in flight and releases everything (caller's thread).
    void finish() {
        for (int b = 0; b < 2; ++b) {
            if (pending[b]) {
                const hipError_t e = hipEventSynchronize(ev[b]);
                if (e != hipSuccess && status == VX_OK) hip_fail(e, "hipEventSynchronize");
            }
            if (ev[b]) (void)hipEventDestroy(ev[b]);
            if (buf[b]) (void)hipHostFree(buf[b]);
        }
        if (stream) (void)hipStreamDestroy(stream);
    }
};

int upload(vx_gguf_file* f, int device, hipStream_t caller, uint64_t file_pos, uint64_t n, uint8_t* dst) {
    int prev = -1;
    hipError_t e;
    if ((e = hipGetDevice(&prev)) != hipSuccess) return vx::fail_hip(e, "hipGetDevice");
    if (prev != device && (e = hipSetDevice(device)) != hipSuccess) return vx::fail_hip(e, "hipSetDevice");
    hipEvent_t after = nullptr;
    if ((e = hipEventCreateWithFlags(&after, hipEventDisableTiming)) != hipSuccess ||
        (e = hipEventRecord(after, caller)) != hipSuccess) {
        if (after) (void)hipEventDestroy(after);
        if (prev != device) (void)hipSetDevice(prev);
        return vx::fail_hip(e, "hipEventRecord (caller stream)");
    }
    const uint64_t chunks = (n + kUploadChunk - 1) / kUploadChunk;
    uint64_t workers = kUploadWorkers;
    if (const char* env = std::getenv("VX_GGUF_UPLOAD_THREADS")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1 && v <= 64) workers = (uint64_t)v;
    }
    const int nw = (int)(chunks < workers ? chunks : workers);
    const uint64_t stage = n < kUploadChunk ? n : kUploadChunk;
    std::vector<UploadWorker> w(nw);
    int status = VX_OK;
    for (int i = 0; i < nw && status == VX_OK; ++i) {
        w[i].device = device;
        status = w[i].setup(stage, after);
    }
    if (status == VX_OK) {
        std::vector<std::thread> th;
        for (int i = 1; i < nw; ++i) {
            try {
                th.emplace_back([&, i] {
                    if (hipSetDevice(device) != hipSuccess) {
                        w[i].status = VX_ERR_HIP;
                        w[i].msg = "hipSetDevice (upload worker)";
                        return;
                    }
                    w[i].run(f->fd, file_pos, n, dst, (uint64_t)i, (uint64_t)nw);
                });
            } catch (...) {  // no thread: this worker's chunks run on the caller's thread below
                w[i].status = -1;
            }
        }
        w[0].run(f->fd, file_pos, n, dst, 0, (uint64_t)nw);
        for (int i = 1; i < nw; ++i) {
            if (w[i].status == -1) {
                w[i].status = VX_OK;
                w[i].run(f->fd, file_pos, n, dst, (uint64_t)i, (uint64_t)nw);
            }
        }
        for (auto& t : th) t.join();
    }
    for (auto& x : w) x.finish();
    (void)hipEventDestroy(after);
    if (prev != device) (void)hipSetDevice(prev);
    for (auto& x : w) {
        if (x.status == VX_ERR_HIP) return vx::fail_hip(x.hip_error, x.msg.c_str());
        if (x.status != VX_OK) return fail(x.status, x.msg.c_str());
    }
    return VX_OK;
}

}  // namespace

extern "C" {

int vx_gguf_type_size(uint32_t ggml_type, uint32_t* block_elems, uint32_t* block_bytes) {
    vx::clear_error();
    if (!block_elems || !block_bytes) return fail(VX_ERR_INVALID, "null output");
    if (!type_size(ggml_type, block_elems, block_bytes))
        return fail(VX_ERR_UNSUPPORTED, ("no block size for ggml type " + std::to_string(ggml_type)).c_str());
    return VX_OK;
}

int vx_gguf_open(const char* path, vx_gguf* out) {
    vx::clear_error();
    if (!path || !out) return fail(VX_ERR_INVALID, "null argument");
    *out = nullptr;
    auto* f = new vx_gguf_file();
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) {
        const int err = errno;
        delete f;
        return fail(VX_ERR_IO, (std::string("cannot open ") + path + ": " + std::strerror(err)).c_str());
    }
    struct stat st;
    if (fstat(f->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        delete f;
        return fail(VX_ERR_IO, (std::string("not a regular file: ") + path).c_str());
    }
    f->size = (uint64_t)st.st_size;
    if (f->size > 0) {
        void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
        if (m == MAP_FAILED) {
            const int err = errno;
            delete f;
            return fail(VX_ERR_IO, (std::string("cannot map ") + path + ": " + std::strerror(err)).c_str());
        }
        f->map = (const uint8_t*)m;
    }
    const int s = parse(f);
    if (s) {
        delete f;
        return s;
    }
    *out = f;
    return VX_OK;
}

int vx_gguf_close(vx_gguf file) {
    vx::clear_error();
    delete file;
    return VX_OK;
}

int vx_gguf_get_header(vx_gguf f, vx_gguf_header* out) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!out) return fail(VX_ERR_INVALID, "null output");
    *out = f->hdr;
    return VX_OK;
}

int vx_gguf_tensor_info(vx_gguf f, uint64_t index, vx_gguf_tensor* out) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!out) return fail(VX_ERR_INVALID, "null output");
    if (index >= f->tensors.size()) return fail(VX_ERR_INVALID, "tensor index out of range");
    const Tensor& t = f->tensors[index];
    std::memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->n_dims = t.n_dims;
    out->type = t.type;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->size_known = t.size_known ? 1u : 0u;
    out->data = t.size_known && t.nbytes ? f->map + f->hdr.data_offset + t.offset : nullptr;
    return VX_OK;
}

int vx_gguf_find_tensor(vx_gguf f, const char* name, uint64_t* index) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!name || !index) return fail(VX_ERR_INVALID, "null argument");
    auto it = f->tensor_index.find(name);
    if (it == f->tensor_index.end()) return fail(VX_ERR_NOT_FOUND, (std::string("no tensor named ") + name).c_str());
    *index = it->second;
    return VX_OK;
}

int vx_gguf_kv_info(vx_gguf f, uint64_t index, vx_gguf_kv* out) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!out) return fail(VX_ERR_INVALID, "null output");
    if (index >= f->kv.size()) return fail(VX_ERR_INVALID, "metadata index out of range");
    const Kv& k = f->kv[index];
    std::memset(out, 0, sizeof(*out));
    out->key = k.key.c_str();
    out->type = k.type;
    out->elem_type = k.elem_type;
    out->count = k.count;
    if (fixed_size(k.elem_type)) {
        out->data = f->map + k.value_pos;
        out->nbytes = k.nbytes;
    }
    return VX_OK;
}

int vx_gguf_find_key(vx_gguf f, const char* key, uint64_t* index) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!key || !index) return fail(VX_ERR_INVALID, "null argument");
    auto it = f->kv_index.find(key);
    if (it == f->kv_index.end()) return fail(VX_ERR_NOT_FOUND, (std::string("no metadata key ") + key).c_str());
    *index = it->second;
    return VX_OK;
}

int vx_gguf_kv_string(vx_gguf f, uint64_t index, uint64_t elem, const char** str, uint64_t* len) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!str || !len) return fail(VX_ERR_INVALID, "null output");
    if (index >= f->kv.size()) return fail(VX_ERR_INVALID, "metadata index out of range");
    const Kv& k = f->kv[index];
    if (k.elem_type != VX_GGUF_STRING) return fail(VX_ERR_INVALID, "metadata value is not a string");
    if (elem >= k.str_pos.size()) return fail(VX_ERR_INVALID, "string element out of range");
    uint64_t n;
    std::memcpy(&n, f->map + k.str_pos[elem], 8);
    *str = (const char*)(f->map + k.str_pos[elem] + 8);
    *len = n;
    return VX_OK;
}

int vx_gguf_qweight(vx_gguf f, uint64_t index, const void* device_data, vx_qweight* out) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!device_data || !out) return fail(VX_ERR_INVALID, "null argument");
    if (index >= f->tensors.size()) return fail(VX_ERR_INVALID, "tensor index out of range");
    const Tensor& t = f->tensors[index];
    if (t.type != VX_Q4_0 && t.type != VX_Q8_0 && t.type != VX_Q4_K)
        return fail(VX_ERR_UNSUPPORTED, ("tensor '" + t.name + "' is not Q4_0, Q8_0 or Q4_K").c_str());
    if (t.ne[2] != 1 || t.ne[3] != 1)
        return fail(VX_ERR_UNSUPPORTED, ("tensor '" + t.name + "' is not a matrix (ne[2] or ne[3] != 1)").c_str());
    if (t.ne[0] > UINT32_MAX || t.ne[1] > UINT32_MAX)
        return fail(VX_ERR_UNSUPPORTED, ("tensor '" + t.name + "' has a dimension >= 2^32").c_str());
    uint32_t be, bb;
    type_size(t.type, &be, &bb);
    std::memset(out, 0, sizeof(*out));
    out->base = (const uint8_t*)device_data + t.offset;
    out->qtype = t.type;
    out->rows = (uint32_t)t.ne[1];
    out->cols = (uint32_t)t.ne[0];
    out->row_stride_bytes = t.ne[0] / be * bb;
    return VX_OK;
}

int vx_gguf_view(vx_gguf f, uint64_t index, const void* device_data, vx_cview* out) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!device_data || !out) return fail(VX_ERR_INVALID, "null argument");
    if (index >= f->tensors.size()) return fail(VX_ERR_INVALID, "tensor index out of range");
    const Tensor& t = f->tensors[index];
    if (t.type != 0) return fail(VX_ERR_UNSUPPORTED, ("tensor '" + t.name + "' is not F32").c_str());
    if (t.offset % 4 || (uintptr_t)device_data % 4)
        return fail(VX_ERR_UNSUPPORTED, ("tensor '" + t.name + "' is not 4-byte aligned").c_str());
    static const uint32_t kGgmlIds[4] = {1, 0, 2, 3};  // src/shapes.rs:15-18
    vx_layout l;
    for (int d = 0; d < 4; ++d) l.size[d] = 1, l.stride[d] = 1;
    l.rank = t.n_dims;
    l.offset = 0;
    uint64_t stride = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
        const uint32_t at = t.n_dims == 1 ? 0 : kGgmlIds[d];
        if (t.ne[d] > UINT32_MAX || stride > UINT32_MAX)
            return fail(VX_ERR_UNSUPPORTED, ("tensor '" + t.name + "' has a size or stride >= 2^32").c_str());
        l.size[at] = (uint32_t)t.ne[d];
        l.stride[at] = (uint32_t)stride;
        stride *= t.ne[d];
    }
    out->base = (const float*)((const uint8_t*)device_data + t.offset);
    out->layout = l;
    return VX_OK;
}

int vx_gguf_upload(vx_ctx ctx, vx_stream stream, vx_gguf f, uint64_t offset, uint64_t nbytes, void* device_dst) {
    vx::clear_error();
    int s;
    if (!get_file(f, &s)) return s;
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    if (offset > f->hdr.data_size || nbytes > f->hdr.data_size - offset)
        return fail(VX_ERR_INVALID, "upload range runs past the data section");
    if (nbytes == 0) return VX_OK;
    if (!device_dst) return fail(VX_ERR_INVALID, "null device destination");
    int device = 0;
    if ((s = vx_device_info(ctx, &device, nullptr))) return s;
    return upload(f, device, (hipStream_t)stream, f->hdr.data_offset + offset, nbytes, (uint8_t*)device_dst);
}

}  // extern "C"
