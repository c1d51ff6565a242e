// vx_host.cpp — runtime and op dispatch of libvortx_hip.so behind the C ABI
// declared in include/vortx_hip.h.
//
// Runtime: the gfx950 code objects built by hipcc --genco are embedded in
// this library (vx_embed.S); vx_init loads them with hipModuleLoadData and
// resolves every kernel once; launches go through hipModuleLaunchKernel with
// the kernel's argument struct (vx_kargs.h) passed by value (kernelParams).
//
// Ops: Gemm::dispatch / dispatch_naive / dispatch_tiled of
// src/linalg/gemm.rs:47-305 (canonicalize, validate, pick a kernel, grid)
// and the block-quantized GEMV / dequantize, which the reference lacks.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "vx_internal.hpp"
#include "vx_kargs.h"

extern "C" {
extern const unsigned char vx_co_gemm[];
extern const unsigned char vx_co_gemm_end[];
extern const unsigned char vx_co_gemv_q[];
extern const unsigned char vx_co_gemv_q_end[];
extern const unsigned char vx_co_copy[];
extern const unsigned char vx_co_copy_end[];
extern const unsigned char vx_co_quantize[];
extern const unsigned char vx_co_quantize_end[];
}

namespace vx {

// --------------------------------------------------------------- errors
static thread_local std::string t_msg;
static thread_local int t_hip = 0;

int fail(int status, const char* msg) {
    t_msg = msg ? msg : "";
    return status;
}

int fail_hip(int hip_error, const char* what) {
    t_hip = hip_error;
    t_msg = std::string(what) + ": " + hipGetErrorString((hipError_t)hip_error);
    return VX_ERR_HIP;
}

void clear_error() {
    t_msg.clear();
    t_hip = 0;
}

// -------------------------------------------------------------- kernels
// Every kernel the library launches; resolved by name at vx_init.
enum Kernel : int {
#define K(name) K_##name,
#include "vx_kernel_list.inc"
#undef K
    K_COUNT
};
static const char* const kKernelNames[K_COUNT] = {
#define K(name) #name,
#include "vx_kernel_list.inc"
#undef K
};
// The embedded code objects; every kernel name is unique across them.
static const unsigned char* const kModules[] = {vx_co_gemm, vx_co_gemv_q, vx_co_copy, vx_co_quantize};
constexpr int kNumModules = 4;
constexpr int kModGemv = 1;  // the module holding vx_scratch

}  // namespace vx

struct vx_context {
    int device = 0;
    int num_cus = 0;
    size_t lds_per_block = 65536;
    hipModule_t mods[vx::kNumModules] = {};
    hipFunction_t fn[vx::K_COUNT] = {};
    // device address of vx_scratch in this context's GEMV module (vx_gemv_q_noalloc)
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Nothing here changes after vx_init: buffers a call needs beyond its
    // operands are the caller's (vx_gemv_q_ws) or the module's scratch.
};

namespace vx {

struct DeviceGuard {
    int prev = -1;
    bool changed = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
            changed = hipSetDevice(dev) == hipSuccess;
        }
    }
    ~DeviceGuard() {
        if (changed) (void)hipSetDevice(prev);
    }
};

// Every kernel takes its vx_*_args struct by value. It is passed through
// kernelParams (an array of pointers to each argument), which the runtime
// copies by the kernel's argument layout at launch, and which stream capture
// copies into the graph node, so the arguments may live on this stack frame.
template <class Args>
static int launch(vx_ctx ctx, int k, dim3 grid, dim3 block, size_t lds, vx_stream stream, const Args& args) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return VX_OK;
    Args copy = args;
    void* params[] = {&copy};
    const hipError_t e = hipModuleLaunchKernel(ctx->fn[k], grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                               (unsigned)lds, (hipStream_t)stream, params, nullptr);
    if (e != hipSuccess) return fail_hip(e, kKernelNames[k]);
    return VX_OK;
}

// The persistent batch-1 kernels (and the read probe and launch floor) take
// the fields a wave needs before its first request as leading scalars, which
// arrive preloaded in SGPRs (VX_B1_PARAMS in gemv_q.hip: w, x, row stride,
// M, units per row, grid size, x layout flag), then the struct.
static int launch_b1(vx_ctx ctx, int k, uint32_t grid, size_t lds, vx_stream stream, const vx_gemv_args& args) {
    if (grid == 0) return VX_OK;
    vx_gemv_args copy = args;
    const uint8_t* w = args.w;
    const float* x = args.x;
    uint64_t rs = args.row_stride;
    uint32_t M = args.M, nu = args.nunits, G = grid, xv = args.x_vec;
    void* params[] = {&w, &x, &rs, &M, &nu, &G, &xv, &copy};
    const hipError_t e = hipModuleLaunchKernel(ctx->fn[k], grid, 1, 1, 1024, 1, 1, (unsigned)lds, (hipStream_t)stream,
                                               params, nullptr);
    if (e != hipSuccess) return fail_hip(e, kKernelNames[k]);
    return VX_OK;
}

// ----------------------------------------------------------------- init
static int init(int device, vx_ctx* out) {
    if (!out) return fail(VX_ERR_INVALID, "null out_ctx");
    *out = nullptr;
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess) return fail_hip(e, "hipGetDeviceCount");
    if (device < 0 || device >= ndev) return fail(VX_ERR_INVALID, "device ordinal out of range");
    DeviceGuard guard(device);
    if (!guard.changed) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess || cur != device) {
            e = hipSetDevice(device);
            if (e != hipSuccess) return fail_hip(e, "hipSetDevice");
        }
    }
    auto* ctx = new vx_context();
    ctx->device = device;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        delete ctx;
        return fail_hip(e, "hipGetDeviceProperties");
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        delete ctx;
        return fail(VX_ERR_UNSUPPORTED, "device is not gfx950 (MI355X); this library ships gfx950 code only");
    }
    ctx->num_cus = prop.multiProcessorCount;
    ctx->lds_per_block = prop.sharedMemPerBlock;
    auto unload = [&]() {
        for (hipModule_t m : ctx->mods)
            if (m) (void)hipModuleUnload(m);
    };
    for (int i = 0; i < kNumModules; ++i) {
        e = hipModuleLoadData(&ctx->mods[i], kModules[i]);
        if (e != hipSuccess) {
            unload();
            t_hip = e;
            t_msg = std::string("hipModuleLoadData: ") + hipGetErrorString(e);
            delete ctx;
            return VX_ERR_NO_CODE_OBJECT;
        }
    }
    for (int k = 0; k < K_COUNT; ++k) {
        e = hipErrorNotFound;
        for (int i = 0; i < kNumModules && e != hipSuccess; ++i) {
            e = hipModuleGetFunction(&ctx->fn[k], ctx->mods[i], kKernelNames[k]);
            // a miss in one module is expected; do not leave it as the
            // runtime's last error for the caller's next HIP call
            if (e != hipSuccess) (void)hipGetLastError();
        }
        if (e != hipSuccess) {
            unload();
            delete ctx;
            t_hip = e;
            t_msg = std::string("hipModuleGetFunction(") + kKernelNames[k] + "): " + hipGetErrorString(e);
            return VX_ERR_NO_CODE_OBJECT;
        }
    }
    // The no-alloc entry point's scratch: a __device__ array of the GEMV code
    // object; its address on this device (current here) is resolved once.
    {
        hipDeviceptr_t p = nullptr;
        size_t bytes = 0;
        e = hipModuleGetGlobal(&p, &bytes, ctx->mods[kModGemv], "vx_scratch");
        if (e != hipSuccess || !p || bytes != VX_SCRATCH_BYTES) {
            if (e == hipSuccess) e = hipErrorNotFound;
            (void)hipGetLastError();
            unload();
            delete ctx;
            t_hip = e;
            t_msg = std::string("hipModuleGetGlobal(vx_scratch): ") + hipGetErrorString(e);
            return VX_ERR_NO_CODE_OBJECT;
        }
        ctx->scratch = (void*)p;
        ctx->scratch_bytes = bytes;
    }
    *out = ctx;
    return VX_OK;
}

// ------------------------------------------------------------ view math
struct Canon {
    vx_layout l;      // canonical rank-4 layout (offset applied to ptr)
    uintptr_t ptr;    // base + original offset, in bytes
};

static int canon_view(const void* base, const vx_layout* in, Canon* c, const char* name) {
    if (!in) return fail(VX_ERR_INVALID, "null view");
    if (in->rank > 4) return fail(VX_ERR_UNSUPPORTED, "tensors of ranks > 4 not supported");
    int s = layout_canonicalize(in, &c->l);
    if (s) return s;
    c->ptr = (uintptr_t)base + 4ull * in->offset;
    uint64_t n = 1;
    for (int k = 0; k < 4; ++k) n *= c->l.size[k];
    if (n && !base) {
        static thread_local std::string m;
        m = std::string("null base pointer for ") + name;
        return fail(VX_ERR_INVALID, m.c_str());
    }
    return VX_OK;
}

static bool aligned16(uintptr_t p) { return (p & 15u) == 0; }

static std::string layout_str(const vx_layout& l) {
    char buf[200];
    std::snprintf(buf, sizeof buf, "{size:[%u,%u,%u,%u], stride:[%u,%u,%u,%u]}", l.size[0], l.size[1], l.size[2],
                  l.size[3], l.stride[0], l.stride[1], l.stride[2], l.stride[3]);
    return buf;
}

// ---------------------------------------------------------------- gemm
enum Force { FORCE_AUTO = -1, FORCE_NAIVE = 0, FORCE_TILED = 1 };

struct GemmPlan {
    Canon o, l, r;
    uint32_t M, N, K, nb, nc;
    int route;
};

// Canonicalize and validate exactly like Gemm::dispatch
// (src/linalg/gemm.rs:66-104), then choose the route (:111-118). With
// `broadcast`, a batch dim (0 or 1) of lhs or rhs may instead be 1 where
// out's is larger: its stride becomes 0, as TensorLayout::broadcast
// (src/shapes.rs:346-391) sets it, so the kernels reuse that operand.
static int plan_gemm(const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs, int force, GemmPlan* p,
                     bool broadcast = false) {
    if (!out || !lhs || !rhs) return fail(VX_ERR_INVALID, "null view");
    int s;
    if ((s = canon_view(out->base, &out->layout, &p->o, "out"))) return s;
    if ((s = canon_view(lhs->base, &lhs->layout, &p->l, "lhs"))) return s;
    if ((s = canon_view(rhs->base, &rhs->layout, &p->r, "rhs"))) return s;
    vx_layout &so = p->o.l, &sl = p->l.l, &sr = p->r.l;
    if (broadcast) {
        for (int d = 0; d < 2; ++d) {
            if (sl.size[d] == 1 && so.size[d] != 1) sl.size[d] = so.size[d], sl.stride[d] = 0;
            if (sr.size[d] == 1 && so.size[d] != 1) sr.size[d] = so.size[d], sr.stride[d] = 0;
        }
    }
    const bool ok = so.size[0] == sl.size[0] && so.size[1] == sl.size[1] && sl.size[0] == sr.size[0] &&
                    sl.size[1] == sr.size[1] && so.size[2] == sl.size[2] && so.size[3] == sr.size[3] &&
                    sl.size[3] == sr.size[2];
    if (!ok) {
        static thread_local std::string m;
        m = "incompatible gemm shapes: " + layout_str(so) + " = " + layout_str(sl) + " x " + layout_str(sr);
        return fail(VX_ERR_SHAPE, m.c_str());
    }
    p->nb = so.size[0];
    p->nc = so.size[1];
    p->M = so.size[2];
    p->N = so.size[3];
    p->K = sl.size[3];
    if ((uint64_t)p->nb * p->nc > 65535u) return fail(VX_ERR_UNSUPPORTED, "more than 65535 batch matrices");
    if (p->M == 0 || p->N == 0 || p->nb == 0 || p->nc == 0) {
        p->route = VX_ROUTE_EMPTY;
        return VX_OK;
    }
    if (force == FORCE_NAIVE) {
        p->route = VX_ROUTE_NAIVE;
    } else if (force == FORCE_TILED) {
        p->route = VX_ROUTE_TILED;
    } else if (p->M < 32 && p->N < 32) {
        p->route = VX_ROUTE_NAIVE;
    } else if (p->N == 1 && sl.stride[3] == 1 && sl.stride[2] % 4 == 0 && (p->nb == 1 || sl.stride[0] % 4 == 0) &&
               (p->nc == 1 || sl.stride[1] % 4 == 0) && aligned16(p->l.ptr)) {
        p->route = VX_ROUTE_GEMV;
    } else {
        p->route = VX_ROUTE_TILED;
    }
    return VX_OK;
}

// Operand mode for the MFMA kernel: 0 = contiguous along K, 1 = contiguous
// along the other dim (M for A, N for B), 2 = generic. 128-bit loads need
// the unit-stride dim plus 4-aligned other strides and a 16-byte base.
static int operand_mode(const Canon& c, int kdim, int xdim, uint32_t nb, uint32_t nc) {
    const vx_layout& l = c.l;
    const bool batch4 = (nb == 1 || l.stride[0] % 4 == 0) && (nc == 1 || l.stride[1] % 4 == 0);
    if (!batch4 || !aligned16(c.ptr)) return 2;
    if (l.stride[kdim] == 1 && l.stride[xdim] % 4 == 0) return 0;
    if (l.stride[xdim] == 1 && l.stride[kdim] % 4 == 0) return 1;
    return 2;
}

static int run_gemm(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs,
                    int force, const vx_gemm_opts* opts = nullptr) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    float alpha = 1.f, beta = 0.f;
    bool broadcast = false;
    if (opts) {
        if (opts->reserved != 0 ||
            (opts->flags & ~(uint32_t)(VX_GEMM_BROADCAST | VX_GEMM_TILE_NARROW | VX_GEMM_TILE_WIDE | VX_GEMM_TILE_SMALL)))
            return fail(VX_ERR_INVALID, "unknown gemm option flags (reserved must be 0)");
        const uint32_t tf = opts->flags & (VX_GEMM_TILE_NARROW | VX_GEMM_TILE_WIDE | VX_GEMM_TILE_SMALL);
        if (tf & (tf - 1u))
            return fail(VX_ERR_INVALID, "VX_GEMM_TILE_NARROW, VX_GEMM_TILE_WIDE and VX_GEMM_TILE_SMALL are exclusive");
        alpha = opts->alpha;
        beta = opts->beta;
        broadcast = (opts->flags & VX_GEMM_BROADCAST) != 0;
    }
    GemmPlan p;
    int s = plan_gemm(out, lhs, rhs, force, &p, broadcast);
    if (s) return s;
    if (opts) {
        // every output element must have its own address: the epilogue reads it, and
        // different (i, j) writing one address would race
        for (int d = 0; d < 4; ++d)
            if (p.o.l.size[d] > 1 && p.o.l.stride[d] == 0)
                return fail(VX_ERR_INVALID, "out has a zero stride on a dimension of size > 1");
    }
    if (p.route == VX_ROUTE_EMPTY) return VX_OK;
    DeviceGuard guard(ctx->device);
    const uint32_t batch = p.nb * p.nc;
    if (p.route == VX_ROUTE_GEMV) {
        vx_gemv_f32_args g{};
        g.a = (const float*)p.l.ptr;
        g.as_m = p.l.l.stride[2];
        g.as_k = p.l.l.stride[3];
        g.x = (const float*)p.r.ptr;
        g.xs_k = p.r.l.stride[2];
        g.y = (float*)p.o.ptr;
        g.ys_m = p.o.l.stride[2];
        g.M = p.M;
        g.K = p.K;
        g.batch_c = p.nc;
        g.a_bs[0] = p.l.l.stride[0];
        g.a_bs[1] = p.l.l.stride[1];
        g.x_bs[0] = p.r.l.stride[0];
        g.x_bs[1] = p.r.l.stride[1];
        g.y_bs[0] = p.o.l.stride[0];
        g.y_bs[1] = p.o.l.stride[1];
        g.alpha = alpha;
        g.beta = beta;
        // one row per workgroup, or four when a row is short (K < 4096: then
        // one row would leave each wave fewer than four loads in flight)
        // (a grid holds fewer than 2^32 threads: 2^24 one-row workgroups)
        if (p.K >= 4096u && p.M < (1u << 24))
            return launch(ctx, K_vx_gemv_f32, dim3(p.M, batch, 1), dim3(VX_WG), 0, stream, g);
        return launch(ctx, K_vx_gemv_f32_r4, dim3((p.M + 3) / 4, batch, 1), dim3(VX_WG), 0, stream, g);
    }
    vx_gemm_args a{};
    a.c = (float*)p.o.ptr;
    a.a = (const float*)p.l.ptr;
    a.b = (const float*)p.r.ptr;
    for (int k = 0; k < 4; ++k) {
        a.cs[k] = p.o.l.stride[k];
        a.as[k] = p.l.l.stride[k];
        a.bs[k] = p.r.l.stride[k];
    }
    a.batch_c = p.nc;
    a.M = p.M;
    a.N = p.N;
    a.K = p.K;
    a.alpha = alpha;
    a.beta = beta;
    if (p.route == VX_ROUTE_NAIVE) {
        return launch(ctx, K_vx_gemm_naive, dim3((p.N + 63) / 64, p.M, batch), dim3(64), 0, stream, a);
    }
    a.tiles_m = (p.M + 127) / 128;
    a.tiles_n = (p.N + 127) / 128;
    const int am = operand_mode(p.l, 3, 2, p.nb, p.nc);
    const int bm = operand_mode(p.r, 2, 3, p.nb, p.nc);
    int k;
    // Tile shape. 128 x 256 tiles (two resident workgroups per CU) instead of
    // 128 x 128 (three) when they fill the last round of resident workgroups
    // clearly better: 4096^3 is 1024 narrow tiles, 1.33 rounds of 768, but 512
    // wide ones, one round (B transposed 131 -> 137 TFLOP/s). 64 x 64 tiles
    // when they spread over the CUs better than either, a CU taking
    // ceil(tiles / CUs) of them, balance = (tiles / CUs) / that, the small
    // kernel weighted 0.9 for its lower rate on large shapes (4096^3: 119 vs
    // 131 TFLOP/s): 1024^3 28 -> 75, 1536^3 65 -> 80, 3072^3 96 -> 109. All
    // give the same bits; VX_GEMM_TILE_* (vx_gemm_f32_ex) force one.
    bool wide = false, small = false;
    if (am == 0 && (bm == 0 || bm == 1)) {
        const uint64_t tn = (uint64_t)a.tiles_m * a.tiles_n * batch;
        const uint64_t tw = (uint64_t)a.tiles_m * ((p.N + 255) / 256) * batch;
        const uint64_t ts = (uint64_t)((p.M + 63) / 64) * ((p.N + 63) / 64) * batch;
        const uint64_t sn = 3ull * (uint64_t)ctx->num_cus, sw = 2ull * (uint64_t)ctx->num_cus;
        const double en = (double)tn / (double)(((tn + sn - 1) / sn) * sn);
        const double ew = (double)tw / (double)(((tw + sw - 1) / sw) * sw);
        wide = ew > en + 0.05;
        const double cus = (double)ctx->num_cus;
        auto balance = [&](uint64_t t) { return ((double)t / cus) / std::ceil((double)t / cus); };
        small = 0.9 * balance(ts) > std::max(balance(tn), balance(tw));
        if (small) wide = false;
        const uint32_t tf = opts ? opts->flags : 0u;
        if (tf & (VX_GEMM_TILE_NARROW | VX_GEMM_TILE_WIDE | VX_GEMM_TILE_SMALL)) {
            wide = (tf & VX_GEMM_TILE_WIDE) != 0;
            small = (tf & VX_GEMM_TILE_SMALL) != 0;
        }
    }
    if (small) {
        a.tiles_m = (p.M + 63) / 64;
        a.tiles_n = (p.N + 63) / 64;
        k = bm == 1 ? K_vx_gemm_mfma_kx_s : K_vx_gemm_mfma_kk_s;
    } else if (wide) {
        a.tiles_n = (p.N + 255) / 256;
        k = bm == 1 ? K_vx_gemm_mfma_kx_w : K_vx_gemm_mfma_kk_w;
    } else if (am == 0 && bm == 1) k = K_vx_gemm_mfma_kx;
    else if (am == 0 && bm == 0) k = K_vx_gemm_mfma_kk;
    else if (am == 1 && bm == 1) k = K_vx_gemm_mfma_xx;
    else if (am == 1 && bm == 0) k = K_vx_gemm_mfma_xk;
    else if (am == 0) k = K_vx_gemm_mfma_kg;
    else if (bm == 1) k = K_vx_gemm_mfma_gx;
    else k = K_vx_gemm_mfma_gg;
    const uint64_t tiles = (uint64_t)a.tiles_m * a.tiles_n;
    if (tiles > 0x7FFFFFFFull) return fail(VX_ERR_UNSUPPORTED, "too many output tiles");
    return launch(ctx, k, dim3((uint32_t)tiles, 1, batch), dim3(VX_WG), 0, stream, a);
}

// ------------------------------------------------------------ quant gemv
static int qinfo(uint32_t qt, uint32_t* qk, uint32_t* bb) {
    switch (qt) {
    case VX_Q4_0: *qk = 32; *bb = 18; return VX_OK;
    case VX_Q8_0: *qk = 32; *bb = 34; return VX_OK;
    case VX_Q4_K: *qk = 256; *bb = 144; return VX_OK;
    default: return fail(VX_ERR_INVALID, "unknown quant type (expected GGML id 2, 8 or 12)");
    }
}

static int check_qweight(const vx_qweight* w, uint32_t* qk, uint32_t* bb) {
    if (!w) return fail(VX_ERR_INVALID, "null weight");
    int s = qinfo(w->qtype, qk, bb);
    if (s) return s;
    if (w->reserved) return fail(VX_ERR_INVALID, "vx_qweight.reserved must be 0");
    if (w->cols % *qk) return fail(VX_ERR_UNSUPPORTED, "cols is not a multiple of the block size");
    if (w->row_stride_bytes < (uint64_t)(w->cols / *qk) * *bb)
        return fail(VX_ERR_INVALID, "row_stride_bytes smaller than one row of blocks");
    if (w->rows && w->cols && !w->base) return fail(VX_ERR_INVALID, "null weight base");
    return VX_OK;
}

static int q_index(uint32_t qt) { return qt == VX_Q4_0 ? 0 : qt == VX_Q8_0 ? 1 : 2; }

static int b1_kernel(uint32_t qt, int R) {
    static const int tab[3][4] = {
        {K_vx_gemv_b1_q4_0_r1, K_vx_gemv_b1_q4_0_r2, K_vx_gemv_b1_q4_0_r4, K_vx_gemv_b1_q4_0_r8},
        {K_vx_gemv_b1_q8_0_r1, K_vx_gemv_b1_q8_0_r2, K_vx_gemv_b1_q8_0_r4, K_vx_gemv_b1_q8_0_r8},
        {K_vx_gemv_b1_q4_k_r1, K_vx_gemv_b1_q4_k_r2, K_vx_gemv_b1_q4_k_r4, K_vx_gemv_b1_q4_k_r8}};
    const int ri = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : 3;
    return tab[q_index(qt)][ri];
}

static int i8b1_kernel(uint32_t qt, int R) {
    static const int tab[3][4] = {
        {K_vx_gemv_i8b1_q4_0_r1, K_vx_gemv_i8b1_q4_0_r2, K_vx_gemv_i8b1_q4_0_r4, K_vx_gemv_i8b1_q4_0_r8},
        {K_vx_gemv_i8b1_q8_0_r1, K_vx_gemv_i8b1_q8_0_r2, K_vx_gemv_i8b1_q8_0_r4, K_vx_gemv_i8b1_q8_0_r8},
        {K_vx_gemv_i8b1_q4_k_r1, K_vx_gemv_i8b1_q4_k_r2, K_vx_gemv_i8b1_q4_k_r4, K_vx_gemv_i8b1_q4_k_r8}};
    const int ri = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : 3;
    return tab[q_index(qt)][ri];
}

static int bn_kernel(uint32_t qt, int NB) {
    static const int tab[3][4] = {
        {K_vx_gemv_b2_q4_0_r2, K_vx_gemv_b4_q4_0_r2, K_vx_gemv_b8_q4_0_r2, K_vx_gemv_b16_q4_0_r2},
        {K_vx_gemv_b2_q8_0_r2, K_vx_gemv_b4_q8_0_r2, K_vx_gemv_b8_q8_0_r2, K_vx_gemv_b16_q8_0_r2},
        {K_vx_gemv_b2_q4_k_r2, K_vx_gemv_b4_q4_k_r2, K_vx_gemv_b8_q4_k_r2, K_vx_gemv_b16_q4_k_r2}};
    const int ni = NB == 2 ? 0 : NB == 4 ? 1 : NB == 8 ? 2 : 3;
    return tab[q_index(qt)][ni];
}

// Persistent batch-1 kernel with f32 x (VX_GEMV_X_F32); xv: x contiguous
// along K and 16-byte aligned (else the _xs form, strided x).
static int p1_kernel(uint32_t qt, bool xv) {
    static const int tab[2][3] = {{K_vx_gemv_p1_q4_0_w1024_xs, K_vx_gemv_p1_q8_0_w1024_xs, K_vx_gemv_p1_q4_k_w1024_xs},
                                  {K_vx_gemv_p1_q4_0_w1024, K_vx_gemv_p1_q8_0_w1024, K_vx_gemv_p1_q4_k_w1024}};
    return tab[xv ? 1 : 0][q_index(qt)];
}

// Persistent batch-1 kernel on the integer-dot path, by ring depth P (1 or
// 2; P = 0: the one-item-per-wave form, _p1e) and x layout (as p1_kernel).
static int p1i_kernel(uint32_t qt, int P, bool xv) {
    static const int tab[2][3][3] = {
        {{K_vx_gemv_p1i_q4_0_p1e_xs, K_vx_gemv_p1i_q4_0_p1_xs, K_vx_gemv_p1i_q4_0_p2_xs},
         {K_vx_gemv_p1i_q8_0_p1e_xs, K_vx_gemv_p1i_q8_0_p1_xs, K_vx_gemv_p1i_q8_0_p2_xs},
         {K_vx_gemv_p1i_q4_k_p1e_xs, K_vx_gemv_p1i_q4_k_p1_xs, K_vx_gemv_p1i_q4_k_p2_xs}},
        {{K_vx_gemv_p1i_q4_0_p1e, K_vx_gemv_p1i_q4_0_p1, K_vx_gemv_p1i_q4_0_p2},
         {K_vx_gemv_p1i_q8_0_p1e, K_vx_gemv_p1i_q8_0_p1, K_vx_gemv_p1i_q8_0_p2},
         {K_vx_gemv_p1i_q4_k_p1e, K_vx_gemv_p1i_q4_k_p1, K_vx_gemv_p1i_q4_k_p2}}};
    return tab[xv ? 1 : 0][q_index(qt)][P <= 0 ? 0 : P >= 2 ? 2 : 1];
}

static int generic_kernel(uint32_t qt) {
    return qt == VX_Q4_0 ? K_vx_gemv_generic_q4_0 : qt == VX_Q8_0 ? K_vx_gemv_generic_q8_0 : K_vx_gemv_generic_q4_k;
}

static int dequant_kernel(uint32_t qt) {
    return qt == VX_Q4_0 ? K_vx_dequant_q4_0 : qt == VX_Q8_0 ? K_vx_dequant_q8_0 : K_vx_dequant_q4_k;
}

// Rows per wave for batch 1: the largest R whose grid still gives every
// CU at least two workgroups.
static int pick_rows_per_wave(vx_ctx ctx, uint32_t qt, uint32_t M) {
    const int maxr = qt == VX_Q8_0 ? 4 : 8;
    for (int r = maxr; r > 1; r >>= 1)
        if ((M + 4u * r - 1) / (4u * r) >= 2u * (uint32_t)ctx->num_cus) return r;
    return 1;
}

// ------------------------------------------------- activation split
// vx_xq layout: levels [ceil(K/256) items][B][2][4][8][8] bytes, then scales
// f32 [K/32][B][2]
static uint64_t xq_levels_bytes(uint32_t K, uint32_t B) { return (uint64_t)((K + 255u) / 256u) * B * 512u; }

static int xq_size(uint32_t K, uint32_t B, uint64_t* bytes) {
    if (K % 32u) return fail(VX_ERR_UNSUPPORTED, "activation split: K is not a multiple of 32");
    *bytes = xq_levels_bytes(K, B) + (uint64_t)(K / 32u) * B * 8u;
    return VX_OK;
}

static int check_xq(const vx_xq* q) {
    if (!q) return fail(VX_ERR_INVALID, "null vx_xq");
    uint64_t nb;
    int s = xq_size(q->K, q->B, &nb);
    if (s) return s;
    if (nb && !q->base) return fail(VX_ERR_INVALID, "null vx_xq base");
    if (((uintptr_t)q->base & 15u) != 0) return fail(VX_ERR_INVALID, "vx_xq base is not 16-byte aligned");
    return VX_OK;
}

// x [K, B] view -> split into q (already checked). x is canonical [.., K, B].
static int launch_quantize_x(vx_ctx ctx, vx_stream stream, const vx_xq* q, const Canon& cx) {
    const uint32_t K = q->K, B = q->B;
    vx_xq_args a{};
    a.x = (const float*)cx.ptr;
    a.xs_k = cx.l.stride[2];
    a.xs_b = cx.l.stride[3];
    a.levels = (int8_t*)q->base;
    a.scales = (float*)((uint8_t*)q->base + xq_levels_bytes(K, B));
    a.K = K;
    a.B = B;
    a.nblk = K / 32u;
    a.x_vec = (a.xs_k == 1 && aligned16(cx.ptr) && (B == 1 || a.xs_b % 4 == 0)) ? 1u : 0u;
    const uint64_t threads = (uint64_t)a.nblk * B * 8u;
    if ((threads + 255u) / 256u > 0x7FFFFFFFull) return fail(VX_ERR_UNSUPPORTED, "activation split too large");
    return launch(ctx, K_vx_quantize_x, dim3((uint32_t)((threads + 255u) / 256u)), dim3(256), 0, stream, a);
}

// canonical [.., K, B] view of a rank-1 or rank-2 x
static int canon_x(const vx_cview* x, Canon* cx) {
    if (!x) return fail(VX_ERR_INVALID, "null view");
    if (x->layout.rank < 1 || x->layout.rank > 2) return fail(VX_ERR_SHAPE, "x must be [K] or [K, B]");
    vx_layout lx = x->layout;
    int s;
    if (lx.rank == 1 && (s = layout_unsqueeze(&x->layout, 1, &lx))) return s;
    return canon_view(x->base, &lx, cx, "x");
}

static int run_quantize_x(vx_ctx ctx, vx_stream stream, const vx_xq* q, const vx_cview* x) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    int s = check_xq(q);
    if (s) return s;
    Canon cx;
    if ((s = canon_x(x, &cx))) return s;
    if (cx.l.size[2] != q->K || cx.l.size[3] != q->B) {
        static thread_local std::string m;
        m = "activation split: x " + layout_str(cx.l) + " is not [K=" + std::to_string(q->K) + ", B=" +
            std::to_string(q->B) + "]";
        return fail(VX_ERR_SHAPE, m.c_str());
    }
    if (q->K == 0 || q->B == 0) return VX_OK;
    DeviceGuard guard(ctx->device);
    return launch_quantize_x(ctx, stream, q, cx);
}

// Batched GEMV kernel on split x: column groups ncg (1: B <= 8, 2: B <= 16),
// items per wave and pass xi, one pass or several (mp; K past 16 xi items).
// The multi-pass kernels use the largest xi of their format.
// Ring depth (tile-works in flight per wave) of each one-pass xq kernel, as
// instantiated in gemv_q.hip.
static int xq_ring(uint32_t qt, int ncg, int xi) {
    switch (q_index(qt)) {
    case 0: return ncg == 2 ? 3 : xi == 1 ? 3 : 1;
    case 1: return ncg == 2 ? 2 : xi == 1 ? 2 : 1;
    default: return ncg == 2 ? 2 : xi == 1 ? 3 : 1;
    }
}

// st: the straight-line kernel (one pass, every CU's tile-works within the
// ring); fx: the kernel that splits x itself (one pass only); fh: its form
// for <= 4 columns, each lane splitting half the blocks
static int xq_kernel(uint32_t qt, int ncg, int xi, bool mp, bool st, bool fx, bool fh = false) {
#define VX_XQK(N) (st ? K_vx_gemv_xq_##N##_st : K_vx_gemv_xq_##N)
#define VX_XQF(N) (fh ? (st ? K_vx_gemv_xq_##N##_st_fx4 : K_vx_gemv_xq_##N##_fx4) \
                      : (st ? K_vx_gemv_xq_##N##_st_fx : K_vx_gemv_xq_##N##_fx))
#define VX_XQF2(N) (st ? K_vx_gemv_xq_##N##_st_fx : K_vx_gemv_xq_##N##_fx)
#define VX_XQF4(N) (st ? K_vx_gemv_xq_##N##_st_fx4 : K_vx_gemv_xq_##N##_fx4)
    if (fx) {  // one pass; the shapes xq_fused_shape admits
        switch (q_index(qt)) {
        case 0:
            if (ncg == 2) return VX_XQF2(q4_0_c2_x1);
            return xi == 1 ? VX_XQF(q4_0_c1_x1) : xi == 2 ? VX_XQF(q4_0_c1_x2) : VX_XQF4(q4_0_c1_x3);
        case 1:
            if (ncg == 2) return VX_XQF2(q8_0_c2_x1);
            return xi == 1 ? VX_XQF(q8_0_c1_x1) : VX_XQF(q8_0_c1_x2);
        default:
            if (ncg == 2) return VX_XQF2(q4_k_c2_x1);
            return xi == 1 ? VX_XQF(q4_k_c1_x1) : VX_XQF(q4_k_c1_x2);
        }
    }
    switch (q_index(qt)) {
    case 0:
        if (ncg == 2) return mp ? K_vx_gemv_xq_q4_0_c2_x1_mp : VX_XQK(q4_0_c2_x1);
        if (mp) return K_vx_gemv_xq_q4_0_c1_x3_mp;
        return xi == 1 ? VX_XQK(q4_0_c1_x1) : xi == 2 ? VX_XQK(q4_0_c1_x2) : VX_XQK(q4_0_c1_x3);
    case 1:
        if (ncg == 2) return mp ? K_vx_gemv_xq_q8_0_c2_x1_mp : VX_XQK(q8_0_c2_x1);
        if (mp) return K_vx_gemv_xq_q8_0_c1_x2_mp;
        return xi == 1 ? VX_XQK(q8_0_c1_x1) : VX_XQK(q8_0_c1_x2);
    default:
        if (ncg == 2) return mp ? K_vx_gemv_xq_q4_k_c2_x1_mp : VX_XQK(q4_k_c2_x1);
        if (mp) return K_vx_gemv_xq_q4_k_c1_x2_mp;
        return xi == 1 ? VX_XQK(q4_k_c1_x1) : VX_XQK(q4_k_c1_x2);
    }
#undef VX_XQK
#undef VX_XQF
#undef VX_XQF2
#undef VX_XQF4
}

// Items per wave and pass for a launch of b columns: the x levels of XI items
// stay in registers (Q8_0's larger weight items leave room for two, Q4_K's
// header for two). Sets *mp when K needs several passes.
static int xq_items(uint32_t qt, uint32_t K, uint32_t b, bool* mp) {
    const uint32_t ipr = (K / 64u + 3u) / 4u;
    const int ximax = qt == VX_Q4_0 ? 3 : 2;
    const int xmax = b > 8u ? 1 : ximax;
    int xi = (int)((ipr + 15u) / 16u);
    *mp = xi > xmax;
    return *mp ? xmax : xi;
}

// Whether a launch of b (<= 16) columns has a kernel that splits x itself:
// one pass, and the split of the wave's slice fits the registers: one item
// per wave (one or two groups of 8 columns), two items with <= 8 columns, or
// three items with <= 4 columns (each lane splitting half the blocks).
static bool xq_fused_shape(uint32_t qt, uint32_t K, uint32_t b) {
    bool mp;
    const int xi = xq_items(qt, K, b, &mp);
    if (mp || b > 16u) return false;
    if (b > 8u) return xi == 1;
    return xi <= 2 || b <= 4u;
}

// y [.., M, B] (canonical) = W x, x given by its split q (q->K == K, q->B ==
// B), or, with q == nullptr, split inside the kernels from x itself (cx:
// stride 1 along K, 16-byte aligned columns; one pass, see xq_fused_ok).
// Launches of up to 16 columns; W is streamed once per launch.
static int launch_gemv_xq(vx_ctx ctx, vx_stream stream, const Canon& cy, const vx_qweight* w, const vx_xq* q,
                          const Canon* cx = nullptr, uint32_t Bx = 0) {
    const uint32_t M = w->rows, K = w->cols, B = q ? q->B : Bx;
    const bool fx = q == nullptr;
    vx_gemv_xq_args a{};
    a.w = (const uint8_t*)w->base;
    a.row_stride = w->row_stride_bytes;
    if (fx) {
        a.x = (const float*)cx->ptr;
        a.xs_b = cx->l.stride[3];
    } else {
        a.levels = (const int8_t*)q->base;
        a.scales = (const float*)((const uint8_t*)q->base + xq_levels_bytes(K, B));
    }
    a.ys_m = cy.l.stride[2];
    a.ys_b = cy.l.stride[3];
    a.M = M;
    a.K = K;
    a.nblk = K / 32u;
    a.nunits = K / 64u;
    a.ipr = (a.nunits + 3u) / 4u;
    a.xcols = B;
    for (uint32_t b0 = 0; b0 < B; b0 += 16u) {
        a.B = B - b0 < 16u ? B - b0 : 16u;
        a.col0 = b0;
        a.y = (float*)(cy.ptr + 4ull * (uint64_t)b0 * (uint64_t)cy.l.stride[3]);
        const int ncg = a.B > 8u ? 2 : 1;
        bool mp;
        const int xi = xq_items(w->qtype, K, a.B, &mp);
        if (fx && !xq_fused_shape(w->qtype, K, a.B))
            return fail(VX_ERR_UNSUPPORTED, "internal: no kernel splits x itself at this shape");
        a.npass = (a.ipr + 16u * (uint32_t)xi - 1u) / (16u * (uint32_t)xi);
        // 64 KB of parked partial sums + each of the 16 waves' scales (+ the
        // fused split's per-wave tables)
        const size_t lds = 65536u + (size_t)16u * 8u * (uint32_t)xi * 8u * (uint32_t)ncg * 8u + (fx ? 16u * 1536u : 0u);
        // the kernels' row split: balanced row ranges for one column group,
        // whole tiles for two (measured: Q4_K 14336x4096 / 32000x4096 B = 16
        // 0.35 / 0.7 us faster whole, B <= 8 0.1-0.35 us faster balanced);
        // every CU's tile-works must fit the ring for the _st kernels
        const uint32_t G = (uint32_t)ctx->num_cus;
        const uint32_t tmax = ncg == 2 ? ((M + 15u) / 16u + G - 1u) / G : ((M + G - 1u) / G + 15u) / 16u;
        const bool st = !mp && tmax <= (uint32_t)xq_ring(w->qtype, ncg, xi);
        int s = launch(ctx, xq_kernel(w->qtype, ncg, xi, mp, st, fx, a.B <= 4u), dim3(G), dim3(1024u), lds, stream, a);
        if (s) return s;
    }
    return VX_OK;
}

// The batched GEMV splits x inside its kernels (one launch, no workspace)
// when x has stride 1 along K with 16-byte aligned columns, B <= 16 and the
// shape has a fused kernel (xq_fused_shape). Measured per step against the
// split-then-GEMV route (graph replay): Q4_0 11008x4096 B = 8 13.0 -> 11.7
// us, 4096x11008 B = 4 (three items, half the blocks per lane) 13.6 -> 11.6
// us, Q4_K 32000x4096 B = 16 (two column groups) 29.6 -> 28.2 us, 14336x4096
// B = 16 18.2 -> 18.7 us (even: kept fused, it needs no workspace).
// With memory for the split (have_mem), two column groups (B = 9..16) take
// the split route below M = 24576: there every CU splitting all of x (16
// columns, two chunks per wave) costs more than the second launch (measured,
// graph-replayed: Q4_K 14336x4096 B = 16 fused 18.9 us, split 2.8 + GEMV
// 14.4 us; 32000x4096 28.2 against 2.8 + 26.2 us).
static bool xq_fused_ok(const vx_qweight* w, const Canon& cx, uint32_t B, bool have_mem = false) {
    if (B > 16u || cx.l.stride[2] != 1 || !aligned16(cx.ptr) || (B > 1u && cx.l.stride[3] % 4 != 0)) return false;
    if (have_mem && B > 8u && w->rows < 24576u) return false;
    return xq_fused_shape(w->qtype, w->cols, B);
}

static bool xq_layout_ok(const vx_qweight* w) {
    return w->cols > 0 && w->cols % 64u == 0 && ((uintptr_t)w->base & 3u) == 0 && w->row_stride_bytes % 4 == 0;
}

// canonical [.., M, B] view of a rank-1 or rank-2 y
static int canon_y(const vx_mview* y, Canon* cy) {
    if (!y) return fail(VX_ERR_INVALID, "null view");
    if (y->layout.rank < 1 || y->layout.rank > 2) return fail(VX_ERR_SHAPE, "y must be [M] or [M, B]");
    vx_layout ly = y->layout;
    int s;
    if (ly.rank == 1 && (s = layout_unsqueeze(&y->layout, 1, &ly))) return s;
    return canon_view(y->base, &ly, cy, "y");
}

static int run_gemv_q_xq(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_xq* q) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    uint32_t qk, bb;
    int s = check_qweight(w, &qk, &bb);
    if (s) return s;
    if ((s = check_xq(q))) return s;
    Canon cy;
    if ((s = canon_y(y, &cy))) return s;
    if (cy.l.size[2] != w->rows || q->K != w->cols || cy.l.size[3] != q->B) {
        static thread_local std::string m;
        m = "incompatible gemv shapes: y " + layout_str(cy.l) + " = W [" + std::to_string(w->rows) + ", " +
            std::to_string(w->cols) + "] x split [K=" + std::to_string(q->K) + ", B=" + std::to_string(q->B) + "]";
        return fail(VX_ERR_SHAPE, m.c_str());
    }
    if (w->rows == 0 || q->B == 0) return VX_OK;
    if (!xq_layout_ok(w))
        return fail(VX_ERR_UNSUPPORTED, "vx_gemv_q_xq needs K a multiple of 64 and 4-byte aligned weight rows");
    DeviceGuard guard(ctx->device);
    return launch_gemv_xq(ctx, stream, cy, w, q);
}

// Where the batched GEMV's activation split may go: nowhere (vx_gemv_q /
// _ex), a caller's workspace (vx_gemv_q_ws) or the module scratch
// (vx_gemv_q_noalloc).
enum SplitMem { SPLIT_NONE = 0, SPLIT_WS = 1, SPLIT_SCRATCH = 2 };

static int run_gemv_q(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_cview* x,
                      uint32_t flags, SplitMem mem = SPLIT_NONE, void* ws = nullptr, uint64_t ws_bytes = 0) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    uint32_t qk, bb;
    int s = check_qweight(w, &qk, &bb);
    if (s) return s;
    if (!y || !x) return fail(VX_ERR_INVALID, "null view");
    if (y->layout.rank < 1 || y->layout.rank > 2 || x->layout.rank < 1 || x->layout.rank > 2)
        return fail(VX_ERR_SHAPE, "y must be [M] or [M, B] and x [K] or [K, B]");
    // A rank-1 y / x is a column ([M] -> [M, 1], [K] -> [K, 1]).
    vx_layout ly = y->layout, lx = x->layout;
    if (ly.rank == 1 && (s = layout_unsqueeze(&y->layout, 1, &ly))) return s;
    if (lx.rank == 1 && (s = layout_unsqueeze(&x->layout, 1, &lx))) return s;
    Canon cy, cx;
    if ((s = canon_view(y->base, &ly, &cy, "y"))) return s;
    if ((s = canon_view(x->base, &lx, &cx, "x"))) return s;
    const uint32_t M = w->rows, K = w->cols;
    const uint32_t B = cy.l.size[3];
    if (cy.l.size[2] != M || cx.l.size[2] != K || cx.l.size[3] != B) {
        static thread_local std::string m;
        m = "incompatible gemv shapes: y " + layout_str(cy.l) + " = W [" + std::to_string(M) + ", " +
            std::to_string(K) + "] x " + layout_str(cx.l);
        return fail(VX_ERR_SHAPE, m.c_str());
    }
    if (M == 0 || B == 0) return VX_OK;
    DeviceGuard guard(ctx->device);

    vx_gemv_args a{};
    a.w = (const uint8_t*)w->base;
    a.row_stride = w->row_stride_bytes;
    a.xs_k = cx.l.stride[2];
    a.xs_b = cx.l.stride[3];
    a.ys_m = cy.l.stride[2];
    a.ys_b = cy.l.stride[3];
    a.M = M;
    a.K = K;
    a.nunits = K / 64;

    const bool fast = K > 0 && K % 64 == 0 && ((uintptr_t)w->base & 3u) == 0 && w->row_stride_bytes % 4 == 0;
    const size_t budget = ctx->lds_per_block < 160u * 1024u ? ctx->lds_per_block : 160u * 1024u;
    // x as two int8 levels per 32-block (the default) or exact f32 (VX_GEMV_X_F32)
    bool x_f32 = (flags & VX_GEMV_X_F32) != 0;
    if (mem == SPLIT_WS && ws && B >= 2 && !x_f32 && K % 64u == 0u) {
        // a caller workspace is checked against what the call may use
        // (vx_gemv_q_ws_size), whichever route the shape then takes
        uint64_t nb;
        if ((s = xq_size(K, B, &nb))) return s;
        if (ws_bytes < nb) {
            static thread_local std::string m;
            m = "vx_gemv_q_ws: x [K=" + std::to_string(K) + ", B=" + std::to_string(B) + "] needs " +
                std::to_string(nb) + " bytes of workspace, " + std::to_string(ws_bytes) + " given";
            return fail(VX_ERR_INVALID, m.c_str());
        }
    }
    const bool have_mem = mem == SPLIT_SCRATCH || (mem == SPLIT_WS && ws);
    if (B >= 2 && !x_f32 && xq_layout_ok(w) && xq_fused_ok(w, cx, B, have_mem)) {
        // the matrix-core GEMV splitting x itself: one launch per 16 columns,
        // W streamed once per launch, no workspace
        return launch_gemv_xq(ctx, stream, cy, w, nullptr, &cx, B);
    }
    if (B >= 2 && !x_f32 && xq_layout_ok(w)) {
        // split x once into memory (the caller's workspace or the module's
        // scratch), then the matrix-core GEMV on the split (W streamed once
        // per 16 columns)
        vx_xq q{nullptr, K, B};
        uint64_t nb;
        if ((s = xq_size(K, B, &nb))) return s;
        static thread_local std::string m;
        if (mem == SPLIT_SCRATCH) {
            // the module's scratch array: no allocation, a fixed maximum
            if (nb > ctx->scratch_bytes) {
                m = "vx_gemv_q_noalloc: the split of x [K=" + std::to_string(K) + ", B=" + std::to_string(B) +
                    "] needs " + std::to_string(nb) + " bytes, more than the " + std::to_string(ctx->scratch_bytes) +
                    "-byte scratch (ceil(K/256) * B * 512 + (K/32) * B * 8 must not exceed it)";
                return fail(VX_ERR_UNSUPPORTED, m.c_str());
            }
            q.base = ctx->scratch;
        } else if (mem == SPLIT_WS && ws) {
            q.base = ws;  // its size was checked above
        } else if (flags & VX_GEMV_X_INT8) {
            m = "the int8 split of x [K=" + std::to_string(K) + ", B=" + std::to_string(B) + "] at this shape needs " +
                std::to_string(nb) + " bytes of device memory: pass a workspace (vx_gemv_q_ws)";
            return fail(VX_ERR_UNSUPPORTED, m.c_str());
        }
        if (q.base) {
            if ((s = launch_quantize_x(ctx, stream, &q, cx))) return s;
            return launch_gemv_xq(ctx, stream, cy, w, &q);
        }
        // no memory for the split: exact f32 x (the VX_GEMV_X_F32 kernels)
        x_f32 = true;
    }
    // batch-1 kernel: the persistent one, or the per-row-group one when x
    // does not fit the persistent kernel's LDS (K > 16384); int8 x unless
    // VX_GEMV_X_F32
    uint32_t b0 = 0;
    while (b0 < B) {
        const uint32_t rem = B - b0;
        const int NB = rem >= 16 ? 16 : rem >= 8 ? 8 : rem >= 4 ? 4 : rem >= 2 ? 2 : 1;
        a.x = (const float*)(cx.ptr + 4ull * (uint64_t)b0 * (uint64_t)cx.l.stride[3]);
        a.y = (float*)(cy.ptr + 4ull * (uint64_t)b0 * (uint64_t)cy.l.stride[3]);
        a.B = NB;
        a.x_vec = (a.xs_k == 1 && aligned16((uintptr_t)a.x) && (NB == 1 || a.xs_b % 4 == 0)) ? 1u : 0u;
        if (!fast) {
            a.B = rem;
            return launch(ctx, generic_kernel(w->qtype), dim3((M + 3) / 4), dim3(VX_WG), 0, stream, a);
        }
        int k;
        uint32_t rows_per_wg;
        size_t lds;
        if (NB == 1 && !x_f32 && a.nunits <= 256u) {
            // persistent integer-dot path: all of x as int8 levels, 152 B per unit
            a.chunk_units = a.nunits;
            a.upitch = a.nunits | 1u;
            lds = (size_t)a.upitch * 152u;
            // Ring of one item per wave where a row is one pass (K <= 4096):
            // fewer requests in flight per wave, and the x loads queue behind
            // fewer weight requests (Q4_0 11008 x 4096 6.90 -> 6.46 us, Q4_K
            // 14336 x 4096 8.27 -> 7.66 us). Several passes keep a ring of two
            // (Q4_0 4096 x 11008 7.82 against 8.18 us with one), except Q8_0
            // (68-byte units) with at most two items per wave, where the
            // second slot would only load a repeat of the last item (2048 x
            // 4096 4.57 -> 4.09 us, 4096 x 8192 8.75 -> 8.45 us).
            const uint32_t waves = (uint32_t)ctx->num_cus * 16u;
            const uint32_t npass = (a.nunits + 63u) / 64u;
            const uint32_t items = (M + waves - 1u) / waves * npass;
            // One item per wave: no barrier between the x and the weight
            // requests (_p1e; Q8_0 4096 x 4096 5.37 -> 5.15 us).
            const int ring = items == 1u ? 0 : (npass == 1u || (w->qtype == VX_Q8_0 && items <= 2u)) ? 1 : 2;
            s = launch_b1(ctx, p1i_kernel(w->qtype, ring, a.x_vec != 0), (uint32_t)ctx->num_cus, lds, stream, a);
            if (s) return s;
            b0 += NB;
            continue;
        } else if (NB == 1 && !x_f32) {
            // integer-dot path: 152 bytes of LDS per staged unit
            const int R = pick_rows_per_wave(ctx, w->qtype, M);
            uint32_t cu = a.nunits;
            const uint32_t cap = (uint32_t)(budget < 65536 ? budget : 65536) / 152u - 1u;
            if (cu > cap) cu = cap;
            a.chunk_units = cu;
            a.upitch = cu | 1u;
            k = i8b1_kernel(w->qtype, R);
            rows_per_wg = 4u * R;
            lds = (size_t)a.upitch * 152u;
        } else if (NB == 1 && a.nunits <= 256u) {
            // Persistent path: one workgroup per CU, all of x in LDS
            // (16 slots x odd pitch x 16 B) plus the per-unit block sums.
            a.chunk_units = a.nunits;
            a.upitch = a.nunits | 1u;
            lds = (size_t)16u * a.upitch * 16u + (size_t)a.nunits * 8u;
            s = launch_b1(ctx, p1_kernel(w->qtype, a.x_vec != 0), (uint32_t)ctx->num_cus, lds, stream, a);
            if (s) return s;
            b0 += NB;
            continue;
        } else if (NB == 1) {
            const int R = pick_rows_per_wave(ctx, w->qtype, M);
            // x chunk: up to 255 units (16 slots x odd pitch x 16 B <= 64 KB)
            uint32_t cu = a.nunits;
            const uint32_t cap = (uint32_t)(budget < 65536 ? budget : 65536) / 256u - 1u;
            if (cu > cap) cu = cap;
            a.chunk_units = cu;
            a.upitch = cu | 1u;
            k = b1_kernel(w->qtype, R);
            rows_per_wg = 4u * R;
            lds = (size_t)NB * 16u * a.upitch * 16u;
        } else {
            const uint32_t LPR = NB <= 4 ? 64u : NB == 8 ? 32u : 16u;
            // Largest multiple of LPR whose [NB][16][pitch] float4 block fits.
            // An odd pitch keeps the staging stores conflict free; an even
            // one is used when the odd pitch would not fit.
            uint32_t cu = LPR;
            while (cu + LPR <= ((a.nunits + LPR - 1) / LPR) * LPR &&
                   (size_t)NB * 16u * (cu + LPR) * 16u <= budget)
                cu += LPR;
            if ((size_t)NB * 16u * cu * 16u > budget) return fail(VX_ERR_UNSUPPORTED, "LDS budget too small");
            a.chunk_units = cu;
            a.upitch = ((size_t)NB * 16u * (cu | 1u) * 16u <= budget) ? (cu | 1u) : cu;
            k = bn_kernel(w->qtype, NB);
            rows_per_wg = 4u * (64u / LPR) * 2u;
            lds = (size_t)NB * 16u * a.upitch * 16u;
        }
        s = launch(ctx, k, dim3((M + rows_per_wg - 1) / rows_per_wg), dim3(VX_WG), lds, stream, a);
        if (s) return s;
        b0 += NB;
    }
    return VX_OK;
}

// Read probe: vx_gemv_p1i's loads of W alone (measurement).
static int run_read_probe(vx_ctx ctx, vx_stream stream, const vx_qweight* w, float* y) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    uint32_t qk, bb;
    int s = check_qweight(w, &qk, &bb);
    if (s) return s;
    if (w->rows && !y) return fail(VX_ERR_INVALID, "null y");
    if (!xq_layout_ok(w))
        return fail(VX_ERR_UNSUPPORTED, "read probe needs K a multiple of 64 and 4-byte aligned weight rows");
    if (w->rows == 0) return VX_OK;
    DeviceGuard guard(ctx->device);
    vx_gemv_args a{};
    a.w = (const uint8_t*)w->base;
    a.row_stride = w->row_stride_bytes;
    a.y = y;
    a.ys_m = 1;
    a.M = w->rows;
    a.K = w->cols;
    a.nunits = w->cols / 64u;
    const int k = q_index(w->qtype) == 0 ? K_vx_read_probe_q4_0 : q_index(w->qtype) == 1 ? K_vx_read_probe_q8_0
                                                                                         : K_vx_read_probe_q4_k;
    return launch_b1(ctx, k, (uint32_t)ctx->num_cus, 0, stream, a);
}

// Launch floor: an empty kernel on the batch-1 GEMV's grid (measurement).
static int run_launch_floor(vx_ctx ctx, vx_stream stream) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    DeviceGuard guard(ctx->device);
    vx_gemv_args a{};
    return launch_b1(ctx, K_vx_launch_floor_k, (uint32_t)ctx->num_cus, 0, stream, a);
}

// ------------------------------------------------------------ contiguous
static vx_udiv make_udiv(uint32_t d) {
    vx_udiv r{};
    if (d <= 1u) {
        r.one = 1u;
        return r;
    }
    uint32_t l = 0;
    while (l < 32u && (1ull << l) < d) ++l;  // ceil(log2 d)
    r.m = (uint32_t)((((1ull << 32) * ((1ull << l) - d)) / d) + 1ull);
    r.s = l - 1u;
    return r;
}

static int run_contiguous(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* src,
                          const uint32_t* dev_offset) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    if (!out || !src) return fail(VX_ERR_INVALID, "null view");
    // src/linalg/contiguous.rs:43-48: equal size arrays, contiguous output
    if (std::memcmp(out->layout.size, src->layout.size, sizeof(out->layout.size)) != 0) {
        static thread_local std::string m;
        m = "contiguous: tensor size " + layout_str(src->layout) + " differs from output size " + layout_str(out->layout);
        return fail(VX_ERR_SHAPE, m.c_str());
    }
    if (out->layout.rank > 4 || src->layout.rank > 4) return fail(VX_ERR_UNSUPPORTED, "rank > 4");
    if (!layout_is_contiguous(&out->layout)) {
        static thread_local std::string m;
        m = "Output tensor must be contiguous: " + layout_str(out->layout) + ".";
        return fail(VX_ERR_SHAPE, m.c_str());
    }
    vx_layout c;
    int s = layout_canonicalize(&src->layout, &c);
    if (s) return s;
    uint64_t total = 1;
    for (int i = 0; i < 4; ++i) total *= c.size[i];
    if (total == 0) return VX_OK;
    if (total >= (1ull << 32)) return fail(VX_ERR_UNSUPPORTED, "contiguous: 2^32 elements or more");
    vx_copy_args a{};
    // Without a device offset the view's own offset is the base shift
    // (TensorRef::buffer); with one, the raw buffer is read at that offset
    // (TensorRef::raw_buffer, contiguous.rs:63-71), as the reference does.
    a.src = (const uint32_t*)src->base + (dev_offset ? 0u : src->layout.offset);
    a.dst = (uint32_t*)out->base + out->layout.offset;
    a.dev_offset = dev_offset;
    for (int i = 0; i < 4; ++i) {
        a.stride[i] = c.stride[i];
        a.size[i] = c.size[i];
    }
    a.total = (uint32_t)total;
    a.dw = make_udiv(c.size[3]);
    a.dh = make_udiv(c.size[2]);
    a.dc = make_udiv(c.size[1]);
    DeviceGuard guard(ctx->device);
    const bool tile = c.stride[2] == 1u && c.stride[3] != 1u && c.size[2] >= 16u && c.size[3] >= 16u;
    // 16-byte tiles: every float4 of a row (along h in, along w out) aligned
    // 128 x 128 tiles (66 KB of LDS, 2 workgroups per CU) when there are at
    // least 8 per CU, else 128 (h) x 64 (w) tiles (33 KB, 4 per CU): 8192^2
    // 4.73 vs 4.64 TB/s, 4096^2 4.27 vs 4.91 TB/s.
    const uint64_t nbig = (uint64_t)((c.size[3] + 127u) / 128u) * ((c.size[2] + 127u) / 128u) * c.size[0] * c.size[1];
    const bool big = nbig >= 8ull * (uint64_t)ctx->num_cus;
    const uint64_t ntiles128 = big ? nbig
                                   : (uint64_t)((c.size[3] + 63u) / 64u) * ((c.size[2] + 127u) / 128u) * c.size[0] *
                                         c.size[1];
    const bool tile16 = tile && !dev_offset && c.size[2] % 4u == 0u && c.size[3] % 4u == 0u &&
                        c.stride[0] % 4 == 0 && c.stride[1] % 4 == 0 && c.stride[3] % 4 == 0 &&
                        aligned16((uintptr_t)a.src) && aligned16((uintptr_t)a.dst) && ntiles128 < (1ull << 32);
    if (tile16) {
        const uint64_t maxb = (uint64_t)ctx->num_cus * 8u;
        return launch(ctx, big ? K_vx_contiguous_t128 : K_vx_contiguous_t128x64,
                      dim3((uint32_t)(ntiles128 < maxb ? ntiles128 : maxb)), dim3(256), 0, stream, a);
    }
    if (tile) {
        auto cap = [](uint64_t v) { return (uint32_t)(v < 65535u ? v : 65535u); };
        return launch(ctx, K_vx_contiguous_t64, dim3(cap((c.size[3] + 63u) / 64u), cap((c.size[2] + 63u) / 64u),
                                                     cap((uint64_t)c.size[0] * c.size[1])),
                      dim3(256), 0, stream, a);
    }
    const bool v4 = !dev_offset && c.stride[3] == 1u && c.size[3] % 4u == 0u && c.stride[0] % 4u == 0u &&
                    c.stride[1] % 4u == 0u && c.stride[2] % 4u == 0u && aligned16((uintptr_t)a.src) &&
                    aligned16((uintptr_t)a.dst);
    uint64_t blocks = ((v4 ? total / 4u : total) + 255u) / 256u;
    const uint64_t maxb = (uint64_t)ctx->num_cus * 32u;
    if (blocks > maxb) blocks = maxb;
    return launch(ctx, v4 ? K_vx_contiguous_v4 : K_vx_contiguous_gen, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
}

// ------------------------------------------------------------- quantize
static int run_quantize(vx_ctx ctx, vx_stream stream, const vx_qweight* out, const vx_cview* x) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    uint32_t qk, bb;
    int s = check_qweight(out, &qk, &bb);
    if (s) return s;
    if (!x) return fail(VX_ERR_INVALID, "null view");
    if (x->layout.rank != 2) return fail(VX_ERR_SHAPE, "quantize input must be a rank-2 [M, K] view");
    Canon cx;
    if ((s = canon_view(x->base, &x->layout, &cx, "x"))) return s;
    if (cx.l.size[2] != out->rows || cx.l.size[3] != out->cols) return fail(VX_ERR_SHAPE, "input view is not [rows, cols]");
    if (out->rows == 0 || out->cols == 0) return VX_OK;
    // block stores: 16-bit (Q8_0, Q4_0) or 32-bit (Q4_K)
    const uint64_t al = out->qtype == VX_Q4_K ? 4u : 2u;
    if (((uintptr_t)out->base % al) || (out->row_stride_bytes % al))
        return fail(VX_ERR_UNSUPPORTED, "quantize output must be 2-byte (Q4_K: 4-byte) aligned");
    vx_quant_args a{};
    a.x = (const float*)cx.ptr;
    a.xs_m = cx.l.stride[2];
    a.xs_k = cx.l.stride[3];
    a.out = (uint8_t*)out->base;
    a.row_stride = out->row_stride_bytes;
    a.M = out->rows;
    a.K = out->cols;
    a.nblk = out->cols / qk;
    a.x_vec = (a.xs_k == 1 && aligned16(cx.ptr) && a.xs_m % 4 == 0) ? 1u : 0u;
    DeviceGuard guard(ctx->device);
    if (out->qtype == VX_Q4_K) {
        // 32 super-blocks of the flattened (row, super-block) sequence per workgroup, grid-stride
        uint64_t blocks = ((uint64_t)a.M * a.nblk + 31u) / 32u;
        const uint64_t maxb = (uint64_t)ctx->num_cus * 64u;
        if (blocks > maxb) blocks = maxb;
        return launch(ctx, K_vx_quantize_q4_k, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
    }
    if (out->qtype == VX_Q8_0) {
        // rounds of 256 blocks of the flattened (row, block) sequence, grid-stride
        uint64_t blocks = ((uint64_t)a.M * a.nblk + 255u) / 256u;
        const uint64_t maxb = (uint64_t)ctx->num_cus * 16u;
        if (blocks > maxb) blocks = maxb;
        return launch(ctx, K_vx_quantize_q8_0, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
    }
    const uint32_t gy = a.M < 65535u ? a.M : 65535u;
    return launch(ctx, K_vx_quantize_q4_0, dim3((a.nblk + 255u) / 256u, gy), dim3(256), 0, stream, a);
}

static int run_dequant(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_qweight* w) {
    clear_error();
    if (!ctx) return fail(VX_ERR_INVALID, "null ctx");
    uint32_t qk, bb;
    int s = check_qweight(w, &qk, &bb);
    if (s) return s;
    if (!out) return fail(VX_ERR_INVALID, "null view");
    if (out->layout.rank != 2) return fail(VX_ERR_SHAPE, "dequantize output must be a rank-2 [M, K] view");
    Canon co;
    if ((s = canon_view(out->base, &out->layout, &co, "out"))) return s;
    if (co.l.size[2] != w->rows || co.l.size[3] != w->cols) return fail(VX_ERR_SHAPE, "output view is not [M, K]");
    const uint64_t groups = (uint64_t)w->rows * (w->cols / 32u);
    if (!groups) return VX_OK;
    if ((groups + VX_WG - 1) / VX_WG > 0x7FFFFFFFull) return fail(VX_ERR_UNSUPPORTED, "matrix too large");
    DeviceGuard guard(ctx->device);
    vx_gemv_args a{};
    a.w = (const uint8_t*)w->base;
    a.row_stride = w->row_stride_bytes;
    a.y = (float*)co.ptr;
    a.ys_m = co.l.stride[2];
    a.ys_b = co.l.stride[3];
    a.M = w->rows;
    a.K = w->cols;
    return launch(ctx, dequant_kernel(w->qtype), dim3((uint32_t)((groups + VX_WG - 1) / VX_WG)), dim3(VX_WG), 0,
                  stream, a);
}

}  // namespace vx

// ================================================================= C ABI
extern "C" {

int vx_init(int device, vx_ctx* out_ctx) {
    vx::clear_error();
    return vx::init(device, out_ctx);
}

int vx_destroy(vx_ctx ctx) {
    vx::clear_error();
    if (!ctx) return VX_OK;
    vx::DeviceGuard guard(ctx->device);
    for (hipModule_t m : ctx->mods)
        if (m) (void)hipModuleUnload(m);
    delete ctx;
    return VX_OK;
}

int vx_device_info(vx_ctx ctx, int* device, int* num_cus) {
    if (!ctx) return vx::fail(VX_ERR_INVALID, "null ctx");
    if (device) *device = ctx->device;
    if (num_cus) *num_cus = ctx->num_cus;
    return VX_OK;
}

int vx_gemm_f32(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs) {
    return vx::run_gemm(ctx, stream, out, lhs, rhs, vx::FORCE_AUTO);
}

int vx_gemm_f32_ex(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs,
                   const vx_gemm_opts* opts) {
    return vx::run_gemm(ctx, stream, out, lhs, rhs, vx::FORCE_AUTO, opts);
}

int vx_gemm_f32_naive(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs) {
    return vx::run_gemm(ctx, stream, out, lhs, rhs, vx::FORCE_NAIVE);
}

int vx_gemm_f32_tiled(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs) {
    return vx::run_gemm(ctx, stream, out, lhs, rhs, vx::FORCE_TILED);
}

int vx_gemm_f32_route(const vx_mview* out, const vx_cview* lhs, const vx_cview* rhs, int* route) {
    vx::clear_error();
    if (!route) return vx::fail(VX_ERR_INVALID, "null route");
    vx::GemmPlan p;
    const int s = vx::plan_gemm(out, lhs, rhs, vx::FORCE_AUTO, &p);
    if (s) return s;
    *route = p.route;
    return VX_OK;
}

int vx_gemv_q(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_cview* x) {
    return vx::run_gemv_q(ctx, stream, y, w, x, 0u);
}

int vx_gemv_q_ex(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_cview* x,
                 uint32_t flags) {
    if (flags & ~(uint32_t)(VX_GEMV_X_INT8 | VX_GEMV_X_F32)) return vx::fail(VX_ERR_INVALID, "unknown vx_gemv_q_ex flags");
    if ((flags & VX_GEMV_X_INT8) && (flags & VX_GEMV_X_F32))
        return vx::fail(VX_ERR_INVALID, "VX_GEMV_X_INT8 and VX_GEMV_X_F32 are exclusive");
    return vx::run_gemv_q(ctx, stream, y, w, x, flags);
}

int vx_gemv_q_ws(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_cview* x,
                 uint32_t flags, void* workspace, uint64_t workspace_bytes) {
    if (flags & ~(uint32_t)(VX_GEMV_X_INT8 | VX_GEMV_X_F32)) return vx::fail(VX_ERR_INVALID, "unknown vx_gemv_q_ws flags");
    if ((flags & VX_GEMV_X_INT8) && (flags & VX_GEMV_X_F32))
        return vx::fail(VX_ERR_INVALID, "VX_GEMV_X_INT8 and VX_GEMV_X_F32 are exclusive");
    if (((uintptr_t)workspace & 15u) != 0) return vx::fail(VX_ERR_INVALID, "workspace is not 16-byte aligned");
    return vx::run_gemv_q(ctx, stream, y, w, x, flags, vx::SPLIT_WS, workspace, workspace_bytes);
}

int vx_gemv_q_ws_size(uint32_t qtype, uint32_t K, uint32_t B, uint32_t flags, uint64_t* bytes) {
    vx::clear_error();
    if (!bytes) return vx::fail(VX_ERR_INVALID, "null bytes");
    uint32_t qk, bb;
    int s = vx::qinfo(qtype, &qk, &bb);
    if (s) return s;
    *bytes = 0;
    if (B < 2 || (flags & VX_GEMV_X_F32) || K % 64u != 0u) return VX_OK;
    return vx::xq_size(K, B, bytes);
}

int vx_xq_size(uint32_t K, uint32_t B, uint64_t* bytes) {
    vx::clear_error();
    if (!bytes) return vx::fail(VX_ERR_INVALID, "null bytes");
    return vx::xq_size(K, B, bytes);
}

int vx_quantize_x(vx_ctx ctx, vx_stream stream, const vx_xq* out, const vx_cview* x) {
    return vx::run_quantize_x(ctx, stream, out, x);
}

int vx_gemv_q_xq(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_xq* x) {
    return vx::run_gemv_q_xq(ctx, stream, y, w, x);
}

int vx_gemv_q_read_probe(vx_ctx ctx, vx_stream stream, const vx_qweight* w, float* y) {
    return vx::run_read_probe(ctx, stream, w, y);
}

int vx_launch_floor(vx_ctx ctx, vx_stream stream) { return vx::run_launch_floor(ctx, stream); }

int vx_dequantize(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_qweight* w) {
    return vx::run_dequant(ctx, stream, out, w);
}

int vx_gemv_q_noalloc(vx_ctx ctx, vx_stream stream, const vx_mview* y, const vx_qweight* w, const vx_cview* x,
                      uint32_t flags) {
    if (flags & ~(uint32_t)(VX_GEMV_X_INT8 | VX_GEMV_X_F32))
        return vx::fail(VX_ERR_INVALID, "unknown vx_gemv_q_noalloc flags");
    if ((flags & VX_GEMV_X_INT8) && (flags & VX_GEMV_X_F32))
        return vx::fail(VX_ERR_INVALID, "VX_GEMV_X_INT8 and VX_GEMV_X_F32 are exclusive");
    return vx::run_gemv_q(ctx, stream, y, w, x, flags, vx::SPLIT_SCRATCH);
}

int vx_quantize(vx_ctx ctx, vx_stream stream, const vx_qweight* out, const vx_cview* x) {
    return vx::run_quantize(ctx, stream, out, x);
}

int vx_contiguous(vx_ctx ctx, vx_stream stream, const vx_mview* out, const vx_cview* src, const uint32_t* dev_offset) {
    return vx::run_contiguous(ctx, stream, out, src, dev_offset);
}

int vx_qtype_info(uint32_t qtype, uint32_t* block_weights, uint32_t* block_bytes) {
    vx::clear_error();
    uint32_t qk, bb;
    const int s = vx::qinfo(qtype, &qk, &bb);
    if (s) return s;
    if (block_weights) *block_weights = qk;
    if (block_bytes) *block_bytes = bb;
    return VX_OK;
}

int vx_layout_contiguous(const uint32_t* size, uint32_t rank, vx_layout* out) {
    vx::clear_error();
    if (!out) return vx::fail(VX_ERR_INVALID, "null out");
    return vx::layout_contiguous(size, rank, out);
}
int vx_layout_canonicalize(const vx_layout* in, vx_layout* out) {
    vx::clear_error();
    if (!in || !out) return vx::fail(VX_ERR_INVALID, "null layout");
    return vx::layout_canonicalize(in, out);
}
int vx_layout_transpose(const vx_layout* in, uint32_t a, uint32_t b, vx_layout* out) {
    vx::clear_error();
    if (!in || !out) return vx::fail(VX_ERR_INVALID, "null layout");
    return vx::layout_transpose(in, a, b, out);
}
int vx_layout_broadcast(const vx_layout* a, const vx_layout* b, vx_layout* a_out, vx_layout* b_out) {
    vx::clear_error();
    if (!a || !b || !a_out || !b_out) return vx::fail(VX_ERR_INVALID, "null layout");
    return vx::layout_broadcast(a, b, a_out, b_out);
}
int vx_layout_view(const vx_layout* in, uint32_t offset, const uint32_t* shape, uint32_t rank,
                   const uint32_t* strides, uint32_t nstrides, vx_layout* out) {
    vx::clear_error();
    if (!in || !out || (rank && !shape)) return vx::fail(VX_ERR_INVALID, "null argument");
    return vx::layout_view(in, offset, shape, rank, strides, nstrides, out);
}
int vx_layout_narrow(const vx_layout* in, uint32_t axis, uint32_t first, uint32_t count, vx_layout* out) {
    vx::clear_error();
    if (!in || !out) return vx::fail(VX_ERR_INVALID, "null layout");
    return vx::layout_narrow(in, axis, first, count, out);
}
int vx_layout_unsqueeze(const vx_layout* in, uint32_t axis, vx_layout* out) {
    vx::clear_error();
    if (!in || !out) return vx::fail(VX_ERR_INVALID, "null layout");
    return vx::layout_unsqueeze(in, axis, out);
}
int vx_layout_is_contiguous(const vx_layout* in) { return in && vx::layout_is_contiguous(in) ? 1 : 0; }

const char* vx_status_string(int status) {
    switch (status) {
    case VX_OK: return "VX_OK";
    case VX_ERR_SHAPE: return "VX_ERR_SHAPE";
    case VX_ERR_UNSUPPORTED: return "VX_ERR_UNSUPPORTED";
    case VX_ERR_INVALID: return "VX_ERR_INVALID";
    case VX_ERR_HIP: return "VX_ERR_HIP";
    case VX_ERR_NO_CODE_OBJECT: return "VX_ERR_NO_CODE_OBJECT";
    case VX_ERR_IO: return "VX_ERR_IO";
    case VX_ERR_FORMAT: return "VX_ERR_FORMAT";
    case VX_ERR_NOT_FOUND: return "VX_ERR_NOT_FOUND";
    default: return "VX_ERR_UNKNOWN";
    }
}

const char* vx_last_error_message(void) { return vx::t_msg.c_str(); }
int vx_last_hip_error(void) { return vx::t_hip; }

}  // extern "C"
