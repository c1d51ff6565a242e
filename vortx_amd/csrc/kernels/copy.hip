// copy.hip — strided -> contiguous copy of 4-byte elements for gfx950.
//
// The op of vortx's Contiguous::launch (src/linalg/contiguous.rs:22-119;
// shader vortx-shaders/src/linalg/contiguous.rs:59-90): out[i] = src[off +
// n*s0 + c*s1 + h*s2 + w*s3] for the canonical [n, c, h, w] view, i the
// row-major index. Indices are 64-bit here (the shader's u32 `it` wraps past
// 2^32 elements).
//
// Four kernels (one in two tile shapes), all HBM-bound (8 bytes of traffic
// per element):
//   vx_contiguous_gen  any strides; one element per lane per step, the
//                      row-major index split with precomputed reciprocals;
//                      reads are coalesced when s3 == 1;
//   vx_contiguous_v4   the same with 16-byte moves for aligned rows with
//                      s3 == 1 and W % 4 == 0;
//   vx_contiguous_t64  views whose h axis is the contiguous one (s2 == 1,
//                      e.g. a transposed matrix): 64 x 64 tiles through LDS
//                      so that both the reads (along h) and the writes
//                      (along w) are coalesced;
//   vx_contiguous_t128 the same views when 16-byte moves are aligned (H, W,
//   (and _t128x64)     s0, s1, s3 multiples of 4, aligned bases): 128 x 128
//                      (or 128 x 64) tiles, float4 reads along h and float4
//                      writes along w (a quarter of the memory instructions,
//                      512-byte segments), a grid-stride loop over tiles.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../vx_kargs.h"
#include "vx_args.hpp"

// q = n / d with a precomputed multiplier (Granlund-Montgomery, as in
// libdivide's branch-free u32 form): for d >= 2, l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, s = l - 1, and
// q = (t + ((n - t) >> 1)) >> s with t = umulhi(n, m); d == 1 is flagged.
__device__ __forceinline__ uint32_t vx_div(uint32_t n, const vx_udiv& d) {
    if (d.one) return n;
    const uint32_t t = __umulhi(n, d.m);
    return (t + ((n - t) >> 1)) >> d.s;
}

extern "C" __global__ __launch_bounds__(256) void vx_contiguous_gen(vx_copy_args a) {
    vx_args_fetch(a);
    const int64_t off = a.dev_offset ? (int64_t)*a.dev_offset : 0;
    // 64-bit loop index: with total just below 2^32, a u32 i + stride would
    // wrap below total and the loop would never end
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t i64 = (uint64_t)blockIdx.x * 256u + threadIdx.x; i64 < a.total; i64 += stride) {
        const uint32_t i = (uint32_t)i64;          // < total < 2^32
        const uint32_t r1 = vx_div(i, a.dw);       // i / W
        const uint32_t w = i - r1 * a.size[3];
        const uint32_t r2 = vx_div(r1, a.dh);      // / H
        const uint32_t h = r1 - r2 * a.size[2];
        const uint32_t n = vx_div(r2, a.dc);       // / C
        const uint32_t c = r2 - n * a.size[1];
        const int64_t k = off + (int64_t)n * a.stride[0] + (int64_t)c * a.stride[1] + (int64_t)h * a.stride[2] +
                          (int64_t)w * a.stride[3];
        a.dst[i] = a.src[k];
    }
}

// 16-byte variant of vx_contiguous_gen for views with s3 == 1, W % 4 == 0
// and 16-byte aligned rows (base, offsets and s0..s2 multiples of 4; the host
// checks): lane i moves elements 4i..4i+3, which share n, c, h.
extern "C" __global__ __launch_bounds__(256) void vx_contiguous_v4(vx_copy_args a) {
    vx_args_fetch(a);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const uint32_t total4 = a.total >> 2;
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t j = (uint64_t)blockIdx.x * 256u + threadIdx.x; j < total4; j += stride) {
        const uint32_t i = (uint32_t)j << 2;
        const uint32_t r1 = vx_div(i, a.dw);
        const uint32_t w = i - r1 * a.size[3];
        const uint32_t r2 = vx_div(r1, a.dh);
        const uint32_t h = r1 - r2 * a.size[2];
        const uint32_t n = vx_div(r2, a.dc);
        const uint32_t c = r2 - n * a.size[1];
        const int64_t k = (int64_t)n * a.stride[0] + (int64_t)c * a.stride[1] + (int64_t)h * a.stride[2] + (int64_t)w;
        *(u32x4*)(a.dst + i) = *(const u32x4*)(a.src + k);
    }
}

// grid: x = tiles along w, y = tiles along h, z = n * c slices (loops past
// the grid limits). Block 256 threads = 4 waves.
extern "C" __global__ __launch_bounds__(256) void vx_contiguous_t64(vx_copy_args a) {
    vx_args_fetch(a);
    __shared__ uint32_t tile[64][65];
    const int64_t off = a.dev_offset ? (int64_t)*a.dev_offset : 0;
    const uint32_t H = a.size[2], W = a.size[3], C = a.size[1];
    const uint32_t nc_total = a.size[0] * C;
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    for (uint32_t nc = blockIdx.z; nc < nc_total; nc += gridDim.z) {
        const uint32_t n = nc / C, c = nc - n * C;
        const int64_t sbase = off + (int64_t)n * a.stride[0] + (int64_t)c * a.stride[1];
        const uint64_t dbase = (uint64_t)nc * H * W;
        for (uint32_t h0 = blockIdx.y * 64u; h0 < H; h0 += gridDim.y * 64u) {
            for (uint32_t w0 = blockIdx.x * 64u; w0 < W; w0 += gridDim.x * 64u) {
                __syncthreads();
                // read: lane = h offset (stride 1 in memory), waves step w
                const uint32_t h = h0 + lane;
#pragma unroll 4
                for (uint32_t j = wv; j < 64u; j += 4u) {
                    const uint32_t w = w0 + j;
                    if (h < H && w < W) tile[j][lane] = a.src[sbase + (int64_t)h + (int64_t)w * a.stride[3]];
                }
                __syncthreads();
                // write: lane = w offset (contiguous in out), waves step h
                const uint32_t w = w0 + lane;
#pragma unroll 4
                for (uint32_t i = wv; i < 64u; i += 4u) {
                    const uint32_t hh = h0 + i;
                    if (hh < H && w < W) a.dst[dbase + (uint64_t)hh * W + w] = tile[lane][i];
                }
            }
        }
    }
}

// grid: a multiple of the CU count, looping over tiles (n c, h-band, w-band)
// with w fastest. 256 threads; each phase moves the TH x TW tile as float4,
// thread t taking float4 t + 256 i. LDS holds the tile as [w][h] with pitch
// TH + 1 so the column reads of the write phase fall in different banks.
template <uint32_t TH, uint32_t TW>
__device__ __forceinline__ void vx_contiguous_tile16(const vx_copy_args& a) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr uint32_t P = TH + 1u, NV = TH * TW / 1024u, QH = TH / 4u, QW = TW / 4u;
    __shared__ uint32_t tile[TW * P];
    const uint32_t H = a.size[2], W = a.size[3], C = a.size[1];
    const uint32_t tw_n = (W + TW - 1u) / TW, th_n = (H + TH - 1u) / TH;
    const uint32_t per_nc = tw_n * th_n;
    const uint32_t ntiles = per_nc * a.size[0] * C;  // < 2^32 (the host checks)
    const uint32_t t = threadIdx.x;
    for (uint32_t id = blockIdx.x; id < ntiles; id += gridDim.x) {
        const uint32_t nc = id / per_nc, r = id - nc * per_nc;
        const uint32_t th = r / tw_n, tw = r - th * tw_n;
        const uint32_t h0 = th * TH, w0 = tw * TW;
        const uint32_t n = nc / C, c = nc - n * C;
        const uint32_t* sb = a.src + (int64_t)n * a.stride[0] + (int64_t)c * a.stride[1];
        uint32_t* db = a.dst + (uint64_t)nc * H * W;
        // read: float4 f = (column f / QH, rows 4 (f % QH) .. + 3)
        u32x4 v[NV];
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t f = t + 256u * i;
            const uint32_t h = h0 + 4u * (f % QH), w = w0 + f / QH;
            v[i] = (h < H && w < W) ? *(const u32x4*)(sb + h + (int64_t)w * a.stride[3]) : u32x4{0u, 0u, 0u, 0u};
        }
        __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t f = t + 256u * i;
            uint32_t* d = tile + (f / QH) * P + 4u * (f % QH);
            d[0] = v[i].x; d[1] = v[i].y; d[2] = v[i].z; d[3] = v[i].w;
        }
        __syncthreads();
        // write: float4 f = (row f / QW, columns 4 (f % QW) .. + 3)
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t f = t + 256u * i;
            const uint32_t hl = f / QW, w4 = f % QW;
            const uint32_t h = h0 + hl, w = w0 + 4u * w4;
            const uint32_t* q = tile + 4u * w4 * P + hl;
            if (h < H && w < W) *(u32x4*)(db + (uint64_t)h * W + w) = u32x4{q[0], q[P], q[2u * P], q[3u * P]};
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void vx_contiguous_t128(vx_copy_args a) {
    vx_args_fetch(a);
    vx_contiguous_tile16<128u, 128u>(a);
}
extern "C" __global__ __launch_bounds__(256) void vx_contiguous_t128x64(vx_copy_args a) {
    vx_args_fetch(a);
    vx_contiguous_tile16<128u, 64u>(a);
}
