// quantize.hip — f32 rows -> GGML Q8_0 / Q4_0 / Q4_K blocks for gfx950.
//
// The algorithms are ggml's reference quantizers (ggml-quants.c:
// quantize_row_q8_0_ref, quantize_row_q4_0_ref, quantize_row_q4_K_ref with
// make_qkx2_quants and nearest_int), evaluated in the same f32 operation
// order with no contraction (the pragma below), IEEE division and square
// root, round-to-nearest-even f32 -> f16: the blocks equal those of a
// sequential CPU run of the same algorithm bit for bit. The reference
// (vortx) has no quantized code; this is the step before its GEMV.
//
//   vx_quantize_q8_0 / _q4_0  one lane per 32-block (HBM-bound; Q8_0's
//                             blocks staged in LDS for 16-byte stores);
//   vx_quantize_q4_k          8 lanes per 256-super-block, lane j running
//                             the scale/min search of sub-block j, the
//                             lanes meeting through shuffles for the
//                             super-block maxima, the 6-bit scale packing
//                             and the nibble pairs (compute-bound: about
//                             20 search passes of 32 elements per lane).
//
// ggml MIT license notice (the quantizers below restate ggml's published
// quantize_row_*_ref / make_qkx2_quants; ggml is distributed under it):
//
//   MIT License
//
//   Copyright (c) 2023-2024 The ggml authors
//
//   Permission is hereby granted, free of charge, to any person obtaining a copy
//   of this software and associated documentation files (the "Software"), to deal
//   in the Software without restriction, including without limitation the rights
//   to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
//   copies of the Software, and to permit persons to whom the Software is
//   furnished to do so, subject to the following conditions:
//
//   The above copyright notice and this permission notice shall be included in all
//   copies or substantial portions of the Software.
//
//   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR
//   IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY,
//   FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT SHALL THE
//   AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER
//   LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM,
//   OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE
//   SOFTWARE.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../vx_kargs.h"
#include "vx_dpp.hpp"
#include "vx_xq.hpp"

#pragma clang fp contract(off)

typedef float f32x4q __attribute__((ext_vector_type(4)));

// The empty asm pins v as an already-rounded f32: without it the backend folds
// a preceding multiply into v_fma_mix (one rounding straight to f16, and a
// +0 addend that turns -0 into +0), which is not ggml's f32 -> f16 of an f32.
__device__ __forceinline__ uint16_t vx_f32_to_f16_bits(float v) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32, round to nearest even
}
__device__ __forceinline__ float vx_f16_bits_to_f32(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}

// ggml nearest_int: round half to even through the 1.5 * 2^23 magic.
__device__ __forceinline__ int vx_nearest_int(float fval) {
    const float val = fval + 12582912.f;
    return (int)(__builtin_bit_cast(uint32_t, val) & 0x007fffffu) - 0x00400000;
}

__device__ __forceinline__ void vx_q_load32(const vx_quant_args& a, uint32_t row, uint32_t k0, float (&x)[32]) {
    const float* xr = a.x + (int64_t)row * a.xs_m;
    if (a.x_vec) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4q v = *(const f32x4q*)(xr + k0 + 4 * i);
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = xr[(int64_t)(k0 + i) * a.xs_k];
    }
}

// One Q8_0 block (quantize_row_q8_0_ref): 17 little-endian u16 words, the
// f16 scale then the 32 int8 values in pairs.
__device__ __forceinline__ void vx_q8_0_block(const float (&x)[32], uint16_t (&w)[17]) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float v = fabsf(x[j]);
        amax = amax > v ? amax : v;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    w[0] = vx_f32_to_f16_bits(d);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t q0 = (uint32_t)(uint8_t)(int8_t)(int)__builtin_roundf(x[2 * j] * id);
        const uint32_t q1 = (uint32_t)(uint8_t)(int8_t)(int)__builtin_roundf(x[2 * j + 1] * id);
        w[1 + j] = (uint16_t)(q0 | (q1 << 8));
    }
}

// One Q4_0 block (quantize_row_q4_0_ref): 9 u16 words, the f16 scale then
// the 16 bytes of nibble pairs (element j low, element j + 16 high).
__device__ __forceinline__ void vx_q4_0_block(const float (&x)[32], uint16_t (&w)[9]) {
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            mx = x[j];
        }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    w[0] = vx_f32_to_f16_bits(d);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t pr = 0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int jj = 2 * j + t;
            int xi0 = (int8_t)(x[jj] * id + 8.5f);
            int xi1 = (int8_t)(x[16 + jj] * id + 8.5f);
            xi0 = xi0 < 15 ? xi0 : 15;
            xi1 = xi1 < 15 ? xi1 : 15;
            pr |= (uint32_t)(xi0 | (xi1 << 4)) << (8 * t);
        }
        w[1 + j] = (uint16_t)pr;
    }
}

// Q8_0: thread t of each round takes block g0 + t of the flattened (row,
// block) sequence (grid-stride over rounds of 256 blocks). With dense rows
// (row stride = nblk blocks) a round's output is one contiguous range: it is
// staged in LDS and written with 16-byte stores, which beats per-lane
// 2-byte stores at a 34-byte lane stride (14336 x 4096: 60.4 -> 54.1 us).
// Padded rows take the 2-byte stores. (Q4_0's 18-byte blocks measured
// faster with its own row-per-workgroup kernel below, staged or not.)
template <int NW>
__device__ __forceinline__ void vx_quantize_blocks(const vx_quant_args& a) {
    __shared__ uint4 stage[(256u * 2u * NW + 15u) / 16u];
    uint16_t* st = (uint16_t*)stage;
    const uint64_t G = (uint64_t)a.M * a.nblk;
    const bool dense = a.row_stride == 2ull * NW * a.nblk;  // uniform
    const bool out16 = (reinterpret_cast<uintptr_t>(a.out) & 15u) == 0u;
    const uint32_t t = threadIdx.x;
    for (uint64_t g0 = (uint64_t)blockIdx.x * 256u; g0 < G; g0 += (uint64_t)gridDim.x * 256u) {
        const uint64_t g = g0 + t;
        if (g < G) {
            const uint32_t row = (uint32_t)(g / a.nblk), b = (uint32_t)(g - (uint64_t)row * a.nblk);
            float x[32];
            vx_q_load32(a, row, 32u * b, x);
            uint16_t w[NW];
            if constexpr (NW == 17) vx_q8_0_block(x, w);
            else vx_q4_0_block(x, w);
            if (dense) {
#pragma unroll
                for (int j = 0; j < NW; ++j) st[NW * t + j] = w[j];
            } else {
                uint16_t* y = (uint16_t*)(a.out + (uint64_t)row * a.row_stride + 2ull * NW * b);
#pragma unroll
                for (int j = 0; j < NW; ++j) y[j] = w[j];
            }
        }
        if (dense) {
            __syncthreads();
            const uint32_t nb = G - g0 < 256u ? (uint32_t)(G - g0) : 256u;
            const uint32_t nh = NW * nb;             // u16 words of this round
            uint8_t* dst = a.out + g0 * 2u * NW;     // 16-byte aligned when out is: 256 blocks = 16 * (32 NW) bytes
            uint32_t done = 0;
            if (out16) {
                const uint32_t n16 = nh / 8u;
                for (uint32_t i = t; i < n16; i += 256u) ((uint4*)dst)[i] = stage[i];
                done = 8u * n16;
            }
            for (uint32_t i = done + t; i < nh; i += 256u) ((uint16_t*)dst)[i] = st[i];
            __syncthreads();  // the next round rewrites the stage
        }
    }
}

// grid: a multiple of the CU count; 256 threads, one 32-block each per round.
extern "C" __global__ __launch_bounds__(256) void vx_quantize_q8_0(vx_quant_args a) {
    vx_quantize_blocks<17>(a);
}

// grid: x covers the blocks of a row (256 per workgroup), y the rows (loop).
extern "C" __global__ __launch_bounds__(256) void vx_quantize_q4_0(vx_quant_args a) {
    const uint32_t b = blockIdx.x * 256u + threadIdx.x;
    if (b >= a.nblk) return;
    for (uint64_t r64 = blockIdx.y; r64 < a.M; r64 += gridDim.y) {  // 64-bit: no wrap near 2^32 rows
        const uint32_t row = (uint32_t)r64;
        float x[32];
        vx_q_load32(a, row, 32u * b, x);
        uint16_t w[9];
        vx_q4_0_block(x, w);
        uint16_t* y = (uint16_t*)(a.out + (uint64_t)row * a.row_stride + 18ull * b);
#pragma unroll
        for (int j = 0; j < 9; ++j) y[j] = w[j];
    }
}

// make_qkx2_quants(32, 15, x, weights, L, &min, Laux, -1, 0.1, 20, false).
// Every loop over the 32 values is unrolled so x, w and the candidate levels
// stay in registers (a rolled loop indexes them through 32-way selects).
// Instead of copying the winning candidate's levels on each improvement, the
// (iscale, min) pair that produced them is kept and the levels are rebuilt
// once by vx_qkx2_levels: the same nearest_int(iscale * (x - min)), clamped.
// (float) MAX(0, MIN(15, nearest_int(v))) of make_qkx2_quants' search for
// |v| < 2^22 (ggml's nearest_int asserts |v| <= 4194303): there its
// 1.5 * 2^23 magic rounds to nearest even exactly like v_rndne_f32, and
// v_med3_f32 clamps in float, so no integer round trip. The only
// difference, a -0 level for v in (-0.5, -0], changes none of the sums or
// squared differences it enters.
__device__ __forceinline__ float vx_level(float v) {
    return __builtin_amdgcn_fmed3f(__builtin_rintf(v), 0.f, 15.f);
}

struct vx_qkx2_best {
    float iscale, mnu;  // the winning candidate's inputs; iscale 0 = all levels 0
};

__device__ __forceinline__ float vx_make_qkx2(const float (&x)[32], const float (&w)[32], vx_qkx2_best& best,
                                              float& the_min) {
    const int nmax = 15;
    const float rmin = -1.f, rdelta = 0.1f;
    const int nstep = 20;
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        best.iscale = 0.f;
        best.mnu = 0.f;
        the_min = -mn;
        return 0.f;
    }
    float iscale = (float)nmax / (mx - mn);
    float scale = 1 / iscale;
    float best_mad = 0;
    best.iscale = iscale;
    best.mnu = mn;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float fl = vx_level(iscale * (x[i] - mn));
        float diff = scale * fl + mn - x[i];
        diff = diff * diff;
        best_mad += w[i] * diff;
    }
    float fl[32];
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            fl[i] = vx_level(iscale * (x[i] - mn));
            sum_l += w[i] * fl[i];
            sum_l2 += w[i] * fl[i] * fl[i];
            sum_xl += w[i] * fl[i] * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                float diff = this_scale * fl[i] + this_min - x[i];
                diff = diff * diff;
                mad += w[i] * diff;
            }
            if (mad < best_mad) {
                best.iscale = iscale;
                best.mnu = mn;
                best_mad = mad;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    the_min = -mn;
    return scale;
}

// The levels make_qkx2_quants leaves in L for the winning candidate.
__device__ __forceinline__ void vx_qkx2_levels(const float (&x)[32], const vx_qkx2_best& best, uint8_t (&L)[32]) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int l = best.iscale == 0.f ? 0 : vx_nearest_int(best.iscale * (x[i] - best.mnu));
        L[i] = (uint8_t)(l < 0 ? 0 : l > 15 ? 15 : l);
    }
}

// 8 lanes per super-block (lane j = sub-block j); 256 threads = 32
// super-blocks of the flattened (row, super-block) sequence; grid-stride.
extern "C" __global__ __launch_bounds__(256) void vx_quantize_q4_k(vx_quant_args a) {
    const uint32_t j = threadIdx.x & 7u;
    const uint64_t total = (uint64_t)a.M * a.nblk;
    for (uint64_t g0 = (uint64_t)blockIdx.x * 32u; g0 < total; g0 += (uint64_t)gridDim.x * 32u) {
        const uint64_t g = g0 + (threadIdx.x >> 3);
        const bool live = g < total;  // whole 8-lane groups agree
        const uint32_t row = live ? (uint32_t)(g / a.nblk) : 0u;
        const uint32_t sb = live ? (uint32_t)(g - (uint64_t)row * a.nblk) : 0u;
        float x[32], w[32];
        uint8_t L[32];
        vx_qkx2_best best{0.f, 0.f};
        float scale = 0.f, mn = 0.f;
        if (live) {
            vx_q_load32(a, row, 256u * sb + 32u * j, x);
            float sum_x2 = 0;
#pragma unroll
            for (int l = 0; l < 32; ++l) sum_x2 += x[l] * x[l];
            const float av_x = __builtin_sqrtf(sum_x2 / 32);
#pragma unroll
            for (int l = 0; l < 32; ++l) w[l] = av_x + fabsf(x[l]);
            scale = vx_make_qkx2(x, w, best, mn);
        }
        // super-block maxima (ggml starts both at 0)
        float max_scale = scale > 0.f ? scale : 0.f, max_min = mn > 0.f ? mn : 0.f;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            const float s2 = __shfl_xor(max_scale, o, 64), m2 = __shfl_xor(max_min, o, 64);
            max_scale = s2 > max_scale ? s2 : max_scale;
            max_min = m2 > max_min ? m2 : max_min;
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        uint32_t ls = (uint32_t)(uint8_t)vx_nearest_int(inv_scale * scale);
        uint32_t lm = (uint32_t)(uint8_t)vx_nearest_int(inv_min * mn);
        ls = ls < 63u ? ls : 63u;
        lm = lm < 63u ? lm : 63u;
        const uint16_t dh = vx_f32_to_f16_bits(max_scale / 63.f), mh = vx_f32_to_f16_bits(max_min / 63.f);
        // the 6-bit pair (ls, lm) round-trips through the packing unchanged
        const float dq = vx_f16_bits_to_f32(dh) * (float)ls;
        if (live && dq != 0.f) {
            const float dm = vx_f16_bits_to_f32(mh) * (float)lm;
#pragma unroll
            for (int ii = 0; ii < 32; ++ii) {
                int l = vx_nearest_int((x[ii] + dm) / dq);
                L[ii] = (uint8_t)(l < 0 ? 0 : l > 15 ? 15 : l);
            }
        } else {
            vx_qkx2_levels(x, best, L);  // ggml keeps make_qkx2_quants' levels when d * sc == 0
        }
        // scales[12]: j < 4: sc[j] = ls_j | (ls_{j+4} >> 4) << 6,
        // sc[j+4] = lm_j | (lm_{j+4} >> 4) << 6; j >= 4: sc[j+4] = (ls_j & 15) | (lm_j & 15) << 4
        const uint32_t ls4 = (uint32_t)__shfl_xor((int)ls, 4, 64), lm4 = (uint32_t)__shfl_xor((int)lm, 4, 64);
        uint32_t Lp[4];  // this lane's 32 nibbles, 8 per dword
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) {
            uint32_t v = 0;
#pragma unroll
            for (int t = 0; t < 8; ++t) v |= (uint32_t)L[8 * d4 + t] << (4 * t);
            Lp[d4] = v;
        }
        uint32_t Lh[4];  // the odd partner's nibbles (sub-block 2c + 1)
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) Lh[d4] = (uint32_t)__shfl_xor((int)Lp[d4], 1, 64);
        if (!live) continue;
        uint8_t* yb = a.out + (uint64_t)row * a.row_stride + 144ull * sb;
        if (j == 0) {
            ((uint16_t*)yb)[0] = dh;
            ((uint16_t*)yb)[1] = mh;
        }
        if (j < 4) {
            yb[4 + j] = (uint8_t)(ls | ((ls4 >> 4) << 6));
            yb[8 + j] = (uint8_t)(lm | ((lm4 >> 4) << 6));
        } else {
            yb[8 + j] = (uint8_t)((ls & 15u) | ((lm & 15u) << 4));
        }
        if ((j & 1u) == 0u) {
            // chunk c = j / 2: byte l = L_{2c}[l] | L_{2c+1}[l] << 4
            uint32_t* q = (uint32_t*)(yb + 16u + 16u * j);
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                uint32_t v = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int l = 4 * d + t;
                    const uint32_t lo = (Lp[l >> 3] >> (4 * (l & 7))) & 15u;
                    const uint32_t hi = (Lh[l >> 3] >> (4 * (l & 7))) & 15u;
                    v |= (lo | (hi << 4)) << (8 * t);
                }
                q[d] = v;
            }
        }
    }
}

// ------------------------------------------------------------------------
// Activation split for the batched GEMV (no reference counterpart): per
// column b of x [K, B] and 32-element block j, two int8 levels and one scale,
//   m = max|v|, S = sum v (a fixed tree: pairs within each 4, then 8 lanes),
//   c1 = m / 126, c2 = c1 / 254, i1 = 126 / m (0 for m < 2^-100 or a
//   non-finite block), i2 = 254 i1,
//   q1 = clamp(rne(v i1), +-127), q2 = clamp(rne(fma(-q1, c1, v) i2), +-127),
// so x ~= c2 (254 q1 + q2), |error| <= ~max|v| / 64008. A block's 32
// positions hold element i at position 8 (i / 4) + i % 4 (i < 16) or
// 8 ((i - 16) / 4) + 4 + i % 4 (i >= 16): the order of a Q4_0 block's nibbles
// (byte t holds elements t and t + 16), so a 32-bit word of Q4_0 nibbles and
// 8 bytes of x levels line up for the int8 matrix cores. Levels are stored
// [item = j / 8][k = (j % 8) / 2][g = position / 8][b][level][j % 2]
// [position % 8]: the 16 bytes one matrix-core lane (column b, level, group
// g) needs from blocks 2k, 2k + 1 of an item sit together, and the lanes of
// one load instruction (fixed k) read consecutive 16-byte pieces, so a
// wave's load of 8 columns covers 1 KB contiguously (8 cache lines rather
// than 64). Scales [j][b] = {c2, S}; a block with a NaN
// or inf stores {m + S, S} and zero levels, so every output of its column
// becomes non-finite.
// Eight lanes per (j, b), lane t holding elements 4t..4t+3; every operation
// is one IEEE rounding (no contraction in this file), so the bytes equal
// the oracle's sequential restatement (orc_quantize_x).
extern "C" __global__ __launch_bounds__(256) void vx_quantize_x(vx_xq_args a) {
    const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t grp = gid >> 3;               // (j, b) = (grp / B, grp % B)
    const uint32_t t = threadIdx.x & 7u;
    const uint64_t ngrp = (uint64_t)a.nblk * a.B;
    // every lane takes part in the DPP reductions; lanes past the end load
    // group 0 and store nothing
    const bool in = grp < ngrp;
    const uint64_t gg = in ? grp : 0u;
    const uint32_t j = (uint32_t)(gg / a.B), b = (uint32_t)(gg - (uint64_t)j * a.B);
    const int64_t k0 = 32 * (int64_t)j + 4 * (int64_t)t;
    f32x4q v;
    if (a.x_vec) {
        v = *(const f32x4q*)(a.x + (int64_t)b * a.xs_b + k0);
    } else {
        const float* p = a.x + (int64_t)b * a.xs_b + k0 * a.xs_k;
        v = f32x4q{p[0], p[a.xs_k], p[2 * a.xs_k], p[3 * a.xs_k]};
    }
    const float m = vx_max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float S = vx_sum8((v.x + v.y) + (v.z + v.w));
    const vx_xq_scale sc = vx_xq_scales(m, S);
    const bool fin = sc.fin;
    const float c2 = sc.c2;
    uint32_t w1, w2;
    vx_xq_levels4(v, sc.c1, sc.i1, sc.i2, fin, w1, w2);
    if (in) {
        // position dword dw (positions 4 dw..4 dw + 3, elements 4t..4t+3) of
        // level L sits at item B 512 + ((j % 8) / 2) B 128 + (dw / 2) B 32 +
        // b 32 + L 16 + (j % 2) 8 + (dw % 2) 4
        const uint32_t dw = t < 4u ? 2u * t : 2u * (t - 4u) + 1u;
        uint8_t* base = (uint8_t*)a.levels + (uint64_t)(j >> 3) * a.B * 512u + ((j & 7u) >> 1) * a.B * 128u +
                        (dw >> 1) * a.B * 32u + b * 32u + (j & 1u) * 8u + (dw & 1u) * 4u;
        *(uint32_t*)base = w1;
        *(uint32_t*)(base + 16u) = w2;
        if (t == 0) *(float2*)(a.scales + 2u * grp) = float2{fin ? c2 : m + S, S};
    }
}
