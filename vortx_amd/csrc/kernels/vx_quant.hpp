// vx_quant.hpp — device-side GGML block decoding for gfx950.
//
// Block formats (public ggml layout; the reference has no quantized code):
//   Q4_0  18 B / 32 weights : f16 d | 16 B nibbles; w_j = (lo(q_j)-8) d,
//                             w_{j+16} = (hi(q_j)-8) d
//   Q8_0  34 B / 32 weights : f16 d | 32 int8;      w_i = d q_i
//   Q4_K 144 B / 256 weights: f16 d | f16 dmin | 12 B packed 6-bit
//                             (scale, min) x 8 | 128 B nibbles;
//                             w = (d sc_s) q - (dmin m_s)
//
// A "unit" is 64 consecutive weights of one row: two Q4_0 / Q8_0 blocks
// (36 / 68 bytes, 4-byte aligned when the row is) or one quarter of a Q4_K
// super-block (its 16-byte header plus 32 bytes of nibbles). Unit u of a
// row covers x[64u .. 64u+64) for every format.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../vx_kargs.h"
#include "vx_args.hpp"
#include "vx_dpp.hpp"

#define VX_Q4_0 2
#define VX_Q8_0 8
#define VX_Q4_K 12

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float vx_f16_to_f32(uint32_t bits) {
    // v_cvt_f32_f16: exact for every binary16 value, subnormals included.
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

// Weight loads (plain cached loads: a non-temporal hint measured slower,
// the x loads then arrive later).
__device__ __forceinline__ u32x4_a4 vx_ld16(const uint8_t* p) { return *(const u32x4_a4*)p; }
__device__ __forceinline__ uint32_t vx_ld4(const uint8_t* p) { return *(const uint32_t*)p; }

// v_and_b32 / v_xor_b32 the optimiser cannot see through: applied to a
// whole dword before byte extraction, they keep each byte->float convert a
// single v_cvt_f32_ubyte{0..3} instead of a per-byte bit-field extract.
__device__ __forceinline__ uint32_t vx_and(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %2, %1" : "=v"(r) : "v"(v), "s"(m));
    return r;
}
__device__ __forceinline__ uint32_t vx_xor(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_xor_b32 %0, %2, %1" : "=v"(r) : "v"(v), "s"(m));
    return r;
}

// Byte b of a dword as float: matches v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float vx_ub(uint32_t v, int b) {
    return (float)((v >> (8 * b)) & 0xFFu);
}

// The four nibbles at bits (sh, sh+8, sh+16, sh+24) of w as floats scaled
// by VX_NIB (= 2^-9), two per v_cvt_pk_f32_fp8: a byte 0..15 read as an
// OCP e4m3 value is exactly q * 2^-9 (subnormals for q < 8, exponent 1
// for q >= 8), so one packed convert replaces two byte converts.
#define VX_NIB_INV 512.0f
__device__ __forceinline__ void vx_nib4(uint32_t w, int sh, float (&o)[4]) {
    const uint32_t b = vx_and(sh ? (w >> 4) : w, 0x0F0F0F0Fu);
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(b, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(b, true);
    o[0] = lo[0];
    o[1] = lo[1];
    o[2] = hi[0];
    o[3] = hi[1];
}

template <int QT> struct vx_unit;
template <> struct vx_unit<VX_Q4_0> { static constexpr int NW = 9;  static constexpr int QK = 32;  static constexpr int BB = 18; };
template <> struct vx_unit<VX_Q8_0> { static constexpr int NW = 17; static constexpr int QK = 32;  static constexpr int BB = 34; };
template <> struct vx_unit<VX_Q4_K> { static constexpr int NW = 12; static constexpr int QK = 256; static constexpr int BB = 144; };

// Raw bytes of unit u of a row into registers (row 4-byte aligned). With
// U24 the caller guarantees u < 2^24, so the byte offset is a full-rate
// 24-bit multiply instead of v_mul_lo_u32.
template <int QT, bool U24 = false>
__device__ __forceinline__ void vx_load_unit(const uint8_t* row, uint32_t u, uint32_t (&r)[vx_unit<QT>::NW]) {
    if constexpr (QT == VX_Q4_0) {
        const uint8_t* p = row + (U24 ? __umul24(u, 36u) : 36u * u);
        u32x4_a4 a = vx_ld16(p), b = vx_ld16(p + 16);
        r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
        r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
        r[8] = vx_ld4(p + 32);
    } else if constexpr (QT == VX_Q8_0) {
        const uint8_t* p = row + (U24 ? __umul24(u, 68u) : 68u * u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4_a4 a = vx_ld16(p + 16 * i);
            r[4 * i + 0] = a.x; r[4 * i + 1] = a.y; r[4 * i + 2] = a.z; r[4 * i + 3] = a.w;
        }
        r[16] = vx_ld4(p + 64);
    } else {
        const uint8_t* sb = row + (U24 ? __umul24(u >> 2, 144u) : 144u * (u >> 2));
        const uint8_t* qs = sb + 16 + 32u * (u & 3u);
        u32x4_a4 h = vx_ld16(sb), a = vx_ld16(qs), b = vx_ld16(qs + 16);
        r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
        r[4] = a.x; r[5] = a.y; r[6] = a.z; r[7] = a.w;
        r[8] = b.x; r[9] = b.y; r[10] = b.z; r[11] = b.w;
    }
}

// Q4_K: the (scale, min) pairs of the two sub-blocks (2c, 2c+1) a unit
// covers, from the 12 packed bytes held in h1 = bytes 0..3, h2 = 4..7,
// h3 = 8..11. Sub-block s < 4: sc = b[s] & 63, m = b[s+4] & 63.
// s >= 4: sc = (b[s+4] & 15) | (b[s-4] >> 6) << 4,
//         m  = (b[s+4] >> 4) | (b[s]   >> 6) << 4.
__device__ __forceinline__ void vx_q4k_scales(uint32_t h1, uint32_t h2, uint32_t h3, uint32_t c,
                                              uint32_t& sc0, uint32_t& m0, uint32_t& sc1, uint32_t& m1) {
    const uint32_t sh = 16u * (c & 1u);
    const uint32_t A = h1 >> sh, Bv = h2 >> sh, Cv = h3 >> sh;
    if (c < 2) {
        sc0 = A & 63u;
        sc1 = (A >> 8) & 63u;
        m0 = Bv & 63u;
        m1 = (Bv >> 8) & 63u;
    } else {
        sc0 = (Cv & 15u) | ((A >> 2) & 0x30u);
        m0 = ((Cv >> 4) & 15u) | ((Bv >> 2) & 0x30u);
        sc1 = ((Cv >> 8) & 15u) | ((A >> 10) & 0x30u);
        m1 = ((Cv >> 12) & 15u) | ((Bv >> 10) & 0x30u);
    }
}

// Dot product of one unit with x (64 floats in registers) for batch 1.
// sx0 / sx1 are the sums of x[0..32) and x[32..64). The offset terms of
// each format (-8 d for Q4_0, the xor-128 bias for Q8_0, dmin m for Q4_K)
// are applied once per 32 weights through those sums, so the inner work
// is one byte->float convert and one FMA per weight.
template <int QT>
__device__ __forceinline__ float vx_unit_dot_b1(const uint32_t (&r)[vx_unit<QT>::NW], const float (&xv)[64],
                                                float sx0, float sx1, uint32_t u) {
    if constexpr (QT == VX_Q4_0) {
        const float d0 = vx_f16_to_f32(r[0]);
        const float d1 = vx_f16_to_f32(r[4] >> 16);
        uint32_t q[8];
        q[0] = __builtin_amdgcn_alignbit(r[1], r[0], 16);
        q[1] = __builtin_amdgcn_alignbit(r[2], r[1], 16);
        q[2] = __builtin_amdgcn_alignbit(r[3], r[2], 16);
        q[3] = __builtin_amdgcn_alignbit(r[4], r[3], 16);
        q[4] = r[5]; q[5] = r[6]; q[6] = r[7]; q[7] = r[8];
        float res = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float slo = 0.f, shi = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float wl[4], wh[4];
                vx_nib4(q[4 * h + i], 0, wl);
                vx_nib4(q[4 * h + i], 4, wh);
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    slo = __builtin_fmaf(wl[b], xv[32 * h + 4 * i + b], slo);
                    shi = __builtin_fmaf(wh[b], xv[32 * h + 16 + 4 * i + b], shi);
                }
            }
            const float d = h ? d1 : d0;
            const float sx = h ? sx1 : sx0;
            res = __builtin_fmaf(d, __builtin_fmaf(slo + shi, VX_NIB_INV, -8.f * sx), res);
        }
        return res;
    } else if constexpr (QT == VX_Q8_0) {
        const float d0 = vx_f16_to_f32(r[0]);
        const float d1 = vx_f16_to_f32(r[8] >> 16);
        float res = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t qd = h ? r[9 + i] : __builtin_amdgcn_alignbit(r[i + 1], r[i], 16);
                const uint32_t uq = vx_xor(qd, 0x80808080u);  // q + 128 per byte
#pragma unroll
                for (int b = 0; b < 4; ++b) s = __builtin_fmaf(vx_ub(uq, b), xv[32 * h + 4 * i + b], s);
            }
            const float d = h ? d1 : d0;
            const float sx = h ? sx1 : sx0;
            res = __builtin_fmaf(d, s - 128.f * sx, res);
        }
        return res;
    } else {
        const float d = vx_f16_to_f32(r[0]);
        const float dmin = vx_f16_to_f32(r[0] >> 16);
        uint32_t sc0, m0, sc1, m1;
        vx_q4k_scales(r[1], r[2], r[3], u & 3u, sc0, m0, sc1, m1);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float wl[4], wh[4];
            vx_nib4(r[4 + i], 0, wl);
            vx_nib4(r[4 + i], 4, wh);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                slo = __builtin_fmaf(wl[b], xv[4 * i + b], slo);
                shi = __builtin_fmaf(wh[b], xv[32 + 4 * i + b], shi);
            }
        }
        const float t0 = __builtin_fmaf(d * (float)sc0 * VX_NIB_INV, slo, -(dmin * (float)m0) * sx0);
        const float t1 = __builtin_fmaf(d * (float)sc1 * VX_NIB_INV, shi, -(dmin * (float)m1) * sx1);
        return t0 + t1;
    }
}

// Per-unit scale terms for the batched path, decoded once per (row, unit):
//   Q4_0: s = {d0, -8 d0, d1, -8 d1}     w = q * s[0|2] + s[1|3]
//   Q8_0: s = {d0, 0, d1, 0}             w = q * s[0|2]
//   Q4_K: s = {d sc0, -dmin m0, d sc1, -dmin m1}
template <int QT>
__device__ __forceinline__ void vx_unit_scales(const uint32_t (&r)[vx_unit<QT>::NW], uint32_t u, float (&s)[4]) {
    if constexpr (QT == VX_Q4_0) {
        s[0] = vx_f16_to_f32(r[0]);
        s[2] = vx_f16_to_f32(r[4] >> 16);
        s[1] = -8.f * s[0];
        s[3] = -8.f * s[2];
    } else if constexpr (QT == VX_Q8_0) {
        s[0] = vx_f16_to_f32(r[0]);
        s[2] = vx_f16_to_f32(r[8] >> 16);
        s[1] = 0.f;
        s[3] = 0.f;
    } else {
        const float d = vx_f16_to_f32(r[0]);
        const float dmin = vx_f16_to_f32(r[0] >> 16);
        uint32_t sc0, m0, sc1, m1;
        vx_q4k_scales(r[1], r[2], r[3], u & 3u, sc0, m0, sc1, m1);
        s[0] = d * (float)sc0;
        s[1] = -(dmin * (float)m0);
        s[2] = d * (float)sc1;
        s[3] = -(dmin * (float)m1);
    }
}

// Decode the 8 weights of group g (0..7) of a unit with its scale terms,
// and the two float4 slots (ja, jb) of x they multiply (weights 0..3 ->
// slot ja, 4..7 -> slot jb). Q4_0 and Q8_0 values are exact; Q4_K values
// are fma(q, d sc, -dmin m) (one rounding, the decoded value itself).
template <int QT>
__device__ __forceinline__ void vx_unit_group(const uint32_t (&r)[vx_unit<QT>::NW], const float (&s)[4], int g,
                                              float (&w)[8], int& ja, int& jb) {
    if constexpr (QT == VX_Q4_0) {
        const int h = g >> 2, i = g & 3;
        const uint32_t qd = h ? r[5 + i] : __builtin_amdgcn_alignbit(r[i + 1], r[i], 16);
        const uint32_t lo = vx_and(qd, 0x0F0F0F0Fu), hi = vx_and(qd >> 4, 0x0F0F0F0Fu);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            w[b] = __builtin_fmaf(vx_ub(lo, b), s[2 * h], s[2 * h + 1]);
            w[4 + b] = __builtin_fmaf(vx_ub(hi, b), s[2 * h], s[2 * h + 1]);
        }
        ja = 8 * h + i;
        jb = 8 * h + 4 + i;
    } else if constexpr (QT == VX_Q8_0) {
        const int h = g >> 2, i = g & 3;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int di = 2 * i + t;
            const uint32_t qd = h ? r[9 + di] : __builtin_amdgcn_alignbit(r[di + 1], r[di], 16);
#pragma unroll
            for (int b = 0; b < 4; ++b) w[4 * t + b] = s[2 * h] * (float)(int8_t)((qd >> (8 * b)) & 0xFFu);
        }
        ja = 8 * h + 2 * i;
        jb = ja + 1;
    } else {
        const uint32_t qd = r[4 + g];
        const uint32_t lo = vx_and(qd, 0x0F0F0F0Fu), hi = vx_and(qd >> 4, 0x0F0F0F0Fu);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            w[b] = __builtin_fmaf(vx_ub(lo, b), s[0], s[1]);
            w[4 + b] = __builtin_fmaf(vx_ub(hi, b), s[2], s[3]);
        }
        ja = g;
        jb = 8 + g;
    }
}

// Byte-level exact decode of the 32 weights kb*32 .. kb*32+32 of a row
// (any alignment). Used by the dequantize kernel and the generic GEMV.
template <int QT>
__device__ __forceinline__ void vx_decode32(const uint8_t* row, uint32_t kb, float (&o)[32]) {
    if constexpr (QT == VX_Q4_0) {
        const uint8_t* blk = row + 18u * kb;
        const float d = vx_f16_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t q = blk[2 + j];
            o[j] = (float)((int)(q & 15u) - 8) * d;
            o[j + 16] = (float)((int)(q >> 4) - 8) * d;
        }
    } else if constexpr (QT == VX_Q8_0) {
        const uint8_t* blk = row + 34u * kb;
        const float d = vx_f16_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
#pragma unroll
        for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)blk[2 + i];
    } else {
        const uint8_t* sb = row + 144u * (kb >> 3);
        const uint32_t s = kb & 7u, c = s >> 1, hi = s & 1u;
        const float d = vx_f16_to_f32((uint32_t)sb[0] | ((uint32_t)sb[1] << 8));
        const float dmin = vx_f16_to_f32((uint32_t)sb[2] | ((uint32_t)sb[3] << 8));
        const uint8_t* sc12 = sb + 4;
        uint32_t sc, m;
        if (s < 4) {
            sc = sc12[s] & 63u;
            m = sc12[s + 4] & 63u;
        } else {
            sc = (sc12[s + 4] & 15u) | ((uint32_t)(sc12[s - 4] >> 6) << 4);
            m = (uint32_t)(sc12[s + 4] >> 4) | ((uint32_t)(sc12[s] >> 6) << 4);
        }
        const float ds = d * (float)sc, mm = dmin * (float)m;
        const uint8_t* qs = sb + 16 + 32u * c;
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t q = hi ? (uint32_t)(qs[l] >> 4) : (uint32_t)(qs[l] & 15u);
            o[l] = __fsub_rn(__fmul_rn(ds, (float)q), mm);
        }
    }
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float vx_group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
