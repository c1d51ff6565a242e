// vx_dpp.hpp — wave64 reductions on DPP lane moves (gfx950).
//
// __shfl_xor lowers to ds_bpermute, a round trip through the LDS crossbar
// per step; a six-step wave sum built from it sits on a wave's critical
// path for ~700 cycles. DPP moves are VALU operand modifiers: the same sum
// takes six dependent VALU adds.
#pragma once

#include <hip/hip_runtime.h>

// DPP controls used here (GFX9 encoding):
//   0xB1  quad_perm [1,0,3,2]   lane i <- i ^ 1
//   0x4E  quad_perm [2,3,0,1]   lane i <- i ^ 2
//   0x141 row_half_mirror       lane i <- 7 - i   within each 8 lanes
//   0x140 row_mirror            lane i <- 15 - i  within each 16 lanes
//   0x142 row_bcast:15          row r <- lane 15 of row r - 1
//   0x143 row_bcast:31          rows 2, 3 <- lane 31
//   0x128 row_ror:8             lane i <- (i + 8) mod 16 within each 16 lanes
// ROWS masks the 16-lane rows that are written; the others (and any lane
// whose source is invalid) receive 0, so v + vx_dpp(v) leaves them as v.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float vx_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}

// Sum over each aligned group of 8 lanes, in every lane of the group.
__device__ __forceinline__ float vx_sum8(float v) {
    v += vx_dpp<0xB1>(v);
    v += vx_dpp<0x4E>(v);
    return v + vx_dpp<0x141>(v);
}

// Maximum over each aligned group of 8 lanes, in every lane of the group.
__device__ __forceinline__ float vx_max8(float v) {
    v = fmaxf(v, vx_dpp<0xB1>(v));
    v = fmaxf(v, vx_dpp<0x4E>(v));
    return fmaxf(v, vx_dpp<0x141>(v));
}

// Sum over the 64 lanes, returned in every lane (wave-uniform).
__device__ __forceinline__ float vx_wave_sum(float v) {
    v = vx_sum8(v);
    v += vx_dpp<0x140>(v);       // each row of 16 holds its row sum
    v += vx_dpp<0x142, 0xA>(v);  // rows 1, 3 += rows 0, 2
    v += vx_dpp<0x143, 0xC>(v);  // rows 2, 3 += lane 31 (rows 0 + 1): lane 63 has the total
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over the four 16-lane rows: lane l gets v[l % 16] + v[l % 16 + 16] +
// v[l % 16 + 32] + v[l % 16 + 48], added as (row 0 + row 1) + (row 2 + row 3).
// v_permlane16_swap exchanges odd rows of its first operand with even rows
// of its second, v_permlane32_swap the upper half of the first with the
// lower half of the second (gfx950 VALU ops); with both operands v, the two
// results of each swap add up to the pairwise row sums in every lane.
// Both operands and both results pass through empty asm: this compiler
// otherwise folds the two results of a swap into one (a[0] + a[1] came out
// as a[0] + a[0]), and the swap needs its operands in two registers.
__device__ __forceinline__ void vx_pin2(unsigned& x, unsigned& y) { asm volatile("" : "+v"(x), "+v"(y)); }

__device__ __forceinline__ float vx_sum_rows4(float v) {
    unsigned u = __builtin_bit_cast(unsigned, v), u2 = u;
    vx_pin2(u, u2);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u2, false, false);
    unsigned a0 = a[0], a1 = a[1];
    vx_pin2(a0, a1);
    const float p = __builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a1);
    unsigned w = __builtin_bit_cast(unsigned, p), w2 = w;
    vx_pin2(w, w2);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w2, false, false);
    unsigned b0 = b[0], b1 = b[1];
    vx_pin2(b0, b1);
    return __builtin_bit_cast(float, b0) + __builtin_bit_cast(float, b1);
}

// vx_sum_rows4 of four values at once: row r (lanes 16r..16r+15) of the
// result holds the row sums of v_r, lane l having v_r[l % 16] + v_r[l % 16
// + 16] + v_r[l % 16 + 32] + v_r[l % 16 + 48], added in the same order as
// vx_sum_rows4. The first permlane16_swap pairs v0 with v1 and v2 with v3
// (row sums of rows 0 + 1 and 2 + 3 of each), the permlane32_swap pairs the
// two results: three swaps and three adds for four values.
__device__ __forceinline__ float vx_sum_rows4x4(float v0, float v1, float v2, float v3) {
    auto pair16 = [](float x, float y) {
        unsigned a = __builtin_bit_cast(unsigned, x), b = __builtin_bit_cast(unsigned, y);
        vx_pin2(a, b);
        const auto s = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        unsigned s0 = s[0], s1 = s[1];
        vx_pin2(s0, s1);
        return __builtin_bit_cast(float, s0) + __builtin_bit_cast(float, s1);
    };
    unsigned p = __builtin_bit_cast(unsigned, pair16(v0, v1)), q = __builtin_bit_cast(unsigned, pair16(v2, v3));
    vx_pin2(p, q);
    const auto t = __builtin_amdgcn_permlane32_swap(p, q, false, false);
    unsigned t0 = t[0], t1 = t[1];
    vx_pin2(t0, t1);
    return __builtin_bit_cast(float, t0) + __builtin_bit_cast(float, t1);
}
