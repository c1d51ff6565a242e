// vx_xq.hpp — the arithmetic of the activation split (no reference
// counterpart), shared by vx_quantize_x (quantize.hip) and the batched GEMV
// that splits x itself (gemv_q.hip), so both produce the same bytes. Per
// 32-element block with m = max|v| and S = sum v (the callers reduce them):
//   c1 = m / 126, c2 = c1 / 254, i1 = 126 / m (0 for m < 2^-100 or a
//   non-finite block), i2 = 254 i1,
//   q1 = clamp(rne(v i1), +-127), q2 = clamp(rne(fma(-q1, c1, v) i2), +-127)
//   (the clamps never act; see vx_xq_levels4),
// so x ~= c2 (254 q1 + q2), |error| <= ~max|v| / 64008. Every operation is
// one IEEE rounding (no contraction); the divisions are IEEE divisions.
#ifndef VX_XQ_HPP
#define VX_XQ_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

#define VX_XQ_MAGIC 12582912.0f  // 1.5 * 2^23

struct vx_xq_scale {
    float c1, c2, i1, i2;
    bool fin;  // m and S finite
};

__device__ __forceinline__ vx_xq_scale vx_xq_scales(float m, float S) {
#pragma clang fp contract(off)
    vx_xq_scale r;
    r.fin = m < __builtin_inff() && S == S;
    r.c1 = m / 126.0f;
    r.c2 = r.c1 / 254.0f;
    r.i1 = (r.fin && m >= 0x1p-100f) ? 126.0f / m : 0.0f;
    r.i2 = r.i1 * 254.0f;
    return r;
}

// The two levels of 4 values (value e in byte e of w1 / w2): fmaf(x, s,
// 1.5 2^23) rounds x s to the nearest integer n (ties to even) for |x s| <
// 2^22 and leaves n's int8 in the float's low byte; v_perm_b32 gathers the
// four low bytes. The clamps to +-127 never act in a finite block, so none
// is computed: |v| <= m and i1 = RN(126 / m) give |v i1| <= 126 (1 + 2^-24),
// which rounds to |q1| <= 126; r = RN(v - q1 c1) with c1 = RN(m / 126) has
// |r / c1| <= 0.5 + 126 2^-23, and i2 = RN(254 i1), so |r i2| <= 127.004
// rounds to |q2| <= 127 (m < 2^-100 has i1 = i2 = 0: both levels 0). A
// non-finite block (fin false) gives zero bytes: its values are computed
// anyway and masked per word.
template <typename V4>
__device__ __forceinline__ void vx_xq_levels4(const V4& v, float c1, float i1, float i2, bool fin, uint32_t& w1,
                                              uint32_t& w2) {
#pragma clang fp contract(off)
    uint32_t b1[4], b2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float t1 = __builtin_fmaf(v[e], i1, VX_XQ_MAGIC);
        const float q1 = t1 - VX_XQ_MAGIC;  // exact
        const float r = __builtin_fmaf(-q1, c1, v[e]);
        const float t2 = __builtin_fmaf(r, i2, VX_XQ_MAGIC);
        b1[e] = __float_as_uint(t1);
        b2[e] = __float_as_uint(t2);
    }
    // bytes 0 of (x0, x1) -> bytes 0, 1; of (x2, x3) -> bytes 2, 3
    const uint32_t p1 = __builtin_amdgcn_perm(b1[1], b1[0], 0x0c0c0400u), q1 = __builtin_amdgcn_perm(b1[3], b1[2], 0x0c0c0400u);
    const uint32_t p2 = __builtin_amdgcn_perm(b2[1], b2[0], 0x0c0c0400u), q2 = __builtin_amdgcn_perm(b2[3], b2[2], 0x0c0c0400u);
    w1 = fin ? __builtin_amdgcn_perm(q1, p1, 0x05040100u) : 0u;
    w2 = fin ? __builtin_amdgcn_perm(q2, p2, 0x05040100u) : 0u;
}

#endif  // VX_XQ_HPP
