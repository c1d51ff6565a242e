// vx_xq.hpp — the arithmetic of the activation split (no reference
// counterpart), shared by vx_quantize_x (quantize.hip) and the batched GEMV
// that splits x itself (gemv_q.hip), so both produce the same bytes. Per
// 32-element block with m = max|v| and S = sum v (the callers reduce them):
//   c1 = m / 126, c2 = c1 / 254, i1 = 126 / m (0 for m < 2^-100 or a
//   non-finite block), i2 = 254 i1,
//   q1 = clamp(rne(v i1), +-127), q2 = clamp(rne(fma(-q1, c1, v) i2), +-127),
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
// 2^22 and leaves n's int8 in the float's low byte.
template <typename V4>
__device__ __forceinline__ void vx_xq_levels4(const V4& v, float c1, float i1, float i2, bool fin, uint32_t& w1,
                                              uint32_t& w2) {
#pragma clang fp contract(off)
    w1 = 0u;
    w2 = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float t1 = fin ? __builtin_fmaf(v[e], i1, VX_XQ_MAGIC) : VX_XQ_MAGIC;
        t1 = fminf(fmaxf(t1, VX_XQ_MAGIC - 127.0f), VX_XQ_MAGIC + 127.0f);
        const float q1 = t1 - VX_XQ_MAGIC;  // exact
        const float r = __builtin_fmaf(-q1, c1, v[e]);
        float t2 = fin ? __builtin_fmaf(r, i2, VX_XQ_MAGIC) : VX_XQ_MAGIC;
        t2 = fminf(fmaxf(t2, VX_XQ_MAGIC - 127.0f), VX_XQ_MAGIC + 127.0f);
        w1 |= (__float_as_uint(t1) & 0xFFu) << (8 * e);
        w2 |= (__float_as_uint(t2) & 0xFFu) << (8 * e);
    }
}

#endif  // VX_XQ_HPP
