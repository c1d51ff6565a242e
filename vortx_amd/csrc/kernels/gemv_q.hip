// gemv_q.hip — block-quantized GEMV y = W x and dequantize, for gfx950.
//
// Work split (batch 1, the HBM-bound case):
//   * workgroup = 4 wave64; wave w owns R consecutive rows;
//   * x (or a chunk of it) is staged once per workgroup in LDS as
//     [16 float4 slots][unit] with an odd unit pitch, so both the staging
//     stores and the per-lane ds_read_b128 are bank-conflict free;
//   * lane l handles unit (64 weights) l of every row in a pass of 64
//     units: per row it issues 128-bit loads of the unit's bytes (36 B for
//     Q4_0, 68 B for Q8_0, 48 B for Q4_K) — a wave's loads for one row
//     cover the row's contiguous bytes, and the R rows' loads are all in
//     flight before any is consumed;
//   * the decoded dot uses one byte->float convert and one FMA per
//     weight; x for the unit stays in 64 VGPRs across the R rows;
//   * partial sums are reduced across the wave with xor shuffles.
// Batch > 1 uses the same staging with exact per-weight decode and x read
// from LDS per 8-weight group; lanes are split into 64/LPR row groups so
// that NB * chunk fits the LDS budget.
#include "vx_quant.hpp"

extern __shared__ f32x4 vx_lds_x[];

// x staging. Units [ub, ub + cu) of the NB batch columns of x go to LDS as
// slot j of unit ul of column b -> vx_lds_x[(b * 16 + j) * upitch + ul].
// Float4 f of the chunk is (b, ul, j) with j fastest, so consecutive
// threads read consecutive 16-byte pieces of x. A thread moves up to four
// float4 per group; all four loads are issued before any store so a group
// costs one round trip, and the caller issues the first group's loads
// before its weight loads so the LDS stores wait only for x.
struct vx_xgroup {
    f32x4 v[4];
};

template <int NB, bool XV>
__device__ __forceinline__ void vx_stage_load(const vx_gemv_args& a, uint32_t ub, uint32_t cu, uint32_t g0,
                                              vx_xgroup& xg) {
    const uint32_t per_col = cu * 16u;
    const uint32_t total = per_col * NB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // Clamped, unconditional loads (no divergent branch between them);
        // entries past the chunk are loaded but never stored.
        const uint32_t f = min(g0 + threadIdx.x + VX_WG * i, total - 1u);
        const uint32_t b = NB == 1 ? 0u : f / per_col;
        const uint32_t rem = f - b * per_col;
        const uint32_t ul = rem >> 4, j = rem & 15u;
        const int64_t k = 64 * (int64_t)(ub + ul) + 4 * j;
        if constexpr (XV) {
            xg.v[i] = *(const f32x4*)(a.x + b * a.xs_b + k);
        } else {
            const float* xp = a.x + b * a.xs_b + k * a.xs_k;
            xg.v[i] = f32x4{xp[0], xp[a.xs_k], xp[2 * a.xs_k], xp[3 * a.xs_k]};
        }
    }
}

template <int NB>
__device__ __forceinline__ void vx_stage_store(const vx_gemv_args& a, uint32_t cu, uint32_t g0, const vx_xgroup& xg) {
    const uint32_t per_col = cu * 16u;
    const uint32_t total = per_col * NB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t f = g0 + threadIdx.x + VX_WG * i;
        if (f < total) {
            const uint32_t b = NB == 1 ? 0u : f / per_col;
            const uint32_t rem = f - b * per_col;
            vx_lds_x[(b * 16u + (rem & 15u)) * a.upitch + (rem >> 4)] = xg.v[i];
        }
    }
}

// Groups after the first (only when a chunk holds more than 1024 float4).
template <int NB, bool XV>
__device__ __forceinline__ void vx_stage_rest(const vx_gemv_args& a, uint32_t ub, uint32_t cu) {
    for (uint32_t g0 = 4 * VX_WG; g0 < cu * 16u * NB; g0 += 4 * VX_WG) {
        vx_xgroup xg;
        vx_stage_load<NB, XV>(a, ub, cu, g0, xg);
        vx_stage_store<NB>(a, cu, g0, xg);
    }
}

template <int QT, int R, bool XV>
__device__ __forceinline__ void vx_gemv_b1(const vx_gemv_args& a) {
    constexpr int NW = vx_unit<QT>::NW;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * 4u + wave) * R;

    const uint8_t* wrow[R];
    bool rok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rok[r] = row0 + r < a.M;
        wrow[r] = a.w + (uint64_t)(rok[r] ? row0 + r : 0u) * a.row_stride;
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;

    for (uint32_t ub = 0; ub < a.nunits; ub += a.chunk_units) {
        const uint32_t cu = min(a.chunk_units, a.nunits - ub);
        // x loads first, then the first pass's weight loads: the LDS stores
        // of x wait only for x, and the weights' HBM latency overlaps the
        // staging round trip and the barrier.
        vx_xgroup xg;
        vx_stage_load<1, XV>(a, ub, cu, 0, xg);
        // Loads are unconditional (rows past M read row 0, lanes past the
        // chunk read its first unit) so no branch hides them from the
        // wait-count bookkeeping; their contributions are discarded below.
        uint32_t wr[R][NW];
#pragma unroll
        for (int r = 0; r < R; ++r) vx_load_unit<QT>(wrow[r], ub + (lane < cu ? lane : 0u), wr[r]);
        if (ub) __syncthreads();
        vx_stage_store<1>(a, cu, 0, xg);
        vx_stage_rest<1, XV>(a, ub, cu);
        __syncthreads();

        for (uint32_t p = 0; p < cu; p += 64) {
            const uint32_t ul = p + lane;
            const bool act = ul < cu;
            if (p) {
#pragma unroll
                for (int r = 0; r < R; ++r) vx_load_unit<QT>(wrow[r], ub + (act ? ul : 0u), wr[r]);
            }
            float xv[64];
            const uint32_t uls = act ? ul : 0u;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const f32x4 t = vx_lds_x[j * a.upitch + uls];
                xv[4 * j + 0] = t.x; xv[4 * j + 1] = t.y; xv[4 * j + 2] = t.z; xv[4 * j + 3] = t.w;
            }
            float sx0 = 0.f, sx1 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) { sx0 += xv[i]; sx1 += xv[32 + i]; }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float d = vx_unit_dot_b1<QT>(wr[r], xv, sx0, sx1, ub + (act ? ul : 0u));
                acc[r] += act ? d : 0.f;
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = vx_wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (rok[r]) a.y[(int64_t)(row0 + r) * a.ys_m] = acc[r];
    }
}

// ------------------------------------------------------------------------
// Batch 1, persistent: one workgroup of WGT threads per CU (grid = CU
// count), wave w of the chip owning rows w, w + W, w + 2W, ... (W = waves
// in the grid). Items (row, pass of 64 units) stream through a P-deep
// register ring.
// Ordering is what makes this fast. x is needed before any arithmetic, an
// x request queued behind the CU's weight requests waits for them, and a
// wave issuing weight loads stalls while the CU's memory queue is full.
// So: every wave issues its share of the x loads; a bare s_barrier (no
// wait) puts all x requests of the CU ahead of every weight request; each
// wave issues one weight item only, stores x to LDS as soon as x alone has
// arrived and reaches the one barrier before any wave can stall on a full
// queue; the rest of the ring is issued after it. The two 32-block sums of
// x per unit (for the offset terms of vx_unit_dot_b1) are reduced in the
// staging step with lane shuffles, so no second barrier is needed.
// WGT = 1024: 16 waves of at most 128 VGPRs; 512: 8 waves with room for a
// deeper ring. x must fit VX_P_XF float4 (K <= 16384).
#define VX_P_XF 4096u

template <int QT, int P, int WGT, bool XV>
__device__ __forceinline__ void vx_gemv_p1(const vx_gemv_args& a) {
    constexpr int NW = vx_unit<QT>::NW;
    constexpr int XPT = (int)(VX_P_XF / WGT);
    const uint32_t t = threadIdx.x, lane = t & 63u;
    // wave-uniform (scalar) so that the item loop runs on scalar branches
    // and the wait counts stay exact
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nwv = gridDim.x * (WGT / 64u);
    const uint32_t gw = blockIdx.x * (WGT / 64u) + wave;
    const uint32_t nunits = a.nunits, npass = (nunits + 63u) >> 6;
    const uint32_t nrows = a.M > gw ? (a.M - gw + nwv - 1u) / nwv : 0u;
    const uint32_t nitems = nrows * npass;
    const uint32_t upitch = a.upitch;
    float* sxs = (float*)(vx_lds_x + 16u * upitch);  // [unit][2]

    // 1. x loads: float4 f of x = slot f & 15 of unit f >> 4 (k = 4 f).
    const uint32_t total = nunits * 16u;
    f32x4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        if ((uint32_t)i * WGT >= total) break;  // uniform: rounds past x
        const uint32_t f = min(t + WGT * (uint32_t)i, total - 1u);
        if constexpr (XV) {
            xr[i] = *(const f32x4*)(a.x + 4 * (int64_t)f);
        } else {
            const float* xp = a.x + 4 * (int64_t)f * a.xs_k;
            xr[i] = f32x4{xp[0], xp[a.xs_k], xp[2 * a.xs_k], xp[3 * a.xs_k]};
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // 2. the first item (clamped: past the end an item repeats the last
    //    one, which the cache serves; y is written only for real rows).
    const uint8_t* wbase = a.w;
    auto item_ptr = [&](uint32_t it, uint32_t& unit) {
        const uint32_t c = nitems ? min(it, nitems - 1u) : 0u;
        const uint32_t ri = c / npass, p = c - ri * npass;
        const uint32_t row = min(gw + ri * nwv, a.M - 1u);
        unit = min(64u * p + lane, nunits - 1u);
        return wbase + (uint64_t)row * a.row_stride;
    };
    uint32_t wr[P][NW];
    {
        uint32_t u;
        const uint8_t* rp = item_ptr(0u, u);
        vx_load_unit<QT>(rp, u, wr[0]);
    }

    // 3. x to LDS (waits for the x loads only) with the per-unit sums:
    //    the 16 slots of a unit sit in 16 consecutive lanes.
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        if ((uint32_t)i * WGT >= total) break;
        const uint32_t f = t + WGT * (uint32_t)i;
        const bool in = f < total;
        float ps = in ? (xr[i].x + xr[i].y) + (xr[i].z + xr[i].w) : 0.f;
        ps += __shfl_xor(ps, 1, 64);
        ps += __shfl_xor(ps, 2, 64);
        ps += __shfl_xor(ps, 4, 64);
        if (in) {
            vx_lds_x[(f & 15u) * upitch + (f >> 4)] = xr[i];
            if ((f & 7u) == 0u) sxs[2u * (f >> 4) + ((f >> 3) & 1u)] = ps;
        }
    }
    __syncthreads();

    // 4. the rest of the ring, then stream the items. The main loop runs
    //    whole rounds of P items so that every path through it issues the
    //    same loads (exact wait counts); the last partial round follows.
#pragma unroll
    for (int j = 1; j < P; ++j) {
        uint32_t u;
        const uint8_t* rp = item_ptr((uint32_t)j, u);
        vx_load_unit<QT>(rp, u, wr[j]);
    }
    float xv[64];
    float sx0 = 0.f, sx1 = 0.f;
    uint32_t cur = ~0u;
    float acc = 0.f;
    auto body = [&](uint32_t it, uint32_t (&w)[NW]) {
        const uint32_t ri = it / npass, p = it - ri * npass;
        const uint32_t u = 64u * p + lane;
        const bool act = u < nunits;
        const uint32_t us = act ? u : nunits - 1u;
        if (p != cur) {
            cur = p;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const f32x4 v = vx_lds_x[q * upitch + us];
                xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
            }
            sx0 = sxs[2u * us];
            sx1 = sxs[2u * us + 1u];
        }
        const float d = vx_unit_dot_b1<QT>(w, xv, sx0, sx1, us);
        acc += act ? d : 0.f;
        uint32_t nu;
        const uint8_t* rp = item_ptr(it + P, nu);
        vx_load_unit<QT>(rp, nu, w);
        if (p == npass - 1u) {
            const float sum = vx_wave_sum(acc);
            if (lane == 0) a.y[(int64_t)(gw + ri * nwv) * a.ys_m] = sum;
            acc = 0.f;
        }
    };
    const uint32_t nfull = nitems - nitems % P;
    for (uint32_t it0 = 0; it0 < nfull; it0 += P) {
#pragma unroll
        for (int j = 0; j < P; ++j) body(it0 + (uint32_t)j, wr[j]);
    }
#pragma unroll
    for (int j = 0; j < P - 1; ++j)
        if (nfull + (uint32_t)j < nitems) body(nfull + (uint32_t)j, wr[j]);
}

// ------------------------------------------------------------------------
// Integer-dot path. During staging every 32-element block of x (per batch
// column) is split into two int8 levels with one f32 scale:
//     x ~= c * (254 * x1 + x2),   c = max|x_blk| / (127 * 254),
//     x1 = rint(x / (254 c)),  x2 = rint((x - 254 c x1) / c)  (both in +-127)
// so |x - c (254 x1 + x2)| <= c / 2 ~ 1.6e-5 * max|x_blk|. A weight block
// then reduces in exact int32 with v_dot4_i32_i8:
//     T = 254 * sum(q * x1) + sum(q * x2)            (q the block's integers)
// and contributes d * c * T (minus the format's zero-point / min term).
// LDS per chunk and batch column: x1 / x2 as [level][4 slots of 16 B][unit]
// (odd unit pitch), then per 32-block: c, sum(x) (f32) and
// O = sum(254 x1 + x2) (int32), indexed 2 * unit + half.
struct vx_i8lds {
    uint32_t upitch, cu;
    __device__ __forceinline__ int4* x8(uint32_t b) const {
        return (int4*)vx_lds_x + (size_t)b * 8u * upitch;
    }
    __device__ __forceinline__ float* cs(uint32_t NB, uint32_t b) const {
        return (float*)((int4*)vx_lds_x + (size_t)NB * 8u * upitch) + (size_t)b * 2u * upitch;
    }
    __device__ __forceinline__ float* sx(uint32_t NB, uint32_t b) const { return cs(NB, NB) + (size_t)b * 2u * upitch; }
    __device__ __forceinline__ int* oz(uint32_t NB, uint32_t b) const {
        return (int*)(cs(NB, 2 * NB)) + (size_t)b * 2u * upitch;
    }
};

__device__ __forceinline__ uint32_t vx_pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

// Quantize one staged group of float4 (see vx_stage_load) and store it.
// The 8 float4 of a 32-block are 8 consecutive lanes.
template <int NB>
__device__ __forceinline__ void vx_stage_store_i8(const vx_gemv_args& a, uint32_t cu, uint32_t g0, const vx_xgroup& xg) {
    const uint32_t per_col = cu * 16u;
    const uint32_t total = per_col * NB;
    const vx_i8lds L{a.upitch, cu};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t f = g0 + threadIdx.x + VX_WG * i;
        const f32x4 v = xg.v[i];
        float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        const float c = m * (1.0f / (127.0f * 254.0f));
        const float inv1 = m > 0.f ? 127.0f / m : 0.f;  // 1 / (254 c)
        const float inv2 = inv1 * 254.0f;               // 1 / c
        const float s1 = 254.0f * c;
        const float e[4] = {v.x, v.y, v.z, v.w};
        int q1[4], q2[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            q1[t] = (int)rintf(e[t] * inv1);
            const float r = __builtin_fmaf(-(float)q1[t], s1, e[t]);
            q2[t] = min(127, max(-127, (int)rintf(r * inv2)));
        }
        float sx = (v.x + v.y) + (v.z + v.w);
        int oz = 254 * (q1[0] + q1[1] + q1[2] + q1[3]) + (q2[0] + q2[1] + q2[2] + q2[3]);
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            sx += __shfl_xor(sx, off, 64);
            oz += __shfl_xor(oz, off, 64);
        }
        if (f < total) {
            const uint32_t b = NB == 1 ? 0u : f / per_col;
            const uint32_t rem = f - b * per_col;
            const uint32_t ul = rem >> 4, j = rem & 15u;
            uint32_t* x8 = (uint32_t*)L.x8(b);
            // dword j of the unit's 64 bytes: slot j/4, dword j%4
            x8[((0u * 4u + (j >> 2)) * a.upitch + ul) * 4u + (j & 3u)] = vx_pack4(q1[0], q1[1], q1[2], q1[3]);
            x8[((1u * 4u + (j >> 2)) * a.upitch + ul) * 4u + (j & 3u)] = vx_pack4(q2[0], q2[1], q2[2], q2[3]);
            if ((j & 7u) == 0) {
                const uint32_t idx = 2u * ul + (j >> 3);
                L.cs(NB, b)[idx] = c;
                L.sx(NB, b)[idx] = sx;
                L.oz(NB, b)[idx] = oz;
            }
        }
    }
}

template <int NB, bool XV>
__device__ __forceinline__ void vx_stage_rest_i8(const vx_gemv_args& a, uint32_t ub, uint32_t cu) {
    for (uint32_t g0 = 4 * VX_WG; g0 < cu * 16u * NB; g0 += 4 * VX_WG) {
        vx_xgroup xg;
        vx_stage_load<NB, XV>(a, ub, cu, g0, xg);
        vx_stage_store_i8<NB>(a, cu, g0, xg);
    }
}

// One unit of one row against the staged int8 x of one batch column.
// x1 / x2: the unit's 16 dwords of each level (dword t = weights 4t..4t+3).
template <int QT>
__device__ __forceinline__ float vx_unit_dot_i8(const uint32_t (&r)[vx_unit<QT>::NW], const uint32_t (&x1)[16],
                                                const uint32_t (&x2)[16], const float (&cb)[2], const float (&sxb)[2],
                                                const int (&ozb)[2], uint32_t u) {
    if constexpr (QT == VX_Q4_0) {
        uint32_t q[8];
        q[0] = __builtin_amdgcn_alignbit(r[1], r[0], 16);
        q[1] = __builtin_amdgcn_alignbit(r[2], r[1], 16);
        q[2] = __builtin_amdgcn_alignbit(r[3], r[2], 16);
        q[3] = __builtin_amdgcn_alignbit(r[4], r[3], 16);
        q[4] = r[5]; q[5] = r[6]; q[6] = r[7]; q[7] = r[8];
        float res = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int i1 = 0, i2 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = vx_and(q[4 * h + i], 0x0F0F0F0Fu);
                const uint32_t hi = vx_and(q[4 * h + i] >> 4, 0x0F0F0F0Fu);
                i1 = __builtin_amdgcn_sdot4((int)lo, (int)x1[8 * h + i], i1, false);
                i1 = __builtin_amdgcn_sdot4((int)hi, (int)x1[8 * h + 4 + i], i1, false);
                i2 = __builtin_amdgcn_sdot4((int)lo, (int)x2[8 * h + i], i2, false);
                i2 = __builtin_amdgcn_sdot4((int)hi, (int)x2[8 * h + 4 + i], i2, false);
            }
            const int t = 254 * i1 + i2 - 8 * ozb[h];
            const float d = vx_f16_to_f32(h ? (r[4] >> 16) : r[0]);
            res = __builtin_fmaf(d * cb[h], (float)t, res);
        }
        return res;
    } else if constexpr (QT == VX_Q8_0) {
        float res = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int i1 = 0, i2 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t qd = h ? r[9 + i] : __builtin_amdgcn_alignbit(r[i + 1], r[i], 16);
                i1 = __builtin_amdgcn_sdot4((int)qd, (int)x1[8 * h + i], i1, false);
                i2 = __builtin_amdgcn_sdot4((int)qd, (int)x2[8 * h + i], i2, false);
            }
            const int t = 254 * i1 + i2;
            const float d = vx_f16_to_f32(h ? (r[8] >> 16) : r[0]);
            res = __builtin_fmaf(d * cb[h], (float)t, res);
        }
        return res;
    } else {
        const float d = vx_f16_to_f32(r[0]);
        const float dmin = vx_f16_to_f32(r[0] >> 16);
        uint32_t sc0, m0, sc1, m1;
        vx_q4k_scales(r[1], r[2], r[3], u & 3u, sc0, m0, sc1, m1);
        int a1 = 0, a2 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = vx_and(r[4 + i], 0x0F0F0F0Fu);
            const uint32_t hi = vx_and(r[4 + i] >> 4, 0x0F0F0F0Fu);
            a1 = __builtin_amdgcn_sdot4((int)lo, (int)x1[i], a1, false);
            a2 = __builtin_amdgcn_sdot4((int)lo, (int)x2[i], a2, false);
            b1 = __builtin_amdgcn_sdot4((int)hi, (int)x1[8 + i], b1, false);
            b2 = __builtin_amdgcn_sdot4((int)hi, (int)x2[8 + i], b2, false);
        }
        const float t0 = (float)(254 * a1 + a2), t1 = (float)(254 * b1 + b2);
        float res = __builtin_fmaf(d * (float)sc0 * cb[0], t0, -(dmin * (float)m0) * sxb[0]);
        res = __builtin_fmaf(d * (float)sc1 * cb[1], t1, res);
        return __builtin_fmaf(-(dmin * (float)m1), sxb[1], res);
    }
}

__device__ __forceinline__ void vx_read_x8(const vx_i8lds& L, uint32_t b, uint32_t ul, uint32_t (&x1)[16],
                                           uint32_t (&x2)[16]) {
    const int4* x8 = L.x8(b);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int4 v1 = x8[(0 * 4 + s) * L.upitch + ul];
        const int4 v2 = x8[(1 * 4 + s) * L.upitch + ul];
        x1[4 * s + 0] = v1.x; x1[4 * s + 1] = v1.y; x1[4 * s + 2] = v1.z; x1[4 * s + 3] = v1.w;
        x2[4 * s + 0] = v2.x; x2[4 * s + 1] = v2.y; x2[4 * s + 2] = v2.z; x2[4 * s + 3] = v2.w;
    }
}

// Batch 1 on the integer-dot path: same work split as vx_gemv_b1.
template <int QT, int R, bool XV>
__device__ __forceinline__ void vx_gemv_i8b1(const vx_gemv_args& a) {
    constexpr int NW = vx_unit<QT>::NW;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * 4u + wave) * R;
    const uint8_t* wrow[R];
    bool rok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rok[r] = row0 + r < a.M;
        wrow[r] = a.w + (uint64_t)(rok[r] ? row0 + r : 0u) * a.row_stride;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;

    for (uint32_t ub = 0; ub < a.nunits; ub += a.chunk_units) {
        const uint32_t cu = min(a.chunk_units, a.nunits - ub);
        const vx_i8lds L{a.upitch, cu};
        vx_xgroup xg;
        vx_stage_load<1, XV>(a, ub, cu, 0, xg);
        uint32_t wr[R][NW];
#pragma unroll
        for (int r = 0; r < R; ++r) vx_load_unit<QT>(wrow[r], ub + (lane < cu ? lane : 0u), wr[r]);
        if (ub) __syncthreads();
        vx_stage_store_i8<1>(a, cu, 0, xg);
        vx_stage_rest_i8<1, XV>(a, ub, cu);
        __syncthreads();

        for (uint32_t p = 0; p < cu; p += 64) {
            const uint32_t ul = p + lane;
            const bool act = ul < cu;
            const uint32_t uls = act ? ul : 0u;
            if (p) {
#pragma unroll
                for (int r = 0; r < R; ++r) vx_load_unit<QT>(wrow[r], ub + uls, wr[r]);
            }
            uint32_t x1[16], x2[16];
            vx_read_x8(L, 0, uls, x1, x2);
            const float2 cb2 = *(const float2*)&L.cs(1, 0)[2 * uls];
            const float2 sx2 = *(const float2*)&L.sx(1, 0)[2 * uls];
            const int2 oz2 = *(const int2*)&L.oz(1, 0)[2 * uls];
            const float cb[2] = {cb2.x, cb2.y}, sxb[2] = {sx2.x, sx2.y};
            const int ozb[2] = {oz2.x, oz2.y};
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float d = vx_unit_dot_i8<QT>(wr[r], x1, x2, cb, sxb, ozb, ub + uls);
                acc[r] += act ? d : 0.f;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = vx_wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (rok[r]) a.y[(int64_t)(row0 + r) * a.ys_m] = acc[r];
    }
}

// Batch NB > 1: lane l serves row group g = l / LPR (R rows each) and unit
// l % LPR of each pass; weights are decoded exactly 8 at a time and
// multiplied with the matching x slots of every batch column from LDS.
template <int QT, int NB, int R, int LPR, bool XV>
__device__ __forceinline__ void vx_gemv_bn(const vx_gemv_args& a) {
    constexpr int NW = vx_unit<QT>::NW;
    constexpr int G = 64 / LPR;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t row0 = ((blockIdx.x * 4u + wave) * G + g) * R;

    const uint8_t* wrow[R];
    bool rok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rok[r] = row0 + r < a.M;
        wrow[r] = a.w + (uint64_t)(rok[r] ? row0 + r : 0u) * a.row_stride;
    }
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;

    for (uint32_t ub = 0; ub < a.nunits; ub += a.chunk_units) {
        const uint32_t cu = min(a.chunk_units, a.nunits - ub);
        vx_xgroup xg;
        vx_stage_load<NB, XV>(a, ub, cu, 0, xg);
        if (ub) __syncthreads();
        vx_stage_store<NB>(a, cu, 0, xg);
        vx_stage_rest<NB, XV>(a, ub, cu);
        __syncthreads();
        for (uint32_t p = 0; p < cu; p += LPR) {
            const uint32_t ul = p + li;
            const bool act = ul < cu;
            const uint32_t uls = act ? ul : 0u;
            uint32_t wr[R][NW];
#pragma unroll
            for (int r = 0; r < R; ++r) vx_load_unit<QT>(wrow[r], ub + uls, wr[r]);
            float sc[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) vx_unit_scales<QT>(wr[r], ub + ul, sc[r]);
#pragma unroll
            for (int grp = 0; grp < 8; ++grp) {
                float wv[R][8];
                int ja = 0, jb = 0;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    vx_unit_group<QT>(wr[r], sc[r], grp, wv[r], ja, jb);
#pragma unroll
                    for (int e = 0; e < 8; ++e) wv[r][e] = act ? wv[r][e] : 0.f;
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const f32x4 xa = vx_lds_x[(b * 16 + ja) * a.upitch + uls];
                    const f32x4 xb = vx_lds_x[(b * 16 + jb) * a.upitch + uls];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float s = acc[r][b];
                        s = __builtin_fmaf(wv[r][0], xa.x, s);
                        s = __builtin_fmaf(wv[r][1], xa.y, s);
                        s = __builtin_fmaf(wv[r][2], xa.z, s);
                        s = __builtin_fmaf(wv[r][3], xa.w, s);
                        s = __builtin_fmaf(wv[r][4], xb.x, s);
                        s = __builtin_fmaf(wv[r][5], xb.y, s);
                        s = __builtin_fmaf(wv[r][6], xb.z, s);
                        s = __builtin_fmaf(wv[r][7], xb.w, s);
                        acc[r][b] = s;
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = vx_group_sum(acc[r][b], LPR);
    if (li == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (rok[r]) {
#pragma unroll
                for (int b = 0; b < NB; ++b) a.y[(int64_t)(row0 + r) * a.ys_m + (int64_t)b * a.ys_b] = acc[r][b];
            }
    }
}

// ------------------------------------------------------------------------
// Batched path on the matrix cores: v_mfma_f32_16x16x4f32 with
//   A = 16 rows x 4 k of exactly decoded f32 weights (lane l: row l%16,
//       k-slot l/16),
//   B = 4 k x 16 batch columns of f32 x from LDS (lane l: k-slot l/16,
//       column l%16; columns >= B read zeros),
//   D = 16 rows x 16 columns in 4 VGPRs (lane l: rows 4(l/16)+v, column
//       l%16),
// so weights, x and the accumulation stay f32 and no per-block rescale is
// needed. A wave owns 16-row tiles; within one MFMA the four k-slots take
// element s of four consecutive units (64-weight groups) of the same rows, so
// lane (r, q) streams unit 4g+q of row r with the same 128-bit loads as the
// batch-1 kernel. KS waves of a workgroup split K (interleaved unit
// groups) and their partial tiles are summed through LDS at the end; x is
// staged per K chunk as [column][k] with a pitch of Kc + 4 floats (bank
// conflict free for the 16 columns a 16-lane phase reads).
template <int QT>
__device__ __forceinline__ void vx_unit_decode64(const uint32_t (&r)[vx_unit<QT>::NW], uint32_t u, float (&w)[64]) {
    if constexpr (QT == VX_Q4_0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float d = vx_f16_to_f32(h ? (r[4] >> 16) : r[0]);
            const float o = -8.f * d;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t qd = h ? r[5 + i] : __builtin_amdgcn_alignbit(r[i + 1], r[i], 16);
                const uint32_t lo = vx_and(qd, 0x0F0F0F0Fu), hi = vx_and(qd >> 4, 0x0F0F0F0Fu);
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    w[32 * h + 4 * i + b] = __builtin_fmaf(vx_ub(lo, b), d, o);
                    w[32 * h + 16 + 4 * i + b] = __builtin_fmaf(vx_ub(hi, b), d, o);
                }
            }
        }
    } else if constexpr (QT == VX_Q8_0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float d = vx_f16_to_f32(h ? (r[8] >> 16) : r[0]);
            const float o = -128.f * d;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t qd = h ? r[9 + i] : __builtin_amdgcn_alignbit(r[i + 1], r[i], 16);
                const uint32_t uq = vx_xor(qd, 0x80808080u);  // q + 128, exact: (q+128) d - 128 d
#pragma unroll
                for (int b = 0; b < 4; ++b) w[32 * h + 4 * i + b] = __builtin_fmaf(vx_ub(uq, b), d, o);
            }
        }
    } else {
        float sc[4];
        vx_unit_scales<QT>(r, u, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = vx_and(r[4 + i], 0x0F0F0F0Fu), hi = vx_and(r[4 + i] >> 4, 0x0F0F0F0Fu);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[4 * i + b] = __builtin_fmaf(vx_ub(lo, b), sc[0], sc[1]);
                w[32 + 4 * i + b] = __builtin_fmaf(vx_ub(hi, b), sc[2], sc[3]);
            }
        }
    }
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

// One 16-row tile per wave. The wave's unit groups (256 k each) are
// g = ks, ks + KS, ...; their weights are loaded PD groups ahead in a
// register ring, across LDS chunk boundaries, so HBM latency overlaps the
// MFMA work. kc / 256 (groups per chunk) is a multiple of KS, so all waves
// of a workgroup cross chunk boundaries - and reach the staging barriers -
// at the same loop step.
template <int QT, int KS, int PD>
__device__ __forceinline__ void vx_gemv_mfma(const vx_gemv_args& a) {
    constexpr int NW = vx_unit<QT>::NW;
    constexpr int TG = 4 / KS;  // tiles per workgroup
    float* xs = (float*)vx_lds_x;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t i16 = lane & 15u, q = lane >> 4;
    const uint32_t ks = wave % KS;
    const uint32_t tile = blockIdx.x * TG + wave / KS;
    const uint32_t kc = a.chunk_units * 64u;  // k per LDS chunk, multiple of 256 * KS
    const uint32_t pitch = kc + 4u;
    const uint32_t ngroups = a.K / 256u;
    const uint32_t nj = ngroups > ks ? (ngroups - ks + KS - 1) / KS : 0u;  // this wave's groups
    const uint32_t row = min(tile * 16u + i16, a.M - 1u);  // rows past M read the last row
    const uint8_t* wrow = a.w + (uint64_t)row * a.row_stride;

    f32x4v acc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = f32x4v{0.f, 0.f, 0.f, 0.f};

    uint32_t wr[PD][NW];
#pragma unroll
    for (int p = 0; p < PD; ++p) {
        const uint32_t g = ks + KS * min((uint32_t)p, nj ? nj - 1u : 0u);
        vx_load_unit<QT>(wrow, 4u * min(g, ngroups - 1u) + q, wr[p]);
    }

    uint32_t cur_chunk = 0xFFFFFFFFu;
    // every wave runs the same number of outer steps (the max over waves) so
    // the staging barriers line up; steps past a wave's last group skip work.
    const uint32_t nj_max = (ngroups + KS - 1) / KS;
    for (uint32_t j0 = 0; j0 < nj_max; j0 += PD) {
#pragma unroll
        for (int p = 0; p < PD; ++p) {
            const uint32_t j = j0 + p;
            if (j >= nj_max) break;  // uniform across the workgroup
            const uint32_t g = ks + KS * j;
            const uint32_t chunk = (KS * j * 256u) / kc;  // same for every ks
            if (chunk != cur_chunk) {
                cur_chunk = chunk;
                const uint32_t k0 = chunk * kc;
                const uint32_t klen = min(kc, a.K - k0);
                __syncthreads();
                for (uint32_t f = threadIdx.x; f < 16u * (kc / 4u); f += VX_WG) {
                    const uint32_t b = f / (kc / 4u), k4 = 4u * (f % (kc / 4u));
                    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (b < a.B && k4 < klen) {
                        const int64_t k = (int64_t)k0 + k4;
                        if (a.x_vec) {
                            v = *(const f32x4*)(a.x + b * a.xs_b + k);
                        } else {
                            const float* xp = a.x + b * a.xs_b + k * a.xs_k;
                            v = f32x4{xp[0], xp[a.xs_k], xp[2 * a.xs_k], xp[3 * a.xs_k]};
                        }
                    }
                    *(f32x4*)(xs + b * pitch + k4) = v;
                }
                __syncthreads();
            }
            if (j < nj) {
                float w[64];
                vx_unit_decode64<QT>(wr[p], 4u * g + q, w);
                // prefetch the group PD steps ahead into the freed slot
                const uint32_t jn = min(j + PD, nj - 1u);
                vx_load_unit<QT>(wrow, 4u * (ks + KS * jn) + q, wr[p]);
                const float* xb = xs + i16 * pitch + (g * 256u - chunk * kc) + 64u * q;
#pragma unroll
                for (int s4 = 0; s4 < 16; ++s4) {
                    const f32x4 xv = *(const f32x4*)(xb + 4 * s4);
                    acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * s4 + 0], xv.x, acc[0], 0, 0, 0);
                    acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * s4 + 1], xv.y, acc[1], 0, 0, 0);
                    acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * s4 + 2], xv.z, acc[2], 0, 0, 0);
                    acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * s4 + 3], xv.w, acc[3], 0, 0, 0);
                }
            }
        }
    }

    // Sum the accumulators, then the KS partial tiles through LDS; store
    // rows 4(l/16)+v, column l%16.
    f32x4v tot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    if constexpr (KS > 1) {
        __syncthreads();
        f32x4v* red = (f32x4v*)vx_lds_x;  // [wave][lane]
        red[wave * 64 + lane] = tot;
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int o = 1; o < KS; ++o) tot += red[(wave + o) * 64 + lane];
        }
    }
    if (ks == 0 && i16 < a.B) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t r = tile * 16u + 4u * q + v;
            if (r < a.M) a.y[(int64_t)r * a.ys_m + (int64_t)i16 * a.ys_b] = tot[v];
        }
    }
}

// ------------------------------------------------------------------------
// Batched path on f16 matrix cores at f32 accuracy (B >= 2, 16 columns per
// launch).
//   D[i][j] = sum_k X[i][k] Wq[k][j] with v_mfma_f32_16x16x32_f16:
//     Wq (B operand) = the block integers of 16 rows j (q - 8 for Q4_0, q
//       for Q8_0 and Q4_K), exact in f16: nibbles / bytes are placed in the
//       mantissa of 1024.0 and the offset is removed with an exact packed
//       f16 subtraction;
//     X (A operand) = 16 batch columns i of x in two f16 levels x1 + x2.
//       Per chunk of 512 k and column, x is first scaled by 2^n so that the
//       chunk's max |x| lies in [2^14, 2^15): then |x s - x1 - x2| <=
//       max(2^-22 |x s|, 2^-25), i.e. finer than f32 rounding relative to
//       the column's scale, with no f16 overflow or loss to subnormals;
//   each level is one MFMA into the block's accumulator, and the lane that
//   loaded row j applies the block scale: acc += d D (Q4_K: + (-dmin m) S,
//   S the scaled block sum of x). At the end of a chunk acc_chunk * 2^-n is
//   added to the running sum.
// Lane l: row j = l%16 of the tile, k-octet o = l/16 of every 32-block
//   (A and B operands), outputs D[4o+v][j] = y[row j][column 4o+v].
// The four lanes of a row load the same 64-weight unit (the TA merges the
// identical addresses) and each takes one octet of every block. Within an
// octet, k follows the order in which the packing yields the pairs:
//   (e0,e2) (e1,e3) (e4,e6) (e5,e7) of the octet's 8 elements, where
//   Q4_0's octet o is elements 4o..4o+3 and 16+4o..16+4o+3 of its block
//   (low and high nibbles of qs dword o), and Q8_0 / Q4_K's octet is
//   elements 8o..8o+7.
// LDS: per 32-block, level and octet, 16 columns x 16 bytes (lane l reads
//   group (o, l%16): conflict free); then the Q4_K block sums [blk][col],
//   the per-wave column maxima and the chunk exponents.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4h __attribute__((ext_vector_type(4)));

#define VX_H_KC 512u  // k per staged chunk
#define VX_H_NG (VX_H_KC / 128u)  // 8-element groups per thread per chunk

// Exact packed f16 subtraction of a small-integer offset from 1024 + q pairs.
__device__ __forceinline__ uint32_t vx_h2_sub(uint32_t bits, float off) {
    const _Float16 o = (_Float16)off;
    const f16x2 v = __builtin_bit_cast(f16x2, bits) - f16x2{o, o};
    return __builtin_bit_cast(uint32_t, v);
}

// f16 pairs (1024 + nibble) of the nibbles at bits (sh, sh + 16) of w.
__device__ __forceinline__ uint32_t vx_nib_pair(uint32_t w, uint32_t sh) {
    return ((w >> sh) & 0x000F000Fu) | 0x64006400u;
}

// x of one 8-element group (block blk, octet o, column col) of the chunk at
// k0, in packing order. Q4_0 groups are two float4 at 4o and 16 + 4o, the
// others at 8o and 8o + 4.
template <int QT, int XV>
__device__ __forceinline__ void vx_h_load(const vx_gemv_args& a, uint32_t k0, uint32_t blk, uint32_t o,
                                          uint32_t col, bool live, float (&e)[8]) {
    const uint32_t ka = k0 + blk * 32u + (QT == VX_Q4_0 ? 4u * o : 8u * o);
    const uint32_t kb = ka + (QT == VX_Q4_0 ? 16u : 4u);
    if constexpr (XV) {
        f32x4 u = f32x4{0.f, 0.f, 0.f, 0.f}, v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (live) {
            const float* xc = a.x + (int64_t)col * a.xs_b;
            u = *(const f32x4*)(xc + ka);
            v = *(const f32x4*)(xc + kb);
        }
        e[0] = u.x; e[1] = u.z; e[2] = u.y; e[3] = u.w;
        e[4] = v.x; e[5] = v.z; e[6] = v.y; e[7] = v.w;
    } else {
        const uint32_t ord[4] = {0u, 2u, 1u, 3u};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t k = (t < 4 ? ka : kb) + ord[t & 3];
            e[t] = live ? a.x[(int64_t)col * a.xs_b + (int64_t)k * a.xs_k] : 0.f;
        }
    }
}

template <int QT, int KS, int XV>
__device__ __forceinline__ void vx_gemv_h16(const vx_gemv_args& a) {
    constexpr int TG = 4 / KS;  // 16-row tiles per workgroup
    constexpr uint32_t NBLK = VX_H_KC / 32u;
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t j16 = lane & 15u, o = lane >> 4;
    const uint32_t ks = wave % KS;
    const uint32_t tile = blockIdx.x * TG + wave / KS;
    const uint32_t row = min(tile * 16u + j16, a.M - 1u);
    const uint8_t* wrow = a.w + (uint64_t)row * a.row_stride;

    uint4* xg = (uint4*)vx_lds_x;                          // [blk][level][octet][col]
    float* sums = (float*)(xg + NBLK * 2u * 64u);           // [blk][col] (Q4_K)
    float* wmax = sums + NBLK * 16u;                        // [wave][col]
    int* nexp = (int*)(wmax + 64);                          // [col]

    f32x4h acc = f32x4h{0.f, 0.f, 0.f, 0.f};
    for (uint32_t k0 = 0; k0 < a.K; k0 += VX_H_KC) {
        const uint32_t klen = min(VX_H_KC, a.K - k0);  // a multiple of 64
        // ---- stage: load the chunk, per-column max |x|
        const uint32_t col = t & 15u;
        float e[VX_H_NG][8];
        float mx = 0.f;
#pragma unroll
        for (uint32_t g = 0; g < VX_H_NG; ++g) {
            const uint32_t f = t + g * VX_WG;
            const uint32_t go = (f >> 4) & 3u, blk = f >> 6;
            vx_h_load<QT, XV>(a, k0, blk, go, col, col < a.B && blk * 32u < klen, e[g]);
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(e[g][i]));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (lane < 16u) wmax[wave * 16u + lane] = mx;
        __syncthreads();  // also: every wave is done with the previous chunk
        const float m = fmaxf(fmaxf(wmax[col], wmax[16u + col]), fmaxf(wmax[32u + col], wmax[48u + col]));
        const int n = (m < __builtin_inff()) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
        if (t < 16u) nexp[t] = n;
#pragma unroll
        for (uint32_t g = 0; g < VX_H_NG; ++g) {
            const uint32_t f = t + g * VX_WG;
            const uint32_t go = (f >> 4) & 3u, blk = f >> 6;
            uint32_t l1[4], l2[4];
            float part = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float v0 = __builtin_amdgcn_ldexpf(e[g][i], n), v1 = __builtin_amdgcn_ldexpf(e[g][i + 1], n);
                part += v0 + v1;
                const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
                const _Float16 r0 = (_Float16)(v0 - (float)h0), r1 = (_Float16)(v1 - (float)h1);
                l1[i / 2] = __builtin_bit_cast(uint32_t, f16x2{h0, h1});
                l2[i / 2] = __builtin_bit_cast(uint32_t, f16x2{r0, r1});
            }
            const uint32_t base = blk * 128u + go * 16u + col;
            xg[base] = uint4{l1[0], l1[1], l1[2], l1[3]};
            xg[base + 64u] = uint4{l2[0], l2[1], l2[2], l2[3]};
            if constexpr (QT == VX_Q4_K) {
                part += __shfl_xor(part, 16, 64);
                part += __shfl_xor(part, 32, 64);
                if (go == 0u) sums[blk * 16u + col] = part;
            }
        }
        __syncthreads();

        // ---- compute: units of this wave's k-slice, two 32-blocks each
        f32x4h accc = f32x4h{0.f, 0.f, 0.f, 0.f};
        const uint32_t u0 = k0 / 64u, un = klen / 64u;
        for (uint32_t ul = ks; ul < un; ul += KS) {
            uint32_t r[vx_unit<QT>::NW];
            vx_load_unit<QT>(wrow, u0 + ul, r);
            float sc[4];
            if constexpr (QT == VX_Q4_K) vx_unit_scales<QT>(r, u0 + ul, sc);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t blk = 2u * ul + h;
                uint32_t p[4];
                float d;
                if constexpr (QT == VX_Q4_0) {
                    const uint32_t qd = h ? r[5 + o] : __builtin_amdgcn_alignbit(r[o + 1], r[o], 16);
                    p[0] = vx_h2_sub(vx_nib_pair(qd, 0), 1032.f);
                    p[1] = vx_h2_sub(vx_nib_pair(qd, 8), 1032.f);
                    p[2] = vx_h2_sub(vx_nib_pair(qd, 4), 1032.f);
                    p[3] = vx_h2_sub(vx_nib_pair(qd, 12), 1032.f);
                    d = vx_f16_to_f32(h ? (r[4] >> 16) : r[0]);
                } else if constexpr (QT == VX_Q8_0) {
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const int di = 2 * (int)o + q;
                        const uint32_t qd = h ? r[9 + di] : __builtin_amdgcn_alignbit(r[di + 1], r[di], 16);
                        const uint32_t u = vx_xor(qd, 0x80808080u);  // q + 128
                        p[2 * q] = vx_h2_sub((u & 0x00FF00FFu) | 0x64006400u, 1152.f);
                        p[2 * q + 1] = vx_h2_sub(((u >> 8) & 0x00FF00FFu) | 0x64006400u, 1152.f);
                    }
                    d = vx_f16_to_f32(h ? (r[8] >> 16) : r[0]);
                } else {
                    const uint32_t w0 = r[4 + 2 * o], w1 = r[5 + 2 * o], sh = 4u * h;
                    p[0] = vx_h2_sub(vx_nib_pair(w0, sh), 1024.f);
                    p[1] = vx_h2_sub(vx_nib_pair(w0, sh + 8u), 1024.f);
                    p[2] = vx_h2_sub(vx_nib_pair(w1, sh), 1024.f);
                    p[3] = vx_h2_sub(vx_nib_pair(w1, sh + 8u), 1024.f);
                    d = sc[2 * h];
                }
                const f16x8 bw = __builtin_bit_cast(f16x8, uint4{p[0], p[1], p[2], p[3]});
                const uint32_t gb = blk * 128u + o * 16u + j16;
                const f16x8 x1 = __builtin_bit_cast(f16x8, xg[gb]);
                const f16x8 x2 = __builtin_bit_cast(f16x8, xg[gb + 64u]);
                f32x4h dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, bw, f32x4h{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(x2, bw, dd, 0, 0, 0);
                if constexpr (QT == VX_Q4_K) {
                    const f32x4 sv = *(const f32x4*)(sums + blk * 16u + 4u * o);
#pragma unroll
                    for (int v = 0; v < 4; ++v) accc[v] = __builtin_fmaf(sc[2 * h + 1], sv[v], accc[v]);
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) accc[v] = __builtin_fmaf(d, dd[v], accc[v]);
            }
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] += __builtin_amdgcn_ldexpf(accc[v], -nexp[4u * o + v]);
    }
    if constexpr (KS > 1) {
        __syncthreads();
        f32x4h* red = (f32x4h*)vx_lds_x;
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int w = 1; w < KS; ++w) acc += red[(wave + w) * 64 + lane];
        }
    }
    if (ks == 0) {
        const uint32_t r0 = tile * 16u + j16;
        if (r0 < a.M) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t c = 4u * o + v;
                if (c < a.B) a.y[(int64_t)r0 * a.ys_m + (int64_t)c * a.ys_b] = acc[v];
            }
        }
    }
}

// Any layout fallback (K a multiple of 32, any alignment, any B): one
// wave per row, lane l decodes 32-weight groups l, l+64, ... byte by byte.
template <int QT>
__device__ __forceinline__ void vx_gemv_generic(const vx_gemv_args& a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= a.M) return;  // wave-uniform; no barrier in this kernel
    const uint8_t* wrow = a.w + (uint64_t)row * a.row_stride;
    const uint32_t ngroups = a.K / 32u;
    for (uint32_t b = 0; b < a.B; ++b) {
        float acc = 0.f;
        for (uint32_t kb = lane; kb < ngroups; kb += 64) {
            float o[32];
            vx_decode32<QT>(wrow, kb, o);
            const float* xp = a.x + (int64_t)b * a.xs_b + (int64_t)(32 * kb) * a.xs_k;
#pragma unroll
            for (int i = 0; i < 32; ++i) acc = __builtin_fmaf(o[i], xp[(int64_t)i * a.xs_k], acc);
        }
        acc = vx_wave_sum(acc);
        if (lane == 0) a.y[(int64_t)row * a.ys_m + (int64_t)b * a.ys_b] = acc;
    }
}

// out[m, k] = decode(W)[m, k]; thread per 32-weight group. Output view:
// element (m, k) at y[m * ys_m + k * ys_b].
template <int QT>
__device__ __forceinline__ void vx_dequant(const vx_gemv_args& a) {
    const uint32_t ngroups = a.K / 32u;
    const uint64_t t = (uint64_t)blockIdx.x * VX_WG + threadIdx.x;
    if (t >= (uint64_t)a.M * ngroups) return;
    const uint32_t m = (uint32_t)(t / ngroups), kb = (uint32_t)(t % ngroups);
    float o[32];
    vx_decode32<QT>(a.w + (uint64_t)m * a.row_stride, kb, o);
    float* op = a.y + (int64_t)m * a.ys_m + (int64_t)(32 * kb) * a.ys_b;
#pragma unroll
    for (int i = 0; i < 32; ++i) op[(int64_t)i * a.ys_b] = o[i];
}

#define VX_GEMV_B1(QT, QN, R)                                                              \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_b1_##QN##_r##R(vx_gemv_args a) { \
        if (a.x_vec) vx_gemv_b1<QT, R, true>(a);                                           \
        else vx_gemv_b1<QT, R, false>(a);                                                  \
    }
#define VX_GEMV_I8B1(QT, QN, R)                                                               \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_i8b1_##QN##_r##R(vx_gemv_args a) { \
        if (a.x_vec) vx_gemv_i8b1<QT, R, true>(a);                                           \
        else vx_gemv_i8b1<QT, R, false>(a);                                                  \
    }
#define VX_GEMV_BN(QT, QN, NB, R, LPR)                                                            \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_b##NB##_##QN##_r##R(vx_gemv_args a) { \
        if (a.x_vec) vx_gemv_bn<QT, NB, R, LPR, true>(a);                                         \
        else vx_gemv_bn<QT, NB, R, LPR, false>(a);                                                \
    }
#define VX_GEMV_MFMA(QT, QN, KS, PD)                                                              \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_mfma_##QN##_s##KS##_p##PD(vx_gemv_args a) { \
        vx_gemv_mfma<QT, KS, PD>(a);                                                              \
    }
#define VX_GEMV_H16(QT, QN, KS)                                                                 \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_h16_##QN##_s##KS(vx_gemv_args a) {  \
        if (a.x_vec) vx_gemv_h16<QT, KS, 1>(a); else vx_gemv_h16<QT, KS, 0>(a);                \
    }
#define VX_GEMV_P1(QT, QN, P, WGT)                                                              \
    extern "C" __global__ __launch_bounds__(WGT) void vx_gemv_p1_##QN##_w##WGT(vx_gemv_args a) {  \
        if (a.x_vec) vx_gemv_p1<QT, P, WGT, true>(a); else vx_gemv_p1<QT, P, WGT, false>(a);   \
    }
#define VX_GEMV_ALL(QT, QN)                                                                         \
    VX_GEMV_B1(QT, QN, 1)                                                                           \
    VX_GEMV_B1(QT, QN, 2)                                                                           \
    VX_GEMV_B1(QT, QN, 4)                                                                           \
    VX_GEMV_B1(QT, QN, 8)                                                                           \
    VX_GEMV_I8B1(QT, QN, 1)                                                                         \
    VX_GEMV_I8B1(QT, QN, 2)                                                                         \
    VX_GEMV_I8B1(QT, QN, 4)                                                                         \
    VX_GEMV_I8B1(QT, QN, 8)                                                                         \
    VX_GEMV_BN(QT, QN, 2, 2, 64)                                                                    \
    VX_GEMV_BN(QT, QN, 4, 2, 64)                                                                    \
    VX_GEMV_BN(QT, QN, 8, 2, 32)                                                                    \
    VX_GEMV_BN(QT, QN, 16, 2, 16)                                                                   \
    VX_GEMV_H16(QT, QN, 1)                                                                         \
    VX_GEMV_H16(QT, QN, 2)                                                                         \
    VX_GEMV_H16(QT, QN, 4)                                                                         \
    VX_GEMV_MFMA(QT, QN, 1, 2)                                                                      \
    VX_GEMV_MFMA(QT, QN, 2, 2)                                                                      \
    VX_GEMV_MFMA(QT, QN, 4, 2)                                                                      \
    VX_GEMV_MFMA(QT, QN, 1, 4)                                                                      \
    VX_GEMV_MFMA(QT, QN, 2, 4)                                                                      \
    VX_GEMV_MFMA(QT, QN, 4, 4)                                                                      \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_generic_##QN(vx_gemv_args a) {     \
        vx_gemv_generic<QT>(a);                                                                     \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_dequant_##QN(vx_gemv_args a) { vx_dequant<QT>(a); }

VX_GEMV_ALL(VX_Q4_0, q4_0)
VX_GEMV_ALL(VX_Q8_0, q8_0)
VX_GEMV_ALL(VX_Q4_K, q4_k)
VX_GEMV_P1(VX_Q4_0, q4_0, 2, 1024)
VX_GEMV_P1(VX_Q8_0, q8_0, 1, 1024)
VX_GEMV_P1(VX_Q4_K, q4_k, 2, 1024)
VX_GEMV_P1(VX_Q4_0, q4_0, 4, 512)
VX_GEMV_P1(VX_Q8_0, q8_0, 3, 512)
VX_GEMV_P1(VX_Q4_K, q4_k, 4, 512)
