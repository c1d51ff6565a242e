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
#include "vx_xq.hpp"

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
// wave issues at most two weight items, stores x to LDS as soon as x alone
// has arrived and reaches the one barrier before any wave can stall on a
// full queue; the rest of a deeper ring is issued after it. The two 32-block sums of
// x per unit (for the offset terms of vx_unit_dot_b1) are reduced in the
// staging step with lane shuffles, so no second barrier is needed.
// WGT = 1024: 16 waves of at most 128 VGPRs. x must fit VX_P_XF float4
// (K <= 16384).
#define VX_P_XF 4096u

template <int QT, int P, int WGT, bool XV, bool XM = false>
__device__ __forceinline__ void vx_gemv_p1(const vx_gemv_args& a, uint32_t G) {
    constexpr int NW = vx_unit<QT>::NW;
    constexpr int XPT = (int)(VX_P_XF / WGT);
    const uint32_t t = threadIdx.x, lane = t & 63u;
    // wave-uniform (scalar) so that the item loop runs on scalar branches
    // and the wait counts stay exact
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nwv = G * (WGT / 64u);
    // waves interleaved over the CUs (wave-major), so the rows left over
    // after whole rounds of nwv spread evenly: at M = 11008 every CU gets 43
    // rows (CU-major numbering gives 176 CUs 48 rows and 80 CUs 32). XM:
    // positions per XCD as in vx_gemv_p1i.
    const uint32_t pb = (XM && (G & 7u) == 0u) ? (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const uint32_t gw = wave * G + pb;
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

    // 2. the first items (clamped: past the end an item repeats the last
    //    one, which the cache serves; y is written only for real rows).
    const uint8_t* wbase = a.w;
    // Past the last item the ring still issues its loads (so that every
    // round issues the same loads and the wait counts stay exact), but all
    // lanes then read unit 0 of the last item's row: one cache line the
    // wave has just fetched, so the wave does not end waiting on a full row.
    auto item_ptr = [&](uint32_t it, uint32_t& unit) {
        const uint32_t c = nitems ? min(it, nitems - 1u) : 0u;
        const uint32_t ri = c / npass, p = c - ri * npass;
        const uint32_t row = min(gw + ri * nwv, a.M - 1u);
        unit = it < nitems ? min(64u * p + lane, nunits - 1u) : 0u;
        return wbase + (uint64_t)row * a.row_stride;
    };
    // PRE items go out before the x barrier: the whole ring when it is at
    // most 2 deep (measured: Q4_K 32000x4096 3 % faster, Q4_0 unchanged);
    // deeper rings issue one, since waves then stall on a full memory queue
    // before reaching the barrier.
    constexpr int PRE = P <= 2 ? P : 1;
    uint32_t wr[P][NW];
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        uint32_t u;
        const uint8_t* rp = item_ptr((uint32_t)j, u);
        vx_load_unit<QT>(rp, u, wr[j]);
    }

    // 3. x to LDS (waits for the x loads only) with the per-unit sums:
    //    the 16 slots of a unit sit in 16 consecutive lanes.
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        if ((uint32_t)i * WGT >= total) break;
        const uint32_t f = t + WGT * (uint32_t)i;
        const bool in = f < total;
        const float ps = vx_sum8(in ? (xr[i].x + xr[i].y) + (xr[i].z + xr[i].w) : 0.f);
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
    for (int j = PRE; j < P; ++j) {
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
            // The LDS addresses derive from a value defined inside this
            // branch, so the compiler cannot hoist their arithmetic into every
            // item (with one pass, K <= 4096, the branch runs once per wave).
            uint32_t ul = us;
            asm volatile("" : "+v"(ul));
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const f32x4 v = vx_lds_x[q * upitch + ul];
                xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
            }
            sx0 = sxs[2u * ul];
            sx1 = sxs[2u * ul + 1u];
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
// -8 O with O = sum(254 x1 + x2) (int32: Q4_0's zero point -8 sum(x) at the
// scale c), indexed 2 * unit + half.
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
        // a non-finite block (fmaxf skips NaN; the sum does not) stores
        // max + sum as its scale, so y is non-finite
        const bool fin = m < __builtin_inff() && sx == sx;
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
                L.cs(NB, b)[idx] = fin ? c : m + sx;
                L.sx(NB, b)[idx] = sx;
                L.oz(NB, b)[idx] = -8 * oz;
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
            int i1 = 0, i2 = ozb[h];  // the zero point -8 O starts the level-2 sum
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = vx_and(q[4 * h + i], 0x0F0F0F0Fu);
                const uint32_t hi = vx_and(q[4 * h + i] >> 4, 0x0F0F0F0Fu);
                i1 = __builtin_amdgcn_sdot4((int)lo, (int)x1[8 * h + i], i1, false);
                i1 = __builtin_amdgcn_sdot4((int)hi, (int)x1[8 * h + 4 + i], i1, false);
                i2 = __builtin_amdgcn_sdot4((int)lo, (int)x2[8 * h + i], i2, false);
                i2 = __builtin_amdgcn_sdot4((int)hi, (int)x2[8 * h + 4 + i], i2, false);
            }
            const int t = __mul24(i1, 254) + i2;
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
            const int t = __mul24(i1, 254) + i2;
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
        const float t0 = (float)(__mul24(a1, 254) + a2), t1 = (float)(__mul24(b1, 254) + b2);
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

// Batch 1: split float4 f of x (slot f & 15 of unit f >> 4) into the two
// int8 levels of vx_i8lds and store them; the 8 float4 of a 32-block are 8
// consecutive lanes, whose max and sums are reduced with DPP (every lane of
// the wave takes part; `in` selects the lanes that store). The block stores
// its scale c, sum(x) and -8 O, O = sum(254 x1 + x2) (|O| < 2^21: exact as a
// float sum).
__device__ __forceinline__ void vx_split_store_b1(const vx_i8lds& L, uint32_t f, f32x4 v, bool in) {
    const float m = vx_max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float c = m * (1.0f / (127.0f * 254.0f));
    const float inv1 = m > 0.f ? 127.0f / m : 0.f;  // 1 / (254 c)
    const float inv2 = inv1 * 254.0f;               // 1 / c
    const float s1 = 254.0f * c;
    int q1[4], q2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        q1[e] = (int)rintf(v[e] * inv1);
        const float r = __builtin_fmaf(-(float)q1[e], s1, v[e]);
        q2[e] = min(127, max(-127, (int)rintf(r * inv2)));
    }
    const float sx = vx_sum8((v.x + v.y) + (v.z + v.w));
    // a non-finite block (fmaxf skips NaN; the sum does not) stores
    // max + sum as its scale, so y is non-finite
    const bool fin = m < __builtin_inff() && sx == sx;
    const float oz = vx_sum8((float)(254 * (q1[0] + q1[1] + q1[2] + q1[3]) + (q2[0] + q2[1] + q2[2] + q2[3])));
    if (in) {
        const uint32_t ul = f >> 4, j = f & 15u;
        uint32_t* x8 = (uint32_t*)L.x8(0);
        x8[((0u * 4u + (j >> 2)) * L.upitch + ul) * 4u + (j & 3u)] = vx_pack4(q1[0], q1[1], q1[2], q1[3]);
        x8[((1u * 4u + (j >> 2)) * L.upitch + ul) * 4u + (j & 3u)] = vx_pack4(q2[0], q2[1], q2[2], q2[3]);
        if ((j & 7u) == 0u) {
            const uint32_t idx = 2u * ul + (j >> 3);
            L.cs(1, 0)[idx] = fin ? c : m + sx;
            L.sx(1, 0)[idx] = sx;
            L.oz(1, 0)[idx] = -8 * (int)oz;
        }
    }
}

// Unsigned maximum over each aligned group of 8 lanes (DPP). Used on the
// bits of |x|: for non-negative floats the integer order is the float order.
__device__ __forceinline__ uint32_t vx_umax8(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
}

// vx_split_store_b1 for N float4 per lane (f, f + stride, ...), the N
// dependency chains interleaved step by step so their DPP reductions and
// divisions overlap, and each level computed with one rounding
// (vx_xq_levels4: q1 = RNE(v inv1) and q2 = RNE(r inv2) from fmaf(., ., 1.5
// 2^23), the bytes gathered with v_perm_b32; 4 VALU per element instead of
// 9). The block maximum runs on the bits of |x| as unsigned: equal to
// fmaxf's for finite blocks; a NaN then wins (fmaxf would skip it), and such
// a block is non-finite either way (its sum is NaN). Scales as in
// vx_split_store_b1 (c = m / (127 254), inv1 = 127 / m); the clamps to +-127
// never act: |v inv1| <= 127 (1 + 2^-24), and with r = RN(v - q1 s1),
// |r inv2| <= 254 (0.5 + 508 2^-24)(1 + 3 2^-24) < 127.01. A block with m <
// 2^-100 (inv1 would overflow) or non-finite stores zero levels; a
// non-finite one stores a non-finite scale, so y is non-finite. Only the
// block sums the format's decode uses are formed: sum(x) for Q4_K's min
// term, O = sum(254 q1 + q2) for Q4_0's zero point (from the packed bytes,
// v_dot4 against 0x01010101), neither for Q8_0. The maximum on the bits
// sees a NaN (it orders above infinity), so m < inf alone tells a finite
// block.
template <int QT, int N>
__device__ __forceinline__ void vx_split_store_bn(const vx_i8lds& L, uint32_t f0, uint32_t stride, uint32_t total,
                                                  const f32x4 (&xv)[N]) {
    constexpr bool SX = QT == VX_Q4_K, OZ = QT == VX_Q4_0;
    float m[N], c[N], inv1[N], inv2[N], s1[N], sx[N], oz[N];
    bool fin[N];
    uint32_t w1[N], w2[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const f32x4 v = xv[i];
        const uint32_t mb = max(max(__float_as_uint(fabsf(v.x)), __float_as_uint(fabsf(v.y))),
                                max(__float_as_uint(fabsf(v.z)), __float_as_uint(fabsf(v.w))));
        m[i] = __uint_as_float(vx_umax8(mb));
        if (SX) sx[i] = (v.x + v.y) + (v.z + v.w);
    }
    if (SX) {
#pragma unroll
        for (int i = 0; i < N; ++i) sx[i] = vx_sum8(sx[i]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        fin[i] = m[i] < __builtin_inff();
        c[i] = m[i] * (1.0f / (127.0f * 254.0f));
        inv1[i] = (fin[i] && m[i] >= 0x1p-100f) ? 127.0f / m[i] : 0.f;
        inv2[i] = inv1[i] * 254.0f;
        s1[i] = 254.0f * c[i];
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        vx_xq_levels4(xv[i], s1[i], inv1[i], inv2[i], fin[i], w1[i], w2[i]);
        if (OZ) {
            const int o = 254 * __builtin_amdgcn_sdot4((int)w1[i], 0x01010101, 0, false) +
                          __builtin_amdgcn_sdot4((int)w2[i], 0x01010101, 0, false);
            oz[i] = (float)o;
        }
    }
    if (OZ) {
#pragma unroll
        for (int i = 0; i < N; ++i) oz[i] = vx_sum8(oz[i]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint32_t f = f0 + stride * (uint32_t)i;
        if (f < total) {
            const uint32_t ul = f >> 4, j = f & 15u;
            uint32_t* x8 = (uint32_t*)L.x8(0);
            x8[((0u * 4u + (j >> 2)) * L.upitch + ul) * 4u + (j & 3u)] = w1[i];
            x8[((1u * 4u + (j >> 2)) * L.upitch + ul) * 4u + (j & 3u)] = w2[i];
            if ((j & 7u) == 0u) {
                const uint32_t idx = 2u * ul + (j >> 3);
                L.cs(1, 0)[idx] = fin[i] ? c[i] : m[i];
                if (SX) L.sx(1, 0)[idx] = sx[i];
                if (OZ) L.oz(1, 0)[idx] = -8 * (int)oz[i];
            }
        }
    }
}

// Batch 1, persistent, on the integer-dot path: the work split, issue order
// and ring of vx_gemv_p1, with x staged in LDS as two int8 levels per
// 32-block (the vx_i8lds layout; x ~= c (254 x1 + x2), error <= c / 2 ~
// 1.6e-5 of the block's max|x|). A unit then reduces in exact int32 with
// v_dot4_i32_i8 (vx_unit_dot_i8): on gfx950 one v_dot4 (4 products) issues
// in about the time of two v_fma_f32, and no weight is converted to float
// (v_cvt_pk_f32_fp8 costs about three times a v_fma_f32), so a unit takes
// about half the VALU time of vx_unit_dot_b1. Each 8 consecutive lanes
// stage one 32-block; its max and sums are reduced with DPP.
// EW (one item per wave): no bare barrier after the x loads, so every wave
// requests its one item as soon as it starts (Q8_0 4096^2 5.37 -> 5.15 us);
// with more items per wave the x must come first (Q4_0 11008 x 4096 6.38
// against 6.54 us without the barrier).
template <int QT, int P, int WGT, bool XV, bool XM = false, bool FS = false, bool EW = false>
__device__ __forceinline__ void vx_gemv_p1i(const vx_gemv_args& a, uint32_t G) {
    constexpr int NW = vx_unit<QT>::NW;
    constexpr uint32_t XW = WGT < 512 ? WGT : 512u;
    constexpr int XPT = (int)(VX_P_XF / XW);
    static_assert(!FS || XPT % 2 == 0, "the paired split takes whole pairs of rounds");
    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nwv = G * (WGT / 64u);
    // XM: workgroups are dealt to the 8 XCDs in turn (workgroup b runs on
    // XCD b % 8), so position pb = (b % 8) G / 8 + b / 8 gives each XCD a
    // contiguous range of positions; with wave-major rows (below) each XCD
    // then streams runs of G / 8 adjacent rows. Identity when G % 8 != 0.
    const uint32_t pb = (XM && (G & 7u) == 0u) ? (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const uint32_t gw = wave * G + pb;  // wave-major, as vx_gemv_p1
    const uint32_t nunits = a.nunits, npass = (nunits + 63u) >> 6;
    const uint32_t nrows = a.M > gw ? (a.M - gw + nwv - 1u) / nwv : 0u;
    const uint32_t nitems = nrows * npass;
    const vx_i8lds L{a.upitch, nunits};

    // 1. x loads (float4 f = slot f & 15 of unit f >> 4), then the bare
    //    barrier that puts them ahead of every weight request of the CU.
    //    Only the first XW threads load and split x (two float4 each at
    //    K = 4096): the requests leave as soon as the first waves of the CU
    //    start, and the later waves only meet the barriers (1-6 % faster
    //    than all 16 waves loading; 4 waves loading is slower).
    const uint32_t total = nunits * 16u;
    f32x4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        // uniform: rounds past x (FS: whole pairs of rounds, the second
        // one's lanes past x re-reading the last float4)
        if ((uint32_t)(FS ? i & ~1 : i) * XW >= total || wave >= XW / 64u) break;
        const uint32_t f = min(t + XW * (uint32_t)i, total - 1u);
        if constexpr (XV) {
            xr[i] = *(const f32x4*)(a.x + 4 * (int64_t)f);
        } else {
            const float* xp = a.x + 4 * (int64_t)f * a.xs_k;
            xr[i] = f32x4{xp[0], xp[a.xs_k], xp[2 * a.xs_k], xp[3 * a.xs_k]};
        }
    }
    asm volatile("" ::: "memory");
    if constexpr (!EW) __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // 2. the first ring items (see vx_gemv_p1 for the clamping).
    const uint8_t* wbase = a.w;
    auto item_ptr = [&](uint32_t it, uint32_t& unit) {
        const uint32_t c = nitems ? min(it, nitems - 1u) : 0u;
        const uint32_t ri = c / npass, p = c - ri * npass;
        const uint32_t row = min(gw + ri * nwv, a.M - 1u);
        unit = it < nitems ? min(64u * p + lane, nunits - 1u) : 0u;
        return wbase + (uint64_t)row * a.row_stride;
    };
    constexpr int PRE = P <= 2 ? P : 1;
    uint32_t wr[P][NW];
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        uint32_t u;
        const uint8_t* rp = item_ptr((uint32_t)j, u);
        vx_load_unit<QT, true>(rp, u, wr[j]);
    }

    // 3. split x into the two levels and store them (vx_split_store_b1;
    //    FS: two rounds at a time, interleaved, vx_split_store_bn).
    if constexpr (FS) {
#pragma unroll
        for (int i = 0; i < XPT; i += 2) {
            if ((uint32_t)i * XW >= total || wave >= XW / 64u) break;
            const f32x4 pr[2] = {xr[i], xr[i + 1]};
            vx_split_store_bn<QT, 2>(L, t + XW * (uint32_t)i, XW, total, pr);
        }
    } else {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
            if ((uint32_t)i * XW >= total || wave >= XW / 64u) break;
            const uint32_t f = t + XW * (uint32_t)i;
            const bool in = f < total;
            vx_split_store_b1(L, f, in ? xr[i] : f32x4{0.f, 0.f, 0.f, 0.f}, in);
        }
    }
    __syncthreads();

    // 4. the rest of the ring, then stream the items (whole rounds of P in
    //    the main loop: exact wait counts; the last partial round follows).
#pragma unroll
    for (int j = PRE; j < P; ++j) {
        uint32_t u;
        const uint8_t* rp = item_ptr((uint32_t)j, u);
        vx_load_unit<QT, true>(rp, u, wr[j]);
    }
    uint32_t x1[16], x2[16];
    float cb[2], sxb[2];
    int ozb[2];
    uint32_t cur = ~0u;
    float acc = 0.f;
    auto body = [&](uint32_t it, uint32_t (&w)[NW]) {
        const uint32_t ri = it / npass, p = it - ri * npass;
        const uint32_t u = 64u * p + lane;
        const bool act = u < nunits;
        const uint32_t us = act ? u : nunits - 1u;
        if (p != cur) {
            cur = p;
            uint32_t ul = us;  // defined in the branch: its LDS addressing stays here
            asm volatile("" : "+v"(ul));
            vx_read_x8(L, 0, ul, x1, x2);
            const float2 cb2 = *(const float2*)&L.cs(1, 0)[2u * ul];
            const float2 sx2 = *(const float2*)&L.sx(1, 0)[2u * ul];
            const int2 oz2 = *(const int2*)&L.oz(1, 0)[2u * ul];
            cb[0] = cb2.x; cb[1] = cb2.y; sxb[0] = sx2.x; sxb[1] = sx2.y; ozb[0] = oz2.x; ozb[1] = oz2.y;
        }
        const float d = vx_unit_dot_i8<QT>(w, x1, x2, cb, sxb, ozb, us);
        acc += act ? d : 0.f;
        uint32_t nu;
        const uint8_t* rp = item_ptr(it + P, nu);
        vx_load_unit<QT, true>(rp, nu, w);
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

// Read probe (measurement only): the loads of vx_gemv_p1i with nothing
// else. Same grid, per-XCD wave-major row numbering and per-lane units; no
// x, no barrier, no arithmetic; every item of a round of P in flight before
// any is used (an empty asm statement consumes each loaded word, so the
// loads stay and their waits are real), nothing loaded past the wave's last
// item. Lane 0 writes its XOR of the row's words to y: the bytes of the
// GEMV without x. Its time is the ceiling of what the GEMV's access pattern
// can stream in one launch. P = 1, the GEMV's ring for one-pass rows, is
// also the fastest depth for the bare loads (Q4_0 11008 x 4096: 6.03 us
// against 6.13 with two items and 6.34 with four).
template <int QT, int P>
__device__ __forceinline__ void vx_read_probe(const vx_gemv_args& a, uint32_t G) {
    constexpr int NW = vx_unit<QT>::NW;
    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nwv = G * 16u;
    const uint32_t pb = (G & 7u) == 0u ? (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const uint32_t gw = wave * G + pb;
    const uint32_t nunits = a.nunits, npass = (nunits + 63u) >> 6;
    const uint32_t nrows = a.M > gw ? (a.M - gw + nwv - 1u) / nwv : 0u;
    const uint32_t nitems = nrows * npass;
    uint32_t acc = 0u;
    for (uint32_t it0 = 0; it0 < nitems; it0 += P) {
        uint32_t wr[P][NW];
#pragma unroll
        for (int j = 0; j < P; ++j) {
            // nothing is loaded past the wave's last item (wave-uniform)
            const uint32_t it = it0 + (uint32_t)j;
            if (it < nitems) {
                const uint32_t ri = it / npass, p = it - ri * npass;
                vx_load_unit<QT, true>(a.w + (uint64_t)(gw + ri * nwv) * a.row_stride, min(64u * p + lane, nunits - 1u),
                                       wr[j]);
            } else {
#pragma unroll
                for (int q = 0; q < NW; ++q) wr[j][q] = 0u;
            }
        }
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const uint32_t it = it0 + (uint32_t)j;
#pragma unroll
            for (int q = 0; q < NW; ++q) {
                asm volatile("" ::"v"(wr[j][q]));
                acc ^= wr[j][q];
            }
            if (it < nitems) {
                const uint32_t ri = it / npass, p = it - ri * npass;
                if (p == npass - 1u) {
                    if (lane == 0) a.y[(int64_t)(gw + ri * nwv) * a.ys_m] = __uint_as_float(acc & 0x007FFFFFu);
                    acc = 0u;
                }
            }
        }
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

typedef int i32x4 __attribute__((ext_vector_type(4)));

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

// Arguments of the persistent batch-1 kernels (and of the read probe and the
// launch floor, which mirror them). What a wave needs before its first x and
// weight requests (W, x, the row stride, M, the units per row, the grid size
// and the x layout flag) comes first as plain scalars, which the compiler
// preloads into SGPRs (built with -amdgpu-kernarg-preload-count): the
// dispatcher writes them with the wave, so no wave waits for a
// kernel-argument fetch (about 0.3 us, serialized before its first request)
// before it starts streaming. The rest stays in the vx_gemv_args struct,
// fetched in the background. The grid size comes in as an argument because
// gridDim is a hidden argument, not preloaded. Same box, graph-replayed:
// Q4_0 11008x4096 6.35 -> 5.96 us, Q8_0 4096^2 (_p1e) 5.15 -> 4.88 us,
// Q4_0 4096x11008 (ring of two) 7.01 -> 6.80 us, Q4_K 14336x4096 7.59 ->
// 7.28 us, outputs identical. Argument structs themselves cannot be
// preloaded.
#define VX_B1_PARAMS                                                                                   \
    const uint8_t *pre_w, const float *pre_x, uint64_t pre_rs, uint32_t pre_M, uint32_t pre_nu, uint32_t pre_G, \
        uint32_t pre_xv, vx_gemv_args pre_a
#define VX_B1_ARGS pre_w, pre_x, pre_rs, pre_M, pre_nu, pre_xv, pre_a
__device__ __forceinline__ vx_gemv_args vx_b1_args(const uint8_t* w, const float* x, uint64_t rs, uint32_t M,
                                                   uint32_t nu, uint32_t xv, const vx_gemv_args& a) {
    vx_gemv_args r = a;
    r.w = w;
    r.x = x;
    r.row_stride = rs;
    r.M = M;
    r.nunits = nu;
    r.x_vec = xv;
    return r;
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
// Persistent batch-1 kernels: rows per XCD in contiguous runs (XM), and
// for the integer-dot path the paired split (FS). Same-box A/B, graph-
// replayed (Q4_0 11008x4096 / Q8_0 4096^2 / Q4_0 4096x11008 / Q4_K
// 14336x4096 / Q4_K 32000x4096, us): int8 x, ring 2 without either 6.96 /
// 5.33 / 8.04 / 8.22 / 15.23, ring 1 with both 6.46 / 5.31 / 8.18 / 7.66 /
// 14.69, ring 2 with both 6.90 / 5.50 / 7.82 / 8.27 / 14.99; f32 x, ring 2
// 7.72 / 6.61 / 8.71 / 9.92 / 18.49, ring 1 with XM 6.57 / 5.47 / 7.96 /
// 8.34 / 15.85. Outputs identical bit for bit across all of them.
// One kernel per x layout (contiguous x: the default; _xs: strided x): with
// both bodies in one kernel behind a run-time flag the contiguous path ran
// slower (same box, graph-replayed: Q4_0 11008x4096 6.18 against 6.06 us,
// 4096x11008 ring of two 7.03 against 6.72 us).
#define VX_GEMV_P1(QT, QN, P, WGT)                                                              \
    extern "C" __global__ __launch_bounds__(WGT) void vx_gemv_p1_##QN##_w##WGT(VX_B1_PARAMS) {     \
        vx_gemv_p1<QT, P, WGT, true, true>(vx_b1_args(VX_B1_ARGS), pre_G);                          \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(WGT) void vx_gemv_p1_##QN##_w##WGT##_xs(VX_B1_PARAMS) { \
        vx_gemv_p1<QT, P, WGT, false, true>(vx_b1_args(VX_B1_ARGS), pre_G);                         \
    }
#define VX_GEMV_P1I(QT, QN, P)                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void vx_gemv_p1i_##QN##_p##P(VX_B1_PARAMS) {     \
        vx_gemv_p1i<QT, P, 1024, true, true, true>(vx_b1_args(VX_B1_ARGS), pre_G);                \
    }                                                                                             \
    extern "C" __global__ __launch_bounds__(1024) void vx_gemv_p1i_##QN##_p##P##_xs(VX_B1_PARAMS) { \
        vx_gemv_p1i<QT, P, 1024, false, true, true>(vx_b1_args(VX_B1_ARGS), pre_G);              \
    }
// _p1e: one item per wave (every row one pass, at most one row per wave)
#define VX_GEMV_P1IE(QT, QN)                                                                    \
    extern "C" __global__ __launch_bounds__(1024) void vx_gemv_p1i_##QN##_p1e(VX_B1_PARAMS) {      \
        vx_gemv_p1i<QT, 1, 1024, true, true, true, true>(vx_b1_args(VX_B1_ARGS), pre_G);          \
    }                                                                                             \
    extern "C" __global__ __launch_bounds__(1024) void vx_gemv_p1i_##QN##_p1e_xs(VX_B1_PARAMS) {   \
        vx_gemv_p1i<QT, 1, 1024, false, true, true, true>(vx_b1_args(VX_B1_ARGS), pre_G);        \
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
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_generic_##QN(vx_gemv_args a) {     \
        vx_args_fetch(a);                                                                           \
        vx_gemv_generic<QT>(a);                                                                     \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(VX_WG) void vx_dequant_##QN(vx_gemv_args a) {          \
        vx_args_fetch(a);                                                                           \
        vx_dequant<QT>(a);                                                                          \
    }

VX_GEMV_ALL(VX_Q4_0, q4_0)
VX_GEMV_ALL(VX_Q8_0, q8_0)
VX_GEMV_ALL(VX_Q4_K, q4_k)
VX_GEMV_P1(VX_Q4_0, q4_0, 1, 1024)
VX_GEMV_P1(VX_Q8_0, q8_0, 1, 1024)
VX_GEMV_P1(VX_Q4_K, q4_k, 1, 1024)
VX_GEMV_P1I(VX_Q4_0, q4_0, 1)
VX_GEMV_P1I(VX_Q4_0, q4_0, 2)
VX_GEMV_P1I(VX_Q8_0, q8_0, 1)
VX_GEMV_P1I(VX_Q8_0, q8_0, 2)
VX_GEMV_P1I(VX_Q4_K, q4_k, 1)
VX_GEMV_P1I(VX_Q4_K, q4_k, 2)
VX_GEMV_P1IE(VX_Q4_0, q4_0)
VX_GEMV_P1IE(VX_Q8_0, q8_0)
VX_GEMV_P1IE(VX_Q4_K, q4_k)
#define VX_READ_PROBE(QT, QN)                                                                     \
    extern "C" __global__ __launch_bounds__(1024) void vx_read_probe_##QN(VX_B1_PARAMS) {         \
        vx_read_probe<QT, 1>(vx_b1_args(VX_B1_ARGS), pre_G);                                      \
    }
// Launch floor (measurement only): no work, the batch-1 GEMV's grid and
// preloaded arguments. In a replayed HIP graph its time per launch is the
// fixed cost every kernel of a step pays (dispatch with its argument
// preload, wave launch, completion) before any byte moves.
extern "C" __global__ __launch_bounds__(1024) void vx_launch_floor_k(VX_B1_PARAMS) {
    if (pre_M == 0xFFFFFFFFu && threadIdx.x == 0) pre_a.y[blockIdx.x] = 0.f;  // never true: keeps the argument
}
VX_READ_PROBE(VX_Q4_0, q4_0)
VX_READ_PROBE(VX_Q8_0, q8_0)
VX_READ_PROBE(VX_Q4_K, q4_k)

// ------------------------------------------------------------------------
// Batched GEMV on split activations (vx_xq, written once per call by
// vx_quantize_x: two int8 levels and {c2, S} per 32-block and column, the
// levels in the order of a Q4_0 block's nibbles) on the int8 matrix cores,
// one v_mfma_i32_16x16x32_i8 per 32-block and group of 8 columns:
//   A (16 x 32): row i = 2 c + L is level L of column 8 h + c; lane (i, g)
//     holds bytes 8g..8g+7 of that block's level array;
//   B (32 x 16): column n is W row n of the 16-row tile; lane (n, g) holds
//     the 8 weights those bytes pair with: the low then the high nibbles of
//     qs dword g (Q4_0), qs dwords g and 4 + g (Q8_0), the low or high
//     nibbles of qs-chunk dwords g and 4 + g (Q4_K sub-block 2c or 2c + 1);
//   D (16 x 16): lane (n, g) receives rows 4g..4g+3, columns 8h + 2g and
//     8h + 2g + 1 with both levels, of W row n, T = 254 D_L0 + D_L1 (exact
//     int32, |D| < 2^20), and applies the block's scales in f32:
//       Q4_0  acc += d (c2 T - 8 S)       (nibbles used unbiased)
//       Q8_0  acc += d (c2 T)
//       Q4_K  acc += d (sum over the item's sub-blocks of sc (c2 T))
//                  - dmin (sum of m S)   (one super-block per item)
// Work split: one workgroup of 16 waves per CU (grid = CU count); CU c owns
// rows [c M / G, (c + 1) M / G) in 16-row tiles, the last one possibly
// partial (its spare lanes repeat the range's last row, which costs no HBM
// bytes), so every CU streams the same bytes to within one row; with two
// column groups, where the arithmetic bounds the kernel, CU c owns the whole
// tiles c, c + G, ... instead (no partial tile's arithmetic on every CU);
// wave w owns the K slice s = (w + c) mod 16:
// items (256 weights) s, s + 16, ... up to XI per pass. The rotation by c
// keeps the waves of the chip from reading the same slice of x at the same
// time. A wave loads its slice's x levels into registers once per pass and
// reuses them for every tile; per tile it streams 16 rows x 256 weights per
// item, lane (n, u) loading quarter u of row n's item (a unit of 64 weights,
// or the Q4_K super-block's header and qs chunk u) with 16-byte loads, and
// 4 x 4 transposes across the four 16-lane rows (v_permlane32_swap +
// v_permlane16_swap) turn quarters into the per-block MFMA layout. Weight
// items flow through a ring of R = XI * TU register slots (TU = 2 tiles when
// XI = 1). At the end of each tile the 16 waves' partial sums meet in LDS and
// one thread per output adds them in slice order (deterministic), adding to
// its own y of the previous passes when K takes several passes.

// v_permlane{16,32}_swap results pass through empty asm: see vx_pin2.
__device__ __forceinline__ void vx_swap32(uint32_t& x, uint32_t& y) {
    vx_pin2(x, y);
    const auto s = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    x = s[0];
    y = s[1];
    vx_pin2(x, y);
}
__device__ __forceinline__ void vx_swap16(uint32_t& x, uint32_t& y) {
    vx_pin2(x, y);
    const auto s = __builtin_amdgcn_permlane16_swap(x, y, false, false);
    x = s[0];
    y = s[1];
    vx_pin2(x, y);
}

// 4 x 4 transpose across the 16-lane rows: on entry row u of r[k] holds
// A[u][k]; on exit row g of r[k] holds A[k][g]. permlane32_swap(x, y)
// exchanges rows 2, 3 of x with rows 0, 1 of y; permlane16_swap(x, y) rows
// 1, 3 of x with rows 0, 2 of y.
__device__ __forceinline__ void vx_t4(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    vx_swap32(r0, r2);  // r0 = [A00 A10 A02 A12], r2 = [A20 A30 A22 A32]
    vx_swap32(r1, r3);  // r1 = [A01 A11 A03 A13], r3 = [A21 A31 A23 A33]
    vx_swap16(r0, r1);  // r0 = [A00 A01 A02 A03], r1 = [A10 A11 A12 A13]
    vx_swap16(r2, r3);  // r2 = [A20 A21 A22 A23], r3 = [A30 A31 A32 A33]
}

// Every row's value of v in every lane: o[u] = v of 16-lane row u.
__device__ __forceinline__ void vx_gather4(uint32_t v, uint32_t (&o)[4]) {
    uint32_t a = v, b = v;
    vx_swap32(a, b);  // a = [v0 v1 v0 v1], b = [v2 v3 v2 v3]
    uint32_t a2 = a, b2 = b;
    vx_swap16(a, a2);  // a = [v0 v0 v0 v0], a2 = [v1 v1 v1 v1]
    vx_swap16(b, b2);  // b = [v2 v2 v2 v2], b2 = [v3 v3 v3 v3]
    o[0] = a;
    o[1] = a2;
    o[2] = b;
    o[3] = b2;
}

// The weights of one item (8 blocks / sub-blocks of 32) in MFMA layout.
template <int QT>
struct vx_xq_item {
    uint32_t lo[8], hi[8];  // B operand of block b: lo[b] | hi[b] << 32 (int8 lanes)
    float ds[8];            // d of block b, this lane's row (Q4_0, Q8_0)
    uint32_t scm[4];        // Q4_K: sub-blocks 2k, 2k + 1: bytes sc, m, sc, m (6-bit)
    float d, dmin;          // Q4_K super-block scales
};

template <int QT>
__device__ __forceinline__ void vx_xq_prepare(uint32_t (&r)[vx_unit<QT>::NW], uint32_t u, vx_xq_item<QT>& it) {
    constexpr uint32_t NIB = 0x0F0F0F0Fu;
    if constexpr (QT == VX_Q4_0) {
        // unit u = blocks 2u (d in bytes 0-1, qs 2..17) and 2u + 1 (d 18-19, qs 20..35)
        uint32_t e0 = __builtin_amdgcn_alignbit(r[1], r[0], 16), e1 = __builtin_amdgcn_alignbit(r[2], r[1], 16);
        uint32_t e2 = __builtin_amdgcn_alignbit(r[3], r[2], 16), e3 = __builtin_amdgcn_alignbit(r[4], r[3], 16);
        uint32_t o0 = r[5], o1 = r[6], o2 = r[7], o3 = r[8];
        vx_t4(e0, e1, e2, e3);  // e_k: qs dword g of block 2k
        vx_t4(o0, o1, o2, o3);  // o_k: qs dword g of block 2k + 1
        const uint32_t q[8] = {e0, o0, e1, o1, e2, o2, e3, o3};
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            it.lo[b] = vx_and(q[b], NIB);
            it.hi[b] = vx_and(q[b] >> 4, NIB);
        }
        uint32_t dd[4];
        vx_gather4((r[0] & 0xFFFFu) | (r[4] & 0xFFFF0000u), dd);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            it.ds[2 * k] = vx_f16_to_f32(dd[k]);
            it.ds[2 * k + 1] = vx_f16_to_f32(dd[k] >> 16);
        }
    } else if constexpr (QT == VX_Q8_0) {
        // unit u = blocks 2u (d 0-1, qs 2..33) and 2u + 1 (d 34-35, qs 36..67)
        uint32_t a[8], b[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            a[k] = __builtin_amdgcn_alignbit(r[k + 1], r[k], 16);
            b[k] = r[9 + k];
        }
        vx_t4(a[0], a[1], a[2], a[3]);  // a[k]: dword g of block 2k
        vx_t4(a[4], a[5], a[6], a[7]);  // a[4 + k]: dword 4 + g of block 2k
        vx_t4(b[0], b[1], b[2], b[3]);
        vx_t4(b[4], b[5], b[6], b[7]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            it.lo[2 * k] = a[k];
            it.hi[2 * k] = a[4 + k];
            it.lo[2 * k + 1] = b[k];
            it.hi[2 * k + 1] = b[4 + k];
        }
        uint32_t dd[4];
        vx_gather4((r[0] & 0xFFFFu) | (r[8] & 0xFFFF0000u), dd);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            it.ds[2 * k] = vx_f16_to_f32(dd[k]);
            it.ds[2 * k + 1] = vx_f16_to_f32(dd[k] >> 16);
        }
    } else {
        // header r[0..3] (d, dmin, 12 scale bytes), qs chunk u in r[4..11]:
        // sub-blocks 2u (low nibbles) and 2u + 1 (high nibbles)
        uint32_t c0 = r[4], c1 = r[5], c2 = r[6], c3 = r[7];
        uint32_t c4 = r[8], c5 = r[9], c6 = r[10], c7 = r[11];
        vx_t4(c0, c1, c2, c3);  // c_k: chunk k dword g
        vx_t4(c4, c5, c6, c7);  // c_{4+k}: chunk k dword 4 + g
        const uint32_t lo4[4] = {c0, c1, c2, c3}, hi4[4] = {c4, c5, c6, c7};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            it.lo[2 * k] = vx_and(lo4[k], NIB);
            it.hi[2 * k] = vx_and(hi4[k], NIB);
            it.lo[2 * k + 1] = vx_and(lo4[k] >> 4, NIB);
            it.hi[2 * k + 1] = vx_and(hi4[k] >> 4, NIB);
        }
        it.d = vx_f16_to_f32(r[0]);
        it.dmin = vx_f16_to_f32(r[0] >> 16);
        // this lane's two sub-blocks' 6-bit (scale, min), packed, then every
        // chunk's from its row
        uint32_t sc0, m0, sc1, m1;
        vx_q4k_scales(r[1], r[2], r[3], u, sc0, m0, sc1, m1);
        vx_gather4(sc0 | (m0 << 8) | (sc1 << 16) | (m1 << 24), it.scm);
    }
}

#define VX_XQ_WG 1024
typedef long i64x2 __attribute__((ext_vector_type(2)));

// Scratch of vx_gemv_q_noalloc (no counterpart in the reference): the
// activation split of x for callers that cannot allocate device memory.
// One copy per loaded module, i.e. per context; vx_init resolves its device
// address once (hipModuleGetGlobal, with the context's device current) and
// the host passes that address to vx_quantize_x / vx_gemv_xq like any other
// buffer. Calls on one context share it, so calls that overlap in time race.
extern "C" {
__device__ __align__(256) uint8_t vx_scratch[VX_SCRATCH_BYTES];
}

// LDS of vx_gemv_xq: per wave, the scales of its K slice in the current
// pass [8 XI blocks][CP columns] float2 {c2, S'} (S' = -8 S for Q4_0); then
// red[RMAX tiles][16 slots][CP][16 rows] partial sums.
// Schedule (measured with per-wave s_memrealtime stamps): the chip's weight
// requests go out together, so their data returns in no useful order; a
// barrier per tile then waits for the last wave's item, by which time most of
// the matrix has arrived, and the compute runs after the stream instead of
// under it. So nothing here waits for other waves while streaming:
//  1. each wave issues the loads of its slice's x levels (registers) and
//     scales; one bare barrier (no wait) puts every x request of the CU
//     ahead of its weight requests, as an x request behind the chip's
//     weight requests returns late;
//  2. then its ring of weight items, and only then the wait for its own x
//     (the scales go to its own LDS region); each item is reduced as it
//     arrives and its partial sums parked in red[tile-work mod RMAX];
//  3. every RMAX tile-works (for the usual shapes once, at the end) the
//     workgroup meets, one thread per output adds the 16 slots in slice
//     order (deterministic) and writes y.
// Wait counts: inside the streaming loop the only memory loads are the ring
// refills, issued unconditionally (clamped inside the matrix past the last
// tile-work) in whole rounds of RD, so each wait covers just its slot. MP
// (several passes, K past 16 XI items) adds loads of the next pass's x and of
// y, which makes those waits conservative; it is compiled separately.
#define VX_XQ_RED_BYTES 65536u
// Per wave, after the scales: the fused split's tables ([64] {m, S}, then
// [64] {c1, i1, i2, fin}), 1536 bytes.
#define VX_XQ_FX_FLOAT2 192u
template <int QT, int NCG, int XI, int RD, bool MP, bool ST, bool FX, bool FH, bool XM = false>
__device__ __forceinline__ void vx_gemv_xq(const vx_gemv_xq_args& a) {
    constexpr int NW = vx_unit<QT>::NW;
    constexpr uint32_t CP = 8u * NCG;             // columns per launch (padded)
    constexpr uint32_t PI = 16u * XI;             // items per pass
    constexpr uint32_t NSW = 8u * XI * CP;        // scale entries per wave and pass
    constexpr int SPL = (int)((NSW + 63u) / 64u);  // ... per lane
    constexpr uint32_t TILE_F = 16u * CP * 16u;   // red floats per tile-work
    constexpr uint32_t RMAX = VX_XQ_RED_BYTES / (TILE_F * 4u);
    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t G = gridDim.x;
    // XM: positions per XCD as in vx_gemv_p1i (workgroup b runs on XCD b % 8)
    const uint32_t cu = (XM && (G & 7u) == 0u) ? (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    // this CU's tile-work ts covers rows rb + ts rs .. + 15, below rlim:
    // rows [r0, r1), M split into G ranges that differ by at most one row,
    // in 16-row tiles (the last one possibly partial), or with two column
    // groups (WHOLE) the whole tiles cu, cu + G, ...: where the arithmetic,
    // not the stream, bounds the kernel, that computes fewer row slots
    constexpr bool WHOLE = NCG == 2;
    uint32_t rb, rs, rlim, nts;
    if constexpr (WHOLE) {
        const uint32_t ntiles = (a.M + 15u) >> 4;
        rb = 16u * cu;
        rs = 16u * G;
        rlim = a.M;
        nts = ntiles > cu ? (ntiles - cu + G - 1u) / G : 0u;
    } else {
        const uint32_t r0 = (uint32_t)((uint64_t)cu * a.M / G), r1 = (uint32_t)((uint64_t)(cu + 1u) * a.M / G);
        rb = r0;
        rs = 16u;
        rlim = r1;
        nts = (r1 - r0 + 15u) >> 4;
    }
    if (nts == 0u) return;  // uniform over the workgroup
    const uint32_t slot = (wave + cu) & 15u;
    const uint32_t B = a.B, nblk = a.nblk, ipr = a.ipr;
    const uint32_t nwork = (MP ? a.npass : 1u) * nts;  // tile-works over all passes

    float* red = (float*)vx_lds_x;                               // [RMAX][16][CP][16]
    float2* scl = (float2*)(red + RMAX * TILE_F) + wave * NSW;   // this wave's [8 XI][CP]
    float2* fxt = (float2*)(red + RMAX * TILE_F) + 16u * NSW + wave * VX_XQ_FX_FLOAT2;  // FX: {m, S}
    float4* fxp = (float4*)(fxt + 64);                                                  // FX: {c1, i1, i2, fin}

    auto row_of = [&](uint32_t ts) { return min(rb + ts * rs + n, rlim - 1u); };
    // W loads of tile-work w, item j of this wave (clamped inside the
    // matrix). Past the wave's last tile-work every lane loads the first unit
    // of the matrix: one cache line, where repeating the last item would add
    // a whole item of L2 reads per ring slot (the loads stay, so the waits
    // stay exact).
    auto wload = [&](uint32_t w, int j, uint32_t (&r)[NW]) {
        const bool past = w >= nwork;  // wave-uniform
        w = min(w, nwork - 1u);
        const uint32_t p = MP ? w / nts : 0u, ts = MP ? w - p * nts : w;
        const uint32_t item = min(p * PI + (uint32_t)XI * slot + (uint32_t)j, ipr - 1u);
        const uint8_t* rp = past ? a.w : a.w + (uint64_t)row_of(ts) * a.row_stride;
        vx_load_unit<QT, true>(rp, past ? 0u : min(4u * item + g, a.nunits - 1u), r);
    };
    // this wave's x levels and scales of pass p, from clamped addresses.
    // Nothing here uses the loaded values (lanes of columns >= B or of blocks
    // past K feed only D rows / MFMAs that are never used; the scales are
    // masked when they go to LDS), so no wait is forced before the caller's.
    float2 sv[SPL];
    long xa[XI][8][NCG];
    auto pass_loads = [&](uint32_t p) {
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            // entry e = (j, b, col): block 8 (p PI + XI slot + j) + b
            const uint32_t e = lane + 64u * (uint32_t)i;
            const uint32_t jb = e / CP, col = e - jb * CP;
            const uint32_t blk = 8u * (p * PI + (uint32_t)XI * slot + (jb >> 3)) + (jb & 7u);
            sv[i] = *(const float2*)(a.scales + 2u * ((uint64_t)min(blk, nblk - 1u) * a.xcols + a.col0 +
                                                      min(col, B - 1u)));
        }
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const uint32_t item = p * PI + (uint32_t)XI * slot + (uint32_t)j;
#pragma unroll
            for (int h = 0; h < NCG; ++h) {
                // lane (i, g): level i % 2 of column 8 h + i / 2, the 8 bytes
                // of position group g of each of the item's 8 blocks, 16
                // bytes (blocks 2k, 2k + 1) per load k; the lanes of one load
                // read consecutive 16-byte pieces (vx_quantize_x's layout)
                const uint32_t col = 8u * (uint32_t)h + (n >> 1);
                const uint8_t* lp = (const uint8_t*)a.levels + (uint64_t)min(item, ipr - 1u) * a.xcols * 512u +
                                    (uint64_t)(g * a.xcols + a.col0 + min(col, B - 1u)) * 32u + (n & 1u) * 16u;
                const uint32_t ks = a.xcols * 128u;  // bytes from one block pair to the next
                const i64x2 v0 = *(const i64x2*)lp, v1 = *(const i64x2*)(lp + ks);
                const i64x2 v2 = *(const i64x2*)(lp + 2u * ks), v3 = *(const i64x2*)(lp + 3u * ks);
                xa[j][0][h] = v0.x; xa[j][1][h] = v0.y; xa[j][2][h] = v1.x; xa[j][3][h] = v1.y;
                xa[j][4][h] = v2.x; xa[j][5][h] = v2.y; xa[j][6][h] = v3.x; xa[j][7][h] = v3.y;
            }
        }
    };
    // the scales to this wave's LDS region (read back by the same wave only)
    auto pass_publish = [&](uint32_t p) {
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const uint32_t e = lane + 64u * (uint32_t)i;
            const uint32_t jb = e / CP, col = e - jb * CP;
            const uint32_t blk = 8u * (p * PI + (uint32_t)XI * slot + (jb >> 3)) + (jb & 7u);
            float2 v = (blk < nblk && col < B) ? sv[i] : float2{0.f, 0.f};
            if constexpr (QT == VX_Q4_0) v.y *= -8.f;
            if (e < NSW) scl[e] = v;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): LDS stores done (vmcnt, expcnt untouched)
        __builtin_amdgcn_wave_barrier();
    };

    // FX: split this wave's slice of x itself (the bytes vx_quantize_x
    // writes, from the same arithmetic, vx_xq.hpp), one (item, column group)
    // at a time. Lane (i, g) holds column 8 h + i / 2 and level L = i % 2 of
    // the MFMA's A operand: positions 8g..8g+7 of each block, i.e. elements
    // 4g..4g+3 and 16+4g..16+4g+3. It loads elements 16 L + 4g..+3 (the two
    // lanes of a column share the loads), so the 32 values of a (block,
    // column) sit in 8 lanes (L, g), four each: max and sum over g (rows,
    // swaps of 16 and 32) and L (adjacent lanes, DPP), the sum in the tree of
    // vx_quantize_x (pairs within each 4; then 4g, 4(g^1); then g, g^2; then
    // the halves). The scale divisions are spread one (block, column) per
    // lane through LDS, the levels are formed per lane and the two lanes of
    // a column swap the halves they need.
    // FH (B <= 4): the spare half of the lanes splits the other half of
    // the blocks: lanes of columns 4 + c (c8 = n / 2 >= 4) take blocks 4..7
    // of column c, so each lane splits 4 blocks instead of 8, and a row
    // rotation by 8 (DPP row_ror:8) hands blocks 4..7 to the lanes of column
    // c. The A rows of columns 4..7 then hold other columns' levels: only
    // outputs of columns < B are written.
    constexpr int NBL = FH ? 4 : 8;  // blocks per lane
    f32x4 xv[XI][NCG][NBL];
    auto pass_split_loads = [&](uint32_t p) {
        const uint32_t c8 = n >> 1, L = n & 1u;
        const uint32_t cl = FH ? (c8 & 3u) : c8, bo = FH ? 4u * (c8 >> 2) : 0u;
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const uint32_t item = p * PI + (uint32_t)XI * slot + (uint32_t)j;
#pragma unroll
            for (int h = 0; h < NCG; ++h) {
                const uint32_t col = 8u * (uint32_t)h + cl;
                const float* xp = a.x + (int64_t)(a.col0 + min(col, B - 1u)) * a.xs_b + 16u * L + 4u * g;
#pragma unroll
                for (int b = 0; b < NBL; ++b)
                    xv[j][h][b] = *(const f32x4*)(xp + 32 * (int64_t)min(8u * item + bo + (uint32_t)b, nblk - 1u));
            }
        }
    };
    auto pass_split_math = [&](uint32_t p) {
        const uint32_t c8 = n >> 1, L = n & 1u;
        const uint32_t cl = FH ? (c8 & 3u) : c8, bo = FH ? 4u * (c8 >> 2) : 0u;
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const uint32_t item = p * PI + (uint32_t)XI * slot + (uint32_t)j;
#pragma unroll
            for (int h = 0; h < NCG; ++h) {
                const f32x4 (&v)[NBL] = xv[j][h];
                // per block: max |v| and sum over the 8 lanes (L, g) of a
                // column, both through one exchange per step: the even rows
                // carry the max, the odd rows the sum. The max runs on the
                // bits (|v| >= 0 orders as unsigned; a NaN then wins, where
                // fmaxf would skip it, but a NaN makes the sum NaN and the
                // block non-finite either way). Afterwards rows 0 and 2 hold
                // m, rows 1 and 3 hold S (S added as vx_quantize_x adds it).
                uint32_t ms[NBL];
#pragma unroll
                for (int b = 0; b < NBL; ++b) {
                    const float am = fmaxf(fmaxf(fabsf(v[b].x), fabsf(v[b].y)), fmaxf(fabsf(v[b].z), fabsf(v[b].w)));
                    const float s4 = (v[b].x + v[b].y) + (v[b].z + v[b].w);
                    const bool odd = (g & 1u) != 0u;
                    // rows r, r ^ 1: x = row (r & 2) of (max, sum), y = row (r & 2) + 1
                    uint32_t x = __float_as_uint(am), y = __float_as_uint(s4);
                    vx_swap16(x, y);
                    uint32_t t = odd ? __float_as_uint(__uint_as_float(x) + __uint_as_float(y)) : max(x, y);
                    // rows r, r ^ 2
                    uint32_t x2 = t, y2 = t;
                    vx_swap32(x2, y2);
                    t = odd ? __float_as_uint(__uint_as_float(x2) + __uint_as_float(y2)) : max(x2, y2);
                    // lanes L, L ^ 1
                    const uint32_t o = __float_as_uint(vx_dpp<0xB1>(__uint_as_float(t)));
                    ms[b] = odd ? __float_as_uint(__uint_as_float(t) + __uint_as_float(o)) : max(t, o);
                }
                __builtin_amdgcn_wave_barrier();  // the previous chunk's table reads are done
                if (L == 0u && g < 2u) {
                    // g = 0 writes m, g = 1 writes S
#pragma unroll
                    for (int b = 0; b < NBL; ++b) ((uint32_t*)fxt)[2u * (8u * (bo + (uint32_t)b) + cl) + g] = ms[b];
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                __builtin_amdgcn_wave_barrier();
                {
                    // lane = (block b2, column c2) of this chunk (FH: the
                    // table holds columns 0..3 only; the others are never
                    // read back and publish zero scales)
                    const float2 ms = (FH && (lane & 7u) >= 4u) ? float2{0.f, 0.f} : fxt[lane];
                    const vx_xq_scale sc = vx_xq_scales(ms.x, ms.y);
                    fxp[lane] = float4{sc.c1, sc.i1, sc.i2, sc.fin ? 1.f : 0.f};
                    const uint32_t b2 = lane >> 3, c2 = lane & 7u;
                    const uint32_t blk = 8u * item + b2, colo = 8u * (uint32_t)h + c2;
                    float2 sv2 = (blk < nblk && colo < B) ? float2{sc.fin ? sc.c2 : ms.x + ms.y, ms.y}
                                                           : float2{0.f, 0.f};
                    if constexpr (QT == VX_Q4_0) sv2.y *= -8.f;
                    scl[(8u * (uint32_t)j + b2) * CP + colo] = sv2;
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int b = 0; b < NBL; ++b) {
                    const float4 q = fxp[8u * (bo + (uint32_t)b) + cl];
                    uint32_t w1, w2;
                    vx_xq_levels4(v[b], q.x, q.y, q.z, q.w != 0.f, w1, w2);
                    // level L of positions 8g..8g+3 (L = 0's elements) and
                    // 8g+4..8g+7 (L = 1's): each lane sends the other level
                    const uint32_t mine = L ? w2 : w1;
                    const uint32_t other = __float_as_uint(vx_dpp<0xB1>(__uint_as_float(L ? w1 : w2)));
                    const uint32_t lo = L ? other : mine, hi = L ? mine : other;
                    xa[j][b][h] = (long)((uint64_t)lo | ((uint64_t)hi << 32));
                    if constexpr (FH) {
                        // lane n + 8 of the row split block 4 + b of this lane's column
                        const uint32_t lo4 = __float_as_uint(vx_dpp<0x128>(__uint_as_float(lo)));
                        const uint32_t hi4 = __float_as_uint(vx_dpp<0x128>(__uint_as_float(hi)));
                        xa[j][4 + b][h] = (long)((uint64_t)lo4 | ((uint64_t)hi4 << 32));
                    }
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    };
    auto pass_split = [&](uint32_t p) {
        pass_split_loads(p);
        pass_split_math(p);
    };

    uint32_t raw[RD * XI][NW];
    auto ring_prologue = [&]() {
#pragma unroll
        for (int u = 0; u < RD; ++u) {
#pragma unroll
            for (int j = 0; j < XI; ++j) wload((uint32_t)u, j, raw[u * XI + j]);
            // slots issue in ring order (the scheduler would otherwise reorder
            // them, and waiting for slot 0 could mean waiting for all of them)
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if constexpr (FX) {
        // (issuing the ring between the x loads and the split arithmetic, to
        // overlap the two, measured 8-13 % slower: as with x levels, weight
        // requests ahead of a CU's x requests delay x more than they gain)
        pass_split(0u);
        ring_prologue();
    } else {
        // x requests first; a bare barrier puts every x request of the CU
        // ahead of every weight request; then the ring, and only then the
        // wait for this wave's x (the scales go to LDS). Measured against
        // waiting for x before issuing the ring (graph-replayed, same box):
        // Q4_0 4096x11008 B = 8 10.2 -> 9.5 us, 11008x4096 B = 8 9.5 -> 8.9 us,
        // Q4_K 32000x4096 B = 16 26.5 -> 25.5 us, 14336x4096 B = 16 even.
        pass_loads(0u);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        ring_prologue();
        pass_publish(0u);
    }

    float acc[NCG][2];
#pragma unroll
    for (int h = 0; h < NCG; ++h) acc[h][0] = acc[h][1] = 0.f;

    // the workgroup meets and writes y for tile-works [w0, w1]: one thread
    // per output of each tile in the range, adding the tile's passes in the
    // range in pass order (with several passes a range can hold one tile more
    // than once); an earlier range's sum of the tile is read back from y
    // (written before that range's closing barrier)
    auto flush = [&](uint32_t w0, uint32_t w1) {
        __syncthreads();
        const uint32_t per = B * 16u;
        const uint32_t ntile = min(w1 - w0 + 1u, nts);  // distinct tiles in the range
        for (uint32_t e = t; e < ntile * per; e += VX_XQ_WG) {
            const uint32_t k = e / per, rem = e - k * per;
            const uint32_t col = rem >> 4, rr = rem & 15u;
            const uint32_t ts = (w0 + k) % nts;
            const uint32_t row = rb + ts * rs + rr;
            float* yp = a.y + (int64_t)min(row, rlim - 1u) * a.ys_m + (int64_t)col * a.ys_b;
            float tot = 0.f;
            for (uint32_t w = w0 + k; w <= w1; w += nts) {
                const float* rb = red + (w % RMAX) * TILE_F;
                float s = 0.f;
#pragma unroll
                for (int q = 0; q < 16; ++q) s += rb[((uint32_t)q * CP + col) * 16u + rr];
                const uint32_t p = MP ? w / nts : 0u;
                tot = (w == w0 + k) ? ((MP && p > 0u && row < rlim) ? *yp + s : s) : tot + s;
            }
            if (row < rlim) *yp = tot;
        }
        __syncthreads();
    };

    uint32_t wflush = 0;  // first tile-work not yet written to y
    auto tile_work = [&](uint32_t w, int u, bool refill) {
        const uint32_t p = MP ? w / nts : 0u, ts = MP ? w - p * nts : w;
        if constexpr (MP) {
            if (ts == 0u && p > 0u) {
                if constexpr (FX) {
                    pass_split(p);
                } else {
                    pass_loads(p);
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    pass_publish(p);
                }
            }
        }
        (void)ts;
#pragma unroll
        for (int j = 0; j < XI; ++j) {
            const uint32_t item = p * PI + (uint32_t)XI * slot + (uint32_t)j;
            uint32_t (&rw)[NW] = raw[u * XI + j];
            if (item < ipr) {
                vx_xq_item<QT> it;
                vx_xq_prepare<QT>(rw, g, it);
                const uint32_t bl0 = 8u * (uint32_t)j;  // first block of the item in this wave's scales
                // Q4_K: the item's sums before its d / dmin (one super-block)
                float q1s[NCG][2], q2s[NCG][2];
#pragma unroll
                for (int h = 0; h < NCG; ++h) q1s[h][0] = q1s[h][1] = q2s[h][0] = q2s[h][1] = 0.f;
                // block b of the item: MFMA per column group, then the scales
                auto block = [&](int b) {
                    const long bw = (long)((uint64_t)it.lo[b] | ((uint64_t)it.hi[b] << 32));
#pragma unroll
                    for (int h = 0; h < NCG; ++h) {
                        const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[j][b][h], bw, i32x4{0, 0, 0, 0}, 0, 0, 0);
                        const f32x4 sc = *(const f32x4*)&scl[(bl0 + (uint32_t)b) * CP + 8u * (uint32_t)h + 2u * g];
#pragma unroll
                        for (int c = 0; c < 2; ++c) {
                            const float T = (float)(__mul24(D[2 * c], 254) + D[2 * c + 1]);
                            const float c2 = c ? sc.z : sc.x, sx = c ? sc.w : sc.y;
                            float v = acc[h][c];
                            if constexpr (QT == VX_Q4_0) {
                                v = __builtin_fmaf(it.ds[b], __builtin_fmaf(c2, T, sx), v);
                            } else if constexpr (QT == VX_Q8_0) {
                                v = __builtin_fmaf(it.ds[b], c2 * T, v);
                            } else {
                                const uint32_t sm = it.scm[b >> 1] >> (16 * (b & 1));
                                q1s[h][c] = __builtin_fmaf((float)(sm & 0xFFu), c2 * T, q1s[h][c]);
                                q2s[h][c] = __builtin_fmaf((float)((sm >> 8) & 0xFFu), sx, q2s[h][c]);
                            }
                            if constexpr (QT != VX_Q4_K) acc[h][c] = v;
                        }
                    }
                };
                if (8u * item + 8u <= nblk) {
                    // a whole item: no branch between the blocks, so the MFMAs
                    // of later blocks issue while earlier epilogues run
#pragma unroll
                    for (int b = 0; b < 8; ++b) block(b);
                } else {
                    const uint32_t nb = nblk - 8u * item;  // the partial last item
#pragma unroll
                    for (int b = 0; b < 8; ++b)
                        if ((uint32_t)b < nb) block(b);
                }
                if constexpr (QT == VX_Q4_K) {
#pragma unroll
                    for (int h = 0; h < NCG; ++h)
#pragma unroll
                        for (int c = 0; c < 2; ++c)
                            acc[h][c] = __builtin_fmaf(-it.dmin, q2s[h][c], __builtin_fmaf(it.d, q1s[h][c], acc[h][c]));
                }
            }
            // refill this ring slot with the same item of the tile-work RD
            // ahead (past the end: one cache line, see wload)
            if (refill) wload(w + RD, j, rw);
        }
        // park this slot's partial sums; the workgroup reduces every RMAX
        float* rb = red + (w % RMAX) * TILE_F;
#pragma unroll
        for (int h = 0; h < NCG; ++h)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                rb[(slot * CP + 8u * (uint32_t)h + 2u * g + (uint32_t)c) * 16u + n] = acc[h][c];
                acc[h][c] = 0.f;
            }
        if (w + 1u == nwork || w + 1u - wflush == RMAX) {
            flush(wflush, w);
            wflush = w + 1u;
        }
    };
    if constexpr (ST) {
        // (_st kernels: the host takes them when every CU's tile-works fit
        // the ring) the whole work is in the ring already: straight-line, no
        // refills. Through the loop below the compiler copies the ring
        // registers at the loop entry and so waits for the whole ring before
        // the first tile-work; here each tile-work waits for its own slot.
#pragma unroll
        for (int u = 0; u < RD; ++u)
            if ((uint32_t)u < nwork) tile_work((uint32_t)u, u, false);
        return;
    }
    // whole rounds of RD tile-works (every path issues the same loads), then
    // the last partial round
    const uint32_t nfull = nwork - nwork % RD;
    for (uint32_t w0 = 0; w0 < nfull; w0 += RD) {
#pragma unroll
        for (int u = 0; u < RD; ++u) tile_work(w0 + (uint32_t)u, u, true);
    }
#pragma unroll
    for (int u = 0; u < RD - 1; ++u)
        if (nfull + (uint32_t)u < nwork) tile_work(nfull + (uint32_t)u, u, true);
}

// One column group: CU positions per XCD (XM; same-box A/B, graph-replayed:
// Q4_0 11008x4096 B = 8 fused 10.25 -> 9.97 us, 4096x11008 B = 8 on a split
// 9.51 -> 9.43, Q8_0 4096^2 B = 8 7.51 -> 7.44). Two column groups keep the
// plain order (Q4_K 32000x4096 B = 16 27.96 against 28.41 us with XM).
#define VX_GEMV_XQ(QT, QN, NCG, XI, RD, MP, ST, FX, SFX, FH)                                       \
    extern "C" __global__ __launch_bounds__(VX_XQ_WG) void vx_gemv_xq_##QN##_c##NCG##_x##XI##SFX(vx_gemv_xq_args a) { \
        vx_gemv_xq<QT, NCG, XI, RD, MP, ST, FX, FH, NCG == 1>(a);                                        \
    }
// (column groups NCG, items per wave and pass XI, ring depth RD in tiles):
// RD * XI weight items in flight per wave, as many as the registers allow
// except Q4_0 with one item (measured best at 3 of the 4 that fit).
// One pass (K <= 4096 XI): exact waits; _mp: several passes; _st: one pass
// with at most RD tile-works per wave (no loop); _fx: x split in the kernel
// (x f32 with stride 1 along K) instead of read from a vx_quantize_x split.
#define VX_GEMV_XQ1(QT, QN, NCG, XI, RD)                       \
    VX_GEMV_XQ(QT, QN, NCG, XI, RD, false, false, false, , false)     \
    VX_GEMV_XQ(QT, QN, NCG, XI, RD, false, true, false, _st, false)
// _fx: x split in the kernel, for the one-pass shapes whose split fits the
// registers: one item per wave (any B <= 16), or 2-3 items with B <= 4
// (_fx4: each lane splits half the blocks) or 2 items with B <= 8
#define VX_GEMV_XQF(QT, QN, NCG, XI, RD)                                           \
    VX_GEMV_XQ(QT, QN, NCG, XI, RD, false, false, true, _fx, false)                \
    VX_GEMV_XQ(QT, QN, NCG, XI, RD, false, true, true, _st_fx, false)
#define VX_GEMV_XQF4(QT, QN, XI, RD)                                              \
    VX_GEMV_XQ(QT, QN, 1, XI, RD, false, false, true, _fx4, true)                 \
    VX_GEMV_XQ(QT, QN, 1, XI, RD, false, true, true, _st_fx4, true)
#define VX_GEMV_XQ1F(QT, QN, RD)                               \
    VX_GEMV_XQ1(QT, QN, 1, 1, RD)                              \
    VX_GEMV_XQF(QT, QN, 1, 1, RD)                              \
    VX_GEMV_XQF4(QT, QN, 1, RD)
// Q4_0, one item per wave: a ring of 3 tile-works (4: 9.97 -> 9.77 us at
// 11008x4096 B = 8, 9.12 -> 8.89 at B = 4; 2: 10.29 us)
VX_GEMV_XQ1F(VX_Q4_0, q4_0, 3)
VX_GEMV_XQ1(VX_Q4_0, q4_0, 1, 2, 1)
VX_GEMV_XQF(VX_Q4_0, q4_0, 1, 2, 1)
VX_GEMV_XQF4(VX_Q4_0, q4_0, 2, 1)
VX_GEMV_XQ1(VX_Q4_0, q4_0, 1, 3, 1)
VX_GEMV_XQF4(VX_Q4_0, q4_0, 3, 1)
VX_GEMV_XQ1(VX_Q4_0, q4_0, 2, 1, 3)
VX_GEMV_XQF(VX_Q4_0, q4_0, 2, 1, 3)
VX_GEMV_XQ(VX_Q4_0, q4_0, 1, 3, 1, true, false, false, _mp, false)
VX_GEMV_XQ(VX_Q4_0, q4_0, 2, 1, 1, true, false, false, _mp, false)
VX_GEMV_XQ1F(VX_Q8_0, q8_0, 2)
VX_GEMV_XQ1(VX_Q8_0, q8_0, 1, 2, 1)
VX_GEMV_XQF(VX_Q8_0, q8_0, 1, 2, 1)
VX_GEMV_XQF4(VX_Q8_0, q8_0, 2, 1)
VX_GEMV_XQ1(VX_Q8_0, q8_0, 2, 1, 2)
VX_GEMV_XQF(VX_Q8_0, q8_0, 2, 1, 2)
VX_GEMV_XQ(VX_Q8_0, q8_0, 1, 2, 1, true, false, false, _mp, false)
VX_GEMV_XQ(VX_Q8_0, q8_0, 2, 1, 1, true, false, false, _mp, false)
VX_GEMV_XQ1F(VX_Q4_K, q4_k, 3)
VX_GEMV_XQ1(VX_Q4_K, q4_k, 1, 2, 1)
VX_GEMV_XQF(VX_Q4_K, q4_k, 1, 2, 1)
VX_GEMV_XQF4(VX_Q4_K, q4_k, 2, 1)
VX_GEMV_XQ1(VX_Q4_K, q4_k, 2, 1, 2)
VX_GEMV_XQF(VX_Q4_K, q4_k, 2, 1, 2)
VX_GEMV_XQ(VX_Q4_K, q4_k, 1, 2, 1, true, false, false, _mp, false)
VX_GEMV_XQ(VX_Q4_K, q4_k, 2, 1, 1, true, false, false, _mp, false)
