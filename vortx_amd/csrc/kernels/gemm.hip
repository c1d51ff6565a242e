// gemm.hip — f32 GEMM kernels for gfx950 on canonical [n, c, rows, cols]
// views (any strides; batch dims n, c folded into grid z).
//
//  vx_gemm_naive   one thread per output, sequential-k f32 sum with one
//                  rounding per multiply and per add: the summation order of
//                  the reference's gemm_naive / gemm_tiled
//                  (vortx-shaders/src/linalg/gemm.rs:84-171, 225-235).
//  vx_gemm_mfma_*  128x128 output tile per workgroup (4 wave64 in 2x2, each
//                  64x64 = 2x2 v_mfma_f32_32x32x2f32 accumulators), K staged
//                  16 at a time through double-buffered LDS (k-major, one
//                  barrier per stage). Operand loads are 128-bit along the
//                  contiguous dimension of each operand; edge tiles are
//                  zero-filled like the reference (gemm.rs:102-106,121-125).
//                  The _w kernels take 128x256 tiles (each wave 64x128, 2x4
//                  accumulators, two workgroups per CU) with the same
//                  per-output summation order, so the same bits.
//  vx_gemv_f32     the N == 1 case: one (or, _r4, four) rows per workgroup,
//                  K split over its four waves, each with all its 128-bit
//                  loads of A in flight; partial sums meet in LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../vx_kargs.h"
#include "vx_args.hpp"
#include "vx_dpp.hpp"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define TBK 16
#define LDS_PAD 4

// Operand access modes (chosen on the host from strides and alignment).
#define MODE_KC 0  // contiguous along K, rows 16-byte aligned
#define MODE_XC 1  // contiguous along M (for A) / N (for B), 16-byte aligned
#define MODE_GEN 2 // anything else: scalar loads

// Output epilogue: alpha * acc + beta * c, where c is read only when
// beta != 0 (the BLAS convention: out may hold NaN when beta == 0). With
// alpha == 1 and beta == 0 the result is acc itself.
__device__ __forceinline__ void vx_epilogue(float* c, float acc, float alpha, float beta) {
    *c = beta == 0.f ? alpha * acc : alpha * acc + beta * *c;
}

// ---------------------------------------------------------------- naive
extern "C" __global__ __launch_bounds__(64) void vx_gemm_naive(vx_gemm_args p) {
    vx_args_fetch(p);
    const uint32_t j = blockIdx.x * 64u + threadIdx.x;
    const uint32_t i = blockIdx.y;
    const uint32_t z = blockIdx.z;
    if (j >= p.N) return;
    const uint32_t bn = z / p.batch_c, bc = z % p.batch_c;
    const float* a = p.a + bn * p.as[0] + bc * p.as[1] + (int64_t)i * p.as[2];
    const float* b = p.b + bn * p.bs[0] + bc * p.bs[1] + (int64_t)j * p.bs[3];
    float sum = 0.f;
    for (uint32_t k = 0; k < p.K; ++k) {
        // One rounding per multiply and per add (no FMA contraction).
#pragma clang fp contract(off)
        sum = sum + a[(int64_t)k * p.as[3]] * b[(int64_t)k * p.bs[2]];
    }
    float* c = p.c + bn * p.cs[0] + bc * p.cs[1] + (int64_t)i * p.cs[2] + (int64_t)j * p.cs[3];
    {
        // the epilogue rounds after each operation too: (alpha * sum) + (beta * c)
#pragma clang fp contract(off)
        *c = p.beta == 0.f ? p.alpha * sum : p.alpha * sum + p.beta * *c;
    }
}

// ----------------------------------------------------------------- mfma
// Global -> register fragment of one TBK slice of an operand tile.
// "x" is the non-K dimension of the operand (M for A, N for B); sx/sk the
// element strides along x and k; X the operand's extent along x.
template <int MODE, int TX>
struct vx_frag {
    float v[TX / 16];
};

template <int MODE, int TX>
__device__ __forceinline__ void vx_load_frag(vx_frag<MODE, TX>& f, const float* base, int64_t sx, int64_t sk,
                                             uint32_t x0, uint32_t X, uint32_t k0, uint32_t K) {
    const uint32_t t = threadIdx.x;
    constexpr uint32_t QX = TX / 4;  // float4 per k-row (MODE_XC)
    if constexpr (MODE == MODE_KC) {
        // TX x-rows of 4 float4 along k: element (x = f>>2, k = 4(f&3)).
#pragma unroll
        for (int i = 0; i < TX / 64; ++i) {
            const uint32_t fi = t + 256u * i;
            const uint32_t x = x0 + (fi >> 2), k = k0 + 4u * (fi & 3u);
            const float* p = base + (int64_t)x * sx + k;
            if (x < X && k + 3 < K) {
                const f32x4 q = *(const f32x4*)p;
                f.v[4 * i + 0] = q.x; f.v[4 * i + 1] = q.y; f.v[4 * i + 2] = q.z; f.v[4 * i + 3] = q.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) f.v[4 * i + e] = (x < X && k + e < K) ? p[e] : 0.f;
            }
        }
    } else if constexpr (MODE == MODE_XC) {
        // 16 k-rows of TX / 4 float4 along x: element (k = f / QX, x = 4(f % QX)).
#pragma unroll
        for (int i = 0; i < TX / 64; ++i) {
            const uint32_t fi = t + 256u * i;
            const uint32_t k = k0 + fi / QX, x = x0 + 4u * (fi % QX);
            const float* p = base + (int64_t)k * sk + x;
            if (k < K && x + 3 < X) {
                const f32x4 q = *(const f32x4*)p;
                f.v[4 * i + 0] = q.x; f.v[4 * i + 1] = q.y; f.v[4 * i + 2] = q.z; f.v[4 * i + 3] = q.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) f.v[4 * i + e] = (k < K && x + e < X) ? p[e] : 0.f;
            }
        }
    } else {
        // scalar: element (k = f / TX, x = f % TX), f = t + 256 i.
#pragma unroll
        for (int i = 0; i < TX / 16; ++i) {
            const uint32_t fi = t + 256u * i;
            const uint32_t k = k0 + fi / TX, x = x0 + fi % TX;
            f.v[i] = (k < K && x < X) ? base[(int64_t)k * sk + (int64_t)x * sx] : 0.f;
        }
    }
}

// The same fragment for a tile that lies inside the operand along x and a
// stage that lies inside K: every load unconditional (no zero fill), so the
// compiler counts outstanding loads exactly across the pipelined loop.
template <int MODE, int TX>
__device__ __forceinline__ void vx_load_frag_full(vx_frag<MODE, TX>& f, const float* base, int64_t sx, int64_t sk,
                                                  uint32_t x0, uint32_t k0) {
    const uint32_t t = threadIdx.x;
    constexpr uint32_t QX = TX / 4;
    if constexpr (MODE == MODE_KC) {
#pragma unroll
        for (int i = 0; i < TX / 64; ++i) {
            const uint32_t fi = t + 256u * i;
            const f32x4 q = *(const f32x4*)(base + (int64_t)(x0 + (fi >> 2)) * sx + k0 + 4u * (fi & 3u));
            f.v[4 * i + 0] = q.x; f.v[4 * i + 1] = q.y; f.v[4 * i + 2] = q.z; f.v[4 * i + 3] = q.w;
        }
    } else if constexpr (MODE == MODE_XC) {
        // the stage's offset k0 * sk is uniform (scalar); the per-thread part
        // is the same every stage, so the compiler keeps it out of the loop
        // (written as one product, it cost a 64-bit multiply per load and stage)
        const float* stage = base + (int64_t)k0 * sk;
#pragma unroll
        for (int i = 0; i < TX / 64; ++i) {
            const uint32_t fi = t + 256u * i;
            const f32x4 q = *(const f32x4*)(stage + ((int64_t)(fi / QX) * sk + x0 + 4u * (fi % QX)));
            f.v[4 * i + 0] = q.x; f.v[4 * i + 1] = q.y; f.v[4 * i + 2] = q.z; f.v[4 * i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < TX / 16; ++i) {
            const uint32_t fi = t + 256u * i;
            f.v[i] = base[(int64_t)(k0 + fi / TX) * sk + (int64_t)(x0 + fi % TX) * sx];
        }
    }
}

// Register fragment -> LDS tile S[k][x] (row pitch LD).
template <int MODE, int TX, int LD>
__device__ __forceinline__ void vx_store_frag(const vx_frag<MODE, TX>& f, float* S) {
    const uint32_t t = threadIdx.x;
    constexpr uint32_t QX = TX / 4;
    if constexpr (MODE == MODE_KC) {
#pragma unroll
        for (int i = 0; i < TX / 64; ++i) {
            const uint32_t fi = t + 256u * i;
            const uint32_t x = fi >> 2, k = 4u * (fi & 3u);
#pragma unroll
            for (int e = 0; e < 4; ++e) S[(k + e) * LD + x] = f.v[4 * i + e];
        }
    } else if constexpr (MODE == MODE_XC) {
#pragma unroll
        for (int i = 0; i < TX / 64; ++i) {
            const uint32_t fi = t + 256u * i;
            const uint32_t k = fi / QX, x = 4u * (fi % QX);
            *(f32x4*)(S + k * LD + x) = f32x4{f.v[4 * i], f.v[4 * i + 1], f.v[4 * i + 2], f.v[4 * i + 3]};
        }
    } else {
#pragma unroll
        for (int i = 0; i < TX / 16; ++i) {
            const uint32_t fi = t + 256u * i;
            S[(fi / TX) * LD + fi % TX] = f.v[i];
        }
    }
}

template <int AMODE, int BMODE, int TM, int TN>
__device__ __forceinline__ void vx_gemm_mfma(const vx_gemm_args& p) {
    // per wave: TM / 2 x TN / 2, MI row and NJ column blocks of 32
    constexpr int LDA = TM + LDS_PAD, LDB = TN + LDS_PAD, MI = TM / 64, NJ = TN / 64;
    __shared__ float As[2][TBK * LDA];
    __shared__ float Bs[2][TBK * LDB];

    // Tile order: consecutive workgroup ids land on different XCDs (round
    // robin over 8), so ids are first regrouped per XCD, then walked in
    // groups of 8 tile-rows so an XCD's resident tiles share A and B panels
    // in its L2.
    const uint32_t nt = p.tiles_m * p.tiles_n;
    uint32_t bid = blockIdx.x;
    if ((nt & 7u) == 0) bid = (bid & 7u) * (nt >> 3) + (bid >> 3);
    const uint32_t group = 8u * p.tiles_n;
    const uint32_t first_m = (bid / group) * 8u;
    const uint32_t gsize = min(p.tiles_m - first_m, 8u);
    const uint32_t tm = first_m + (bid % group) % gsize;
    const uint32_t tn = (bid % group) / gsize;
    const uint32_t m0 = tm * TM, n0 = tn * TN;

    const uint32_t z = blockIdx.z;
    const uint32_t bn = z / p.batch_c, bc = z % p.batch_c;
    const float* A = p.a + bn * p.as[0] + bc * p.as[1];
    const float* B = p.b + bn * p.bs[0] + bc * p.bs[1];
    float* Cp = p.c + bn * p.cs[0] + bc * p.cs[1];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;
    const uint32_t l32 = lane & 31u, lk = lane >> 5;

    f32x16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // k-pairs [k0, k1) of one TBK stage from LDS buffer `buf`.
    auto mma_part = [&](uint32_t buf, int k0, int k1) {
        const float* as = As[buf] + wm * (TM / 2u) + l32;
        const float* bs = Bs[buf] + wn * (TN / 2u) + l32;
#pragma unroll
        for (int ks = k0; ks < k1; ++ks) {
            const uint32_t kk = 2u * ks + lk;
            float a[MI], b[NJ];
#pragma unroll
            for (int i = 0; i < MI; ++i) a[i] = as[kk * LDA + 32 * i];
#pragma unroll
            for (int j = 0; j < NJ; ++j) b[j] = bs[kk * LDB + 32 * j];
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int i = 0; i < MI; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };
    auto mma = [&](uint32_t buf) { mma_part(buf, 0, TBK / 2); };

    const uint32_t nkf = p.K / TBK;  // whole stages
    if (m0 + TM <= p.M && n0 + TN <= p.N) {
        // Tile inside M and N: the loads for stage s + 2 are issued while
        // stage s is multiplied (two register buffers), so each load has two
        // stages of MFMAs to arrive before its LDS store waits for it. Stage
        // indices are clamped to the last whole stage (the extra loads at the
        // end are harmless). Unrolled by two so each buffer is named.
        if (nkf) {
            vx_frag<AMODE, TM> ra0, ra1;
            vx_frag<BMODE, TN> rb0, rb1;
            auto ld = [&](uint32_t st, vx_frag<AMODE, TM>& fa_, vx_frag<BMODE, TN>& fb_) {
                const uint32_t k0 = min(st, nkf - 1u) * TBK;
                vx_load_frag_full<AMODE, TM>(fa_, A, p.as[2], p.as[3], m0, k0);
                vx_load_frag_full<BMODE, TN>(fb_, B, p.bs[3], p.bs[2], n0, k0);
            };
            ld(0u, ra0, rb0);
            ld(1u, ra1, rb1);
            vx_store_frag<AMODE, TM, LDA>(ra0, As[0]);
            vx_store_frag<BMODE, TN, LDB>(rb0, Bs[0]);
            __syncthreads();
            // Invariant at the top: stage st in buffer 0, stage st + 1 in
            // flight to ra1 / rb1.
            // The other buffer's stores go in among the stage's MFMAs (its
            // last readers finished before the previous barrier): A's after
            // the first k-pair, B's after the third, so the matrix pipes
            // still hold the stage's remaining MFMAs when the wave reaches
            // the barrier. Stores after all eight k-pairs, then after two,
            // then split 1 / 3 (same-box A/B, TFLOP/s): 4096 x 11008 x 4096
            // 127.3 -> 131.9 -> 133.0, 4096^3 (wide) 137.5 -> 139.6 -> 141.3,
            // 2048^3 113.5 -> 118.6 -> 121.7. The bits do not change.
            // Narrow and small tiles (TN <= 128) issue the next loads after
            // B's stores, wide tiles at the top of the stage (same-box A/B,
            // TFLOP/s, loads at the top / after B's stores: 128 x 128 tiles
            // 4096 x 11008 x 4096 132.9 / 135.2, 4096^3 134.8 / 137.0, 2048^3
            // 117.6 / 124.0; 128 x 256 tiles 4096^3 140.8 / 140.3).
            constexpr bool LATE_LD = TN <= 128;
            auto half = [&](uint32_t buf, vx_frag<AMODE, TM>& sa, vx_frag<BMODE, TN>& sb, vx_frag<AMODE, TM>& la,
                            vx_frag<BMODE, TN>& lb, uint32_t ns) {
                if (!LATE_LD) {
                    ld(ns, la, lb);
                    // keep the loads above the MFMAs (the scheduler would sink
                    // them below the other buffer's store and share its registers)
                    __builtin_amdgcn_sched_barrier(0);
                }
                mma_part(buf, 0, 1);
                vx_store_frag<AMODE, TM, LDA>(sa, As[buf ^ 1u]);
                mma_part(buf, 1, 3);
                vx_store_frag<BMODE, TN, LDB>(sb, Bs[buf ^ 1u]);
                if (LATE_LD) {
                    __builtin_amdgcn_sched_barrier(0);
                    ld(ns, la, lb);
                    __builtin_amdgcn_sched_barrier(0);
                }
                mma_part(buf, 3, TBK / 2);
                __syncthreads();
            };
            uint32_t st = 0;
            for (; st + 2u <= nkf; st += 2u) {
                half(0u, ra1, rb1, ra0, rb0, st + 2u);
                half(1u, ra0, rb0, ra1, rb1, st + 3u);
            }
            if (st < nkf) mma(0u);  // an odd stage count: the last one
        }
        if (p.K % TBK) {
            // the K tail: one stage zero-filled past K, through buffer 1
            // (its last reader finished before a barrier)
            vx_frag<AMODE, TM> fa;
            vx_frag<BMODE, TN> fb;
            vx_load_frag<AMODE, TM>(fa, A, p.as[2], p.as[3], m0, p.M, nkf * TBK, p.K);
            vx_load_frag<BMODE, TN>(fb, B, p.bs[3], p.bs[2], n0, p.N, nkf * TBK, p.K);
            vx_store_frag<AMODE, TM, LDA>(fa, As[1]);
            vx_store_frag<BMODE, TN, LDB>(fb, Bs[1]);
            __syncthreads();
            mma(1u);
        }
    } else {
        // Edge tile: zero-filled loads of the next stage during this one.
        vx_frag<AMODE, TM> fa;
        vx_frag<BMODE, TN> fb;
        const uint32_t nk = (p.K + TBK - 1) / TBK;
        if (nk) {
            vx_load_frag<AMODE, TM>(fa, A, p.as[2], p.as[3], m0, p.M, 0, p.K);
            vx_load_frag<BMODE, TN>(fb, B, p.bs[3], p.bs[2], n0, p.N, 0, p.K);
            vx_store_frag<AMODE, TM, LDA>(fa, As[0]);
            vx_store_frag<BMODE, TN, LDB>(fb, Bs[0]);
            __syncthreads();
        }
        for (uint32_t kt = 0; kt < nk; ++kt) {
            const uint32_t cur = kt & 1u;
            const bool more = kt + 1 < nk;
            if (more) {
                vx_load_frag<AMODE, TM>(fa, A, p.as[2], p.as[3], m0, p.M, (kt + 1) * TBK, p.K);
                vx_load_frag<BMODE, TN>(fb, B, p.bs[3], p.bs[2], n0, p.N, (kt + 1) * TBK, p.K);
            }
            mma(cur);
            if (more) {
                vx_store_frag<AMODE, TM, LDA>(fa, As[cur ^ 1u]);
                vx_store_frag<BMODE, TN, LDB>(fb, Bs[cur ^ 1u]);
            }
            __syncthreads();
        }
    }

    // D layout of v_mfma_f32_32x32x2f32: register v of lane l holds
    // row 8*(v/4) + 4*(l/32) + v%4, column l%32 of the 32x32 tile.
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const uint32_t col = n0 + wn * (TN / 2u) + 32u * j + l32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t row = m0 + wm * (TM / 2u) + 32u * i + 8u * (v >> 2) + 4u * lk + (v & 3);
                if (row < p.M && col < p.N)
                    vx_epilogue(Cp + (int64_t)row * p.cs[2] + (int64_t)col * p.cs[3], acc[i][j][v], p.alpha, p.beta);
            }
        }
}

// WPE 3 (amdgpu_waves_per_eu(3, 4)) caps a kernel at 168 registers: three
// 256-thread workgroups per CU (the wide kernels use ~245 under WPE 2: two). The two-stage prefetch's second register
// buffer needs ~150-166 registers; squeezed into WPE 4's 128 (four
// workgroups per CU) it ran slower: 4096^3 118.7 vs 123.5 TFLOP/s, B
// transposed 126.4 vs 134.9, 1024^3 25.5 vs 29.8 (same-box A/B). The
// all-scalar mode needs more and is left uncapped (WPE 1).
#define VX_GEMM_MFMA(AM, BM, NAME, WPE)                                                              \
    extern "C" __global__ __launch_bounds__(VX_WG) __attribute__((amdgpu_waves_per_eu(WPE, 4)))    \
    void vx_gemm_mfma_##NAME(vx_gemm_args p) {                                                       \
        vx_gemm_mfma<AM, BM, 128, 128>(p);                                                              \
    }
#define VX_GEMM_MFMA_W(AM, BM, NAME)                                                                 \
    extern "C" __global__ __launch_bounds__(VX_WG) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
    void vx_gemm_mfma_##NAME##_w(vx_gemm_args p) {                                                   \
        vx_gemm_mfma<AM, BM, 128, 256>(p);                                                              \
    }
// 64 x 64 tiles (each wave 32 x 32, one accumulator) for shapes with fewer
// 128 x 128 tiles than CUs: 1024^3 is 64 such tiles but 256 small ones.
#define VX_GEMM_MFMA_S(AM, BM, NAME)                                                                 \
    extern "C" __global__ __launch_bounds__(VX_WG) __attribute__((amdgpu_waves_per_eu(4, 8)))      \
    void vx_gemm_mfma_##NAME##_s(vx_gemm_args p) {                                                   \
        vx_gemm_mfma<AM, BM, 64, 64>(p);                                                             \
    }
// Suffix letters: A mode then B mode; k = contiguous along K,
// x = contiguous along M / N, g = generic.
VX_GEMM_MFMA(MODE_KC, MODE_XC, kx, 3)  // row-major A, row-major B
VX_GEMM_MFMA(MODE_KC, MODE_KC, kk, 3)  // row-major A, B = transposed view of [N, K]
VX_GEMM_MFMA(MODE_XC, MODE_XC, xx, 3)
VX_GEMM_MFMA(MODE_XC, MODE_KC, xk, 3)
VX_GEMM_MFMA(MODE_GEN, MODE_GEN, gg, 1)
VX_GEMM_MFMA(MODE_KC, MODE_GEN, kg, 3)
VX_GEMM_MFMA(MODE_GEN, MODE_XC, gx, 3)
VX_GEMM_MFMA_W(MODE_KC, MODE_XC, kx)
VX_GEMM_MFMA_W(MODE_KC, MODE_KC, kk)
VX_GEMM_MFMA_S(MODE_KC, MODE_XC, kx)
VX_GEMM_MFMA_S(MODE_KC, MODE_KC, kk)

// ---------------------------------------------------------------- gemv
// y[m] = sum_k A[m, k] x[k]; A contiguous along K with 16-byte aligned
// rows (as_k == 1); x any stride. Grid: (ceil(M/4), batch).
// f32 GEMV y = alpha A x + beta y, A [M, K] rows contiguous along K and
// 16-byte aligned (the host's route condition), x any stride. HBM-bound: A is
// read once (4 M K bytes). A workgroup owns R rows; its four waves split K:
// wave w takes the 256-element steps w, w + 4, ... and issues S of them (R S
// 128-bit loads, x beside them from global: L1 hits after the first
// workgroup of a CU) before it uses any, so a row's bytes are all in flight
// at once up to K = 4096 (R = 1) or 1024 (R = 4); the four partial sums per
// row meet in LDS in wave order. Lanes past K load nothing and add zero.
// (Measured at 11008 x 4096: 75 % of HBM peak, against 60 % for one wave per
// two rows with x staged in LDS and 62 % for a persistent row-streaming
// grid: the split keeps four times more rows' bytes in flight per CU.)
#define VX_GEMV_S 4
template <uint32_t R>
__device__ __forceinline__ void vx_gemv_f32_rows(const vx_gemv_f32_args& p) {
    constexpr uint32_t S = VX_GEMV_S;
    __shared__ float red[4][R];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t z = blockIdx.y;
    const uint32_t bn = z / p.batch_c, bc = z % p.batch_c;
    const float* x = p.x + bn * p.x_bs[0] + bc * p.x_bs[1];
    const uint32_t row0 = blockIdx.x * R;
    const float* arow[R];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r)
        arow[r] = p.a + bn * p.a_bs[0] + bc * p.a_bs[1] + (int64_t)min(row0 + r, p.M - 1u) * p.as_m;
    const uint32_t K4 = p.K & ~3u;
    const uint32_t nst = (K4 + 255u) >> 8;  // 256-element steps
    float acc[R];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) acc[r] = 0.f;
    for (uint32_t j0 = wave; j0 < nst; j0 += 4u * S) {
        f32x4 av[S][R], xv[S];
#pragma unroll
        for (uint32_t u = 0; u < S; ++u) {
            const uint32_t k = 256u * (j0 + 4u * u) + 4u * lane;
            const bool in = j0 + 4u * u < nst && k < K4;
#pragma unroll
            for (uint32_t r = 0; r < R; ++r) av[u][r] = in ? *(const f32x4*)(arow[r] + k) : f32x4{0.f, 0.f, 0.f, 0.f};
            if (!in) xv[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            else if (p.xs_k == 1) xv[u] = *(const f32x4*)(x + k);
            else xv[u] = f32x4{x[(int64_t)k * p.xs_k], x[(int64_t)(k + 1) * p.xs_k], x[(int64_t)(k + 2) * p.xs_k],
                               x[(int64_t)(k + 3) * p.xs_k]};
        }
#pragma unroll
        for (uint32_t u = 0; u < S; ++u)
#pragma unroll
            for (uint32_t r = 0; r < R; ++r) {
                acc[r] = __builtin_fmaf(av[u][r].x, xv[u].x, acc[r]);
                acc[r] = __builtin_fmaf(av[u][r].y, xv[u].y, acc[r]);
                acc[r] = __builtin_fmaf(av[u][r].z, xv[u].z, acc[r]);
                acc[r] = __builtin_fmaf(av[u][r].w, xv[u].w, acc[r]);
            }
    }
    if (wave == 0u && K4 + lane < p.K) {  // K % 4 tail
        const float xt = x[(int64_t)(K4 + lane) * p.xs_k];
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) acc[r] = __builtin_fmaf(arow[r][K4 + lane], xt, acc[r]);
    }
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
        const float v = vx_wave_sum(acc[r]);
        if (lane == 0) red[wave][r] = v;
    }
    __syncthreads();
    if (t < R && row0 + t < p.M) {
        const float v = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
        vx_epilogue(p.y + bn * p.y_bs[0] + bc * p.y_bs[1] + (int64_t)(row0 + t) * p.ys_m, v, p.alpha, p.beta);
    }
}
extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_f32(vx_gemv_f32_args p) { vx_gemv_f32_rows<1>(p); }
extern "C" __global__ __launch_bounds__(VX_WG) void vx_gemv_f32_r4(vx_gemv_f32_args p) { vx_gemv_f32_rows<4>(p); }

