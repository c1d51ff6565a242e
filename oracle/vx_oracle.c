/*
 * vx_oracle.c — CPU ORACLE for the vortx linalg hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product path (libvortx_hip.so) neither links nor calls it.
 *
 * What it restates, and what pins each part (checks live in tests/):
 *
 *  - orc_quantize: f32 rows -> Q8_0 / Q4_0 / Q4_K blocks, restating ggml's
 *    published reference quantizers (ggml-quants.c quantize_row_q8_0_ref,
 *    quantize_row_q4_0_ref, quantize_row_q4_K_ref with make_qkx2_quants and
 *    nearest_int, in the form they have had since k-quants landed in June
 *    2023). ggml is not a dependency of vortx and is not in the reference,
 *    and no ggml-produced vectors exist here, so parity with ggml itself is
 *    unpinned; the restatement is pinned by invariants (error bounds, exact
 *    round trips of representable blocks, hand-computed blocks) and
 *    orc_f32_to_f16 against numpy's float16 rounding.
 *  - orc_contiguous_u32: vortx's contiguous shader (vortx-shaders/src/
 *    linalg/contiguous.rs:59-90): thread i writes dest[i] = src[offset +
 *    it(n, c, h, w)] with (n, c, h, w) the row-major split of i over the
 *    canonical sizes and it() in u32 arithmetic (shape.rs:46-48), as the
 *    shader does. Pinned against numpy's as_strided copy.
 *  - orc_f16_to_f32: IEEE-754 binary16 -> binary32, from the format's
 *    definition. Pinned exhaustively (all 65536 bit patterns) against
 *    numpy's float16 conversion.
 *  - orc_dequant_*: GGML block formats Q8_0 / Q4_0 / Q4_K (public ggml
 *    block_q8_0 / block_q4_0 / block_q4_K layout). The reference has NO
 *    quantized code (no file to cite), so relative to the reference this is
 *    "parity unpinned"; the decode is pinned instead by hand-built known-
 *    answer blocks with literal expected values (tests/golden), one-hot
 *    position sweeps, exact scale linearity and cross-format identities.
 *  - orc_gemm_ref_f32: the f32 summation order of the reference kernels,
 *    gemm_naive (vortx-shaders/src/linalg/gemm.rs:225-235: sum += l*r over
 *    k, sequential) and gemm_tiled (:84-171: per output acc += a*b over
 *    k, tile after tile; zero padding adds +0 which leaves the value
 *    unchanged). Built with -ffp-contract=off: one rounding per mul and per
 *    add. Index math follows Shape::it (vortx-shaders/src/linalg/shape.rs:
 *    46-48) in 64 bits. Pinned against numpy float64 matmul (BLAS) and the
 *    closed forms identity / zero / K=0 / K=1 / integer-exact products.
 *  - orc_gemm_f64: the same contraction accumulated in double (the parity
 *    reference for GPU outputs, tolerance stated in each test).
 *  - orc_gemv_q_f64: y = W x over exactly decoded weights, in double.
 *  - orc_gemm_tiled_f32_omp / orc_gemv_q_f32_omp: CPU-parallel restatements
 *    used only as bench.py's cpu_baseline ("port"): the first keeps
 *    gemm_tiled's 64x64x16 tiling and k order with one output tile per
 *    OpenMP task (vortx-shaders/src/linalg/gemm.rs:14-34, 84-192); the second
 *    is a dequant-dot with no reference equivalent.
 *
 * oracle/_ref: the reference is Rust (crate vortx 0.3.0 + rust-gpu shaders,
 * Cargo.toml:1-58) and this image has no Rust toolchain and no crates.io
 * registry, so the reference itself is unbuildable here; nothing is built
 * into oracle/_ref.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_Q4_0 2
#define ORC_Q8_0 8
#define ORC_Q4_K 12

/* ---------------------------------------------------------------- */
/* binary16 -> binary32                                             */
/* ---------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) & 1u;
    const uint32_t e = (uint32_t)(h >> 10) & 0x1Fu;
    const uint32_t m = (uint32_t)h & 0x3FFu;
    float mag;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in f32 */
        mag = ldexpf((float)m, -24);
    } else if (e == 31) {
        mag = m ? NAN : INFINITY;
    } else {
        /* normal: (1024 + m) * 2^(e - 25), exact in f32 */
        mag = ldexpf((float)(1024u + m), (int)e - 25);
    }
    return sign ? -mag : mag;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

int orc_qtype_info(uint32_t qtype, uint32_t* qk, uint32_t* bytes) {
    switch (qtype) {
    case ORC_Q4_0: *qk = 32; *bytes = 18; return 0;
    case ORC_Q8_0: *qk = 32; *bytes = 34; return 0;
    case ORC_Q4_K: *qk = 256; *bytes = 144; return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- */
/* Block decoders (one block -> QK floats)                          */
/* ---------------------------------------------------------------- */

/* block_q8_0 { half d; int8 qs[32]; }  value_i = d * qs[i] */
static void dq_q8_0(const uint8_t* blk, float* out) {
    const float d = orc_f16_to_f32(rd16(blk));
    for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)blk[2 + i];
}

/* block_q4_0 { half d; uint8 qs[16]; }
 * value_j = (lo(qs[j]) - 8) * d, value_{j+16} = (hi(qs[j]) - 8) * d */
static void dq_q4_0(const uint8_t* blk, float* out) {
    const float d = orc_f16_to_f32(rd16(blk));
    for (int j = 0; j < 16; ++j) {
        const uint8_t q = blk[2 + j];
        out[j] = (float)((int)(q & 0xF) - 8) * d;
        out[j + 16] = (float)((int)(q >> 4) - 8) * d;
    }
}

/* 6-bit scale and min of sub-block s (0..7) from the 12 packed bytes. */
void orc_q4k_scale_min(const uint8_t* sc12, int s, uint8_t* sc, uint8_t* mn) {
    if (s < 4) {
        *sc = sc12[s] & 63;
        *mn = sc12[s + 4] & 63;
    } else {
        *sc = (uint8_t)((sc12[s + 4] & 0xF) | ((sc12[s - 4] >> 6) << 4));
        *mn = (uint8_t)((sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4));
    }
}

/* block_q4_K { half d; half dmin; uint8 scales[12]; uint8 qs[128]; }
 * chunk c (0..3) = qs[32c .. 32c+32): low nibbles -> sub-block 2c
 * (elements 64c + l), high nibbles -> sub-block 2c+1 (elements 64c+32+l).
 * value = (d*sc)*q - (dmin*m). Both products are exact in f32; the
 * subtraction rounds once. */
static void dq_q4_k(const uint8_t* blk, float* out) {
    const float d = orc_f16_to_f32(rd16(blk));
    const float dmin = orc_f16_to_f32(rd16(blk + 2));
    const uint8_t* sc12 = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int c = 0; c < 4; ++c) {
        uint8_t sc0, m0, sc1, m1;
        orc_q4k_scale_min(sc12, 2 * c, &sc0, &m0);
        orc_q4k_scale_min(sc12, 2 * c + 1, &sc1, &m1);
        const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
        const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = qs[32 * c + l];
            out[64 * c + l] = d0 * (float)(q & 0xF) - mm0;
            out[64 * c + 32 + l] = d1 * (float)(q >> 4) - mm1;
        }
    }
}

static int dq_block(uint32_t qtype, const uint8_t* blk, float* out) {
    switch (qtype) {
    case ORC_Q4_0: dq_q4_0(blk, out); return 0;
    case ORC_Q8_0: dq_q8_0(blk, out); return 0;
    case ORC_Q4_K: dq_q4_k(blk, out); return 0;
    default: return -1;
    }
}

/* W[M, K] (rows row_stride bytes apart) -> out[M*K] row-major f32. */
int orc_dequant(uint32_t qtype, const uint8_t* w, uint32_t M, uint32_t K,
                uint64_t row_stride, float* out) {
    uint32_t qk, bb;
    if (orc_qtype_info(qtype, &qk, &bb)) return -1;
    if (K % qk) return -2;
    const uint32_t nb = K / qk;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; ++m) {
        const uint8_t* row = w + (uint64_t)m * row_stride;
        for (uint32_t b = 0; b < nb; ++b)
            dq_block(qtype, row + (uint64_t)b * bb, out + (uint64_t)m * K + (uint64_t)b * qk);
    }
    return 0;
}

/* y[m*ys_m + b*ys_b] = sum_k W[m,k] * x[k*xs_k + b*xs_b], in double. */
int orc_gemv_q_f64(uint32_t qtype, const uint8_t* w, uint32_t M, uint32_t K,
                   uint64_t row_stride, const float* x, int64_t xs_k,
                   int64_t xs_b, uint32_t B, double* y, int64_t ys_m,
                   int64_t ys_b) {
    uint32_t qk, bb;
    if (orc_qtype_info(qtype, &qk, &bb)) return -1;
    if (K % qk) return -2;
    const uint32_t nb = K / qk;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t m = 0; m < (int64_t)M; ++m) {
        float blk[256];
        double acc[64];
        for (uint32_t b0 = 0; b0 < B; b0 += 64) {
            const uint32_t bn = (B - b0) < 64 ? (B - b0) : 64;
            for (uint32_t b = 0; b < bn; ++b) acc[b] = 0.0;
            const uint8_t* row = w + (uint64_t)m * row_stride;
            for (uint32_t ib = 0; ib < nb; ++ib) {
                dq_block(qtype, row + (uint64_t)ib * bb, blk);
                for (uint32_t i = 0; i < qk; ++i) {
                    const int64_t k = (int64_t)ib * qk + i;
                    for (uint32_t b = 0; b < bn; ++b)
                        acc[b] += (double)blk[i] * (double)x[k * xs_k + (int64_t)(b0 + b) * xs_b];
                }
            }
            for (uint32_t b = 0; b < bn; ++b) y[m * ys_m + (int64_t)(b0 + b) * ys_b] = acc[b];
        }
    }
    return 0;
}

/* CPU baseline: f32 dequant-dot, OpenMP over rows, x contiguous [B, K]. */
int orc_gemv_q_f32_omp(uint32_t qtype, const uint8_t* w, uint32_t M, uint32_t K,
                       uint64_t row_stride, const float* x, uint32_t B, float* y,
                       int nthreads) {
    uint32_t qk, bb;
    if (orc_qtype_info(qtype, &qk, &bb)) return -1;
    if (K % qk || B > 64) return -2;
    const uint32_t nb = K / qk;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; ++m) {
        float blk[256];
        float acc[64];
        for (uint32_t b = 0; b < B; ++b) acc[b] = 0.0f;
        const uint8_t* row = w + (uint64_t)m * row_stride;
        for (uint32_t ib = 0; ib < nb; ++ib) {
            dq_block(qtype, row + (uint64_t)ib * bb, blk);
            for (uint32_t b = 0; b < B; ++b) {
                const float* xb = x + (uint64_t)b * K + (uint64_t)ib * qk;
                float s = 0.0f;
                for (uint32_t i = 0; i < qk; ++i) s += blk[i] * xb[i];
                acc[b] += s;
            }
        }
        for (uint32_t b = 0; b < B; ++b) y[(uint64_t)m * B + b] = acc[b];
    }
    return 0;
}

/* ---------------------------------------------------------------- */
/* GEMM on canonical rank-4 views                                    */
/* ---------------------------------------------------------------- */

/* A canonical [n, c, h, w] view: element (i0,i1,i2,i3) at
 * base[i0*s0 + i1*s1 + i2*s2 + i3*s3] (Shape::it, shape.rs:46-48). */
typedef struct orc_view {
    const float* base;
    uint32_t size[4];
    int64_t stride[4];
} orc_view;

static inline float at(const orc_view* v, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return v->base[(int64_t)a * v->stride[0] + (int64_t)b * v->stride[1] +
                   (int64_t)c * v->stride[2] + (int64_t)d * v->stride[3]];
}

/* out (f32 view, written through `out_base` with its strides) =
 * lhs * rhs in the reference's f32 order: per output, sum starts at +0
 * and adds l*r for k = 0..K-1 sequentially, one rounding per op. */
int orc_gemm_ref_f32(float* out_base, const int64_t* out_stride,
                     const orc_view* lhs, const orc_view* rhs) {
    const uint32_t N0 = lhs->size[0], C = lhs->size[1], M = lhs->size[2], K = lhs->size[3];
    const uint32_t N = rhs->size[3];
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t bn = 0; bn < (int64_t)N0; ++bn)
        for (int64_t bc = 0; bc < (int64_t)C; ++bc)
            for (uint32_t i = 0; i < M; ++i)
                for (uint32_t j = 0; j < N; ++j) {
                    float sum = 0.0f;
                    for (uint32_t k = 0; k < K; ++k) {
                        const float p = at(lhs, bn, bc, i, k) * at(rhs, bn, bc, k, j);
                        sum = sum + p;
                    }
                    out_base[bn * out_stride[0] + bc * out_stride[1] + (int64_t)i * out_stride[2] +
                             (int64_t)j * out_stride[3]] = sum;
                }
    return 0;
}

/* Double-precision contraction. out is a dense [n, c, nrows_sel, N]
 * array. rows == NULL selects every row; otherwise only rows[r],
 * r < nrows (used to check large GPU outputs on a sample of rows). */
int orc_gemm_f64(double* out, const orc_view* lhs, const orc_view* rhs,
                 const uint32_t* rows, uint32_t nrows) {
    const uint32_t N0 = lhs->size[0], C = lhs->size[1], M = lhs->size[2], K = lhs->size[3];
    const uint32_t N = rhs->size[3];
    const uint32_t R = rows ? nrows : M;
#pragma omp parallel for collapse(3) schedule(dynamic, 4)
    for (int64_t bn = 0; bn < (int64_t)N0; ++bn)
        for (int64_t bc = 0; bc < (int64_t)C; ++bc)
            for (int64_t r = 0; r < (int64_t)R; ++r) {
                const uint32_t i = rows ? rows[r] : (uint32_t)r;
                double* o = out + ((bn * C + bc) * (int64_t)R + r) * N;
                for (uint32_t j = 0; j < N; ++j) o[j] = 0.0;
                for (uint32_t k = 0; k < K; ++k) {
                    const double a = (double)at(lhs, bn, bc, i, k);
                    for (uint32_t j = 0; j < N; ++j) o[j] += a * (double)at(rhs, bn, bc, k, j);
                }
            }
    (void)M;
    return 0;
}

/* CPU baseline: restatement of gemm_tiled (vortx-shaders/src/linalg/
 * gemm.rs:41-194) for contiguous row-major A [M,K], B [K,N], C [M,N].
 * One OpenMP task per 64x64 output tile; inside a task the 256
 * "invocations" of a workgroup run one after another between the two
 * barriers, with the same 64x16 / 16x64 staging (padded strides 17 and 65)
 * and the same k order. */
int orc_gemm_tiled_f32_omp(float* c, const float* a, const float* b, uint32_t M,
                           uint32_t N, uint32_t K, int nthreads) {
    enum { TM = 64, TN = 64, TK = 16, SA = TK + 1, SB = TN + 1 };
    const uint32_t tiles_m = (M + TM - 1) / TM, tiles_n = (N + TN - 1) / TN;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < (int64_t)tiles_m * tiles_n; ++t) {
        const uint32_t tile_row = (uint32_t)(t / tiles_n) * TM;
        const uint32_t tile_col = (uint32_t)(t % tiles_n) * TN;
        float sa[TM * SA], sb[TK * SB];
        float acc[TM][TN];
        memset(acc, 0, sizeof(acc));
        for (uint32_t kt = 0; kt < K; kt += TK) {
            for (uint32_t r = 0; r < TM; ++r)
                for (uint32_t q = 0; q < TK; ++q) {
                    const uint32_t gr = tile_row + r, gc = kt + q;
                    sa[r * SA + q] = (gr < M && gc < K) ? a[(uint64_t)gr * K + gc] : 0.0f;
                }
            for (uint32_t r = 0; r < TK; ++r)
                for (uint32_t q = 0; q < TN; ++q) {
                    const uint32_t gr = kt + r, gc = tile_col + q;
                    sb[r * SB + q] = (gr < K && gc < N) ? b[(uint64_t)gr * N + gc] : 0.0f;
                }
            for (uint32_t i = 0; i < TM; ++i)
                for (uint32_t kk = 0; kk < TK; ++kk) {
                    const float av = sa[i * SA + kk];
                    for (uint32_t j = 0; j < TN; ++j) acc[i][j] = acc[i][j] + av * sb[kk * SB + j];
                }
        }
        for (uint32_t i = 0; i < TM; ++i) {
            const uint32_t row = tile_row + i;
            if (row >= M) continue;
            for (uint32_t j = 0; j < TN; ++j) {
                const uint32_t col = tile_col + j;
                if (col < N) c[(uint64_t)row * N + col] = acc[i][j];
            }
        }
    }
    return 0;
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* vortx-shaders/src/linalg/contiguous.rs:70-90 (contiguous_impl): size and
 * stride are the canonical [n, c, h, w] Shape fields; offset is the extra
 * element offset (0 for the plain `contiguous` entry point). u32 index
 * arithmetic like the shader. */
int orc_contiguous_u32(uint32_t* dest, const uint32_t* src, const uint32_t* size, const uint32_t* stride,
                       uint32_t offset) {
    const uint32_t len = size[0] * size[1] * size[2] * size[3];
    const uint32_t h_stride = size[3];
    const uint32_t c_stride = size[2] * size[3];
    const uint32_t n_stride = size[1] * size[2] * size[3];
    for (uint32_t t = 0; t < len; ++t) {
        const uint32_t n = t / n_stride;
        const uint32_t c = (t % n_stride) / c_stride;
        const uint32_t h = (t % c_stride) / h_stride;
        const uint32_t w = t % h_stride;
        const uint32_t it = n * stride[0] + c * stride[1] + h * stride[2] + w * stride[3];
        dest[t] = src[offset + it];
    }
    return 0;
}

/* ------------------------------------------------------------- quantize */
/*
 * ggml MIT license notice (the quantizers below restate ggml's published
 * quantize_row_*_ref / make_qkx2_quants; ggml is distributed under it):
 *
 *   MIT License
 *
 *   Copyright (c) 2023-2024 The ggml authors
 *
 *   Permission is hereby granted, free of charge, to any person obtaining a copy
 *   of this software and associated documentation files (the "Software"), to deal
 *   in the Software without restriction, including without limitation the rights
 *   to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
 *   copies of the Software, and to permit persons to whom the Software is
 *   furnished to do so, subject to the following conditions:
 *
 *   The above copyright notice and this permission notice shall be included in all
 *   copies or substantial portions of the Software.
 *
 *   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR
 *   IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY,
 *   FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT SHALL THE
 *   AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER
 *   LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM,
 *   OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE
 *   SOFTWARE.
 */
/* IEEE binary32 -> binary16, round to nearest even (what ggml's
 * GGML_FP32_TO_FP16 does with F16C or its software path). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const uint32_t exp = (b >> 23) & 0xFFu;
    uint32_t man = b & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    const int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h += 1u;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

/* ggml nearest_int: round half to even through the 1.5 * 2^23 magic. */
static int orc_nearest_int(float fval) {
    const float val = fval + 12582912.f;
    int32_t i;
    memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* ggml make_qkx2_quants (asymmetric 4-bit search over 20 scale candidates,
 * weighted squared error). */
static float orc_make_qkx2(int n, int nmax, const float* x, const float* weights, uint8_t* L, float* the_min,
                           uint8_t* Laux, float rmin, float rdelta, int nstep) {
    float mn = x[0], mx = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -mn;
        return 0.f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        int l = orc_nearest_int(iscale * (x[i] - mn));
        L[i] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
        float diff = scale * L[i] + mn - x[i];
        diff = diff * diff;
        best_mad += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = orc_nearest_int(iscale * (x[i] - mn));
            l = l < 0 ? 0 : l > nmax ? nmax : l;
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
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
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                mad += weights[i] * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

static void orc_put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFFu);
    p[1] = (uint8_t)(v >> 8);
}

static void orc_quant_q8_0(const float* x, uint8_t* y) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(x[j]);
        amax = amax > a ? amax : a;
    }
    const float d = amax / ((1 << 7) - 1);
    const float id = d ? 1.0f / d : 0.0f;
    orc_put16(y, orc_f32_to_f16(d));
    for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

static void orc_quant_q4_0(const float* x, uint8_t* y) {
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float v = x[j];
        if (amax < fabsf(v)) {
            amax = fabsf(v);
            mx = v;
        }
    }
    const float d = mx / -8;
    const float id = d ? 1.0f / d : 0.0f;
    orc_put16(y, orc_f32_to_f16(d));
    for (int j = 0; j < 16; ++j) {
        const float x0 = x[j] * id, x1 = x[16 + j] * id;
        int xi0 = (int8_t)(x0 + 8.5f), xi1 = (int8_t)(x1 + 8.5f);
        xi0 = xi0 < 15 ? xi0 : 15;
        xi1 = xi1 < 15 ? xi1 : 15;
        y[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

/* ggml's search constants for Q4_K sub-blocks (quantize_row_q4_K_ref calls
 * make_qkx2_quants(32, 15, x, weights, L, &min, Laux, -1, 0.1, 20)):
 * candidate inverse scales (15 + rmin + rdelta k) / (max - min), k = 0..20. */
#define ORC_Q4K_RMIN (-1.f)
#define ORC_Q4K_RDELTA 0.1f
#define ORC_Q4K_NSTEP 20

/* One sub-block's scale search, as orc_quant_q4_k runs it (test hook). */
int orc_q4k_fit(const float* x, const float* weights, uint8_t* L, float* scale, float* min) {
    uint8_t Laux[32];
    *scale = orc_make_qkx2(32, 15, x, weights, L, min, Laux, ORC_Q4K_RMIN, ORC_Q4K_RDELTA, ORC_Q4K_NSTEP);
    return 0;
}

static void orc_quant_q4_k(const float* x, uint8_t* y) {
    uint8_t L[256], Laux[32];
    float weights[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = orc_make_qkx2(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, ORC_Q4K_RMIN,
                                  ORC_Q4K_RDELTA, ORC_Q4K_NSTEP);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t* sc = y + 4;
    memset(sc, 0, 12);
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)orc_nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)orc_nearest_int(inv_min * mins[j]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        if (j < 4) {
            sc[j] = ls;
            sc[j + 4] = lm;
        } else {
            sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc[j - 0] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t dh = orc_f32_to_f16(max_scale / 63.f), mh = orc_f32_to_f16(max_min / 63.f);
    orc_put16(y, dh);
    orc_put16(y + 2, mh);
    for (int j = 0; j < 8; ++j) {
        uint8_t scv, mv;
        orc_q4k_scale_min(sc, j, &scv, &mv);
        const float d = orc_f16_to_f32(dh) * scv;
        if (!d) continue;
        const float dm = orc_f16_to_f32(mh) * mv;
        for (int ii = 0; ii < 32; ++ii) {
            int l = orc_nearest_int((x[32 * j + ii] + dm) / d);
            l = l < 0 ? 0 : l > 15 ? 15 : l;
            L[32 * j + ii] = (uint8_t)l;
        }
    }
    uint8_t* q = y + 16;
    for (int j = 0; j < 256; j += 64) {
        for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
        q += 32;
    }
}

/* x: M rows of K f32 (row i at x + i * x_row_stride elements); out: M rows
 * of blocks, row_stride_bytes apart. K must be a multiple of the block. */
int orc_quantize(uint32_t qtype, const float* x, uint32_t M, uint32_t K, uint64_t x_row_stride, uint8_t* out,
                 uint64_t row_stride_bytes) {
    uint32_t qk, bb;
    if (orc_qtype_info(qtype, &qk, &bb)) return -1;
    if (K % qk) return -2;
    for (uint32_t i = 0; i < M; ++i) {
        const float* xr = x + (uint64_t)i * x_row_stride;
        uint8_t* yr = out + (uint64_t)i * row_stride_bytes;
        for (uint32_t b = 0; b < K / qk; ++b) {
            if (qtype == 8) orc_quant_q8_0(xr + (uint64_t)b * 32, yr + (uint64_t)b * 34);
            else if (qtype == 2) orc_quant_q4_0(xr + (uint64_t)b * 32, yr + (uint64_t)b * 18);
            else orc_quant_q4_k(xr + (uint64_t)b * 256, yr + (uint64_t)b * 144);
        }
    }
    return 0;
}

/* ------------------------------------------------------ activation split */
/* The activation format of the library's batched GEMV (vx_quantize_x in
 * include/vortx_hip.h; no reference counterpart: vortx has no quantized
 * path). Column b of x [K, B], 32-element block j, v[i] = x[32 j + i, b]:
 *   m  = max_i |v_i|
 *   s4[q] = (v[4q] + v[4q+1]) + (v[4q+2] + v[4q+3])          q = 0..7
 *   S  = ((s4[0] + s4[1]) + (s4[2] + s4[3])) + ((s4[4] + s4[5]) + (s4[6] + s4[7]))
 *   fin = m < inf and S == S
 *   c1 = m / 126, c2 = c1 / 254, i1 = (fin and m >= 2^-100) ? 126 / m : 0,
 *   i2 = i1 * 254 (every operation one IEEE rounding)
 *   q1_i = clamp(rne(v_i * i1), -127, 127),  r_i = fma(-q1_i, c1, v_i),
 *   q2_i = clamp(rne(r_i * i2), -127, 127)   (rne of the exact product)
 *   (a non-finite block stores q1 = q2 = 0)
 * so x ~= c2 (254 q1 + q2) with |error| <= ~c2 / 2 = max|v| / 64008.
 * Storage: levels int8 [K/32][B][2][32], element i of the block at byte
 * position p(i) = 8 (i / 4) + i % 4 for i < 16 and 8 ((i - 16) / 4) + 4 +
 * (i - 16) % 4 for i >= 16 (the order in which a 32-block's nibbles sit in
 * a Q4_0 block's 16 bytes: byte t holds elements t and t + 16); scales f32
 * [K/32][B][2] = {fin ? c2 : m + S, S}. */
int orc_quantize_x(const float* x, int64_t xs_k, int64_t xs_b, uint32_t K, uint32_t B, int8_t* levels,
                   float* scales) {
    if (K % 32) return -2;
    const uint32_t nblk = K / 32;
    for (uint32_t j = 0; j < nblk; ++j) {
        for (uint32_t b = 0; b < B; ++b) {
            float v[32];
            for (int i = 0; i < 32; ++i) v[i] = x[(int64_t)(32 * j + i) * xs_k + (int64_t)b * xs_b];
            float m = 0.0f;
            for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(v[i]));
            float s4[8];
            for (int q = 0; q < 8; ++q) s4[q] = (v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]);
            const float S = ((s4[0] + s4[1]) + (s4[2] + s4[3])) + ((s4[4] + s4[5]) + (s4[6] + s4[7]));
            const int fin = m < INFINITY && S == S;
            const float c1 = m / 126.0f, c2 = c1 / 254.0f;
            const float i1 = (fin && m >= 0x1p-100f) ? 126.0f / m : 0.0f, i2 = i1 * 254.0f;
            int8_t* l1 = levels + ((size_t)j * B + b) * 64;
            int8_t* l2 = l1 + 32;
            for (int i = 0; i < 32; ++i) {
                const int p = i < 16 ? 8 * (i / 4) + i % 4 : 8 * ((i - 16) / 4) + 4 + (i - 16) % 4;
                float q1 = 0.0f, q2 = 0.0f;
                if (fin) {
                    /* fmaf(p, s, 1.5 * 2^23) - 1.5 * 2^23 is the exact product p s
                     * rounded once to the nearest integer, ties to even (|p s|
                     * stays below ~127, far inside the 2^22 range of the trick) */
                    q1 = fmaf(v[i], i1, 12582912.0f) - 12582912.0f;
                    q1 = q1 < -127.0f ? -127.0f : q1 > 127.0f ? 127.0f : q1;
                    const float r = fmaf(-q1, c1, v[i]);
                    q2 = fmaf(r, i2, 12582912.0f) - 12582912.0f;
                    q2 = q2 < -127.0f ? -127.0f : q2 > 127.0f ? 127.0f : q2;
                }
                l1[p] = (int8_t)q1;
                l2[p] = (int8_t)q2;
            }
            float* sc = scales + ((size_t)j * B + b) * 2;
            sc[0] = fin ? c2 : m + S;
            sc[1] = S;
        }
    }
    return 0;
}
