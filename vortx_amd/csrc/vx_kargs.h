/*
 * vx_kargs.h — kernel argument blocks shared by the host library (g++)
 * and the gfx950 kernels (hipcc). Each kernel takes one of these structs
 * by value; the host passes it to hipModuleLaunchKernel through
 * kernelParams, so the layout must be identical on both sides: only
 * fixed-width integers and pointers, naturally aligned.
 */
#ifndef VX_KARGS_H
#define VX_KARGS_H

#include <stdint.h>

#define VX_WG 256          /* threads per workgroup (4 wave64) */
#define VX_LDS_X_BYTES 65536 /* LDS budget for staged activations */

/* Dense f32 GEMM on canonical [n, c, rows, cols] operands. Base pointers
 * already include each view's element offset. Strides in elements. */
typedef struct vx_gemm_args {
    float* c;
    const float* a;
    const float* b;
    int64_t cs[4];
    int64_t as[4];
    int64_t bs[4];
    uint32_t batch_c;  /* size of dim 1; grid z = n * batch_c */
    uint32_t M, N, K;
    uint32_t tiles_m, tiles_n;
    float alpha, beta;  /* c = alpha * acc + beta * c (c not read when beta == 0) */
} vx_gemm_args;

/* Block-quantized GEMV / dequantize. */
typedef struct vx_gemv_args {
    const uint8_t* w;
    uint64_t row_stride;   /* bytes between rows of W */
    const float* x;        /* x[k, b] at x[k*xs_k + b*xs_b] */
    int64_t xs_k, xs_b;
    float* y;              /* y[m, b] at y[m*ys_m + b*ys_b] */
    int64_t ys_m, ys_b;
    uint32_t M, K, B;      /* B = batch columns handled by this launch */
    uint32_t nunits;       /* K / 64 (units of 64 weights) */
    uint32_t chunk_units;  /* units staged in LDS per chunk */
    uint32_t upitch;       /* LDS pitch (in float4) of one unit-column, odd */
    uint32_t x_vec;        /* 1: x has stride 1 along K and 16-byte aligned rows */
    uint32_t pad0;
} vx_gemv_args;

/* f32 GEMV (the N == 1 route of the GEMM op): y[m] = sum_k A[m,k] x[k]. */
typedef struct vx_gemv_f32_args {
    const float* a;
    int64_t as_m, as_k;
    const float* x;
    int64_t xs_k;
    float* y;
    int64_t ys_m;
    uint32_t M, K;
    uint32_t batch_c;
    float alpha, beta;  /* y = alpha * acc + beta * y (y not read when beta == 0) */
    uint32_t pad0;
    int64_t a_bs[2], x_bs[2], y_bs[2]; /* batch strides (dims n, c) */
} vx_gemv_f32_args;

/* Unsigned division by a fixed divisor d >= 1 (round-up multiplier m and
 * shift s; `one` marks d == 1). */
typedef struct vx_udiv {
    uint32_t m, s, one, pad;
} vx_udiv;

/* Strided -> contiguous copy of 4-byte elements over the canonical
 * [n, c, h, w] view (strides in elements, 64-bit). */
typedef struct vx_copy_args {
    uint32_t* dst;
    const uint32_t* src;
    const uint32_t* dev_offset; /* null, or a device u32 added to every source index */
    int64_t stride[4];
    uint32_t size[4];
    uint32_t total;             /* elements (< 2^32) */
    uint32_t pad0;
    vx_udiv dw, dh, dc;         /* divisions by size[3], size[2], size[1] */
} vx_copy_args;

/* f32 [M, K] -> quantized blocks (row i at out + i * row_stride). */
typedef struct vx_quant_args {
    const float* x;
    int64_t xs_m, xs_k;
    uint8_t* out;
    uint64_t row_stride;
    uint32_t M, K;
    uint32_t nblk;   /* blocks (Q4_K: super-blocks) per row */
    uint32_t x_vec;  /* 1: xs_k == 1 and 16-byte aligned rows */
} vx_quant_args;

/* Activation split x [K, B] f32 -> levels int8 [nblk][B][2][32] and scales
 * f32 [nblk][B][2] (the layout of vx_xq in include/vortx_hip.h). */
typedef struct vx_xq_args {
    const float* x;        /* x[k, b] at x[k*xs_k + b*xs_b] */
    int64_t xs_k, xs_b;
    int8_t* levels;
    float* scales;
    uint32_t K, B;
    uint32_t nblk;         /* K / 32 */
    uint32_t x_vec;        /* 1: xs_k == 1, 16-byte aligned columns */
} vx_xq_args;

/* Batched GEMV on split activations: y[m, b] = sum_k W[m, k] x[k, b]. */
typedef struct vx_gemv_xq_args {
    const uint8_t* w;
    uint64_t row_stride;   /* bytes between rows of W */
    const int8_t* levels;  /* the vx_xq levels of x */
    const float* scales;   /* the vx_xq scales of x */
    float* y;              /* y[m, b] at y[m*ys_m + b*ys_b] */
    int64_t ys_m, ys_b;
    uint32_t M, K, B;      /* B: columns of this launch, <= 16 */
    uint32_t nblk;         /* K / 32 */
    uint32_t nunits;       /* K / 64 */
    uint32_t ipr;          /* items (256 weights) per row, the last one possibly partial */
    uint32_t npass;        /* passes over K: ceil(ipr / (16 * items per wave)) */
    uint32_t xcols;        /* columns of the split x (its layout pitch) */
    uint32_t col0;         /* first split-x column of this launch (y is already offset) */
    uint32_t pad0;
    const float* x;        /* kernels that split x themselves (_fx): x[k, b] at x[k + b*xs_b] */
    int64_t xs_b;
} vx_gemv_xq_args;

/* Bytes of the device scratch array of vx_gemv_q_noalloc (vx_scratch in
 * the GEMV code object): the largest activation split it can hold. */
#define VX_SCRATCH_BYTES (4u << 20)

#endif /* VX_KARGS_H */
