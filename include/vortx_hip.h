/*
 * vortx_hip.h — C ABI of the MI355X (gfx950) linalg hot path.
 *
 * Drop-in boundary for vortx's GEMM op on tensor views
 * (reference: src/linalg/gemm.rs:34-321, src/shapes.rs:51-60) plus a
 * GGUF block-quantized dequant-GEMV (Q8_0, Q4_0, Q4_K) that the reference
 * does not have. Plain pointers and sizes only; no C++ or HIP types cross
 * this boundary. Device pointers are HIP device addresses; streams are
 * hipStream_t values passed as void*.
 *
 * Conventions shared by every entry point:
 *  - Every function returns a vx_status (0 == VX_OK). Nothing throws.
 *    vx_last_error_message() gives a human-readable reason for the last
 *    failure on the calling thread; vx_last_hip_error() the hipError_t.
 *  - Launches are asynchronous on the given stream (NULL = null stream).
 *    The caller keeps every buffer alive until the stream work completes;
 *    the library never frees or retains caller memory.
 *  - A vx_ctx is immutable after vx_init and may be shared by threads and
 *    streams (as the reference's `Gemm` is `&self`). No entry point of this
 *    header allocates, frees or synchronizes device memory after vx_init,
 *    except vx_gemv_q_noalloc's shared scratch array (see there): memory a
 *    call needs beyond its operands is passed in by the caller
 *    (vx_gemv_q_ws), like the reference's caller-owned
 *    `shapes: &mut TensorLayoutBuffers` (src/linalg/gemm.rs:47-56).
 */
#ifndef VORTX_HIP_H
#define VORTX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* Status codes                                                        */
/* ------------------------------------------------------------------ */
typedef enum vx_status {
    VX_OK = 0,
    /* Operand shapes are incompatible. The reference panics on the same
     * condition (assert_eq!, src/linalg/gemm.rs:70-104); a Rust shim maps
     * this code to panic!. */
    VX_ERR_SHAPE = 1,
    /* Valid request that this build does not support (rank > 4, an index
     * beyond 2^63, K not a multiple of the block size, ...). */
    VX_ERR_UNSUPPORTED = 2,
    /* Invalid argument: NULL pointer, unknown quant type, bad axis. */
    VX_ERR_INVALID = 3,
    /* A HIP runtime call failed; vx_last_hip_error() returns its code.
     * Maps to the reference's Err(GpuBackendError). */
    VX_ERR_HIP = 4,
    /* The embedded gfx950 code object failed to load (hipModuleLoadData). */
    VX_ERR_NO_CODE_OBJECT = 5,
    /* A file could not be opened, sized or mapped (vortx_gguf.h). */
    VX_ERR_IO = 6,
    /* A file is not a well-formed GGUF file (vortx_gguf.h). */
    VX_ERR_FORMAT = 7,
    /* No tensor or metadata key of the requested name (vortx_gguf.h). */
    VX_ERR_NOT_FOUND = 8
} vx_status;

/* ------------------------------------------------------------------ */
/* Tensor views                                                        */
/* ------------------------------------------------------------------ */

/* Byte-compatible with vortx's TensorLayout (src/shapes.rs:51-60):
 * sizes and strides in ELEMENTS, row-major, rank <= 4, offset in elements
 * from the buffer base. Dimensions at index >= rank are ignored. */
typedef struct vx_layout {
    uint32_t size[4];
    uint32_t stride[4];
    uint32_t rank;
    uint32_t offset;
} vx_layout;

/* Read-only f32 view = TensorRef<f32> (src/tensor/tensor_ref.rs:11-14).
 * `base` is the buffer start; the element at index (i0,i1,i2,i3) lives at
 * base[offset + sum_k i_k * stride[k]] (offset applied like
 * TensorRef::buffer(), src/tensor/tensor_ref.rs:101-103). */
typedef struct vx_cview {
    const float* base;
    vx_layout layout;
} vx_cview;

/* Writable f32 view = TensorMut<f32> (src/tensor/tensor_mut.rs:10-13). */
typedef struct vx_mview {
    float* base;
    vx_layout layout;
} vx_mview;

/* GGML type ids of the supported block formats. */
typedef enum vx_qtype {
    VX_Q4_0 = 2,  /* 32 weights / 18 bytes: f16 d, 16 B of nibbles      */
    VX_Q8_0 = 8,  /* 32 weights / 34 bytes: f16 d, 32 int8              */
    VX_Q4_K = 12  /* 256 weights / 144 bytes: f16 d, f16 dmin, 12 B of
                     6-bit scales/mins, 128 B of nibbles               */
} vx_qtype;

/* A row-major block-quantized matrix W[rows, cols]: each row is cols/QK
 * consecutive blocks, rows are row_stride_bytes apart. This is a GGUF
 * tensor with ne = [cols, rows] (vortx maps ggml dim 0 to its column
 * dimension: GGML_IDS, src/shapes.rs:15-18). */
typedef struct vx_qweight {
    const void* base;
    uint32_t qtype;             /* a vx_qtype */
    uint32_t rows;              /* M */
    uint32_t cols;              /* K, a multiple of the block size */
    uint32_t reserved;          /* must be 0 */
    uint64_t row_stride_bytes;  /* >= (cols/QK) * block_bytes */
} vx_qweight;

typedef struct vx_context* vx_ctx;
typedef void* vx_stream; /* hipStream_t */

/* ------------------------------------------------------------------ */
/* Context                                                             */
/* ------------------------------------------------------------------ */

/* Loads the embedded gfx950 code objects on `device` (hipModuleLoadData)
 * and resolves every kernel. Counterpart of Gemm::from_backend (khal
 * #[derive(Shader)], used at src/linalg/gemm.rs:366). */
int vx_init(int device, vx_ctx* out_ctx);
int vx_destroy(vx_ctx ctx);
/* Device ordinal and compute-unit count the context was built for. */
int vx_device_info(vx_ctx ctx, int* device, int* num_cus);

/* ------------------------------------------------------------------ */
/* GEMM: out = lhs * rhs, f32                                          */
/* ------------------------------------------------------------------ */

/* Replaces Gemm::dispatch (src/linalg/gemm.rs:47-187). Each view is
 * canonicalized to rank 4 [n, c, rows, cols] (TensorLayout::canonicalize,
 * src/shapes.rs:145-155); n and c must match across the three operands,
 * out is [.., M, N], lhs [.., M, K], rhs [.., K, N]. Arbitrary strides
 * (transposed views included). Kernel choice by shape: the naive kernel
 * when M < 32 and N < 32 (the reference's rule, :111-112), an f32 GEMV
 * when N == 1, otherwise the MFMA tiled kernel. out is only written. */
int vx_gemm_f32(vx_ctx ctx, vx_stream stream, const vx_mview* out,
                const vx_cview* lhs, const vx_cview* rhs);

/* Replaces Gemm::dispatch_naive (src/linalg/gemm.rs:190-246): forces the
 * one-thread-per-output kernel with sequential-k f32 accumulation (the
 * order of gemm_naive, vortx-shaders/src/linalg/gemm.rs:196-237). Unlike
 * the reference this variant validates shapes. */
int vx_gemm_f32_naive(vx_ctx ctx, vx_stream stream, const vx_mview* out,
                      const vx_cview* lhs, const vx_cview* rhs);

/* Replaces Gemm::dispatch_tiled (src/linalg/gemm.rs:249-305): forces the
 * MFMA tiled kernel (never the GEMV route). Validates shapes. */
int vx_gemm_f32_tiled(vx_ctx ctx, vx_stream stream, const vx_mview* out,
                      const vx_cview* lhs, const vx_cview* rhs);

/* Options of vx_gemm_f32_ex. */
typedef enum vx_gemm_flags {
    /* Batch dims broadcast: after canonicalization (rank 4, leading 1s),
     * each of lhs's and rhs's dims 0 and 1 may be 1 where out's is larger;
     * that operand is then reused along the dim (stride 0), the semantics
     * of TensorLayout::broadcast (src/shapes.rs:346-391) that the reference
     * leaves as a TODO in Gemm::dispatch (src/linalg/gemm.rs:64). */
    VX_GEMM_BROADCAST = 1,
    /* Tile shape of the MFMA kernel, for callers that pin it (all give the
     * same bits; by default the one that fills the GPU best is taken):
     * 128 x 128, 128 x 256 or 64 x 64 output tiles. Exclusive; ignored on
     * the naive and GEMV routes; WIDE and SMALL apply to operands whose A is
     * contiguous along K and B along K or N (others keep 128 x 128). */
    VX_GEMM_TILE_NARROW = 2,
    VX_GEMM_TILE_WIDE = 4,
    VX_GEMM_TILE_SMALL = 8
} vx_gemm_flags;

typedef struct vx_gemm_opts {
    float alpha;       /* out = alpha * (lhs x rhs) + beta * out */
    float beta;        /* 0: out is only written (NaN / inf in out do not propagate) */
    uint32_t flags;    /* bitwise OR of vx_gemm_flags */
    uint32_t reserved; /* must be 0 */
} vx_gemm_opts;

/* Gemm::dispatch with an alpha / beta epilogue and optional batch
 * broadcasting (no reference counterpart: the reference's out is only
 * written, :70-104 require equal batch dims). Same routes and kernels as
 * vx_gemm_f32; opts == NULL means alpha 1, beta 0, no flags, which is
 * vx_gemm_f32. out must not overlap itself (a dim of size > 1 with stride
 * 0 is VX_ERR_INVALID). With beta != 0 each output element is read once
 * before it is written. */
int vx_gemm_f32_ex(vx_ctx ctx, vx_stream stream, const vx_mview* out,
                   const vx_cview* lhs, const vx_cview* rhs, const vx_gemm_opts* opts);

/* Kernel route vx_gemm_f32 takes for these views, without launching
 * (host logic only; usable without a GPU). */
typedef enum vx_gemm_route {
    VX_ROUTE_NAIVE = 0,
    VX_ROUTE_TILED = 1,
    VX_ROUTE_GEMV = 2,
    VX_ROUTE_EMPTY = 3 /* M, N or a batch size is 0: nothing to launch */
} vx_gemm_route;
int vx_gemm_f32_route(const vx_mview* out, const vx_cview* lhs,
                      const vx_cview* rhs, int* route);

/* ------------------------------------------------------------------ */
/* Block-quantized GEMV: y = W * x   (no reference counterpart)        */
/* ------------------------------------------------------------------ */

/* y[m, b] = sum_k W[m, k] * x[k, b] with W decoded exactly from its
 * blocks. y is an [M, B] view, x a [K, B] view (rank 1 views mean B = 1);
 * any strides. Fast path: x with stride 1 along K (activations stored
 * [B, K]). Same operand roles as Gemm::dispatch(out = y, lhs = W, rhs = x).
 * Arithmetic: this is vx_gemv_q_ex with flags 0, so x is NOT kept in f32:
 * each 32-element block of each column is rounded to two int8 levels with
 * one f32 scale (|error| <= ~1.6e-5 of the block's max|x|), the products
 * with the weights are exact int32 and the scaling and accumulation are
 * f32. vx_gemv_q_ex(..., VX_GEMV_X_F32) keeps x in f32.
 * Batches (B >= 2) run on the int8 matrix cores; where the GEMV kernel
 * can split x itself (2 <= B <= 8, K <= 4096 — one 256-element item per
 * wave — and x of stride 1 along K with 16-byte aligned columns) that is one
 * launch. Other batched shapes need the split in device memory: this entry
 * point has none, so they are computed with x kept in f32 (the
 * VX_GEMV_X_F32 kernels); vx_gemv_q_ws with a caller workspace keeps the
 * int8 split there (the fused and the two-launch route give the same bits).
 * Empty shapes: K = 0 writes y = 0 (as vx_gemm_f32 with K = 0); M = 0 or
 * B = 0 returns VX_OK and launches nothing. The same holds for _ex, _ws
 * and _noalloc; vx_gemv_q_xq also returns VX_OK for M = 0 or B = 0 but
 * refuses K = 0 (VX_ERR_UNSUPPORTED), and vx_dequantize of 0 rows is a
 * no-op.
 * Uses no memory beyond its operands; safe to call concurrently on any
 * streams, and to capture. */
int vx_gemv_q(vx_ctx ctx, vx_stream stream, const vx_mview* y,
              const vx_qweight* w, const vx_cview* x);

/* vx_gemv_q with options; flags is a bitwise OR of vx_gemv_flags.
 * By default x is split, per 32-element block of each column, into two
 * int8 levels with one f32 scale, x ~= c (254 x1 + x2), |error| <= c/2 ~
 * 1.6e-5 max|x_block|; products and block sums with the exactly decoded
 * weights are exact in int32 and the scaling is f32. Batch 1 reduces with
 * v_dot4_i32_i8, batches (B >= 2) on the int8 matrix cores. VX_GEMV_X_F32
 * keeps x in f32 instead (f32 FMA on the exactly decoded weights; slower);
 * VX_GEMV_X_INT8 names the default split and may not be combined with it. */
typedef enum vx_gemv_flags { VX_GEMV_X_INT8 = 1, VX_GEMV_X_F32 = 2 } vx_gemv_flags;
/* With VX_GEMV_X_INT8, a batched shape whose split needs device memory
 * (see vx_gemv_q) returns VX_ERR_UNSUPPORTED here instead of falling back
 * to f32 x. */
int vx_gemv_q_ex(vx_ctx ctx, vx_stream stream, const vx_mview* y,
                 const vx_qweight* w, const vx_cview* x, uint32_t flags);

/* vx_gemv_q_ex with a device workspace owned by the caller. No counterpart
 * in the reference (it has no quantized code); the workspace plays the part
 * of Gemm::dispatch's caller-owned `shapes: &mut TensorLayoutBuffers`
 * (src/linalg/gemm.rs:47-56): per-caller mutable state kept outside the
 * (immutable) context. Where a batched call needs its activation split in
 * memory (see vx_gemv_q), x is split into `workspace` by the vx_quantize_x
 * kernel and the GEMV reads it (two launches on `stream`); elsewhere the
 * workspace is not touched. workspace: device memory, 16-byte aligned, at
 * least vx_gemv_q_ws_size(...) bytes (a smaller non-NULL workspace is
 * VX_ERR_INVALID; NULL behaves as vx_gemv_q_ex). The library never
 * allocates, frees or retains it; its contents need not start at zero.
 * Calls that share one workspace must be ordered (one stream, or events);
 * calls with different workspaces may run concurrently on any streams of
 * one context. A captured HIP graph records the workspace address: keep the
 * buffer alive and unshared while the graph can be replayed. */
int vx_gemv_q_ws(vx_ctx ctx, vx_stream stream, const vx_mview* y,
                 const vx_qweight* w, const vx_cview* x, uint32_t flags,
                 void* workspace, uint64_t workspace_bytes);

/* Workspace bytes vx_gemv_q_ws may use for W of `qtype` with K columns
 * and B batch columns under `flags`: vx_xq_size(K, B) for the int8 route at
 * B >= 2 (K a multiple of 64), else 0 (it needs none). */
int vx_gemv_q_ws_size(uint32_t qtype, uint32_t K, uint32_t B, uint32_t flags,
                      uint64_t* bytes);

/* ---- activation split: x -> two int8 levels per 32-block (VX_XQ) -----
 * No counterpart in the reference (it has no quantized code): the step
 * before the batched GEMV, done once per x so that every CU of the GEMV
 * reads 2.25 bytes per element instead of re-splitting 4.
 * Column b of x [K, B], 32-element block j, values v[0..31]:
 *   m = max|v|, S = sum v (pairs within each 4, then the 8 partial sums
 *   pairwise), c1 = m / 126, c2 = c1 / 254, i1 = 126 / m (0 when m < 2^-100
 *   or the block holds a NaN / inf), i2 = 254 i1,
 *   q1 = clamp(rne(v i1), +-127), q2 = clamp(rne(fma(-q1, c1, v) i2), +-127)
 * (every operation one IEEE f32 rounding), so x ~= c2 (254 q1 + q2) with
 * |error| <= ~max|v| / 64008 per element. Element i of a block sits at
 * position p(i) = 8 (i/4) + i%4 (i < 16) or 8 ((i-16)/4) + 4 + i%4 (i >= 16),
 * the order of a Q4_0 block's nibbles. Layout in one device buffer, with
 * NI = ceil(K / 256) items of 8 blocks:
 *   levels int8 at byte 0: level L of column b, block j, position p at
 *     (j/8) B 512 + ((j%8)/2) B 128 + (p/8) B 32 + b 32 + L 16 + (j%2) 8
 *     + p%8 (the 16 bytes one matrix-core lane takes from a block pair lie
 *     together, and the lanes of one load read consecutive 16-byte pieces;
 *     blocks past K/32 in the last item are unused);
 *   scales f32 [K/32][B][2] at byte NI B 512: {c2, S}, or {m + S, S}
 *     (non-finite) for a block holding a NaN or inf.
 * The bytes are deterministic and equal a sequential CPU evaluation of the
 * formulas (the tests check them byte for byte). */
typedef struct vx_xq {
    void* base;   /* device buffer, 16-byte aligned, >= vx_xq_size(K, B) bytes */
    uint32_t K;   /* elements per column, a multiple of 32 */
    uint32_t B;   /* columns */
} vx_xq;

/* Bytes of the vx_xq of a [K, B] x: ceil(K/256) * B * 512 + (K/32) * B * 8
 * (72 bytes per 32 elements when K is a multiple of 256). VX_ERR_UNSUPPORTED
 * when K is not a multiple of 32. */
int vx_xq_size(uint32_t K, uint32_t B, uint64_t* bytes);

/* Write the split of x (a [K, B] f32 view, any strides; rank 1 means B = 1)
 * into out. Asynchronous on `stream`. */
int vx_quantize_x(vx_ctx ctx, vx_stream stream, const vx_xq* out, const vx_cview* x);

/* y = W x with x given by its split (written by vx_quantize_x; out->K ==
 * w->cols): the batched GEMV without the split, for callers that reuse one
 * x for several matrices (a layer's q / k / v or gate / up projections) and
 * quantize it once. y is an [M, B] view, any strides. Needs K a multiple
 * of 64 and W rows 4-byte aligned, else VX_ERR_UNSUPPORTED. Products of the
 * levels with the exactly decoded weights are exact int32 on the int8
 * matrix cores; scaling and accumulation are f32. The library allocates
 * nothing here. */
int vx_gemv_q_xq(vx_ctx ctx, vx_stream stream, const vx_mview* y,
                 const vx_qweight* w, const vx_xq* x);

/* vx_gemv_q_ws without a caller workspace, allocating nothing. No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc) yet want the int8 split at every batched shape. Same
 * arguments and flags as vx_gemv_q_ex, and the kernels and results of
 * vx_gemv_q_ws: where that one splits x into the caller's workspace
 * (B >= 2), this one uses a fixed
 * device array of VX_NOALLOC_SCRATCH_BYTES (4 MiB) that the library's GEMV
 * code object holds per context from vx_init to vx_destroy, so the split of
 * x, vx_xq_size(K, B) bytes (72 per 32 elements of x), must fit it (else
 * VX_ERR_UNSUPPORTED, nothing launched): B = 16 up to K = 116480, B = 64 up
 * to K = 28928. Every call on
 * one context uses the same array: calls that overlap in time on one
 * context race (serialize them on one stream, or use one context per
 * stream); nothing in it needs to start at zero. */
#define VX_NOALLOC_SCRATCH_BYTES (4u << 20)
int vx_gemv_q_noalloc(vx_ctx ctx, vx_stream stream, const vx_mview* y,
                      const vx_qweight* w, const vx_cview* x, uint32_t flags);

/* Measurement only, no counterpart in the reference: the loads of the
 * batch-1 GEMV (vx_gemv_q at B = 1) with nothing else — the same grid, row
 * order, per-lane 64-weight units and preloaded kernel arguments, one item
 * per wave in flight (the GEMV's ring for K <= 4096), no x, no barrier, no
 * arithmetic. Reads every byte of W once and
 * writes one word per row to y[0..M) (contents unspecified). Its time is
 * the ceiling of what that access pattern streams in one launch. Needs K a
 * multiple of 64 and 4-byte aligned rows (else VX_ERR_UNSUPPORTED). */
int vx_gemv_q_read_probe(vx_ctx ctx, vx_stream stream, const vx_qweight* w,
                         float* y);

/* Measurement only, no counterpart in the reference: one launch of an
 * empty kernel on the batch-1 GEMV's grid (one workgroup of 1024 threads
 * per CU) with its preloaded kernel arguments. Its time per launch in a
 * replayed HIP graph is the fixed cost of such a launch on this device, the
 * floor under every per-step time of the batch-1 GEMV. */
int vx_launch_floor(vx_ctx ctx, vx_stream stream);

/* out[m, k] = W[m, k] decoded to f32 (bit-exact: every block value is
 * exactly representable in f32). out is an [M, K] view, any strides. */
int vx_dequantize(vx_ctx ctx, vx_stream stream, const vx_mview* out,
                  const vx_qweight* w);

/* ---- quantize: f32 -> Q8_0 / Q4_0 / Q4_K -----------------------------
 * No counterpart in the reference (it has no quantized code): the step
 * before the GEMV. x is an [rows, cols] f32 view (any strides); the blocks
 * of row i are written at out->base + i * out->row_stride_bytes. The
 * algorithms are ggml's reference quantizers (ggml-quants.c
 * quantize_row_q8_0_ref / quantize_row_q4_0_ref / quantize_row_q4_K_ref,
 * the latter with make_qkx2_quants), evaluated in their f32 operation order
 * without contraction, so the bytes equal a sequential CPU run of the same
 * algorithm. The output must be 2-byte aligned (Q4_K: 4-byte) or
 * VX_ERR_UNSUPPORTED. Asynchronous on `stream`. */
int vx_quantize(vx_ctx ctx, vx_stream stream, const vx_qweight* out,
                const vx_cview* x);

/* ---- strided -> contiguous copy (4-byte elements) --------------------
 * Replaces Contiguous::launch (src/linalg/contiguous.rs:22-119; shader
 * vortx-shaders/src/linalg/contiguous.rs:59-90): out[i] = src[it(n,c,h,w)]
 * over the canonicalized src view, i the row-major index. out must have the
 * same size array as src and a contiguous layout (VX_ERR_SHAPE otherwise,
 * where the reference panics). dev_offset is the optional `offset` tensor:
 * null reads src at its view offset (TensorRef::buffer); non-null reads the
 * raw buffer at the device u32 *dev_offset, ignoring the view offset
 * (TensorRef::raw_buffer), as the reference does. Elements are copied as
 * bits (f32, i32, u32 alike); indices are 64-bit (the shader's u32 index
 * wraps past 2^32 elements); views of 2^32 elements or more return
 * VX_ERR_UNSUPPORTED. Asynchronous on `stream`. */
int vx_contiguous(vx_ctx ctx, vx_stream stream, const vx_mview* out,
                  const vx_cview* src, const uint32_t* dev_offset);

/* Block geometry of a vx_qtype: weights per block and bytes per block. */
int vx_qtype_info(uint32_t qtype, uint32_t* block_weights,
                  uint32_t* block_bytes);

/* ------------------------------------------------------------------ */
/* Layout algebra (host only) — TensorLayout, src/shapes.rs            */
/* ------------------------------------------------------------------ */

/* TensorLayout::contiguous (src/shapes.rs:85-99). rank <= 4. */
int vx_layout_contiguous(const uint32_t* size, uint32_t rank, vx_layout* out);
/* TensorLayout::canonicalize (src/shapes.rs:145-155): prepend size-1
 * dims to rank 4; the offset is reset to 0 exactly as the reference does
 * (the view offset is carried by the buffer slice instead). */
int vx_layout_canonicalize(const vx_layout* in, vx_layout* out);
/* TensorLayout::transpose (src/shapes.rs:238-254). */
int vx_layout_transpose(const vx_layout* in, uint32_t axis_a,
                        uint32_t axis_b, vx_layout* out);
/* TensorLayout::broadcast (src/shapes.rs:346-391): VX_ERR_SHAPE when the
 * shapes are incompatible (the reference returns None). */
int vx_layout_broadcast(const vx_layout* a, const vx_layout* b,
                        vx_layout* a_out, vx_layout* b_out);
/* TensorLayout::view (src/shapes.rs:407-441). `strides` may be NULL; a
 * stride of 0xFFFFFFFF means None (use the contiguous default). */
int vx_layout_view(const vx_layout* in, uint32_t offset,
                   const uint32_t* shape, uint32_t rank,
                   const uint32_t* strides, uint32_t nstrides, vx_layout* out);
/* TensorLayout::narrow (src/shapes.rs:443-464). */
int vx_layout_narrow(const vx_layout* in, uint32_t axis, uint32_t first,
                     uint32_t count, vx_layout* out);
/* TensorLayout::unsqueeze (src/shapes.rs:161-178). */
int vx_layout_unsqueeze(const vx_layout* in, uint32_t axis, vx_layout* out);
/* TensorLayout::is_contiguous (src/shapes.rs:332-343): 1 or 0. */
int vx_layout_is_contiguous(const vx_layout* in);

/* ------------------------------------------------------------------ */
/* Errors                                                              */
/* ------------------------------------------------------------------ */
const char* vx_status_string(int status);
/* Message of the last failure on this thread ("" if none). */
const char* vx_last_error_message(void);
/* hipError_t of the last VX_ERR_HIP on this thread (0 if none). */
int vx_last_hip_error(void);

#ifdef __cplusplus
}
#endif

#endif /* VORTX_HIP_H */
