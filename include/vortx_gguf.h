/*
 * vortx_gguf.h — GGUF model-file reader of libvortx_hip.so.
 *
 * The reference has no file format for quantized weights (its GGML support
 * is the dimension convention GGML_IDS, src/shapes.rs:15-18, and the
 * size_ggml / stride_ggml accessors, src/tensor/tensor_impl.rs:159-171).
 * This reader feeds GGUF files (the llama.cpp / ggml container, versions 2
 * and 3, little-endian) to vx_gemv_q: it maps the file, validates every
 * header field against the file size, exposes the metadata and the tensor
 * table, streams tensor data into caller-owned device memory, and turns a
 * tensor into a vx_qweight or an f32 view.
 *
 * File layout (the public GGUF specification):
 *   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
 *   n_kv x { string key, u32 value_type, value },
 *   n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type,
 *                 u64 offset },
 *   padding to `general.alignment` (u32 metadata key, default 32),
 *   data section; tensor i lives at data_offset + offset_i.
 * A string is u64 length + bytes (no terminator). An array value is
 * u32 element type + u64 count + elements.
 *
 * All functions return a vx_status from vortx_hip.h; the reason for a
 * failure is in vx_last_error_message(). Host-only functions (everything
 * except vx_gguf_upload) make no HIP call and run without a GPU.
 */
#ifndef VORTX_GGUF_H
#define VORTX_GGUF_H

#include <stdint.h>

#include "vortx_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF metadata value types (the specification's gguf_type). */
typedef enum vx_gguf_type {
    VX_GGUF_UINT8 = 0,
    VX_GGUF_INT8 = 1,
    VX_GGUF_UINT16 = 2,
    VX_GGUF_INT16 = 3,
    VX_GGUF_UINT32 = 4,
    VX_GGUF_INT32 = 5,
    VX_GGUF_FLOAT32 = 6,
    VX_GGUF_BOOL = 7,
    VX_GGUF_STRING = 8,
    VX_GGUF_ARRAY = 9,
    VX_GGUF_UINT64 = 10,
    VX_GGUF_INT64 = 11,
    VX_GGUF_FLOAT64 = 12
} vx_gguf_type;

/* An open, mapped GGUF file. Immutable after vx_gguf_open: every query may
 * run concurrently; vx_gguf_close must not overlap any other call. */
typedef struct vx_gguf_file* vx_gguf;

typedef struct vx_gguf_header {
    uint32_t version;      /* 2 or 3 */
    uint32_t reserved;
    uint64_t n_tensors;
    uint64_t n_kv;
    uint64_t alignment;    /* general.alignment, default 32 */
    uint64_t data_offset;  /* file offset of the data section */
    uint64_t data_size;    /* file size - data_offset (0 without tensors) */
    uint64_t file_size;
} vx_gguf_header;

typedef struct vx_gguf_tensor {
    const char* name;      /* NUL-terminated, owned by the handle */
    uint32_t n_dims;       /* 1..4 */
    uint32_t type;         /* ggml type id (VX_Q4_0, VX_Q8_0, VX_Q4_K, 0 = F32, ...) */
    uint64_t ne[4];        /* ggml order: ne[0] is the innermost dimension; 1 past n_dims */
    uint64_t offset;       /* bytes from the start of the data section */
    uint64_t nbytes;       /* 0 when size_known == 0 */
    uint32_t size_known;   /* 1 when this reader knows the type's block size */
    uint32_t reserved;
    const void* data;      /* host address inside the mapping (NULL if !size_known) */
} vx_gguf_tensor;

typedef struct vx_gguf_kv {
    const char* key;       /* NUL-terminated, owned by the handle */
    uint32_t type;         /* a vx_gguf_type */
    uint32_t elem_type;    /* arrays: the element type; otherwise == type */
    uint64_t count;        /* arrays: element count; otherwise 1 */
    /* Scalars and arrays of fixed-size elements: the little-endian values
     * inside the mapping (NOT aligned: copy them out with memcpy); strings
     * and arrays of strings or arrays: NULL (use vx_gguf_kv_string). */
    const void* data;
    uint64_t nbytes;       /* bytes at data */
} vx_gguf_kv;

/* Maps and validates `path`. Fails with VX_ERR_IO when the file cannot be
 * opened or mapped, VX_ERR_FORMAT when it is not a well-formed GGUF v2/v3
 * little-endian file: bad magic or version, a field running past the end
 * of the file, general.alignment not a power of two, duplicate keys or
 * tensor names, n_dims outside 1..4, element counts that overflow, a
 * tensor offset that is not a multiple of the alignment, or tensor data
 * past the end of the file. */
int vx_gguf_open(const char* path, vx_gguf* out);
int vx_gguf_close(vx_gguf file);

int vx_gguf_get_header(vx_gguf file, vx_gguf_header* out);

/* Tensor `index` (0 <= index < n_tensors), in file order. */
int vx_gguf_tensor_info(vx_gguf file, uint64_t index, vx_gguf_tensor* out);
/* VX_ERR_NOT_FOUND when no tensor has that name. */
int vx_gguf_find_tensor(vx_gguf file, const char* name, uint64_t* index);

/* Metadata entry `index` (0 <= index < n_kv), in file order. */
int vx_gguf_kv_info(vx_gguf file, uint64_t index, vx_gguf_kv* out);
/* VX_ERR_NOT_FOUND when no key has that name. */
int vx_gguf_find_key(vx_gguf file, const char* key, uint64_t* index);
/* The bytes of a string value (elem == 0) or of element `elem` of an array
 * of strings; not NUL-terminated. VX_ERR_INVALID for other types. */
int vx_gguf_kv_string(vx_gguf file, uint64_t index, uint64_t elem, const char** str, uint64_t* len);

/* Block geometry of a ggml type: (elements per block, bytes per block).
 * VX_ERR_UNSUPPORTED for a type this reader has no size for. */
int vx_gguf_type_size(uint32_t ggml_type, uint32_t* block_elems, uint32_t* block_bytes);

/* Copies bytes [offset, offset + nbytes) of the data section into device
 * memory at `device_dst` (any device address of the context's device).
 * Two host threads (VX_GGUF_UPLOAD_THREADS, 1..64, overrides) each pread
 * 16 MB chunks of the file into two pinned staging buffers of their own
 * (hipHostMalloc, allocated per call) and copy them with hipMemcpyAsync on a
 * stream of their own, so reading the file overlaps the DMA. Those streams first wait for the work already queued
 * on `stream`; the call returns after every copy has completed and the
 * staging is freed. Uploading the whole data section once (offset 0,
 * nbytes = data_size) keeps every tensor at device_dst + tensor.offset
 * with the file's alignment. VX_ERR_IO if the file cannot be read. */
int vx_gguf_upload(vx_ctx ctx, vx_stream stream, vx_gguf file, uint64_t offset, uint64_t nbytes,
                   void* device_dst);

/* The vx_qweight of quantized tensor `index` whose data section was
 * uploaded to `device_data` (so the tensor is at device_data + offset):
 * rows = ne[1], cols = ne[0], dense row stride. Requires type Q4_0, Q8_0
 * or Q4_K, ne[2] == ne[3] == 1 and rows, cols < 2^32 (VX_ERR_UNSUPPORTED). */
int vx_gguf_qweight(vx_gguf file, uint64_t index, const void* device_data, vx_qweight* out);

/* A read-only f32 view of F32 tensor `index` uploaded as above, in vortx's
 * GGML dimension convention (GGML_IDS = [1, 0, 2, 3], src/shapes.rs:15-18):
 * rank = n_dims, size[GGML_IDS[i]] = ne[i] and stride[GGML_IDS[i]] = the
 * ggml element stride of dim i (ne[0] is contiguous). A 2-D tensor with
 * ne = [K, M] is the row-major [M, K] matrix; a 1-D tensor is [ne[0]].
 * VX_ERR_UNSUPPORTED for other types or sizes/strides >= 2^32. */
int vx_gguf_view(vx_gguf file, uint64_t index, const void* device_data, vx_cview* out);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* VORTX_GGUF_H */
