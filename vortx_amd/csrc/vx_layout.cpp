// vx_layout.cpp — TensorLayout view algebra (host only), restating the
// semantics of vortx's src/shapes.rs for the C ABI: row-major element
// strides, rank <= 4, offset in elements.
#include <cstring>

#include "vx_internal.hpp"

namespace vx {

// TensorLayout::contiguous (src/shapes.rs:85-99): sizes beyond the rank are
// 1; strides are row-major products, 1 beyond the rank.
int layout_contiguous(const uint32_t* size, uint32_t rank, vx_layout* out) {
    if (rank > 4) return fail(VX_ERR_UNSUPPORTED, "tensors of ranks > 4 not supported");
    if (rank && !size) return fail(VX_ERR_INVALID, "null size");
    vx_layout l{};
    for (int k = 0; k < 4; ++k) {
        l.size[k] = 1;
        l.stride[k] = 1;
    }
    for (uint32_t k = 0; k < rank; ++k) l.size[k] = size[k];
    uint32_t cur = 1;
    for (int k = (int)rank - 1; k >= 0; --k) {
        l.stride[k] = cur;
        cur *= l.size[k];
    }
    l.rank = rank;
    l.offset = 0;
    *out = l;
    return VX_OK;
}

// TensorLayout::canonicalize (src/shapes.rs:145-155): prepend size-1 dims up
// to rank 4. For rank < 4 the result is built from contiguous(size) with the
// original strides copied into the trailing dims, so the prepended dims get
// contiguous strides and the offset becomes 0.
int layout_canonicalize(const vx_layout* in, vx_layout* out) {
    if (in->rank > 4) return fail(VX_ERR_UNSUPPORTED, "tensors of ranks > 4 not supported");
    if (in->rank == 4) {
        *out = *in;
        return VX_OK;
    }
    const uint32_t diff = 4 - in->rank;
    uint32_t size[4] = {1, 1, 1, 1};
    for (uint32_t k = 0; k < in->rank; ++k) size[diff + k] = in->size[k];
    vx_layout r;
    layout_contiguous(size, 4, &r);
    for (uint32_t k = 0; k < in->rank; ++k) r.stride[diff + k] = in->stride[k];
    *out = r;
    return VX_OK;
}

// TensorLayout::transpose (src/shapes.rs:238-254).
int layout_transpose(const vx_layout* in, uint32_t a, uint32_t b, vx_layout* out) {
    if (a >= in->rank || b >= in->rank) return fail(VX_ERR_INVALID, "transpose axis index out of bounds");
    vx_layout r = *in;
    std::swap(r.size[a], r.size[b]);
    std::swap(r.stride[a], r.stride[b]);
    *out = r;
    return VX_OK;
}

// TensorLayout::is_contiguous (src/shapes.rs:332-343): zero strides are
// accepted on any dim.
bool layout_is_contiguous(const vx_layout* l) {
    uint32_t stride = 1;
    for (int i = (int)l->rank - 1; i >= 0; --i) {
        if (l->stride[i] != 0 && l->stride[i] != stride) return false;
        stride *= l->size[i];
    }
    return true;
}

// TensorLayout::broadcast (src/shapes.rs:346-391). The lower-rank operand is
// right-aligned to the higher rank, every size-1 dim gets stride 0, and the
// shapes are compatible when each dim pair is equal or has a 1.
int layout_broadcast(const vx_layout* a_in, const vx_layout* b_in, vx_layout* a_out, vx_layout* b_out) {
    vx_layout s = *a_in, o = *b_in;
    if (s.rank > 4 || o.rank > 4) return fail(VX_ERR_UNSUPPORTED, "tensors of ranks > 4 not supported");
    const bool flip = s.rank > o.rank;
    if (flip) std::swap(s, o);
    const uint32_t diff = o.rank - s.rank;
    for (int k = (int)s.rank - 1; k >= 0; --k) {
        s.size[k + diff] = s.size[k];
        s.stride[k + diff] = s.stride[k];
    }
    for (uint32_t k = 0; k < diff; ++k) s.size[k] = 1;
    s.rank = o.rank;
    for (uint32_t k = 0; k < s.rank; ++k) {
        if (s.size[k] == 1) s.stride[k] = 0;
        if (o.size[k] == 1) o.stride[k] = 0;
    }
    for (uint32_t k = 0; k < s.rank; ++k)
        if (s.size[k] != 1 && o.size[k] != 1 && s.size[k] != o.size[k])
            return fail(VX_ERR_SHAPE, "incompatible broadcast shapes");
    if (flip) {
        *a_out = o;
        *b_out = s;
    } else {
        *a_out = s;
        *b_out = o;
    }
    return VX_OK;
}

// TensorLayout::view (src/shapes.rs:407-441): only from a contiguous source;
// missing strides default to the contiguous ones of the new shape.
int layout_view(const vx_layout* in, uint32_t offset, const uint32_t* shape, uint32_t rank,
                const uint32_t* strides, uint32_t nstrides, vx_layout* out) {
    if (rank > 4 || nstrides > rank) return fail(VX_ERR_UNSUPPORTED, "view rank > 4 or too many strides");
    if (!layout_is_contiguous(in)) return fail(VX_ERR_INVALID, "Cannot take a view of a non-contiguous tensor");
    uint64_t avail = 1, need = 1;
    for (int k = 0; k < 4; ++k) avail *= in->size[k];
    for (uint32_t k = 0; k < rank; ++k) need *= shape[k];
    need += offset;
    if (need > avail) return fail(VX_ERR_SHAPE, "Source tensor is too small for reshaping");
    vx_layout r{};
    for (int k = 0; k < 4; ++k) {
        r.size[k] = 1;
        r.stride[k] = 0;
    }
    for (uint32_t k = 0; k < rank; ++k) r.size[k] = shape[k];
    uint32_t cur = 1;
    for (int k = (int)rank - 1; k >= 0; --k) {
        const bool given = strides && (uint32_t)k < nstrides && strides[k] != 0xFFFFFFFFu;
        r.stride[k] = given ? strides[k] : cur;
        cur = r.stride[k] * r.size[k];
    }
    r.rank = rank;
    r.offset = in->offset + offset;
    *out = r;
    return VX_OK;
}

// TensorLayout::narrow (src/shapes.rs:443-465).
int layout_narrow(const vx_layout* in, uint32_t axis, uint32_t first, uint32_t count, vx_layout* out) {
    if (axis >= in->rank) return fail(VX_ERR_INVALID, "Axis index out of bounds.");
    if ((uint64_t)first + count > in->size[axis]) return fail(VX_ERR_SHAPE, "narrow range out of bounds");
    vx_layout r = *in;
    r.size[axis] = count;
    r.offset = in->offset + in->stride[axis] * first;
    *out = r;
    return VX_OK;
}

// TensorLayout::unsqueeze (src/shapes.rs:161-175): shift dims right from
// `axis`, insert size 1 whose stride copies its right neighbour. axis == 3
// has no right neighbour (the reference indexes stride[4] and panics): an
// error here.
int layout_unsqueeze(const vx_layout* in, uint32_t axis, vx_layout* out) {
    if (in->rank >= 4 || axis > in->rank || axis >= 3)
        return fail(VX_ERR_INVALID, "unsqueeze axis out of bounds or rank 4");
    vx_layout r = *in;
    for (int i = 2; i >= (int)axis; --i) {
        r.size[i + 1] = r.size[i];
        r.stride[i + 1] = r.stride[i];
    }
    r.size[axis] = 1;
    r.stride[axis] = r.stride[axis + 1];
    r.rank += 1;
    *out = r;
    return VX_OK;
}

}  // namespace vx
