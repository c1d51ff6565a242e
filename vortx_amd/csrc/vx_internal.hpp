// vx_internal.hpp — declarations shared by the host sources of
// libvortx_hip.so (not part of the public C ABI).
#pragma once

#include <cstdint>
#include <utility>

#include "vortx_hip.h"

namespace vx {

// Records `msg` as this thread's last error and returns `status`.
int fail(int status, const char* msg);
int fail_hip(int hip_error, const char* what);
// Clears this thread's last error (every entry point starts with it).
void clear_error();

int layout_contiguous(const uint32_t* size, uint32_t rank, vx_layout* out);
int layout_canonicalize(const vx_layout* in, vx_layout* out);
int layout_transpose(const vx_layout* in, uint32_t a, uint32_t b, vx_layout* out);
bool layout_is_contiguous(const vx_layout* l);
int layout_broadcast(const vx_layout* a, const vx_layout* b, vx_layout* a_out, vx_layout* b_out);
int layout_view(const vx_layout* in, uint32_t offset, const uint32_t* shape, uint32_t rank,
                const uint32_t* strides, uint32_t nstrides, vx_layout* out);
int layout_narrow(const vx_layout* in, uint32_t axis, uint32_t first, uint32_t count, vx_layout* out);
int layout_unsqueeze(const vx_layout* in, uint32_t axis, vx_layout* out);

}  // namespace vx
