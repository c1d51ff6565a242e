// vx_args.hpp — fetch a kernel's arguments in one batch at entry.
//
// Kernel arguments sit in memory that a wave reads through the scalar
// cache, and on MI355X a miss there costs about a third of a microsecond.
// The compiler loads each argument where it is first needed, so an argument
// on a 64-byte line that the first loads did not touch (the hidden grid size
// after a large argument struct, or a field used only after the first wait)
// is a second miss, paid in series by every wave before its first data
// request. Measured on a 25 MB read (graph-replayed, same code otherwise):
// 5.71 us with the arguments on two lines fetched one after the other, 5.38
// us with both fetched together. vx_args_fetch touches every dword of the
// argument struct and the grid size in one group, so all their lines are
// requested before any wait and later reads hit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

template <typename T>
__device__ __forceinline__ void vx_args_fetch(const T& a) {
    static_assert(sizeof(T) % 4 == 0, "argument structs are whole dwords");
    constexpr int N = (int)(sizeof(T) / 4);
    const uint32_t* u = reinterpret_cast<const uint32_t*>(&a);
    uint32_t v[N + 1];
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = u[i];
    v[N] = gridDim.x;
#pragma unroll
    for (int i = 0; i <= N; ++i) asm volatile("" ::"s"(v[i]));
}
