// Internal helpers shared by the treeverify translation units (host + gfx950 device).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "treeverify.h"

namespace tv {

// ---------------------------------------------------------------- host side
// Records a printf-style message for tv_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
// Clears the message at the start of an entry point.
void clear_error();
// Converts a launch result into TV_OK / TV_ERR_LAUNCH.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Flags word of an attention work item (both planners write it, the kernel checks it
// against the live metadata): the last prefix chunk of its (request, head group, node
// block), which also covers the tree; the last node block of its request; and the query
// heads per KV head the plan was made for.
constexpr int kItemLastChunk = 1;
constexpr int kItemLastBlock = 2;
constexpr int kItemGroupShift = 8;

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ---------------------------------------------------------------- device side
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void set_status(int32_t* status, int32_t bits) {
    if (status) atomicOr(status, bits);
}

}  // namespace tv
