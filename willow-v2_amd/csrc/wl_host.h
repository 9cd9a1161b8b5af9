// Host-side argument validation shared by the C-ABI entry points. Every check runs before anything is enqueued.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/willow_hip.h"

namespace wl {

constexpr int64_t kMaxRows = 1 << 24;
constexpr int64_t kMaxK = 1 << 16;

inline int block_bytes(int type) {
    if (type == WL_TYPE_Q4_K) return 144;
    if (type == WL_TYPE_Q6_K) return 210;
    return -1;
}

// Base alignment the kernels rely on: Q4_K blocks are read with 16-byte loads (144 = 9 x 16), Q6_K blocks with
// dword loads realigned in registers, which needs an even block start on a dword-aligned base.
inline int64_t base_alignment(int type) { return type == WL_TYPE_Q4_K ? 16 : 4; }

inline int check_matrix(int type, const void* w, int64_t rows, int64_t k, int64_t row_stride) {
    const int bb = block_bytes(type);
    if (bb < 0) return WL_EINVAL_TYPE;
    if (!w) return WL_EINVAL_NULL;
    if (rows <= 0 || rows > kMaxRows || k <= 0 || k > kMaxK || k % 256 != 0) return WL_EINVAL_SHAPE;
    if (row_stride < k / 256 * bb) return WL_EINVAL_SHAPE;
    if (reinterpret_cast<uintptr_t>(w) % base_alignment(type) != 0) return WL_EINVAL_ALIGN;
    if (row_stride % (type == WL_TYPE_Q4_K ? 16 : 2) != 0) return WL_EINVAL_ALIGN;
    return WL_OK;
}

inline int launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? WL_OK : static_cast<int>(e);
}

}  // namespace wl
