// linear_workspace.h -- the optional split-K scratch of mlk_linear_quant /
// mlk_linear_f32, taken from the caching device allocator, so that a call
// with few token rows still fills the GPU and repeated calls cost no device
// allocation after the first.
#pragma once

#include "include/cuda_runtime.h"
#include "include/minilamma_hip.h"

#include <cstdint>

namespace yan_lamma {

inline CudaDeviceBuffer LinearWorkspace(int64_t rows, int64_t in_features, int64_t out_features,
                                        int device_id) {
    CudaDeviceBuffer ws;
    const int64_t bytes = mlk_linear_workspace_bytes(rows, in_features, out_features);
    if (bytes > 0) ws.Reset(static_cast<size_t>(bytes), device_id);
    return ws;
}

}  // namespace yan_lamma
