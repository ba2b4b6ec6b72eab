// prune_kernels.h -- launch interface of the final RobustPrune (prune.hip),
// shared with the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

constexpr uint32_t kPruneMaxPool = 256;  // row_stride and max_degree limit (LDS lists)

struct RobustPruneParams {
    const float *data;        // num_points x dim
    uint32_t num_points;
    uint32_t dim;
    const uint32_t *targets;  // num_points x row_stride
    const uint32_t *counts;
    uint32_t row_stride;
    uint32_t max_degree;
    uint32_t max_occlusion;
    float alpha;
    uint32_t saturate;
    uint32_t *out_targets;    // num_points x max_degree
    uint32_t *out_counts;
};

int launch_robust_prune(const RobustPruneParams &p, hipStream_t stream);

}  // namespace tessa
