// assign_kernels.h -- launch parameters of the assignment replay kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

struct AssignParams {
    const int8_t *codes;
    const float *scales;
    const float *norms;
    const uint32_t *gids;
    uint64_t rows;
    uint32_t padded_dim;
    const uint32_t *members;
    const uint32_t *leaders;
    const uint32_t *member_offsets;
    const uint32_t *member_counts;
    const uint32_t *leader_offsets;
    const uint32_t *leader_counts;
    const uint32_t *r_h;
    const uint64_t *output_offsets;
    uint32_t task_count;
    uint32_t max_members;
    uint32_t *out_ids;
    float *out_dists;
    uint64_t *counters;
};

int launch_assign_replay(const AssignParams &p, hipStream_t stream);
int launch_sq8_quantize(const float *x, uint64_t rows, uint32_t dim, uint32_t padded_dim, uint32_t bits,
                        int8_t *codes, float *scales, float *norms, uint64_t *bad_row, hipStream_t stream);

}  // namespace tessa
