// d0_kernels.h -- launch interface of the global D0 assignment (d0_assign.hip),
// shared with the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

constexpr uint32_t kD0MaxFanout = 32;
// The leader ranking is quadratic in the leader count (65,536 leaders: 4.3e9
// compares, a few ms); the reference caps root leaders at 10,000 by default.
constexpr uint32_t kD0MaxLeaders = 1u << 16;

struct D0AssignParams {
    const int8_t *codes;         // rows x padded_dim
    const float *scales;
    const float *norms;
    const uint32_t *global_ids;  // rows
    uint64_t rows;
    uint32_t padded_dim;         // a multiple of 16, <= 1024
    const int8_t *leader_codes;  // leaders x padded_dim
    const float *leader_scales;
    const float *leader_norms;
    const uint32_t *leader_ids;  // leaders (global ids: the tie order)
    uint32_t leaders;
    uint32_t fanout;
    uint32_t *leader_rank;       // leaders: position in (id, index) order
    uint32_t *rank_leader;       // leaders: the inverse
    uint32_t *out_child;         // rows x fanout leader indices
    uint32_t *out_point;         // rows x fanout global ids
};

int launch_d0_assign(const D0AssignParams &p, hipStream_t stream);

// Grouping of the fragments by child (stable, so rows stay ascending):
// child_offsets [leaders + 1], child_points [rows * fanout].
size_t d0_group_temp_bytes(uint64_t items, uint32_t leaders);
int launch_d0_group(const D0AssignParams &p, uint64_t *child_offsets, uint32_t *child_points, void *temp,
                    size_t temp_bytes, hipStream_t stream);

}  // namespace tessa
