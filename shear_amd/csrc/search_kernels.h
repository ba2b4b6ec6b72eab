// search_kernels.h -- launch interface of the greedy graph search (search.hip),
// shared with the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

constexpr uint32_t kSearchMaxL = 256;   // search list capacity held in LDS
constexpr uint32_t kSearchWaves = 4;    // waves (query slots) per workgroup

struct GraphSearchParams {
    const float *data;        // num_points x dim, or null with SQ8 rows
    const int8_t *codes;      // SQ8 rows: num_points x padded_dim codes (when data is null)
    const float *scales;      // SQ8 rows: num_points scales; a row reads as scale * code
    uint32_t padded_dim;
    uint32_t num_points;
    uint32_t dim;
    const uint32_t *targets;  // num_points x row_stride neighbour ids
    const uint32_t *counts;   // num_points (clipped to row_stride)
    uint32_t row_stride;
    uint32_t start;
    const float *queries;     // num_queries x dim
    uint32_t num_queries;
    uint32_t L;
    uint32_t K;
    uint32_t *out_ids;        // num_queries x K (0xFFFFFFFF past the list)
    float *out_dists;         // num_queries x K, or null
    uint32_t *out_cmps;       // num_queries, or null
    uint32_t *tags;           // slots x num_points visited tags (query index + 1)
    uint32_t slots;           // a multiple of kSearchWaves
};

// Query slots for a call: each slot owns num_points tags of scratch.
uint32_t search_slots(uint32_t num_points, uint32_t num_queries);
int launch_graph_search(const GraphSearchParams &p, hipStream_t stream);

}  // namespace tessa
