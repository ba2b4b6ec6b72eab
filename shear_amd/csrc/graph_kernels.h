// graph_kernels.h -- launch interface of the `_mem.index` packing kernels
// (graph.hip), shared with the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

struct GraphPackParams {
    const uint32_t *targets;  // num_points x row_stride neighbour ids
    const uint32_t *counts;   // num_points (clipped to row_stride)
    uint32_t num_points;
    uint32_t row_stride;
    uint32_t start;
    uint64_t num_frozen;
    uint32_t *out_words;      // index_size / 4 words
    uint64_t *block_sums;     // graph_scan_blocks(num_points)
    uint64_t *row_off;        // num_points: first word of each row after the header
    uint64_t *total_words;    // device u64: sum over rows of 1 + degree
    uint32_t *max_degree;     // device u32
};

uint64_t graph_scan_blocks(uint32_t num_points);
// Row sums and the max degree (total_words, max_degree); then the image.
int launch_graph_size(const GraphPackParams &p, hipStream_t stream);
int launch_graph_pack(const GraphPackParams &p, hipStream_t stream);

}  // namespace tessa
