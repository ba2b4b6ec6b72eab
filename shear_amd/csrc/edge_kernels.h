// edge_kernels.h -- launch parameters of the candidate-record -> edge-record
// kernels (edge_records.hip) shared with the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

// Largest leaf the edge kernels take (LDS: row counts, member ids and a
// membership table of 2x that size, 64 KB at this bound).
constexpr uint32_t kEdgeMaxLeafRows = 4096;

// Status words written by the edge kernels (device u64[4]).
enum EdgeStatusWord : uint32_t {
    kEdgeRecordCount = 0,  // records the batch needs (2 per valid slot)
    kEdgeFirstError = 1,   // smallest error key, UINT64_MAX when none (see edge_error_key)
    kEdgeCapacityHit = 2,  // 1 when out_capacity was too small (nothing written)
    kEdgeLeafTooLarge = 3, // 1 + largest leaf above max_leaf_rows (such leaves emit nothing)
    kEdgeKept = 4,         // unique grouped order: records written (the leaves' cursor)
    kEdgeStatusWords = 5
};

// Error keys order errors as the reference meets them: leaf by leaf, the
// sketch prefetch of the leaf's points before its slots, slots in row-major
// order.  key = leaf << 20 | kind << 19 | row << 6 | rank (row < 4096, rank < 64).
constexpr uint64_t kEdgeErrSketch = 0;   // a leaf point has no sketch row; row field = member row
constexpr uint64_t kEdgeErrOutside = 1;  // a top-k id is not a member of the leaf
__host__ __device__ inline uint64_t edge_error_key(uint64_t leaf, uint64_t kind, uint64_t row, uint64_t rank) {
    return (leaf << 20) | (kind << 19) | (row << 6) | rank;
}

struct EdgeParams {
    const uint32_t *gids;            // global id per resident row
    uint64_t resident_rows;
    const uint32_t *members;         // resident rows, per leaf
    const uint64_t *member_offsets;
    const uint32_t *member_counts;
    const uint64_t *output_offsets;  // slot of (leaf, row 0, rank 0)
    uint32_t leaf_count;
    uint32_t max_leaf_rows;          // <= kEdgeMaxLeafRows; larger leaves are reported, not emitted
    uint32_t table_bits;             // edge_table_bits(max_leaf_rows)
    uint32_t k;                      // slot stride; per leaf k = min(k, n - 1)
    const uint32_t *topk_ids;
    const float *topk_dists;
    const float *sketches;           // sketch_rows x width, row = global id
    uint64_t sketch_rows;
    uint32_t width;
    uint32_t m_bits;
    uint4 *out;                      // 16-byte records
    uint64_t out_capacity;           // records
    uint32_t *leaf_totals;           // workspace: valid slots per leaf
    uint64_t *leaf_base;             // leaf_count + 1: first record of each leaf, then the total
    uint64_t *status;                // kEdgeStatusWords
    // Source-grouped order (segments != null): inside each leaf the records
    // with the same source are adjacent, one segment per member row; segment
    // of (leaf, row r) = {src, first record (lo, hi words), record count} at
    // segments[leaf_seg_base[leaf] + r].
    uint4 *segments;
    uint64_t segment_capacity;
    uint64_t *leaf_seg_base;         // leaf_count + 1: first segment of each leaf, then the total
    // Grouped order only: leave out the reverse record of a slot (r -> j)
    // whose leaf row j lists r at the same distance (j's forward record is
    // the same record); the leaves then take their places in the output from
    // a cursor (status[kEdgeKept]) and the output has no gaps.
    uint32_t unique;
};

// log2 of the LDS membership table size: >= 2 x max_leaf_rows, >= 64.
uint32_t edge_table_bits(uint32_t max_leaf_rows);
int launch_edge_records(const EdgeParams &p, hipStream_t stream);

}  // namespace tessa
