// hashprune_kernels.h -- launch interface of the HashPrune reservoir kernels
// (hashprune.hip), shared with the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

// Largest reservoir (l_max) the reduce kernel takes: one wave merges at most
// kHpMergeCap candidates per round, l_max of them the reservoir's own slots.
constexpr uint32_t kHpMergeCap = 512;
constexpr uint32_t kHpMaxLMax = 256;

struct HashPruneState {
    uint32_t num_points = 0;
    uint32_t l_max = 0;
    uint64_t *slot_keys = nullptr;  // num_points x l_max: total-order dist key << 32 | target
    uint16_t *slot_hash = nullptr;  // num_points x l_max
    uint32_t *slot_count = nullptr; // num_points
    uint32_t *bucket = nullptr;     // num_points: records per source in the batch (zero between batches)
    uint32_t *offsets = nullptr;    // num_points + 1: first grouped record of each source
    uint32_t *block_sums = nullptr; // scan partials
    uint64_t block_sums_capacity = 0;
    uint4 *grouped = nullptr;       // the batch's records grouped by source
    uint64_t grouped_capacity = 0;
    uint64_t *status = nullptr;     // [0] first record with src >= num_points (UINT64_MAX: none)
    void *seg_ws = nullptr;          // segment mode workspace (hashprune_segment_workspace_bytes)
    uint64_t seg_ws_bytes = 0;
    // Named R-half backfill (rhalf_mode != 0): per slot the next rhalf_quota
    // distinct targets of its hash, ascending keys (~0: none), kept while the
    // reservoir has a free slot; the export appends up to rhalf_capacity of
    // them to an underfull row by the mode's priority.
    uint32_t rhalf_mode = 0;         // kRhalf*
    uint32_t rhalf_quota = 0;        // 1..3
    uint32_t rhalf_capacity = 0;     // min(row cap, l_max / 2)
    double rhalf_alpha_sq = 1.0;     // SoftTier priority alpha squared
    uint64_t *grp_keys = nullptr;    // num_points x l_max x kRhalfGroup
};

constexpr uint32_t kRhalfHashSlot1 = 1;
constexpr uint32_t kRhalfDistanceFirstQ3 = 2;
constexpr uint32_t kRhalfSoftTierQ3 = 3;
constexpr uint32_t kRhalfHardTierQ3 = 4;
constexpr uint32_t kRhalfGroup = 3;  // group keys stored per slot (the largest quota)

// Groups `count` records by source and merges each source's new candidates
// into its reservoir.  Returns 0, or -1 when a launch failed.
int launch_hashprune_insert(HashPruneState &s, const uint4 *records, uint64_t count, hipStream_t stream);
// The same for records described by segments {src, first lo, first hi, count}
// (records left in place; the segments, not the records, are sorted by
// source, so the work is proportional to the batch, not to num_points).
uint64_t hashprune_segment_workspace_bytes(uint64_t nseg, uint32_t num_points);
int launch_hashprune_insert_segments(HashPruneState &s, const uint4 *records, const uint4 *segs, uint64_t nseg,
                                     hipStream_t stream);
// Zeroes the per-source counters (all reservoirs empty).
int launch_hashprune_clear(HashPruneState &s, hipStream_t stream);
// Slot targets / hashes / distances (ascending hash) and counts per point,
// then, with a backfill policy, the row's backups in priority order.
int launch_hashprune_export(const HashPruneState &s, uint32_t *targets, uint16_t *hashes, float *dists,
                            uint32_t *counts, hipStream_t stream);
uint64_t hashprune_scan_blocks(uint32_t num_points);

}  // namespace tessa
