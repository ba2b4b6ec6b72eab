// leaf_kernels.h -- launch parameters shared by the leaf kernels and the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tessa {

struct LeafParams {
    const int8_t *codes;
    const float *scales;
    const float *norms;
    const uint32_t *gids;
    uint64_t rows;
    uint32_t padded_dim;
    uint32_t k;
    const uint32_t *members;
    const uint64_t *member_offsets;
    const uint32_t *member_counts;
    const uint64_t *output_offsets;
    uint32_t leaf_count;
    uint32_t max_leaf_rows;
    uint32_t *out_ids;
    float *out_dists;
    uint64_t *counters;
    // Rows the MFMA kernel could not certify, re-run by the exact kernel:
    // pairs (leaf, row); count is a device u32; capacity is the pair count.
    uint32_t *fallback;
    uint32_t *fallback_count;
    uint32_t fallback_capacity;
    // Test knob: rows whose leaf position is a multiple of this value skip
    // certification and are re-run by the exact kernel (0 = off).
    uint32_t debug_rerun_every;
    // Rows whose certified candidate set G holds an eps-tie chain: header
    // (output offset lo/hi, pool offset, |G| | k_eff << 8) plus |G| pool
    // entries (f32 bits, column, global id, 0) at pool offset + 64 i (the
    // sets of 64 consecutive queue entries interleaved), replayed in column
    // order by the chain kernel.  chain_pool_used is not used.
    uint4 *chain_rows;
    uint32_t *chain_count;
    uint32_t chain_capacity;
    uint4 *chain_pool;
    uint32_t *chain_pool_used;
    uint32_t chain_pool_capacity;
    // Work tickets of the filter kernel: words 0..7 one counter per XCD, word
    // 8 the count of finished workgroups.  Zero before the first launch; the
    // last workgroup of each launch zeroes them again.
    uint32_t *item_tickets;
    // The batch's work items, listed: entry g = (leaf, block) for g below
    // *item_total (the leaves' non-empty blocks, a leaf's blocks in a row);
    // batches cover list positions [item_begin, item_begin + item_count) and
    // positions at or past *item_total are empty.
    const uint2 *item_list;
    const uint32_t *item_total;
    // Work items are (leaf, block of kLeafBlockRows member rows), at most
    // blocks_per_leaf per leaf.  The filter kernel writes, per block row of
    // the batch's item w (list position item_begin + w), 2 * log_capacity
    // survivor entries (raw dot, column) at survivor_log[(w * kLeafBlockRows
    // + row) * 2 * log_capacity], entry e of the row's lane h at 2e + h, and a row_meta
    // word set (threshold F bits, the two lanes' entry counts); the select
    // kernel reads both.
    uint32_t item_begin;
    uint32_t item_count;
    uint32_t blocks_per_leaf;
    uint2 *survivor_log;
    uint32_t log_capacity;
    uint4 *row_meta;
};

constexpr uint32_t kLeafBlockRows = 256;       // member rows per work item
constexpr uint32_t kLeafFilterThreads = 512;   // filter workgroup: 8 waves, 32 rows each
constexpr uint32_t kLeafLogCapacity = 128;     // survivor entries per filter thread
constexpr uint64_t kLeafLogBytesPerItem = (uint64_t)kLeafFilterThreads * kLeafLogCapacity * 8u;
constexpr uint32_t kLeafChainSetEntries = 40;  // chain pool entries per queued row (k + 8)

// Chain rows the queue and the pool can both hold: a queued row needs its
// header slot and its candidate set in a whole 64-row pool group.  The
// select kernel only writes a header when both fit, and the chain kernel
// replays every header below min(count, capacity), so the capacity passed to
// both must not exceed what the pool holds.
inline uint64_t leaf_chain_rows_usable(uint64_t queue_capacity, uint64_t pool_entries) {
    const uint64_t pool_rows = pool_entries / ((uint64_t)kLeafChainSetEntries * 64u) * 64u;
    return queue_capacity < pool_rows ? queue_capacity : pool_rows;
}

// Host-side launchers (leaf_exact.hip / leaf_mfma.hip).
int launch_leaf_exact_all(const LeafParams &p, hipStream_t stream);
int launch_leaf_exact_fallback(const LeafParams &p, hipStream_t stream);
int launch_leaf_mfma(const LeafParams &p, hipStream_t stream);
int launch_leaf_select(const LeafParams &p, hipStream_t stream);
int launch_leaf_chain(const LeafParams &p, hipStream_t stream);
int leaf_mfma_supported(uint32_t padded_dim, uint32_t max_leaf_rows);

}  // namespace tessa
