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
    // entries (f32 bits, column, global id, 0), replayed in column order by
    // the chain kernel.
    uint4 *chain_rows;
    uint32_t *chain_count;
    uint32_t chain_capacity;
    uint4 *chain_pool;
    uint32_t *chain_pool_used;
    uint32_t chain_pool_capacity;
    // MFMA kernel survivor log: one slot per persistent workgroup, holding
    // log_capacity (raw dot, column) entries per thread.
    uint2 *survivor_log;
    uint32_t log_capacity;
    uint32_t log_slots;
};

constexpr uint32_t kLeafLogCapacity = 128;
constexpr uint32_t kLeafLogSlots = 2048;

// Host-side launchers (leaf_exact.hip / leaf_mfma.hip).
int launch_leaf_exact_all(const LeafParams &p, hipStream_t stream);
int launch_leaf_exact_fallback(const LeafParams &p, hipStream_t stream);
int launch_leaf_mfma(const LeafParams &p, hipStream_t stream);
int launch_leaf_chain(const LeafParams &p, hipStream_t stream);
int leaf_mfma_supported(uint32_t padded_dim, uint32_t max_leaf_rows);

}  // namespace tessa
