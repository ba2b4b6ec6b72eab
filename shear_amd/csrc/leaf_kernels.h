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
    // Debug/test knob: lowers the per-lane candidate list capacity so the
    // overflow -> exact fallback path runs on ordinary inputs (0 = default).
    uint32_t list_cap_override;
};

// Host-side launchers (leaf_exact.hip / leaf_mfma.hip).
int launch_leaf_exact_all(const LeafParams &p, hipStream_t stream);
int launch_leaf_exact_fallback(const LeafParams &p, hipStream_t stream);
int launch_leaf_mfma(const LeafParams &p, hipStream_t stream);
int leaf_mfma_supported(uint32_t padded_dim, uint32_t max_leaf_rows);

}  // namespace tessa
