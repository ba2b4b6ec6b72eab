/*
 * tessa_d0.c -- CPU restatement of the global D0 assignment (SQ8 rows against
 * the global D0 leaders, each row to its fanout_top nearest).
 * TEST INFRASTRUCTURE ONLY (see tessa_oracle.h): the parity checker for
 * shear_amd/csrc/d0_assign.hip.
 *
 * Paths relative to shear-core/src/algorithm/pipnn/:
 *   distance   sq_int8_approx_l2, dco_sq_int8.rs:2950-2965: the i32 code dot
 *              as f32, dist = (norm_r + norm_l) - ((2 * scale_r) * scale_l) * dot,
 *              0 when <= 0 (each operation rounded, no contraction)
 *   order      the GPU path's partial and merge kernels, compute_backend.rs:
 *              18083-18099 and 18446-18511: ascending (dist, leader global id),
 *              strict.  (quantize_sq8_and_assign_global_d0_reference,
 *              dco_sq_int8.rs:2016-2033, sorts with stable_distance_order's
 *              2e-5 tie band instead; the two differ only for leaders within
 *              2e-5 of each other.)
 *   fragments  row-major [rows x fanout_top] (child = leader index, point =
 *              global id), as the merge kernel writes them (:18503-18510);
 *   children   grouped by child, rows ascending within a child.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "tessa_oracle.h"

static float d0_dist(const int8_t *a, float sa, float na, const int8_t *b, float sb, float nb, size_t pd) {
    int32_t dot = 0;
    for (size_t i = 0; i < pd; ++i) dot += (int32_t)a[i] * (int32_t)b[i];
    const float sum = na + nb;
    const float s2 = 2.0f * sa;
    const float s3 = s2 * sb;
    const float prod = s3 * (float)dot;
    const float d = sum - prod;
    return d <= 0.0f ? 0.0f : d;
}

int orc_d0_assign(const int8_t *codes, const float *scales, const float *norms, const uint32_t *global_ids,
                  size_t rows, size_t padded_dim, const int8_t *leader_codes, const float *leader_scales,
                  const float *leader_norms, const uint32_t *leader_ids, size_t leader_count, size_t fanout,
                  uint32_t *out_child, uint32_t *out_point, uint64_t *child_offsets, uint32_t *child_points) {
    if (fanout == 0 || fanout > 32 || fanout > leader_count) return -1;
    int rc = 0;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        float bd[32];
        uint32_t bl[32], bid[32];
        size_t have = 0;
        for (size_t l = 0; l < leader_count; ++l) {
            const float d = d0_dist(codes + r * padded_dim, scales[r], norms[r], leader_codes + l * padded_dim,
                                    leader_scales[l], leader_norms[l], padded_dim);
            const uint32_t id = leader_ids[l];
            size_t pos = have;
            while (pos > 0 && (d < bd[pos - 1] || (d == bd[pos - 1] && id < bid[pos - 1]))) --pos;
            if (pos >= fanout) continue;
            const size_t last = have < fanout ? have : fanout - 1;
            for (size_t s = last; s > pos; --s) {
                bd[s] = bd[s - 1];
                bl[s] = bl[s - 1];
                bid[s] = bid[s - 1];
            }
            bd[pos] = d;
            bl[pos] = (uint32_t)l;
            bid[pos] = id;
            if (have < fanout) ++have;
        }
        for (size_t s = 0; s < fanout; ++s) {
            out_child[r * fanout + s] = bl[s];
            out_point[r * fanout + s] = global_ids[r];
        }
    }
    if (child_offsets) {
        memset(child_offsets, 0, (leader_count + 1) * sizeof(uint64_t));
        for (size_t i = 0; i < rows * fanout; ++i) child_offsets[out_child[i] + 1]++;
        for (size_t c = 0; c < leader_count; ++c) child_offsets[c + 1] += child_offsets[c];
        uint64_t *fill = (uint64_t *)malloc((leader_count ? leader_count : 1) * sizeof(uint64_t));
        if (!fill) return -2;
        memcpy(fill, child_offsets, leader_count * sizeof(uint64_t));
        for (size_t i = 0; i < rows * fanout; ++i) child_points[fill[out_child[i]]++] = out_point[i];
        free(fill);
    }
    return rc;
}
