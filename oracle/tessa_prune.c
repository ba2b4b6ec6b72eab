/*
 * tessa_prune.c -- CPU restatement of the final RobustPrune pass over a
 * neighbour table.  TEST INFRASTRUCTURE ONLY (see tessa_oracle.h): the parity
 * checker for shear_amd/csrc/prune.hip.
 *
 * Paths relative to shear-core/src/:
 *   per node     index/inmem_index/pipnn_builder.rs:287-330 (final_prune_pipnn:
 *                pool = the node's neighbours with their distance to it; an empty
 *                row stays empty)
 *   robust_prune algorithm/prune/prune.rs:146-214 (pool sorted by (distance, id),
 *                model/neighbor/neighbor.rs:46-70; saturate only with alpha > 1)
 *   occlude_list prune.rs:17-96 (truncate to max_candidate_size; alpha passes
 *                1.0, x1.2, .. <= alpha; a candidate whose factor exceeds the pass's
 *                alpha waits; a picked one is marked f32::MAX and added unless it
 *                is the node itself; later candidates whose factor is <= alpha
 *                take max(factor, d_j / d(j, picked)), f32::MAX when that
 *                distance is 0)
 *   distances    squared L2 summed over the coordinates in order in f32, each
 *                product rounded before the add (the reference's SIMD distance
 *                may associate differently: pinned to this order).
 */
#include <float.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "tessa_oracle.h"

static float rp_l2(const float *a, const float *b, size_t dim) {
    float s = 0.0f;
    for (size_t i = 0; i < dim; ++i) {
        const float t = a[i] - b[i];
        const float sq = t * t;
        s = s + sq;
    }
    return s;
}

typedef struct {
    float d;
    uint32_t id;
} rp_nbr;

static int rp_cmp(const void *a, const void *b) {
    const rp_nbr *x = (const rp_nbr *)a, *y = (const rp_nbr *)b;
    if (x->d < y->d) return -1;
    if (x->d > y->d) return 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

int orc_robust_prune(const float *data, size_t num_points, size_t dim, const uint32_t *targets,
                     const uint32_t *counts, size_t row_stride, size_t max_degree, size_t max_occlusion,
                     float alpha, int saturate, uint32_t *out_targets, uint32_t *out_counts) {
    if (max_degree == 0) return -1;
    int bad = 0;
#pragma omp parallel
    {
        rp_nbr *pool = (rp_nbr *)malloc((row_stride ? row_stride : 1) * sizeof(rp_nbr));
        float *occ = (float *)malloc((row_stride ? row_stride : 1) * sizeof(float));
        if (!pool || !occ) {
#pragma omp atomic write
            bad = 1;
        }
#pragma omp for schedule(dynamic, 64)
        for (size_t v = 0; v < num_points; ++v) {
            if (!pool || !occ) continue;
            const float *xv = data + v * dim;
            const uint32_t deg = counts[v] < row_stride ? counts[v] : (uint32_t)row_stride;
            size_t n = 0;
            for (uint32_t s = 0; s < deg; ++s) {
                const uint32_t id = targets[v * row_stride + s];
                if (id >= num_points) continue;
                pool[n].d = rp_l2(xv, data + (size_t)id * dim, dim);
                pool[n].id = id;
                ++n;
            }
            uint32_t *res = out_targets + v * max_degree;
            size_t rl = 0;
            if (n > 0) {
                qsort(pool, n, sizeof(rp_nbr), rp_cmp);
                if (n > max_occlusion) n = max_occlusion;
                for (size_t i = 0; i < n; ++i) occ[i] = 0.0f;
                float cur = 1.0f;
                while (cur <= alpha && rl < max_degree) {
                    for (size_t i = 0; i < n; ++i) {
                        if (rl >= max_degree) break;
                        if (occ[i] > cur) continue;
                        occ[i] = FLT_MAX;
                        if (pool[i].id != (uint32_t)v) res[rl++] = pool[i].id;
                        const float *xi = data + (size_t)pool[i].id * dim;
                        for (size_t j = i + 1; j < n; ++j) {
                            if (occ[j] > alpha) continue;
                            const float djk = rp_l2(data + (size_t)pool[j].id * dim, xi, dim);
                            if (djk == 0.0f) {
                                occ[j] = FLT_MAX;
                            } else {
                                const float q = pool[j].d / djk;
                                occ[j] = occ[j] > q ? occ[j] : q;
                            }
                        }
                    }
                    cur *= 1.2f;
                }
                if (saturate && alpha > 1.0f) {
                    for (size_t i = 0; i < n && rl < max_degree; ++i) {
                        int seen = pool[i].id == (uint32_t)v;
                        for (size_t r = 0; r < rl && !seen; ++r) seen = res[r] == pool[i].id;
                        if (!seen) res[rl++] = pool[i].id;
                    }
                }
            }
            for (size_t r = rl; r < max_degree; ++r) res[r] = 0xFFFFFFFFu;
            out_counts[v] = (uint32_t)rl;
        }
        free(pool);
        free(occ);
    }
    return bad ? -2 : 0;
}
