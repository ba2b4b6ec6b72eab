/*
 * tessa_edges.c -- CPU restatement of the reference's candidate-record to
 * HashPrune-edge conversion.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker for shear_amd's edge-record
 * kernels; see tessa_oracle.h).  Paths are relative to
 * shear-core/src/algorithm/pipnn/ in the reference.
 */
#include <math.h>
#include <string.h>

#include "tessa_oracle.h"

/* hash_prune.rs:2239-2251 */
uint16_t orc_compute_hash(const float *sketch_p, const float *sketch_c, unsigned m_bits) {
    uint16_t h = 0;
    for (unsigned i = 0; i < m_bits; ++i) {
        const float diff = sketch_c[i] - sketch_p[i];
        if (diff >= 0.0f) h |= (uint16_t)(1u << i);
    }
    return h;
}

/* leaf_build.rs:330-346 compact_local_index: the j_local of a global id (the
 * linear form; the hash form agrees for batches without repeated ids). */
static long local_index(const uint32_t *point_ids, size_t rows, uint32_t id) {
    for (size_t i = 0; i < rows; ++i)
        if (point_ids[i] == id) return (long)i;
    return -1;
}

/* leaf_build.rs:1679-1829 */
long long orc_flush_compact_topk_into_edges(const uint32_t *point_ids, size_t rows, size_t k,
                                            const uint32_t *topk_ids, const float *topk_dists,
                                            const float *sketches, size_t sketch_rows, size_t width,
                                            unsigned m_bits, orc_edge_record *out, size_t capacity,
                                            uint32_t *bad_point) {
    if (rows == 0 || k == 0) return 0; /* :1695-1698 */
    if (m_bits > 16 || m_bits > width) return -2; /* hash_prune.rs:2240 assert, slice bound */
    /* :1758-1763 LeafSketchCache::prefetch reads one sketch row per point */
    for (size_t i = 0; i < rows; ++i)
        if (point_ids[i] >= sketch_rows) {
            if (bad_point) *bad_point = point_ids[i];
            return -3;
        }
    size_t n = 0;
    for (size_t i = 0; i < rows; ++i) { /* :1766 */
        const uint32_t i_global = point_ids[i];
        const float *sketch_i = sketches + (size_t)i_global * width;
        for (size_t rank = 0; rank < k; ++rank) { /* :1771 */
            const uint32_t j = topk_ids[i * k + rank];
            const float d = topk_dists[i * k + rank];
            if (j == ORC_EMPTY_ID || !isfinite(d)) continue; /* :1774-1776 */
            if (local_index(point_ids, rows, j) < 0) {        /* :1796-1801 */
                if (bad_point) *bad_point = j;
                return -1;
            }
            const float *sketch_j = sketches + (size_t)j * width; /* row(j_local) = sketch of j */
            if (n + 2 > capacity) return -2;
            out[n].src = i_global; /* :1797-1812: forward then reverse */
            out[n].dst = j;
            out[n].hash = orc_compute_hash(sketch_i, sketch_j, m_bits);
            out[n].flags = 0;
            out[n].dist = d;
            out[n + 1].src = j;
            out[n + 1].dst = i_global;
            out[n + 1].hash = orc_compute_hash(sketch_j, sketch_i, m_bits);
            out[n + 1].flags = 0;
            out[n + 1].dist = d;
            n += 2;
        }
    }
    return (long long)n;
}
