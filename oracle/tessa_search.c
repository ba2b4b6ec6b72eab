/*
 * tessa_search.c -- CPU restatement of the in-memory index's greedy search.
 * TEST INFRASTRUCTURE ONLY (see tessa_oracle.h): the parity checker for
 * shear_amd/csrc/search.hip and the recall harness's reference.
 *
 * Paths relative to shear-core/src/ in the reference:
 *   gs_insert / gs_closest  model/neighbor/neighbor_priority_queue.rs:50-85
 *                           (capacity-L sorted list, reject when full and the
 *                           last is smaller, cursor = first not-visited)
 *   order                   model/neighbor/neighbor.rs:46-70 (distance, then id)
 *   orc_greedy_search       algorithm/search/search.rs:26-43 and :137-233
 *                           (start point seeded and marked visited; expand the
 *                           closest not-visited node; unvisited neighbours are
 *                           marked and inserted; until none is left), results
 *                           as index/inmem_index/inmem_index.rs:559-580 (the
 *                           first K entries)
 *   gs_l2                   squared L2 as one sequential f32 sum over the
 *                           coordinates, each term (x - q) * (x - q) rounded
 *                           before the add.  The reference's SIMD distance
 *                           may sum in another order: distances are pinned to
 *                           this order, not to the reference's bits.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "tessa_oracle.h"

typedef struct {
    float d;
    uint32_t id;
    int visited;
} gs_nbr;

static int gs_lt(float ad, uint32_t aid, float bd, uint32_t bid) {
    return ad < bd || (ad == bd && aid < bid);
}

static float gs_l2(const float *x, const float *q, size_t dim) {
    float s = 0.0f;
    for (size_t i = 0; i < dim; ++i) {
        const float t = x[i] - q[i];
        const float sq = t * t;
        s = s + sq;
    }
    return s;
}

static void gs_insert(gs_nbr *list, size_t *size, size_t cap, size_t *cur, float d, uint32_t id) {
    if (*size == cap && gs_lt(list[*size - 1].d, list[*size - 1].id, d, id)) return;
    size_t lo = 0, hi = *size;
    while (lo < hi) { /* first position whose element is not less than (d, id) */
        const size_t mid = lo + (hi - lo) / 2;
        if (gs_lt(list[mid].d, list[mid].id, d, id)) lo = mid + 1;
        else hi = mid;
    }
    if (lo < *size && list[lo].d == d && list[lo].id == id) return;
    if (lo >= cap) return;
    const size_t move = (*size < cap ? *size : cap - 1) - lo;
    memmove(&list[lo + 1], &list[lo], move * sizeof(gs_nbr));
    list[lo] = (gs_nbr){d, id, 0};
    if (*size < cap) (*size)++;
    if (lo < *cur) *cur = lo;
}

int orc_greedy_search(const float *data, size_t num_points, size_t dim, const uint32_t *targets,
                      const uint32_t *counts, size_t row_stride, uint32_t start, const float *queries,
                      size_t num_queries, size_t L, size_t K, uint32_t *out_ids, float *out_dists,
                      uint32_t *out_cmps) {
    if (L == 0 || K == 0 || K > L || start >= num_points) return -1;
    gs_nbr *list = (gs_nbr *)malloc((L + 1) * sizeof(gs_nbr));
    uint8_t *visited = (uint8_t *)malloc(num_points ? num_points : 1);
    uint32_t *fresh = (uint32_t *)malloc((row_stride ? row_stride : 1) * sizeof(uint32_t));
    if (!list || !visited || !fresh) {
        free(list);
        free(visited);
        free(fresh);
        return -2;
    }
    for (size_t qi = 0; qi < num_queries; ++qi) {
        const float *q = queries + qi * dim;
        memset(visited, 0, num_points);
        size_t size = 0, cur = 0;
        uint32_t cmps = 0;
        visited[start] = 1;
        gs_insert(list, &size, L, &cur, gs_l2(data + (size_t)start * dim, q, dim), start);
        while (cur < size) {
            /* closest_notvisited */
            list[cur].visited = 1;
            const uint32_t node = list[cur].id;
            while (cur < size && list[cur].visited) ++cur;
            const uint32_t deg = counts[node] < row_stride ? counts[node] : (uint32_t)row_stride;
            size_t nf = 0;
            for (uint32_t s = 0; s < deg; ++s) {
                const uint32_t id = targets[(size_t)node * row_stride + s];
                if (id >= num_points || visited[id]) continue;
                visited[id] = 1;
                fresh[nf++] = id;
            }
            for (size_t m = 0; m < nf; ++m)
                gs_insert(list, &size, L, &cur, gs_l2(data + (size_t)fresh[m] * dim, q, dim), fresh[m]);
            cmps += (uint32_t)nf;
        }
        for (size_t i = 0; i < K; ++i) {
            out_ids[qi * K + i] = i < size ? list[i].id : 0xFFFFFFFFu;
            if (out_dists) out_dists[qi * K + i] = i < size ? list[i].d : 0.0f;
        }
        if (out_cmps) out_cmps[qi] = cmps;
    }
    free(list);
    free(visited);
    free(fresh);
    return 0;
}
