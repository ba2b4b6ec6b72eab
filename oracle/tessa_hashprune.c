/*
 * tessa_hashprune.c -- CPU restatement of the HashPrune reservoir and of the
 * spill reducer's per-point reduction.  TEST INFRASTRUCTURE ONLY (see
 * tessa_oracle.h): the parity checker for shear_amd/csrc/hashprune.hip.
 *
 * Paths are relative to shear-core/src/algorithm/pipnn/ in the reference.
 *
 *   hp_order             hash_prune.rs:2094-2106 hashprune_candidate_total_order:
 *                        dist by f32 total_cmp, then target, then hash.
 *   hp_insert            hash_prune.rs:1333-1453 insert_inner (backfill and
 *                        evidence policies off, their defaults params.rs:3346-3350):
 *                        binary search by hash; a hash hit keeps the better
 *                        candidate; a miss inserts in hash order while below
 *                        l_max, else replaces the farthest slot when better and
 *                        re-sorts it into hash order; recompute_farthest :467-478.
 *   orc_hashprune_reduce spill_hashprune.rs:2686-2719 reduce_segment_group_in_range_off
 *                        (reservoir.insert per edge in stream order) and :3203-3221
 *                        emit_shard (copy_neighbors_and_clear: slot targets in slot
 *                        order, i.e. ascending hash).
 *
 * The slots are a sorted array exactly as in the reference; this file is a
 * sequential restatement, not the GPU algorithm (which sorts per point).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "tessa_oracle.h"

typedef struct {
    uint32_t target;
    float dist;
    uint16_t hash;
} hp_slot;

/* f32 total_cmp as an unsigned key: negative values reversed below positive ones. */
static uint32_t total_key(float d) {
    uint32_t b;
    memcpy(&b, &d, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* -1, 0, 1 like Ordering: (dist total_cmp, target, hash). */
static int hp_order(uint32_t lt, uint16_t lh, float ld, uint32_t rt, uint16_t rh, float rd) {
    const uint32_t lk = total_key(ld), rk = total_key(rd);
    if (lk != rk) return lk < rk ? -1 : 1;
    if (lt != rt) return lt < rt ? -1 : 1;
    if (lh != rh) return lh < rh ? -1 : 1;
    return 0;
}

typedef struct {
    hp_slot *slots; /* l_max capacity, sorted by hash */
    size_t len;
    size_t farthest;
} hp_reservoir;

static void hp_recompute_farthest(hp_reservoir *r) {
    size_t idx = 0;
    for (size_t i = 1; i < r->len; ++i) {
        const hp_slot *s = &r->slots[i], *f = &r->slots[idx];
        if (hp_order(s->target, s->hash, s->dist, f->target, f->hash, f->dist) > 0) idx = i;
    }
    r->farthest = idx;
}

/* first index whose hash is >= h (partition_point of hash < h) */
static size_t hp_lower_bound(const hp_slot *s, size_t lo, size_t hi, uint16_t h) {
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (s[mid].hash < h) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

static void hp_insert(hp_reservoir *r, size_t l_max, uint32_t target, uint16_t hash, float dist) {
    const size_t pos = hp_lower_bound(r->slots, 0, r->len, hash);
    if (pos < r->len && r->slots[pos].hash == hash) {
        hp_slot *s = &r->slots[pos];
        if (hp_order(target, hash, dist, s->target, s->hash, s->dist) < 0) {
            s->target = target;
            s->dist = dist;
            if (pos == r->farthest) hp_recompute_farthest(r);
        }
        return;
    }
    if (r->len < l_max) {
        memmove(&r->slots[pos + 1], &r->slots[pos], (r->len - pos) * sizeof(hp_slot));
        r->slots[pos] = (hp_slot){target, dist, hash};
        r->len++;
        if (r->len == 1) {
            r->farthest = 0;
        } else {
            if (pos <= r->farthest) r->farthest++;
            const hp_slot *n = &r->slots[pos], *f = &r->slots[r->farthest];
            if (hp_order(n->target, n->hash, n->dist, f->target, f->hash, f->dist) > 0) r->farthest = pos;
        }
        return;
    }
    const hp_slot *f = &r->slots[r->farthest];
    if (hp_order(target, hash, dist, f->target, f->hash, f->dist) >= 0) return;
    /* overwrite the farthest slot, then rotate it into hash order */
    const size_t fi = r->farthest;
    const hp_slot ns = {target, dist, hash};
    if (fi > 0 && r->slots[fi - 1].hash > hash) {
        const size_t tp = hp_lower_bound(r->slots, 0, fi, hash);
        memmove(&r->slots[tp + 1], &r->slots[tp], (fi - tp) * sizeof(hp_slot));
        r->slots[tp] = ns;
    } else if (fi + 1 < r->len && r->slots[fi + 1].hash < hash) {
        const size_t tp = hp_lower_bound(r->slots, fi + 1, r->len, hash);
        memmove(&r->slots[fi], &r->slots[fi + 1], (tp - fi - 1) * sizeof(hp_slot));
        r->slots[tp - 1] = ns;
    } else {
        r->slots[fi] = ns;
    }
    hp_recompute_farthest(r);
}

int orc_hashprune_reduce(size_t num_points, size_t l_max, const orc_edge_record *records, size_t count,
                         uint32_t *out_targets, uint16_t *out_hashes, float *out_dists, uint32_t *out_counts,
                         uint32_t *bad_record) {
    if (l_max == 0) return -1;
    hp_slot *pool = (hp_slot *)calloc(num_points ? num_points * l_max : 1, sizeof(hp_slot));
    hp_reservoir *res = (hp_reservoir *)calloc(num_points ? num_points : 1, sizeof(hp_reservoir));
    if (!pool || !res) {
        free(pool);
        free(res);
        return -2;
    }
    for (size_t p = 0; p < num_points; ++p) res[p].slots = pool + p * l_max;
    for (size_t i = 0; i < count; ++i) {
        const orc_edge_record *e = &records[i];
        if (e->src >= num_points) {
            if (bad_record) *bad_record = (uint32_t)i;
            free(pool);
            free(res);
            return -3;
        }
        hp_insert(&res[e->src], l_max, e->dst, e->hash, e->dist);
    }
    for (size_t p = 0; p < num_points; ++p) {
        out_counts[p] = (uint32_t)res[p].len;
        for (size_t s = 0; s < l_max; ++s) {
            const int live = s < res[p].len;
            out_targets[p * l_max + s] = live ? res[p].slots[s].target : 0xFFFFFFFFu;
            if (out_hashes) out_hashes[p * l_max + s] = live ? res[p].slots[s].hash : 0;
            if (out_dists) out_dists[p * l_max + s] = live ? res[p].slots[s].dist : 0.0f;
        }
    }
    free(pool);
    free(res);
    return 0;
}
