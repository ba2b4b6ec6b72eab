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

/* ---- named R-half backfill policies (SoftTier-Q3 and its siblings) -------
 *
 * hash_prune_backfill.rs:44-83 (from_params: the hash quota of the named
 * modes, 1 for rhalf-hash-slot-1 and 3 for the Q3 modes; the SoftTier
 * priority alpha, 1.1 unless given, with alpha^2 exactly 1.21 for that
 * value :62-66), :299-336 (budget_for = floor(R/2); candidate_capacity_for =
 * min(row cap, budget, R - primaries)), :375-386 (priority_score: the
 * squared distance in f64, times alpha^2 per hit layer past the first, for
 * SoftTier only), hash_prune.rs:655-685 (rhalf_priority_order).
 *
 * The result is the reference's own order-independent characterization of
 * the streaming reservoir (hash_prune.rs:2601-2682 reference_tiered_rhalf_slots,
 * which the reference's tests hold the streaming insert and finish to for
 * every insertion order, :3019-3085, :3243-3290): the primaries are the
 * ordinary HashPrune reservoir; when there are some but fewer than l_max,
 * each primary hash's other candidates (distinct targets, each at its best
 * distance, the primary's own target excluded) are sorted by the candidate
 * order and cut to the quota, a member's hit layer being its rank (1-based);
 * all members are sorted by the priority order and cut to the capacity; the
 * row is the primaries (ascending hash) then the shortlist (priority order),
 * as finish_soft_tier_q3_fast emits it (:1458-1555).  No alpha gate applies
 * to the named modes (uses_alpha_gate is false for them, :388-391). */

typedef struct {
    uint32_t target;
    float dist;
    uint16_t hash;
    uint32_t layer;
} rh_member;

static uint64_t total_key64(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    return (b & 0x8000000000000000ull) ? ~b : (b | 0x8000000000000000ull);
}

typedef struct {
    int mode;          /* ORC_RHALF_* */
    double alpha_sq;   /* SoftTier priority alpha squared */
} rh_policy;

static double rh_priority_score(const rh_policy *p, float dist, uint32_t layer) {
    const double d = (double)dist;
    if (p->mode != ORC_RHALF_SOFT_TIER_Q3) return d;
    if (layer == 2) return d * p->alpha_sq;
    if (layer == 3) return d * p->alpha_sq * p->alpha_sq;
    return d;
}

static int rh_cmp_u64(uint64_t a, uint64_t b) { return a < b ? -1 : (a > b ? 1 : 0); }
static int rh_cmp_u32(uint32_t a, uint32_t b) { return a < b ? -1 : (a > b ? 1 : 0); }

/* hash_prune.rs:655-685 */
static int rh_priority_order(const rh_policy *p, const rh_member *l, const rh_member *r) {
    int c;
    switch (p->mode) {
        case ORC_RHALF_SOFT_TIER_Q3:
            c = rh_cmp_u64(total_key64(rh_priority_score(p, l->dist, l->layer)),
                           total_key64(rh_priority_score(p, r->dist, r->layer)));
            if (c) return c;
            if ((c = rh_cmp_u32(l->layer, r->layer))) return c;
            if ((c = rh_cmp_u32(l->target, r->target))) return c;
            return rh_cmp_u32(l->hash, r->hash);
        case ORC_RHALF_HARD_TIER_Q3:
            if ((c = rh_cmp_u32(l->layer, r->layer))) return c;
            return hp_order(l->target, l->hash, l->dist, r->target, r->hash, r->dist);
        default: /* hash-slot-1, distance-first-q3 */
            if ((c = rh_cmp_u32(total_key(l->dist), total_key(r->dist)))) return c;
            if ((c = rh_cmp_u32(l->layer, r->layer))) return c;
            if ((c = rh_cmp_u32(l->target, r->target))) return c;
            return rh_cmp_u32(l->hash, r->hash);
    }
}

static const rh_policy *g_rh_policy; /* for qsort */
static int rh_qsort_priority(const void *a, const void *b) {
    return rh_priority_order(g_rh_policy, (const rh_member *)a, (const rh_member *)b);
}
static int rh_qsort_candidate(const void *a, const void *b) {
    const rh_member *l = (const rh_member *)a, *r = (const rh_member *)b;
    return hp_order(l->target, l->hash, l->dist, r->target, r->hash, r->dist);
}
/* records of one source by (hash, target), then the candidate order */
static int rh_qsort_hash_target(const void *a, const void *b) {
    const rh_member *l = (const rh_member *)a, *r = (const rh_member *)b;
    if (l->hash != r->hash) return l->hash < r->hash ? -1 : 1;
    if (l->target != r->target) return l->target < r->target ? -1 : 1;
    return hp_order(l->target, l->hash, l->dist, r->target, r->hash, r->dist);
}

int orc_hashprune_rhalf_reduce(size_t num_points, size_t l_max, const orc_edge_record *records, size_t count,
                               int mode, unsigned hash_quota, unsigned row_cap, float priority_alpha,
                               uint32_t *out_targets, uint16_t *out_hashes, float *out_dists, uint32_t *out_counts,
                               uint32_t *out_primary_counts, uint32_t *bad_record) {
    if (l_max == 0 || mode < ORC_RHALF_HASH_SLOT_1 || mode > ORC_RHALF_HARD_TIER_Q3) return -1;
    const unsigned quota = hash_quota ? hash_quota : (mode == ORC_RHALF_HASH_SLOT_1 ? 1u : 3u);
    if (quota > 3) return -1;
    rh_policy pol;
    pol.mode = mode;
    if (mode == ORC_RHALF_SOFT_TIER_Q3) {
        const float a = priority_alpha > 0.0f ? priority_alpha : 1.1f;
        pol.alpha_sq = a == 1.1f ? 1.21 : (double)a * (double)a;
    } else {
        pol.alpha_sq = 1.0;
    }
    /* primaries: the ordinary reservoir */
    int rc = orc_hashprune_reduce(num_points, l_max, records, count, out_targets, out_hashes, out_dists, out_counts,
                                  bad_record);
    if (rc) return rc;
    /* each source's records, grouped (counting sort by source) */
    size_t *start = (size_t *)calloc(num_points + 1, sizeof(size_t));
    rh_member *mem = (rh_member *)malloc((count ? count : 1) * sizeof(rh_member));
    rh_member *tmp = (rh_member *)malloc((count ? count : 1) * sizeof(rh_member));
    if (!start || !mem || !tmp) {
        free(start);
        free(mem);
        free(tmp);
        return -2;
    }
    for (size_t i = 0; i < count; ++i) start[records[i].src + 1]++;
    for (size_t p = 0; p < num_points; ++p) start[p + 1] += start[p];
    {
        size_t *fill = (size_t *)malloc((num_points ? num_points : 1) * sizeof(size_t));
        if (!fill) {
            free(start);
            free(mem);
            free(tmp);
            return -2;
        }
        memcpy(fill, start, num_points * sizeof(size_t));
        for (size_t i = 0; i < count; ++i) {
            const orc_edge_record *e = &records[i];
            mem[fill[e->src]++] = (rh_member){e->dst, e->dist, e->hash, 0};
        }
        free(fill);
    }
    const size_t budget = l_max / 2;
    const size_t cap_row = (row_cap && row_cap < budget) ? row_cap : budget;
    g_rh_policy = &pol;
    for (size_t p = 0; p < num_points; ++p) {
        const size_t pc = out_counts[p];
        out_primary_counts[p] = (uint32_t)pc;
        if (pc == 0 || pc == l_max) continue;
        const size_t spare = l_max - pc;
        const size_t capacity = cap_row < spare ? cap_row : spare;
        rh_member *m = mem + start[p];
        const size_t n = start[p + 1] - start[p];
        qsort(m, n, sizeof(rh_member), rh_qsort_hash_target);
        size_t nt = 0; /* shortlist candidates, in tmp */
        const uint32_t *pt = out_targets + p * l_max;
        const uint16_t *ph = out_hashes + p * l_max;
        size_t i = 0, slot = 0;
        while (i < n) {
            const uint16_t h = m[i].hash;
            size_t j = i;
            while (j < n && m[j].hash == h) ++j;
            while (slot < pc && ph[slot] < h) ++slot;
            if (slot < pc && ph[slot] == h) {
                /* distinct targets at their best distance, primary's target excluded */
                const size_t g0 = nt;
                for (size_t a = i; a < j;) {
                    size_t b = a + 1;
                    while (b < j && m[b].target == m[a].target) ++b; /* m[a] is the target's best */
                    if (m[a].target != pt[slot]) tmp[nt++] = m[a];
                    a = b;
                }
                qsort(tmp + g0, nt - g0, sizeof(rh_member), rh_qsort_candidate);
                size_t keep = nt - g0 < quota ? nt - g0 : quota;
                for (size_t q = 0; q < keep; ++q) tmp[g0 + q].layer = (uint32_t)(q + 1);
                nt = g0 + keep;
            }
            i = j;
        }
        qsort(tmp, nt, sizeof(rh_member), rh_qsort_priority);
        const size_t take = nt < capacity ? nt : capacity;
        for (size_t q = 0; q < take; ++q) {
            out_targets[p * l_max + pc + q] = tmp[q].target;
            if (out_hashes) out_hashes[p * l_max + pc + q] = tmp[q].hash;
            if (out_dists) out_dists[p * l_max + pc + q] = tmp[q].dist;
        }
        out_counts[p] = (uint32_t)(pc + take);
    }
    free(start);
    free(mem);
    free(tmp);
    return 0;
}
