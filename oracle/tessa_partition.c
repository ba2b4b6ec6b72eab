/*
 * tessa_partition.c -- CPU restatement of the persistent subtree partition
 * (recursive RBC split of one resident subtree into leaves).
 *
 * TEST INFRASTRUCTURE ONLY (see tessa_oracle.h).
 *
 * Reference (paths relative to shear-core/src/algorithm/pipnn/):
 *   compute_backend.rs:12456-12646  gpu_persistent_stage_large_node
 *   compute_backend.rs:15047-15727  large task COUNT / EMIT / SCATTER / PUBLISH
 *   compute_backend.rs:12648-13078  gpu_persistent_process_node (small nodes)
 *   compute_backend.rs:5991-6019    gpu_persistent_sample_large_retry_leaders
 *   compute_backend.rs:6524-6580    gpu_persistent_assignment_insert_candidate
 *   compute_backend.rs:7044-7121    adaptive psamp, terminal limit,
 *                                   meaningful split, sort_unique
 *   compute_backend.rs:11735-11839  gpu_persistent_push_leaf (leaf layout)
 *
 * Order.  The reference walks the tree through a concurrent queue and
 * scatters child rows with atomics, so its leaf numbering and the member
 * order inside a leaf depend on timing (atomicAdd at :15615/:15625 and
 * :11752-11760).  This restatement fixes one legal schedule of that
 * algorithm: nodes are processed level by level in publication order, a
 * node's children are published in leader-slot order, and the rows of a child
 * keep the order they had in the parent.  The HIP implementation follows the
 * same schedule, so the two agree row for row.
 */
#include "tessa_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define P_MAX_LEADERS 128u /* GPU_QUEUE_LEADER_STRIDE compute_backend.rs:371 */

typedef struct {
    uint32_t *rows; /* owned */
    uint32_t n;
    uint32_t depth;
    uint64_t seed;
} pnode;

typedef struct {
    const int8_t *codes;
    const float *scales;
    const float *norms;
    size_t resident_rows;
    size_t padded_dim;
    const orc_subtree_cfg *cfg;
    uint64_t *ctr;
    uint32_t *leaf_row_ids;
    uint64_t *leaf_starts;
    uint64_t *leaf_sizes;
    uint64_t leaf_count;
    uint64_t leaf_rows;
    pnode *next;
    size_t next_len, next_cap;
    int oom;
} pctx;

static void flag(pctx *c, uint64_t f) { c->ctr[ORC_P_OVERFLOW_FLAGS] |= f; }
static void cmax(pctx *c, int i, uint64_t v) { if (v > c->ctr[i]) c->ctr[i] = v; }
static void cmin(pctx *c, int i, uint64_t v) { if (v < c->ctr[i]) c->ctr[i] = v; }

/* compute_backend.rs:7044-7075 */
float orc_adaptive_psamp(float base, uint32_t cluster_size, uint32_t depth) {
    float frac = base;
    if (cluster_size >= 20000000u) frac *= 0.05f;
    else if (cluster_size >= 10000000u) frac *= 0.1f;
    else if (cluster_size >= 5000000u) frac *= 0.2f;
    else if (cluster_size >= 1000000u) frac *= 0.4f;
    else if (cluster_size >= 100000u) frac *= 0.7f;
    if (depth > 4u) frac *= 0.35f;
    else if (depth > 2u) frac *= 0.5f;
    else if (depth > 0u) frac *= 0.8f;
    if (frac < 0.00005f) frac = 0.00005f;
    if (frac > 0.1f) frac = 0.1f;
    return frac;
}

/* compute_backend.rs:7082-7101 */
int orc_meaningful_split(uint32_t parent_rows, uint32_t max_child_rows, uint32_t terminal_limit) {
    if (parent_rows <= terminal_limit || max_child_rows <= terminal_limit) return 1;
    if (max_child_rows >= parent_rows) return 0;
    uint32_t min_shrink = parent_rows >> 5;
    if (min_shrink < 32u) min_shrink = 32u;
    if (min_shrink >= parent_rows) min_shrink = 1u;
    return max_child_rows + min_shrink <= parent_rows;
}

/* (uint32)(psamp * (float)n + 0.5f) with the multiply and add rounded
 * separately (compute_backend.rs:12542, :12761), clamped to [2, max]. */
static uint32_t base_leader_count(float psamp, uint32_t n, uint32_t max_leaders) {
    float prod = psamp * (float)n;
    float sum = prod + 0.5f;
    uint32_t b = (uint32_t)sum;
    if (b < 2u) b = 2u;
    if (b > max_leaders) b = max_leaders;
    return b;
}

/* compute_backend.rs:6524-6580 with `slots` = local fanout (1..4) and the
 * SQ8 distance of :6400-6411 evaluated without contraction. */
static void best_slots(const pctx *c, uint32_t point, const uint32_t *leaders, uint32_t nl,
                       uint32_t slots, uint32_t *out_slots) {
    float bd[4] = {FLT_MAX, FLT_MAX, FLT_MAX, FLT_MAX};
    uint32_t bs[4] = {ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID};
    uint32_t bl[4] = {ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID};
    const size_t pd = c->padded_dim;
    for (uint32_t s = 0; s < nl; ++s) {
        const uint32_t l = leaders[s];
        int32_t dot = orc_sq8_dot(c->codes + (size_t)point * pd, c->codes + (size_t)l * pd, pd);
        float d = orc_sq8_assign_l2(dot, c->scales[point], c->norms[point], c->scales[l], c->norms[l]);
        if (!orc_assign_before(d, point, l, bd[slots - 1], bl[slots - 1])) continue;
        uint32_t pos = slots - 1;
        while (pos > 0 && orc_assign_before(d, point, l, bd[pos - 1], bl[pos - 1])) {
            bd[pos] = bd[pos - 1];
            bs[pos] = bs[pos - 1];
            bl[pos] = bl[pos - 1];
            --pos;
        }
        bd[pos] = d;
        bs[pos] = s;
        bl[pos] = l;
    }
    for (uint32_t k = 0; k < slots; ++k) out_slots[k] = bs[k];
}

/* compute_backend.rs:11735-11763 + :7123-7131: one leaf descriptor. */
static int push_leaf(pctx *c, const uint32_t *rows, uint32_t n) {
    uint64_t idx = c->leaf_count++;
    c->ctr[ORC_P_OUTPUT_LEAF_COUNT] = c->leaf_count;
    if (idx >= c->cfg->max_leaf_count) {
        flag(c, ORC_OVF_LEAF_DESC);
        return -1;
    }
    uint64_t start = c->leaf_rows;
    c->leaf_rows += n;
    c->ctr[ORC_P_OUTPUT_ROWS] = c->leaf_rows;
    if (start + n > c->cfg->max_leaf_rows) {
        flag(c, ORC_OVF_LEAF_ROW);
        return -1;
    }
    cmin(c, ORC_P_LEAF_SIZE_MIN, n);
    cmax(c, ORC_P_LEAF_SIZE_MAX, n);
    c->ctr[ORC_P_LEAF_SIZE_SUM] += n;
    c->ctr[ORC_P_LEAF_SIZE_COUNT] += 1;
    c->leaf_starts[idx] = start;
    c->leaf_sizes[idx] = n;
    memcpy(c->leaf_row_ids + start, rows, (size_t)n * 4);
    return 0;
}

static int publish(pctx *c, const uint32_t *rows, uint32_t n, uint32_t depth, uint64_t seed) {
    if (c->next_len == c->next_cap) {
        size_t cap = c->next_cap ? 2 * c->next_cap : 16;
        pnode *p = (pnode *)realloc(c->next, cap * sizeof(pnode));
        if (!p) { c->oom = 1; return -1; }
        c->next = p;
        c->next_cap = cap;
    }
    uint32_t *copy = (uint32_t *)malloc((size_t)(n ? n : 1) * 4);
    if (!copy) { c->oom = 1; return -1; }
    memcpy(copy, rows, (size_t)n * 4);
    pnode *q = &c->next[c->next_len++];
    q->rows = copy;
    q->n = n;
    q->depth = depth;
    q->seed = seed;
    return 0;
}

static uint32_t rel_depth(const pctx *c, uint32_t depth) {
    return depth >= c->cfg->root_depth ? depth - c->cfg->root_depth : 0u;
}

static int grow_u32(uint32_t **v, size_t *cap, size_t need) {
    if (need <= *cap) return 0;
    size_t cap2 = *cap ? *cap : 1024;
    while (cap2 < need) cap2 *= 2;
    uint32_t *p = (uint32_t *)realloc(*v, cap2 * 4);
    if (!p) return -1;
    *v = p;
    *cap = cap2;
    return 0;
}

void orc_pass_trace_free(orc_pass_trace *t) {
    if (!t) return;
    free(t->passes);
    free(t->rows);
    memset(t, 0, sizeof(*t));
}

/* One COUNT pass into the trace (test infrastructure; no reference code). */
static void trace_pass(pctx *c, const pnode *nd, uint32_t attempt, uint32_t fanout, const uint32_t *leaders,
                       uint32_t nl) {
    orc_pass_trace *t = c->cfg->trace;
    if (!t || nd->n < c->cfg->trace_min_members) return;
    if (grow_u32(&t->passes, &t->pass_cap, t->pass_len + 5) ||
        grow_u32(&t->rows, &t->row_cap, t->row_len + nd->n + nl)) {
        c->oom = 1;
        return;
    }
    uint32_t *w = t->passes + t->pass_len;
    w[0] = nd->depth;
    w[1] = attempt;
    w[2] = fanout;
    w[3] = nd->n;
    w[4] = nl;
    t->pass_len += 5;
    memcpy(t->rows + t->row_len, nd->rows, (size_t)nd->n * 4);
    memcpy(t->rows + t->row_len + nd->n, leaders, (size_t)nl * 4);
    t->row_len += (size_t)nd->n + nl;
}

/* compute_backend.rs:12456-12646 (stage) + :15047-15727 (COUNT, EMIT,
 * SCATTER, PUBLISH) for one node. */
static void process_large(pctx *c, const pnode *nd) {
    const orc_subtree_cfg *cfg = c->cfg;
    const uint32_t n = nd->n;
    if (n == 0) return;
    if (nd->depth >= cfg->max_depth) { flag(c, ORC_OVF_OVERSIZED_TERMINAL_NODE); return; }
    if ((uint64_t)n > cfg->large_scratch_rows) { flag(c, ORC_OVF_QUEUE_ROW); return; }
    c->ctr[ORC_P_LARGE_NODE_CLAIMS] += 1;
    c->ctr[ORC_P_LARGE_NODE_ROWS] += n;
    cmax(c, ORC_P_LARGE_NODE_MAX_ROWS, n);
    uint32_t retry_max = n < 2u ? 2u : n;
    if (retry_max > P_MAX_LEADERS) retry_max = P_MAX_LEADERS;
    uint32_t max_leaders = cfg->max_leaders < retry_max ? cfg->max_leaders : retry_max;
    if (max_leaders < 2u) max_leaders = 2u;
    const uint32_t rel = rel_depth(c, nd->depth);
    const int use_root = rel == 0 && cfg->root_leader_count > 0;
    const float psamp = orc_adaptive_psamp(cfg->psamp_fraction, n, nd->depth);
    uint32_t nl = use_root ? cfg->root_leader_count : base_leader_count(psamp, n, max_leaders);
    if (nl > max_leaders) nl = max_leaders;
    uint32_t req = rel == 0 ? cfg->fanout_second : 1u;
    if (req < 1u) req = 1u;
    if (req > 4u) { flag(c, ORC_OVF_FANOUT_OVER_32); return; }
    uint32_t fanout = req < nl ? req : nl;
    cmax(c, ORC_P_EFFECTIVE_ROOT_FANOUT, rel == 0 ? fanout : 0u);
    cmax(c, ORC_P_EFFECTIVE_DEEPER_FANOUT, rel > 0 ? fanout : 1u);

    uint32_t leaders[P_MAX_LEADERS];
    for (uint32_t s = 0; s < nl; ++s) {
        if (use_root) {
            leaders[s] = cfg->root_leaders[s];
        } else {
            uint32_t ord = (uint32_t)(((uint64_t)s * n) / nl);
            if (ord >= n) ord = n - 1u;
            leaders[s] = nd->rows[ord];
        }
    }
    uint32_t *slots = (uint32_t *)malloc((size_t)n * 4 * sizeof(uint32_t));
    uint32_t counts[P_MAX_LEADERS];
    if (!slots) { c->oom = 1; return; }
    const int retry_allowed = !use_root;
    uint32_t attempt = 0;
    int balanced = 0;
    for (;;) {
        memset(counts, 0, sizeof(counts));
        trace_pass(c, nd, attempt, fanout, leaders, nl);
        c->ctr[ORC_P_LARGE_PHYSICAL_TILES] += (n + 15u) / 16u;
        /* rows are independent: OpenMP over rows, counted afterwards */
#pragma omp parallel for schedule(static)
        for (long long r = 0; r < (long long)n; ++r)
            best_slots(c, nd->rows[r], leaders, nl, fanout, slots + (size_t)r * 4);
        for (uint32_t r = 0; r < n; ++r) {
            for (uint32_t k = 0; k < fanout; ++k) {
                uint32_t s = slots[(size_t)r * 4 + k];
                if (s < nl) counts[s]++;
                else flag(c, ORC_OVF_QUEUE_ROW);
            }
        }
        /* EMIT :15402-15420 */
        uint64_t running = 0;
        uint32_t nonempty = 0, max_child = 0;
        for (uint32_t s = 0; s < nl; ++s) {
            running += counts[s];
            if (counts[s]) {
                nonempty++;
                if (counts[s] > max_child) max_child = counts[s];
            }
        }
        if (running > cfg->large_scratch_rows) { flag(c, ORC_OVF_QUEUE_ROW); free(slots); return; }
        if (nonempty > 1u && orc_meaningful_split(n, max_child, cfg->leaf_max)) break;
        if (retry_allowed && (attempt == 0u || nl < max_leaders)) {
            /* :15424-15440 leader count for the retry */
            uint32_t next = nl;
            if (attempt > 0u) {
                uint32_t doubled = next << 1;
                next = (doubled > next && doubled < max_leaders) ? doubled : max_leaders;
            }
            if (next > max_leaders) next = max_leaders;
            attempt += 1u;
            orc_sample_retry_leaders(nd->rows, n, next, nd->seed, attempt, leaders);
            nl = next;
            c->ctr[ORC_P_LARGE_SPLIT_RETRIES] += 1;
            continue;
        }
        /* :15485-15510 balanced even/odd fallback */
        balanced = 1;
        nl = 2u;
        fanout = 1u;
        c->ctr[ORC_P_LARGE_BALANCED_FALLBACKS] += 1;
        break;
    }
    if (balanced) {
        c->ctr[ORC_P_FANOUT_ASSIGNMENT_SLOTS] += n;
        c->ctr[ORC_P_REPLICATED_ROWS] += n;
    } else {
        c->ctr[ORC_P_FANOUT_ASSIGNMENT_SLOTS] += (uint64_t)n * fanout;
        c->ctr[ORC_P_REPLICATED_ROWS] += (uint64_t)n * fanout;
    }
    /* SCATTER (:15556-15648) in parent row order, then PUBLISH (:15650-15727). */
    uint32_t *child = (uint32_t *)malloc((size_t)n * 4);
    if (!child) { free(slots); c->oom = 1; return; }
    c->ctr[ORC_P_ASSIGNMENT_PASSES] += 1;
    c->ctr[ORC_P_LARGE_NODE_SPLITS] += 1;
    for (uint32_t s = 0; s < nl; ++s) {
        uint32_t len = 0;
        for (uint32_t r = 0; r < n; ++r) {
            int hit = 0;
            if (balanced) {
                hit = (r & 1u) == s;
            } else {
                for (uint32_t k = 0; k < fanout; ++k) hit |= slots[(size_t)r * 4 + k] == s;
            }
            if (hit) child[len++] = nd->rows[r];
        }
        if (len == 0) continue;
        if (len <= cfg->leaf_max) {
            if (push_leaf(c, child, len)) break;
        } else if (nd->depth + 1u >= cfg->max_depth) {
            flag(c, ORC_OVF_OVERSIZED_TERMINAL_NODE);
            break;
        } else {
            uint64_t cs = nd->seed ^ ((uint64_t)s * 0x94d049bb133111ebull) ^ (((uint64_t)len) << 23);
            if (publish(c, child, len, nd->depth + 1u, cs)) break;
        }
    }
    free(child);
    free(slots);
}

/* compute_backend.rs:12648-13078 gpu_persistent_process_node.  Only a subtree
 * root can reach it: every published child is larger than leaf_max. */
static void process_small(pctx *c, const pnode *nd) {
    const orc_subtree_cfg *cfg = c->cfg;
    uint32_t n = nd->n;
    if (n == 0) return;
    if (n > cfg->small_node_limit) { flag(c, ORC_OVF_QUEUE_ROW); return; }
    uint32_t *pts = (uint32_t *)malloc((size_t)n * 4);
    if (!pts) { c->oom = 1; return; }
    memcpy(pts, nd->rows, (size_t)n * 4);
    orc_sort_unique(pts, &n);
    if (n == 0) { free(pts); return; }
    cmax(c, ORC_P_MAX_ACTIVE, n);
    const uint32_t terminal = cfg->leaf_max;
    const uint32_t merge_min = cfg->leaf_min;
    const uint32_t rel = rel_depth(c, nd->depth);
    const int probe = rel == 0 && cfg->fanout_second > 1u && n > 1u;
    if (n <= terminal && !probe) { push_leaf(c, pts, n); free(pts); return; }
    if (nd->depth >= cfg->max_depth) { flag(c, ORC_OVF_OVERSIZED_TERMINAL_NODE); free(pts); return; }
    uint32_t max_leaders = cfg->max_leaders < n ? cfg->max_leaders : n;
    if (max_leaders < 2u) max_leaders = 2u;
    if (max_leaders > P_MAX_LEADERS) { flag(c, ORC_OVF_LEADER); free(pts); return; }
    const float psamp = orc_adaptive_psamp(cfg->psamp_fraction, n, nd->depth);
    const uint32_t base = base_leader_count(psamp, n, max_leaders);
    const int use_root = rel == 0 && cfg->root_leader_count > 0;
    const uint32_t attempts = use_root ? 1u : 6u;

    uint32_t *slots = (uint32_t *)malloc((size_t)n * 4 * sizeof(uint32_t));
    uint32_t *clustered = (uint32_t *)malloc(4096 * 4);
    uint32_t *merged = (uint32_t *)malloc(2 * 4096 * 4);
    uint32_t *small = (uint32_t *)malloc(2 * 4096 * 4);
    uint32_t leaders[P_MAX_LEADERS], child_off[P_MAX_LEADERS + 1], child_cnt[P_MAX_LEADERS + 1];
    uint32_t start[P_MAX_LEADERS], cnt[P_MAX_LEADERS];
    uint32_t split = 0;
    int ok = 0;
    if (!slots || !clustered || !merged || !small) { c->oom = 1; goto done; }
    for (uint32_t attempt = 0; attempt < attempts; ++attempt) {
        uint32_t nl = use_root ? cfg->root_leader_count : (base << attempt);
        if (nl > max_leaders) nl = max_leaders;
        if (use_root) {
            for (uint32_t s = 0; s < nl; ++s) leaders[s] = cfg->root_leaders[s];
        } else {
            orc_hash_rank_leaders(pts, n, nl, nd->seed, attempt, nd->depth, leaders);
        }
        uint32_t req = rel == 0 ? cfg->fanout_second : 1u;
        if (req < 1u) req = 1u;
        if (req > 4u) { flag(c, ORC_OVF_FANOUT_OVER_32); goto done; }
        uint32_t fanout = req < nl ? req : nl;
        cmax(c, ORC_P_EFFECTIVE_ROOT_FANOUT, rel == 0 ? fanout : 0u);
        cmax(c, ORC_P_EFFECTIVE_DEEPER_FANOUT, rel > 0 ? fanout : 1u);
        memset(cnt, 0, sizeof(cnt));
        for (uint32_t r = 0; r < n; ++r) {
            best_slots(c, pts[r], leaders, nl, fanout, slots + (size_t)r * 4);
            for (uint32_t k = 0; k < fanout; ++k) {
                uint32_t s = slots[(size_t)r * 4 + k];
                if (s >= nl) { flag(c, ORC_OVF_QUEUE_ROW); goto done; }
                cnt[s]++;
            }
        }
        c->ctr[ORC_P_FANOUT_ASSIGNMENT_SLOTS] += (uint64_t)n * fanout;
        c->ctr[ORC_P_REPLICATED_ROWS] += (uint64_t)n * fanout;
        uint32_t running = 0;
        for (uint32_t s = 0; s < nl; ++s) {
            start[s] = running;
            running += cnt[s];
        }
        if (running > 4096u) { flag(c, ORC_OVF_QUEUE_ROW); goto done; }
        {
            uint32_t w[P_MAX_LEADERS];
            memcpy(w, start, sizeof(uint32_t) * nl);
            for (uint32_t r = 0; r < n; ++r)
                for (uint32_t k = 0; k < fanout; ++k) clustered[w[slots[(size_t)r * 4 + k]]++] = pts[r];
        }
        c->ctr[ORC_P_ASSIGNMENT_PASSES] += 1;
        /* :12923-12996 children with small-child merging */
        split = 0;
        uint32_t merged_rows = 0, small_len = 0, max_child = 0;
        for (uint32_t s = 0; s < nl; ++s) {
            uint32_t count = cnt[s];
            if (count == 0u) continue;
            uint32_t *ch = clustered + start[s];
            orc_sort_unique(ch, &count);
            if (count == 0u) continue;
            if (count < merge_min) {
                memcpy(small + small_len, ch, (size_t)count * 4);
                small_len += count;
                orc_sort_unique(small, &small_len);
                if (small_len >= merge_min) {
                    memcpy(merged + merged_rows, small, (size_t)small_len * 4);
                    child_off[split] = merged_rows;
                    child_cnt[split] = small_len;
                    merged_rows += small_len;
                    if (small_len > max_child) max_child = small_len;
                    split++;
                    small_len = 0;
                }
            } else {
                child_off[split] = merged_rows;
                child_cnt[split] = count;
                memcpy(merged + merged_rows, ch, (size_t)count * 4);
                merged_rows += count;
                if (count > max_child) max_child = count;
                split++;
            }
        }
        if (small_len > 0u) {
            if (split > 0u) {
                uint32_t last = split - 1u;
                uint32_t last_count = child_cnt[last];
                if (last_count + small_len <= terminal) {
                    uint32_t dst = child_off[last] + last_count;
                    memcpy(merged + dst, small, (size_t)small_len * 4);
                    uint32_t mc = last_count + small_len;
                    orc_sort_unique(merged + child_off[last], &mc);
                    child_cnt[last] = mc;
                    if (mc > max_child) max_child = mc;
                    small_len = 0;
                }
            }
            if (small_len > 0u) {
                memcpy(merged + merged_rows, small, (size_t)small_len * 4);
                child_off[split] = merged_rows;
                child_cnt[split] = small_len;
                merged_rows += small_len;
                if (small_len > max_child) max_child = small_len;
                split++;
            }
        }
        if (split > 1u && orc_meaningful_split(n, max_child, terminal)) { ok = 1; break; }
        if (nl >= max_leaders) break;
    }
    if (!ok) {
        if (n > terminal) flag(c, ORC_OVF_OVERSIZED_TERMINAL_NODE | ORC_OVF_NO_PROGRESS_SPLIT);
        else push_leaf(c, pts, n);
        goto done;
    }
    for (uint32_t ci = 0; ci < split; ++ci) {
        uint32_t len = child_cnt[ci];
        if (len == 0u) continue;
        if (len <= terminal) {
            if (push_leaf(c, merged + child_off[ci], len)) break;
        } else if (nd->depth + 1u >= cfg->max_depth) {
            flag(c, ORC_OVF_OVERSIZED_TERMINAL_NODE);
            break;
        } else {
            uint64_t cs = nd->seed ^ ((uint64_t)ci * 0x94d049bb133111ebull) ^ (((uint64_t)len) << 23);
            if (publish(c, merged + child_off[ci], len, nd->depth + 1u, cs)) break;
        }
    }
done:
    free(slots);
    free(clustered);
    free(merged);
    free(small);
    free(pts);
}

/* compute_backend.rs:7103-7121 (insertion sort, then drop repeats). */
void orc_sort_unique(uint32_t *v, uint32_t *len) {
    uint32_t n = *len;
    for (uint32_t i = 1; i < n; ++i) {
        uint32_t key = v[i], j = i;
        while (j > 0 && v[j - 1] > key) {
            v[j] = v[j - 1];
            --j;
        }
        v[j] = key;
    }
    uint32_t out = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (i == 0 || v[i] != v[i - 1]) v[out++] = v[i];
    *len = out;
}

/* compute_backend.rs:5991-6019 */
void orc_sample_retry_leaders(const uint32_t *rows, uint32_t row_count, uint32_t num_leaders,
                              uint64_t seed, uint32_t attempt, uint32_t *leaders) {
    for (uint32_t s = 0; s < num_leaders; ++s) {
        uint32_t b = (uint32_t)(((uint64_t)s * row_count) / num_leaders);
        uint32_t e = (uint32_t)(((uint64_t)(s + 1u) * row_count) / num_leaders);
        if (e <= b) e = b + 1u;
        uint32_t span = e - b;
        uint64_t key = orc_hash64(seed ^ ((uint64_t)attempt * 0xd6e8feb86659fd93ull) ^
                                  ((uint64_t)s * 0x9e3779b97f4a7c15ull));
        leaders[s] = rows[b + (uint32_t)(key % span)];
    }
}

/* compute_backend.rs:12770-12800: keep the num_leaders smallest (key, point)
 * in ascending order by bounded insertion. */
void orc_hash_rank_leaders(const uint32_t *pts, uint32_t n, uint32_t num_leaders, uint64_t seed,
                           uint32_t attempt, uint32_t depth, uint32_t *leaders) {
    uint64_t score[P_MAX_LEADERS];
    for (uint32_t s = 0; s < num_leaders; ++s) {
        leaders[s] = ORC_EMPTY_ID;
        score[s] = UINT64_MAX;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t point = pts[i];
        const uint64_t key = orc_hash64(seed ^ ((uint64_t)attempt * 0xbf58476d1ce4e5b9ull) ^
                                        (((uint64_t)depth) << 19) ^ (((uint64_t)i) << 7) ^
                                        (((uint64_t)point) << 31));
        uint32_t ins = num_leaders;
        for (uint32_t pos = 0; pos < num_leaders; ++pos) {
            if (key < score[pos] || (key == score[pos] && point < leaders[pos])) {
                ins = pos;
                break;
            }
        }
        if (ins < num_leaders) {
            for (uint32_t pos = num_leaders - 1u; pos > ins; --pos) {
                score[pos] = score[pos - 1u];
                leaders[pos] = leaders[pos - 1u];
            }
            score[ins] = key;
            leaders[ins] = point;
        }
    }
}

/* compute_backend.rs:1597-1603 gpu_queue_root_seed */
uint64_t orc_subtree_root_seed(uint64_t random_seed, uint64_t depth, uint64_t point_count,
                               uint64_t parent_points, uint64_t min_recurse_size) {
#define ROTL(x, r) (((x) << (r)) | ((x) >> (64 - (r))))
    return random_seed ^ (depth * 0x9e3779b97f4a7c15ull) ^ ROTL(point_count, 17) ^
           ROTL(parent_points, 7) ^ ROTL(min_recurse_size, 29);
#undef ROTL
}

int orc_subtree_partition(const int8_t *codes, const float *scales, const float *norms,
                          size_t resident_rows, size_t padded_dim, const orc_subtree_cfg *cfg,
                          uint32_t *leaf_row_ids, uint64_t *leaf_starts, uint64_t *leaf_sizes,
                          uint64_t *counters, uint64_t *leaf_count, uint64_t *leaf_rows) {
    if (!cfg || !counters || !leaf_count || !leaf_rows) return -1;
    if (cfg->leaf_max == 0 || cfg->leaf_min == 0 || cfg->max_leaders == 0) return -2;
    if (resident_rows > 0xffffffffull) return -2;
    for (uint32_t i = 0; i < cfg->root_leader_count; ++i)
        if (cfg->root_leaders[i] >= resident_rows) return -3;
    memset(counters, 0, sizeof(uint64_t) * ORC_P_COUNTER_WORDS);
    counters[ORC_P_LEAF_SIZE_MIN] = UINT64_MAX;
    counters[ORC_P_UNIQUE_RESIDENT_ROWS] = resident_rows;
    pctx c;
    memset(&c, 0, sizeof(c));
    c.codes = codes;
    c.scales = scales;
    c.norms = norms;
    c.resident_rows = resident_rows;
    c.padded_dim = padded_dim;
    c.cfg = cfg;
    c.ctr = counters;
    c.leaf_row_ids = leaf_row_ids;
    c.leaf_starts = leaf_starts;
    c.leaf_sizes = leaf_sizes;
    pnode *level = NULL;
    size_t level_len = 0;
    if (resident_rows > 0) {
        level = (pnode *)malloc(sizeof(pnode));
        uint32_t *rows = (uint32_t *)malloc(resident_rows * 4);
        if (!level || !rows) { free(level); free(rows); return -4; }
        for (size_t r = 0; r < resident_rows; ++r) rows[r] = (uint32_t)r;
        level[0].rows = rows;
        level[0].n = (uint32_t)resident_rows;
        level[0].depth = cfg->root_depth;
        level[0].seed = cfg->seed;
        level_len = 1;
    }
    /* compute_backend.rs:16835-16842 routing: nodes above leaf_max, and a
     * root whose fanout probe would overflow the small-node scratch, take the
     * large-task path; the rest go to process_node. */
    while (level_len > 0) {
        counters[ORC_P_PARTITION_LEVEL_ROUNDS] += 1;
        c.next = NULL;
        c.next_len = c.next_cap = 0;
        for (size_t i = 0; i < level_len; ++i) {
            const pnode *nd = &level[i];
            counters[ORC_P_PARTITION_POPS] += 1;
            const uint32_t rel = rel_depth(&c, nd->depth);
            const int probe = rel == 0 && cfg->fanout_second > 1u && nd->n > 1u;
            const int probe_overflow =
                probe && (uint64_t)nd->n * cfg->fanout_second > (uint64_t)cfg->small_node_limit;
            if (nd->n > cfg->leaf_max || probe_overflow) process_large(&c, nd);
            else process_small(&c, nd);
            if (c.oom) break;
        }
        for (size_t i = 0; i < level_len; ++i) free(level[i].rows);
        free(level);
        level = c.next;
        level_len = c.next_len;
        if (c.oom || counters[ORC_P_OVERFLOW_FLAGS] != 0) break;
    }
    for (size_t i = 0; i < level_len; ++i) free(level[i].rows);
    free(level);
    if (c.oom) return -4;
    *leaf_count = c.leaf_count;
    *leaf_rows = c.leaf_rows;
    return 0;
}
