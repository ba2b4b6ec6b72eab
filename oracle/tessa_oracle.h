/*
 * tessa_oracle.h -- CPU restatement of the reference TESSA operator semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * implementation in shear_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product path never calls it.
 *
 * Every function names the reference file:line whose behaviour it restates
 * (paths are relative to shear-core/src/algorithm/pipnn/ in the reference).
 *
 * Pinning (what checks each function, besides retyping the formula):
 *   orc_sq8_quantize      reference KATs dco_sq_int8.rs:3261-3299 (codes, scale
 *                         bits, norm, zero row), round-half-away-from-zero and
 *                         clamp cases, bit-width variants (4-bit KAT).
 *   orc_sq8_dot*          brute-force int64 sum; VNNI/AVX2 == scalar on random
 *                         and extreme (+-127) codes; KAT dco_sq_int8.rs:3301-3325.
 *   orc_sq8_leaf_l2       KAT 127*64+64*127 dot; closed form evaluated in
 *                         float64 then rounded step by step; d<=0 -> 0 clamp.
 *   orc_rowtopk_push      brute force: with no eps-ties the result equals a
 *                         stable sort by distance; tie KAT (smaller id wins
 *                         within 2e-5); non-transitive chain example whose
 *                         answer is worked by hand (order dependence).
 *   orc_leaf_topk_batch   brute force on tiny leaves via an independent numpy
 *                         restatement; invariants (self never listed, ids are
 *                         members, k_eff = min(k, n-1)).
 *   orc_assign_replay     hash64 == SplitMix64 finalizer known outputs; without
 *                         near-ties equals the strict (dist, id) order of the
 *                         CPU D0 path (orc_assign_strict).
 *   orc_compute_hash /    the reference's own fixture batch (leaf_build.rs:3126-3137
 *   orc_flush_compact_    with build_test_sketches :2900-2908), whose edges follow
 *   topk_into_edges       in closed form; an independent numpy restatement on random
 *                         batches; the empty-slot, non-finite and outside-leaf cases.
 *   orc_hashprune_reduce  the reference's reservoir KATs (hash_prune.rs:4803-4875:
 *                         exact-distance replacement inside one BF16 bucket, same-hash
 *                         collision, 1.5e-5 band, permutation-independent epsilon
 *                         cycle); brute force: the l_max best (dist, target, hash)
 *                         among each hash's best candidate, listed by ascending hash;
 *                         invariance under every shuffle of the record stream.
 *   orc_d0_assign         brute force in f64 on well-separated distances, a row's own
 *                         leader first, ties by leader id on duplicated leaders,
 *                         fanout = leader count giving the full order, the grouping
 *                         against a sort of the fragments.
 *   orc_robust_prune      hand-worked occlusions (a point behind a kept one dropped, two
 *                         orthogonal ones kept, one kept only in the alpha = 1.2 pass),
 *                         the degree cap, self-loops and zero distances, saturation.
 *   orc_greedy_search     brute force: on a complete graph (every point lists every
 *                         other) with L >= n the search visits everything and
 *                         returns the exact K nearest; the neighbour-queue rules
 *                         (full-list rejection, cursor rewind on an insert in front
 *                         of it) on hand-built graphs whose search is worked by hand.
 */
#ifndef TESSA_ORACLE_H
#define TESSA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* mod.rs:74 STABLE_DISTANCE_TIE_EPS */
#define ORC_TIE_EPS 2.0e-5f
/* dco_sq_int8.rs:14 SQ_INT8_DEFAULT_K_ALIGN */
#define ORC_SQ8_K_ALIGN 16u
#define ORC_EMPTY_ID 0xffffffffu

/* dco_sq_int8.rs:1216-1224 sq_int8_padded_dim (0 on dim == 0). */
size_t orc_sq8_padded_dim(size_t dim, size_t k_align);

/* dco_sq_int8.rs:1340-1375 + 1431-1467: per-vector symmetric quantizer.
 * Returns 0, or -1 when a value is non-finite (its row in *bad_row), or -2 on
 * bad arguments.  codes is rows*padded_dim, zero padded. */
int orc_sq8_quantize(const float *x, size_t rows, size_t dim, size_t padded_dim,
                     unsigned bits, int8_t *codes, float *scales, float *norms,
                     size_t *bad_row);

/* dco_sq_int8.rs:2685-2691 scalar dot; the dispatching version uses the best
 * SIMD path present (dco_sq_int8.rs:2813-2948 analogue). */
int32_t orc_sq8_dot_scalar(const int8_t *a, const int8_t *b, size_t n);
int32_t orc_sq8_dot(const int8_t *a, const int8_t *b, size_t n);
/* Which dot path orc_sq8_dot uses: 0 scalar, 1 avx2, 2 avx512-vnni. */
int orc_sq8_dot_kernel(void);
/* Force a path (for the SIMD == scalar tests); returns the previous one. */
int orc_sq8_set_dot_kernel(int kernel);

/* compute_backend.rs:8987-9002 (== dco_sq_int8.rs:2950-2965):
 * (rn + cn) + (-2 * ((rs * cs) * (float)dot)), then d <= 0 -> 0. */
float orc_sq8_leaf_l2(int32_t dot, float row_scale, float row_norm,
                      float col_scale, float col_norm);

/* rbc_partition.rs:17630-17639 (== compute_backend.rs:6400-6411 without
 * contraction): (pn + ln) - ((2 * ps) * ls) * (float)dot, then d <= 0 -> 0. */
float orc_sq8_assign_l2(int32_t dot, float point_scale, float point_norm,
                        float leader_scale, float leader_norm);

/* mod.rs:417-428 stable_distance_order(...).is_lt(): candidate c beats s. */
int orc_beats(float dc, uint32_t idc, float ds, uint32_t ids);

/* leaf_build.rs:887-957 RowTopK::push (k <= 32). */
void orc_rowtopk_push(uint32_t k, float d, uint32_t id, float *best_d,
                      uint32_t *best_id, uint32_t *len);

/* Leaf operator over replay layouts (tessa_replay.rs:1021-1057 TessaLeafLayout,
 * semantics leaf_build.rs:1566-1590 with the SQ8 distance): for every member
 * row, every other member column in member order is pushed into RowTopK.
 * Output slot [output_offset + row*k + rank] = (global id, distance); slots
 * past k_eff = min(k, n-1) are (0xffffffff, FLT_MAX).
 * threads <= 0 uses all OpenMP threads.  Returns 0 or a negative error. */
int orc_leaf_topk_batch(const int8_t *codes, const float *scales,
                        const float *norms, const uint32_t *global_ids,
                        size_t resident_rows, size_t padded_dim,
                        const uint32_t *members, const uint64_t *member_offsets,
                        const uint32_t *member_counts,
                        const uint64_t *output_offsets, size_t leaf_count,
                        uint32_t k, uint32_t *out_ids, float *out_dists,
                        int threads);

/* compute_backend.rs:5983-5989 gpu_persistent_hash64 (SplitMix64 finalizer). */
uint64_t orc_hash64(uint64_t x);
/* compute_backend.rs:6513-6522 tie key. */
uint64_t orc_assign_tie_key(uint32_t point, uint32_t leader);

/* Assignment replay (compute_backend.rs:15729-15943 with best_slots4_no_dco
 * :6618-6699 and insert :6524-6580): per member, leaders visited in slot
 * order into 4 slots with the 2e-5 eps / hash tie key rule; output rank r of
 * member row m at output_offset + m*r_h + r = (global id of leader, dist). */
int orc_assign_replay(const int8_t *codes, const float *scales,
                      const float *norms, const uint32_t *global_ids,
                      size_t resident_rows, size_t padded_dim,
                      const uint32_t *members, const uint32_t *leaders,
                      const uint32_t *member_offsets,
                      const uint32_t *member_counts,
                      const uint32_t *leader_offsets,
                      const uint32_t *leader_counts, const uint32_t *r_h,
                      const uint64_t *output_offsets, size_t task_count,
                      uint32_t *out_ids, float *out_dists, int threads);

/* CPU D0 path (rbc_partition.rs:17453-17608, compare :17714-17733): strict
 * (dist, leader global id) order, same output layout as orc_assign_replay. */
int orc_assign_strict(const int8_t *codes, const float *scales,
                      const float *norms, const uint32_t *global_ids,
                      size_t resident_rows, size_t padded_dim,
                      const uint32_t *members, const uint32_t *leaders,
                      const uint32_t *member_offsets,
                      const uint32_t *member_counts,
                      const uint32_t *leader_offsets,
                      const uint32_t *leader_counts, const uint32_t *r_h,
                      const uint64_t *output_offsets, size_t task_count,
                      uint32_t *out_ids, float *out_dists, int threads);

/* compute_backend.rs:6541-6568: does (d, leader) go before (od, oleader)
 * for this point?  Within 2e-5 the SplitMix64 tie key, then leader id. */
int orc_assign_before(float d, uint32_t point, uint32_t leader, float od, uint32_t oleader);

/* ---- subtree partition (tessa_partition.c) ------------------------------ */

/* Overflow bits, compute_backend.rs:4843-4860 */
#define ORC_OVF_QUEUE_NODE              (1ull << 0)
#define ORC_OVF_QUEUE_ROW               (1ull << 1)
#define ORC_OVF_LEAF_DESC               (1ull << 2)
#define ORC_OVF_LEAF_ROW                (1ull << 3)
#define ORC_OVF_LEADER                  (1ull << 4)
#define ORC_OVF_FANOUT_OVER_32          (1ull << 5)
#define ORC_OVF_NO_PROGRESS_SPLIT       (1ull << 7)
#define ORC_OVF_OVERSIZED_TERMINAL_NODE (1ull << 10)

/* Counter words used by the partition, at the reference's indices
 * (compute_backend.rs:5028-5187, 159 words). */
#define ORC_P_COUNTER_WORDS 159
enum {
    ORC_P_LEAF_PUSHES = 9,
    ORC_P_OVERFLOW_FLAGS = 7,
    ORC_P_PARTITION_POPS = 8,
    ORC_P_OUTPUT_ROWS = 12,
    ORC_P_OUTPUT_LEAF_COUNT = 13,
    ORC_P_ASSIGNMENT_PASSES = 14,
    ORC_P_MAX_ACTIVE = 15,
    ORC_P_EFFECTIVE_ROOT_FANOUT = 17,
    ORC_P_EFFECTIVE_DEEPER_FANOUT = 18,
    ORC_P_FANOUT_ASSIGNMENT_SLOTS = 19,
    ORC_P_REPLICATED_ROWS = 20,
    ORC_P_UNIQUE_RESIDENT_ROWS = 21,
    ORC_P_LARGE_NODE_CLAIMS = 27,
    ORC_P_LARGE_NODE_SPLITS = 28,
    ORC_P_LARGE_NODE_ROWS = 29,
    ORC_P_LARGE_NODE_MAX_ROWS = 30,
    ORC_P_LEAF_SIZE_MIN = 33,
    ORC_P_LEAF_SIZE_MAX = 34,
    ORC_P_LEAF_SIZE_SUM = 35,
    ORC_P_LEAF_SIZE_COUNT = 36,
    ORC_P_PARTITION_LEVEL_ROUNDS = 119,
    ORC_P_LARGE_SPLIT_RETRIES = 130,
    ORC_P_LARGE_BALANCED_FALLBACKS = 131,
    ORC_P_LARGE_PHYSICAL_TILES = 145
};

typedef struct orc_subtree_cfg {
    const uint32_t *root_leaders; /* resident row ids; NULL when count == 0 */
    uint32_t root_leader_count;
    uint32_t root_depth;          /* request.depth */
    uint32_t max_depth;           /* params.max_depth */
    uint32_t max_leaders;         /* params.max_leaders */
    uint32_t fanout_second;       /* params.fanout_second (1..4) */
    uint32_t leaf_min;            /* plan leaf_min (merge threshold) */
    uint32_t leaf_max;            /* plan leaf_max = max(256, c_max) */
    uint32_t small_node_limit;    /* plan small_node_limit (4096) */
    uint64_t large_scratch_rows;  /* plan large_scratch_rows */
    uint64_t max_leaf_count;
    uint64_t max_leaf_rows;
    float psamp_fraction;         /* params.psamp_fraction as f32 */
    uint64_t seed;                /* orc_subtree_root_seed(...) */
    /* Optional trace of the COUNT passes of nodes with >= trace_min_members
     * rows (NULL: off): the passes the reference's in-kernel sampler sees
     * (compute_backend.rs:5415-5546), for checking a GPU capture. */
    uint32_t trace_min_members;
    struct orc_pass_trace *trace;
} orc_subtree_cfg;

/* Growable trace: per pass 5 words (depth, attempt, fanout, members,
 * leaders) in `passes`; members then leaders (resident rows) in `rows`. */
typedef struct orc_pass_trace {
    uint32_t *passes;
    size_t pass_len, pass_cap;
    uint32_t *rows;
    size_t row_len, row_cap;
} orc_pass_trace;
void orc_pass_trace_free(orc_pass_trace *t);

/* compute_backend.rs:7044-7075, 7082-7101, 7103-7121 */
float orc_adaptive_psamp(float base, uint32_t cluster_size, uint32_t depth);
int orc_meaningful_split(uint32_t parent_rows, uint32_t max_child_rows, uint32_t terminal_limit);
void orc_sort_unique(uint32_t *v, uint32_t *len);
/* compute_backend.rs:5991-6019 */
void orc_sample_retry_leaders(const uint32_t *rows, uint32_t row_count, uint32_t num_leaders,
                              uint64_t seed, uint32_t attempt, uint32_t *leaders);
/* compute_backend.rs:12770-12800 hash-ranked leaders of a small node. */
void orc_hash_rank_leaders(const uint32_t *pts, uint32_t n, uint32_t num_leaders, uint64_t seed,
                           uint32_t attempt, uint32_t depth, uint32_t *leaders);
/* compute_backend.rs:1597-1603 */
uint64_t orc_subtree_root_seed(uint64_t random_seed, uint64_t depth, uint64_t point_count,
                               uint64_t parent_points, uint64_t min_recurse_size);

/* Recursive partition of resident rows 0..resident_rows-1 into leaves
 * (leaf_row_ids / leaf_starts / leaf_sizes, compute_backend.rs:11735-11839
 * layout), in the level / slot / parent-row order described in
 * tessa_partition.c.  Overflow bits land in counters[ORC_P_OVERFLOW_FLAGS]
 * and stop the walk after the level that raised them.  Returns 0, or a
 * negative value on bad arguments (-2), bad root leaders (-3), or when out
 * of host memory (-4). */
int orc_subtree_partition(const int8_t *codes, const float *scales, const float *norms,
                          size_t resident_rows, size_t padded_dim, const orc_subtree_cfg *cfg,
                          uint32_t *leaf_row_ids, uint64_t *leaf_starts, uint64_t *leaf_sizes,
                          uint64_t *counters, uint64_t *leaf_count, uint64_t *leaf_rows);

/* ---- candidate records -> HashPrune edges ------------------------------ */

/* spill_hashprune.rs:137-145 SpillRecord16, the 16-byte form of PendingEdge
 * (leaf_build.rs:59-65; flags = HashPruneMeta spill flags). */
typedef struct orc_edge_record {
    uint32_t src;
    uint32_t dst;
    uint16_t hash;
    uint16_t flags;
    float dist;
} orc_edge_record;

/* hash_prune.rs:2239-2251 compute_hash: bit i = (sketch_c[i] - sketch_p[i] >= 0). */
uint16_t orc_compute_hash(const float *sketch_p, const float *sketch_c, unsigned m_bits);

/* leaf_build.rs:1679-1829 flush_compact_topk_batch_into_edges for one
 * CompactTopKBatch (leaf_build.rs:271-282), evidence annotation and compact
 * lune pruning off (their defaults).  Sketch rows are indexed by global point
 * id (LeafSketchCache::prefetch over batch.point_ids).  Appends 2 records per
 * valid slot to out[0..capacity).  Returns the number written, or
 *   -1  a top-k id is not a member of the batch (*bad_point = that id),
 *   -2  m_bits > 16 or > width, or capacity too small,
 *   -3  a point id has no sketch row (*bad_point = that id). */
long long orc_flush_compact_topk_into_edges(const uint32_t *point_ids, size_t rows, size_t k,
                                            const uint32_t *topk_ids, const float *topk_dists,
                                            const float *sketches, size_t sketch_rows, size_t width,
                                            unsigned m_bits, orc_edge_record *out, size_t capacity,
                                            uint32_t *bad_point);

/* HashPrune reservoirs of num_points points (l_max slots each) after inserting
 * `records` in order (spill_hashprune.rs:2686-2719 with hash_prune.rs:1333-1453
 * insert_inner, backfill and evidence off).  Per point: out_counts[p] slots, then
 * out_targets/out_hashes/out_dists[p*l_max + s] in slot order (ascending hash),
 * unused slots 0xFFFFFFFF / 0 / 0.  out_hashes and out_dists may be NULL.
 * Returns 0, or -3 with *bad_record set when a record's src >= num_points. */
int orc_hashprune_reduce(size_t num_points, size_t l_max, const orc_edge_record *records, size_t count,
                         uint32_t *out_targets, uint16_t *out_hashes, float *out_dists, uint32_t *out_counts,
                         uint32_t *bad_record);

/* HashPrune with a named R-half backfill policy (hash_prune_backfill.rs,
 * hash_prune.rs:2601-2682): the ordinary reservoirs of `records` (as
 * orc_hashprune_reduce), then for each point with some but fewer than l_max
 * primaries a shortlist of its primary hashes' other candidates (quota per
 * hash, hit layers by rank) in the mode's priority order, cut to
 * min(row_cap, floor(l_max / 2), l_max - primaries), appended after the
 * primaries.  mode: ORC_RHALF_*; hash_quota 0 = the mode's (1 or 3);
 * row_cap 0 = none; priority_alpha <= 0 = 1.1 (SoftTier only).
 * out_counts = primaries + shortlist, out_primary_counts = primaries.
 * Returns 0, -1 on bad arguments, -2 on allocation failure, -3 as
 * orc_hashprune_reduce. */
#define ORC_RHALF_HASH_SLOT_1 1
#define ORC_RHALF_DISTANCE_FIRST_Q3 2
#define ORC_RHALF_SOFT_TIER_Q3 3
#define ORC_RHALF_HARD_TIER_Q3 4
int orc_hashprune_rhalf_reduce(size_t num_points, size_t l_max, const orc_edge_record *records, size_t count,
                               int mode, unsigned hash_quota, unsigned row_cap, float priority_alpha,
                               uint32_t *out_targets, uint16_t *out_hashes, float *out_dists, uint32_t *out_counts,
                               uint32_t *out_primary_counts, uint32_t *bad_record);

/* Greedy search of a [num_points x row_stride] neighbour table (row p =
 * targets[p*row_stride .. + counts[p]]) over f32 vectors, search list L,
 * from `start` (algorithm/search/search.rs:137-233 with the capacity-L
 * neighbour queue, model/neighbor/neighbor_priority_queue.rs:50-85): per
 * query the first K entries (ids, squared L2), 0xFFFFFFFF past the list, and
 * the number of distance evaluations.  Returns 0, -1 on bad arguments. */
int orc_greedy_search(const float *data, size_t num_points, size_t dim, const uint32_t *targets,
                      const uint32_t *counts, size_t row_stride, uint32_t start, const float *queries,
                      size_t num_queries, size_t L, size_t K, uint32_t *out_ids, float *out_dists,
                      uint32_t *out_cmps);

/* Global D0 assignment (GPU path, compute_backend.rs:18016-18511; distance
 * dco_sq_int8.rs:2950-2965): each row's fanout_top (<= 32) nearest leaders
 * by (dist, leader id) as row-major fragments (out_child = leader index,
 * out_point = global id) and, when child_offsets is given, the fragments
 * grouped by child (child_offsets [leader_count + 1], child_points [rows *
 * fanout], rows ascending within a child).  Returns 0, -1 on bad fanout. */
int orc_d0_assign(const int8_t *codes, const float *scales, const float *norms, const uint32_t *global_ids,
                  size_t rows, size_t padded_dim, const int8_t *leader_codes, const float *leader_scales,
                  const float *leader_norms, const uint32_t *leader_ids, size_t leader_count, size_t fanout,
                  uint32_t *out_child, uint32_t *out_point, uint64_t *child_offsets, uint32_t *child_points);

/* Final RobustPrune of every row of a [num_points x row_stride] neighbour
 * table (index/inmem_index/pipnn_builder.rs:287-330, algorithm/prune/
 * prune.rs:17-214): out_targets [num_points x max_degree] (0xFFFFFFFF past
 * out_counts).  Returns 0, -1 on bad arguments. */
int orc_robust_prune(const float *data, size_t num_points, size_t dim, const uint32_t *targets,
                     const uint32_t *counts, size_t row_stride, size_t max_degree, size_t max_occlusion,
                     float alpha, int saturate, uint32_t *out_targets, uint32_t *out_counts);

#ifdef __cplusplus
}
#endif
#endif
