/*
 * tessa_hip.h -- C ABI of the MI355X (gfx950) TESSA construction operator.
 *
 * This is the drop-in boundary for SHEAR's CUDA operator path.  It is plain C:
 * integers, floats and pointers; device pointers are `void*`/typed pointers
 * into HIP device memory and `stream` is a hipStream_t passed as `void*`.
 * Nothing here panics or throws across the boundary: every entry point returns
 * a tessa_status whose `code` is 0 on success.
 *
 * Reference interfaces each entry point replaces (paths relative to
 * shear-core/src/algorithm/pipnn/ in SHEAR):
 *   tessa_query_caps             compute_backend.rs:3696-3702 validate_gpu_subtree_hardware
 *                                / gpu_hardware_adaptation_profile
 *   tessa_session_create/destroy compute_backend.rs:34648 TessaCudaReplaySession::new,
 *                                :31510 CudaComputeBackend::new
 *   tessa_session_upload_sq8     compute_backend.rs:26844 upload_quantized_resident_subtree
 *                                (H2D of GpuSubtreeQuantizedInput :1871-1883)
 *   tessa_leaf_topk              compute_backend.rs:16146-16334 gpu_persistent_subtree_topk_only
 *                                (launched by TessaCudaReplaySession::run_mode :34841,
 *                                layouts tessa_replay.rs:1021-1057)
 *   tessa_assign_replay          compute_backend.rs:15729-15943 gpu_tessa_assignment_replay
 *   tessa_sq8_quantize           dco_sq_int8.rs:1331-1467 quantize_sq_int8_matrix (its GPU
 *                                twin compute_backend.rs:17955-18014 tree-reduces the norm;
 *                                this one keeps the CPU's sequential sum, so bits match)
 *   tessa_session_leaf_topk /    TessaCudaReplaySession::run_mode leaf / assignment legs
 *   tessa_session_assign_replay  (tessa_replay.rs:190-200 TessaCudaModeResult)
 *   tessa_overflow_labels        compute_backend.rs:2249-2296 gpu_persistent_overflow_labels
 *   tessa_session_submit_subtree compute_backend.rs:3807-3815 submit_owned_quantized_subtree_l2_compact_topk
 *   / _wait / _release           (Deferred result, pinned slot ring :31432-31497)
 *   tessa_emit_edge_records      leaf_build.rs:1679-1829 flush_compact_topk_batch_into_edges
 *                                (records: spill_hashprune.rs:137-145 SpillRecord16)
 */
#ifndef TESSA_HIP_H
#define TESSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TESSA_ABI_VERSION 1u

/* ---- status ----------------------------------------------------------- */
enum tessa_code {
    TESSA_OK = 0,
    TESSA_ERR_INVALID_ARGUMENT = 1,
    TESSA_ERR_HIP = 2,              /* a HIP runtime call failed */
    TESSA_ERR_OVERFLOW = 3,         /* device set overflow_flags (see bits) */
    TESSA_ERR_UNSUPPORTED = 4,      /* shape outside the kernels' limits */
    TESSA_ERR_OUT_OF_MEMORY = 5,
    TESSA_ERR_NO_DEVICE = 6
};

typedef struct tessa_status {
    int32_t code;
    uint32_t reserved;
    uint64_t overflow_flags;  /* same bit meanings as the reference word */
    char msg[512];            /* "overflow_flags=0x.. overflow_labels=..." tokens kept */
} tessa_status;

/* Overflow bits: identical to compute_backend.rs:4843-4860 / host :252-272. */
#define TESSA_OVF_QUEUE_NODE               (1ull << 0)
#define TESSA_OVF_QUEUE_ROW                (1ull << 1)
#define TESSA_OVF_LEAF_DESC                (1ull << 2)
#define TESSA_OVF_LEAF_ROW                 (1ull << 3)
#define TESSA_OVF_LEADER                   (1ull << 4)
#define TESSA_OVF_FANOUT_OVER_32           (1ull << 5)
#define TESSA_OVF_NO_PROGRESS_SPLIT        (1ull << 7)
#define TESSA_OVF_WORKSPACE_BUDGET         (1ull << 8)
#define TESSA_OVF_OVERSIZED_TERMINAL_NODE  (1ull << 10)
#define TESSA_OVF_WATCHDOG_STALLED         (1ull << 11)
#define TESSA_OVF_ACTIVE_WORK_BUDGET       (1ull << 12)
#define TESSA_OVF_INVALID_TOPK_ROW_ID      (1ull << 13)
#define TESSA_OVF_INVALID_TOPK_COL_ID      (1ull << 14)
#define TESSA_OVF_INVALID_ASSIGN_POINT_ID  (1ull << 15)
#define TESSA_OVF_INVALID_ASSIGN_LEADER_ID (1ull << 16)
#define TESSA_OVF_UNSUPPORTED_EXPLICIT_KERNEL (1ull << 18)

/* ---- counters (u64 words, device-resident, accumulated by kernels) ----- */
#define TESSA_COUNTER_WORDS 32
enum tessa_counter {
    TESSA_C_OVERFLOW_FLAGS = 0,
    TESSA_C_LEAF_ROWS = 1,             /* rows whose top-k was written */
    TESSA_C_LEAF_MFMA_TILES = 2,       /* 32x32 candidate tiles on the MFMA path */
    TESSA_C_LEAF_EXACT_ROWS = 3,       /* rows evaluated by the exact scalar kernel */
    TESSA_C_LEAF_FALLBACK_ROWS = 4,    /* MFMA rows re-run exactly (list overflow / gap) */
    TESSA_C_LEAF_LIST_OVERFLOW_ROWS = 5,
    TESSA_C_LEAF_GAP_FALLBACK_ROWS = 6,
    TESSA_C_LEAF_REFINES = 7,          /* threshold refinements (wave-level) */
    TESSA_C_LEAF_SURVIVORS = 8,        /* candidates that passed the running threshold */
    TESSA_C_LEAF_FINAL_CANDIDATES = 9, /* entries fed to the final ordered insertion */
    TESSA_C_ASSIGN_ROWS = 10,
    TESSA_C_ASSIGN_PAIRS = 11,
    TESSA_C_ASSIGN_TIE_EVENTS = 12,    /* insertions decided by the eps tie key */
    TESSA_C_LEAF_CHAIN_ROWS = 13       /* MFMA rows whose eps-tie chains were replayed
                                          in column order over their candidate set */
};

/* ---- executors (mirrors tessa_replay.rs:20-86 leaf_executor_code) ------ */
#define TESSA_EXEC_EXACT 1u  /* scalar integer-dot kernel, reference "DP4A" role */
#define TESSA_EXEC_MFMA  2u  /* int8 MFMA 32x32x32 kernel, reference "WMMA" role */

/* ---- device capabilities ---------------------------------------------- */
typedef struct tessa_caps {
    int32_t device;
    int32_t compute_units;
    int32_t max_threads_per_block;
    int32_t lds_bytes_per_block;
    uint64_t hbm_bytes;
    char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t supported;      /* 1 when the arch is gfx950 */
    int32_t max_leaf_rows;  /* MFMA leaf path limit */
    int32_t max_k;          /* 32 */
    int32_t max_padded_dim; /* 1024 */
} tessa_caps;

tessa_status tessa_query_caps(int32_t device, tessa_caps *out);

/* ---- SQ8 input (GpuSubtreeQuantizedInput, compute_backend.rs:1871-1883) --
 * codes: rows x code_row_bytes int8 (DenseI8 layout, code_row_bytes ==
 * padded_dim, padded_dim % 16 == 0); scales/norms: f32 per row; global_ids:
 * u32 per row (ids written into candidate records). */
typedef struct tessa_sq8_view {
    const int8_t *codes;
    const float *scales;
    const float *norms;
    const uint32_t *global_ids;
    uint64_t rows;
    uint32_t dim;
    uint32_t padded_dim;
} tessa_sq8_view;

/* ---- leaf layouts (TessaLeafLayout, tessa_replay.rs:1041-1047) ---------
 * members: local row ids (index into the SQ8 arrays), concatenated per leaf;
 * member_offsets[l] / member_counts[l] / output_offsets[l]; output slot of
 * (leaf l, member row r, rank q) is output_offsets[l] + r*k + q. */
typedef struct tessa_leaf_batch {
    const uint32_t *members;
    const uint64_t *member_offsets;
    const uint32_t *member_counts;
    const uint64_t *output_offsets;
    uint32_t leaf_count;
    uint32_t max_leaf_rows;   /* upper bound of member_counts (checked on device) */
    uint32_t k;               /* 1..32; per leaf k_eff = min(k, n-1) */
    uint32_t executor;        /* TESSA_EXEC_MFMA or TESSA_EXEC_EXACT */
    uint32_t debug_rerun_every; /* 0 = off; else rows whose leaf position is a
                                   multiple of it take the exact re-run path
                                   (test knob for the MFMA executor) */
    uint32_t reserved;
} tessa_leaf_batch;

/* Leaf all-pairs SQ8 evaluation + per-row top-k (candidate records).
 * All pointers are device pointers; work is enqueued on `stream` (hipStream_t,
 * NULL = default stream).  out_ids/out_dists receive (global id, f32 distance)
 * per slot: bit-identical to the reference RowTopK order (eps 2e-5, ties by
 * global id, columns in member order); unused slots are (0xffffffff, FLT_MAX).
 * counters: TESSA_COUNTER_WORDS u64 (accumulated; caller zeroes), may be NULL.
 * The call allocates its workspace on first use (grows, kept per device). */
tessa_status tessa_leaf_topk(const tessa_sq8_view *sq8, const tessa_leaf_batch *leaves,
                             uint32_t *out_ids, float *out_dists,
                             uint64_t *counters, void *stream);

/* tessa_leaf_topk that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and errors as tessa_leaf_topk; all scratch (queue
 * counters, re-run and chain queues, survivor logs, work-item list) lives
 * in one static device array of about 39 MB per GPU, held until the process ends, so a
 * call of the MFMA executor may cover at most 65,536 member rows
 * (leaf_count * max_leaf_rows); larger batches are rejected with
 * TESSA_ERR_UNSUPPORTED.  The exact executor uses no scratch and takes any
 * batch.  Once a first call on a device has returned, calls may be captured
 * into a HIP graph (the first call looks up the array's address and sets
 * the kernels' LDS limits; later calls only launch kernels).  Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller. */
tessa_status tessa_leaf_topk_noalloc(const tessa_sq8_view *sq8, const tessa_leaf_batch *leaves,
                                     uint32_t *out_ids, float *out_dists,
                                     uint64_t *counters, void *stream);

/* tessa_leaf_topk with hipEvents around its kernels (the reference reports
 * the same split as persistent_kernel_event_ms / leaf DCO clocks in
 * GpuSubtreeTopKProfile, compute_backend.rs:2198-2247).  Synchronises on the
 * last event; phase_ms[0..3] = MFMA filter kernel and select kernel (summed
 * over the call's batches of work items), chain replay, exact re-run;
 * phase_ms[4] = the number of batches (launches of each of the first two). */
tessa_status tessa_leaf_topk_profiled(const tessa_sq8_view *sq8, const tessa_leaf_batch *leaves,
                                      uint32_t *out_ids, float *out_dists,
                                      uint64_t *counters, void *stream, float *phase_ms);

/* ---- assignment tasks (TessaAssignmentLayout, tessa_replay.rs:1031-1039) -
 * For member row m of task t, leaders of the task are visited in slot order;
 * best r_h[t] <= 4 ranks are written at output_offsets[t] + m*r_h[t] + rank as
 * (leader global id, f32 SQ8 distance). */
typedef struct tessa_assign_batch {
    const uint32_t *members;
    const uint32_t *leaders;
    const uint32_t *member_offsets;
    const uint32_t *member_counts;
    const uint32_t *leader_offsets;
    const uint32_t *leader_counts;   /* each <= 128 */
    const uint32_t *r_h;             /* each 1..4, <= leader count */
    const uint64_t *output_offsets;
    uint32_t task_count;
    uint32_t max_members;            /* upper bound of member_counts */
} tessa_assign_batch;

tessa_status tessa_assign_replay(const tessa_sq8_view *sq8, const tessa_assign_batch *tasks,
                                 uint32_t *out_ids, float *out_dists,
                                 uint64_t *counters, void *stream);

/* SQ8 quantizer on device: x is rows x dim f32 (device); codes rows x
 * padded_dim int8, scales/norms f32.  Bit-identical to the reference CPU
 * quantizer (sequential f32 norm, round half away from zero).  *bad_row_out
 * (device u64, may be NULL) receives the first row holding a non-finite value
 * or UINT64_MAX; such rows are left zero. */
tessa_status tessa_sq8_quantize(const float *x, uint64_t rows, uint32_t dim,
                                uint32_t padded_dim, uint32_t bits, int8_t *codes,
                                float *scales, float *norms, uint64_t *bad_row_out,
                                void *stream);

/* ---- sessions (TessaCudaReplaySession / CudaComputeBackend role) --------
 * A session owns one device, one stream and device copies of an SQ8 resident
 * set.  Sessions are single-threaded: callers serialise, as the reference's
 * Mutex<CudaGemmEngine> does. */
typedef struct tessa_session tessa_session;

typedef struct tessa_config {
    int32_t device;
    uint32_t reserved;
} tessa_config;

tessa_status tessa_session_create(const tessa_config *cfg, tessa_session **out);
tessa_status tessa_session_destroy(tessa_session *session);
/* Copy of an SQ8 resident set into session-owned device buffers; the view's
 * arrays may be host or device memory (the copy direction follows the
 * pointers). */
tessa_status tessa_session_upload_sq8(tessa_session *session, const tessa_sq8_view *host);

/* Host-layout leaf replay: host arrays in, host arrays out; event_ms gets the
 * kernel time measured with hipEvents on the session stream. */
tessa_status tessa_session_leaf_topk(tessa_session *session,
                                     const uint32_t *members, const uint64_t *member_offsets,
                                     const uint32_t *member_counts,
                                     const uint64_t *output_offsets, uint32_t leaf_count,
                                     uint32_t k, uint32_t executor, uint32_t *out_ids,
                                     float *out_dists, uint64_t *counters, float *event_ms);

tessa_status tessa_session_assign_replay(tessa_session *session, const uint32_t *members,
                                         const uint32_t *leaders,
                                         const uint32_t *member_offsets,
                                         const uint32_t *member_counts,
                                         const uint32_t *leader_offsets,
                                         const uint32_t *leader_counts, const uint32_t *r_h,
                                         const uint64_t *output_offsets, uint32_t task_count,
                                         uint32_t *out_ids, float *out_dists,
                                         uint64_t *counters, float *event_ms);

/* ---- resident subtree: recursive partition + leaf top-k -----------------
 * Replaces PiPNNComputeBackend::process_quantized_subtree_l2_compact_topk
 * (compute_backend.rs:3794-3805; request GpuSubtreePartitionRequest
 * :1818-1826, result GpuSubtreeTopKResult :1945-1951) as executed by
 * gpu_persistent_subtree_topk (:16336-17380) after plan_gpu_persistent_subtree
 * (:1309-1488).  The session's uploaded SQ8 rows are the resident subtree
 * (local row r = upload row r, global id = global_ids[r]). */

/* Counter words of a subtree run, at the reference's indices
 * (compute_backend.rs:5028-5187).  Words with no counterpart in this
 * implementation (queue heads, polls, locks, most clocks) stay 0.  The phase
 * clocks of the persistent partition walk are in ticks of the device's
 * 100 MHz wall clock, measured by workgroup 0 between grid barriers (the
 * reference counts SM clock cycles): BUSY the whole walk, WAIT workgroup 0's
 * barrier waits, COUNT_DISTANCE the COUNT passes, COUNT_COMMIT the stage,
 * item plan and EMIT passes, SCATTER the scatter, PUBLISH the child layout
 * and numbering scans
 * (all 0 when the partition runs level by level for a capture). */
#define TESSA_SUBTREE_COUNTER_WORDS 159
enum tessa_subtree_counter {
    TESSA_P_OVERFLOW_FLAGS = 7,
    TESSA_P_PARTITION_POPS = 8,
    TESSA_P_OUTPUT_ROWS = 12,
    TESSA_P_OUTPUT_LEAF_COUNT = 13,
    TESSA_P_ASSIGNMENT_PASSES = 14,
    TESSA_P_MAX_ACTIVE = 15,
    TESSA_P_EFFECTIVE_ROOT_FANOUT = 17,
    TESSA_P_EFFECTIVE_DEEPER_FANOUT = 18,
    TESSA_P_FANOUT_ASSIGNMENT_SLOTS = 19,
    TESSA_P_REPLICATED_ROWS = 20,
    TESSA_P_UNIQUE_RESIDENT_ROWS = 21,
    TESSA_P_LARGE_NODE_CLAIMS = 27,
    TESSA_P_LARGE_NODE_SPLITS = 28,
    TESSA_P_LARGE_NODE_ROWS = 29,
    TESSA_P_LARGE_NODE_MAX_ROWS = 30,
    TESSA_P_LEAF_SIZE_MIN = 33,
    TESSA_P_LEAF_SIZE_MAX = 34,
    TESSA_P_LEAF_SIZE_SUM = 35,
    TESSA_P_LEAF_SIZE_COUNT = 36,
    TESSA_P_PARTITION_LEVEL_ROUNDS = 119,
    TESSA_P_PARTITION_BUSY_CLOCKS = 120,
    TESSA_P_PARTITION_WAIT_CLOCKS = 121,
    TESSA_P_LARGE_SPLIT_RETRIES = 130,
    TESSA_P_LARGE_BALANCED_FALLBACKS = 131,
    TESSA_P_LARGE_COUNT_DISTANCE_CLOCKS = 140,
    TESSA_P_LARGE_COUNT_COMMIT_CLOCKS = 141,
    TESSA_P_LARGE_SCATTER_CLOCKS = 142,
    TESSA_P_LARGE_PUBLISH_CLOCKS = 143,
    TESSA_P_LARGE_PHYSICAL_TILES = 145,
    TESSA_P_LEAF_SQ8_WMMA_TILES = 158
};

/* plan_gpu_persistent_subtree (compute_backend.rs:1309-1488): capacities and
 * admission.  required_bytes is this implementation's device workspace plus
 * outputs; the fallback reasons keep the reference's bits. */
/* GPU_PERSISTENT_FALLBACK_REASON_* (compute_backend.rs:375-383) */
#define TESSA_PLAN_FALLBACK_UNSUPPORTED_K       (1u << 2)
#define TESSA_PLAN_FALLBACK_UNSUPPORTED_FANOUT  (1u << 3)
#define TESSA_PLAN_FALLBACK_UNSUPPORTED_LEADERS (1u << 4)
#define TESSA_PLAN_FALLBACK_WORKSPACE           (1u << 5)
typedef struct tessa_subtree_plan {
    int32_t supported;
    uint32_t fallback_reason_flags;
    uint64_t overflow_flags;
    uint32_t leaf_min;            /* 64 (GPU_PERSISTENT_LEAF_MIN) */
    uint32_t leaf_target;         /* 128 */
    uint32_t leaf_max;            /* max(256, c_max) */
    uint32_t small_node_limit;    /* 4096 */
    uint32_t effective_root_fanout;
    uint32_t effective_deeper_fanout;
    uint32_t fanout_amplification;
    uint32_t large_child_slots;   /* 128 */
    uint64_t max_queue_nodes;
    uint64_t max_leaf_count;      /* capacity of leaf_starts / leaf_sizes */
    uint64_t max_leaf_rows;       /* capacity of leaf_row_ids; top-k rows */
    uint64_t large_scratch_rows;
    uint64_t required_bytes;
    uint64_t budget_bytes;
} tessa_subtree_plan;

tessa_status tessa_plan_subtree(uint64_t resident_rows, uint32_t leaf_knn,
                                uint32_t max_leaders_per_node, uint32_t max_fanout,
                                uint64_t budget_bytes /* 0 = unlimited */, uint32_t c_max,
                                tessa_subtree_plan *plan);

/* ---- GPU-memory-aware task formation -----------------------------------------
 * plan_gpu_persistent_subtree_resident_admission (compute_backend.rs:
 * 1490-1522): the plan above plus the resident rows' bytes
 * (estimate_gpu_resident_subtree_device_bytes[_for_params] :898-930: f32 rows
 * + id + norm, the reference default; or SQ8 codes padded to 16 bytes, or
 * packed int4, + id + scale + norm); a task whose resident + workspace bytes
 * exceed device_budget_bytes (0 = none) is unsupported with the workspace
 * fallback and overflow bits.  Budgets of 0 mean "none". */
#define TESSA_RESIDENT_F32 0u
#define TESSA_RESIDENT_SQ8 1u
#define TESSA_RESIDENT_SQ4 2u
typedef struct tessa_resident_admission {
    tessa_subtree_plan plan;
    uint64_t resident_device_bytes;
    uint64_t device_admission_required_bytes;
    uint64_t device_admission_budget_bytes;  /* UINT64_MAX without a budget */
} tessa_resident_admission;
tessa_status tessa_plan_subtree_resident_admission(uint64_t resident_rows, uint32_t dim, uint32_t leaf_knn,
                                                   uint32_t max_leaders_per_node, uint32_t max_fanout,
                                                   uint64_t workspace_budget_bytes, uint64_t device_budget_bytes,
                                                   uint32_t c_max, uint32_t resident_format,
                                                   tessa_resident_admission *out);
/* find_max_admissible_rows (d0_capacity.rs:55-102): the largest resident row
 * count (< 2^31 by doubling, then bisection) the admission supports; 0 when
 * dim is 0 or one row does not fit. */
uint64_t tessa_find_max_admissible_rows(uint32_t dim, uint32_t leaf_knn, uint32_t max_leaders_per_node,
                                        uint32_t max_fanout, uint64_t workspace_budget_bytes,
                                        uint64_t device_budget_bytes, uint32_t c_max, uint32_t resident_format);
/* D0 capacity (d0_capacity.rs:201-299): thresholds from the admitted row
 * count (ratios clamped high in [0.01, 1], target in [0.01, high], low in
 * [0, target]; c_low lifted to min_efficient_rows, capped at c_target);
 * root leader plan (k_capacity = ceil(points * fanout / c_target), the
 * quality floor and the leader cap); split leader count of an oversized
 * child; nearest-rank child size summary. */
typedef struct tessa_d0_thresholds {
    uint64_t c_gpu, c_high, c_target, c_low;
} tessa_d0_thresholds;
#define TESSA_D0_LEADERS_CAPACITY      0u  /* "capacity" */
#define TESSA_D0_LEADERS_QUALITY_FLOOR 1u  /* "quality_floor" */
#define TESSA_D0_LEADERS_ROOT_CAP      2u  /* "root_leader_cap" */
typedef struct tessa_d0_leader_plan {
    uint64_t k_capacity, k_initial, root_leader_cap;
    uint32_t source;
} tessa_d0_leader_plan;
typedef struct tessa_d0_child_summary {
    uint64_t max_rows, p50_rows, p95_rows, p99_rows;
    uint64_t oversized_count, small_count, small_rows;
} tessa_d0_child_summary;
tessa_d0_thresholds tessa_d0_compute_thresholds(uint64_t c_gpu, double high_ratio, double target_ratio,
                                                double low_ratio, uint64_t min_efficient_rows);
tessa_d0_leader_plan tessa_d0_plan_root_leaders(uint64_t total_points, uint64_t root_fanout,
                                                const tessa_d0_thresholds *t, uint64_t quality_min_root_leaders,
                                                uint64_t root_leader_cap);
uint64_t tessa_d0_split_leader_count(uint64_t rows, const tessa_d0_thresholds *t);
tessa_d0_child_summary tessa_d0_observe_child_sizes(const uint64_t *sizes, uint64_t count,
                                                    const tessa_d0_thresholds *t);

/* gpu_queue_root_seed (compute_backend.rs:1597-1603). */
uint64_t tessa_subtree_root_seed(uint64_t random_seed, uint64_t depth, uint64_t point_count,
                                 uint64_t parent_points, uint64_t min_recurse_size);

typedef struct tessa_subtree_request {
    const uint32_t *root_leaders;  /* host array of resident row ids, or NULL */
    uint32_t root_leader_count;    /* <= min(max_leaders, 128) */
    uint32_t root_depth;           /* request.depth */
    uint64_t seed;                 /* tessa_subtree_root_seed(...) */
    uint32_t leaf_knn;             /* 1..32 (k = min(leaf_knn, rows-1)) */
    uint32_t fanout_second;        /* 1..4, root-level replication */
    uint32_t max_depth;
    uint32_t max_leaders;          /* params.max_leaders */
    uint32_t leaf_min;             /* plan.leaf_min */
    uint32_t leaf_max;             /* plan.leaf_max (<= 4096 for the top-k) */
    uint32_t small_node_limit;     /* plan.small_node_limit */
    float psamp_fraction;          /* params.psamp_fraction as f32 */
    uint32_t executor;             /* TESSA_EXEC_MFMA or TESSA_EXEC_EXACT */
    uint32_t partition_only;       /* 1: leaves only, no top-k */
    uint64_t max_leaf_count;       /* output capacities (plan values) */
    uint64_t max_leaf_rows;
} tessa_subtree_request;

/* Device output buffers (caller-owned, sized from the plan) and results.
 * Leaf l holds leaf_row_ids[leaf_starts[l] .. + leaf_sizes[l]] (resident row
 * ids); the top-k of its member row r is at (leaf_starts[l] + r) * k + rank,
 * k = min(leaf_knn, rows - 1), unused slots (0xffffffff, FLT_MAX).  Leaves
 * are numbered level by level, each node's children in leader-slot order,
 * and the rows of every leaf are ascending (one legal order of the
 * reference's concurrent walk, which has none fixed). */
typedef struct tessa_subtree_output {
    uint32_t *leaf_row_ids;        /* device, max_leaf_rows */
    uint64_t *leaf_starts;         /* device, max_leaf_count */
    uint64_t *leaf_sizes;          /* device, max_leaf_count */
    uint32_t *topk_ids;            /* device, max_leaf_rows * k (unused if partition_only) */
    float *topk_dists;
    uint64_t *counters;            /* host, TESSA_SUBTREE_COUNTER_WORDS, may be NULL */
    uint64_t *leaf_counters;       /* host, TESSA_COUNTER_WORDS, may be NULL */
    uint64_t leaf_count;           /* out */
    uint64_t leaf_rows;            /* out */
    uint32_t k;                    /* out: top-k row stride */
    uint32_t levels;               /* out: partition levels walked */
    float partition_ms;            /* out: hipEvent time of the partition */
    float leaf_ms;                 /* out: hipEvent time of the leaf top-k */
} tessa_subtree_output;

tessa_status tessa_session_run_subtree(tessa_session *session, const tessa_subtree_request *req,
                                       tessa_subtree_output *out);

/* ---- many subtree roots in one partition run ------------------------------
 * Replaces the build's loop over D1+ children, one
 * process_quantized_subtree_l2_compact_topk call each (the loop
 * rbc_partition.rs:10261-10352 run_gpu_subtree_d1plus_producer_with_context,
 * the call at :15076-15087): every root's rows are partitioned
 * in one level-synchronous run, all roots' nodes of a level together, with no
 * upload of the roots' SQ8 rows (they are read in place from `sq8`, device
 * arrays, through `rows`).  Root i owns rows[root_offsets[i] ..
 * root_offsets[i+1]) (SQ8 row ids, ascending within a root) and starts from
 * root_seeds[i] at depth root_depth; its leaves are exactly those a
 * tessa_session_run_subtree call over that root's rows alone (uploaded in
 * that order, same seed and parameters) would publish, with member rows given
 * as SQ8 row ids.  Leaves of different roots interleave in the output.  Every
 * root must be a large node: at least 2 rows and more than leaf_max rows or
 * more than small_node_limit / fanout_second (smaller roots go through
 * tessa_session_run_subtree).  Leaf outputs (device): leaf_rows
 * [max_leaf_rows] SQ8 row ids, leaf_starts [max_leaf_count], leaf_sizes
 * [max_leaf_count] (u32, ready as a tessa_leaf_batch's member_counts).
 * Overflow is reported as by tessa_session_run_subtree; no leaf top-k runs. */
typedef struct tessa_roots_request {
    const uint32_t *rows;          /* device: the roots' SQ8 row ids, concatenated */
    const uint64_t *root_offsets;  /* host: root_count + 1 */
    const uint64_t *root_seeds;    /* host: root_count */
    uint32_t root_count;
    uint32_t root_depth;
    uint32_t fanout_second;
    uint32_t max_depth;
    uint32_t max_leaders;
    uint32_t leaf_min;
    uint32_t leaf_max;
    uint32_t small_node_limit;
    float psamp_fraction;
    uint32_t reserved;
    uint64_t max_leaf_count;
    uint64_t max_leaf_rows;
} tessa_roots_request;

typedef struct tessa_roots_output {
    uint32_t *leaf_rows;           /* device, max_leaf_rows: SQ8 row ids */
    uint64_t *leaf_starts;         /* device, max_leaf_count */
    uint32_t *leaf_sizes;          /* device, max_leaf_count */
    uint32_t *leaf_roots;          /* device, max_leaf_count, may be NULL: each leaf's root index */
    uint32_t *leaf_depths;         /* device, max_leaf_count, may be NULL: each leaf's depth (a
                                      root's leaves are one level below the deepest node split;
                                      a run with max_depth M fails for a root iff one of its
                                      leaves is deeper than M) */
    uint64_t *counters;            /* host, TESSA_SUBTREE_COUNTER_WORDS, may be NULL */
    uint64_t leaf_count;           /* out */
    uint64_t leaf_rows_total;      /* out */
    uint32_t levels;               /* out */
    float partition_ms;            /* out */
} tessa_roots_output;

tessa_status tessa_session_partition_roots(tessa_session *session, const tessa_sq8_view *sq8,
                                           const tessa_roots_request *req, tessa_roots_output *out);

/* ---- candidate records -> HashPrune edge records ------------------------
 * Replaces the host conversion flush_compact_topk_batch_into_edges
 * (leaf_build.rs:1679-1829) that SHEAR runs on every CompactTopKBatch the
 * subtree operator returns (compute_backend.rs:32243-32339 builds one per
 * leaf: leaf_id = leaf index, point_ids = global ids of the leaf's rows,
 * k = min(leaf_knn, rows - 1)).  Each slot (j, d) of member row i with
 * j != 0xffffffff and finite d yields two records, in the reference's order
 * (leaf, row, rank; forward then reverse):
 *   {src i, dst j, hash compute_hash(s_i, s_j), flags 0, d}
 *   {src j, dst i, hash compute_hash(s_j, s_i), flags 0, d}
 * compute_hash (hash_prune.rs:2239-2251): bit b = (s_c[b] - s_p[b] >= 0),
 * b < m_bits.  Records use the SpillRecord16 layout
 * (spill_hashprune.rs:137-145).  flags is 0: HashPrune evidence annotation and
 * compact lune pruning (reference options, off by default) are not offered. */
typedef struct tessa_edge_record {
    uint32_t src;    /* PendingEdge.p */
    uint32_t dst;    /* PendingEdge.c */
    uint16_t hash;
    uint16_t flags;  /* HashPruneMeta spill flags */
    float dist;
} tessa_edge_record;

/* SketchAccessor rows (hash_prune.rs:21-36, SketchStore :60-72) on device:
 * sketch_rows x width f32, row = global point id; m_bits = params.m_hash_bits
 * (1..16, <= width). */
typedef struct tessa_sketch_view {
    const float *rows;
    uint64_t sketch_rows;
    uint32_t width;
    uint32_t m_bits;
} tessa_sketch_view;

/* Device arrays in, device records out; leaves/topk as written by
 * tessa_leaf_topk (output slot of (leaf l, row r, rank q) =
 * output_offsets[l] + r*k + q; per leaf k = min(k, n-1); max_leaf_rows <=
 * 4096), global_ids[resident_rows] maps member rows to point ids.  out holds
 * out_capacity records; leaf_record_offsets (device, leaf_count + 1, may be
 * NULL) receives each leaf's first record index and, last, the total.
 * Synchronises `stream`; *record_count = records written.  Errors: a top-k id
 * outside its leaf ("Compact top-k batch references point J outside leaf L",
 * leaf_build.rs:1796-1801), a point without a sketch row, out_capacity below
 * the record count (nothing written). */
tessa_status tessa_emit_edge_records(const uint32_t *global_ids, uint64_t resident_rows,
                                     const tessa_leaf_batch *leaves, const uint32_t *topk_ids,
                                     const float *topk_dists, const tessa_sketch_view *sketches,
                                     tessa_edge_record *out, uint64_t out_capacity,
                                     uint64_t *leaf_record_offsets, uint64_t *record_count,
                                     void *stream);

/* The same records in source-grouped order, for the GPU reservoirs: inside
 * each leaf the records of one source are adjacent (member row r's forward
 * records in rank order, then the reverse records naming it), and
 * segments[i] describes the run of the i-th member row of the batch (leaves
 * in order, rows in order): {src, first record (low and high words), record
 * count}.  The records are the reference's (the multiset per leaf is the one
 * tessa_emit_edge_records writes); only their order differs, and the order of
 * the reverse records inside a run is not fixed.  It has no counterpart in the
 * reference: it lets tessa_hashprune_insert_segments merge without grouping
 * records.  segment_capacity must cover every member row (rows of leaves
 * above max_leaf_rows excluded). */
typedef struct tessa_edge_segment {
    uint32_t src;
    uint32_t first_lo;
    uint32_t first_hi;
    uint32_t count;
} tessa_edge_segment;
tessa_status tessa_emit_edge_segments(const uint32_t *global_ids, uint64_t resident_rows,
                                      const tessa_leaf_batch *leaves, const uint32_t *topk_ids,
                                      const float *topk_dists, const tessa_sketch_view *sketches,
                                      tessa_edge_record *out, uint64_t out_capacity, tessa_edge_segment *segments,
                                      uint64_t segment_capacity, uint64_t *record_count, uint64_t *segment_count,
                                      void *stream);
/* tessa_emit_edge_segments without the repeats of mutual pairs: when leaf
 * row r names j and row j names r at the same distance, the reverse record
 * of r's slot, (j -> r, compute_hash(s_j, s_r), d), is bit for bit j's
 * forward record and is left out (and likewise for j's slot).  Per leaf the
 * records written are the reference's multiset less those repeats: every
 * distinct record is kept, so HashPrune reservoirs (whose state depends only
 * on the set of records inserted) end the same.  The leaves take their
 * places in `out` in completion order, without gaps; *record_count = the
 * records written (the sum of the segment counts).  out_capacity must still
 * cover 2 records per valid slot.  No counterpart in the reference (whose
 * reservoirs see both copies and ignore the second). */
tessa_status tessa_emit_edge_segments_unique(const uint32_t *global_ids, uint64_t resident_rows,
                                             const tessa_leaf_batch *leaves, const uint32_t *topk_ids,
                                             const float *topk_dists, const tessa_sketch_view *sketches,
                                             tessa_edge_record *out, uint64_t out_capacity,
                                             tessa_edge_segment *segments, uint64_t segment_capacity,
                                             uint64_t *record_count, uint64_t *segment_count, void *stream);

/* ---- HashPrune reservoirs: the consumer of the record stream ---------------
 * One HashPruneReservoir per point (hash_prune.rs:266-280, l_max slots, insert
 * :1243-1246 / insert_inner :1333-1453, total order :2094-2106), fed as
 * ExternalHashPruneReducer::reduce_spill_artifacts_ordered feeds it
 * (spill_hashprune.rs:875-892; per edge reservoir.insert :2686-2719; emitted
 * by copy_neighbors_and_clear :3203-3221), backfill and evidence policies off
 * (their defaults, params.rs:3346-3350).  The reservoirs live in device
 * memory; records are merged batch by batch, in any order (the reservoir's
 * final state depends only on the candidates inserted).
 *   create     reservoirs for points [0, num_points), l_max in [1, 256];
 *   insert     device records; synchronises `stream`; a record with
 *              src >= num_points fails the call (the reference's "edge p=...
 *              outside shard range") after the batch's valid records are in;
 *   neighbors  per point up to l_max slots in slot order (ascending hash):
 *              targets / hashes / dists [num_points * l_max] (unused slots
 *              0xFFFFFFFF / 0 / 0.0) and counts [num_points], device pointers,
 *              each may be NULL; enqueued on `stream`;
 *   clear      empties every reservoir (enqueued on `stream`). */
typedef struct tessa_hashprune tessa_hashprune;
tessa_status tessa_hashprune_create(uint32_t num_points, uint32_t l_max, tessa_hashprune **out);
tessa_status tessa_hashprune_destroy(tessa_hashprune *hp);
tessa_status tessa_hashprune_insert(tessa_hashprune *hp, const tessa_edge_record *records, uint64_t count,
                                    void *stream);
tessa_status tessa_hashprune_neighbors(const tessa_hashprune *hp, uint32_t *targets, uint16_t *hashes,
                                       float *dists, uint32_t *counts, void *stream);
tessa_status tessa_hashprune_clear(tessa_hashprune *hp, void *stream);
/* insert for records described by segments (tessa_emit_edge_segments): each
 * segment's records share its src; a source's segments are merged together,
 * reading the records in place (no grouping pass over the records).  Same
 * result as tessa_hashprune_insert of the same records; same errors. */
tessa_status tessa_hashprune_insert_segments(tessa_hashprune *hp, const tessa_edge_record *records,
                                             const tessa_edge_segment *segments, uint64_t segment_count,
                                             void *stream);

/* create with a named R-half backfill policy (PiPNNParams
 * hashprune_backfill_mode rhalf-hash-slot-1 / rhalf-distance-first-q3 /
 * rhalf-soft-tier-q3 / rhalf-hard-tier-q3 with hashprune_rhalf_hash_quota,
 * hashprune_rhalf_max_backfill_per_row and
 * hashprune_soft_tier_priority_alpha: shear-core/src/algorithm/pipnn/
 * params.rs:2070-2083, validated as :2696-2729; the build_shear_index
 * binary's default is SoftTier-Q3, alpha 1.02, 3 per row,
 * apps/build_shear_index/src/main.rs:2360-2374).  A row that ends with some
 * but fewer than l_max primaries takes up to min(row cap, floor(l_max / 2),
 * l_max - primaries) backups from each primary hash's next `quota` distinct
 * targets, ranked by the mode's priority (hash_prune.rs:655-685,
 * hash_prune_backfill.rs:299-386) and emitted after the primaries
 * (hash_prune.rs:1458-1555); the result is the reference's
 * order-independent characterization hash_prune.rs:2601-2682, so batches
 * still merge in any order.  Zero fields take the reference's defaults
 * (quota 1 for hash-slot-1, else 3; cap floor(l_max / 2); alpha 1.1).
 * Extra device memory: num_points * l_max * 24 bytes.  insert,
 * insert_segments, clear and destroy are as above; neighbors writes
 * primaries then backups and counts them both. */
#define TESSA_HP_BACKFILL_OFF 0u
#define TESSA_HP_BACKFILL_RHALF_HASH_SLOT_1 1u
#define TESSA_HP_BACKFILL_RHALF_DISTANCE_FIRST_Q3 2u
#define TESSA_HP_BACKFILL_RHALF_SOFT_TIER_Q3 3u
#define TESSA_HP_BACKFILL_RHALF_HARD_TIER_Q3 4u
typedef struct tessa_hashprune_backfill {
    uint32_t mode;                    /* TESSA_HP_BACKFILL_* */
    uint32_t hash_quota;              /* 0 or 1..3 */
    uint32_t max_backfill_per_row;    /* 0 or 1..floor(l_max / 2) */
    float soft_tier_priority_alpha;   /* 0, or finite >= 1.0 (SoftTier only) */
} tessa_hashprune_backfill;
tessa_status tessa_hashprune_create_backfill(uint32_t num_points, uint32_t l_max,
                                             const tessa_hashprune_backfill *policy, tessa_hashprune **out);

/* ---- TierLift: the bounded host reducer of the record stream ---------------
 * Replaces SpillEdgeSink + ExternalHashPruneReducer
 * (shear-core/src/algorithm/pipnn/spill_hashprune.rs:349-651 routing, shard
 * buffers and segment flush; :727-851 part files and manifest; :853-892
 * shard-by-shard reduction).  Records leave the device as the leaves emit
 * them and are held on the host, bounded by host_budget_bytes, in
 * source-range shards (src / shard_points); past the budget the shard with
 * the most buffered records is written to spill files as the reference
 * writes them: segments of at most 1,000,000 records sorted by src, in
 * `{stem}_shard{shard:05}_part{part:03}.log` next to spill_base (rolled over
 * past 4 GiB), listed in `candidate_segments.manifest` (shard, file, offset,
 * bytes, records, src_min, src_max, sorted=1; ordered by shard, file,
 * offset).  With spill_base NULL or "" exceeding the budget is an error
 * (overflow label WORKSPACE_BUDGET).
 *   create   num_points in [1, 2^32), shard_points >= 1 (the reference's
 *            default is 1,000,000), l_max in [1, 256], staging_records per
 *            pinned slot (two slots), threads for host routing / spill sorting
 *            (0: up to 16);
 *   push     device records (count of them) produced on `stream`: enqueues,
 *            on the reducer's own stream after the work already on `stream`
 *            (never making `stream` wait), a sort of the batch by (src, dst)
 *            that drops exact repeats of a record (the same pair seen forward
 *            and reverse; a reservoir ignores a repeat, so the reduction is
 *            unchanged) and the D2H copy of what is kept; blocks only while
 *            both staging slots are still being routed; *seq_out = the
 *            sequence number of the batch's last slot;
 *   copied   *seq = the highest sequence number whose batch has been read
 *            on the device (the device records of every push up to it may be
 *            reused);
 *   wait     blocks until batch `seq` has been read;
 *   finish   writes the manifest, then reduces shard by shard on the device
 *            (spilled segments, then buffered records, through HashPrune
 *            reservoirs as tessa_hashprune_*) into targets [num_points * l_max]
 *            and counts [num_points] (device pointers, the layout
 *            tessa_hashprune_neighbors writes); enqueued on and synchronises
 *            `stream`; equal to one tessa_hashprune reduction of every record
 *            pushed.  Once only; no push after it;
 *   destroy  stops the worker and frees every buffer (spill files remain).
 * Spilling runs on a thread of its own: past 7/8 of the budget the shard with
 * the most buffered records is handed to it while routing goes on; pushes
 * block only past the budget itself.  When expected_records says the stream
 * will not fit the budget, the shards beyond those that fit are spilled from
 * the start (whenever one has 256 MB buffered), so the disk writes overlap
 * the whole stream; the reduction is the same either way, only which records
 * sit in which part file differs.
 * A record with src >= num_points fails the push that carried it, and every
 * later call, with "Spill reducer encountered edge p=... outside shard
 * range". */
typedef struct tessa_tierlift tessa_tierlift;
typedef struct tessa_tierlift_config {
    uint64_t num_points;
    uint64_t shard_points;
    uint64_t host_budget_bytes;   /* bytes of host record blocks (1,000,000 records each) */
    uint64_t staging_records;     /* records per pinned staging slot */
    const char *spill_base;       /* candidate path whose directory and stem name the spill files */
    uint32_t l_max;
    uint32_t threads;
    uint64_t expected_records;    /* 0, or about how many records will be pushed (see below) */
} tessa_tierlift_config;
typedef struct tessa_tierlift_stats {
    uint64_t records;             /* records pushed */
    uint64_t pushes;              /* staging slots filled */
    uint64_t host_peak_bytes;     /* largest host block allocation */
    uint64_t spilled_records;
    uint64_t spilled_bytes;
    uint64_t segments;
    uint64_t reread_records;      /* records read back from spill files at finish */
    uint32_t shards;
    uint32_t threads;
    double route_s;               /* worker time routing records to shards */
    double spill_s;               /* spill-thread time sorting and writing segments */
    double reduce_s;              /* finish: manifest, uploads, reservoir merges */
    uint64_t unique_records;      /* records kept after dropping exact repeats within each batch */
} tessa_tierlift_stats;
tessa_status tessa_tierlift_create(const tessa_tierlift_config *cfg, tessa_tierlift **out);
tessa_status tessa_tierlift_push(tessa_tierlift *t, const tessa_edge_record *records, uint64_t count, void *stream,
                                 uint64_t *seq_out);
tessa_status tessa_tierlift_copied(tessa_tierlift *t, uint64_t *seq);
tessa_status tessa_tierlift_wait(tessa_tierlift *t, uint64_t seq);
tessa_status tessa_tierlift_finish(tessa_tierlift *t, uint32_t *targets, uint32_t *counts, void *stream,
                                   tessa_tierlift_stats *stats);
tessa_status tessa_tierlift_destroy(tessa_tierlift *t);

/* ---- graph emission ----------------------------------------------------------
 * The `_mem.index` byte image DirectMemGraphWriter writes
 * (index/inmem_index/pipnn_oom_writer.rs:23-72: create, write_node per point
 * in id order, finish rewriting the header), built on the GPU from a
 * neighbour table: point p's row is targets[p * row_stride .. + counts[p]]
 * (counts clipped to row_stride), e.g. the HashPrune reservoirs' slot
 * targets.  Layout (little-endian): index_size u64 (the file size),
 * max_degree u32, start u32, num_frozen_pts u64, then per point degree u32
 * and its ids.  Device pointers; `out` 8-byte aligned, or NULL to get only
 * *index_size.  Synchronises `stream` once (to read the size). */
tessa_status tessa_graph_pack(const uint32_t *targets, const uint32_t *counts, uint32_t num_points,
                              uint32_t row_stride, uint32_t start, uint64_t num_frozen_pts, void *out,
                              uint64_t out_capacity, uint64_t *index_size, void *stream);

/* ---- assignment-task capture ------------------------------------------------
 * The partition side of the TESSA capture (the in-kernel sampler
 * gpu_tessa_capture_assignment, compute_backend.rs:5415-5546): with capture
 * on (min_members > 0; the reference samples tasks of >= 256 members and 1..128
 * leaders), each run_subtree records every assignment pass of a node with at
 * least min_members rows: depth, retry (attempt), r_h (fanout), padded_dim,
 * members and leaders as global ids, in pass order.  Nodes of a small root
 * (one kernel, <= leaf_max rows) are not recorded.  Fetch after the run: a
 * first call with tasks and ids NULL gives the counts.  The bottom-k
 * selection and the fixture files are the host sampler's (tessa_capture.rs).
 * The session keeps the passes of its most recent subtree run only: every
 * run (synchronous, or a submitted job when the worker starts it) replaces
 * them, and an SQ8 upload clears them.  Ids are translated to global ids
 * when the run ends, so they name the resident set that run used.  With
 * submissions, fetch after tessa_session_wait of the job whose passes are
 * wanted and before the next job is submitted.  A run records at most 2^27 member and
 * leader ids (512 MB of host memory); passes past that bound are not
 * recorded (the reference's in-kernel sampler keeps a bounded set per bin;
 * here the host sampler chooses among what was recorded). */
typedef struct tessa_captured_assignment {
    uint32_t depth, retry, r_h, padded_dim, member_count, leader_count;
    uint64_t member_offset, leader_offset;  /* into ids[] */
} tessa_captured_assignment;
tessa_status tessa_session_set_assignment_capture(tessa_session *s, uint32_t min_members);
tessa_status tessa_session_captured_assignments(tessa_session *s, tessa_captured_assignment *tasks,
                                                uint64_t task_capacity, uint32_t *ids, uint64_t id_capacity,
                                                uint64_t *task_count, uint64_t *id_count);

/* ---- global D0 assignment: task formation above the subtrees --------------
 * The GPU-D0 SQ8 assignment (shear-core/src/algorithm/pipnn/compute_backend.rs:
 * sq8_global_d0_*_partial_kernel :18016-18275 + the tile merge :18446-18511;
 * CPU statement quantize_sq8_and_assign_global_d0_reference,
 * dco_sq_int8.rs:1929-2064): every SQ8 row to its fanout_top nearest leaders
 * by sq_int8_approx_l2 (dco_sq_int8.rs:2950-2965), ordered by (distance,
 * leader global id).  Outputs row-major [rows x fanout_top] fragments:
 * out_child (leader index = D0 child), out_point (the row's global id).  With
 * child_offsets [leader_count + 1] and child_points [rows * fanout_top] (both
 * or neither) the fragments are also grouped by child, rows ascending within
 * a child (the D0 children's point lists).  Leader payload: SQ8 codes /
 * scales / norms of the leaders (same padded_dim) and their global ids.
 * fanout_top in [1, min(32, leader_count)] (the reference's "SQ GPU-D0 staging
 * fanout must be in 1..=min(32, leaders)"); at most 65,536 leaders; padded_dim a
 * multiple of 16 up to 1024; rows * fanout_top < 2^31 when grouping.  Device pointers; enqueued on
 * `stream`. */
tessa_status tessa_global_d0_assign(const int8_t *codes, const float *scales, const float *norms,
                                    const uint32_t *global_ids, uint64_t rows, uint32_t padded_dim,
                                    const int8_t *leader_codes, const float *leader_scales,
                                    const float *leader_norms, const uint32_t *leader_ids, uint32_t leader_count,
                                    uint32_t fanout_top, uint32_t *out_child, uint32_t *out_point,
                                    uint64_t *child_offsets, uint32_t *child_points, void *stream);

/* ---- final RobustPrune -------------------------------------------------------
 * final_prune_pipnn (index/inmem_index/pipnn_builder.rs:287-330) with
 * robust_prune / occlude_list (algorithm/prune/prune.rs:17-214) over every
 * row of a neighbour table (row p = targets[p * row_stride .. + counts[p]],
 * ids >= num_points skipped): the pool sorted by (distance, id), cut to
 * max_occlusion (the reference's max_occlusion_size, default 750), alpha
 * passes 1.0, x1.2, .. <= alpha (index_write_parameter.alpha, default 1.2),
 * at most max_degree kept (default 64); saturate != 0 fills up from the pool
 * when alpha > 1 (saturate_graph, default off).  Distances: squared L2 of
 * f32 rows summed in coordinate order without contraction.  Outputs
 * out_targets [num_points x max_degree] (0xFFFFFFFF past out_counts[p]) and
 * out_counts [num_points].  row_stride and max_degree <= 256.  Device
 * pointers; enqueued on `stream`. */
tessa_status tessa_robust_prune(const float *data, uint32_t num_points, uint32_t dim, const uint32_t *targets,
                                const uint32_t *counts, uint32_t row_stride, uint32_t max_degree,
                                uint32_t max_occlusion, float alpha, int saturate, uint32_t *out_targets,
                                uint32_t *out_counts, void *stream);

/* ---- greedy search: the recall harness ---------------------------------------
 * InmemIndex::search (index/inmem_index/inmem_index.rs:523-590) over a
 * neighbour table (row p = targets[p * row_stride .. + counts[p]], ids >=
 * num_points skipped): greedy_search (algorithm/search/search.rs:137-233) from
 * `start` with the capacity-L queue of neighbor_priority_queue.rs:50-85,
 * ordered by (distance, id); per query the first K entries.  Distances are
 * squared L2 over f32 vectors, summed in coordinate order without
 * contraction.  Outputs, row-major [num_queries x K]: out_ids (0xFFFFFFFF
 * past the list's end), out_dists (may be NULL); out_cmps [num_queries]
 * distance evaluations after the start's (may be NULL).  L in [1, 256], K in
 * [1, L] (K > L: the reference's "Set L: .. to a value of at least K: .."),
 * start < num_points < 0xFFFFFFFF, finite data.  Device pointers; enqueued
 * on `stream`; workspace: up to 1 GiB of visited tags. */
tessa_status tessa_graph_search(const float *data, uint32_t num_points, uint32_t dim, const uint32_t *targets,
                                const uint32_t *counts, uint32_t row_stride, uint32_t start, const float *queries,
                                uint32_t num_queries, uint32_t L, uint32_t K, uint32_t *out_ids, float *out_dists,
                                uint32_t *out_cmps, void *stream);
/* The same search over SQ8 rows, for point sets whose f32 vectors do not
 * stay resident (the out-of-memory configuration): row p reads as the f32
 * products scales[p] * codes[p * padded_dim + i] (each rounded), i < dim, so
 * the result is the search over the dequantized vectors.  It has no
 * counterpart in the reference, whose search loads full-precision vectors;
 * it serves the recall harness only.  padded_dim >= dim. */
tessa_status tessa_graph_search_sq8(const int8_t *codes, const float *scales, uint32_t padded_dim, uint32_t num_points,
                                    uint32_t dim, const uint32_t *targets, const uint32_t *counts, uint32_t row_stride,
                                    uint32_t start, const float *queries, uint32_t num_queries, uint32_t L, uint32_t K,
                                    uint32_t *out_ids, float *out_dists, uint32_t *out_cmps, void *stream);

/* ---- asynchronous subtree submissions ----------------------------------
 * Replaces submit_owned_quantized_subtree_l2_compact_topk
 * (compute_backend.rs:3807-3815) with its Deferred result and pinned host-slot
 * ring (CudaDeferredPinnedQuantizedScatter, :31432-31497): the device work of
 * one task overlaps the caller's host-side use of the previous result.
 * A session runs submissions in order on a worker thread of its own and holds
 * two pinned host result slots.  submit copies the request (and its root
 * leader ids); `host_sq8` (may be NULL: keep the current upload) is uploaded
 * by the job, so its arrays must stay valid until tessa_session_wait returns.
 * submit fails when both slots hold unreleased results.  The request's
 * output capacities (max_leaf_count, max_leaf_rows) size the session's device
 * outputs.  wait blocks until the job is done and returns its status; the
 * result arrays stay valid until tessa_session_release(seq).  Other session
 * calls wait for a running job. */
typedef struct tessa_subtree_host_result {
    const uint32_t *leaf_row_ids;   /* pinned host, leaf_rows (resident rows) */
    const uint64_t *leaf_starts;    /* leaf_count */
    const uint64_t *leaf_sizes;     /* leaf_count */
    const uint32_t *topk_ids;       /* leaf_rows * k, global ids */
    const float *topk_dists;        /* leaf_rows * k */
    const uint64_t *counters;       /* TESSA_SUBTREE_COUNTER_WORDS */
    const uint64_t *leaf_counters;  /* TESSA_COUNTER_WORDS */
    uint64_t leaf_count;
    uint64_t leaf_rows;
    uint32_t k;
    uint32_t levels;
    float partition_ms;
    float leaf_ms;
} tessa_subtree_host_result;

tessa_status tessa_session_submit_subtree(tessa_session *session, const tessa_sq8_view *host_sq8,
                                          const tessa_subtree_request *req, uint64_t *seq);
tessa_status tessa_session_wait(tessa_session *session, uint64_t seq, tessa_subtree_host_result *out);
tessa_status tessa_session_release(tessa_session *session, uint64_t seq);

/* Diagnostic, no counterpart in the reference: the sustained int8 MFMA rate
 * of the current GPU (v_mfma_i32_32x32x32_i8 chains on random register
 * operands, no memory traffic; `chains` in {2, 4, 8} per wave, 256-thread
 * workgroups) and the shader clock it ran at, the fastest of three runs.  It
 * is the practical ceiling the leaf filter's roofline is read against; it
 * allocates and synchronises the device. */
tessa_status tessa_probe_mfma_rate(uint32_t workgroups, uint32_t chains, uint64_t iters, double *tops,
                                   double *mhz);

/* "QUEUE_NODE|LEAF_ROW|..." or "none" (same labels as the reference). */
void tessa_overflow_labels(uint64_t flags, char *buf, size_t len);
uint32_t tessa_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
