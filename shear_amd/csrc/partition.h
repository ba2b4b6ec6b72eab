// partition.h -- the recursive subtree partition (leader assignment, split
// control, scatter and leaf publication) on gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace tessa {

constexpr uint32_t kPartMaxLeaders = 128;  // GPU_QUEUE_LEADER_STRIDE compute_backend.rs:371
constexpr uint32_t kPartItemRows = 512;    // rows of one assignment / scatter work item
constexpr uint32_t kChildEmpty = 0xffffffffu;
constexpr uint32_t kChildNodeBit = 0x80000000u;

enum NodeStatus : uint32_t {
    kNodeIdle = 0,      // dropped (overflow) or not staged
    kNodeCounting = 1,  // leaders staged; COUNT pending
    kNodeAccepted = 2,  // split accepted (compute_backend.rs:15527-15549)
    kNodeBalanced = 3,  // even/odd fallback (compute_backend.rs:15485-15510)
};

// One node of the current level (the reference's 7-word queue node plus the
// large-task words it carries through COUNT / EMIT / SCATTER / PUBLISH).
struct NodeDesc {
    uint64_t row_start;  // offset of the node's rows in the level arena
    uint64_t seed;
    uint32_t n;
    uint32_t depth;
    uint32_t num_leaders;
    uint32_t fanout;
    uint32_t attempt;
    uint32_t max_leaders;
    uint32_t status;
    uint32_t retry_allowed;
    uint32_t item_base;
    uint32_t items;
    uint32_t leaf_children;
    uint32_t node_children;
    uint64_t leaf_rows;
    uint64_t node_rows;
    uint64_t leaf_base;      // absolute index of the node's first leaf
    uint64_t leaf_row_base;  // absolute offset of its first leaf row
    uint64_t node_base;      // index of its first child in the next level
    uint64_t node_row_base;  // offset of that child's rows in the next arena
    uint64_t root_base;      // resident index of its root's first row (0 for a single root)
    uint32_t root_index;     // its root (0 for a single root)
    uint32_t pad;
};

constexpr uint32_t kPartMaxAttempts = 16;  // COUNT / EMIT passes per level

// Walk outcome words (LevelHeader::walk_status).
enum WalkStatus : uint32_t {
    kWalkOk = 0,
    kWalkBound = 2,     // level or attempt bound exceeded
    kWalkCapacity = 3,  // the next level's work items exceed the workspace
    kWalkStalled = 4,   // a grid barrier outlived the watchdog (WATCHDOG_STALLED)
};

// Level summary and the walk's control words, in device memory; the host
// reads it once the partition has finished (and, on the capture path,
// after every level).
struct LevelHeader {
    uint64_t leaf_count;
    uint64_t leaf_rows;
    uint64_t next_rows;
    uint64_t overflow;
    uint32_t next_nodes;
    uint32_t items;
    uint32_t retry_nodes;
    uint32_t pad;
    // persistent walk: grid barrier arrivals (monotonic over the launch),
    // EMIT retries per attempt of the current level, and the walk's result
    uint32_t barrier;
    uint32_t walk_status;
    uint32_t levels;
    uint32_t count_passes;
    uint32_t retry[kPartMaxAttempts];
};

struct PartArgs {
    // resident rows 0..rows-1; row r's SQ8 row is row_map[r] (r when row_map is null)
    const int8_t *codes;
    const float *scales;
    const float *norms;
    const uint32_t *row_map;
    uint32_t rows;
    uint32_t padded_dim;
    // several roots in one run (root_count > 0): root i owns resident rows
    // [root_offsets[i], root_offsets[i+1]) and starts from root_seeds[i];
    // each root's rows are partitioned exactly as a single-root run over
    // those rows alone would partition them (assignment tie keys use the
    // row's index within its root)
    const uint64_t *root_offsets;  // device
    const uint64_t *root_seeds;    // device
    uint32_t root_count;
    // request
    const uint32_t *root_leaders;  // device, may be null
    uint32_t root_leader_count;
    uint32_t root_depth;
    uint32_t max_depth;
    uint32_t max_leaders;
    uint32_t fanout_second;
    uint32_t leaf_min;
    uint32_t leaf_max;
    uint32_t small_node_limit;
    uint32_t k;  // top-k row stride used for leaf output offsets
    float psamp;
    uint64_t seed;
    uint64_t large_scratch_rows;
    uint64_t max_leaf_count;
    uint64_t max_leaf_rows;
    // leaf layout outputs
    uint32_t *leaf_row_ids;
    uint64_t *leaf_starts;
    uint64_t *leaf_sizes;
    uint32_t *leaf_sizes32;
    uint64_t *leaf_out_offsets;
    uint32_t *leaf_root;   // optional: each leaf's root index
    uint32_t *leaf_depth;  // optional: each leaf's depth
    uint64_t *counters;  // TESSA_SUBTREE_COUNTER_WORDS, reference layout
    LevelHeader *hdr;
    // workspace
    uint32_t *arena[2];
    NodeDesc *nodes[2];
    uint32_t *leaders;       // node_cap x 128
    uint32_t *child_counts;  // node_cap x 128
    uint32_t *child_idx;     // node_cap x 128: leaf or next-node index within the node
    uint32_t *child_rel;     // node_cap x 128: row offset within the node's leaf / node rows
    uint32_t *slots;         // arena_cap: 4 packed 8-bit leader slots per row
    uint32_t *item_counts;   // item_cap x 128
    uint32_t *item_node;     // item_cap: the level's item -> node map
    uint64_t arena_cap;
    uint64_t item_cap;
    uint32_t node_cap;
    // persistent walk: a grid barrier that waits longer than this many
    // wall-clock ticks flags WATCHDOG_STALLED and ends the walk
    uint64_t watchdog_ticks;
};

struct PartResult {
    uint64_t leaf_count;
    uint64_t leaf_rows;
    uint32_t levels;
    uint32_t count_launches;
    // on a -1 return: the failing HIP call's error and what it was doing
    int hip_error;
    const char *failed_step;
};

// Assignment tasks seen by the COUNT passes (capture, host side): per task
// depth, attempt, fanout and its member / leader resident rows.  Filled only
// when a PartCapture is passed; tasks outside the capture bins (fewer than
// min_members members, no leaders or more than 128) are not kept.
struct PartCaptureTask {
    uint32_t depth, retry, r_h, member_count, leader_count;
    uint64_t member_offset, leader_offset;  // into rows[]
};
struct PartCapture {
    uint32_t min_members = 256;
    uint64_t max_rows = 1ull << 27;  // host bound: members + leaders kept per run (512 MB)
    uint64_t dropped_tasks = 0;      // passes past max_rows, not recorded
    std::vector<PartCaptureTask> tasks;
    std::vector<uint32_t> rows;  // members then leaders of each task, resident rows
};

// Workspace sizes for `rows` resident rows with root fanout `famp`.
void partition_capacity(uint64_t rows, uint32_t famp, uint32_t leaf_max, uint64_t *arena_cap, uint32_t *node_cap,
                        uint64_t *item_cap);

// Runs the whole partition on `stream`: one persistent walk kernel for the
// level loop (no host round trip between levels), or, when `capture` is
// given, the level-by-level launches with a host copy before each COUNT
// pass.  Returns 0, or -1 on a launch failure, -2 when the level loop
// exceeds its bound, -3 when a workspace capacity is exceeded, -4 when the
// walk's watchdog fired (also flagged as WATCHDOG_STALLED).
int run_partition(const PartArgs &a, hipStream_t stream, LevelHeader *host_hdr, PartResult *res,
                  PartCapture *capture = nullptr);

}  // namespace tessa
