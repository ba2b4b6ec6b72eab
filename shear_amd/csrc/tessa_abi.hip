// tessa_abi.hip -- the extern "C" boundary declared in include/tessa_hip.h.
//
// Host-side validation, per-device workspace and sessions.  Nothing here
// throws or aborts across the boundary: every failure becomes a tessa_status
// with a message that keeps the reference's "overflow_flags=0x.." and label
// tokens (compute_backend.rs:2198-2296), which SHEAR's orchestration matches
// by substring (rbc_partition.rs:2982-2998).
#include <hip/hip_runtime.h>

#include <cmath>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "../../include/tessa_hip.h"
#include "assign_kernels.h"
#include "d0_kernels.h"
#include "edge_kernels.h"
#include "graph_kernels.h"
#include "hashprune_kernels.h"
#include "leaf_kernels.h"
#include "partition.h"
#include "prune_kernels.h"
#include "search_kernels.h"
#include "tessa_device.h"


using namespace tessa;

namespace {

tessa_status make_status(int32_t code, uint64_t flags, const char *fmt, ...) {
    tessa_status s;
    std::memset(&s, 0, sizeof(s));
    s.code = code;
    s.overflow_flags = flags;
    if (fmt) {
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(s.msg, sizeof(s.msg), fmt, ap);
        va_end(ap);
    }
    return s;
}

tessa_status ok_status() { return make_status(TESSA_OK, 0, nullptr); }

#define TESSA_HIP_TRY(expr)                                                                       \
    do {                                                                                          \
        hipError_t _e = (expr);                                                                   \
        if (_e != hipSuccess)                                                                     \
            return make_status(TESSA_ERR_HIP, 0, "%s failed: %s", #expr, hipGetErrorString(_e));  \
    } while (0)

__global__ void fill_u32_kernel(uint32_t *p, uint32_t n, uint32_t v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// out[0] = largest value of a[0, n) (out[0] starts at 0).
__global__ void max_u32_kernel(const uint32_t *a, uint64_t n, uint32_t *out) {
    uint32_t m = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        m = a[i] > m ? a[i] : m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = __shfl_xor(m, off);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63u) == 0u) atomicMax(out, m);
}

// x[i] = map[x[i]] for i < n (resident indices -> SQ8 rows).
__global__ void map_rows_kernel(uint32_t *x, uint64_t n, const uint32_t *map) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        x[i] = map[x[i]];
}

// Per-device workspace of the MFMA leaf path: the exact re-run queue (pairs
// (leaf, row)), the chain queue (headers + candidate pool) and their three
// counters.  Grown on demand; kept until the process ends (other callers may
// share the device).
struct DeviceWorkspace {
    uint32_t *queue_counts = nullptr;  // [0] fallback, [1] chain rows, [2] chain pool used, [4..12] filter
                                       // tickets, [13] listed work items
    uint2 *item_list = nullptr;        // (leaf, block) work items of a call
    uint64_t item_list_capacity = 0;
    uint32_t *fallback = nullptr;
    uint64_t fallback_capacity = 0;
    uint4 *chain_rows = nullptr;
    uint64_t chain_capacity = 0;
    uint4 *chain_pool = nullptr;
    uint64_t pool_capacity = 0;
    uint2 *survivor_log = nullptr;  // batch items x kLeafFilterThreads x kLeafLogCapacity entries
    uint64_t log_entries = 0;
    uint4 *row_meta = nullptr;      // batch items x kLeafBlockRows
    uint64_t row_meta_capacity = 0;
    // edge-record kernels: per-leaf totals, leaf record offsets, status words
    uint32_t *edge_totals = nullptr;
    uint64_t edge_totals_capacity = 0;
    uint64_t *edge_base = nullptr;
    uint64_t edge_base_capacity = 0;
    uint64_t *edge_seg_base = nullptr;  // source-grouped order: first segment of each leaf
    uint64_t edge_seg_base_capacity = 0;
    uint64_t *edge_status = nullptr;
    uint64_t edge_status_capacity = 0;
    // graph packing: scan partials, row offsets, (total words, max degree)
    uint64_t *graph_sums = nullptr;
    uint64_t graph_sums_capacity = 0;
    uint64_t *graph_row_off = nullptr;
    uint64_t graph_row_off_capacity = 0;
    uint64_t *graph_scalars = nullptr;
    uint64_t graph_scalars_capacity = 0;
    // greedy search: visited tags, slots x points
    uint32_t *search_tags = nullptr;
    uint64_t search_tags_capacity = 0;
    // D0 assignment: leader ranks and their inverse, grouping scratch
    uint32_t *d0_rank = nullptr;
    uint64_t d0_rank_capacity = 0;
    uint8_t *d0_temp = nullptr;
    uint64_t d0_temp_capacity = 0;
};
std::mutex g_ws_mutex;
std::vector<DeviceWorkspace> g_ws;

template <typename T>
tessa_status grow(T **ptr, uint64_t *cap, uint64_t need, size_t elem_bytes, const char *what) {
    if (*cap >= need) return ok_status();
    if (*ptr) {
        TESSA_HIP_TRY(hipDeviceSynchronize());
        TESSA_HIP_TRY(hipFree(*ptr));
        *ptr = nullptr;
        *cap = 0;
    }
    const uint64_t n = need < 4096 ? 4096 : need;
    if (hipMalloc((void **)ptr, n * elem_bytes) != hipSuccess)
        return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                           "%s allocation of %llu entries failed overflow_flags=0x%llx "
                           "overflow_labels=WORKSPACE_BUDGET",
                           what, (unsigned long long)n, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
    *cap = n;
    return ok_status();
}

// Work items per filter/select batch for `rows` member rows: the survivor
// logs of a batch take kLeafLogBytesPerItem each, at most kLeafLogBudget in
// all (the filter addresses a batch's logs with 32-bit byte offsets below
// 2^31, its out-of-range marker: 4,096 items of 512 KB).
constexpr uint64_t kLeafMaxBatchItems = 4096;
constexpr uint64_t kLeafLogBudget = kLeafMaxBatchItems * kLeafLogBytesPerItem;
uint64_t leaf_batch_items(uint64_t rows) {
    const uint64_t cap = kLeafLogBudget / kLeafLogBytesPerItem;
    const uint64_t want = (rows + kLeafBlockRows - 1) / kLeafBlockRows + 1;
    return want < cap ? want : cap;
}

tessa_status get_workspace(uint64_t rows, DeviceWorkspace **out, uint64_t list_items = 0) {
    int dev = 0;
    TESSA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    DeviceWorkspace &ws = g_ws[dev];
    if (ws.queue_counts == nullptr) TESSA_HIP_TRY(hipMalloc(&ws.queue_counts, 64));
    tessa_status st = grow(&ws.fallback, &ws.fallback_capacity, rows, 2 * sizeof(uint32_t), "re-run queue");
    if (st.code) return st;
    // Chain rows are a fraction of all rows; a row that finds the chain queue
    // full takes the exact re-run instead, so these sizes bound speed, not
    // correctness.
    st = grow(&ws.chain_rows, &ws.chain_capacity, rows / 2 + 1, sizeof(uint4), "chain queue");
    if (st.code) return st;
    // candidate sets of 64 queue entries interleaved: whole groups of 64 x 40
    st = grow(&ws.chain_pool, &ws.pool_capacity, (rows / 2 + 64) / 64 * 64 * kLeafChainSetEntries, sizeof(uint4), "chain pool");
    if (st.code) return st;
    // survivor logs and row thresholds of one batch of work items
    const uint64_t items = leaf_batch_items(rows);
    st = grow(&ws.survivor_log, &ws.log_entries, items * kLeafFilterThreads * kLeafLogCapacity, sizeof(uint2),
              "survivor log");
    if (st.code) return st;
    st = grow(&ws.row_meta, &ws.row_meta_capacity, items * kLeafBlockRows, sizeof(uint4), "row thresholds");
    if (st.code) return st;
    if (list_items) {
        st = grow(&ws.item_list, &ws.item_list_capacity, list_items, sizeof(uint2), "work-item list");
        if (st.code) return st;
    }
    *out = &ws;
    return ok_status();
}

// The status of a failed run_partition call.
tessa_status partition_failure(int rc, const tessa::PartResult &pr) {
    if (rc == -1 && pr.failed_step)
        return make_status(TESSA_ERR_HIP, 0, "subtree partition failed (code -1: %s: %s)", pr.failed_step,
                           hipGetErrorName((hipError_t)pr.hip_error));
    if (rc == -4)
        return make_status(TESSA_ERR_HIP, TESSA_OVF_WATCHDOG_STALLED,
                           "CUDA persistent subtree overflow: partition walk stalled overflow_flags=0x%llx "
                           "overflow_labels=WATCHDOG_STALLED",
                           (unsigned long long)TESSA_OVF_WATCHDOG_STALLED);
    return make_status(TESSA_ERR_HIP, 0, "subtree partition failed (code %d: %s)", rc,
                       rc == -2 ? "level/attempt bound exceeded"
                                : rc == -3 ? "workspace capacity exceeded" : "HIP launch failure");
}

tessa_status device_workspace(DeviceWorkspace **out) {
    int dev = 0;
    TESSA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    *out = &g_ws[dev];
    return ok_status();
}

tessa_status check_view(const tessa_sq8_view *v) {
    if (!v || !v->codes || !v->scales || !v->norms || !v->global_ids)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "sq8 view has a null pointer");
    if (v->padded_dim == 0 || v->padded_dim % 16 != 0 || v->dim == 0 || v->dim > v->padded_dim)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "sq8 view dim=%u padded_dim=%u: padded_dim must be a positive multiple of 16 >= dim",
                           v->dim, v->padded_dim);
    if (v->rows == 0 || v->rows > 0xffffffffull)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "sq8 view rows=%llu outside [1, 2^32)",
                           (unsigned long long)v->rows);
    return ok_status();
}

}  // namespace

extern "C" {

uint32_t tessa_abi_version(void) { return TESSA_ABI_VERSION; }

void tessa_overflow_labels(uint64_t flags, char *buf, size_t len) {
    static const struct {
        uint64_t bit;
        const char *label;
    } kLabels[] = {
        {TESSA_OVF_QUEUE_NODE, "QUEUE_NODE"},
        {TESSA_OVF_QUEUE_ROW, "QUEUE_ROW"},
        {TESSA_OVF_LEAF_DESC, "LEAF_DESC"},
        {TESSA_OVF_LEAF_ROW, "LEAF_ROW"},
        {TESSA_OVF_LEADER, "LEADER"},
        {TESSA_OVF_FANOUT_OVER_32, "FANOUT_OVER_32"},
        {TESSA_OVF_NO_PROGRESS_SPLIT, "NO_PROGRESS_SPLIT"},
        {TESSA_OVF_WORKSPACE_BUDGET, "WORKSPACE_BUDGET"},
        {TESSA_OVF_OVERSIZED_TERMINAL_NODE, "OVERSIZED_TERMINAL_NODE"},
        {TESSA_OVF_WATCHDOG_STALLED, "WATCHDOG_STALLED"},
        {TESSA_OVF_ACTIVE_WORK_BUDGET, "ACTIVE_WORK_BUDGET"},
        {TESSA_OVF_INVALID_TOPK_ROW_ID, "INVALID_TOPK_ROW_ID"},
        {TESSA_OVF_INVALID_TOPK_COL_ID, "INVALID_TOPK_COL_ID"},
        {TESSA_OVF_INVALID_ASSIGN_POINT_ID, "INVALID_ASSIGN_POINT_ID"},
        {TESSA_OVF_INVALID_ASSIGN_LEADER_ID, "INVALID_ASSIGN_LEADER_ID"},
        {1ull << 17, "WMMA_DEBUG_ABORT"},
        {TESSA_OVF_UNSUPPORTED_EXPLICIT_KERNEL, "UNSUPPORTED_EXPLICIT_KERNEL"},
        {1ull << 19, "LARGE_TILE_CAPACITY"},
    };
    if (!buf || len == 0) return;
    buf[0] = '\0';
    uint64_t known = 0;
    size_t used = 0;
    for (const auto &l : kLabels) {
        known |= l.bit;
        if (flags & l.bit) {
            int w = std::snprintf(buf + used, len - used, "%s%s", used ? "|" : "", l.label);
            if (w < 0 || (size_t)w >= len - used) return;
            used += (size_t)w;
        }
    }
    uint64_t unknown = flags & ~known;
    if (unknown) {
        int w = std::snprintf(buf + used, len - used, "%sUNKNOWN_0x%llx", used ? "|" : "",
                              (unsigned long long)unknown);
        if (w < 0 || (size_t)w >= len - used) return;
        used += (size_t)w;
    }
    if (used == 0) std::snprintf(buf, len, "none");
}

tessa_status tessa_query_caps(int32_t device, tessa_caps *out) {
    if (!out) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "caps output is null");
    std::memset(out, 0, sizeof(*out));
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return make_status(TESSA_ERR_NO_DEVICE, 0, "no HIP device visible");
    if (device < 0 || device >= count)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "device %d outside [0, %d)", device, count);
    hipDeviceProp_t prop;
    TESSA_HIP_TRY(hipGetDeviceProperties(&prop, device));
    out->device = device;
    out->compute_units = prop.multiProcessorCount;
    out->max_threads_per_block = prop.maxThreadsPerBlock;
    out->lds_bytes_per_block = (int32_t)prop.sharedMemPerBlock;
    out->hbm_bytes = prop.totalGlobalMem;
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    out->supported = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    out->max_leaf_rows = 4096;
    out->max_k = kMaxK;
    out->max_padded_dim = 1024;
    return ok_status();
}

}  // extern "C"

namespace {

// Events bracketing the leaf kernels: per batch the filter and the select
// kernel (three events), then the chain replay and the exact re-run; one
// set per device, created on first use and grown with the batch count.
struct PhaseEvents {
    std::vector<hipEvent_t> e;
};
std::mutex g_ev_mutex;
std::vector<PhaseEvents> g_events;

tessa_status phase_events(PhaseEvents **out) {
    int dev = 0;
    TESSA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ev_mutex);
    if ((int)g_events.size() <= dev) g_events.resize(dev + 1);
    *out = &g_events[dev];
    return ok_status();
}

tessa_status ensure_events(PhaseEvents *pe, size_t count) {
    while (pe->e.size() < count) {
        hipEvent_t ev = nullptr;
        TESSA_HIP_TRY(hipEventCreate(&ev));
        pe->e.push_back(ev);
    }
    return ok_status();
}

// Device buffers of the MFMA leaf path: queue counters (16 words), the exact
// re-run queue, the chain queue and pool, one batch of survivor logs and row
// thresholds (log_items work items) and the call's work-item list.
struct LeafScratch {
    uint32_t *queue_counts;
    uint32_t *fallback;
    uint64_t fallback_capacity;
    uint4 *chain_rows;
    uint64_t chain_capacity;
    uint4 *chain_pool;
    uint64_t pool_capacity;
    uint2 *log;
    uint64_t log_items;
    uint4 *row_meta;
    uint2 *item_list;
    uint64_t item_list_capacity;
};

// The call's work items: each leaf's non-empty blocks (an oversized leaf
// keeps its first blocks, so the filter flags it), reserved with one atomic
// per wave; a leaf's blocks are listed in a row.
__global__ void leaf_item_list_kernel(const uint32_t *counts, uint32_t leaf_count, uint32_t blocks_per_leaf,
                                      uint2 *list, uint32_t *total) {
    const uint32_t l = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n = l < leaf_count ? counts[l] : 0u;
    uint32_t nb = (n + kLeafBlockRows - 1u) / kLeafBlockRows;
    nb = nb < blocks_per_leaf ? nb : blocks_per_leaf;
    uint32_t incl = nb;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t v = __shfl_up(incl, d);
        incl += lane >= (uint32_t)d ? v : 0u;
    }
    uint32_t base = 0u;
    if (lane == 63u && incl) base = atomicAdd(total, incl);
    base = __shfl(base, 63);
    const uint32_t first = base + incl - nb;
    for (uint32_t b = 0; b < nb; ++b) list[first + b] = make_uint2(l, b);
}

// Leaf top-k over device layouts; `rows_bound` bounds the member rows and
// sizes the re-run / chain queues.  `ev` (optional) brackets the kernels.
// `fixed` (optional) supplies the scratch buffers; else the per-device
// workspace is grown to fit.
tessa_status leaf_topk_impl(const tessa_sq8_view *sq8, const tessa_leaf_batch *lb, uint64_t rows_bound,
                            uint32_t *out_ids, float *out_dists, uint64_t *counters, void *stream,
                            PhaseEvents *ev, uint64_t *batches_out = nullptr, const LeafScratch *fixed = nullptr) {
    tessa_status st = check_view(sq8);
    if (st.code) return st;
    if (!lb || !lb->members || !lb->member_offsets || !lb->member_counts || !lb->output_offsets || !out_ids ||
        !out_dists)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf batch has a null pointer");
    if (lb->k == 0 || lb->k > (uint32_t)kMaxK)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf k=%u outside [1, 32]", lb->k);
    if (lb->leaf_count == 0) return ok_status();
    if (lb->max_leaf_rows == 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "max_leaf_rows must be positive");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    LeafParams p{};
    p.codes = sq8->codes;
    p.scales = sq8->scales;
    p.norms = sq8->norms;
    p.gids = sq8->global_ids;
    p.rows = sq8->rows;
    p.padded_dim = sq8->padded_dim;
    p.k = lb->k;
    p.members = lb->members;
    p.member_offsets = lb->member_offsets;
    p.member_counts = lb->member_counts;
    p.output_offsets = lb->output_offsets;
    p.leaf_count = lb->leaf_count;
    p.max_leaf_rows = lb->max_leaf_rows;
    p.out_ids = out_ids;
    p.out_dists = out_dists;
    p.counters = counters;
    p.debug_rerun_every = lb->debug_rerun_every;
    const uint32_t exec = lb->executor;
    if (exec == TESSA_EXEC_EXACT) {
        if (launch_leaf_exact_all(p, s) != 0)
            return make_status(TESSA_ERR_HIP, 0, "exact leaf kernel launch failed");
        return ok_status();
    }
    if (exec != TESSA_EXEC_MFMA)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_UNSUPPORTED_EXPLICIT_KERNEL,
                           "unknown leaf executor %u overflow_flags=0x%llx overflow_labels=UNSUPPORTED_EXPLICIT_KERNEL",
                           exec, (unsigned long long)TESSA_OVF_UNSUPPORTED_EXPLICIT_KERNEL);
    if (!leaf_mfma_supported(sq8->padded_dim, lb->max_leaf_rows))
        return make_status(TESSA_ERR_UNSUPPORTED, 0,
                           "MFMA leaf path needs padded_dim <= 1024 and max_leaf_rows <= 4096 (got %u, %u)",
                           sq8->padded_dim, lb->max_leaf_rows);
    const uint32_t bpl = (lb->max_leaf_rows + kLeafBlockRows - 1) / kLeafBlockRows;
    const uint64_t items = (uint64_t)bpl * lb->leaf_count;  // bound of the listed items
    if (items > 0xffffff00ull) return make_status(TESSA_ERR_UNSUPPORTED, 0, "more than 2^32 leaf work items");
    LeafScratch sc{};
    if (fixed) {
        sc = *fixed;
        if (items > sc.item_list_capacity)
            return make_status(TESSA_ERR_UNSUPPORTED, 0, "%llu leaf work items exceed the %llu of the fixed scratch",
                               (unsigned long long)items, (unsigned long long)sc.item_list_capacity);
    } else {
        DeviceWorkspace *ws = nullptr;
        st = get_workspace(rows_bound, &ws, items);
        if (st.code) return st;
        sc = LeafScratch{ws->queue_counts,
                         ws->fallback,
                         ws->fallback_capacity,
                         ws->chain_rows,
                         ws->chain_capacity,
                         ws->chain_pool,
                         ws->pool_capacity,
                         ws->survivor_log,
                         ws->log_entries / ((uint64_t)kLeafFilterThreads * kLeafLogCapacity),
                         ws->row_meta,
                         ws->item_list,
                         ws->item_list_capacity};
    }
    auto clamp32 = [](uint64_t v) { return (uint32_t)(v < 0xffffffffull ? v : 0xffffffffull); };
    p.fallback = sc.fallback;
    p.fallback_count = sc.queue_counts;
    p.fallback_capacity = clamp32(sc.fallback_capacity);
    p.chain_rows = sc.chain_rows;
    p.chain_count = sc.queue_counts + 1;
    p.chain_capacity = clamp32(leaf_chain_rows_usable(sc.chain_capacity, sc.pool_capacity));
    p.chain_pool = sc.chain_pool;
    p.chain_pool_used = sc.queue_counts + 2;
    p.item_tickets = sc.queue_counts + 4;
    p.chain_pool_capacity = clamp32(sc.pool_capacity);
    p.survivor_log = sc.log;
    p.log_capacity = kLeafLogCapacity;
    p.row_meta = sc.row_meta;
    p.blocks_per_leaf = bpl;
    p.item_list = sc.item_list;
    p.item_total = sc.queue_counts + 13;
    const uint64_t batch_cap = sc.log_items < kLeafMaxBatchItems ? sc.log_items : kLeafMaxBatchItems;
    if (batch_cap == 0) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf workspace holds no survivor log");
    // as few batches as the logs allow, of equal size (no short last batch)
    const uint64_t nbatch = (items + batch_cap - 1) / batch_cap;
    const uint64_t batch = (items + nbatch - 1) / nbatch;
    if (ev) {
        st = ensure_events(ev, 3 * nbatch + 2);
        if (st.code) return st;
    }
    // Zero the queue counters with a kernel (capture-safe, unlike a memset node).
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s, sc.queue_counts, 16u, 0u);
    // the work-item list; batches past its length find no items and return
    hipLaunchKernelGGL(leaf_item_list_kernel, dim3((lb->leaf_count + 255u) / 256u), dim3(256), 0, s,
                       lb->member_counts, lb->leaf_count, bpl, sc.item_list, sc.queue_counts + 13);
    for (uint64_t b = 0; b < nbatch; ++b) {
        p.item_begin = (uint32_t)(b * batch);
        p.item_count = (uint32_t)(items - b * batch < batch ? items - b * batch : batch);
        if (ev) TESSA_HIP_TRY(hipEventRecord(ev->e[3 * b], s));
        if (launch_leaf_mfma(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "MFMA leaf kernel launch failed");
        if (ev) TESSA_HIP_TRY(hipEventRecord(ev->e[3 * b + 1], s));
        if (launch_leaf_select(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "leaf select kernel launch failed");
        if (ev) TESSA_HIP_TRY(hipEventRecord(ev->e[3 * b + 2], s));
    }
    if (launch_leaf_chain(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "leaf chain kernel launch failed");
    if (ev) TESSA_HIP_TRY(hipEventRecord(ev->e[3 * nbatch], s));
    if (launch_leaf_exact_fallback(p, s) != 0)
        return make_status(TESSA_ERR_HIP, 0, "leaf fallback kernel launch failed");
    if (ev) TESSA_HIP_TRY(hipEventRecord(ev->e[3 * nbatch + 1], s));
    if (batches_out) *batches_out = nbatch;
    return ok_status();
}

}  // namespace

extern "C" {

tessa_status tessa_leaf_topk(const tessa_sq8_view *sq8, const tessa_leaf_batch *lb, uint32_t *out_ids,
                             float *out_dists, uint64_t *counters, void *stream) {
    if (!lb) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf batch has a null pointer");
    return leaf_topk_impl(sq8, lb, (uint64_t)lb->leaf_count * lb->max_leaf_rows, out_ids, out_dists, counters,
                          stream, nullptr);
}

tessa_status tessa_leaf_topk_profiled(const tessa_sq8_view *sq8, const tessa_leaf_batch *lb, uint32_t *out_ids,
                                      float *out_dists, uint64_t *counters, void *stream, float *phase_ms) {
    if (!lb) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf batch has a null pointer");
    if (!phase_ms) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "phase_ms is null");
    for (int i = 0; i < 5; ++i) phase_ms[i] = 0.0f;
    PhaseEvents *ev = nullptr;
    tessa_status st = phase_events(&ev);
    if (st.code) return st;
    uint64_t nb = 0;
    st = leaf_topk_impl(sq8, lb, (uint64_t)lb->leaf_count * lb->max_leaf_rows, out_ids, out_dists, counters, stream,
                        ev, &nb);
    if (st.code || nb == 0) return st;  // exact executor or no leaves: no MFMA phases
    TESSA_HIP_TRY(hipEventSynchronize(ev->e[3 * nb + 1]));
    auto span = [&](size_t a, size_t b) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ev->e[a], ev->e[b]);
        return ms;
    };
    for (uint64_t b = 0; b < nb; ++b) {
        phase_ms[0] += span(3 * b, 3 * b + 1);
        phase_ms[1] += span(3 * b + 1, 3 * b + 2);
    }
    phase_ms[2] = span(3 * nb - 1, 3 * nb);
    phase_ms[3] = span(3 * nb, 3 * nb + 1);
    phase_ms[4] = (float)nb;
    return ok_status();
}

// ---- leaf top-k without allocation -------------------------------------------
// All scratch of the MFMA leaf path in one static device array per GPU:
// queue counters, re-run queue, chain queue and pool for up to
// kNoAllocMaxRows member rows, and survivor logs for kNoAllocLogItems work
// items per filter/select batch.
}  // extern "C"
namespace {
constexpr uint64_t kNoAllocMaxRows = 65536;
constexpr uint64_t kNoAllocLogItems = 32;
constexpr uint64_t kNoAllocChainRows = kNoAllocMaxRows / 2 + 1;
constexpr size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }
constexpr size_t kNaOffFallback = 256;
constexpr size_t kNaOffChainRows = kNaOffFallback + a256(kNoAllocMaxRows * 2 * sizeof(uint32_t));
constexpr size_t kNaOffChainPool = kNaOffChainRows + a256(kNoAllocChainRows * sizeof(uint4));
constexpr uint64_t kNoAllocPoolEntries = (kNoAllocChainRows + 63) / 64 * 64 * kLeafChainSetEntries;  // whole groups of 64 x 40
constexpr size_t kNaOffRowMeta = kNaOffChainPool + a256(kNoAllocPoolEntries * sizeof(uint4));
constexpr size_t kNaOffLog = kNaOffRowMeta + a256(kNoAllocLogItems * kLeafBlockRows * sizeof(uint4));
// work items: leaf_count * blocks_per_leaf <= rows / kLeafBlockRows + leaf_count
constexpr uint64_t kNoAllocListItems = kNoAllocMaxRows / kLeafBlockRows + kNoAllocMaxRows;
constexpr size_t kNaOffItems = kNaOffLog + a256(kNoAllocLogItems * kLeafLogBytesPerItem);
constexpr size_t kNoAllocBytes = kNaOffItems + a256(kNoAllocListItems * sizeof(uint2));

__device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_ptr[kMaxDevices] = {};

// The device address of this GPU's `scratch` (the host-side name is only a
// stand-in), looked up once per device with that device current.
tessa_status scratch_for_device(unsigned char **out) {
    int dev = 0;
    TESSA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "device %d beyond the no-allocation path's %d devices", dev,
                           kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        TESSA_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        g_scratch_ptr[dev] = static_cast<unsigned char *>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return ok_status();
}
}  // namespace
extern "C" {

tessa_status tessa_leaf_topk_noalloc(const tessa_sq8_view *sq8, const tessa_leaf_batch *lb, uint32_t *out_ids,
                                     float *out_dists, uint64_t *counters, void *stream) {
    if (!lb) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf batch has a null pointer");
    const uint64_t rows = (uint64_t)lb->leaf_count * lb->max_leaf_rows;
    // the exact executor uses no scratch: any batch size
    if (lb->executor == TESSA_EXEC_EXACT)
        return leaf_topk_impl(sq8, lb, rows, out_ids, out_dists, counters, stream, nullptr);
    if (rows > kNoAllocMaxRows)
        return make_status(TESSA_ERR_UNSUPPORTED, 0,
                           "leaf batch of %u leaves x %u rows exceeds the no-allocation limit of %llu member rows",
                           lb->leaf_count, lb->max_leaf_rows, (unsigned long long)kNoAllocMaxRows);
    unsigned char *base = nullptr;
    tessa_status st = scratch_for_device(&base);
    if (st.code) return st;
    const LeafScratch sc{reinterpret_cast<uint32_t *>(base),
                         reinterpret_cast<uint32_t *>(base + kNaOffFallback),
                         kNoAllocMaxRows,
                         reinterpret_cast<uint4 *>(base + kNaOffChainRows),
                         kNoAllocChainRows,
                         reinterpret_cast<uint4 *>(base + kNaOffChainPool),
                         kNoAllocPoolEntries,
                         reinterpret_cast<uint2 *>(base + kNaOffLog),
                         kNoAllocLogItems,
                         reinterpret_cast<uint4 *>(base + kNaOffRowMeta),
                         reinterpret_cast<uint2 *>(base + kNaOffItems),
                         kNoAllocListItems};
    return leaf_topk_impl(sq8, lb, rows, out_ids, out_dists, counters, stream, nullptr, nullptr, &sc);
}

tessa_status tessa_assign_replay(const tessa_sq8_view *sq8, const tessa_assign_batch *tb, uint32_t *out_ids,
                                 float *out_dists, uint64_t *counters, void *stream) {
    tessa_status st = check_view(sq8);
    if (st.code) return st;
    if (!tb || !tb->members || !tb->leaders || !tb->member_offsets || !tb->member_counts || !tb->leader_offsets ||
        !tb->leader_counts || !tb->r_h || !tb->output_offsets || !out_ids || !out_dists)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "assignment batch has a null pointer");
    if (tb->task_count == 0 || tb->max_members == 0) return ok_status();
    if (sq8->padded_dim > 1024)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "assignment path needs padded_dim <= 1024 (got %u)",
                           sq8->padded_dim);
    AssignParams p{};
    p.codes = sq8->codes;
    p.scales = sq8->scales;
    p.norms = sq8->norms;
    p.gids = sq8->global_ids;
    p.rows = sq8->rows;
    p.padded_dim = sq8->padded_dim;
    p.members = tb->members;
    p.leaders = tb->leaders;
    p.member_offsets = tb->member_offsets;
    p.member_counts = tb->member_counts;
    p.leader_offsets = tb->leader_offsets;
    p.leader_counts = tb->leader_counts;
    p.r_h = tb->r_h;
    p.output_offsets = tb->output_offsets;
    p.task_count = tb->task_count;
    p.max_members = tb->max_members;
    p.out_ids = out_ids;
    p.out_dists = out_dists;
    p.counters = counters;
    if (launch_assign_replay(p, reinterpret_cast<hipStream_t>(stream)) != 0)
        return make_status(TESSA_ERR_HIP, 0, "assignment kernel launch failed");
    return ok_status();
}

tessa_status tessa_sq8_quantize(const float *x, uint64_t rows, uint32_t dim, uint32_t padded_dim, uint32_t bits,
                                int8_t *codes, float *scales, float *norms, uint64_t *bad_row_out, void *stream) {
    if (!x || !codes || !scales || !norms)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "quantize has a null pointer");
    if (bits < 4 || bits > 8)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "SQ-int8 bits=%u outside [4, 8]", bits);
    if (dim == 0 || padded_dim < dim || padded_dim % 16 != 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "quantize dim=%u padded_dim=%u invalid", dim, padded_dim);
    if (launch_sq8_quantize(x, rows, dim, padded_dim, bits, codes, scales, norms, bad_row_out,
                            reinterpret_cast<hipStream_t>(stream)) != 0)
        return make_status(TESSA_ERR_HIP, 0, "quantize kernel launch failed");
    return ok_status();
}

}  // extern "C"

// ---- sessions ------------------------------------------------------------

struct tessa_session {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    int8_t *codes = nullptr;
    float *scales = nullptr, *norms = nullptr;
    uint32_t *gids = nullptr;
    uint64_t rows = 0;
    uint32_t dim = 0, padded_dim = 0;
    // growable scratch for layouts / outputs
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    uint64_t *counters = nullptr;
    // subtree partition workspace (one device block carved into arrays)
    void *part = nullptr;
    size_t part_bytes = 0;
    uint64_t *part_counters = nullptr;  // TESSA_SUBTREE_COUNTER_WORDS
    tessa::LevelHeader *part_hdr = nullptr;
    tessa::LevelHeader *part_hdr_host = nullptr;  // pinned
    hipEvent_t ev2 = nullptr;
    // Held by every call (and by the async worker for a whole job) that uses
    // the stream, the uploaded rows or the workspaces above.
    std::mutex exec_mu;
    // ---- asynchronous submissions (tessa_session_submit_subtree) ----
    struct AsyncSlot {
        int state = 0;  // 0 free, 1 queued or running, 2 result ready
        uint64_t seq = 0;
        bool upload = false;
        tessa_sq8_view host{};
        tessa_subtree_request req{};
        std::vector<uint32_t> roots;
        tessa_status status{};
        // results, in pinned host memory grown to the largest result seen
        uint32_t *rows_h = nullptr;
        uint64_t *starts_h = nullptr, *sizes_h = nullptr;
        uint32_t *ids_h = nullptr;
        float *dists_h = nullptr;
        uint64_t rows_cap = 0, starts_cap = 0, sizes_cap = 0, ids_cap = 0, dists_cap = 0;
        uint64_t counters[TESSA_SUBTREE_COUNTER_WORDS] = {};
        uint64_t leaf_counters[TESSA_COUNTER_WORDS] = {};
        uint64_t leaf_count = 0, leaf_rows = 0;
        uint32_t k = 0, levels = 0;
        float partition_ms = 0.0f, leaf_ms = 0.0f;
        // device outputs of this slot's job: the next job computes into the
        // other slot's while this one's D2H runs on the copy stream
        uint32_t *rows_d = nullptr;
        uint64_t *starts_d = nullptr, *sizes_d = nullptr;
        uint32_t *ids_d = nullptr;
        float *dists_d = nullptr;
        uint64_t rows_dcap = 0, starts_dcap = 0, sizes_dcap = 0, ids_dcap = 0, dists_dcap = 0;
        hipEvent_t computed = nullptr, copied = nullptr;
        bool copy_pending = false;
    };
    static constexpr int kAsyncSlots = 2;
    AsyncSlot slots[kAsyncSlots];
    std::mutex q_mu;
    std::condition_variable q_cv;
    std::deque<int> queue;
    std::thread worker;
    bool worker_started = false;
    bool stop = false;
    uint64_t next_seq = 1;
    // side stream for the results' D2H copies (default priority)
    hipStream_t copy_stream = nullptr;
    // assignment tasks of the last run's COUNT passes, when capture is on
    uint32_t capture_min_members = 0;  // 0: off
    tessa::PartCapture capture;        // rows[] hold global ids once the run has finished
    uint32_t capture_padded_dim = 0;
};

namespace {

void stop_async(tessa_session *s);  // asynchronous submissions, below

void free_sq8(tessa_session *s) {
    if (s->codes) (void)hipFree(s->codes);
    if (s->scales) (void)hipFree(s->scales);
    if (s->norms) (void)hipFree(s->norms);
    if (s->gids) (void)hipFree(s->gids);
    s->codes = nullptr;
    s->scales = s->norms = nullptr;
    s->gids = nullptr;
    s->rows = 0;
}

tessa_status ensure_scratch(tessa_session *s, size_t bytes) {
    if (s->scratch_bytes >= bytes) return ok_status();
    if (s->scratch) {
        TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
        TESSA_HIP_TRY(hipFree(s->scratch));
        s->scratch = nullptr;
        s->scratch_bytes = 0;
    }
    if (hipMalloc(&s->scratch, bytes) != hipSuccess)
        return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                           "session scratch of %zu bytes failed overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                           bytes, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
    s->scratch_bytes = bytes;
    return ok_status();
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

tessa_status finish_with_counters(tessa_session *s, uint64_t *host_counters, const char *what) {
    uint64_t c[TESSA_COUNTER_WORDS];
    TESSA_HIP_TRY(hipMemcpyAsync(c, s->counters, sizeof(c), hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    if (host_counters) std::memcpy(host_counters, c, sizeof(c));
    if (c[TESSA_C_OVERFLOW_FLAGS] != 0) {
        char labels[256];
        tessa_overflow_labels(c[TESSA_C_OVERFLOW_FLAGS], labels, sizeof(labels));
        return make_status(TESSA_ERR_OVERFLOW, c[TESSA_C_OVERFLOW_FLAGS],
                           "HIP %s overflow: resident_rows=%llu overflow_flags=0x%llx overflow_labels=%s", what,
                           (unsigned long long)s->rows, (unsigned long long)c[TESSA_C_OVERFLOW_FLAGS], labels);
    }
    return ok_status();
}

}  // namespace

extern "C" {

tessa_status tessa_session_create(const tessa_config *cfg, tessa_session **out) {
    if (!cfg || !out) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session config/output is null");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return make_status(TESSA_ERR_NO_DEVICE, 0, "no HIP device visible");
    if (cfg->device < 0 || cfg->device >= count)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "device %d outside [0, %d)", cfg->device, count);
    tessa_session *s = new (std::nothrow) tessa_session();
    if (!s) return make_status(TESSA_ERR_OUT_OF_MEMORY, 0, "session allocation failed");
    s->device = cfg->device;
    hipError_t e = hipSetDevice(s->device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&s->ev0);
    if (e == hipSuccess) e = hipEventCreate(&s->ev1);
    if (e == hipSuccess) e = hipEventCreate(&s->ev2);
    if (e == hipSuccess) e = hipMalloc(&s->counters, TESSA_COUNTER_WORDS * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc(&s->part_counters, TESSA_SUBTREE_COUNTER_WORDS * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc(&s->part_hdr, sizeof(tessa::LevelHeader));
    if (e == hipSuccess) e = hipHostMalloc(&s->part_hdr_host, sizeof(tessa::LevelHeader), hipHostMallocDefault);
    if (e != hipSuccess) {
        tessa_session_destroy(s);
        return make_status(TESSA_ERR_HIP, 0, "session setup failed: %s", hipGetErrorString(e));
    }
    *out = s;
    return ok_status();
}

tessa_status tessa_session_destroy(tessa_session *s) {
    if (!s) return ok_status();
    (void)hipSetDevice(s->device);
    stop_async(s);  // finishes the queued jobs, joins the worker, frees the result slots
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    free_sq8(s);
    if (s->scratch) (void)hipFree(s->scratch);
    if (s->counters) (void)hipFree(s->counters);
    if (s->part) (void)hipFree(s->part);
    if (s->part_counters) (void)hipFree(s->part_counters);
    if (s->part_hdr) (void)hipFree(s->part_hdr);
    if (s->part_hdr_host) (void)hipHostFree(s->part_hdr_host);
    if (s->ev2) (void)hipEventDestroy(s->ev2);
    if (s->ev0) (void)hipEventDestroy(s->ev0);
    if (s->ev1) (void)hipEventDestroy(s->ev1);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return ok_status();
}

static tessa_status tessa_session_upload_sq8_locked(tessa_session *s, const tessa_sq8_view *host) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    tessa_status st = check_view(host);
    if (st.code) return st;
    TESSA_HIP_TRY(hipSetDevice(s->device));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    free_sq8(s);
    // captured passes name rows of the set being replaced
    s->capture.tasks.clear();
    s->capture.rows.clear();
    const uint64_t rows = host->rows;
    if (hipMalloc(&s->codes, rows * host->padded_dim) != hipSuccess ||
        hipMalloc(&s->scales, rows * 4) != hipSuccess || hipMalloc(&s->norms, rows * 4) != hipSuccess ||
        hipMalloc(&s->gids, rows * 4) != hipSuccess) {
        free_sq8(s);
        return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                           "SQ8 upload of %llu rows failed overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                           (unsigned long long)rows, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
    }
    TESSA_HIP_TRY(hipMemcpyAsync(s->codes, host->codes, rows * host->padded_dim, hipMemcpyDefault, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(s->scales, host->scales, rows * 4, hipMemcpyDefault, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(s->norms, host->norms, rows * 4, hipMemcpyDefault, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(s->gids, host->global_ids, rows * 4, hipMemcpyDefault, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    s->rows = rows;
    s->dim = host->dim;
    s->padded_dim = host->padded_dim;
    return ok_status();
}

tessa_status tessa_session_upload_sq8(tessa_session *s, const tessa_sq8_view *host) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    return tessa_session_upload_sq8_locked(s, host);
}

static tessa_status tessa_session_leaf_topk_locked(tessa_session *s, const uint32_t *members, const uint64_t *member_offsets,
                                     const uint32_t *member_counts, const uint64_t *output_offsets,
                                     uint32_t leaf_count, uint32_t k, uint32_t executor, uint32_t *out_ids,
                                     float *out_dists, uint64_t *counters, float *event_ms) {
    if (!s || !s->codes) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session has no SQ8 upload");
    if (!members || !member_offsets || !member_counts || !output_offsets || !out_ids || !out_dists)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf replay has a null pointer");
    if (leaf_count == 0) return ok_status();
    if (k == 0 || k > (uint32_t)kMaxK) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "k=%u outside [1,32]", k);
    uint64_t total_members = 0, total_out = 0;
    uint32_t max_rows = 0;
    for (uint32_t l = 0; l < leaf_count; ++l) {
        uint64_t end_m = member_offsets[l] + member_counts[l];
        uint64_t end_o = output_offsets[l] + (uint64_t)member_counts[l] * k;
        if (end_m > total_members) total_members = end_m;
        if (end_o > total_out) total_out = end_o;
        if (member_counts[l] > max_rows) max_rows = member_counts[l];
    }
    for (uint64_t i = 0; i < total_members; ++i)
        if (members[i] >= s->rows)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_INVALID_TOPK_ROW_ID,
                               "leaf member %llu = %u outside resident rows %llu overflow_flags=0x%llx "
                               "overflow_labels=INVALID_TOPK_ROW_ID",
                               (unsigned long long)i, members[i], (unsigned long long)s->rows,
                               (unsigned long long)TESSA_OVF_INVALID_TOPK_ROW_ID);
    TESSA_HIP_TRY(hipSetDevice(s->device));
    const size_t b_mem = align256(total_members * 4), b_off = align256(leaf_count * 8ull),
                 b_cnt = align256(leaf_count * 4ull), b_ids = align256(total_out * 4), b_d = align256(total_out * 4);
    tessa_status st = ensure_scratch(s, b_mem + 2 * b_off + b_cnt + b_ids + b_d);
    if (st.code) return st;
    char *base = static_cast<char *>(s->scratch);
    uint32_t *d_mem = reinterpret_cast<uint32_t *>(base);
    uint64_t *d_moff = reinterpret_cast<uint64_t *>(base + b_mem);
    uint64_t *d_ooff = reinterpret_cast<uint64_t *>(base + b_mem + b_off);
    uint32_t *d_cnt = reinterpret_cast<uint32_t *>(base + b_mem + 2 * b_off);
    uint32_t *d_ids = reinterpret_cast<uint32_t *>(base + b_mem + 2 * b_off + b_cnt);
    float *d_d = reinterpret_cast<float *>(base + b_mem + 2 * b_off + b_cnt + b_ids);
    TESSA_HIP_TRY(hipMemcpyAsync(d_mem, members, total_members * 4, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_moff, member_offsets, leaf_count * 8ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_ooff, output_offsets, leaf_count * 8ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_cnt, member_counts, leaf_count * 4ull, hipMemcpyHostToDevice, s->stream));
    hipLaunchKernelGGL(fill_u32_kernel, dim3((TESSA_COUNTER_WORDS * 2 + 63) / 64), dim3(64), 0, s->stream,
                       reinterpret_cast<uint32_t *>(s->counters), (uint32_t)(TESSA_COUNTER_WORDS * 2), 0u);
    tessa_sq8_view view{s->codes, s->scales, s->norms, s->gids, s->rows, s->dim, s->padded_dim};
    tessa_leaf_batch lb{d_mem, d_moff, d_cnt, d_ooff, leaf_count, max_rows, k, executor, 0u, 0u};
    TESSA_HIP_TRY(hipEventRecord(s->ev0, s->stream));
    st = tessa_leaf_topk(&view, &lb, d_ids, d_d, s->counters, s->stream);
    if (st.code) return st;
    TESSA_HIP_TRY(hipEventRecord(s->ev1, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(out_ids, d_ids, total_out * 4, hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(out_dists, d_d, total_out * 4, hipMemcpyDeviceToHost, s->stream));
    st = finish_with_counters(s, counters, "leaf top-k");
    if (event_ms) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, s->ev0, s->ev1);
        *event_ms = ms;
    }
    return st;
}

tessa_status tessa_session_leaf_topk(tessa_session *s, const uint32_t *members, const uint64_t *member_offsets,
                                     const uint32_t *member_counts, const uint64_t *output_offsets,
                                     uint32_t leaf_count, uint32_t k, uint32_t executor, uint32_t *out_ids,
                                     float *out_dists, uint64_t *counters, float *event_ms) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    return tessa_session_leaf_topk_locked(s, members, member_offsets, member_counts, output_offsets, leaf_count, k,
                                          executor, out_ids, out_dists, counters, event_ms);
}

static tessa_status tessa_session_assign_replay_locked(tessa_session *s, const uint32_t *members, const uint32_t *leaders,
                                         const uint32_t *member_offsets, const uint32_t *member_counts,
                                         const uint32_t *leader_offsets, const uint32_t *leader_counts,
                                         const uint32_t *r_h, const uint64_t *output_offsets, uint32_t task_count,
                                         uint32_t *out_ids, float *out_dists, uint64_t *counters, float *event_ms) {
    if (!s || !s->codes) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session has no SQ8 upload");
    if (!members || !leaders || !member_offsets || !member_counts || !leader_offsets || !leader_counts || !r_h ||
        !output_offsets || !out_ids || !out_dists)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "assignment replay has a null pointer");
    if (task_count == 0) return ok_status();
    uint64_t tm = 0, tl = 0, to = 0;
    uint32_t max_members = 0;
    for (uint32_t t = 0; t < task_count; ++t) {
        if (r_h[t] == 0 || r_h[t] > 4 || leader_counts[t] < r_h[t] || leader_counts[t] > 128)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                               "assignment task %u has invalid r_h=%u for %u leaders (leaders <= 128)", t, r_h[t],
                               leader_counts[t]);
        uint64_t em = (uint64_t)member_offsets[t] + member_counts[t];
        uint64_t el = (uint64_t)leader_offsets[t] + leader_counts[t];
        uint64_t eo = output_offsets[t] + (uint64_t)member_counts[t] * r_h[t];
        tm = em > tm ? em : tm;
        tl = el > tl ? el : tl;
        to = eo > to ? eo : to;
        max_members = member_counts[t] > max_members ? member_counts[t] : max_members;
    }
    for (uint64_t i = 0; i < tm; ++i)
        if (members[i] >= s->rows)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_INVALID_ASSIGN_POINT_ID,
                               "assignment member %llu outside resident rows overflow_flags=0x%llx "
                               "overflow_labels=INVALID_ASSIGN_POINT_ID",
                               (unsigned long long)i, (unsigned long long)TESSA_OVF_INVALID_ASSIGN_POINT_ID);
    for (uint64_t i = 0; i < tl; ++i)
        if (leaders[i] >= s->rows)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_INVALID_ASSIGN_LEADER_ID,
                               "assignment leader %llu outside resident rows overflow_flags=0x%llx "
                               "overflow_labels=INVALID_ASSIGN_LEADER_ID",
                               (unsigned long long)i, (unsigned long long)TESSA_OVF_INVALID_ASSIGN_LEADER_ID);
    TESSA_HIP_TRY(hipSetDevice(s->device));
    const size_t bm = align256(tm * 4), bl = align256(tl * 4), bt4 = align256(task_count * 4ull),
                 bt8 = align256(task_count * 8ull), bo = align256(to * 4);
    tessa_status st = ensure_scratch(s, bm + bl + 5 * bt4 + bt8 + 2 * bo);
    if (st.code) return st;
    char *p = static_cast<char *>(s->scratch);
    uint32_t *d_m = reinterpret_cast<uint32_t *>(p); p += bm;
    uint32_t *d_l = reinterpret_cast<uint32_t *>(p); p += bl;
    uint32_t *d_mo = reinterpret_cast<uint32_t *>(p); p += bt4;
    uint32_t *d_mc = reinterpret_cast<uint32_t *>(p); p += bt4;
    uint32_t *d_lo = reinterpret_cast<uint32_t *>(p); p += bt4;
    uint32_t *d_lc = reinterpret_cast<uint32_t *>(p); p += bt4;
    uint32_t *d_rh = reinterpret_cast<uint32_t *>(p); p += bt4;
    uint64_t *d_oo = reinterpret_cast<uint64_t *>(p); p += bt8;
    uint32_t *d_ids = reinterpret_cast<uint32_t *>(p); p += bo;
    float *d_d = reinterpret_cast<float *>(p);
    TESSA_HIP_TRY(hipMemcpyAsync(d_m, members, tm * 4, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_l, leaders, tl * 4, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_mo, member_offsets, task_count * 4ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_mc, member_counts, task_count * 4ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_lo, leader_offsets, task_count * 4ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_lc, leader_counts, task_count * 4ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_rh, r_h, task_count * 4ull, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_oo, output_offsets, task_count * 8ull, hipMemcpyHostToDevice, s->stream));
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s->stream, reinterpret_cast<uint32_t *>(s->counters),
                       (uint32_t)(TESSA_COUNTER_WORDS * 2), 0u);
    tessa_sq8_view view{s->codes, s->scales, s->norms, s->gids, s->rows, s->dim, s->padded_dim};
    tessa_assign_batch tb{d_m, d_l, d_mo, d_mc, d_lo, d_lc, d_rh, d_oo, task_count, max_members};
    TESSA_HIP_TRY(hipEventRecord(s->ev0, s->stream));
    st = tessa_assign_replay(&view, &tb, d_ids, d_d, s->counters, s->stream);
    if (st.code) return st;
    TESSA_HIP_TRY(hipEventRecord(s->ev1, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(out_ids, d_ids, to * 4, hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(out_dists, d_d, to * 4, hipMemcpyDeviceToHost, s->stream));
    st = finish_with_counters(s, counters, "assignment replay");
    if (event_ms) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, s->ev0, s->ev1);
        *event_ms = ms;
    }
    return st;
}

tessa_status tessa_session_assign_replay(tessa_session *s, const uint32_t *members, const uint32_t *leaders,
                                         const uint32_t *member_offsets, const uint32_t *member_counts,
                                         const uint32_t *leader_offsets, const uint32_t *leader_counts,
                                         const uint32_t *r_h, const uint64_t *output_offsets, uint32_t task_count,
                                         uint32_t *out_ids, float *out_dists, uint64_t *counters, float *event_ms) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    return tessa_session_assign_replay_locked(s, members, leaders, member_offsets, member_counts, leader_offsets,
                                             leader_counts, r_h, output_offsets, task_count, out_ids, out_dists,
                                             counters, event_ms);
}

}  // extern "C"

// ---- resident subtree ------------------------------------------------------

namespace {

constexpr uint32_t kLeafMin = 64;          // GPU_PERSISTENT_LEAF_MIN compute_backend.rs:385
constexpr uint32_t kLeafTarget = 128;      // :387
constexpr uint32_t kLeafMaxFloor = 256;    // :389
constexpr uint32_t kSmallNodeLimit = 4096; // plan small_node_limit :1341
constexpr uint32_t kLeaderStride = 128;    // GPU_QUEUE_LEADER_STRIDE :371

uint64_t div_ceil(uint64_t a, uint64_t b) { return b ? (a + b - 1) / b : 0; }

// Byte layout of the partition workspace for the given capacities.
struct PartLayout {
    uint64_t arena_cap = 0, item_cap = 0, leaf_cap = 0;
    uint32_t node_cap = 0;
    size_t off_arena[2] = {0, 0}, off_nodes[2] = {0, 0}, off_leaders = 0, off_ccount = 0, off_cidx = 0,
           off_crel = 0, off_slots = 0, off_items = 0, off_item_node = 0, off_sizes32 = 0, off_outoff = 0, bytes = 0;
};

PartLayout part_layout(uint64_t rows, uint32_t famp, uint32_t leaf_max, uint64_t leaf_cap) {
    PartLayout L;
    partition_capacity(rows, famp, leaf_max, &L.arena_cap, &L.node_cap, &L.item_cap);
    L.leaf_cap = leaf_cap ? leaf_cap : 1;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += align256(bytes);
        return at;
    };
    const uint64_t nc = L.node_cap;
    L.off_arena[0] = take(L.arena_cap * 4);
    L.off_arena[1] = take(L.arena_cap * 4);
    L.off_nodes[0] = take(nc * sizeof(NodeDesc));
    L.off_nodes[1] = take(nc * sizeof(NodeDesc));
    L.off_leaders = take(nc * kPartMaxLeaders * 4);
    L.off_ccount = take(nc * kPartMaxLeaders * 4);
    L.off_cidx = take(nc * kPartMaxLeaders * 4);
    L.off_crel = take(nc * kPartMaxLeaders * 4);
    L.off_slots = take(L.arena_cap * 4);
    L.off_items = take(L.item_cap * kPartMaxLeaders * 4);
    L.off_item_node = take(L.item_cap * 4);
    L.off_sizes32 = take(L.leaf_cap * 4);
    L.off_outoff = take(L.leaf_cap * 8);
    L.bytes = o + kLeaderStride * 4;  // root leaders
    return L;
}

// Re-run / chain queues of the MFMA leaf path for `rows` leaf rows.
uint64_t leaf_workspace_bytes(uint64_t rows) {
    return rows * 8 + (rows / 2 + 1) * 16 + (rows / 2 + 1) * 40 * 8;
}

tessa_status subtree_overflow(const tessa_session *s, const uint64_t *c, float ms) {
    char labels[256];
    const uint64_t f = c[TESSA_P_OVERFLOW_FLAGS];
    tessa_overflow_labels(f, labels, sizeof(labels));
    // "CUDA persistent subtree overflow" is the token rbc_partition.rs:2982-2998
    // classifies as a capacity error; it is kept verbatim for that caller.
    return make_status(TESSA_ERR_OVERFLOW, f,
                       "CUDA persistent subtree overflow: resident_rows=%llu overflow_flags=0x%llx "
                       "overflow_labels=%s leaf_rows=%llu leaf_count=%llu partition_pops=%llu "
                       "assignment_passes=%llu max_active_points=%llu persistent_kernel_event_ms=%.3f "
                       "partition_level_rounds=%llu (HIP gfx950 persistent partition walk)",
                       (unsigned long long)s->rows, (unsigned long long)f, labels,
                       (unsigned long long)c[TESSA_P_OUTPUT_ROWS], (unsigned long long)c[TESSA_P_OUTPUT_LEAF_COUNT],
                       (unsigned long long)c[TESSA_P_PARTITION_POPS],
                       (unsigned long long)c[TESSA_P_ASSIGNMENT_PASSES], (unsigned long long)c[TESSA_P_MAX_ACTIVE],
                       ms, (unsigned long long)c[TESSA_P_PARTITION_LEVEL_ROUNDS]);
}

}  // namespace

extern "C" {

uint64_t tessa_subtree_root_seed(uint64_t random_seed, uint64_t depth, uint64_t point_count, uint64_t parent_points,
                                 uint64_t min_recurse_size) {
    auto rotl = [](uint64_t x, int r) { return (x << r) | (x >> (64 - r)); };
    return random_seed ^ (depth * 0x9e3779b97f4a7c15ull) ^ rotl(point_count, 17) ^ rotl(parent_points, 7) ^
           rotl(min_recurse_size, 29);
}

tessa_status tessa_plan_subtree(uint64_t resident_rows, uint32_t leaf_knn, uint32_t max_leaders_per_node,
                                uint32_t max_fanout, uint64_t budget_bytes, uint32_t c_max,
                                tessa_subtree_plan *plan) {
    if (!plan) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "plan output is null");
    tessa_subtree_plan p;
    std::memset(&p, 0, sizeof(p));
    const uint64_t r1 = resident_rows ? resident_rows : 1;
    const uint32_t persistent_fanout = max_fanout ? max_fanout : 1;
    const uint32_t famp = persistent_fanout < 4 ? persistent_fanout : 4;
    p.leaf_min = kLeafMin;
    p.leaf_target = kLeafTarget;
    p.leaf_max = (c_max ? c_max : 1) > kLeafMaxFloor ? (c_max ? c_max : 1) : kLeafMaxFloor;
    p.small_node_limit = kSmallNodeLimit;
    p.effective_root_fanout = famp;
    p.effective_deeper_fanout = 1;
    p.fanout_amplification = famp;
    p.large_child_slots = kLeaderStride;
    // compute_backend.rs:1351-1380
    p.max_queue_nodes = r1 * famp + div_ceil(r1, p.leaf_min);
    p.max_leaf_rows = resident_rows * famp;
    const uint64_t semantic_leaf_count = div_ceil(p.max_leaf_rows ? p.max_leaf_rows : 1, p.leaf_min) * 8;
    p.max_leaf_count = semantic_leaf_count ? semantic_leaf_count : 1;
    p.large_scratch_rows = r1 * famp;
    const uint32_t k = leaf_knn < 32 ? leaf_knn : 32;
    const PartLayout L = part_layout(resident_rows, famp, p.leaf_max, p.max_leaf_count);
    p.required_bytes = L.bytes + TESSA_SUBTREE_COUNTER_WORDS * 8 + p.max_leaf_rows * 4 + p.max_leaf_count * 16 +
                       p.max_leaf_rows * (uint64_t)k * 8 + leaf_workspace_bytes(p.max_leaf_rows);
    p.budget_bytes = budget_bytes ? budget_bytes : UINT64_MAX;
    if (resident_rows != 0 && budget_bytes != 0 && p.required_bytes > budget_bytes) {
        p.fallback_reason_flags |= TESSA_PLAN_FALLBACK_WORKSPACE;
        p.overflow_flags |= TESSA_OVF_WORKSPACE_BUDGET;
    }
    if (leaf_knn > 32) {
        p.fallback_reason_flags |= TESSA_PLAN_FALLBACK_UNSUPPORTED_K;
        p.overflow_flags |= TESSA_OVF_LEAF_DESC;
    }
    if (persistent_fanout > 4) {
        p.fallback_reason_flags |= TESSA_PLAN_FALLBACK_UNSUPPORTED_FANOUT;
        p.overflow_flags |= TESSA_OVF_FANOUT_OVER_32;
    }
    if (max_leaders_per_node > kLeaderStride) {
        p.fallback_reason_flags |= TESSA_PLAN_FALLBACK_UNSUPPORTED_LEADERS;
        p.overflow_flags |= TESSA_OVF_LEADER;
    }
    p.supported = p.fallback_reason_flags == 0;
    *plan = p;
    return ok_status();
}

static tessa_status tessa_session_run_subtree_locked(tessa_session *s, const tessa_subtree_request *rq,
                                       tessa_subtree_output *out) {
    if (!s || !s->codes) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session has no SQ8 upload");
    if (!rq || !out) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "subtree request/output is null");
    const uint64_t rows = s->rows;
    out->leaf_count = out->leaf_rows = 0;
    out->k = 0;
    out->levels = 0;
    out->partition_ms = out->leaf_ms = 0.0f;
    const bool partition_only = rq->partition_only != 0;
    if (!partition_only && (rq->leaf_knn == 0 || rq->leaf_knn > (uint32_t)kMaxK))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_LEAF_DESC,
                           "CUDA persistent strict error: unsupported subtree leaf_knn=%u (1..32) "
                           "fallback_reason_flags=0x%x",
                           rq->leaf_knn, TESSA_PLAN_FALLBACK_UNSUPPORTED_K);
    if (rq->fanout_second == 0 || rq->fanout_second > 4)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_FANOUT_OVER_32,
                           "CUDA persistent strict error: unsupported subtree fanout_second=%u (1..4) "
                           "fallback_reason_flags=0x%x",
                           rq->fanout_second, TESSA_PLAN_FALLBACK_UNSUPPORTED_FANOUT);
    if (rq->max_leaders == 0 || rq->leaf_min == 0 || rq->leaf_max == 0 || rq->small_node_limit == 0 ||
        rq->small_node_limit > kSmallNodeLimit)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "subtree request needs max_leaders, leaf_min, leaf_max >= 1 and "
                           "small_node_limit in [1, 4096]");
    if (!partition_only && rq->executor == TESSA_EXEC_MFMA && rq->leaf_max > 4096)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "MFMA leaf path needs leaf_max <= 4096 (got %u)", rq->leaf_max);
    if (s->padded_dim > 1024)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "subtree path needs padded_dim <= 1024 (got %u)", s->padded_dim);
    const uint32_t leader_cap = rq->max_leaders < kLeaderStride ? rq->max_leaders : kLeaderStride;
    if (rq->root_leader_count > leader_cap)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "CUDA persistent root leader override has %u leaders, exceeding per-node limit %u",
                           rq->root_leader_count, leader_cap);
    if (rq->root_leader_count > 0 && !rq->root_leaders)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "root leader count without root leader ids");
    for (uint32_t i = 0; i < rq->root_leader_count; ++i)
        if (rq->root_leaders[i] >= rows)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                               "CUDA persistent root leader override row %u exceeds resident rows %llu",
                               rq->root_leaders[i], (unsigned long long)rows);
    const uint32_t famp = rq->fanout_second;
    if (rows * famp > 0xffffffffull)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "resident rows x fanout must stay below 2^32");
    if (!out->leaf_row_ids || !out->leaf_starts || !out->leaf_sizes ||
        (!partition_only && (!out->topk_ids || !out->topk_dists)))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "subtree output has a null device pointer");
    if (rq->max_leaf_count == 0 || rq->max_leaf_rows == 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "subtree output capacities must be positive");
    TESSA_HIP_TRY(hipSetDevice(s->device));

    const PartLayout L = part_layout(rows, famp, rq->leaf_max, rq->max_leaf_count);
    if (s->part_bytes < L.bytes) {
        TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
        if (s->part) (void)hipFree(s->part);
        s->part = nullptr;
        s->part_bytes = 0;
        if (hipMalloc(&s->part, L.bytes) != hipSuccess)
            return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                               "Failed to allocate CUDA GPU persistent subtree workspace (HIP, %zu bytes) "
                               "overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                               L.bytes, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
        s->part_bytes = L.bytes;
    }
    char *base = static_cast<char *>(s->part);
    PartArgs a{};
    a.codes = s->codes;
    a.scales = s->scales;
    a.norms = s->norms;
    a.rows = (uint32_t)rows;
    a.padded_dim = s->padded_dim;
    uint32_t *d_root = reinterpret_cast<uint32_t *>(base + L.bytes - kLeaderStride * 4);
    if (rq->root_leader_count)
        TESSA_HIP_TRY(hipMemcpyAsync(d_root, rq->root_leaders, rq->root_leader_count * 4ull,
                                     hipMemcpyHostToDevice, s->stream));
    a.root_leaders = d_root;
    a.root_leader_count = rq->root_leader_count;
    a.root_depth = rq->root_depth;
    a.max_depth = rq->max_depth;
    a.max_leaders = rq->max_leaders;
    a.fanout_second = rq->fanout_second;
    a.leaf_min = rq->leaf_min;
    a.leaf_max = rq->leaf_max;
    a.small_node_limit = rq->small_node_limit;
    const uint32_t k = partition_only ? 0u
                                      : (uint32_t)(rq->leaf_knn < rows - 1 ? rq->leaf_knn : (rows ? rows - 1 : 0));
    a.k = k;
    a.psamp = rq->psamp_fraction;
    a.seed = rq->seed;
    a.large_scratch_rows = rows * famp;
    a.max_leaf_count = rq->max_leaf_count;
    a.max_leaf_rows = rq->max_leaf_rows;
    a.leaf_row_ids = out->leaf_row_ids;
    a.leaf_starts = out->leaf_starts;
    a.leaf_sizes = out->leaf_sizes;
    a.leaf_sizes32 = reinterpret_cast<uint32_t *>(base + L.off_sizes32);
    a.leaf_out_offsets = reinterpret_cast<uint64_t *>(base + L.off_outoff);
    a.counters = s->part_counters;
    a.hdr = s->part_hdr;
    for (int i = 0; i < 2; ++i) {
        a.arena[i] = reinterpret_cast<uint32_t *>(base + L.off_arena[i]);
        a.nodes[i] = reinterpret_cast<NodeDesc *>(base + L.off_nodes[i]);
    }
    a.leaders = reinterpret_cast<uint32_t *>(base + L.off_leaders);
    a.child_counts = reinterpret_cast<uint32_t *>(base + L.off_ccount);
    a.child_idx = reinterpret_cast<uint32_t *>(base + L.off_cidx);
    a.child_rel = reinterpret_cast<uint32_t *>(base + L.off_crel);
    a.slots = reinterpret_cast<uint32_t *>(base + L.off_slots);
    a.item_counts = reinterpret_cast<uint32_t *>(base + L.off_items);
    a.item_node = reinterpret_cast<uint32_t *>(base + L.off_item_node);
    a.arena_cap = L.arena_cap;
    a.item_cap = L.item_cap;
    a.node_cap = L.node_cap;

    TESSA_HIP_TRY(hipEventRecord(s->ev0, s->stream));
    PartResult pr{};
    s->capture.tasks.clear();
    s->capture.rows.clear();
    s->capture.min_members = s->capture_min_members;
    const int rc = run_partition(a, s->stream, s->part_hdr_host, &pr,
                                 s->capture_min_members ? &s->capture : nullptr);
    if (rc != 0)
        return partition_failure(rc, pr);
    if (s->capture_min_members && !s->capture.rows.empty()) {
        // Resident rows -> global ids now, while the resident set is the one
        // this run used (a later upload may replace it before the fetch).
        std::vector<uint32_t> gids(s->rows);
        TESSA_HIP_TRY(hipMemcpyAsync(gids.data(), s->gids, s->rows * 4ull, hipMemcpyDeviceToHost, s->stream));
        TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
        for (uint32_t &r : s->capture.rows) {
            if (r >= s->rows)
                return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "capture: row %u outside the resident set", r);
            r = gids[r];
        }
    }
    s->capture_padded_dim = s->padded_dim;
    TESSA_HIP_TRY(hipEventRecord(s->ev1, s->stream));
    uint64_t c[TESSA_SUBTREE_COUNTER_WORDS];
    TESSA_HIP_TRY(hipMemcpyAsync(c, s->part_counters, sizeof(c), hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    float part_ms = 0.0f;
    (void)hipEventElapsedTime(&part_ms, s->ev0, s->ev1);
    out->partition_ms = part_ms;
    out->levels = pr.levels;
    out->leaf_count = pr.leaf_count;
    out->leaf_rows = pr.leaf_rows;
    out->k = k;
    if (out->counters) std::memcpy(out->counters, c, sizeof(c));
    if (c[TESSA_P_OVERFLOW_FLAGS] != 0) return subtree_overflow(s, c, part_ms);
    if (partition_only || k == 0 || pr.leaf_count == 0) return ok_status();

    // Leaf top-k over the published leaves (the top-k CTAs' role,
    // compute_backend.rs:17113-17370).
    if (pr.leaf_count > 0xffffffffull)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "more than 2^32 leaves");
    const uint32_t max_rows = (uint32_t)c[TESSA_P_LEAF_SIZE_MAX];
    hipLaunchKernelGGL(fill_u32_kernel, dim3((TESSA_COUNTER_WORDS * 2 + 63) / 64), dim3(64), 0, s->stream,
                       reinterpret_cast<uint32_t *>(s->counters), (uint32_t)(TESSA_COUNTER_WORDS * 2), 0u);
    tessa_sq8_view view{s->codes, s->scales, s->norms, s->gids, s->rows, s->dim, s->padded_dim};
    tessa_leaf_batch lb{out->leaf_row_ids, out->leaf_starts, a.leaf_sizes32, a.leaf_out_offsets,
                        (uint32_t)pr.leaf_count, max_rows, k, rq->executor, 0u, 0u};
    tessa_status st = leaf_topk_impl(&view, &lb, pr.leaf_rows, out->topk_ids, out->topk_dists, s->counters,
                                     s->stream, nullptr);
    if (st.code) return st;
    TESSA_HIP_TRY(hipEventRecord(s->ev2, s->stream));
    uint64_t lc[TESSA_COUNTER_WORDS];
    TESSA_HIP_TRY(hipMemcpyAsync(lc, s->counters, sizeof(lc), hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    float leaf_ms = 0.0f;
    (void)hipEventElapsedTime(&leaf_ms, s->ev1, s->ev2);
    out->leaf_ms = leaf_ms;
    if (out->leaf_counters) std::memcpy(out->leaf_counters, lc, sizeof(lc));
    if (out->counters) out->counters[TESSA_P_LEAF_SQ8_WMMA_TILES] = lc[TESSA_C_LEAF_MFMA_TILES];
    if (lc[TESSA_C_OVERFLOW_FLAGS] != 0) {
        char labels[256];
        tessa_overflow_labels(lc[TESSA_C_OVERFLOW_FLAGS], labels, sizeof(labels));
        return make_status(TESSA_ERR_OVERFLOW, lc[TESSA_C_OVERFLOW_FLAGS],
                           "CUDA persistent subtree overflow: resident_rows=%llu overflow_flags=0x%llx "
                           "overflow_labels=%s (leaf top-k)",
                           (unsigned long long)rows, (unsigned long long)lc[TESSA_C_OVERFLOW_FLAGS], labels);
    }
    return ok_status();
}

tessa_status tessa_session_run_subtree(tessa_session *s, const tessa_subtree_request *rq, tessa_subtree_output *out) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    return tessa_session_run_subtree_locked(s, rq, out);
}

static tessa_status tessa_session_partition_roots_locked(tessa_session *s, const tessa_sq8_view *sq8,
                                                         const tessa_roots_request *rq, tessa_roots_output *out) {
    if (!sq8 || !rq || !out) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "partition roots: null argument");
    out->leaf_count = out->leaf_rows_total = 0;
    out->levels = 0;
    out->partition_ms = 0.0f;
    if (!sq8->codes || !sq8->scales || !sq8->norms || sq8->rows == 0 || sq8->rows > 0xffffffffull)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "partition roots: SQ8 view needs device codes, scales and "
                                                          "norms of 1..2^32-1 rows");
    if (sq8->padded_dim == 0 || sq8->padded_dim % 16 != 0 || sq8->padded_dim > 1024)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "partition roots: padded_dim %u (multiple of 16, <= 1024)",
                           sq8->padded_dim);
    if (!rq->rows || !rq->root_offsets || !rq->root_seeds || rq->root_count == 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "partition roots: rows, offsets and seeds of >= 1 root");
    if (rq->fanout_second == 0 || rq->fanout_second > 4)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_FANOUT_OVER_32,
                           "CUDA persistent strict error: unsupported subtree fanout_second=%u (1..4) "
                           "fallback_reason_flags=0x%x",
                           rq->fanout_second, TESSA_PLAN_FALLBACK_UNSUPPORTED_FANOUT);
    if (rq->max_leaders == 0 || rq->leaf_min == 0 || rq->leaf_max == 0 || rq->small_node_limit == 0 ||
        rq->small_node_limit > kSmallNodeLimit)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "partition roots needs max_leaders, leaf_min, leaf_max >= 1 and "
                           "small_node_limit in [1, 4096]");
    if (!out->leaf_rows || !out->leaf_starts || !out->leaf_sizes || rq->max_leaf_count == 0 || rq->max_leaf_rows == 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "partition roots: null output or zero capacity");
    if (rq->root_offsets[0] != 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "partition roots: root_offsets[0] must be 0");
    for (uint32_t i = 0; i < rq->root_count; ++i) {
        const uint64_t a = rq->root_offsets[i], b = rq->root_offsets[i + 1];
        if (b < a + 2)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "partition roots: root %u has %lld rows (>= 2 needed)", i,
                               (long long)(b - a));
        const uint64_t n = b - a;
        const bool large = n > rq->leaf_max ||
                           (rq->fanout_second > 1 && n * rq->fanout_second > (uint64_t)rq->small_node_limit);
        if (!large)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                               "partition roots: root %u of %llu rows is a small root (run it with "
                               "tessa_session_run_subtree)",
                               i, (unsigned long long)n);
    }
    const uint64_t rows = rq->root_offsets[rq->root_count];
    const uint32_t famp = rq->fanout_second;
    if (rows * famp > 0xffffffffull)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "partition roots: rows x fanout must stay below 2^32");
    TESSA_HIP_TRY(hipSetDevice(s->device));

    // workspace: the partition arrays, then the roots' offsets and seeds,
    // 64-bit leaf sizes and one check word
    const PartLayout L = part_layout(rows, famp, rq->leaf_max, rq->max_leaf_count);
    const size_t off_roff = align256(L.bytes), off_seed = off_roff + align256((rq->root_count + 1ull) * 8),
                 off_sz64 = off_seed + align256(rq->root_count * 8ull),
                 off_chk = off_sz64 + align256(rq->max_leaf_count * 8ull), need = off_chk + 256;
    if (s->part_bytes < need) {
        TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
        if (s->part) (void)hipFree(s->part);
        s->part = nullptr;
        s->part_bytes = 0;
        if (hipMalloc(&s->part, need) != hipSuccess)
            return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                               "Failed to allocate CUDA GPU persistent subtree workspace (HIP, %zu bytes) "
                               "overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                               need, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
        s->part_bytes = need;
    }
    char *base = static_cast<char *>(s->part);
    uint64_t *d_roff = reinterpret_cast<uint64_t *>(base + off_roff);
    uint64_t *d_seed = reinterpret_cast<uint64_t *>(base + off_seed);
    uint32_t *d_chk = reinterpret_cast<uint32_t *>(base + off_chk);
    TESSA_HIP_TRY(hipMemcpyAsync(d_roff, rq->root_offsets, (rq->root_count + 1ull) * 8, hipMemcpyHostToDevice,
                                 s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(d_seed, rq->root_seeds, rq->root_count * 8ull, hipMemcpyHostToDevice, s->stream));
    // every row id must be an SQ8 row (the kernels read codes through it)
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s->stream, d_chk, 1u, 0u);
    hipLaunchKernelGGL(max_u32_kernel, dim3(1024), dim3(256), 0, s->stream, rq->rows, rows, d_chk);
    uint32_t max_row = 0;
    TESSA_HIP_TRY(hipMemcpyAsync(&max_row, d_chk, 4, hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    if (max_row >= sq8->rows)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_INVALID_ASSIGN_POINT_ID,
                           "partition roots: row id %u outside the %llu SQ8 rows overflow_flags=0x%llx "
                           "overflow_labels=INVALID_ASSIGN_POINT_ID",
                           max_row, (unsigned long long)sq8->rows, (unsigned long long)TESSA_OVF_INVALID_ASSIGN_POINT_ID);

    PartArgs a{};
    a.codes = sq8->codes;
    a.scales = sq8->scales;
    a.norms = sq8->norms;
    a.row_map = rq->rows;
    a.rows = (uint32_t)rows;
    a.padded_dim = sq8->padded_dim;
    a.root_offsets = d_roff;
    a.root_seeds = d_seed;
    a.root_count = rq->root_count;
    a.root_leaders = nullptr;
    a.root_leader_count = 0;
    a.root_depth = rq->root_depth;
    a.max_depth = rq->max_depth;
    a.max_leaders = rq->max_leaders;
    a.fanout_second = rq->fanout_second;
    a.leaf_min = rq->leaf_min;
    a.leaf_max = rq->leaf_max;
    a.small_node_limit = rq->small_node_limit;
    a.k = 0;
    a.psamp = rq->psamp_fraction;
    a.seed = 0;
    a.large_scratch_rows = rows * famp;
    a.max_leaf_count = rq->max_leaf_count;
    a.max_leaf_rows = rq->max_leaf_rows;
    a.leaf_row_ids = out->leaf_rows;
    a.leaf_starts = out->leaf_starts;
    a.leaf_sizes = reinterpret_cast<uint64_t *>(base + off_sz64);
    a.leaf_sizes32 = out->leaf_sizes;
    a.leaf_out_offsets = reinterpret_cast<uint64_t *>(base + L.off_outoff);
    a.leaf_root = out->leaf_roots;
    a.leaf_depth = out->leaf_depths;
    a.counters = s->part_counters;
    a.hdr = s->part_hdr;
    for (int i = 0; i < 2; ++i) {
        a.arena[i] = reinterpret_cast<uint32_t *>(base + L.off_arena[i]);
        a.nodes[i] = reinterpret_cast<NodeDesc *>(base + L.off_nodes[i]);
    }
    a.leaders = reinterpret_cast<uint32_t *>(base + L.off_leaders);
    a.child_counts = reinterpret_cast<uint32_t *>(base + L.off_ccount);
    a.child_idx = reinterpret_cast<uint32_t *>(base + L.off_cidx);
    a.child_rel = reinterpret_cast<uint32_t *>(base + L.off_crel);
    a.slots = reinterpret_cast<uint32_t *>(base + L.off_slots);
    a.item_counts = reinterpret_cast<uint32_t *>(base + L.off_items);
    a.item_node = reinterpret_cast<uint32_t *>(base + L.off_item_node);
    a.arena_cap = L.arena_cap;
    a.item_cap = L.item_cap;
    a.node_cap = L.node_cap;

    TESSA_HIP_TRY(hipEventRecord(s->ev0, s->stream));
    PartResult pr{};
    const int rc = run_partition(a, s->stream, s->part_hdr_host, &pr, nullptr);
    if (rc != 0)
        return partition_failure(rc, pr);
    uint64_t c[TESSA_SUBTREE_COUNTER_WORDS];
    TESSA_HIP_TRY(hipMemcpyAsync(c, s->part_counters, sizeof(c), hipMemcpyDeviceToHost, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    if (out->counters) std::memcpy(out->counters, c, sizeof(c));
    out->levels = pr.levels;
    out->leaf_count = pr.leaf_count;
    out->leaf_rows_total = pr.leaf_rows;
    if (c[TESSA_P_OVERFLOW_FLAGS] != 0) {
        TESSA_HIP_TRY(hipEventRecord(s->ev1, s->stream));
        TESSA_HIP_TRY(hipEventSynchronize(s->ev1));
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, s->ev0, s->ev1);
        out->partition_ms = ms;
        return subtree_overflow(s, c, ms);
    }
    // leaf members: resident indices -> SQ8 row ids
    if (pr.leaf_rows)
        hipLaunchKernelGGL(map_rows_kernel, dim3((uint32_t)std::min<uint64_t>((pr.leaf_rows + 255) / 256, 8192)),
                           dim3(256), 0, s->stream, out->leaf_rows, pr.leaf_rows, rq->rows);
    TESSA_HIP_TRY(hipEventRecord(s->ev1, s->stream));
    TESSA_HIP_TRY(hipEventSynchronize(s->ev1));
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, s->ev0, s->ev1);
    out->partition_ms = ms;
    return ok_status();
}

tessa_status tessa_session_partition_roots(tessa_session *s, const tessa_sq8_view *sq8, const tessa_roots_request *rq,
                                           tessa_roots_output *out) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    return tessa_session_partition_roots_locked(s, sq8, rq, out);
}

}  // extern "C"

// ---- asynchronous subtree submissions --------------------------------------
//
// The reference's submit_owned_quantized_subtree_l2_compact_topk
// (compute_backend.rs:3807-3815) returns a Deferred result whose finish()
// waits for the device work and the D2H copy into a pinned host slot taken
// from a small ring (CudaDeferredPinnedQuantizedScatter, :31432-31497), so the
// caller's host-side scatter of one task overlaps the device work of the next.
// Here a session owns one worker thread and two pinned result slots: submit
// queues a job (upload of the task's SQ8 rows, partition, leaf top-k, D2H of
// the leaf layout and top-k into the slot) and returns its sequence number;
// wait blocks until that job is done and hands out the slot's host arrays;
// release returns the slot to the ring.

namespace {

template <typename T>
tessa_status grow_pinned(T **p, uint64_t *cap, uint64_t need) {
    if (*cap >= need) return ok_status();
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
    const uint64_t n = need < 1024 ? 1024 : need;
    if (hipHostMalloc((void **)p, n * sizeof(T), hipHostMallocDefault) != hipSuccess)
        return make_status(TESSA_ERR_OUT_OF_MEMORY, 0, "pinned host result slot of %llu entries failed",
                           (unsigned long long)n);
    *cap = n;
    return ok_status();
}

template <typename T>
tessa_status grow_device(T **p, uint64_t *cap, uint64_t need) {
    if (*cap >= need) return ok_status();
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    const uint64_t n = need < 1024 ? 1024 : need;
    if (hipMalloc((void **)p, n * sizeof(T)) != hipSuccess)
        return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                           "Failed to allocate CUDA GPU persistent subtree output (HIP, %llu entries) "
                           "overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                           (unsigned long long)n, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
    *cap = n;
    return ok_status();
}

// One queued job, run by the worker with exec_mu held.
tessa_status run_async_job(tessa_session *s, tessa_session::AsyncSlot &slot) {
    if (slot.upload) {
        tessa_status st = tessa_session_upload_sq8_locked(s, &slot.host);
        if (st.code) return st;
    }
    const tessa_subtree_request &rq = slot.req;
    const uint64_t k_cap = rq.partition_only ? 1 : (rq.leaf_knn ? rq.leaf_knn : 1);
    // this slot's previous copy finished before it was released (wait syncs it)
    tessa_status st = grow_device(&slot.rows_d, &slot.rows_dcap, rq.max_leaf_rows);
    if (!st.code) st = grow_device(&slot.starts_d, &slot.starts_dcap, rq.max_leaf_count);
    if (!st.code) st = grow_device(&slot.sizes_d, &slot.sizes_dcap, rq.max_leaf_count);
    if (!st.code) st = grow_device(&slot.ids_d, &slot.ids_dcap, rq.max_leaf_rows * k_cap);
    if (!st.code) st = grow_device(&slot.dists_d, &slot.dists_dcap, rq.max_leaf_rows * k_cap);
    if (st.code) return st;
    if (!s->copy_stream) TESSA_HIP_TRY(hipStreamCreateWithFlags(&s->copy_stream, hipStreamNonBlocking));
    if (!slot.computed) TESSA_HIP_TRY(hipEventCreateWithFlags(&slot.computed, hipEventDisableTiming));
    if (!slot.copied) TESSA_HIP_TRY(hipEventCreateWithFlags(&slot.copied, hipEventDisableTiming));
    tessa_subtree_request req = rq;
    req.root_leaders = slot.roots.empty() ? nullptr : slot.roots.data();
    tessa_subtree_output out{};
    out.leaf_row_ids = slot.rows_d;
    out.leaf_starts = slot.starts_d;
    out.leaf_sizes = slot.sizes_d;
    out.topk_ids = slot.ids_d;
    out.topk_dists = slot.dists_d;
    out.counters = slot.counters;
    out.leaf_counters = slot.leaf_counters;
    std::memset(slot.counters, 0, sizeof(slot.counters));
    std::memset(slot.leaf_counters, 0, sizeof(slot.leaf_counters));
    st = tessa_session_run_subtree_locked(s, &req, &out);
    slot.leaf_count = out.leaf_count;
    slot.leaf_rows = out.leaf_rows;
    slot.k = out.k;
    slot.levels = out.levels;
    slot.partition_ms = out.partition_ms;
    slot.leaf_ms = out.leaf_ms;
    if (st.code) return st;
    const uint64_t nslots = out.leaf_rows * out.k;
    st = grow_pinned(&slot.rows_h, &slot.rows_cap, out.leaf_rows);
    if (!st.code) st = grow_pinned(&slot.starts_h, &slot.starts_cap, out.leaf_count);
    if (!st.code) st = grow_pinned(&slot.sizes_h, &slot.sizes_cap, out.leaf_count);
    if (!st.code) st = grow_pinned(&slot.ids_h, &slot.ids_cap, nslots);
    if (!st.code) st = grow_pinned(&slot.dists_h, &slot.dists_cap, nslots);
    if (st.code) return st;
    // the D2H runs on the copy stream once the compute stream has produced the
    // results; the worker goes on to the next job, which computes into the
    // other slot's buffers meanwhile; wait() synchronises on `copied`
    hipStream_t q = s->copy_stream;
    TESSA_HIP_TRY(hipEventRecord(slot.computed, s->stream));
    TESSA_HIP_TRY(hipStreamWaitEvent(q, slot.computed, 0));
    TESSA_HIP_TRY(hipMemcpyAsync(slot.rows_h, slot.rows_d, out.leaf_rows * 4, hipMemcpyDeviceToHost, q));
    TESSA_HIP_TRY(hipMemcpyAsync(slot.starts_h, slot.starts_d, out.leaf_count * 8, hipMemcpyDeviceToHost, q));
    TESSA_HIP_TRY(hipMemcpyAsync(slot.sizes_h, slot.sizes_d, out.leaf_count * 8, hipMemcpyDeviceToHost, q));
    if (nslots) {
        TESSA_HIP_TRY(hipMemcpyAsync(slot.ids_h, slot.ids_d, nslots * 4, hipMemcpyDeviceToHost, q));
        TESSA_HIP_TRY(hipMemcpyAsync(slot.dists_h, slot.dists_d, nslots * 4, hipMemcpyDeviceToHost, q));
    }
    TESSA_HIP_TRY(hipEventRecord(slot.copied, q));
    slot.copy_pending = true;
    return ok_status();
}

void async_worker(tessa_session *s) {
    (void)hipSetDevice(s->device);
    while (true) {
        int idx = -1;
        {
            std::unique_lock<std::mutex> lk(s->q_mu);
            s->q_cv.wait(lk, [s] { return s->stop || !s->queue.empty(); });
            if (s->queue.empty()) return;  // stop requested and nothing left
            idx = s->queue.front();
            s->queue.pop_front();
        }
        tessa_session::AsyncSlot &slot = s->slots[idx];
        tessa_status st;
        {
            std::lock_guard<std::mutex> lock(s->exec_mu);
            st = run_async_job(s, slot);
        }
        {
            std::lock_guard<std::mutex> lk(s->q_mu);
            slot.status = st;
            slot.state = 2;
        }
        s->q_cv.notify_all();
    }
}

void stop_async(tessa_session *s) {
    {
        std::lock_guard<std::mutex> lk(s->q_mu);
        s->stop = true;
    }
    s->q_cv.notify_all();
    if (s->worker_started && s->worker.joinable()) s->worker.join();
    s->worker_started = false;
    if (s->copy_stream) (void)hipStreamSynchronize(s->copy_stream);
    for (auto &slot : s->slots) {
        if (slot.rows_d) (void)hipFree(slot.rows_d);
        if (slot.starts_d) (void)hipFree(slot.starts_d);
        if (slot.sizes_d) (void)hipFree(slot.sizes_d);
        if (slot.ids_d) (void)hipFree(slot.ids_d);
        if (slot.dists_d) (void)hipFree(slot.dists_d);
        if (slot.computed) (void)hipEventDestroy(slot.computed);
        if (slot.copied) (void)hipEventDestroy(slot.copied);
        if (slot.rows_h) (void)hipHostFree(slot.rows_h);
        if (slot.starts_h) (void)hipHostFree(slot.starts_h);
        if (slot.sizes_h) (void)hipHostFree(slot.sizes_h);
        if (slot.ids_h) (void)hipHostFree(slot.ids_h);
        if (slot.dists_h) (void)hipHostFree(slot.dists_h);
        slot = tessa_session::AsyncSlot{};
    }
    if (s->copy_stream) (void)hipStreamDestroy(s->copy_stream);
    s->copy_stream = nullptr;
}

}  // namespace

extern "C" {

tessa_status tessa_session_submit_subtree(tessa_session *s, const tessa_sq8_view *host_sq8,
                                          const tessa_subtree_request *req, uint64_t *seq) {
    if (!s || !req || !seq) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "submit: null argument");
    *seq = 0;
    if (host_sq8) {
        tessa_status st = check_view(host_sq8);
        if (st.code) return st;
    }
    if (req->root_leader_count > kLeaderStride)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "CUDA persistent root leader override has %u leaders, exceeding per-node limit %u",
                           req->root_leader_count, kLeaderStride);
    if (req->root_leader_count > 0 && !req->root_leaders)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "root leader count without root leader ids");
    std::lock_guard<std::mutex> lk(s->q_mu);
    int idx = -1;
    for (int i = 0; i < tessa_session::kAsyncSlots; ++i)
        if (s->slots[i].state == 0) {
            idx = i;
            break;
        }
    if (idx < 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "both pinned host result slots are held: wait for and release a submission first");
    tessa_session::AsyncSlot &slot = s->slots[idx];
    slot.state = 1;
    slot.seq = s->next_seq++;
    slot.upload = host_sq8 != nullptr;
    if (host_sq8) slot.host = *host_sq8;
    slot.req = *req;
    slot.roots.assign(req->root_leaders, req->root_leaders + req->root_leader_count);
    slot.req.root_leaders = nullptr;
    slot.status = ok_status();
    if (!s->worker_started) {
        s->stop = false;
        s->worker = std::thread(async_worker, s);
        s->worker_started = true;
    }
    s->queue.push_back(idx);
    *seq = slot.seq;
    s->q_cv.notify_all();
    return ok_status();
}

tessa_status tessa_session_wait(tessa_session *s, uint64_t seq, tessa_subtree_host_result *out) {
    if (!s || !out) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "wait: null argument");
    std::memset(out, 0, sizeof(*out));
    std::unique_lock<std::mutex> lk(s->q_mu);
    int idx = -1;
    for (int i = 0; i < tessa_session::kAsyncSlots; ++i)
        if (s->slots[i].state != 0 && s->slots[i].seq == seq) idx = i;
    if (idx < 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "no pending or unreleased submission %llu",
                           (unsigned long long)seq);
    tessa_session::AsyncSlot &slot = s->slots[idx];
    s->q_cv.wait(lk, [&slot] { return slot.state == 2; });
    if (slot.copy_pending) {
        // the D2H into the pinned slot; the lock is dropped so the worker can
        // start the next job meanwhile (the slot stays held until release)
        const hipEvent_t ev = slot.copied;
        lk.unlock();
        const hipError_t e = hipEventSynchronize(ev);
        lk.lock();
        slot.copy_pending = false;
        if (e != hipSuccess && slot.status.code == 0)
            slot.status = make_status(TESSA_ERR_HIP, 0, "result copy failed: %s", hipGetErrorString(e));
    }
    out->leaf_row_ids = slot.rows_h;
    out->leaf_starts = slot.starts_h;
    out->leaf_sizes = slot.sizes_h;
    out->topk_ids = slot.ids_h;
    out->topk_dists = slot.dists_h;
    out->counters = slot.counters;
    out->leaf_counters = slot.leaf_counters;
    out->leaf_count = slot.leaf_count;
    out->leaf_rows = slot.leaf_rows;
    out->k = slot.k;
    out->levels = slot.levels;
    out->partition_ms = slot.partition_ms;
    out->leaf_ms = slot.leaf_ms;
    return slot.status;
}

tessa_status tessa_session_set_assignment_capture(tessa_session *s, uint32_t min_members) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    s->capture_min_members = min_members;
    s->capture.tasks.clear();
    s->capture.rows.clear();
    return ok_status();
}

tessa_status tessa_session_captured_assignments(tessa_session *s, tessa_captured_assignment *tasks,
                                                uint64_t task_capacity, uint32_t *ids, uint64_t id_capacity,
                                                uint64_t *task_count, uint64_t *id_count) {
    if (!s || !task_count || !id_count) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "capture: null argument");
    std::lock_guard<std::mutex> lock(s->exec_mu);
    *task_count = s->capture.tasks.size();
    *id_count = s->capture.rows.size();
    if (!tasks && !ids) return ok_status();
    if (task_capacity < *task_count || id_capacity < *id_count || !tasks || !ids)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "capture: outputs of %llu tasks / %llu ids below %llu / %llu",
                           (unsigned long long)task_capacity, (unsigned long long)id_capacity,
                           (unsigned long long)*task_count, (unsigned long long)*id_count);
    // global ids, translated when the run finished
    std::memcpy(ids, s->capture.rows.data(), *id_count * sizeof(uint32_t));
    for (uint64_t t = 0; t < *task_count; ++t) {
        const tessa::PartCaptureTask &c = s->capture.tasks[t];
        tasks[t] = tessa_captured_assignment{c.depth, c.retry, c.r_h, s->capture_padded_dim, c.member_count,
                                             c.leader_count, c.member_offset, c.leader_offset};
    }
    return ok_status();
}

tessa_status tessa_session_release(tessa_session *s, uint64_t seq) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    std::lock_guard<std::mutex> lk(s->q_mu);
    for (auto &slot : s->slots)
        if (slot.state != 0 && slot.seq == seq) {
            if (slot.state != 2)
                return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "submission %llu is still running: wait first",
                                   (unsigned long long)seq);
            // released without a wait: its copy must land before the slot's
            // buffers can be reused
            if (slot.copy_pending) (void)hipEventSynchronize(slot.copied);
            slot.copy_pending = false;
            slot.state = 0;
            return ok_status();
        }
    return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "no unreleased submission %llu", (unsigned long long)seq);
}

}  // extern "C"

// ---- candidate records -> edge records -----------------------------------------

extern "C" {

static tessa_status emit_edge_records_impl(const uint32_t *global_ids, uint64_t resident_rows,
                                           const tessa_leaf_batch *lb, const uint32_t *topk_ids,
                                           const float *topk_dists, const tessa_sketch_view *sk,
                                           tessa_edge_record *out, uint64_t out_capacity,
                                           uint64_t *leaf_record_offsets, uint64_t *record_count,
                                           tessa_edge_segment *segments, uint64_t segment_capacity,
                                           uint64_t *segment_count, bool unique, void *stream) {
    static_assert(sizeof(tessa_edge_record) == 16, "SpillRecord16 is 16 bytes");
    static_assert(sizeof(tessa_edge_segment) == 16, "segment descriptors are 16 bytes");
    if (record_count) *record_count = 0;
    if (segment_count) *segment_count = 0;
    if (!global_ids || !lb || !topk_ids || !topk_dists || !sk || !sk->rows || !record_count)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "edge records: null argument");
    if (!lb->members || !lb->member_offsets || !lb->member_counts || !lb->output_offsets)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf batch has a null pointer");
    if (lb->k == 0 || lb->k > (uint32_t)kMaxK)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf k=%u outside [1, 32]", lb->k);
    if (sk->m_bits == 0 || sk->m_bits > 16 || sk->m_bits > sk->width)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "m_hash_bits=%u must be in [1, min(16, width=%u)]",
                           sk->m_bits, sk->width);
    if (lb->max_leaf_rows > kEdgeMaxLeafRows)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "edge records: max_leaf_rows=%u above %u", lb->max_leaf_rows,
                           kEdgeMaxLeafRows);
    if (lb->leaf_count > 0 && !out && out_capacity > 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "edge records: null output with capacity %llu",
                           (unsigned long long)out_capacity);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    DeviceWorkspace *ws = nullptr;
    tessa_status st = device_workspace(&ws);
    if (st.code) return st;
    const uint64_t leaves = lb->leaf_count;
    st = grow(&ws->edge_totals, &ws->edge_totals_capacity, leaves + 1, sizeof(uint32_t), "edge leaf totals");
    if (st.code) return st;
    st = grow(&ws->edge_status, &ws->edge_status_capacity, kEdgeStatusWords, sizeof(uint64_t), "edge status");
    if (st.code) return st;
    if (!leaf_record_offsets) {
        st = grow(&ws->edge_base, &ws->edge_base_capacity, leaves + 1, sizeof(uint64_t), "edge leaf offsets");
        if (st.code) return st;
    }
    if (segments) {
        st = grow(&ws->edge_seg_base, &ws->edge_seg_base_capacity, leaves + 1, sizeof(uint64_t),
                  "edge segment offsets");
        if (st.code) return st;
    }
    EdgeParams p{};
    p.gids = global_ids;
    p.resident_rows = resident_rows;
    p.members = lb->members;
    p.member_offsets = lb->member_offsets;
    p.member_counts = lb->member_counts;
    p.output_offsets = lb->output_offsets;
    p.leaf_count = lb->leaf_count;
    p.max_leaf_rows = lb->max_leaf_rows;
    p.table_bits = edge_table_bits(lb->max_leaf_rows);
    p.k = lb->k;
    p.topk_ids = topk_ids;
    p.topk_dists = topk_dists;
    p.sketches = sk->rows;
    p.sketch_rows = sk->sketch_rows;
    p.width = sk->width;
    p.m_bits = sk->m_bits;
    p.out = reinterpret_cast<uint4 *>(out);
    p.out_capacity = out ? out_capacity : 0;
    p.leaf_totals = ws->edge_totals;
    p.leaf_base = leaf_record_offsets ? leaf_record_offsets : ws->edge_base;
    p.status = ws->edge_status;
    p.segments = reinterpret_cast<uint4 *>(segments);
    p.segment_capacity = segments ? segment_capacity : 0;
    p.leaf_seg_base = segments ? ws->edge_seg_base : nullptr;
    p.unique = segments && unique ? 1u : 0u;
    if (launch_edge_records(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "edge record kernel launch failed");
    uint64_t w[kEdgeStatusWords];
    TESSA_HIP_TRY(hipMemcpyAsync(w, p.status, sizeof(w), hipMemcpyDeviceToHost, s));
    uint64_t nseg = 0;
    if (segments) TESSA_HIP_TRY(hipMemcpyAsync(&nseg, ws->edge_seg_base + leaves, 8, hipMemcpyDeviceToHost, s));
    TESSA_HIP_TRY(hipStreamSynchronize(s));
    if (segment_count) *segment_count = nseg;
    if (w[kEdgeLeafTooLarge])
        return make_status(TESSA_ERR_OVERFLOW, TESSA_OVF_LEAF_ROW,
                           "edge records: a leaf of %llu rows exceeds max_leaf_rows=%u overflow_flags=0x%llx "
                           "overflow_labels=LEAF_ROW",
                           (unsigned long long)(w[kEdgeLeafTooLarge] - 1), lb->max_leaf_rows,
                           (unsigned long long)TESSA_OVF_LEAF_ROW);
    if (w[kEdgeFirstError] != ~0ull) {
        const uint64_t key = w[kEdgeFirstError];
        const uint64_t leaf = key >> 20;
        const uint64_t kind = (key >> 19) & 1u;
        const uint32_t row = (uint32_t)((key >> 6) & 0x1fffu);
        const uint32_t rank = (uint32_t)(key & 63u);
        if (kind == kEdgeErrOutside) {
            uint64_t out0 = 0;
            uint32_t j = 0;
            TESSA_HIP_TRY(hipMemcpy(&out0, lb->output_offsets + leaf, sizeof(out0), hipMemcpyDeviceToHost));
            TESSA_HIP_TRY(hipMemcpy(&j, topk_ids + out0 + (uint64_t)row * lb->k + rank, sizeof(j),
                                    hipMemcpyDeviceToHost));
            return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                               "Compact top-k batch references point %u outside leaf %llu", j,
                               (unsigned long long)leaf);
        }
        uint64_t moff = 0;
        uint32_t mr = 0, g = 0xffffffffu;
        TESSA_HIP_TRY(hipMemcpy(&moff, lb->member_offsets + leaf, sizeof(moff), hipMemcpyDeviceToHost));
        TESSA_HIP_TRY(hipMemcpy(&mr, lb->members + moff + row, sizeof(mr), hipMemcpyDeviceToHost));
        if (mr < resident_rows) TESSA_HIP_TRY(hipMemcpy(&g, global_ids + mr, sizeof(g), hipMemcpyDeviceToHost));
        if (mr >= resident_rows)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, TESSA_OVF_INVALID_TOPK_ROW_ID,
                               "leaf %llu row %u: resident row %u outside %llu rows overflow_flags=0x%llx "
                               "overflow_labels=INVALID_TOPK_ROW_ID",
                               (unsigned long long)leaf, row, mr, (unsigned long long)resident_rows,
                               (unsigned long long)TESSA_OVF_INVALID_TOPK_ROW_ID);
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "leaf %llu point %u has no sketch row (sketch rows %llu)",
                           (unsigned long long)leaf, g, (unsigned long long)sk->sketch_rows);
    }
    if (w[kEdgeCapacityHit]) {
        if (segments && nseg > segment_capacity)
            return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "edge segment capacity %llu below the %llu segments needed",
                               (unsigned long long)segment_capacity, (unsigned long long)nseg);
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "edge record capacity %llu below the %llu records needed",
                           (unsigned long long)p.out_capacity, (unsigned long long)w[kEdgeRecordCount]);
    }
    *record_count = p.unique ? w[kEdgeKept] : w[kEdgeRecordCount];
    return ok_status();
}

tessa_status tessa_emit_edge_records(const uint32_t *global_ids, uint64_t resident_rows, const tessa_leaf_batch *lb,
                                     const uint32_t *topk_ids, const float *topk_dists,
                                     const tessa_sketch_view *sk, tessa_edge_record *out, uint64_t out_capacity,
                                     uint64_t *leaf_record_offsets, uint64_t *record_count, void *stream) {
    return emit_edge_records_impl(global_ids, resident_rows, lb, topk_ids, topk_dists, sk, out, out_capacity,
                                  leaf_record_offsets, record_count, nullptr, 0, nullptr, false, stream);
}

tessa_status tessa_emit_edge_segments(const uint32_t *global_ids, uint64_t resident_rows, const tessa_leaf_batch *lb,
                                      const uint32_t *topk_ids, const float *topk_dists,
                                      const tessa_sketch_view *sk, tessa_edge_record *out, uint64_t out_capacity,
                                      tessa_edge_segment *segments, uint64_t segment_capacity,
                                      uint64_t *record_count, uint64_t *segment_count, void *stream) {
    if (!segments || !segment_count)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "edge segments: null segment output");
    return emit_edge_records_impl(global_ids, resident_rows, lb, topk_ids, topk_dists, sk, out, out_capacity, nullptr,
                                  record_count, segments, segment_capacity, segment_count, false, stream);
}

tessa_status tessa_emit_edge_segments_unique(const uint32_t *global_ids, uint64_t resident_rows,
                                             const tessa_leaf_batch *lb, const uint32_t *topk_ids,
                                             const float *topk_dists, const tessa_sketch_view *sk,
                                             tessa_edge_record *out, uint64_t out_capacity,
                                             tessa_edge_segment *segments, uint64_t segment_capacity,
                                             uint64_t *record_count, uint64_t *segment_count, void *stream) {
    if (!segments || !segment_count)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "edge segments: null segment output");
    return emit_edge_records_impl(global_ids, resident_rows, lb, topk_ids, topk_dists, sk, out, out_capacity, nullptr,
                                  record_count, segments, segment_capacity, segment_count, true, stream);
}

}  // extern "C"

// ---- HashPrune reservoirs --------------------------------------------------------

struct tessa_hashprune {
    int device = 0;
    tessa::HashPruneState st;
};

namespace {

void free_hashprune(tessa_hashprune *hp) {
    auto &s = hp->st;
    for (void *ptr : {(void *)s.slot_keys, (void *)s.slot_hash, (void *)s.slot_count, (void *)s.bucket,
                      (void *)s.offsets, (void *)s.block_sums, (void *)s.grouped, (void *)s.status,
                      (void *)s.seg_ws, (void *)s.grp_keys})
        if (ptr) (void)hipFree(ptr);
    delete hp;
}

tessa_status hp_alloc(void **ptr, uint64_t bytes, const char *what) {
    if (hipMalloc(ptr, bytes ? bytes : 16) != hipSuccess) {
        *ptr = nullptr;
        return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                           "%s allocation of %llu bytes failed overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                           what, (unsigned long long)bytes, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
    }
    return ok_status();
}

// The named R-half policy's parameters, validated as PiPNNParams::validate
// validates them (shear-core/src/algorithm/pipnn/params.rs:2696-2729) and
// resolved as HashPruneBackfillPolicy::from_params resolves them
// (hash_prune_backfill.rs:44-83: quota 1 for hash-slot-1 else 3, SoftTier
// alpha 1.1 with alpha^2 exactly 1.21, capacity min(row cap, floor(l_max / 2))
// by :299-336).
tessa_status resolve_backfill(const tessa_hashprune_backfill *bf, uint32_t l_max, tessa::HashPruneState &s) {
    if (!bf || bf->mode == TESSA_HP_BACKFILL_OFF) return ok_status();
    if (bf->mode < TESSA_HP_BACKFILL_RHALF_HASH_SLOT_1 || bf->mode > TESSA_HP_BACKFILL_RHALF_HARD_TIER_Q3)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "hashprune_backfill_mode %u is not a named R-half policy",
                           bf->mode);
    const uint32_t budget = l_max / 2;
    if (bf->max_backfill_per_row && bf->max_backfill_per_row > budget)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "hashprune_rhalf_max_backfill_per_row: named R-half maximum backfill per row must be in "
                           "1..=floor(l_max/2), got cap=%u l_max=%u",
                           bf->max_backfill_per_row, l_max);
    if (bf->hash_quota > 3)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "hashprune_rhalf_hash_quota: named R-half hash quota must be in 1..=3");
    const float a = bf->soft_tier_priority_alpha;
    if (a != 0.0f && (bf->mode != TESSA_HP_BACKFILL_RHALF_SOFT_TIER_Q3 || !std::isfinite(a) || a < 1.0f))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "hashprune_soft_tier_priority_alpha: SoftTier priority alpha must be finite and >= 1.0");
    s.rhalf_mode = bf->mode;
    s.rhalf_quota = bf->hash_quota ? bf->hash_quota : (bf->mode == TESSA_HP_BACKFILL_RHALF_HASH_SLOT_1 ? 1u : 3u);
    s.rhalf_capacity = bf->max_backfill_per_row ? bf->max_backfill_per_row : budget;
    if (bf->mode == TESSA_HP_BACKFILL_RHALF_SOFT_TIER_Q3) {
        const float alpha = a != 0.0f ? a : 1.1f;
        s.rhalf_alpha_sq = alpha == 1.1f ? 1.21 : (double)alpha * (double)alpha;
    }
    return ok_status();
}

tessa_status hashprune_make(uint32_t num_points, uint32_t l_max, const tessa_hashprune_backfill *bf,
                            tessa_hashprune **out) {
    if (!out) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune: null output");
    *out = nullptr;
    if (l_max == 0) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "l_max must be > 0");
    if (l_max > tessa::kHpMaxLMax)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "hashprune: l_max=%u above %u", l_max, tessa::kHpMaxLMax);
    tessa::HashPruneState probe;
    tessa_status st = resolve_backfill(bf, l_max, probe);
    if (st.code) return st;
    auto *hp = new (std::nothrow) tessa_hashprune();
    if (!hp) return make_status(TESSA_ERR_OUT_OF_MEMORY, 0, "hashprune: host allocation failed");
    if (hipGetDevice(&hp->device) != hipSuccess) {
        delete hp;
        return make_status(TESSA_ERR_HIP, 0, "hashprune: hipGetDevice failed");
    }
    auto &s = hp->st;
    s = probe;
    s.num_points = num_points;
    s.l_max = l_max;
    const uint64_t slots = (uint64_t)num_points * l_max;
    st = hp_alloc((void **)&s.slot_keys, slots * 8, "hashprune slot keys");
    if (!st.code && s.rhalf_mode)
        st = hp_alloc((void **)&s.grp_keys, slots * 8 * tessa::kRhalfGroup, "hashprune backfill groups");
    if (!st.code) st = hp_alloc((void **)&s.slot_hash, slots * 2, "hashprune slot hashes");
    if (!st.code) st = hp_alloc((void **)&s.slot_count, (uint64_t)num_points * 4, "hashprune slot counts");
    if (!st.code) st = hp_alloc((void **)&s.bucket, (uint64_t)num_points * 4, "hashprune source counts");
    if (!st.code) st = hp_alloc((void **)&s.offsets, ((uint64_t)num_points + 1) * 4, "hashprune source offsets");
    if (!st.code) {
        s.block_sums_capacity = tessa::hashprune_scan_blocks(num_points);
        st = hp_alloc((void **)&s.block_sums, s.block_sums_capacity * 4, "hashprune scan partials");
    }
    if (!st.code) st = hp_alloc((void **)&s.status, 8 * 4, "hashprune status");
    if (!st.code && tessa::launch_hashprune_clear(s, nullptr) != 0)
        st = make_status(TESSA_ERR_HIP, 0, "hashprune clear launch failed");
    if (!st.code && hipStreamSynchronize(nullptr) != hipSuccess)
        st = make_status(TESSA_ERR_HIP, 0, "hashprune clear failed");
    if (st.code) {
        free_hashprune(hp);
        return st;
    }
    *out = hp;
    return ok_status();
}

}  // namespace

extern "C" {

tessa_status tessa_hashprune_create(uint32_t num_points, uint32_t l_max, tessa_hashprune **out) {
    return hashprune_make(num_points, l_max, nullptr, out);
}

tessa_status tessa_hashprune_create_backfill(uint32_t num_points, uint32_t l_max,
                                             const tessa_hashprune_backfill *policy, tessa_hashprune **out) {
    return hashprune_make(num_points, l_max, policy, out);
}

tessa_status tessa_hashprune_destroy(tessa_hashprune *hp) {
    if (!hp) return ok_status();
    TESSA_HIP_TRY(hipSetDevice(hp->device));
    TESSA_HIP_TRY(hipDeviceSynchronize());
    free_hashprune(hp);
    return ok_status();
}

tessa_status tessa_hashprune_clear(tessa_hashprune *hp, void *stream) {
    if (!hp) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune is null");
    if (tessa::launch_hashprune_clear(hp->st, reinterpret_cast<hipStream_t>(stream)) != 0)
        return make_status(TESSA_ERR_HIP, 0, "hashprune clear launch failed");
    return ok_status();
}

tessa_status tessa_hashprune_insert(tessa_hashprune *hp, const tessa_edge_record *records, uint64_t count,
                                    void *stream) {
    if (!hp) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune is null");
    if (count && !records) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune: null records");
    if (count >= 0xffffffffull)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "hashprune: %llu records in one batch (limit 2^32-2)",
                           (unsigned long long)count);
    auto &s = hp->st;
    hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    if (count > s.grouped_capacity) {
        TESSA_HIP_TRY(hipStreamSynchronize(hs));
        if (s.grouped) TESSA_HIP_TRY(hipFree(s.grouped));
        s.grouped = nullptr;
        s.grouped_capacity = 0;
        tessa_status st = hp_alloc((void **)&s.grouped, count * 16, "hashprune grouped records");
        if (st.code) return st;
        s.grouped_capacity = count;
    }
    if (tessa::launch_hashprune_insert(s, reinterpret_cast<const uint4 *>(records), count, hs) != 0)
        return make_status(TESSA_ERR_HIP, 0, "hashprune insert launch failed");
    uint64_t bad = 0;
    TESSA_HIP_TRY(hipMemcpyAsync(&bad, s.status, sizeof(bad), hipMemcpyDeviceToHost, hs));
    TESSA_HIP_TRY(hipStreamSynchronize(hs));
    if (bad != ~0ull) {
        tessa_edge_record r{};
        TESSA_HIP_TRY(hipMemcpy(&r, records + bad, sizeof(r), hipMemcpyDeviceToHost));
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "Spill reducer encountered edge p=%u outside shard range [0, %u) (record %llu; the "
                           "batch's valid records were inserted)",
                           r.src, s.num_points, (unsigned long long)bad);
    }
    return ok_status();
}

}  // extern "C"

namespace tessa {

// tessa_hashprune_insert without the read-back of the out-of-range check: no
// stream synchronisation once the grouped buffer holds `count` records (it
// grows, synchronising, on the first larger batch).  For callers whose
// records are known to be in range (TierLift routes only those).
tessa_status hashprune_insert_async(tessa_hashprune *hp, const tessa_edge_record *records, uint64_t count,
                                    hipStream_t hs) {
    if (!hp) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune is null");
    if (count >= 0xffffffffull)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "hashprune: %llu records in one batch (limit 2^32-2)",
                           (unsigned long long)count);
    auto &s = hp->st;
    if (count > s.grouped_capacity) {
        TESSA_HIP_TRY(hipStreamSynchronize(hs));
        if (s.grouped) TESSA_HIP_TRY(hipFree(s.grouped));
        s.grouped = nullptr;
        s.grouped_capacity = 0;
        tessa_status st = hp_alloc((void **)&s.grouped, count * 16, "hashprune grouped records");
        if (st.code) return st;
        s.grouped_capacity = count;
    }
    if (tessa::launch_hashprune_insert(s, reinterpret_cast<const uint4 *>(records), count, hs) != 0)
        return make_status(TESSA_ERR_HIP, 0, "hashprune insert launch failed");
    return ok_status();
}

}  // namespace tessa

extern "C" {

tessa_status tessa_hashprune_insert_segments(tessa_hashprune *hp, const tessa_edge_record *records,
                                             const tessa_edge_segment *segments, uint64_t segment_count,
                                             void *stream) {
    if (!hp) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune is null");
    if (segment_count && (!records || !segments))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune: null records or segments");
    if (segment_count >= 0x7fffffffull)
        return make_status(TESSA_ERR_UNSUPPORTED, 0, "hashprune: %llu segments in one batch (limit 2^31-2)",
                           (unsigned long long)segment_count);
    auto &s = hp->st;
    hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    const uint64_t need = tessa::hashprune_segment_workspace_bytes(segment_count, s.num_points);
    if (need > s.seg_ws_bytes) {
        TESSA_HIP_TRY(hipStreamSynchronize(hs));
        if (s.seg_ws) TESSA_HIP_TRY(hipFree(s.seg_ws));
        s.seg_ws = nullptr;
        s.seg_ws_bytes = 0;
        tessa_status st = hp_alloc(&s.seg_ws, need, "hashprune segment workspace");
        if (st.code) return st;
        s.seg_ws_bytes = need;
    }
    if (tessa::launch_hashprune_insert_segments(s, reinterpret_cast<const uint4 *>(records),
                                                reinterpret_cast<const uint4 *>(segments), segment_count, hs) != 0)
        return make_status(TESSA_ERR_HIP, 0, "hashprune segment insert launch failed");
    uint64_t bad = 0;
    TESSA_HIP_TRY(hipMemcpyAsync(&bad, s.status, sizeof(bad), hipMemcpyDeviceToHost, hs));
    TESSA_HIP_TRY(hipStreamSynchronize(hs));
    if (bad != ~0ull) {
        tessa_edge_record r{};
        TESSA_HIP_TRY(hipMemcpy(&r, records + bad, sizeof(r), hipMemcpyDeviceToHost));
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "Spill reducer encountered edge p=%u outside shard range [0, %u) (record %llu; the "
                           "batch's other segments were inserted)",
                           r.src, s.num_points, (unsigned long long)bad);
    }
    return ok_status();
}

tessa_status tessa_hashprune_neighbors(const tessa_hashprune *hp, uint32_t *targets, uint16_t *hashes,
                                       float *dists, uint32_t *counts, void *stream) {
    if (!hp) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "hashprune is null");
    if (tessa::launch_hashprune_export(hp->st, targets, hashes, dists, counts, reinterpret_cast<hipStream_t>(stream)) != 0)
        return make_status(TESSA_ERR_HIP, 0, "hashprune export launch failed");
    return ok_status();
}

}  // extern "C"

// ---- graph emission ---------------------------------------------------------------

extern "C" {

tessa_status tessa_graph_pack(const uint32_t *targets, const uint32_t *counts, uint32_t num_points,
                              uint32_t row_stride, uint32_t start, uint64_t num_frozen_pts, void *out,
                              uint64_t out_capacity, uint64_t *index_size, void *stream) {
    if (!index_size) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph pack: null index_size");
    *index_size = 0;
    if (num_points && (!counts || (row_stride && !targets)))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph pack: null neighbour table");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    DeviceWorkspace *ws = nullptr;
    tessa_status st = device_workspace(&ws);
    if (st.code) return st;
    st = grow(&ws->graph_sums, &ws->graph_sums_capacity, tessa::graph_scan_blocks(num_points), sizeof(uint64_t),
              "graph scan partials");
    if (st.code) return st;
    st = grow(&ws->graph_row_off, &ws->graph_row_off_capacity, (uint64_t)num_points + 1, sizeof(uint64_t),
              "graph row offsets");
    if (st.code) return st;
    st = grow(&ws->graph_scalars, &ws->graph_scalars_capacity, 2, sizeof(uint64_t), "graph scalars");
    if (st.code) return st;
    tessa::GraphPackParams p{};
    p.targets = targets;
    p.counts = counts;
    p.num_points = num_points;
    p.row_stride = row_stride;
    p.start = start;
    p.num_frozen = num_frozen_pts;
    p.out_words = reinterpret_cast<uint32_t *>(out);
    p.block_sums = ws->graph_sums;
    p.row_off = ws->graph_row_off;
    p.total_words = ws->graph_scalars;
    p.max_degree = reinterpret_cast<uint32_t *>(ws->graph_scalars + 1);
    if (tessa::launch_graph_size(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "graph size launch failed");
    uint64_t words = 0;
    TESSA_HIP_TRY(hipMemcpyAsync(&words, p.total_words, sizeof(words), hipMemcpyDeviceToHost, s));
    TESSA_HIP_TRY(hipStreamSynchronize(s));
    *index_size = 24ull + 4ull * words;
    if (!out) return ok_status();
    if (out_capacity < *index_size)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph pack: output of %llu bytes below the %llu needed",
                           (unsigned long long)out_capacity, (unsigned long long)*index_size);
    if (reinterpret_cast<uintptr_t>(out) % 8 != 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph pack: output must be 8-byte aligned");
    if (tessa::launch_graph_pack(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "graph pack launch failed");
    return ok_status();
}

static tessa_status graph_search_impl(const float *data, const int8_t *codes, const float *scales,
                                      uint32_t padded_dim, uint32_t num_points, uint32_t dim,
                                      const uint32_t *targets, const uint32_t *counts, uint32_t row_stride,
                                      uint32_t start, const float *queries, uint32_t num_queries, uint32_t L,
                                      uint32_t K, uint32_t *out_ids, float *out_dists, uint32_t *out_cmps,
                                      void *stream) {
    if (K > L)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "Set L: %u to a value of at least K: %u", L, K);
    if (L == 0 || K == 0 || L > tessa::kSearchMaxL)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph search: L=%u, K=%u outside 1 <= K <= L <= %u", L,
                           K, tessa::kSearchMaxL);
    if (num_points == 0 || num_points == 0xFFFFFFFFu || start >= num_points || dim == 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph search: start %u, %u points of dim %u", start,
                           num_points, dim);
    if (num_queries == 0) return ok_status();
    if ((!data && (!codes || !scales)) || !counts || (row_stride && !targets) || !queries || !out_ids)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph search: null pointer");
    if (!data && padded_dim < dim)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph search: padded_dim %u below dim %u", padded_dim, dim);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    DeviceWorkspace *ws = nullptr;
    tessa_status st = device_workspace(&ws);
    if (st.code) return st;
    tessa::GraphSearchParams p{};
    p.slots = tessa::search_slots(num_points, num_queries);
    st = grow(&ws->search_tags, &ws->search_tags_capacity, (uint64_t)p.slots * num_points, sizeof(uint32_t),
              "search visited tags");
    if (st.code) return st;
    p.data = data;
    p.codes = codes;
    p.scales = scales;
    p.padded_dim = padded_dim;
    p.num_points = num_points;
    p.dim = dim;
    p.targets = targets;
    p.counts = counts;
    p.row_stride = row_stride;
    p.start = start;
    p.queries = queries;
    p.num_queries = num_queries;
    p.L = L;
    p.K = K;
    p.out_ids = out_ids;
    p.out_dists = out_dists;
    p.out_cmps = out_cmps;
    p.tags = ws->search_tags;
    if (tessa::launch_graph_search(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "graph search launch failed");
    return ok_status();
}

tessa_status tessa_graph_search(const float *data, uint32_t num_points, uint32_t dim, const uint32_t *targets,
                                const uint32_t *counts, uint32_t row_stride, uint32_t start, const float *queries,
                                uint32_t num_queries, uint32_t L, uint32_t K, uint32_t *out_ids, float *out_dists,
                                uint32_t *out_cmps, void *stream) {
    if (!data) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph search: null pointer");
    return graph_search_impl(data, nullptr, nullptr, 0, num_points, dim, targets, counts, row_stride, start, queries,
                             num_queries, L, K, out_ids, out_dists, out_cmps, stream);
}

tessa_status tessa_graph_search_sq8(const int8_t *codes, const float *scales, uint32_t padded_dim, uint32_t num_points,
                                    uint32_t dim, const uint32_t *targets, const uint32_t *counts, uint32_t row_stride,
                                    uint32_t start, const float *queries, uint32_t num_queries, uint32_t L, uint32_t K,
                                    uint32_t *out_ids, float *out_dists, uint32_t *out_cmps, void *stream) {
    if (!codes || !scales) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "graph search: null pointer");
    return graph_search_impl(nullptr, codes, scales, padded_dim, num_points, dim, targets, counts, row_stride, start,
                             queries, num_queries, L, K, out_ids, out_dists, out_cmps, stream);
}

tessa_status tessa_global_d0_assign(const int8_t *codes, const float *scales, const float *norms,
                                    const uint32_t *global_ids, uint64_t rows, uint32_t padded_dim,
                                    const int8_t *leader_codes, const float *leader_scales,
                                    const float *leader_norms, const uint32_t *leader_ids, uint32_t leader_count,
                                    uint32_t fanout_top, uint32_t *out_child, uint32_t *out_point,
                                    uint64_t *child_offsets, uint32_t *child_points, void *stream) {
    if (leader_count == 0)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "SQ GPU-D0 staging requires at least one global D0 leader");
    if (fanout_top == 0 || fanout_top > leader_count || fanout_top > tessa::kD0MaxFanout)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0,
                           "SQ GPU-D0 staging fanout must be in 1..=min(32, leaders), got fanout=%u leaders=%u",
                           fanout_top, leader_count);
    if (leader_count > tessa::kD0MaxLeaders || padded_dim == 0 || padded_dim % 16 != 0 || padded_dim > 1024)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "D0 assign: %u leaders, padded_dim %u unsupported",
                           leader_count, padded_dim);
    if ((child_offsets == nullptr) != (child_points == nullptr))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "D0 assign: child_offsets and child_points go together");
    const uint64_t items = rows * fanout_top;
    if (child_offsets && items >= 0x7fffffffull)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "D0 assign: %llu fragments exceed one grouping pass",
                           (unsigned long long)items);
    if ((rows && (!codes || !scales || !norms || !global_ids || !out_child || !out_point)) || !leader_codes ||
        !leader_scales || !leader_norms || !leader_ids)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "D0 assign: null pointer");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    DeviceWorkspace *ws = nullptr;
    tessa_status st = device_workspace(&ws);
    if (st.code) return st;
    st = grow(&ws->d0_rank, &ws->d0_rank_capacity, 2ull * leader_count, sizeof(uint32_t), "D0 leader ranks");
    if (st.code) return st;
    tessa::D0AssignParams p{};
    p.codes = codes;
    p.scales = scales;
    p.norms = norms;
    p.global_ids = global_ids;
    p.rows = rows;
    p.padded_dim = padded_dim;
    p.leader_codes = leader_codes;
    p.leader_scales = leader_scales;
    p.leader_norms = leader_norms;
    p.leader_ids = leader_ids;
    p.leaders = leader_count;
    p.fanout = fanout_top;
    p.leader_rank = ws->d0_rank;
    p.rank_leader = ws->d0_rank + leader_count;
    p.out_child = out_child;
    p.out_point = out_point;
    if (tessa::launch_d0_assign(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "D0 assign launch failed");
    if (!child_offsets) return ok_status();
    const size_t temp = tessa::d0_group_temp_bytes(items, leader_count);
    st = grow(&ws->d0_temp, &ws->d0_temp_capacity, temp, 1, "D0 grouping scratch");
    if (st.code) return st;
    if (tessa::launch_d0_group(p, child_offsets, child_points, ws->d0_temp, ws->d0_temp_capacity, s) != 0)
        return make_status(TESSA_ERR_HIP, 0, "D0 grouping launch failed");
    return ok_status();
}

tessa_status tessa_robust_prune(const float *data, uint32_t num_points, uint32_t dim, const uint32_t *targets,
                                const uint32_t *counts, uint32_t row_stride, uint32_t max_degree,
                                uint32_t max_occlusion, float alpha, int saturate, uint32_t *out_targets,
                                uint32_t *out_counts, void *stream) {
    if (max_degree == 0 || max_degree > tessa::kPruneMaxPool || row_stride > tessa::kPruneMaxPool)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "robust prune: max_degree %u / row_stride %u outside 1..%u",
                           max_degree, row_stride, tessa::kPruneMaxPool);
    if (num_points == 0) return ok_status();
    if (num_points == 0xFFFFFFFFu || dim == 0 || !(alpha == alpha))
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "robust prune: %u points of dim %u", num_points, dim);
    if (!data || !counts || (row_stride && !targets) || !out_targets || !out_counts)
        return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "robust prune: null pointer");
    tessa::RobustPruneParams p{};
    p.data = data;
    p.num_points = num_points;
    p.dim = dim;
    p.targets = targets;
    p.counts = counts;
    p.row_stride = row_stride;
    p.max_degree = max_degree;
    p.max_occlusion = max_occlusion;
    p.alpha = alpha;
    p.saturate = saturate ? 1u : 0u;
    p.out_targets = out_targets;
    p.out_counts = out_counts;
    if (tessa::launch_robust_prune(p, reinterpret_cast<hipStream_t>(stream)) != 0)
        return make_status(TESSA_ERR_HIP, 0, "robust prune launch failed");
    return ok_status();
}

}  // extern "C"
