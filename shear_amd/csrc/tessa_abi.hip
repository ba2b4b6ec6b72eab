// tessa_abi.hip -- the extern "C" boundary declared in include/tessa_hip.h.
//
// Host-side validation, per-device workspace and sessions.  Nothing here
// throws or aborts across the boundary: every failure becomes a tessa_status
// with a message that keeps the reference's "overflow_flags=0x.." and label
// tokens (compute_backend.rs:2198-2296), which SHEAR's orchestration matches
// by substring (rbc_partition.rs:2982-2998).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/tessa_hip.h"
#include "assign_kernels.h"
#include "leaf_kernels.h"
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

// Per-device workspace of the MFMA leaf path: the exact re-run queue (pairs
// (leaf, row)), the chain queue (headers + candidate pool) and their three
// counters.  Grown on demand; kept until the process ends (other callers may
// share the device).
struct DeviceWorkspace {
    uint32_t *queue_counts = nullptr;  // [0] fallback, [1] chain rows, [2] chain pool used
    uint32_t *fallback = nullptr;
    uint64_t fallback_capacity = 0;
    uint4 *chain_rows = nullptr;
    uint64_t chain_capacity = 0;
    uint2 *chain_pool = nullptr;
    uint64_t pool_capacity = 0;
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

tessa_status get_workspace(uint64_t rows, DeviceWorkspace **out) {
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
    st = grow(&ws.chain_pool, &ws.pool_capacity, (rows / 2 + 1) * 40, sizeof(uint2), "chain pool");
    if (st.code) return st;
    *out = &ws;
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

tessa_status tessa_leaf_topk(const tessa_sq8_view *sq8, const tessa_leaf_batch *lb, uint32_t *out_ids,
                             float *out_dists, uint64_t *counters, void *stream) {
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
    DeviceWorkspace *ws = nullptr;
    st = get_workspace((uint64_t)lb->leaf_count * lb->max_leaf_rows, &ws);
    if (st.code) return st;
    auto clamp32 = [](uint64_t v) { return (uint32_t)(v < 0xffffffffull ? v : 0xffffffffull); };
    p.fallback = ws->fallback;
    p.fallback_count = ws->queue_counts;
    p.fallback_capacity = clamp32(ws->fallback_capacity);
    p.chain_rows = ws->chain_rows;
    p.chain_count = ws->queue_counts + 1;
    p.chain_capacity = clamp32(ws->chain_capacity);
    p.chain_pool = ws->chain_pool;
    p.chain_pool_used = ws->queue_counts + 2;
    p.chain_pool_capacity = clamp32(ws->pool_capacity);
    // Zero the queue counters with a kernel (capture-safe, unlike a memset node).
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s, ws->queue_counts, 3u, 0u);
    if (launch_leaf_mfma(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "MFMA leaf kernel launch failed");
    if (launch_leaf_chain(p, s) != 0) return make_status(TESSA_ERR_HIP, 0, "leaf chain kernel launch failed");
    if (launch_leaf_exact_fallback(p, s) != 0)
        return make_status(TESSA_ERR_HIP, 0, "leaf fallback kernel launch failed");
    return ok_status();
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
};

namespace {

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
    if (e == hipSuccess) e = hipMalloc(&s->counters, TESSA_COUNTER_WORDS * sizeof(uint64_t));
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
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    free_sq8(s);
    if (s->scratch) (void)hipFree(s->scratch);
    if (s->counters) (void)hipFree(s->counters);
    if (s->ev0) (void)hipEventDestroy(s->ev0);
    if (s->ev1) (void)hipEventDestroy(s->ev1);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return ok_status();
}

tessa_status tessa_session_upload_sq8(tessa_session *s, const tessa_sq8_view *host) {
    if (!s) return make_status(TESSA_ERR_INVALID_ARGUMENT, 0, "session is null");
    tessa_status st = check_view(host);
    if (st.code) return st;
    TESSA_HIP_TRY(hipSetDevice(s->device));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    free_sq8(s);
    const uint64_t rows = host->rows;
    if (hipMalloc(&s->codes, rows * host->padded_dim) != hipSuccess ||
        hipMalloc(&s->scales, rows * 4) != hipSuccess || hipMalloc(&s->norms, rows * 4) != hipSuccess ||
        hipMalloc(&s->gids, rows * 4) != hipSuccess) {
        free_sq8(s);
        return make_status(TESSA_ERR_OUT_OF_MEMORY, TESSA_OVF_WORKSPACE_BUDGET,
                           "SQ8 upload of %llu rows failed overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                           (unsigned long long)rows, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
    }
    TESSA_HIP_TRY(hipMemcpyAsync(s->codes, host->codes, rows * host->padded_dim, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(s->scales, host->scales, rows * 4, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(s->norms, host->norms, rows * 4, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipMemcpyAsync(s->gids, host->global_ids, rows * 4, hipMemcpyHostToDevice, s->stream));
    TESSA_HIP_TRY(hipStreamSynchronize(s->stream));
    s->rows = rows;
    s->dim = host->dim;
    s->padded_dim = host->padded_dim;
    return ok_status();
}

tessa_status tessa_session_leaf_topk(tessa_session *s, const uint32_t *members, const uint64_t *member_offsets,
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

tessa_status tessa_session_assign_replay(tessa_session *s, const uint32_t *members, const uint32_t *leaders,
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

}  // extern "C"
