// partition.hip -- recursive subtree partition on gfx950.
//
// Reference: the partition side of gpu_persistent_subtree_topk
// (compute_backend.rs:16555-17112): gpu_persistent_stage_large_node
// (:12456-12646), the large task's COUNT / EMIT / SCATTER / PUBLISH phases
// (:15047-15727), gpu_persistent_process_node for small nodes (:12648-13078)
// and gpu_persistent_push_leaf (:11735-11839).
//
// The reference walks the tree with one persistent kernel whose CTAs spin on
// a node queue and serialise every large node through a single large-task
// descriptor.  Here the walk is level-synchronous: every node of a level is
// staged, counted, split and scattered by the same few launches, so all of
// the chip works on all nodes of a level at once and no workgroup ever waits
// on another.  The schedule is deterministic: nodes are numbered in
// publication order, children in leader-slot order, and a child's rows keep
// the parent's row order (stable scatter by per-item prefix counts).
//
// Kernels per level:
//   stage      one workgroup per node: split parameters and leaders
//   item_plan  one workgroup: 512-row work items per node (prefix sum)
//   count      one workgroup per item: best leader slots on int8 MFMA
//   emit       one workgroup per node: accept / retry / balanced fallback
//   node_scan  one workgroup per node: child offsets, per-item prefixes
//   pub_scan   one workgroup: leaf and next-level numbering (prefix sums)
//   scatter    one workgroup per item: rows to leaves / next arena
#include <type_traits>

#include "partition.h"
#include "tessa_device.h"

namespace tessa {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ void pc_add(uint64_t *c, int idx, uint64_t v) {
    if (v) atomicAdd((unsigned long long *)&c[idx], (unsigned long long)v);
}
__device__ __forceinline__ void pc_max(uint64_t *c, int idx, uint64_t v) {
    atomicMax((unsigned long long *)&c[idx], (unsigned long long)v);
}
__device__ __forceinline__ void pc_min(uint64_t *c, int idx, uint64_t v) {
    atomicMin((unsigned long long *)&c[idx], (unsigned long long)v);
}
__device__ __forceinline__ void pc_flag(uint64_t *c, uint64_t bits) {
    atomicOr((unsigned long long *)&c[TESSA_P_OVERFLOW_FLAGS], (unsigned long long)bits);
}

// compute_backend.rs:7044-7075 (f32, each product rounded).
__device__ float adaptive_psamp(float base, uint32_t n, uint32_t depth) {
    float f = base;
    if (n >= 20000000u) f = __fmul_rn(f, 0.05f);
    else if (n >= 10000000u) f = __fmul_rn(f, 0.1f);
    else if (n >= 5000000u) f = __fmul_rn(f, 0.2f);
    else if (n >= 1000000u) f = __fmul_rn(f, 0.4f);
    else if (n >= 100000u) f = __fmul_rn(f, 0.7f);
    if (depth > 4u) f = __fmul_rn(f, 0.35f);
    else if (depth > 2u) f = __fmul_rn(f, 0.5f);
    else if (depth > 0u) f = __fmul_rn(f, 0.8f);
    if (f < 0.00005f) f = 0.00005f;
    if (f > 0.1f) f = 0.1f;
    return f;
}

// (uint32)(psamp * n + 0.5f), clamped to [2, max] (:12542-12549 / :12761-12767).
__device__ uint32_t base_leader_count(float psamp, uint32_t n, uint32_t max_leaders) {
    const float v = __fadd_rn(__fmul_rn(psamp, (float)n), 0.5f);
    uint32_t b = (uint32_t)v;
    if (b < 2u) b = 2u;
    if (b > max_leaders) b = max_leaders;
    return b;
}

// compute_backend.rs:7082-7101
__device__ bool meaningful_split(uint32_t parent, uint32_t max_child, uint32_t terminal) {
    if (parent <= terminal || max_child <= terminal) return true;
    if (max_child >= parent) return false;
    uint32_t min_shrink = parent >> 5;
    if (min_shrink < 32u) min_shrink = 32u;
    if (min_shrink >= parent) min_shrink = 1u;
    return max_child + min_shrink <= parent;
}

// compute_backend.rs:6541-6568
__device__ __forceinline__ bool assign_before(float d, uint32_t point, uint32_t leader, float od, uint32_t oleader) {
    if (fabsf(__fsub_rn(d, od)) <= kTieEps) {
        const uint64_t ck = assign_tie_key(point, leader);
        const uint64_t ok = assign_tie_key(point, oleader);
        return ck < ok || (ck == ok && leader < oleader);
    }
    return d < od;
}

// compute_backend.rs:6524-6580 with F (1..4) live slots: compare with the
// last live slot, then shift towards the front.  F is a template argument so
// the slot registers are never indexed dynamically.
template <int F>
__device__ __forceinline__ void insert_slot(float d, uint32_t point, uint32_t leader, uint32_t slot,
                                            float (&bd)[4], uint32_t (&bs)[4], uint32_t (&bl)[4]) {
    if (!assign_before(d, point, leader, bd[F - 1], bl[F - 1])) return;
    int pos = F - 1;
#pragma unroll
    for (int q = F - 1; q >= 1; --q) {
        if (pos == q && assign_before(d, point, leader, bd[q - 1], bl[q - 1])) {
            bd[q] = bd[q - 1];
            bs[q] = bs[q - 1];
            bl[q] = bl[q - 1];
            pos = q - 1;
        }
    }
#pragma unroll
    for (int q = 0; q < F; ++q)
        if (q == pos) {
            bd[q] = d;
            bs[q] = slot;
            bl[q] = leader;
        }
}

// Exclusive prefix sum over the workgroup (blockDim.x threads, power of 2).
__device__ uint64_t block_exclusive_scan(uint64_t v, uint64_t *sh, uint64_t *total) {
    const uint32_t t = threadIdx.x;
    sh[t] = v;
    __syncthreads();
    for (uint32_t off = 1; off < blockDim.x; off <<= 1) {
        const uint64_t x = t >= off ? sh[t - off] : 0ull;
        __syncthreads();
        sh[t] += x;
        __syncthreads();
    }
    const uint64_t incl = sh[t];
    *total = sh[blockDim.x - 1];
    __syncthreads();
    return incl - v;
}

// Item -> node: the last node whose item_base <= item (nodes with no items
// share the next node's base, so the last such node owns the item).
__device__ uint32_t find_item_node(const NodeDesc *nodes, uint32_t level_nodes, uint32_t item) {
    uint32_t lo = 0, hi = level_nodes - 1u;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) >> 1;
        if (nodes[mid].item_base <= item) lo = mid;
        else hi = mid - 1u;
    }
    return lo;
}

// ---------------------------------------------------------------------------
__global__ void init_kernel(PartArgs a) {
    for (uint32_t i = threadIdx.x; i < TESSA_SUBTREE_COUNTER_WORDS; i += blockDim.x) a.counters[i] = 0ull;
    __syncthreads();
    if (threadIdx.x == 0) {
        a.counters[TESSA_P_LEAF_SIZE_MIN] = ~0ull;
        a.counters[TESSA_P_UNIQUE_RESIDENT_ROWS] = a.rows;
        LevelHeader h{};
        *a.hdr = h;
    }
}

// Root node: rows 0..R-1 in the first arena (compute_backend.rs:16503-16519).
__global__ void root_kernel(PartArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.rows) a.arena[0][i] = (uint32_t)i;
    if (i == 0) {
        NodeDesc nd{};
        nd.row_start = 0;
        nd.seed = a.seed;
        nd.n = a.rows;
        nd.depth = a.root_depth;
        nd.status = kNodeIdle;
        a.nodes[0][0] = nd;
    }
}

// Several roots: resident rows 0..rows-1 in the first arena, node i = root i.
__global__ void multi_root_kernel(PartArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.rows) a.arena[0][i] = (uint32_t)i;
    if (i < a.root_count) {
        NodeDesc nd{};
        nd.row_start = a.root_offsets[i];
        nd.root_base = a.root_offsets[i];
        nd.root_index = (uint32_t)i;
        nd.seed = a.root_seeds[i];
        nd.n = (uint32_t)(a.root_offsets[i + 1] - a.root_offsets[i]);
        nd.depth = a.root_depth;
        nd.status = kNodeIdle;
        a.nodes[0][i] = nd;
    }
}

__global__ void reset_retry_kernel(LevelHeader *h) { h->retry_nodes = 0u; }

// ---- stage (compute_backend.rs:12456-12646) ---------------------------------
__global__ __launch_bounds__(128) void stage_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    const uint32_t ni = blockIdx.x;
    NodeDesc *nd = a.nodes[cur] + ni;
    __shared__ uint32_t s_nl, s_use_root;
    if (threadIdx.x == 0) {
        if (ni == 0) {
            pc_add(a.counters, TESSA_P_PARTITION_POPS, level_nodes);
            pc_add(a.counters, TESSA_P_PARTITION_LEVEL_ROUNDS, 1);
        }
        const uint32_t n = nd->n, depth = nd->depth;
        uint32_t status = kNodeIdle, nl = 0, use_root = 0;
        if (n == 0u) {
        } else if (depth >= a.max_depth) {
            pc_flag(a.counters, TESSA_OVF_OVERSIZED_TERMINAL_NODE);
        } else if ((uint64_t)n > a.large_scratch_rows) {
            pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
        } else {
            pc_add(a.counters, TESSA_P_LARGE_NODE_CLAIMS, 1);
            pc_add(a.counters, TESSA_P_LARGE_NODE_ROWS, n);
            pc_max(a.counters, TESSA_P_LARGE_NODE_MAX_ROWS, n);
            uint32_t retry_max = n < 2u ? 2u : n;
            if (retry_max > kPartMaxLeaders) retry_max = kPartMaxLeaders;
            uint32_t max_leaders = a.max_leaders < retry_max ? a.max_leaders : retry_max;
            if (max_leaders < 2u) max_leaders = 2u;
            const uint32_t rel = depth >= a.root_depth ? depth - a.root_depth : 0u;
            use_root = (rel == 0u && a.root_leader_count > 0u) ? 1u : 0u;
            const float psamp = adaptive_psamp(a.psamp, n, depth);
            nl = use_root ? a.root_leader_count : base_leader_count(psamp, n, max_leaders);
            if (nl > max_leaders) nl = max_leaders;
            uint32_t req = rel == 0u ? a.fanout_second : 1u;
            if (req < 1u) req = 1u;
            if (req > 4u) {
                pc_flag(a.counters, TESSA_OVF_FANOUT_OVER_32);
                nl = 0;
            } else {
                const uint32_t fanout = req < nl ? req : nl;
                pc_max(a.counters, TESSA_P_EFFECTIVE_ROOT_FANOUT, rel == 0u ? fanout : 0u);
                pc_max(a.counters, TESSA_P_EFFECTIVE_DEEPER_FANOUT, rel > 0u ? fanout : 1u);
                nd->num_leaders = nl;
                nd->fanout = fanout;
                nd->attempt = 0u;
                nd->max_leaders = max_leaders;
                nd->retry_allowed = use_root ? 0u : 1u;
                status = kNodeCounting;
            }
        }
        nd->status = status;
        s_nl = status == kNodeCounting ? nl : 0u;
        s_use_root = use_root;
    }
    __syncthreads();
    const uint32_t t = threadIdx.x;
    const uint32_t nl = s_nl;
    uint32_t leader = 0u;
    if (t < nl) {
        if (s_use_root) {
            leader = a.root_leaders[t];
        } else {
            const uint32_t n = nd->n;
            uint32_t ord = (uint32_t)(((uint64_t)t * n) / nl);
            if (ord >= n) ord = n - 1u;
            leader = a.arena[cur][nd->row_start + ord];
        }
    }
    a.leaders[(uint64_t)ni * kPartMaxLeaders + t] = leader;
    a.child_counts[(uint64_t)ni * kPartMaxLeaders + t] = 0u;
}

// ---- item plan ---------------------------------------------------------------
__global__ __launch_bounds__(1024) void item_plan_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    __shared__ uint64_t sh[1024];
    NodeDesc *nodes = a.nodes[cur];
    const uint32_t per = (level_nodes + 1023u) / 1024u;
    const uint32_t b = threadIdx.x * per;
    const uint32_t e = b + per < level_nodes ? b + per : level_nodes;
    uint64_t local = 0;
    for (uint32_t i = b; i < e; ++i)
        if (nodes[i].status == kNodeCounting) local += (nodes[i].n + kPartItemRows - 1u) / kPartItemRows;
    uint64_t total = 0;
    uint64_t base = block_exclusive_scan(local, sh, &total);
    for (uint32_t i = b; i < e; ++i) {
        const uint32_t items =
            nodes[i].status == kNodeCounting ? (nodes[i].n + kPartItemRows - 1u) / kPartItemRows : 0u;
        nodes[i].item_base = (uint32_t)base;
        nodes[i].items = items;
        base += items;
    }
    if (threadIdx.x == 0) {
        if (total > a.item_cap) {
            pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
            total = 0;
        }
        a.hdr->items = (uint32_t)total;
        a.hdr->retry_nodes = 0u;
    }
}

// ---- COUNT: best leader slots per row on int8 MFMA --------------------------
// (compute_backend.rs:14705-14918 role; insertion :6524-6580).  A workgroup
// takes one 512-row item of one node.  The node's leaders (<= 128) sit in
// LDS as the A operand; each wave keeps 32 rows' codes in VGPRs as B.  Per
// 32-leader tile the distances go through LDS so one lane per row can apply
// the order-dependent insertion in leader-slot order.
// waves of a COUNT workgroup: 8 (two per SIMD) when their distance buffers
// fit beside the leaders, else 4
template <int KS>
constexpr int count_waves() {
    return (KS * 32 + 16) * 128 + 5 * 128 * 4 + 8 * 32 * 33 * 4 <= 160 * 1024 ? 8 : 4;
}
constexpr uint32_t kCountGrid = 512;  // persistent COUNT grid (items are taken grid-stride)

template <int KS>
struct CountLayout {
    static constexpr int kWaves = count_waves<KS>();
    static constexpr int kThreads = kWaves * 64;
    static constexpr int kChunk = kWaves * 32;  // rows per chunk
    static constexpr int kChunks = kPartItemRows / kChunk;
    static constexpr int kStride = KS * 32 + 16;
    static constexpr int kLeaderBytes = kPartMaxLeaders * kStride;
    static constexpr int kMetaOff = kLeaderBytes;  // scales, norms, ids [128] each
    static constexpr int kCntOff = kMetaOff + 3 * kPartMaxLeaders * 4;
    static constexpr int kDistOff = kCntOff + kPartMaxLeaders * 4;
    static constexpr int kBytes = kDistOff + kWaves * 32 * 33 * 4;
    static_assert(kBytes <= 160 * 1024, "LDS budget");
    static_assert(kPartItemRows % kChunk == 0, "item rows");
};

// LDS hand-off inside one wave: its lanes' LDS writes are seen by its other
// lanes' later reads (and reads finish before later writes).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Persistent over the level's items: a workgroup takes items blockIdx.x,
// + gridDim.x, ...; the leaders of an item's node are staged in LDS only when
// the node differs from the previous item's (a large node's items reuse them).
// Each wave owns 32 rows at a time and its own distance buffer, so inside an
// item the waves only synchronise with themselves.
template <int KS>
__global__ __launch_bounds__(CountLayout<KS>::kThreads, 1) void count_kernel(PartArgs a, uint32_t cur,
                                                                             uint32_t level_nodes) {
    using L = CountLayout<KS>;
    constexpr uint32_t kThr = L::kThreads;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    int8_t *lcodes = reinterpret_cast<int8_t *>(smem);
    float *ls = reinterpret_cast<float *>(smem + L::kMetaOff);
    float *ln = ls + kPartMaxLeaders;
    uint32_t *lid = reinterpret_cast<uint32_t *>(ln + kPartMaxLeaders);
    uint32_t *cnt = reinterpret_cast<uint32_t *>(smem + L::kCntOff);
    float *dbuf = reinterpret_cast<float *>(smem + L::kDistOff);
    __shared__ uint32_t s_node;

    const uint32_t items = a.hdr->items;
    const uint32_t pd = a.padded_dim;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t j = lane & 31u;
    const uint32_t h = lane >> 5;
    const uint32_t *arena = a.arena[cur];
    // resident row -> SQ8 row; tie keys use the row's index within its root
    const uint32_t *rmap = a.row_map;
    uint32_t staged = 0xffffffffu;  // node whose leaders are in LDS
    for (uint32_t item = blockIdx.x; item < items; item += gridDim.x) {
        if (tid == 0) s_node = find_item_node(a.nodes[cur], level_nodes, item);
        __syncthreads();
        const uint32_t ni = s_node;
        const NodeDesc *nd = a.nodes[cur] + ni;
        if (nd->status != kNodeCounting) {
            __syncthreads();  // s_node is rewritten by the next item
            continue;
        }
        const uint32_t n = nd->n;
        const uint32_t nl = nd->num_leaders;
        const uint32_t fanout = nd->fanout;
        const uint64_t row_start = nd->row_start;
        const uint32_t first = (item - nd->item_base) * kPartItemRows;
        const uint32_t rb = (uint32_t)nd->root_base;
        if (ni != staged) {
            const uint32_t *node_leaders = a.leaders + (uint64_t)ni * kPartMaxLeaders;
            for (uint32_t q = tid; q < (uint32_t)kPartMaxLeaders * KS * 2; q += kThr) {
                const uint32_t li = q / (KS * 2);
                const uint32_t off = (q % (KS * 2)) * 16u;
                v4i z = {0, 0, 0, 0};
                if (li < nl && off < pd) {
                    const uint32_t g = node_leaders[li];
                    if (g < a.rows)
                        z = *reinterpret_cast<const v4i *>(a.codes + (uint64_t)(rmap ? rmap[g] : g) * pd + off);
                }
                *reinterpret_cast<v4i *>(lcodes + li * L::kStride + off) = z;
            }
            for (uint32_t li = tid; li < (uint32_t)kPartMaxLeaders; li += kThr) {
                uint32_t g = li < nl ? node_leaders[li] : rb;
                if (li < nl && g >= a.rows) {
                    pc_flag(a.counters, TESSA_OVF_INVALID_ASSIGN_LEADER_ID);
                    g = rb;
                }
                const uint32_t sg = rmap ? rmap[g] : g;
                ls[li] = li < nl ? a.scales[sg] : 0.0f;
                ln[li] = li < nl ? a.norms[sg] : 0.0f;
                lid[li] = g - rb;
            }
            staged = ni;
        }
        for (uint32_t li = tid; li < (uint32_t)kPartMaxLeaders; li += kThr) cnt[li] = 0u;
        __syncthreads();

        const uint32_t ntiles = (nl + 31) / 32;
        float *wb = dbuf + wave * 32 * 33;
        for (int ch = 0; ch < L::kChunks; ++ch) {
            if (first + ch * L::kChunk >= n) break;  // uniform across the block
            const uint32_t m = first + ch * L::kChunk + wave * 32u + j;
            bool ok = m < n;
            uint32_t pt = ok ? arena[row_start + m] : rb;
            if (ok && pt >= a.rows) {
                pc_flag(a.counters, TESSA_OVF_INVALID_ASSIGN_POINT_ID);
                ok = false;
                pt = rb;
            }
            if (__ballot(ok) == 0ull) continue;  // this wave's rows are past the node's end
            const uint32_t spt = rmap ? rmap[pt] : pt;
            v4i bfrag[KS];
            const int8_t *mc = a.codes + (uint64_t)spt * pd;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const uint32_t off = 32u * s + 16u * h;
                v4i z = {0, 0, 0, 0};
                if (ok && off < pd) z = *reinterpret_cast<const v4i *>(mc + off);
                bfrag[s] = z;
            }
            const float ps = ok ? a.scales[spt] : 0.0f;
            const float pn = ok ? a.norms[spt] : 0.0f;
            const uint32_t lpt = pt - rb;  // the row's index within its root
            // compute_backend.rs:6357-6368 reset: (FLT_MAX, empty)
            float bd[4] = {kEmptyDist, kEmptyDist, kEmptyDist, kEmptyDist};
            uint32_t bs[4] = {kEmptyId, kEmptyId, kEmptyId, kEmptyId};
            uint32_t bl[4] = {kEmptyId, kEmptyId, kEmptyId, kEmptyId};
            for (uint32_t t = 0; t < ntiles; ++t) {
                v16i acc = {};
                const int8_t *arow = lcodes + (32u * t + j) * L::kStride + 16u * h;
                // A operands read two steps ahead of their MFMA
                v4i ring[3];
                ring[0] = *reinterpret_cast<const v4i *>(arow);
                if constexpr (KS > 1) ring[1] = *reinterpret_cast<const v4i *>(arow + 32);
#pragma unroll
                for (int s = 0; s < KS; ++s) {
                    if (s + 2 < KS) ring[(s + 2) % 3] = *reinterpret_cast<const v4i *>(arow + 32 * (s + 2));
                    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ring[s % 3], bfrag[s], acc, 0, 0, 0);
                }
                // the lane's 16 leaders are 4 runs of 4 (8g + 4h + e): their
                // scales and norms in 8 vector reads, then every distance
                float4 lsv[4], lnv[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    lsv[g] = *reinterpret_cast<const float4 *>(ls + 32u * t + 8u * g + 4u * h);
                    lnv[g] = *reinterpret_cast<const float4 *>(ln + 32u * t + 8u * g + 4u * h);
                }
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t li = 8u * (v / 4) + 4u * h + (v % 4);  // leader within the tile
                    const uint32_t gl = 32u * t + li;
                    const int e = v % 4, g = v / 4;
                    const float lsc = e == 0 ? lsv[g].x : e == 1 ? lsv[g].y : e == 2 ? lsv[g].z : lsv[g].w;
                    const float lno = e == 0 ? lnv[g].x : e == 1 ? lnv[g].y : e == 2 ? lnv[g].z : lnv[g].w;
                    const float d = assign_l2(acc[v], ps, pn, lsc, lno);
                    wb[li * 33 + j] = gl < nl ? d : kEmptyDist;
                }
                wave_lds_sync();
                if (h == 0u && ok) {
                    const uint32_t lim = (nl - 32u * t) < 32u ? (nl - 32u * t) : 32u;
                    // leaders in slot order, 8 at a time: the 8 distances and
                    // leader ids of a step are read before its insertions
                    auto run = [&](auto fc) {
                        constexpr int F = decltype(fc)::value;
                        for (uint32_t l0 = 0; l0 < lim; l0 += 8u) {
                            float dv[8];
                            uint32_t idv[8];
#pragma unroll
                            for (int q = 0; q < 8; ++q) {
                                dv[q] = wb[(l0 + q) * 33 + j];
                                idv[q] = lid[32u * t + l0 + q];
                            }
#pragma unroll
                            for (int q = 0; q < 8; ++q)
                                if (l0 + q < lim) insert_slot<F>(dv[q], lpt, idv[q], 32u * t + l0 + q, bd, bs, bl);
                        }
                    };
                    switch (fanout) {
                        case 1: run(std::integral_constant<int, 1>{}); break;
                        case 2: run(std::integral_constant<int, 2>{}); break;
                        case 3: run(std::integral_constant<int, 3>{}); break;
                        default: run(std::integral_constant<int, 4>{}); break;
                    }
                }
                wave_lds_sync();
            }
            if (h == 0u && ok) {
                uint32_t packed = 0xffffffffu;
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    if (k < fanout) {
                        const uint32_t s = bs[k];
                        if (s < nl) {
                            packed = (packed & ~(0xffu << (8u * k))) | (s << (8u * k));
                            atomicAdd(&cnt[s], 1u);
                        } else {
                            pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
                        }
                    }
                }
                a.slots[row_start + m] = packed;
            }
        }
        __syncthreads();
        for (uint32_t s = tid; s < nl; s += kThr) {
            const uint32_t c = cnt[s];
            a.item_counts[(uint64_t)item * kPartMaxLeaders + s] = c;
            if (c) atomicAdd(&a.child_counts[(uint64_t)ni * kPartMaxLeaders + s], c);
        }
        if (tid == 0) {
            const uint32_t rows_here = (n - first) < kPartItemRows ? (n - first) : kPartItemRows;
            pc_add(a.counters, TESSA_P_LARGE_PHYSICAL_TILES, (rows_here + 15u) / 16u);
        }
        __syncthreads();  // cnt and s_node are reused by the next item
    }
}

// ---- EMIT (compute_backend.rs:15396-15555) -----------------------------------
__global__ __launch_bounds__(128) void emit_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    const uint32_t ni = blockIdx.x;
    NodeDesc *nd = a.nodes[cur] + ni;
    if (nd->status != kNodeCounting) return;
    __shared__ uint64_t s_sum[2];
    __shared__ uint32_t s_nonempty[2], s_max[2];
    __shared__ uint32_t s_act, s_next, s_attempt;
    const uint32_t t = threadIdx.x;
    const uint32_t nl = nd->num_leaders;
    const uint32_t n = nd->n;
    uint32_t *counts = a.child_counts + (uint64_t)ni * kPartMaxLeaders;
    const uint32_t c = t < nl ? counts[t] : 0u;
    uint64_t sum = c;
    uint32_t ne = c ? 1u : 0u, mx = c;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        sum += __shfl_xor(sum, off);
        ne += __shfl_xor(ne, off);
        const uint32_t o = __shfl_xor(mx, off);
        mx = o > mx ? o : mx;
    }
    if ((t & 63u) == 0u) {
        s_sum[t >> 6] = sum;
        s_nonempty[t >> 6] = ne;
        s_max[t >> 6] = mx;
    }
    __syncthreads();
    if (t == 0) {
        const uint64_t running = s_sum[0] + s_sum[1];
        const uint32_t nonempty = s_nonempty[0] + s_nonempty[1];
        const uint32_t max_child = s_max[0] > s_max[1] ? s_max[0] : s_max[1];
        s_act = 0u;
        if (running > a.large_scratch_rows) {
            pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
            nd->status = kNodeIdle;
        } else if (nonempty > 1u && meaningful_split(n, max_child, a.leaf_max)) {
            nd->status = kNodeAccepted;
            pc_add(a.counters, TESSA_P_FANOUT_ASSIGNMENT_SLOTS, (uint64_t)n * nd->fanout);
            pc_add(a.counters, TESSA_P_REPLICATED_ROWS, (uint64_t)n * nd->fanout);
        } else if (nd->retry_allowed && (nd->attempt == 0u || nl < nd->max_leaders)) {
            const uint32_t max_leaders = nd->max_leaders;
            uint32_t next = nl;
            if (nd->attempt > 0u) {
                const uint32_t doubled = next << 1;
                next = (doubled > next && doubled < max_leaders) ? doubled : max_leaders;
            }
            if (next > max_leaders) next = max_leaders;
            nd->num_leaders = next;
            nd->attempt += 1u;
            s_act = 1u;
            s_next = next;
            s_attempt = nd->attempt;
            pc_add(a.counters, TESSA_P_LARGE_SPLIT_RETRIES, 1);
            atomicAdd(&a.hdr->retry_nodes, 1u);
        } else {
            nd->status = kNodeBalanced;
            nd->num_leaders = 2u;
            nd->fanout = 1u;
            counts[0] = (n + 1u) >> 1;
            counts[1] = n >> 1;
            pc_add(a.counters, TESSA_P_LARGE_BALANCED_FALLBACKS, 1);
            pc_add(a.counters, TESSA_P_FANOUT_ASSIGNMENT_SLOTS, n);
            pc_add(a.counters, TESSA_P_REPLICATED_ROWS, n);
        }
    }
    __syncthreads();
    if (s_act == 1u) {
        // compute_backend.rs:5991-6019 hash-sampled retry leaders, one per span.
        const uint32_t next = s_next;
        uint32_t leader = 0u;
        if (t < next) {
            uint32_t b = (uint32_t)(((uint64_t)t * n) / next);
            uint32_t e = (uint32_t)(((uint64_t)(t + 1u) * n) / next);
            if (e <= b) e = b + 1u;
            const uint32_t span = e - b;
            const uint64_t key = hash64(nd->seed ^ ((uint64_t)s_attempt * 0xd6e8feb86659fd93ull) ^
                                        ((uint64_t)t * 0x9e3779b97f4a7c15ull));
            leader = a.arena[cur][nd->row_start + b + (uint32_t)(key % span)];
        }
        a.leaders[(uint64_t)ni * kPartMaxLeaders + t] = leader;
        counts[t] = 0u;
    }
}

// ---- child layout and per-item prefixes ----------------------------------
// 8 groups of 128 threads (one thread per leader slot) split the node's items
// into 8 ranges; each group sums its range, the groups' sums are scanned in
// LDS, then each group writes the exclusive prefixes of its range.  Item
// counts are read 16 items at a time, so the loads of a batch are in flight
// together.
constexpr uint32_t kScanGroups = 8;
constexpr uint32_t kScanBatch = 16;

__global__ __launch_bounds__(kScanGroups * kPartMaxLeaders) void node_scan_kernel(PartArgs a, uint32_t cur,
                                                                                 uint32_t level_nodes) {
    __shared__ uint32_t group_sum[kScanGroups][kPartMaxLeaders];
    const uint32_t ni = blockIdx.x;
    NodeDesc *nd = a.nodes[cur] + ni;
    const uint32_t status = nd->status;
    if (status != kNodeAccepted && status != kNodeBalanced) return;
    const uint32_t t = threadIdx.x % kPartMaxLeaders;
    const uint32_t g = threadIdx.x / kPartMaxLeaders;
    const uint32_t nl = nd->num_leaders;
    const uint64_t cbase = (uint64_t)ni * kPartMaxLeaders;
    if (status == kNodeAccepted) {
        // Stable scatter: exclusive prefix of this slot's count over the items.
        const uint32_t items = nd->items;
        const uint32_t per = (items + kScanGroups - 1u) / kScanGroups;
        const uint32_t i0 = g * per < items ? g * per : items;
        const uint32_t i1 = i0 + per < items ? i0 + per : items;
        uint32_t *col = a.item_counts + (uint64_t)nd->item_base * kPartMaxLeaders + t;
        uint32_t sum = 0u;
        if (t < nl) {
            for (uint32_t i = i0; i < i1; i += kScanBatch) {
                uint32_t v[kScanBatch];
#pragma unroll
                for (uint32_t u = 0; u < kScanBatch; ++u) v[u] = i + u < i1 ? col[(uint64_t)(i + u) * kPartMaxLeaders] : 0u;
#pragma unroll
                for (uint32_t u = 0; u < kScanBatch; ++u) sum += v[u];
            }
        }
        group_sum[g][t] = sum;
        __syncthreads();
        uint32_t run = 0u;
        for (uint32_t h = 0; h < g; ++h) run += group_sum[h][t];
        if (t < nl) {
            for (uint32_t i = i0; i < i1; i += kScanBatch) {
                uint32_t v[kScanBatch];
#pragma unroll
                for (uint32_t u = 0; u < kScanBatch; ++u) v[u] = i + u < i1 ? col[(uint64_t)(i + u) * kPartMaxLeaders] : 0u;
#pragma unroll
                for (uint32_t u = 0; u < kScanBatch; ++u) {
                    if (i + u < i1) col[(uint64_t)(i + u) * kPartMaxLeaders] = run;
                    run += v[u];
                }
            }
        }
    }
    if (threadIdx.x == 0) {
        // compute_backend.rs:15666-15718: children in slot order.
        uint32_t leaf_children = 0, node_children = 0;
        uint64_t leaf_rows = 0, node_rows = 0;
        bool stop = false;
        for (uint32_t s = 0; s < kPartMaxLeaders; ++s) {
            const uint32_t c = s < nl ? a.child_counts[cbase + s] : 0u;
            uint32_t idx = kChildEmpty;
            uint32_t rel = 0;
            if (c != 0u && !stop) {
                if (c <= a.leaf_max) {
                    idx = leaf_children++;
                    rel = (uint32_t)leaf_rows;
                    leaf_rows += c;
                } else if (nd->depth + 1u >= a.max_depth) {
                    pc_flag(a.counters, TESSA_OVF_OVERSIZED_TERMINAL_NODE);
                    stop = true;
                } else {
                    idx = kChildNodeBit | node_children++;
                    rel = (uint32_t)node_rows;
                    node_rows += c;
                }
            }
            a.child_idx[cbase + s] = idx;
            a.child_rel[cbase + s] = rel;
        }
        nd->leaf_children = leaf_children;
        nd->node_children = node_children;
        nd->leaf_rows = leaf_rows;
        nd->node_rows = node_rows;
        pc_add(a.counters, TESSA_P_ASSIGNMENT_PASSES, 1);
        pc_add(a.counters, TESSA_P_LARGE_NODE_SPLITS, 1);
    }
}

// ---- numbering of leaves and next-level nodes -------------------------------
__global__ __launch_bounds__(1024) void pub_scan_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    __shared__ uint64_t sh[1024];
    NodeDesc *nodes = a.nodes[cur];
    const uint32_t per = (level_nodes + 1023u) / 1024u;
    const uint32_t b = threadIdx.x * per;
    const uint32_t e = b + per < level_nodes ? b + per : level_nodes;
    auto live = [&](uint32_t i) { return nodes[i].status == kNodeAccepted || nodes[i].status == kNodeBalanced; };
    uint64_t lc = 0, lr = 0, nc = 0, nr = 0;
    for (uint32_t i = b; i < e; ++i)
        if (live(i)) {
            lc += nodes[i].leaf_children;
            lr += nodes[i].leaf_rows;
            nc += nodes[i].node_children;
            nr += nodes[i].node_rows;
        }
    uint64_t tlc, tlr, tnc, tnr;
    uint64_t blc = block_exclusive_scan(lc, sh, &tlc);
    uint64_t blr = block_exclusive_scan(lr, sh, &tlr);
    uint64_t bnc = block_exclusive_scan(nc, sh, &tnc);
    uint64_t bnr = block_exclusive_scan(nr, sh, &tnr);
    const uint64_t leaf0 = a.hdr->leaf_count, row0 = a.hdr->leaf_rows;
    for (uint32_t i = b; i < e; ++i) {
        nodes[i].leaf_base = leaf0 + blc;
        nodes[i].leaf_row_base = row0 + blr;
        nodes[i].node_base = bnc;
        nodes[i].node_row_base = bnr;
        if (live(i)) {
            blc += nodes[i].leaf_children;
            blr += nodes[i].leaf_rows;
            bnc += nodes[i].node_children;
            bnr += nodes[i].node_rows;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        LevelHeader *h = a.hdr;
        h->leaf_count = leaf0 + tlc;
        h->leaf_rows = row0 + tlr;
        h->next_nodes = (uint32_t)(tnc < 0xffffffffull ? tnc : 0xffffffffull);
        h->next_rows = tnr;
        // compute_backend.rs:11752-11760 leaf capacity; :12398-12403 queue.
        if (h->leaf_count > a.max_leaf_count) pc_flag(a.counters, TESSA_OVF_LEAF_DESC);
        if (h->leaf_rows > a.max_leaf_rows) pc_flag(a.counters, TESSA_OVF_LEAF_ROW);
        if (tnc > a.node_cap) pc_flag(a.counters, TESSA_OVF_QUEUE_NODE);
        if (tnr > a.arena_cap) pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
        a.counters[TESSA_P_OUTPUT_LEAF_COUNT] = h->leaf_count;
        a.counters[TESSA_P_OUTPUT_ROWS] = h->leaf_rows;
        h->overflow = atomicOr((unsigned long long *)&a.counters[TESSA_P_OVERFLOW_FLAGS], 0ull);
    }
}

// ---- SCATTER + PUBLISH (compute_backend.rs:15556-15727) ---------------------
__global__ __launch_bounds__(256) void scatter_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    __shared__ uint32_t s_node;
    __shared__ uint32_t cidx[kPartMaxLeaders];
    __shared__ uint32_t crel[kPartMaxLeaders];
    __shared__ uint32_t run[kPartMaxLeaders];
    __shared__ uint32_t wcnt[4][kPartMaxLeaders];
    __shared__ uint32_t wpre[4][kPartMaxLeaders];
    const uint32_t item = blockIdx.x;
    if (item >= a.hdr->items) return;
    if (a.counters[TESSA_P_OVERFLOW_FLAGS] != 0ull) return;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) s_node = find_item_node(a.nodes[cur], level_nodes, item);
    __syncthreads();
    const uint32_t ni = s_node;
    const NodeDesc *nd = a.nodes[cur] + ni;
    const uint32_t status = nd->status;
    if (status != kNodeAccepted && status != kNodeBalanced) return;
    const uint64_t cbase = (uint64_t)ni * kPartMaxLeaders;
    const uint32_t nl = nd->num_leaders;
    const uint32_t fanout = nd->fanout;
    const uint32_t n = nd->n;
    const uint32_t first = (item - nd->item_base) * kPartItemRows;
    const uint32_t rows_here = (n - first) < kPartItemRows ? (n - first) : kPartItemRows;
    const uint32_t *src = a.arena[cur] + nd->row_start;
    uint32_t *next_arena = a.arena[cur ^ 1u];
    if (tid < kPartMaxLeaders) {
        cidx[tid] = a.child_idx[cbase + tid];
        crel[tid] = a.child_rel[cbase + tid];
        run[tid] = (status == kNodeAccepted && tid < nl) ? a.item_counts[(uint64_t)item * kPartMaxLeaders + tid] : 0u;
    }
    __syncthreads();
    auto put = [&](uint32_t s, uint64_t pos, uint32_t row) {
        const uint32_t ci = cidx[s];
        if (ci == kChildEmpty) return;
        if (ci & kChildNodeBit) next_arena[nd->node_row_base + crel[s] + pos] = row;
        else a.leaf_row_ids[nd->leaf_row_base + crel[s] + pos] = row;
    };
    if (status == kNodeBalanced) {
        // even rows -> child 0, odd rows -> child 1, in row order
        for (uint32_t r = first + tid; r < first + rows_here; r += blockDim.x) put(r & 1u, r >> 1, src[r]);
    } else {
        const uint32_t wave = tid >> 6, lane = tid & 63u;
        const uint64_t lt = (1ull << lane) - 1ull;
        for (uint32_t round = 0; round < kPartItemRows / 256u; ++round) {
            const uint32_t r = first + round * 256u + tid;
            const bool valid = r < first + rows_here;
            const uint32_t packed = valid ? a.slots[nd->row_start + r] : 0xffffffffu;
            uint32_t my[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) my[k] = (valid && k < fanout) ? ((packed >> (8u * k)) & 0xffu) : 0xffu;
            for (uint32_t s = lane; s < kPartMaxLeaders; s += 64u) wcnt[wave][s] = 0u;
            __syncthreads();
            // Stable rank within the wave: one pass per distinct slot value.
            uint32_t rank[4] = {0u, 0u, 0u, 0u};
            uint64_t pend[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) pend[k] = __ballot(my[k] != 0xffu);
            while (true) {
                uint32_t k0 = 4u;
                uint64_t m0 = 0ull;
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k)
                    if (k0 == 4u && pend[k] != 0ull) {
                        k0 = k;
                        m0 = pend[k];
                    }
                if (k0 == 4u) break;
                const int lane0 = __ffsll((long long)m0) - 1;
                uint32_t v = my[0];
#pragma unroll
                for (uint32_t k = 1; k < 4; ++k)
                    if (k == k0) v = my[k];
                const uint32_t s0 = __shfl(v, lane0);
                uint64_t any = 0ull;
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    const uint64_t mk = __ballot(my[k] == s0);
                    any |= mk;
                    pend[k] &= ~mk;
                }
                const uint32_t before = (uint32_t)__popcll(any & lt);
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k)
                    if (my[k] == s0) rank[k] = before;
                if ((int)lane == lane0) wcnt[wave][s0] = (uint32_t)__popcll(any);
            }
            __syncthreads();
            if (tid < kPartMaxLeaders) {
                uint32_t acc = run[tid];
#pragma unroll
                for (uint32_t w = 0; w < 4; ++w) {
                    wpre[w][tid] = acc;
                    acc += wcnt[w][tid];
                }
                run[tid] = acc;
            }
            __syncthreads();
            if (valid) {
                const uint32_t row = src[r];
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k)
                    if (my[k] != 0xffu) put(my[k], (uint64_t)wpre[wave][my[k]] + rank[k], row);
            }
            __syncthreads();
        }
    }
    // The node's first item publishes its children (push_leaf / publish child).
    if (item == nd->item_base && tid < nl) {
        const uint32_t s = tid;
        const uint32_t ci = cidx[s];
        if (ci != kChildEmpty) {
            const uint32_t c = a.child_counts[cbase + s];
            if (ci & kChildNodeBit) {
                NodeDesc child{};
                child.row_start = nd->node_row_base + crel[s];
                child.n = c;
                child.depth = nd->depth + 1u;
                child.seed = nd->seed ^ ((uint64_t)s * 0x94d049bb133111ebull) ^ (((uint64_t)c) << 23);
                child.root_base = nd->root_base;
                child.root_index = nd->root_index;
                child.status = kNodeIdle;
                a.nodes[cur ^ 1u][nd->node_base + (ci & ~kChildNodeBit)] = child;
            } else {
                const uint64_t li = nd->leaf_base + ci;
                const uint64_t start = nd->leaf_row_base + crel[s];
                a.leaf_starts[li] = start;
                a.leaf_sizes[li] = c;
                a.leaf_sizes32[li] = c;
                a.leaf_out_offsets[li] = start * a.k;
                if (a.leaf_root) a.leaf_root[li] = nd->root_index;
                if (a.leaf_depth) a.leaf_depth[li] = nd->depth + 1u;
                pc_min(a.counters, TESSA_P_LEAF_SIZE_MIN, c);
                pc_max(a.counters, TESSA_P_LEAF_SIZE_MAX, c);
                pc_add(a.counters, TESSA_P_LEAF_SIZE_SUM, c);
                pc_add(a.counters, TESSA_P_LEAF_SIZE_COUNT, 1);
            }
        }
    }
}

// ---- small root (compute_backend.rs:12648-13078) -----------------------------
// A subtree root with n <= leaf_max rows (and n * fanout within the 4096-row
// small-node scratch) is split by gpu_persistent_process_node: hash-ranked
// leaders, up to 6 attempts, children below leaf_min merged.  Its rows are
// 0..n-1 (already sorted and unique), so every child is a set of row ids
// kept here as a 4096-bit bitmap, and sort_unique / merge become bitwise ORs.
constexpr int kSmallThreads = 1024;
constexpr uint32_t kSmallMaxRows = 4096;
constexpr uint32_t kSmallWords = kSmallMaxRows / 32;  // 128
constexpr size_t kSmallLdsBytes = kSmallMaxRows * 8                                  // keys
                                  + (size_t)kPartMaxLeaders * kSmallWords * 4;       // child bitmaps

__device__ void push_leaf_rows_from_bitmap(PartArgs &a, const uint32_t *bm, uint32_t size, uint64_t li,
                                           uint64_t start, uint32_t *wpref) {
    // rows in ascending order: prefix popcount over the 128 words
    const uint32_t t = threadIdx.x;
    if (t < kSmallWords) wpref[t] = __popc(bm[t]);
    __syncthreads();
    if (t == 0) {
        uint32_t acc = 0;
        for (uint32_t w = 0; w < kSmallWords; ++w) {
            const uint32_t c = wpref[w];
            wpref[w] = acc;
            acc += c;
        }
    }
    __syncthreads();
    if (t < kSmallWords) {
        uint32_t bits = bm[t];
        uint32_t pos = wpref[t];
        while (bits) {
            const uint32_t b = __ffs(bits) - 1u;
            bits &= bits - 1u;
            a.leaf_row_ids[start + pos++] = t * 32u + b;
        }
    }
    if (t == 0) {
        a.leaf_starts[li] = start;
        a.leaf_sizes[li] = size;
        a.leaf_sizes32[li] = size;
        a.leaf_out_offsets[li] = start * a.k;
        pc_min(a.counters, TESSA_P_LEAF_SIZE_MIN, size);
        pc_max(a.counters, TESSA_P_LEAF_SIZE_MAX, size);
        pc_add(a.counters, TESSA_P_LEAF_SIZE_SUM, size);
        pc_add(a.counters, TESSA_P_LEAF_SIZE_COUNT, 1);
    }
    __syncthreads();
}

__global__ __launch_bounds__(kSmallThreads) void small_root_kernel(PartArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint64_t *keys = reinterpret_cast<uint64_t *>(smem);
    uint32_t *bm = reinterpret_cast<uint32_t *>(smem + kSmallMaxRows * 8);  // [128][128]
    __shared__ uint32_t leaders[kPartMaxLeaders];
    __shared__ uint32_t child_cnt[kPartMaxLeaders + 1];
    __shared__ uint32_t wpref[kSmallWords];
    __shared__ uint32_t s_split, s_ok, s_stop;

    const uint32_t t = threadIdx.x;
    const uint32_t n = a.rows;  // root rows 0..n-1
    const uint32_t terminal = a.leaf_max;
    const uint32_t merge_min = a.leaf_min;
    const bool probe = a.fanout_second > 1u && n > 1u;  // relative depth 0
    if (t == 0) {
        pc_add(a.counters, TESSA_P_PARTITION_POPS, 1);
        pc_add(a.counters, TESSA_P_PARTITION_LEVEL_ROUNDS, 1);
        s_stop = 0u;
        if (n > a.small_node_limit || n > kSmallMaxRows) {
            pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
            s_stop = 1u;
        } else {
            pc_max(a.counters, TESSA_P_MAX_ACTIVE, n);
        }
    }
    __syncthreads();
    if (s_stop) return;
    // all rows as one bitmap (child slot 0)
    auto whole_leaf = [&]() {
        if (t < kSmallWords) {
            const uint32_t lo = t * 32u;
            bm[t] = lo >= n ? 0u : (n - lo >= 32u ? 0xffffffffu : ((1u << (n - lo)) - 1u));
        }
        __syncthreads();
        if (1ull > a.max_leaf_count || (uint64_t)n > a.max_leaf_rows) {
            if (t == 0) pc_flag(a.counters, 1ull > a.max_leaf_count ? TESSA_OVF_LEAF_DESC : TESSA_OVF_LEAF_ROW);
            return;
        }
        push_leaf_rows_from_bitmap(a, bm, n, 0, 0, wpref);
        if (t == 0) {
            a.hdr->leaf_count = 1;
            a.hdr->leaf_rows = n;
            a.counters[TESSA_P_OUTPUT_LEAF_COUNT] = 1;
            a.counters[TESSA_P_OUTPUT_ROWS] = n;
        }
    };
    if (!probe) {  // n <= terminal here
        whole_leaf();
        return;
    }
    if (a.root_depth >= a.max_depth) {
        if (t == 0) pc_flag(a.counters, TESSA_OVF_OVERSIZED_TERMINAL_NODE);
        return;
    }
    uint32_t max_leaders = a.max_leaders < n ? a.max_leaders : n;
    if (max_leaders < 2u) max_leaders = 2u;
    if (max_leaders > kPartMaxLeaders) {
        if (t == 0) pc_flag(a.counters, TESSA_OVF_LEADER);
        return;
    }
    const float psamp = adaptive_psamp(a.psamp, n, a.root_depth);
    const uint32_t base = base_leader_count(psamp, n, max_leaders);
    const bool use_root = a.root_leader_count > 0u;
    const uint32_t attempts = use_root ? 1u : 6u;
    uint32_t req = a.fanout_second;
    if (req > 4u) {
        if (t == 0) pc_flag(a.counters, TESSA_OVF_FANOUT_OVER_32);
        return;
    }
    const uint32_t pd = a.padded_dim;
    bool ok = false;
    uint32_t split = 0;
    for (uint32_t attempt = 0; attempt < attempts; ++attempt) {
        uint32_t nl = use_root ? a.root_leader_count : (base << attempt);
        if (nl > max_leaders) nl = max_leaders;
        if (use_root) {
            if (t < nl) leaders[t] = a.root_leaders[t];
        } else {
            // compute_backend.rs:12770-12800: the nl smallest (key, point)
            for (uint32_t i = t; i < n; i += kSmallThreads)
                keys[i] = hash64(a.seed ^ ((uint64_t)attempt * 0xbf58476d1ce4e5b9ull) ^
                                 (((uint64_t)a.root_depth) << 19) ^ (((uint64_t)i) << 7) ^ (((uint64_t)i) << 31));
            __syncthreads();
            for (uint32_t i = t; i < n; i += kSmallThreads) {
                const uint64_t ki = keys[i];
                uint32_t rank = 0;
                for (uint32_t jj = 0; jj < n; ++jj) {
                    const uint64_t kj = keys[jj];
                    rank += (kj < ki || (kj == ki && jj < i)) ? 1u : 0u;
                }
                if (rank < nl) leaders[rank] = i;
            }
        }
        const uint32_t fanout = req < nl ? req : nl;
        for (uint32_t w = t; w < nl * kSmallWords; w += kSmallThreads) bm[w] = 0u;
        if (t == 0) {
            pc_max(a.counters, TESSA_P_EFFECTIVE_ROOT_FANOUT, fanout);
            pc_max(a.counters, TESSA_P_EFFECTIVE_DEEPER_FANOUT, 1u);
        }
        __syncthreads();
        // assignment: one thread per row, leaders in slot order
        for (uint32_t i = t; i < n; i += kSmallThreads) {
            float bd[4] = {kEmptyDist, kEmptyDist, kEmptyDist, kEmptyDist};
            uint32_t bs[4] = {kEmptyId, kEmptyId, kEmptyId, kEmptyId};
            uint32_t bl[4] = {kEmptyId, kEmptyId, kEmptyId, kEmptyId};
            const int8_t *ci = a.codes + (uint64_t)i * pd;
            const float ps = a.scales[i], pn = a.norms[i];
            auto run = [&](auto fc) {
                constexpr int F = decltype(fc)::value;
                for (uint32_t s = 0; s < nl; ++s) {
                    const uint32_t l = leaders[s];
                    const int dot = dot_i8_rows(ci, a.codes + (uint64_t)l * pd, pd);
                    insert_slot<F>(assign_l2(dot, ps, pn, a.scales[l], a.norms[l]), i, l, s, bd, bs, bl);
                }
            };
            switch (fanout) {
                case 1: run(std::integral_constant<int, 1>{}); break;
                case 2: run(std::integral_constant<int, 2>{}); break;
                case 3: run(std::integral_constant<int, 3>{}); break;
                default: run(std::integral_constant<int, 4>{}); break;
            }
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                if (k < fanout && bs[k] < nl) atomicOr(&bm[bs[k] * kSmallWords + (i >> 5)], 1u << (i & 31u));
        }
        __syncthreads();
        if (t == 0) {
            pc_add(a.counters, TESSA_P_FANOUT_ASSIGNMENT_SLOTS, (uint64_t)n * fanout);
            pc_add(a.counters, TESSA_P_REPLICATED_ROWS, (uint64_t)n * fanout);
            pc_add(a.counters, TESSA_P_ASSIGNMENT_PASSES, 1);
            s_stop = (uint64_t)n * fanout > 4096ull ? 1u : 0u;
            if (s_stop) pc_flag(a.counters, TESSA_OVF_QUEUE_ROW);
        }
        __syncthreads();
        if (s_stop) return;
        // compute_backend.rs:12923-12996 children; wave 0, 2 bitmap words per lane
        if (t < 64) {
            uint32_t sm0 = 0u, sm1 = 0u, small_len = 0u, max_child = 0u, sp = 0u;
            auto wave_pop = [](uint32_t x0, uint32_t x1) {
                uint32_t c = __popc(x0) + __popc(x1);
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off);
                return c;
            };
            for (uint32_t s = 0; s < nl; ++s) {
                const uint32_t w0 = bm[s * kSmallWords + t], w1 = bm[s * kSmallWords + t + 64u];
                const uint32_t c = wave_pop(w0, w1);
                if (c == 0u) continue;
                if (c < merge_min) {
                    sm0 |= w0;
                    sm1 |= w1;
                    small_len = wave_pop(sm0, sm1);
                    if (small_len >= merge_min) {
                        bm[sp * kSmallWords + t] = sm0;
                        bm[sp * kSmallWords + t + 64u] = sm1;
                        if (t == 0) child_cnt[sp] = small_len;
                        max_child = small_len > max_child ? small_len : max_child;
                        ++sp;
                        sm0 = sm1 = 0u;
                        small_len = 0u;
                    }
                } else {
                    bm[sp * kSmallWords + t] = w0;
                    bm[sp * kSmallWords + t + 64u] = w1;
                    if (t == 0) child_cnt[sp] = c;
                    max_child = c > max_child ? c : max_child;
                    ++sp;
                }
            }
            if (small_len > 0u) {
                if (sp > 0u) {
                    const uint32_t last = sp - 1u;
                    const uint32_t last_count = __shfl(child_cnt[last], 0);
                    if (last_count + small_len <= terminal) {
                        const uint32_t m0 = bm[last * kSmallWords + t] | sm0;
                        const uint32_t m1 = bm[last * kSmallWords + t + 64u] | sm1;
                        bm[last * kSmallWords + t] = m0;
                        bm[last * kSmallWords + t + 64u] = m1;
                        const uint32_t mc = wave_pop(m0, m1);
                        if (t == 0) child_cnt[last] = mc;
                        max_child = mc > max_child ? mc : max_child;
                        small_len = 0u;
                    }
                }
                if (small_len > 0u) {
                    bm[sp * kSmallWords + t] = sm0;
                    bm[sp * kSmallWords + t + 64u] = sm1;
                    if (t == 0) child_cnt[sp] = small_len;
                    max_child = small_len > max_child ? small_len : max_child;
                    ++sp;
                }
            }
            if (t == 0) {
                s_split = sp;
                s_ok = (sp > 1u && meaningful_split(n, max_child, terminal)) ? 1u : 0u;
            }
        }
        __syncthreads();
        ok = s_ok != 0u;
        split = s_split;
        if (ok) break;
        if (nl >= max_leaders) break;
        __syncthreads();
    }
    if (!ok) {  // n <= terminal: the whole node is one leaf (:13000-13021)
        whole_leaf();
        return;
    }
    // Every child has <= n <= leaf_max rows, so all become leaves (:13023-13045).
    uint64_t rows_total = 0;
    for (uint32_t c = 0; c < split; ++c) rows_total += child_cnt[c];
    if ((uint64_t)split > a.max_leaf_count || rows_total > a.max_leaf_rows) {
        if (t == 0) pc_flag(a.counters, (uint64_t)split > a.max_leaf_count ? TESSA_OVF_LEAF_DESC : TESSA_OVF_LEAF_ROW);
        return;
    }
    uint64_t start = 0;
    for (uint32_t c = 0; c < split; ++c) {
        push_leaf_rows_from_bitmap(a, bm + c * kSmallWords, child_cnt[c], c, start, wpref);
        start += child_cnt[c];
    }
    if (t == 0) {
        a.hdr->leaf_count = split;
        a.hdr->leaf_rows = rows_total;
        a.counters[TESSA_P_OUTPUT_LEAF_COUNT] = split;
        a.counters[TESSA_P_OUTPUT_ROWS] = rows_total;
    }
}

template <int KS>
int launch_count_ks(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint32_t grid, hipStream_t s) {
    using L = CountLayout<KS>;
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute((const void *)count_kernel<KS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                L::kBytes) != hipSuccess)
            return -1;
        attr = true;
    }
    // persistent: at most two workgroups' worth of items per CU at a time
    const uint32_t g = grid < kCountGrid ? grid : kCountGrid;
    hipLaunchKernelGGL(count_kernel<KS>, dim3(g), dim3(L::kThreads), L::kBytes, s, a, cur, level_nodes);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_count(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint32_t grid, hipStream_t s) {
    const uint32_t ks = (a.padded_dim + 31) / 32;
    if (ks <= 4) return launch_count_ks<4>(a, cur, level_nodes, grid, s);
    if (ks <= 8) return launch_count_ks<8>(a, cur, level_nodes, grid, s);
    if (ks <= 12) return launch_count_ks<12>(a, cur, level_nodes, grid, s);
    if (ks <= 16) return launch_count_ks<16>(a, cur, level_nodes, grid, s);
    if (ks <= 24) return launch_count_ks<24>(a, cur, level_nodes, grid, s);
    if (ks <= 32) return launch_count_ks<32>(a, cur, level_nodes, grid, s);
    return -3;
}

}  // namespace

void partition_capacity(uint64_t rows, uint32_t famp, uint32_t leaf_max, uint64_t *arena_cap, uint32_t *node_cap,
                        uint64_t *item_cap) {
    const uint64_t ac = (rows ? rows : 1) * (famp ? famp : 1);
    // every next-level node holds more than leaf_max rows
    const uint64_t nc = ac / ((uint64_t)leaf_max + 1u) + 2u;
    *arena_cap = ac;
    *node_cap = (uint32_t)(nc < 0xffffffffull ? nc : 0xffffffffull);
    *item_cap = ac / kPartItemRows + nc + 1u;
}

// Copy the level's counting nodes (members and leaders, resident rows) to the
// host before a COUNT pass; every launch on `s` before it has completed.
static int capture_level(const PartArgs &a, hipStream_t s, uint32_t cur, uint32_t level_nodes, PartCapture *cap) {
    std::vector<NodeDesc> nodes(level_nodes);
    if (hipMemcpyAsync(nodes.data(), a.nodes[cur], level_nodes * sizeof(NodeDesc), hipMemcpyDeviceToHost, s) !=
            hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return -1;
    // First pass: the level's tasks and their row offsets, so the host
    // buffer is sized once before any copy into it is queued (a resize
    // between queued copies could move the buffer under them).
    auto wanted = [&](const NodeDesc &nd) {
        return nd.status == kNodeCounting && nd.n >= cap->min_members && nd.num_leaders != 0 &&
               nd.num_leaders <= kPartMaxLeaders;
    };
    const size_t first_task = cap->tasks.size();
    uint64_t total = cap->rows.size();
    std::vector<uint32_t> picked;  // node of each task recorded at this level
    for (uint32_t ni = 0; ni < level_nodes; ++ni) {
        const NodeDesc &nd = nodes[ni];
        if (!wanted(nd)) continue;
        if (total + nd.n + nd.num_leaders > cap->max_rows) {
            cap->dropped_tasks += 1;  // host memory bound reached: the pass is not recorded
            continue;
        }
        PartCaptureTask t{nd.depth, nd.attempt, nd.fanout, nd.n, nd.num_leaders, total, total + nd.n};
        total += (uint64_t)nd.n + nd.num_leaders;
        cap->tasks.push_back(t);
        picked.push_back(ni);
    }
    cap->rows.resize(total);
    for (size_t i = 0; i < picked.size(); ++i) {
        const uint32_t ni = picked[i];
        const NodeDesc &nd = nodes[ni];
        const PartCaptureTask &t = cap->tasks[first_task + i];
        if (hipMemcpyAsync(cap->rows.data() + t.member_offset, a.arena[cur] + nd.row_start, nd.n * 4ull,
                           hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipMemcpyAsync(cap->rows.data() + t.leader_offset, a.leaders + (uint64_t)ni * kPartMaxLeaders,
                           nd.num_leaders * 4ull, hipMemcpyDeviceToHost, s) != hipSuccess)
            return -1;
    }
    return hipStreamSynchronize(s) == hipSuccess ? 0 : -1;
}

// Level bound: the terminal-depth retry runs with max_depth up to 1024, so a
// tree may be that deep.
constexpr uint32_t kMaxLevels = 1100u;
static int run_levels(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture,
                      uint32_t level_nodes, uint64_t level_rows);

int run_partition(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture) {
    *res = PartResult{};
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return -1;
    auto read_header = [&]() -> int {
        if (hipMemcpyAsync(hh, a.hdr, sizeof(LevelHeader), hipMemcpyDeviceToHost, s) != hipSuccess) return -1;
        return hipStreamSynchronize(s) == hipSuccess ? 0 : -1;
    };
    if (a.rows == 0) return read_header();
    uint32_t level_nodes = 1;
    const uint64_t level_rows = a.rows;
    if (a.root_count > 0) {
        // every root is a large node (more than leaf_max rows, or a fanout
        // probe beyond the small-node scratch); the caller checked it
        if ((uint64_t)a.rows > a.arena_cap || a.root_count > a.node_cap) return -3;
        const uint64_t n = (uint64_t)a.rows > a.root_count ? a.rows : a.root_count;
        hipLaunchKernelGGL(multi_root_kernel, dim3((uint32_t)((n + 255u) / 256u)), dim3(256), 0, s, a);
        if (hipGetLastError() != hipSuccess) return -1;
        level_nodes = a.root_count;
        return run_levels(a, s, hh, res, capture, level_nodes, level_rows);
    }
    const bool probe = a.fanout_second > 1u && a.rows > 1u;
    const bool probe_overflow = probe && (uint64_t)a.rows * a.fanout_second > (uint64_t)a.small_node_limit;
    if (a.rows <= a.leaf_max && !probe_overflow) {
        static bool attr = false;
        if (!attr) {
            if (hipFuncSetAttribute((const void *)small_root_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)kSmallLdsBytes) != hipSuccess)
                return -1;
            attr = true;
        }
        hipLaunchKernelGGL(small_root_kernel, dim3(1), dim3(kSmallThreads), kSmallLdsBytes, s, a);
        if (hipGetLastError() != hipSuccess) return -1;
        res->levels = 1;
        if (read_header()) return -1;
        res->leaf_count = hh->leaf_count;
        res->leaf_rows = hh->leaf_rows;
        return 0;
    }
    if ((uint64_t)a.rows > a.arena_cap) return -3;
    hipLaunchKernelGGL(root_kernel, dim3((a.rows + 255u) / 256u), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return -1;
    return run_levels(a, s, hh, res, capture, level_nodes, level_rows);
}

// The level loop from the nodes of level 0 (in the first arena).
static int run_levels(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture,
                      uint32_t level_nodes, uint64_t level_rows) {
    auto read_header = [&]() -> int {
        if (hipMemcpyAsync(hh, a.hdr, sizeof(LevelHeader), hipMemcpyDeviceToHost, s) != hipSuccess) return -1;
        return hipStreamSynchronize(s) == hipSuccess ? 0 : -1;
    };
    uint32_t cur = 0;
    for (uint32_t level = 0; level < kMaxLevels; ++level) {
        const uint64_t items_bound = level_rows / kPartItemRows + level_nodes + 1u;
        if (items_bound > a.item_cap || items_bound > 0x7fffffffull) return -3;
        const uint32_t grid = (uint32_t)items_bound;
        hipLaunchKernelGGL(stage_kernel, dim3(level_nodes), dim3(128), 0, s, a, cur, level_nodes);
        hipLaunchKernelGGL(item_plan_kernel, dim3(1), dim3(1024), 0, s, a, cur, level_nodes);
        if (hipGetLastError() != hipSuccess) return -1;
        uint32_t attempt = 0;
        for (; attempt < 16u; ++attempt) {
            if (capture && capture_level(a, s, cur, level_nodes, capture)) return -1;
            if (launch_count(a, cur, level_nodes, grid, s)) return -1;
            res->count_launches += 1;
            hipLaunchKernelGGL(emit_kernel, dim3(level_nodes), dim3(128), 0, s, a, cur, level_nodes);
            if (hipGetLastError() != hipSuccess) return -1;
            if (read_header()) return -1;
            if (hh->retry_nodes == 0u) break;
            hipLaunchKernelGGL(reset_retry_kernel, dim3(1), dim3(1), 0, s, a.hdr);
        }
        if (attempt == 16u) return -2;
        hipLaunchKernelGGL(node_scan_kernel, dim3(level_nodes), dim3(kScanGroups * kPartMaxLeaders), 0, s, a, cur,
                           level_nodes);
        hipLaunchKernelGGL(pub_scan_kernel, dim3(1), dim3(1024), 0, s, a, cur, level_nodes);
        hipLaunchKernelGGL(scatter_kernel, dim3(grid), dim3(256), 0, s, a, cur, level_nodes);
        if (hipGetLastError() != hipSuccess) return -1;
        if (read_header()) return -1;
        res->levels = level + 1u;
        res->leaf_count = hh->leaf_count;
        res->leaf_rows = hh->leaf_rows;
        if (hh->overflow != 0ull) return 0;
        level_nodes = hh->next_nodes;
        level_rows = hh->next_rows;
        cur ^= 1u;
        if (level_nodes == 0u) return 0;
    }
    return -2;
}

}  // namespace tessa
