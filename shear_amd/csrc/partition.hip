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

#include "kernel_attr.h"
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
// One node per wave: lane 0 takes the node's split parameters, the lanes
// write its 128 leader words.
__device__ __forceinline__ void stage_node_wave(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint32_t ni) {
    const uint32_t lane = threadIdx.x & 63u;
    NodeDesc *nd = a.nodes[cur] + ni;
    uint32_t s_nl = 0u, s_use_root = 0u;
    if (lane == 0u) {
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
    const uint32_t nl = __shfl(s_nl, 0);
    const uint32_t use_root = __shfl(s_use_root, 0);
    for (uint32_t t = lane; t < kPartMaxLeaders; t += 64u) {
        uint32_t leader = 0u;
        if (t < nl) {
            if (use_root) {
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
}

__global__ __launch_bounds__(64) void stage_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    stage_node_wave(a, cur, level_nodes, blockIdx.x);
}

// ---- item plan ---------------------------------------------------------------
// One block of any power-of-two size; sh holds blockDim.x words.
__device__ __forceinline__ void item_plan_block(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint64_t *sh) {
    NodeDesc *nodes = a.nodes[cur];
    const uint32_t per = (level_nodes + blockDim.x - 1u) / blockDim.x;
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
    __syncthreads();
}

__global__ __launch_bounds__(1024) void item_plan_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    __shared__ uint64_t sh[1024];
    item_plan_block(a, cur, level_nodes, sh);
}

// The level's item -> node map, one node per wave (items past the planned
// total are never listed).
__device__ __forceinline__ void item_map_wave(const PartArgs &a, uint32_t cur, uint32_t ni) {
    const NodeDesc *nd = a.nodes[cur] + ni;
    const uint32_t total = a.hdr->items;
    const uint32_t base = nd->item_base, items = nd->items;
    for (uint32_t it = threadIdx.x & 63u; it < items; it += 64u)
        if (base + it < total) a.item_node[base + it] = ni;
}

__global__ __launch_bounds__(64) void item_map_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    item_map_wave(a, cur, blockIdx.x);
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

// v[c] for a wave-uniform c, by selects (the array stays in registers)
template <int N>
__device__ __forceinline__ uint32_t pick(const uint32_t (&v)[N], int c) {
    uint32_t r = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) r = c == i ? v[i] : r;
    return r;
}

// A row's F slots are empty when its first leader tile starts, so in-order
// insertion would visit every leader of that tile.  Let T be the row's F-th
// smallest distance in the tile.  When no distance lies above T by at most
// the tie band, a leader above T is after every leader at or below T under
// assign_before, in both directions (the rounded difference only grows as
// the smaller distance falls).  Such a leader then only ever sits behind
// those leaders in the slots and never moves one of them, and at least F of
// them fill the slots by the tile's end.  Inserting only the leaders at or
// below T, in slot order, leaves the same slots.
// `dl` holds the lane's 16 distances of the tile (kEmptyDist past the node's
// leaders) and `all` the lane's half of the full visit mask.  Returns the
// lane's half of the visit mask: the leaders at or below T, or `all` when a
// distance of the row lies in the band, is NaN, or fewer than F are finite.
// Both lanes of a row return masks of the same choice.
template <int F>
__device__ __forceinline__ uint32_t first_tile_visits(const float (&dl)[16], uint32_t h, uint32_t all) {
    float s[F];  // smallest distances seen, ascending
#pragma unroll
    for (int k = 0; k < F; ++k) s[k] = kEmptyDist;
    auto push = [&](float x) {
#pragma unroll
        for (int k = 0; k < F; ++k) {
            const float lo = fminf(s[k], x);
            if (k + 1 < F) x = fmaxf(s[k], x);
            s[k] = lo;
        }
    };
#pragma unroll
    for (int v = 0; v < 16; ++v) push(dl[v]);
    float o[F];  // the other lane's smallest, for the row's 32 leaders
#pragma unroll
    for (int k = 0; k < F; ++k) o[k] = __shfl_xor(s[k], 32);
#pragma unroll
    for (int k = 0; k < F; ++k) push(o[k]);
    const float T = s[F - 1];
    uint32_t near = 0u;
    bool band = !(T < kEmptyDist);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const uint32_t li = 8u * (v / 4) + 4u * h + (v % 4);
        if (dl[v] <= T) near |= 1u << li;
        else if (!(__fsub_rn(dl[v], T) > kTieEps)) band = true;
    }
    // every lane takes part in the exchange (a lane left out of it hands its
    // partner no value)
    const int other_band = __shfl_xor(band ? 1 : 0, 32);
    return band || other_band != 0 ? all : near;
}

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
// One COUNT pass over the level's items first_item, + stride, ...; `smem` is
// the CountLayout<KS> buffer and `s_node` a shared word.  The block has
// CountLayout<KS>::kThreads threads.
template <int KS>
__device__ __forceinline__ void count_items(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint32_t first_item,
                            uint32_t stride, unsigned char *smem, uint32_t *s_node_ptr) {
    using L = CountLayout<KS>;
    constexpr uint32_t kThr = L::kThreads;
    uint32_t &s_node = *s_node_ptr;
    int8_t *lcodes = reinterpret_cast<int8_t *>(smem);
    float *ls = reinterpret_cast<float *>(smem + L::kMetaOff);
    float *ln = ls + kPartMaxLeaders;
    uint32_t *lid = reinterpret_cast<uint32_t *>(ln + kPartMaxLeaders);
    uint32_t *cnt = reinterpret_cast<uint32_t *>(smem + L::kCntOff);
    float *dbuf = reinterpret_cast<float *>(smem + L::kDistOff);

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
    for (uint32_t item = first_item; item < items; item += stride) {
        if (tid == 0) s_node = a.item_node[item];
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
        // The row ids and SQ8 rows of all the item's chunks are read before
        // its first chunk computes, and a chunk's codes, scales and norms are
        // requested as soon as the chunk before it has issued its last MFMA:
        // that chunk's insertion covers their latency.
        uint32_t cpt[L::kChunks], cspt[L::kChunks];
        uint32_t okbits = 0u;  // bit c: the lane's row of chunk c is valid
#pragma unroll
        for (int c = 0; c < L::kChunks; ++c) {
            const uint32_t m = first + c * L::kChunk + wave * 32u + j;
            cpt[c] = m < n ? arena[row_start + m] : rb;
        }
#pragma unroll
        for (int c = 0; c < L::kChunks; ++c) {
            const uint32_t m = first + c * L::kChunk + wave * 32u + j;
            bool ok = m < n;
            if (ok && cpt[c] >= a.rows) {
                pc_flag(a.counters, TESSA_OVF_INVALID_ASSIGN_POINT_ID);
                ok = false;
                cpt[c] = rb;
            }
            okbits |= ok ? 1u << c : 0u;
            cspt[c] = rmap ? rmap[cpt[c]] : cpt[c];
        }
        v4i bfrag[KS];
        float nps = 0.0f, npn = 0.0f;  // scale and norm of the lane's row in bfrag
        auto load_chunk = [&](int c) {
            const bool ok = (okbits >> c) & 1u;
            const uint32_t spt = pick(cspt, c);
            const int8_t *mc = a.codes + (uint64_t)spt * pd;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const uint32_t off = 32u * s + 16u * h;
                v4i z = {0, 0, 0, 0};
                if (ok && off < pd) z = *reinterpret_cast<const v4i *>(mc + off);
                bfrag[s] = z;
            }
            nps = ok ? a.scales[spt] : 0.0f;
            npn = ok ? a.norms[spt] : 0.0f;
        };
        int loaded = -1;  // chunk whose rows bfrag holds (wave-uniform)
        for (int ch = 0; ch < L::kChunks; ++ch) {
            if (first + ch * L::kChunk >= n) break;  // uniform across the block
            const uint32_t m = first + ch * L::kChunk + wave * 32u + j;
            const bool ok = (okbits >> ch) & 1u;
            if (__ballot(ok) == 0ull) continue;  // this wave's rows are past the node's end
            if (loaded != ch) load_chunk(ch);
            const float ps = nps;
            const float pn = npn;
            const uint32_t lpt = pick(cpt, ch) - rb;  // the row's index within its root
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
                if (t + 1 == ntiles && ch + 1 < L::kChunks) {
                    load_chunk(ch + 1);
                    loaded = ch + 1;
                }
                // the lane's 16 leaders are 4 runs of 4 (8g + 4h + e): their
                // scales and norms in 8 vector reads, then every distance
                float4 lsv[4], lnv[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    lsv[g] = *reinterpret_cast<const float4 *>(ls + 32u * t + 8u * g + 4u * h);
                    lnv[g] = *reinterpret_cast<const float4 *>(ln + 32u * t + 8u * g + 4u * h);
                }
                // The row's last live slot as the tile starts (both lanes of
                // the row hold the same slots).  A leader whose distance lies more than
                // the tie band above it is not assign_before it, nor before
                // any smaller last slot, so its insertion changes nothing
                // while the last slot stays at or below it.  Only the other
                // leaders are visited, in slot order; if an insertion ever
                // raises the last slot (a tie resolved by the hash key can
                // leave a slot up to the band above the next), every later
                // leader of the tile is visited.
                const int fl = (fanout < 4u ? (int)fanout : 4) - 1;
                const float last = fl == 0 ? bd[0] : fl == 1 ? bd[1] : fl == 2 ? bd[2] : bd[3];
                uint32_t visit = 0u;
                float dl[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t li = 8u * (v / 4) + 4u * h + (v % 4);  // leader within the tile
                    const uint32_t gl = 32u * t + li;
                    const int e = v % 4, g = v / 4;
                    const float lsc = e == 0 ? lsv[g].x : e == 1 ? lsv[g].y : e == 2 ? lsv[g].z : lsv[g].w;
                    const float lno = e == 0 ? lnv[g].x : e == 1 ? lnv[g].y : e == 2 ? lnv[g].z : lnv[g].w;
                    const float d = assign_l2(acc[v], ps, pn, lsc, lno);
                    dl[v] = gl < nl ? d : kEmptyDist;
                    wb[li * 33 + j] = dl[v];
                    if (gl < nl && !(__fsub_rn(d, last) > kTieEps)) visit |= 1u << li;
                }
                if (t == 0u) {  // the slots are empty
                    switch (fanout) {
                        case 1: visit = first_tile_visits<1>(dl, h, visit); break;
                        case 2: visit = first_tile_visits<2>(dl, h, visit); break;
                        case 3: visit = first_tile_visits<3>(dl, h, visit); break;
                        default: visit = first_tile_visits<4>(dl, h, visit); break;
                    }
                }
                visit |= __shfl_xor(visit, 32);  // the row's other half of the tile's leaders
                wave_lds_sync();
                if (ok) {  // both lanes of a row insert: each keeps the row's slots
                    const uint32_t lim = (nl - 32u * t) < 32u ? (nl - 32u * t) : 32u;
                    const uint32_t in_tile = lim >= 32u ? ~0u : (1u << lim) - 1u;
                    auto run = [&](auto fc) {
                        constexpr int F = decltype(fc)::value;
                        float bound = last;
                        uint32_t mask = visit;
                        while (mask != 0u) {
                            const uint32_t q = (uint32_t)__builtin_ctz(mask);
                            mask &= mask - 1u;
                            insert_slot<F>(wb[q * 33 + j], lpt, lid[32u * t + q], 32u * t + q, bd, bs, bl);
                            if (bd[F - 1] > bound) {
                                mask |= in_tile & (q >= 31u ? 0u : ~0u << (q + 1u));
                                bound = kEmptyDist;
                            }
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

template <int KS>
__global__ __launch_bounds__(CountLayout<KS>::kThreads, 1) void count_kernel(PartArgs a, uint32_t cur,
                                                                             uint32_t level_nodes) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ uint32_t s_node;
    count_items<KS>(a, cur, level_nodes, blockIdx.x, gridDim.x, smem, &s_node);
}

// ---- EMIT (compute_backend.rs:15396-15555) -----------------------------------
// One node per wave; a retry adds 1 to *retry_ctr.  Lane l holds slots l
// and l + 64; lane 0 decides.
__device__ __forceinline__ void emit_node_wave(const PartArgs &a, uint32_t cur, uint32_t ni, uint32_t *retry_ctr) {
    const uint32_t lane = threadIdx.x & 63u;
    NodeDesc *nd = a.nodes[cur] + ni;
    if (nd->status != kNodeCounting) return;  // one word, read by the whole wave
    const uint32_t nl = nd->num_leaders;
    const uint32_t n = nd->n;
    uint32_t *counts = a.child_counts + (uint64_t)ni * kPartMaxLeaders;
    const uint32_t c0 = lane < nl ? counts[lane] : 0u;
    const uint32_t c1 = lane + 64u < nl ? counts[lane + 64u] : 0u;
    uint64_t sum = (uint64_t)c0 + c1;
    uint32_t ne = (c0 ? 1u : 0u) + (c1 ? 1u : 0u), mx = c0 > c1 ? c0 : c1;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        sum += __shfl_xor(sum, off);
        ne += __shfl_xor(ne, off);
        const uint32_t o = __shfl_xor(mx, off);
        mx = o > mx ? o : mx;
    }
    uint32_t act = 0u, s_next = 0u, s_attempt = 0u;
    if (lane == 0u) {
        const uint64_t running = sum;
        const uint32_t nonempty = ne;
        const uint32_t max_child = mx;
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
            act = 1u;
            s_next = next;
            s_attempt = nd->attempt;
            pc_add(a.counters, TESSA_P_LARGE_SPLIT_RETRIES, 1);
            atomicAdd(retry_ctr, 1u);
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
    if (__shfl(act, 0) == 1u) {
        // compute_backend.rs:5991-6019 hash-sampled retry leaders, one per span.
        const uint32_t next = __shfl(s_next, 0);
        const uint32_t attempt = __shfl(s_attempt, 0);
        const uint64_t seed = nd->seed;
        const uint64_t row_start = nd->row_start;
        for (uint32_t t = lane; t < kPartMaxLeaders; t += 64u) {
            uint32_t leader = 0u;
            if (t < next) {
                uint32_t b = (uint32_t)(((uint64_t)t * n) / next);
                uint32_t e = (uint32_t)(((uint64_t)(t + 1u) * n) / next);
                if (e <= b) e = b + 1u;
                const uint32_t span = e - b;
                const uint64_t key = hash64(seed ^ ((uint64_t)attempt * 0xd6e8feb86659fd93ull) ^
                                            ((uint64_t)t * 0x9e3779b97f4a7c15ull));
                leader = a.arena[cur][row_start + b + (uint32_t)(key % span)];
            }
            a.leaders[(uint64_t)ni * kPartMaxLeaders + t] = leader;
            counts[t] = 0u;
        }
    }
}

__global__ __launch_bounds__(64) void emit_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    emit_node_wave(a, cur, blockIdx.x, &a.hdr->retry_nodes);
}

// ---- child layout and per-item prefixes ----------------------------------
// Stable scatter needs, per item and slot, the exclusive prefix of the
// slot's count over the node's earlier items.  A node with many items is
// scanned by a whole workgroup: groups of 128 threads (one thread per leader
// slot) split its items into ranges, each group sums its range, the groups'
// sums are scanned in LDS, then each group writes the prefixes of its range.
// A node with few items is scanned by one wave (lane l owns slots l and
// l + 64).  Item counts are read 16 items at a time, so the loads of a batch
// are in flight together.
constexpr uint32_t kScanGroups = 8;
constexpr uint32_t kScanBatch = 16;
constexpr uint32_t kWaveScanItems = 16;  // nodes with at most this many items: one wave

__device__ __forceinline__ void node_item_prefix_block(const PartArgs &a, const NodeDesc *nd, uint32_t nl,
                                       uint32_t (*group_sum)[kPartMaxLeaders]) {
    const uint32_t groups = blockDim.x / kPartMaxLeaders;
    const uint32_t t = threadIdx.x % kPartMaxLeaders;
    const uint32_t g = threadIdx.x / kPartMaxLeaders;
    const uint32_t items = nd->items;
    const uint32_t per = (items + groups - 1u) / groups;
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
    __syncthreads();  // group_sum is reused by the next node
}

__device__ __forceinline__ void node_item_prefix_wave(const PartArgs &a, const NodeDesc *nd, uint32_t nl) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t items = nd->items;
    uint32_t *col = a.item_counts + (uint64_t)nd->item_base * kPartMaxLeaders + lane;
    const bool live0 = lane < nl, live1 = lane + 64u < nl;
    uint32_t run0 = 0u, run1 = 0u;
    for (uint32_t i = 0; i < items; i += kScanBatch) {
        uint32_t v0[kScanBatch], v1[kScanBatch];
#pragma unroll
        for (uint32_t u = 0; u < kScanBatch; ++u) {
            const bool in = i + u < items;
            v0[u] = (in && live0) ? col[(uint64_t)(i + u) * kPartMaxLeaders] : 0u;
            v1[u] = (in && live1) ? col[(uint64_t)(i + u) * kPartMaxLeaders + 64u] : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kScanBatch; ++u) {
            if (i + u < items) {
                if (live0) col[(uint64_t)(i + u) * kPartMaxLeaders] = run0;
                if (live1) col[(uint64_t)(i + u) * kPartMaxLeaders + 64u] = run1;
            }
            run0 += v0[u];
            run1 += v1[u];
        }
    }
}

// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const uint64_t y = __shfl_up(v, off);
        v += lane >= off ? y : 0ull;
    }
    return v;
}

// compute_backend.rs:15666-15718: children in slot order, one wave.  A child
// of more than leaf_max rows at the depth limit flags OVERSIZED_TERMINAL_NODE
// and, with every later slot, gets no child.  Slot s = lane + 64 h.
__device__ __forceinline__ void node_layout_wave(const PartArgs &a, NodeDesc *nd, uint32_t ni) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nl = nd->num_leaders;
    const uint64_t cbase = (uint64_t)ni * kPartMaxLeaders;
    const bool terminal = nd->depth + 1u >= a.max_depth;
    uint32_t c[2];
    uint32_t kind[2];  // 0 empty, 1 leaf, 2 next-level node, 3 oversized at the depth limit
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t sl = lane + 64u * h;
        c[h] = sl < nl ? a.child_counts[cbase + sl] : 0u;
        kind[h] = c[h] == 0u ? 0u : (c[h] <= a.leaf_max ? 1u : (terminal ? 3u : 2u));
    }
    const uint64_t ovf0 = __ballot(kind[0] == 3u), ovf1 = __ballot(kind[1] == 3u);
    const uint32_t first_ovf = ovf0 ? (uint32_t)__builtin_ctzll(ovf0)
                                    : (ovf1 ? 64u + (uint32_t)__builtin_ctzll(ovf1) : kPartMaxLeaders);
    uint64_t leaf_base = 0ull, leaf_rows_base = 0ull, node_base = 0ull, node_rows_base = 0ull;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t sl = lane + 64u * h;
        const bool alive = sl < first_ovf;
        const bool leaf = alive && kind[h] == 1u;
        const bool node = alive && kind[h] == 2u;
        const uint64_t il = wave_incl_scan(leaf ? 1ull : 0ull);
        const uint64_t rl = wave_incl_scan(leaf ? c[h] : 0ull);
        const uint64_t in_ = wave_incl_scan(node ? 1ull : 0ull);
        const uint64_t rn = wave_incl_scan(node ? c[h] : 0ull);
        uint32_t idx = kChildEmpty, rel = 0u;
        if (leaf) {
            idx = (uint32_t)(leaf_base + il - 1ull);
            rel = (uint32_t)(leaf_rows_base + rl - c[h]);
        } else if (node) {
            idx = kChildNodeBit | (uint32_t)(node_base + in_ - 1ull);
            rel = (uint32_t)(node_rows_base + rn - c[h]);
        }
        a.child_idx[cbase + sl] = idx;
        a.child_rel[cbase + sl] = rel;
        leaf_base += __shfl(il, 63);
        leaf_rows_base += __shfl(rl, 63);
        node_base += __shfl(in_, 63);
        node_rows_base += __shfl(rn, 63);
    }
    if (lane == 0u) {
        if (first_ovf < kPartMaxLeaders) pc_flag(a.counters, TESSA_OVF_OVERSIZED_TERMINAL_NODE);
        nd->leaf_children = (uint32_t)leaf_base;
        nd->node_children = (uint32_t)node_base;
        nd->leaf_rows = leaf_rows_base;
        nd->node_rows = node_rows_base;
        pc_add(a.counters, TESSA_P_ASSIGNMENT_PASSES, 1);
        pc_add(a.counters, TESSA_P_LARGE_NODE_SPLITS, 1);
    }
}

__device__ __forceinline__ bool node_split(uint32_t status) {
    return status == kNodeAccepted || status == kNodeBalanced;
}

// One node, a whole workgroup (a multiple of 128 threads, at most
// kScanGroups x 128); group_sum holds kScanGroups x 128 words.
__device__ __forceinline__ void node_scan_block(const PartArgs &a, uint32_t cur, uint32_t ni, uint32_t (*group_sum)[kPartMaxLeaders]) {
    NodeDesc *nd = a.nodes[cur] + ni;
    const uint32_t status = nd->status;
    if (!node_split(status)) return;
    if (status == kNodeAccepted) node_item_prefix_block(a, nd, nd->num_leaders, group_sum);
    if (threadIdx.x < 64u) node_layout_wave(a, nd, ni);
}

// One node, one wave.
__device__ __forceinline__ void node_scan_wave(const PartArgs &a, uint32_t cur, uint32_t ni) {
    NodeDesc *nd = a.nodes[cur] + ni;
    const uint32_t status = nd->status;
    if (!node_split(status)) return;
    if (status == kNodeAccepted) node_item_prefix_wave(a, nd, nd->num_leaders);
    node_layout_wave(a, nd, ni);
}

__global__ __launch_bounds__(kScanGroups * kPartMaxLeaders) void node_scan_kernel(PartArgs a, uint32_t cur,
                                                                                 uint32_t level_nodes) {
    __shared__ uint32_t group_sum[kScanGroups][kPartMaxLeaders];
    node_scan_block(a, cur, blockIdx.x, group_sum);
}

// ---- numbering of leaves and next-level nodes -------------------------------
// One block of any power-of-two size; sh holds blockDim.x words.
__device__ __forceinline__ void pub_scan_block(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint64_t *sh) {
    NodeDesc *nodes = a.nodes[cur];
    const uint32_t per = (level_nodes + blockDim.x - 1u) / blockDim.x;
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
    __syncthreads();
}

__global__ __launch_bounds__(1024) void pub_scan_kernel(PartArgs a, uint32_t cur, uint32_t level_nodes) {
    __shared__ uint64_t sh[1024];
    pub_scan_block(a, cur, level_nodes, sh);
}

// ---- SCATTER + PUBLISH (compute_backend.rs:15556-15727) ---------------------
// One item per wave.  The item's rows go to their children in row order, in
// rounds of 64 rows.  Inside a round a row's rank among the rows bound for
// the same child comes from a bit-sliced match: per fanout entry, one ballot
// per bit of the 7-bit slot number, so lanes holding the same slot are found
// with a fixed number of ballots however many slots the round touches.  The
// wave keeps each slot's child index, child row offset and running position
// (from the item's prefix) in its own 1.5 KB of LDS.  The node's first item
// publishes its children.
constexpr uint32_t kScatterWaveWords = 3 * kPartMaxLeaders;  // per-wave LDS: child idx, child rel, running position

__device__ __forceinline__ void scatter_item_wave(const PartArgs &a, uint32_t cur, uint32_t item, uint32_t ni,
                                                  uint32_t *wl) {
    const uint32_t lane = threadIdx.x & 63u;
    const NodeDesc *nd = a.nodes[cur] + ni;
    const uint32_t status = nd->status;
    if (!node_split(status)) return;
    const uint64_t cbase = (uint64_t)ni * kPartMaxLeaders;
    const uint32_t nl = nd->num_leaders;
    const uint32_t fanout = nd->fanout;
    const uint32_t n = nd->n;
    const uint32_t first = (item - nd->item_base) * kPartItemRows;
    const uint32_t rows_here = (n - first) < kPartItemRows ? (n - first) : kPartItemRows;
    const uint64_t row_start = nd->row_start;
    const uint32_t *src = a.arena[cur] + row_start;
    uint32_t *next_arena = a.arena[cur ^ 1u];
    const uint64_t node_row_base = nd->node_row_base, leaf_row_base = nd->leaf_row_base;
    const bool counted = status == kNodeAccepted;
    uint32_t *w_idx = wl, *w_rel = wl + kPartMaxLeaders, *w_run = wl + 2 * kPartMaxLeaders;
    // the lane's two slots
    const uint32_t ci0 = a.child_idx[cbase + lane], ci1 = a.child_idx[cbase + lane + 64u];
    const uint32_t cr0 = a.child_rel[cbase + lane], cr1 = a.child_rel[cbase + lane + 64u];
    const uint32_t run0 = (counted && lane < nl) ? a.item_counts[(uint64_t)item * kPartMaxLeaders + lane] : 0u;
    const uint32_t run1 =
        (counted && lane + 64u < nl) ? a.item_counts[(uint64_t)item * kPartMaxLeaders + lane + 64u] : 0u;
    wave_lds_sync();  // the previous item's reads of wl are done
    w_idx[lane] = ci0;
    w_idx[lane + 64u] = ci1;
    w_rel[lane] = cr0;
    w_rel[lane + 64u] = cr1;
    w_run[lane] = run0;
    w_run[lane + 64u] = run1;
    wave_lds_sync();
    auto put = [&](uint32_t s, uint64_t pos, uint32_t row) {
        const uint32_t ci = w_idx[s];
        if (ci == kChildEmpty) return;
        if (ci & kChildNodeBit) next_arena[node_row_base + w_rel[s] + pos] = row;
        else a.leaf_row_ids[leaf_row_base + w_rel[s] + pos] = row;
    };
    if (!counted) {
        // balanced: even rows -> child 0, odd rows -> child 1, in row order
        for (uint32_t r = first + lane; r < first + rows_here; r += 64u) put(r & 1u, r >> 1, src[r]);
    } else {
        const uint64_t lt = (1ull << lane) - 1ull;
        // every round's slot word and row requested before the first round
        constexpr uint32_t kRounds = kPartItemRows / 64u;
        uint32_t pk[kRounds], rw[kRounds];
#pragma unroll
        for (uint32_t q = 0; q < kRounds; ++q) {
            const uint32_t r = first + q * 64u + lane;
            const bool valid = q * 64u + lane < rows_here;
            pk[q] = valid ? a.slots[row_start + r] : 0xffffffffu;
            rw[q] = valid ? src[r] : 0u;
        }
#pragma unroll
        for (uint32_t q = 0; q < kRounds; ++q) {
            if (q * 64u >= rows_here) break;
            const bool valid = q * 64u + lane < rows_here;
            uint32_t my[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) my[k] = (valid && k < fanout) ? ((pk[q] >> (8u * k)) & 0xffu) : 0xffu;
            // bit planes of every fanout entry's slot number (a lane's slots
            // are distinct leaders, so a lane matches a slot at most once)
            uint64_t live[4], plane[4][7];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                live[k] = __ballot(my[k] != 0xffu);
#pragma unroll
                for (uint32_t b = 0; b < 7u; ++b) plane[k][b] = __ballot((my[k] >> b) & 1u);
            }
            uint32_t pos[4], grow[4];
            bool lead[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                const uint32_t v = my[k] == 0xffu ? 0u : my[k];
                uint64_t same = 0ull;  // lanes holding slot v in any entry
#pragma unroll
                for (uint32_t k2 = 0; k2 < 4; ++k2) {
                    uint64_t m = live[k2];
#pragma unroll
                    for (uint32_t b = 0; b < 7u; ++b) m &= ((v >> b) & 1u) ? plane[k2][b] : ~plane[k2][b];
                    same |= m;
                }
                const uint64_t below = same & lt;
                const uint32_t base = my[k] != 0xffu ? w_run[v] : 0u;
                pos[k] = base + (uint32_t)__popcll(below);
                lead[k] = my[k] != 0xffu && below == 0ull;  // the slot's first lane advances its position
                grow[k] = base + (uint32_t)__popcll(same);
            }
            wave_lds_sync();  // every lane has read its bases
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                if (lead[k]) w_run[my[k]] = grow[k];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                if (my[k] != 0xffu) put(my[k], pos[k], rw[q]);
            wave_lds_sync();  // the advanced positions are seen by the next round
        }
    }
    // The node's first item publishes its children (push_leaf / publish child).
    if (item == nd->item_base) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t sl = lane + 64u * h;
            const uint32_t ci = h ? ci1 : ci0;
            const uint32_t cr = h ? cr1 : cr0;
            if (sl < nl && ci != kChildEmpty) {
                const uint32_t c = a.child_counts[cbase + sl];
                if (ci & kChildNodeBit) {
                    NodeDesc child{};
                    child.row_start = node_row_base + cr;
                    child.n = c;
                    child.depth = nd->depth + 1u;
                    child.seed = nd->seed ^ ((uint64_t)sl * 0x94d049bb133111ebull) ^ (((uint64_t)c) << 23);
                    child.root_base = nd->root_base;
                    child.root_index = nd->root_index;
                    child.status = kNodeIdle;
                    a.nodes[cur ^ 1u][nd->node_base + (ci & ~kChildNodeBit)] = child;
                } else {
                    const uint64_t li = nd->leaf_base + ci;
                    const uint64_t start = leaf_row_base + cr;
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
}

// Level-by-level launches: four items per 256-thread workgroup; the whole
// scatter is skipped once an overflow is flagged.
constexpr uint32_t kScatterWavesPerBlock = 4;
__global__ __launch_bounds__(64 * kScatterWavesPerBlock) void scatter_kernel(PartArgs a, uint32_t cur,
                                                                             uint32_t level_nodes) {
    __shared__ uint32_t wl[kScatterWavesPerBlock][kScatterWaveWords];
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t item = blockIdx.x * kScatterWavesPerBlock + wave;
    if (item >= a.hdr->items || a.counters[TESSA_P_OVERFLOW_FLAGS] != 0ull) return;  // whole waves
    scatter_item_wave(a, cur, item, a.item_node[item], wl[wave]);
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

// ---- the persistent walk ----------------------------------------------------
// One cooperative launch runs the whole level loop (the reference's
// persistent partition loop, compute_backend.rs:16555-17112): every phase of
// a level (stage, item plan, COUNT / EMIT attempts, node scan, publication
// scan, scatter) is a grid-stride loop over the level's nodes or items,
// separated by grid barriers, and every decision the host loop used to read
// back (retry or not, the next level's size, overflow) is read from the level
// header by all workgroups after a barrier, so they take the same branch.
// The schedule, and with it the leaves and counters, is the level-by-level
// launches' schedule.

// Levels: the terminal-depth retry runs with max_depth up to 1024, so a tree
// may be that deep.
constexpr uint32_t kMaxLevels = 1100u;

__device__ __forceinline__ uint32_t load_ctl(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Grid barrier over gridDim.x co-resident workgroups: arrivals count up a
// monotonic word, so barrier i waits for (i + 1) * gridDim.x arrivals and no
// reset is needed.  Memory: every wave waits until its global stores are
// acknowledged by L2 before the workgroup barrier; thread 0 then arrives with
// an agent-scope release (the L2 written back, so the other XCDs, which have
// L2s of their own, can see the workgroup's writes), polls with relaxed
// loads (an acquiring load would invalidate the caches on every poll, under
// workgroups still at work), and acquires once the count is reached (this
// CU's L1 and its XCD's L2 invalidated) before the workgroup moves on.
// A wait longer than watchdog_ticks of the 100 MHz wall clock flags
// WATCHDOG_STALLED (compute_backend.rs:5883-5929 role) and returns false;
// every workgroup then leaves the walk.
constexpr int kWaitStores = 0x0F70;  // s_waitcnt vmcnt(0): the wave's memory operations complete

__device__ __forceinline__ bool grid_barrier(const PartArgs &a, uint32_t target, uint32_t *s_ok,
                                             uint64_t *wait_ticks = nullptr) {
    __builtin_amdgcn_s_waitcnt(kWaitStores);
    __syncthreads();
    if (threadIdx.x == 0) {
        LevelHeader *h = a.hdr;
        uint32_t ok = 1u;
        __hip_atomic_fetch_add(&h->barrier, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t t0 = wall_clock64();
        if (wait_ticks) *wait_ticks -= t0;
        while (__hip_atomic_load(&h->barrier, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (load_ctl(&h->walk_status) == kWalkStalled) {
                ok = 0u;
                break;
            }
            if (wall_clock64() - t0 > a.watchdog_ticks) {
                __hip_atomic_store(&h->walk_status, (uint32_t)kWalkStalled, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                pc_flag(a.counters, TESSA_OVF_WATCHDOG_STALLED);
                ok = 0u;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (wait_ticks) *wait_ticks += wall_clock64();
        *s_ok = ok;
    }
    __syncthreads();
    return *s_ok != 0u;
}

template <int KS>
__global__ __launch_bounds__(CountLayout<KS>::kThreads, 1) void walk_kernel(PartArgs a, uint32_t level_nodes,
                                                                            uint64_t level_rows) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];  // CountLayout<KS>, reused per phase
    __shared__ uint32_t s_node, s_ok;
    static_assert(CountLayout<KS>::kThreads * 8 <= CountLayout<KS>::kBytes, "scan scratch fits the LDS");
    static_assert(kScanGroups * kPartMaxLeaders * 4 <= CountLayout<KS>::kBytes, "node scan scratch fits the LDS");
    static_assert(CountLayout<KS>::kWaves * kScatterWaveWords * 4 <= CountLayout<KS>::kBytes,
                  "scatter scratch fits the LDS");
    static_assert(CountLayout<KS>::kThreads % kPartMaxLeaders == 0 &&
                      CountLayout<KS>::kThreads / kPartMaxLeaders <= kScanGroups,
                  "node scan groups");
    LevelHeader *h = a.hdr;
    const uint32_t G = gridDim.x, b = blockIdx.x, tid = threadIdx.x;
    // waves as workers for the per-node and per-item phases
    const uint32_t GW = G * (blockDim.x >> 6), gw = b * (blockDim.x >> 6) + (tid >> 6);
    uint32_t target = 0u;
    uint32_t cur = 0u, levels = 0u, passes = 0u, status = kWalkBound;
    // phase clocks (workgroup 0, thread 0, kept in LDS): spans between
    // barrier exits; clk[kClkMark] is the last exit, clk[kClkStart] the start
    enum { kClkCount, kClkEmit, kClkScatter, kClkPublish, kClkWait, kClkMark, kClkStart, kClkN };
    __shared__ uint64_t clk[kClkN];
    const bool timer = b == 0u && tid == 0u;
    if (timer) {
        for (int i = 0; i < kClkN; ++i) clk[i] = 0ull;
        clk[kClkStart] = clk[kClkMark] = (uint64_t)wall_clock64();
    }
    auto barrier = [&](int phase) -> bool {
        const bool ok = grid_barrier(a, target += G, &s_ok, timer ? &clk[kClkWait] : nullptr);
        if (timer) {
            const uint64_t now = wall_clock64();
            clk[phase] += now - clk[kClkMark];
            clk[kClkMark] = now;
        }
        return ok;
    };
    for (uint32_t level = 0; level < kMaxLevels; ++level) {
        const uint64_t items_bound = level_rows / kPartItemRows + level_nodes + 1u;
        if (items_bound > a.item_cap || items_bound > 0x7fffffffull) {
            status = kWalkCapacity;
            break;
        }
        if (b == 0u && tid < kPartMaxAttempts) h->retry[tid] = 0u;
        for (uint32_t ni = gw; ni < level_nodes; ni += GW) stage_node_wave(a, cur, level_nodes, ni);
        if (!barrier(kClkEmit)) return;
        if (b == 0u) item_plan_block(a, cur, level_nodes, reinterpret_cast<uint64_t *>(smem));
        if (!barrier(kClkEmit)) return;
        for (uint32_t ni = gw; ni < level_nodes; ni += GW) item_map_wave(a, cur, ni);
        if (!barrier(kClkEmit)) return;
        uint32_t attempt = 0;
        for (; attempt < kPartMaxAttempts; ++attempt) {
            count_items<KS>(a, cur, level_nodes, b, G, smem, &s_node);
            passes += 1u;
            if (!barrier(kClkCount)) return;
            for (uint32_t ni = gw; ni < level_nodes; ni += GW) emit_node_wave(a, cur, ni, &h->retry[attempt]);
            if (!barrier(kClkEmit)) return;
            if (load_ctl(&h->retry[attempt]) == 0u) break;
        }
        if (attempt == kPartMaxAttempts) {
            status = kWalkBound;
            break;
        }
        // nodes of many items: a workgroup each; the rest: a wave each
        for (uint32_t ni = b; ni < level_nodes; ni += G)
            if (a.nodes[cur][ni].items > kWaveScanItems)
                node_scan_block(a, cur, ni, reinterpret_cast<uint32_t(*)[kPartMaxLeaders]>(smem));
        for (uint32_t ni = gw; ni < level_nodes; ni += GW)
            if (a.nodes[cur][ni].items <= kWaveScanItems) node_scan_wave(a, cur, ni);
        if (!barrier(kClkPublish)) return;
        if (b == 0u) pub_scan_block(a, cur, level_nodes, reinterpret_cast<uint64_t *>(smem));
        if (!barrier(kClkPublish)) return;
        const uint32_t items =
            __hip_atomic_load(&a.counters[TESSA_P_OVERFLOW_FLAGS], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0ull
                ? 0u
                : load_ctl(&h->items);
        uint32_t *wl = reinterpret_cast<uint32_t *>(smem) + (tid >> 6) * kScatterWaveWords;
        for (uint32_t item = gw; item < items; item += GW) scatter_item_wave(a, cur, item, a.item_node[item], wl);
        if (!barrier(kClkScatter)) return;
        levels = level + 1u;
        const uint64_t overflow = __hip_atomic_load(&h->overflow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        level_nodes = load_ctl(&h->next_nodes);
        level_rows = __hip_atomic_load(&h->next_rows, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        cur ^= 1u;
        if (overflow != 0ull || level_nodes == 0u) {
            status = kWalkOk;
            break;
        }
    }
    if (timer) {
        h->levels = levels;
        h->count_passes = passes;
        if (load_ctl(&h->walk_status) != kWalkStalled) h->walk_status = status;
        a.counters[TESSA_P_PARTITION_BUSY_CLOCKS] = (uint64_t)wall_clock64() - clk[kClkStart];
        a.counters[TESSA_P_PARTITION_WAIT_CLOCKS] = clk[kClkWait];
        a.counters[TESSA_P_LARGE_COUNT_DISTANCE_CLOCKS] = clk[kClkCount];
        a.counters[TESSA_P_LARGE_COUNT_COMMIT_CLOCKS] = clk[kClkEmit];
        a.counters[TESSA_P_LARGE_SCATTER_CLOCKS] = clk[kClkScatter];
        a.counters[TESSA_P_LARGE_PUBLISH_CLOCKS] = clk[kClkPublish];
    }
}

// Co-resident workgroups of the walk: the occupancy the runtime reports,
// times the CUs.
// A failed HIP call of the walk's launch path: records it and returns -1.
int part_fail(PartResult *res, hipError_t e, const char *step) {
    res->hip_error = (int)e;
    res->failed_step = step;
    return -1;
}

template <int KS>
int launch_walk_ks(const PartArgs &a, uint32_t level_nodes, uint64_t level_rows, hipStream_t s, PartResult *res) {
    using L = CountLayout<KS>;
    const void *fn = reinterpret_cast<const void *>(walk_kernel<KS>);
    if (ensure_lds_limit(fn, L::kBytes)) return part_fail(res, hipErrorInvalidValue, "walk LDS limit");
    int dev = 0, cus = 0, per = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, walk_kernel<KS>, L::kThreads, L::kBytes);
    if (e != hipSuccess) return part_fail(res, e, "walk occupancy query");
    if (per < 1 || cus < 1) return part_fail(res, hipErrorInvalidConfiguration, "walk occupancy is zero");
    PartArgs args = a;
    void *params[] = {&args, &level_nodes, &level_rows};
    e = hipLaunchCooperativeKernel(fn, dim3((uint32_t)(cus * per)), dim3(L::kThreads), params, L::kBytes, s);
    if (e != hipSuccess) return part_fail(res, e, "walk cooperative launch");
    return 0;
}

int launch_walk(const PartArgs &a, uint32_t level_nodes, uint64_t level_rows, hipStream_t s, PartResult *res) {
    const uint32_t ks = (a.padded_dim + 31) / 32;
    if (ks <= 4) return launch_walk_ks<4>(a, level_nodes, level_rows, s, res);
    if (ks <= 8) return launch_walk_ks<8>(a, level_nodes, level_rows, s, res);
    if (ks <= 12) return launch_walk_ks<12>(a, level_nodes, level_rows, s, res);
    if (ks <= 16) return launch_walk_ks<16>(a, level_nodes, level_rows, s, res);
    if (ks <= 24) return launch_walk_ks<24>(a, level_nodes, level_rows, s, res);
    if (ks <= 32) return launch_walk_ks<32>(a, level_nodes, level_rows, s, res);
    return -3;
}

template <int KS>
int launch_count_ks(const PartArgs &a, uint32_t cur, uint32_t level_nodes, uint32_t grid, hipStream_t s) {
    using L = CountLayout<KS>;
    if (ensure_lds_limit(reinterpret_cast<const void *>(count_kernel<KS>), L::kBytes)) return -1;
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

static int run_levels(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture,
                      uint32_t level_nodes, uint64_t level_rows);

int run_partition(const PartArgs &args, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture) {
    *res = PartResult{};
    PartArgs a = args;
    if (a.watchdog_ticks == 0) {
        // 10 s of the device's wall clock (its rate in kHz)
        int dev = 0, khz = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
        if (e != hipSuccess) return part_fail(res, e, "wall clock rate query");
        if (khz <= 0) khz = 100000;  // the gfx9 wall clock runs at 100 MHz
        a.watchdog_ticks = (uint64_t)khz * 10000ull;
    }
    hipLaunchKernelGGL(init_kernel, dim3(1), dim3(256), 0, s, a);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return part_fail(res, e, "init launch");
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
        if (ensure_lds_limit(reinterpret_cast<const void *>(small_root_kernel), (int)kSmallLdsBytes)) return -1;
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

// The level loop from the nodes of level 0 (in the first arena): the
// persistent walk, read back once it has finished; with a capture, the
// level-by-level launches.
static int run_levels_host(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture,
                           uint32_t level_nodes, uint64_t level_rows);

static int run_levels(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture,
                      uint32_t level_nodes, uint64_t level_rows) {
    if (capture) return run_levels_host(a, s, hh, res, capture, level_nodes, level_rows);
    const int rc = launch_walk(a, level_nodes, level_rows, s, res);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(hh, a.hdr, sizeof(LevelHeader), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return part_fail(res, e, "walk header read-back");
    res->levels = hh->levels;
    res->count_launches = hh->count_passes;
    res->leaf_count = hh->leaf_count;
    res->leaf_rows = hh->leaf_rows;
    switch (hh->walk_status) {
        case kWalkOk: return 0;
        case kWalkCapacity: return -3;
        case kWalkStalled: return -4;
        default: return -2;
    }
}

static int run_levels_host(const PartArgs &a, hipStream_t s, LevelHeader *hh, PartResult *res, PartCapture *capture,
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
        hipLaunchKernelGGL(stage_kernel, dim3(level_nodes), dim3(64), 0, s, a, cur, level_nodes);
        hipLaunchKernelGGL(item_plan_kernel, dim3(1), dim3(1024), 0, s, a, cur, level_nodes);
        hipLaunchKernelGGL(item_map_kernel, dim3(level_nodes), dim3(64), 0, s, a, cur, level_nodes);
        if (hipGetLastError() != hipSuccess) return -1;
        uint32_t attempt = 0;
        for (; attempt < kPartMaxAttempts; ++attempt) {
            if (capture && capture_level(a, s, cur, level_nodes, capture)) return -1;
            if (launch_count(a, cur, level_nodes, grid, s)) return -1;
            res->count_launches += 1;
            hipLaunchKernelGGL(emit_kernel, dim3(level_nodes), dim3(64), 0, s, a, cur, level_nodes);
            if (hipGetLastError() != hipSuccess) return -1;
            if (read_header()) return -1;
            if (hh->retry_nodes == 0u) break;
            hipLaunchKernelGGL(reset_retry_kernel, dim3(1), dim3(1), 0, s, a.hdr);
        }
        if (attempt == kPartMaxAttempts) return -2;
        hipLaunchKernelGGL(node_scan_kernel, dim3(level_nodes), dim3(kScanGroups * kPartMaxLeaders), 0, s, a, cur,
                           level_nodes);
        hipLaunchKernelGGL(pub_scan_kernel, dim3(1), dim3(1024), 0, s, a, cur, level_nodes);
        hipLaunchKernelGGL(scatter_kernel, dim3((grid + kScatterWavesPerBlock - 1) / kScatterWavesPerBlock),
                           dim3(64 * kScatterWavesPerBlock), 0, s, a, cur, level_nodes);
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
