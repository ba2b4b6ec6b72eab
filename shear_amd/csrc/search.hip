// search.hip -- greedy search of a neighbour graph: the recall harness's
// search, one wavefront per query.
//
// Reference (paths relative to shear-core/src/): algorithm/search/search.rs:
// 137-233 (seed the list with the start point, mark it visited; repeatedly
// expand the closest not-visited entry; its unvisited neighbours are marked
// and inserted; stop when every listed entry is visited) over the capacity-L
// queue of model/neighbor/neighbor_priority_queue.rs:50-85, ordered by
// (distance, id) (model/neighbor/neighbor.rs:46-70); results as
// index/inmem_index/inmem_index.rs:559-580 (the first K entries).
//
// Inserting one expansion's neighbours one by one into the capacity-L sorted
// list leaves the L smallest of (list, neighbours) under the total order
// (distance, id), and the queue's cursor is then the first not-visited entry
// (an insert in front of the cursor moves it there; entries before it are all
// visited).  So the wave inserts a whole batch at once: the up-to-64 new
// neighbours of a chunk of the row are scored one per lane, sorted across the
// wave, and merged with the list by rank (each entry's new position is its
// old one plus the number of entries of the other side below it); entries
// ranked L and past drop off.  Same list, same cursor as the one-by-one
// inserts.
//
// Distances: squared L2 summed over the coordinates in order in f32, each
// product rounded before the add (no contraction), one lane per candidate
// (the harness's stated order; the reference's SIMD kernel may associate
// differently).  With SQ8 rows (sets too large to keep as f32) a row's
// coordinate i is the f32 product scale * code[i], rounded, then the same sum:
// the search over the dequantized vectors.  Keys are (distance bits << 32 | id): for the non-negative
// distances this computes, the integer order is (distance, id).
//
// Visited set: a tag per (slot, point) holding query index + 1; tags are
// zeroed once per call, so a slot's next query needs no clearing.  The tag is
// claimed with an atomic exchange so a point listed twice in one row enters
// the list once.
#include "search_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

constexpr uint32_t kThreads = kSearchWaves * 64;
constexpr uint64_t kNoKey = ~0ull;

struct alignas(16) WaveLists {
    uint64_t key[2][kSearchMaxL];     // double-buffered list, ascending
    uint32_t visited[2][kSearchMaxL];
    uint64_t fresh[64];               // one chunk's new neighbours, sorted
};

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, uint32_t src) {
    const uint32_t lo = __shfl((uint32_t)v, src), hi = __shfl((uint32_t)(v >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}

// Ascending bitonic sort of one u64 per lane across the wave.
__device__ __forceinline__ uint64_t wave_sort64(uint64_t v, uint32_t lane) {
#pragma unroll
    for (uint32_t k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            const uint64_t o = shfl_u64(v, lane ^ j);
            const bool lower = (lane & j) == 0;
            const bool up = (lane & k) == 0;
            const uint64_t lo = v < o ? v : o, hi = v < o ? o : v;
            v = (lower == up) ? lo : hi;
        }
    }
    return v;
}

// number of entries of a[0, n) (ascending, distinct from x) below x
__device__ __forceinline__ uint32_t rank_in(const uint64_t *a, uint32_t n, uint64_t x) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (a[mid] < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Squared L2 of the dequantized SQ8 row (scale * code[i], rounded) and the
// query, coordinates in order; 16 codes per load when kVec16.
template <bool kVec16>
__device__ float sq8_l2_ordered(const int8_t *__restrict__ c, float sc, const float *__restrict__ q, uint32_t dim) {
    float s = 0.0f;
    if constexpr (kVec16) {
        typedef int v4i_t __attribute__((ext_vector_type(4)));
        const v4i_t *cv = reinterpret_cast<const v4i_t *>(c);
        const float4 *qv = reinterpret_cast<const float4 *>(q);
        for (uint32_t i = 0; i < dim / 16; ++i) {
            const v4i_t w = cv[i];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 b = qv[4 * i + g];
                const uint32_t word = (uint32_t)w[g];
                const float bq[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = __fmul_rn(sc, (float)(int8_t)(word >> (8 * e)));
                    const float t = __fsub_rn(x, bq[e]);
                    s = __fadd_rn(s, __fmul_rn(t, t));
                }
            }
        }
    } else {
        for (uint32_t i = 0; i < dim; ++i) {
            const float t = __fsub_rn(__fmul_rn(sc, (float)c[i]), q[i]);
            s = __fadd_rn(s, __fmul_rn(t, t));
        }
    }
    return s;
}

// kMode 0: f32 rows, scalar; 1: f32 rows, float4 loads; 2: SQ8 rows, scalar;
// 3: SQ8 rows, 16 codes per load.
template <int kMode>
__device__ __forceinline__ float row_dist(const GraphSearchParams &p, uint32_t id, const float *q) {
    if constexpr (kMode < 2) return l2_ordered<kMode == 1>(p.data + (uint64_t)id * p.dim, q, p.dim);
    else return sq8_l2_ordered<kMode == 3>(p.codes + (uint64_t)id * p.padded_dim, p.scales[id], q, p.dim);
}

template <int kMode>
__global__ __launch_bounds__(kThreads) void graph_search_kernel(GraphSearchParams p) {
    __shared__ WaveLists lists[kSearchWaves];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = blockIdx.x * kSearchWaves + wave;
    WaveLists &w = lists[wave];
    uint32_t *tags = p.tags + (uint64_t)slot * p.num_points;

    for (uint32_t qi = slot; qi < p.num_queries; qi += p.slots) {
        const float *q = p.queries + (uint64_t)qi * p.dim;
        const uint32_t epoch = qi + 1u;
        uint32_t buf = 0, size = 1, cur = 0, cmps = 0;
        if (lane == 0) {
            tags[p.start] = epoch;
            const float d0 = row_dist<kMode>(p, p.start, q);
            w.key[0][0] = ((uint64_t)__float_as_uint(d0) << 32) | p.start;
            w.visited[0][0] = 0u;
        }
        wave_lds_sync();
        while (cur < size) {
            // closest_notvisited: expand the entry at the cursor
            const uint32_t node = (uint32_t)w.key[buf][cur];
            wave_lds_sync();
            if (lane == 0) w.visited[buf][cur] = 1u;
            const uint32_t cnt = p.counts[node];
            const uint32_t deg = cnt < p.row_stride ? cnt : p.row_stride;
            const uint32_t *row = p.targets + (uint64_t)node * p.row_stride;
            for (uint32_t s0 = 0; s0 < deg; s0 += 64) {
                const uint32_t s = s0 + lane;
                const uint32_t id = s < deg ? row[s] : 0xFFFFFFFFu;
                bool fresh = id < p.num_points;
                if (fresh) fresh = atomicExch(&tags[id], epoch) != epoch;
                uint64_t key = kNoKey;
                if (fresh) {
                    const float d = row_dist<kMode>(p, id, q);
                    key = ((uint64_t)__float_as_uint(d) << 32) | id;
                }
                const uint32_t nf = (uint32_t)__popcll(__ballot(fresh));
                if (nf == 0) continue;
                cmps += nf;
                key = wave_sort64(key, lane);
                w.fresh[lane] = key;
                wave_lds_sync();
                const uint32_t nb = buf ^ 1u;
                const uint32_t new_size = size + nf < p.L ? size + nf : p.L;
                for (uint32_t i = lane; i < size; i += 64) {
                    const uint64_t k = w.key[buf][i];
                    const uint32_t pos = i + rank_in(w.fresh, nf, k);
                    if (pos < p.L) {
                        w.key[nb][pos] = k;
                        w.visited[nb][pos] = w.visited[buf][i];
                    }
                }
                if (lane < nf) {
                    const uint32_t pos = lane + rank_in(w.key[buf], size, key);
                    if (pos < p.L) {
                        w.key[nb][pos] = key;
                        w.visited[nb][pos] = 0u;
                    }
                }
                wave_lds_sync();
                buf = nb;
                size = new_size;
            }
            // the cursor: first entry not yet expanded
            wave_lds_sync();
            cur = size;
            for (uint32_t c = 0; c < size; c += 64) {
                const uint32_t i = c + lane;
                const uint64_t open = __ballot(i < size && w.visited[buf][i] == 0u);
                if (open) {
                    cur = c + (uint32_t)__ffsll((unsigned long long)open) - 1u;
                    break;
                }
            }
        }
        for (uint32_t i = lane; i < p.K; i += 64) {
            const uint64_t k = i < size ? w.key[buf][i] : kNoKey;
            p.out_ids[(uint64_t)qi * p.K + i] = i < size ? (uint32_t)k : 0xFFFFFFFFu;
            if (p.out_dists) p.out_dists[(uint64_t)qi * p.K + i] = i < size ? __uint_as_float((uint32_t)(k >> 32)) : 0.0f;
        }
        if (p.out_cmps && lane == 0) p.out_cmps[qi] = cmps;
        wave_lds_sync();
    }
}

__global__ void zero_tags(uint32_t *tags, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        tags[i] = 0u;
}

}  // namespace

uint32_t search_slots(uint32_t num_points, uint32_t num_queries) {
    // at most 1 GiB of tags and 4096 slots, at least one workgroup
    const uint64_t by_mem = (1ull << 30) / (4ull * (num_points ? num_points : 1));
    uint64_t s = num_queries < 4096u ? num_queries : 4096u;
    if (s > by_mem) s = by_mem;
    s = (s + kSearchWaves - 1) / kSearchWaves * kSearchWaves;
    return (uint32_t)(s < kSearchWaves ? kSearchWaves : s);
}

int launch_graph_search(const GraphSearchParams &p, hipStream_t stream) {
    const uint64_t ntags = (uint64_t)p.slots * p.num_points;
    uint64_t zg = (ntags + 255) / 256;
    zg = zg < 1 ? 1 : (zg > 8192 ? 8192 : zg);
    hipLaunchKernelGGL(zero_tags, dim3((uint32_t)zg), dim3(256), 0, stream, p.tags, ntags);
    const dim3 grid(p.slots / kSearchWaves);
    if (p.data) {
        const bool vec4 = p.dim % 4 == 0 && reinterpret_cast<uintptr_t>(p.data) % 16 == 0 &&
                          reinterpret_cast<uintptr_t>(p.queries) % 16 == 0;
        if (vec4) hipLaunchKernelGGL(graph_search_kernel<1>, grid, dim3(kThreads), 0, stream, p);
        else hipLaunchKernelGGL(graph_search_kernel<0>, grid, dim3(kThreads), 0, stream, p);
    } else {
        const bool vec16 = p.dim % 16 == 0 && p.padded_dim % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(p.codes) % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(p.queries) % 16 == 0;
        if (vec16) hipLaunchKernelGGL(graph_search_kernel<3>, grid, dim3(kThreads), 0, stream, p);
        else hipLaunchKernelGGL(graph_search_kernel<2>, grid, dim3(kThreads), 0, stream, p);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
