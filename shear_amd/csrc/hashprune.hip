// hashprune.hip -- HashPrune reservoirs on the GPU: the reducer that consumes
// the edge-record stream (SpillRecord16) and keeps, per source point, at most
// l_max neighbours.
//
// Reference semantics (shear-core/src/algorithm/pipnn/): HashPruneReservoir
// insert (hash_prune.rs:1333-1453) under the total order (dist by total_cmp,
// target, hash; :2094-2106), fed edge by edge by the spill reducer
// (spill_hashprune.rs:2686-2719) and emitted as the slot targets in slot
// order, ascending hash (:3203-3221 emit_shard).  With the backfill and
// evidence policies off (params.rs:3346-3350) that reservoir ends in a state
// that depends only on the set of candidates inserted: each hash keeps its
// best candidate (a hit keeps the better one), and of those the l_max best
// remain (an evicted or rejected candidate is worse than l_max others of
// distinct hashes, and those are only ever replaced by better ones).  So a
// batch of records can be merged in any order, which is what makes it a GPU
// reduction.  Record batches:
//   1. count records per source (atomics), exclusive scan, scatter the records
//      grouped by source (the per-source counters return to zero);
//   2. one wave per source with new records merges its current slots with them
//      (in registers up to 256 candidates, else in LDS up to kHpMergeCap at a
//      time): a bitonic sort by (hash, total order: dist key, target) puts
//      each hash's best first; when more than l_max hashes remain, a sort of
//      those by the total order gives the l_max-th as a threshold; the
//      survivors are the new slots.
// Segment batches (records left where the emitter wrote them, described by
// per-source runs) are merged by streaming each source's records through its
// reservoir held in registers (hp_merge_stream_kernel).  Between merges the
// slots are kept in no particular order; the export sorts each reservoir by
// hash, the reference's emit order.
#include <hipcub/hipcub.hpp>

#include "hashprune_kernels.h"

namespace tessa {

namespace {

constexpr int kHpWaves = 4;                 // waves per workgroup of the merge kernels
constexpr uint32_t kHpRegMax = 256;         // largest merge done in registers (4 candidates per lane)
constexpr int kHpThreads = kHpWaves * 64;
constexpr int kScanThreads = 1024;
constexpr int kScanPerThread = 4;
constexpr uint32_t kScanBlock = kScanThreads * kScanPerThread;

__device__ __forceinline__ uint32_t total_key(float d) {
    const uint32_t b = __float_as_uint(d);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_dist(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v, uint32_t lane, uint32_t &total) {
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off);
        if (lane >= (uint32_t)off) x += y;
    }
    total = __shfl(x, 63);
    return x - v;
}

__global__ void hp_fill_u32(uint32_t *a, uint64_t n, uint32_t v) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        a[i] = v;
}

__global__ void hp_status_init(uint64_t *status) { status[0] = ~0ull; }

// Lanes of a wave holding the same source as the wave's first active lane
// share one atomic (the edge stream interleaves one row's outgoing records
// with its reverse ones, so about half a wave has the same source).
__device__ __forceinline__ uint64_t same_as_leader(uint32_t src, bool active, uint32_t &leader_src) {
    const uint64_t act = __ballot(active);
    const uint32_t leader = act ? (uint32_t)__builtin_ctzll(act) : 0u;
    leader_src = __shfl(src, leader);
    return __ballot(active && src == leader_src);
}

__global__ void hp_count_kernel(const uint4 *rec, uint64_t count, uint32_t num_points, uint32_t *bucket,
                                uint64_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    // uniform trip count per wave: lanes past the end stay inactive
    for (uint64_t i0 = (uint64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~63u); i0 < count; i0 += stride) {
        const uint64_t i = i0 + lane;
        const bool in = i < count;
        const uint32_t src = in ? rec[i].x : 0u;
        const bool bad = in && src >= num_points;
        if (bad) atomicMin((unsigned long long *)status, (unsigned long long)i);
        uint32_t lsrc;
        const uint64_t grp = same_as_leader(src, in && !bad, lsrc);
        const bool in_grp = (grp >> lane) & 1ull;
        if (in_grp && lane == (uint32_t)__builtin_ctzll(grp)) atomicAdd(&bucket[lsrc], (uint32_t)__popcll(grp));
        if (in && !bad && !in_grp) atomicAdd(&bucket[src], 1u);
    }
}

// Block sums of `bucket` over kScanBlock elements each.
__global__ __launch_bounds__(kScanThreads) void hp_scan_reduce(const uint32_t *bucket, uint32_t n, uint32_t *sums) {
    __shared__ uint32_t ws[kScanThreads / 64];
    const uint32_t base = blockIdx.x * kScanBlock + threadIdx.x * kScanPerThread;
    uint32_t v = 0;
#pragma unroll
    for (int e = 0; e < kScanPerThread; ++e) v += base + e < n ? bucket[base + e] : 0u;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if ((threadIdx.x & 63u) == 0) ws[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < kScanThreads / 64; ++w) t += ws[w];
        sums[blockIdx.x] = t;
    }
}

// Exclusive scan of the block sums in place (one workgroup); offsets[n] = total.
__global__ __launch_bounds__(kScanThreads) void hp_scan_partials(uint32_t *sums, uint32_t nb, uint32_t *offsets,
                                                                 uint32_t n) {
    __shared__ uint32_t ws[kScanThreads / 64];
    __shared__ uint32_t carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (uint32_t b0 = 0; b0 < nb; b0 += kScanThreads) {
        const uint32_t i = b0 + threadIdx.x;
        const uint32_t v = i < nb ? sums[i] : 0u;
        uint32_t wt;
        const uint32_t ex = wave_excl_scan(v, lane, wt);
        if (lane == 0) ws[wave] = wt;
        __syncthreads();
        uint32_t before = 0, all = 0;
        for (uint32_t w = 0; w < kScanThreads / 64; ++w) {
            before += w < wave ? ws[w] : 0u;
            all += ws[w];
        }
        if (i < nb) sums[i] = carry + before + ex;
        __syncthreads();
        if (threadIdx.x == 0) carry += all;
        __syncthreads();
    }
    if (threadIdx.x == 0) offsets[n] = carry;
}

__global__ __launch_bounds__(kScanThreads) void hp_scan_apply(const uint32_t *bucket, uint32_t n, const uint32_t *sums,
                                                              uint32_t *offsets) {
    __shared__ uint32_t ws[kScanThreads / 64];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t base = blockIdx.x * kScanBlock + threadIdx.x * kScanPerThread;
    uint32_t v[kScanPerThread], t = 0;
#pragma unroll
    for (int e = 0; e < kScanPerThread; ++e) {
        v[e] = base + e < n ? bucket[base + e] : 0u;
        t += v[e];
    }
    uint32_t wt;
    const uint32_t ex = wave_excl_scan(t, lane, wt);
    if (lane == 0) ws[wave] = wt;
    __syncthreads();
    uint32_t before = sums[blockIdx.x];
    for (uint32_t w = 0; w < wave; ++w) before += ws[w];
    uint32_t run = before + ex;
#pragma unroll
    for (int e = 0; e < kScanPerThread; ++e) {
        if (base + e < n) offsets[base + e] = run;
        run += v[e];
    }
}

// Records grouped by source; the per-source counters count back down to zero.
__global__ void hp_scatter_kernel(const uint4 *rec, uint64_t count, uint32_t num_points, uint32_t *bucket,
                                  const uint32_t *offsets, uint4 *grouped) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i0 = (uint64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~63u); i0 < count; i0 += stride) {
        const uint64_t i = i0 + lane;
        const bool in = i < count;
        const uint4 r = in ? rec[i] : make_uint4(0u, 0u, 0u, 0u);
        const bool ok = in && r.x < num_points;
        uint32_t lsrc;
        const uint64_t grp = same_as_leader(r.x, ok, lsrc);
        const bool in_grp = (grp >> lane) & 1ull;
        // the group takes popcount(grp) positions with one atomic; lane order inside it
        const uint32_t first = grp ? (uint32_t)__builtin_ctzll(grp) : 0u;
        uint32_t top = 0;
        if (in_grp && lane == first) top = atomicSub(&bucket[lsrc], (uint32_t)__popcll(grp));
        top = __shfl(top, first);
        if (in_grp) {
            const uint32_t below = (uint32_t)__popcll(grp & ((1ull << lane) - 1ull));
            grouped[offsets[lsrc] + top - 1u - below] = r;
        } else if (ok) {
            grouped[offsets[r.x] + atomicSub(&bucket[r.x], 1u) - 1u] = r;
        }
    }
}

// Ascending bitonic sort of (key, payload) pairs, lexicographic, over
// [0, P) (P a power of two >= 64), by one wave on its LDS region.  LDS
// operations of one wave complete in order, so stages need no barrier.
template <typename K>
__device__ void wave_bitonic(K *key, uint32_t *val, uint32_t P, uint32_t lane) {
    for (uint32_t k = 2; k <= P; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t c = lane; c < P / 2; c += 64) {
                const uint32_t i = ((c & ~(j - 1u)) << 1) | (c & (j - 1u));
                const uint32_t l = i + j;
                const bool up = (i & k) == 0;
                const K a = key[i], b = key[l];
                const uint32_t va = val[i], vb = val[l];
                const bool b_less = b < a || (b == a && vb < va);
                const bool a_less = a < b || (a == b && va < vb);
                if (up ? b_less : a_less) {
                    key[i] = b;
                    key[l] = a;
                    val[i] = vb;
                    val[l] = va;
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// Ascending bitonic sort of (hash, key) pairs, hash first, over [0, P).
__device__ void wave_bitonic_hk(uint32_t *hash, uint64_t *key, uint32_t P, uint32_t lane) {
    for (uint32_t k = 2; k <= P; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t c = lane; c < P / 2; c += 64) {
                const uint32_t i = ((c & ~(j - 1u)) << 1) | (c & (j - 1u));
                const uint32_t l = i + j;
                const bool up = (i & k) == 0;
                const uint32_t ha = hash[i], hb = hash[l];
                const uint64_t a = key[i], b = key[l];
                const bool b_less = hb < ha || (hb == ha && b < a);
                const bool a_less = ha < hb || (ha == hb && a < b);
                if (up ? b_less : a_less) {
                    hash[i] = hb;
                    hash[l] = ha;
                    key[i] = b;
                    key[l] = a;
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// Register bitonic sort of P = 64*E elements, element q*64 + lane in lane
// `lane`'s slot q, by (hash, key) when kHashFirst, else by (key, hash).
template <int E, bool kHashFirst>
__device__ __forceinline__ void reg_bitonic(uint32_t (&h)[E], uint64_t (&k)[E], uint32_t lane) {
    auto less = [](uint32_t ha, uint64_t ka, uint32_t hb, uint64_t kb) {
        return kHashFirst ? (ha < hb || (ha == hb && ka < kb)) : (ka < kb || (ka == kb && ha < hb));
    };
#pragma unroll
    for (uint32_t kk = 2; kk <= 64u * E; kk <<= 1) {
#pragma unroll
        for (uint32_t j = kk >> 1; j > 0; j >>= 1) {
            if (j >= 64) {
                const uint32_t jq = j / 64;
#pragma unroll
                for (int q = 0; q < E; ++q) {
                    if ((q & jq) != 0) continue;
                    const int l = q | jq;
                    const bool up = (((uint32_t)q * 64u + lane) & kk) == 0;
                    const bool sw = up ? less(h[l], k[l], h[q], k[q]) : less(h[q], k[q], h[l], k[l]);
                    const uint32_t th = h[q];
                    const uint64_t tk = k[q];
                    h[q] = sw ? h[l] : h[q];
                    k[q] = sw ? k[l] : k[q];
                    h[l] = sw ? th : h[l];
                    k[l] = sw ? tk : k[l];
                }
            } else {
#pragma unroll
                for (int q = 0; q < E; ++q) {
                    const uint32_t ph = __shfl_xor(h[q], (int)j);
                    const uint32_t plo = __shfl_xor((uint32_t)k[q], (int)j);
                    const uint32_t phi = __shfl_xor((uint32_t)(k[q] >> 32), (int)j);
                    const uint64_t pk = ((uint64_t)phi << 32) | plo;
                    const bool up = (((uint32_t)q * 64u + lane) & kk) == 0;
                    const bool want_min = ((lane & j) == 0) == up;
                    const bool take = want_min ? less(ph, pk, h[q], k[q]) : less(h[q], k[q], ph, pk);
                    h[q] = take ? ph : h[q];
                    k[q] = take ? pk : k[q];
                }
            }
        }
    }
}

// Of the candidates in h/k (E register slots per lane; an empty entry is
// h = 0xffffffff, k = ~0, after every real hash <= 0xffff), keeps each hash's
// best and, of those, the l_max best in total order; leaves them in h/k at
// positions [0, n) (position q*64 + lane in slot q of lane), ascending in
// total order, empty entries after them, and returns n.
template <int E>
__device__ __forceinline__ uint32_t select_sorted(uint32_t (&h)[E], uint64_t (&k)[E], uint32_t l_max, uint32_t lane) {
    reg_bitonic<E, true>(h, k, lane);
    // kept = first of its hash (the predecessor of element 64*q is lane 63 of slot q-1)
    uint32_t n_kept = 0;
    bool kept[E];
#pragma unroll
    for (int q = 0; q < E; ++q) {
        uint32_t prev = __shfl_up(h[q], 1);
        if (q > 0) {
            const uint32_t last = __shfl(h[q - 1], 63);
            prev = lane == 0 ? last : prev;
        }
        const uint32_t e = (uint32_t)q * 64u + lane;
        kept[q] = h[q] != 0xffffffffu && (e == 0 || prev != h[q]);
        n_kept += (uint32_t)__popcll(__ballot(kept[q]));
    }
#pragma unroll
    for (int q = 0; q < E; ++q) {
        h[q] = kept[q] ? h[q] : 0xffffffffu;
        k[q] = kept[q] ? k[q] : ~0ull;
    }
    reg_bitonic<E, false>(h, k, lane);
    const uint32_t n = n_kept < l_max ? n_kept : l_max;
#pragma unroll
    for (int q = 0; q < E; ++q) {
        const bool live = (uint32_t)q * 64u + lane < n;
        h[q] = live ? h[q] : 0xffffffffu;
        k[q] = live ? k[q] : ~0ull;
    }
    return n;
}

// One merge of a source's n_old slots and n_new records (n_old + n_new <= 64*E)
// entirely in registers; writes the new slots and returns their count.
// fetch(q, t) returns new record t (t < n_new) for register slot q.
template <int E, typename Fetch>
__device__ uint32_t reg_merge_f(const uint64_t *slot_keys_in, const uint16_t *slot_hash_in, uint32_t n_old,
                                uint32_t n_new, Fetch &&fetch, uint32_t l_max, uint32_t lane,
                                uint64_t *slot_keys_out, uint16_t *slot_hash_out) {
    const uint32_t N = n_old + n_new;
    uint32_t h[E];
    uint64_t k[E];
#pragma unroll
    for (int q = 0; q < E; ++q) {
        const uint32_t e = (uint32_t)q * 64u + lane;
        h[q] = 0xffffffffu;
        k[q] = ~0ull;
        if (e < n_old) {
            k[q] = slot_keys_in[e];
            h[q] = slot_hash_in[e];
        } else if (e < N) {
            const uint4 r = fetch(q, e - n_old);
            k[q] = ((uint64_t)total_key(__uint_as_float(r.w)) << 32) | r.y;
            h[q] = r.z & 0xffffu;
        }
    }
    const uint32_t n = select_sorted<E>(h, k, l_max, lane);
#pragma unroll
    for (int q = 0; q < E; ++q) {
        const uint32_t e = (uint32_t)q * 64u + lane;
        if (e < n) {
            slot_keys_out[e] = k[q];
            slot_hash_out[e] = (uint16_t)h[q];
        }
    }
    return n;
}

// Records contiguous at recs; the first 64 were prefetched into r0 (they line
// up with register slot q when n_old == 64*q).
template <int E>
__device__ uint32_t reg_merge(const uint64_t *slot_keys_in, const uint16_t *slot_hash_in, uint32_t n_old,
                              const uint4 *recs, uint32_t n_new, const uint4 &r0, uint32_t l_max, uint32_t lane,
                              uint64_t *slot_keys_out, uint16_t *slot_hash_out) {
    auto fetch = [&](int q, uint32_t t) -> uint4 { return (n_old == (uint32_t)q * 64u) ? r0 : recs[t]; };
    return reg_merge_f<E>(slot_keys_in, slot_hash_in, n_old, n_new, fetch, l_max, lane, slot_keys_out,
                          slot_hash_out);
}

struct HpWaveLds {
    uint64_t key[kHpMergeCap];      // candidates: total-order key (dist key << 32 | target)
    uint32_t val[kHpMergeCap];      // their hashes
    uint64_t tkey[kHpMergeCap];     // each hash's best, sorted by total order: the merged
    uint32_t thash[kHpMergeCap];    // reservoir is their first min(count, l_max)
};

// Sources with at most kHpRegMax candidates (slots + new records): register
// merges, no LDS, so occupancy is set by registers alone.
__global__ __launch_bounds__(kHpThreads) void hp_merge_small_kernel(const uint4 *grouped, const uint32_t *offsets,
                                                                    uint32_t num_points, uint32_t l_max,
                                                                    uint64_t *slot_keys, uint16_t *slot_hash,
                                                                    uint32_t *slot_count) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t waves = gridDim.x * kHpWaves;
    // the next source's offsets and first 64 records are loaded one iteration
    // ahead, so their latency overlaps the current merge
    uint32_t src = blockIdx.x * kHpWaves + (threadIdx.x >> 6);
    uint32_t p_off = 0, p_n = 0;
    uint4 p_rec = make_uint4(0u, 0u, 0u, 0u);
    if (src < num_points) {
        p_off = offsets[src];
        p_n = offsets[src + 1] - p_off;
        if (lane < p_n) p_rec = grouped[p_off + lane];
    }
    for (; src < num_points; src += waves) {
        const uint32_t off = p_off;
        const uint32_t n_new = p_n;
        const uint4 r0 = p_rec;
        const uint32_t nsrc = src + waves;
        if (nsrc < num_points) {
            p_off = offsets[nsrc];
            p_n = offsets[nsrc + 1] - p_off;
            if (lane < p_n) p_rec = grouped[p_off + lane];
        }
        if (n_new == 0) continue;
        const uint32_t n_old = slot_count[src];
        const uint64_t sbase = (uint64_t)src * l_max;
        uint32_t c;
        if (n_old + n_new <= 64u)
            c = reg_merge<1>(slot_keys + sbase, slot_hash + sbase, n_old, grouped + off, n_new, r0, l_max, lane,
                             slot_keys + sbase, slot_hash + sbase);
        else if (n_old + n_new <= 128u)
            c = reg_merge<2>(slot_keys + sbase, slot_hash + sbase, n_old, grouped + off, n_new, r0, l_max, lane,
                             slot_keys + sbase, slot_hash + sbase);
        else if (n_old + n_new <= kHpRegMax)
            c = reg_merge<4>(slot_keys + sbase, slot_hash + sbase, n_old, grouped + off, n_new, r0, l_max, lane,
                             slot_keys + sbase, slot_hash + sbase);
        else
            continue;  // hp_merge_large_kernel
        if (lane == 0) slot_count[src] = c;
    }
}

// Sources with more than kHpRegMax candidates: merged in LDS, kHpMergeCap at a
// time.
// One LDS merge round: the wave's reservoir w.key/w.val[0, n_old) and new
// candidates w.key/w.val[n_old, N) become the merged reservoir in
// w.tkey/w.thash[0, result), ascending in total order; returns its size.
__device__ uint32_t lds_merge_round(HpWaveLds &w, uint32_t n_old, uint32_t N, uint32_t l_max, uint32_t lane) {
    uint32_t P = 64;
    while (P < N) P <<= 1;
    for (uint32_t e = N + lane; e < P; e += 64) {
        w.key[e] = ~0ull;
        w.val[e] = 0xffffffffu;  // after every real hash (<= 0xffff)
    }
    __builtin_amdgcn_wave_barrier();
    // each hash's best first: sort by (hash, total-order key)
    wave_bitonic_hk(w.val, w.key, P, lane);
    const uint32_t E = P / 64;
    const uint32_t eb = lane * E;
    // kept = first of its hash, compacted into tkey / thash
    uint32_t kcount = 0;
    for (uint32_t q = 0; q < E; ++q) {
        const uint32_t e = eb + q;
        kcount += (e < N && (e == 0 || w.val[e - 1] != w.val[e])) ? 1u : 0u;
    }
    uint32_t n_kept;
    uint32_t run = wave_excl_scan(kcount, lane, n_kept);
    for (uint32_t q = 0; q < E; ++q) {
        const uint32_t e = eb + q;
        if (e < N && (e == 0 || w.val[e - 1] != w.val[e])) {
            w.tkey[run] = w.key[e];
            w.thash[run] = w.val[e];
            ++run;
        }
    }
    // the kept by total order; the first l_max of them remain
    uint32_t P2 = 64;
    while (P2 < n_kept) P2 <<= 1;
    for (uint32_t e = n_kept + lane; e < P2; e += 64) {
        w.tkey[e] = ~0ull;
        w.thash[e] = 0xffffffffu;
    }
    __builtin_amdgcn_wave_barrier();
    wave_bitonic<uint64_t>(w.tkey, w.thash, P2, lane);
    __builtin_amdgcn_wave_barrier();
    return n_kept < l_max ? n_kept : l_max;
}

// Sources with more than kHpRegMax candidates: merged in LDS, kHpMergeCap at a
// time.
__global__ __launch_bounds__(kHpThreads) void hp_merge_large_kernel(const uint4 *grouped, const uint32_t *offsets,
                                                                    uint32_t num_points, uint32_t l_max,
                                                                    uint64_t *slot_keys, uint16_t *slot_hash,
                                                                    uint32_t *slot_count) {
    __shared__ HpWaveLds lds[kHpWaves];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    HpWaveLds &w = lds[wave];
    const uint32_t waves = gridDim.x * kHpWaves;
    for (uint32_t src = blockIdx.x * kHpWaves + wave; src < num_points; src += waves) {
        const uint32_t off = offsets[src];
        const uint32_t n_new = offsets[src + 1] - off;
        if (n_new == 0) continue;
        uint32_t n_old = slot_count[src];
        if (n_old + n_new <= kHpRegMax) continue;  // merged by hp_merge_small_kernel
        const uint64_t sbase = (uint64_t)src * l_max;
        for (uint32_t e = lane; e < n_old; e += 64) {
            w.key[e] = slot_keys[sbase + e];
            w.val[e] = slot_hash[sbase + e];
        }
        uint32_t used = 0;
        while (used < n_new) {
            const uint32_t take = (n_new - used < kHpMergeCap - n_old) ? n_new - used : kHpMergeCap - n_old;
            for (uint32_t e = lane; e < take; e += 64) {
                const uint4 r = grouped[off + used + e];
                w.key[n_old + e] = ((uint64_t)total_key(__uint_as_float(r.w)) << 32) | r.y;
                w.val[n_old + e] = r.z & 0xffffu;
            }
            n_old = lds_merge_round(w, n_old, n_old + take, l_max, lane);
            used += take;
            if (used < n_new) {
                for (uint32_t e = lane; e < n_old; e += 64) {
                    w.key[e] = w.tkey[e];
                    w.val[e] = w.thash[e];
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        for (uint32_t e = lane; e < n_old; e += 64) {
            slot_keys[sbase + e] = w.tkey[e];
            slot_hash[sbase + e] = (uint16_t)w.thash[e];
        }
        if (lane == 0) slot_count[src] = n_old;
        __builtin_amdgcn_wave_barrier();
    }
}

// ---- segment mode: records left where the emitter put them ------------------
// A segment {src, first record lo/hi, count} names a run of records of one
// source.  The batch's segments are sorted by source (radix sort of the
// segment indices), each run of equal sources becomes one active source, and
// the merges walk the active sources only, reading each one's records in
// place: the work follows the batch size, with no pass over all points and
// no atomics per record.

__global__ void hp_seg_keys_kernel(const uint4 *segs, uint64_t nseg, uint32_t num_points, uint32_t *keys,
                                   uint32_t *vals, uint64_t *status) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nseg; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint4 g = segs[i];
        const bool bad = g.w != 0u && g.x >= num_points;
        // the first record of the segment carries the bad source
        if (bad) atomicMin((unsigned long long *)status, (unsigned long long)(((uint64_t)g.z << 32) | g.y));
        keys[i] = (g.w == 0u || bad) ? num_points : g.x;  // empty and bad segments sort last, unused
        vals[i] = (uint32_t)i;
    }
}

// The segment descriptors in sorted order (one gather, so the merge reads a
// source's segments contiguously).
__global__ void hp_seg_gather_kernel(const uint4 *segs, const uint32_t *order, uint64_t nseg, uint4 *sorted) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nseg; i += (uint64_t)gridDim.x * blockDim.x)
        sorted[i] = segs[order[i]];
}

// ---- streaming merge of a source's segments ----------------------------------
// Every merge leaves a reservoir's slots ascending in total order (the export
// sorts them by hash, the reference's emit order).  One wave per active source
// holds the reservoir in registers (slot position q*64 + lane in register q,
// ER = ceil(l_max / 64) registers) and streams the source's records through
// it 64 at a time.  A full reservoir's last slot bounds what can still enter:
// a candidate no better than it either repeats a slot's hash with a worse (or
// equal) key or is worse than l_max slots of distinct hashes, so it is
// dropped by one compare.  The candidates that pass are inserted one at a time
// (the reference's insert: a hash hit keeps the better, a new hash fills a
// free slot or replaces the worst) by a rank ballot and a one-position shift;
// a first chunk into an empty reservoir is sorted instead.

constexpr uint32_t kBatchMin = 24;  // passing candidates of a chunk into an empty reservoir that are sorted

__device__ __forceinline__ bool ent_less(uint64_t ka, uint32_t ha, uint64_t kb, uint32_t hb) {
    return ka < kb || (ka == kb && ha < hb);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, uint32_t l) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), (int)l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, (int)l);
}
__device__ __forceinline__ uint32_t readlane32(uint32_t v, uint32_t l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}
__device__ __forceinline__ uint64_t ballot64(bool pred) { return __builtin_amdgcn_ballot_w64(pred); }

template <int ER>
struct Reservoir {
    uint64_t k[ER];  // live positions [0, c) ascending by (k, h); the rest k = ~0, h = 0xffffffff
    uint32_t h[ER];
    uint32_t c;
};

// Key / hash at position pos (the same in every lane).
template <int ER>
__device__ __forceinline__ void res_at(const Reservoir<ER> &r, uint32_t pos, uint64_t &k, uint32_t &h) {
    uint64_t kk = r.k[0];
    uint32_t hh = r.h[0];
#pragma unroll
    for (int q = 1; q < ER; ++q) {
        kk = pos / 64u == (uint32_t)q ? r.k[q] : kk;
        hh = pos / 64u == (uint32_t)q ? r.h[q] : hh;
    }
    k = readlane64(kk, pos & 63u);
    h = readlane32(hh, pos & 63u);
}

// Positions (p, end] take the entry before them; position p takes (bk, bh).
template <int ER>
__device__ __forceinline__ void res_shift_in(Reservoir<ER> &r, uint32_t p, uint32_t end, uint64_t bk, uint32_t bh,
                                             uint32_t lane) {
#pragma unroll
    for (int q = ER - 1; q >= 0; --q) {
        if ((uint32_t)q * 64u > end || (uint32_t)q * 64u + 63u < p) continue;  // register untouched
        const uint32_t lo = __shfl_up((uint32_t)r.k[q], 1);
        const uint32_t hi = __shfl_up((uint32_t)(r.k[q] >> 32), 1);
        uint64_t uk = ((uint64_t)hi << 32) | lo;
        uint32_t uh = __shfl_up(r.h[q], 1);
        if (q > 0) {
            const uint64_t ck = readlane64(r.k[q - 1], 63);
            const uint32_t ch = readlane32(r.h[q - 1], 63);
            uk = lane == 0 ? ck : uk;
            uh = lane == 0 ? ch : uh;
        }
        const uint32_t e = (uint32_t)q * 64u + lane;
        const bool mv = e > p && e <= end;
        r.k[q] = e == p ? bk : (mv ? uk : r.k[q]);
        r.h[q] = e == p ? bh : (mv ? uh : r.h[q]);
    }
}

// Inserts candidate (bk, bh), the same in every lane (r.c, p, hit and the
// decision are wave-uniform, so they stay scalar).
template <int ER>
__device__ __forceinline__ void res_insert(Reservoir<ER> &r, uint64_t bk, uint32_t bh, uint32_t l_max,
                                           uint32_t lane) {
    uint32_t p = 0;                // slots before the candidate in total order
    uint32_t hit = 0xffffffffu;    // the slot of its hash
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        const bool live = (uint32_t)q * 64u + lane < r.c;
        p += (uint32_t)__popcll(ballot64(live && ent_less(r.k[q], r.h[q], bk, bh)));
        const uint64_t m = ballot64(live && r.h[q] == bh);
        hit = m ? (uint32_t)q * 64u + (uint32_t)__builtin_ctzll(m) : hit;
    }
    bool go;
    uint32_t end;
    if (hit != 0xffffffffu) {
        // a hash hit: the candidate replaces the slot when it is better (a
        // better or equal slot sorts before it, hit < p, or is the same key)
        uint64_t ek;
        uint32_t eh;
        res_at(r, hit, ek, eh);
        go = hit >= p && ek != bk;
        end = hit;
    } else if (r.c < l_max) {
        go = true;  // a free slot
        end = r.c;
        r.c = r.c + 1u;
    } else {
        go = p < l_max;  // the worst slot goes unless the candidate is worse than every slot
        end = l_max - 1u;
    }
    if (go) res_shift_in(r, p, end, bk, bh, lane);
}

// Merges one chunk (candidate (ck, ch) in each lane where v) into the reservoir.
template <int ER>
__device__ __forceinline__ void res_chunk(Reservoir<ER> &r, uint64_t ck, uint32_t ch, bool v, uint32_t l_max, uint32_t lane) {
    bool pass = v;
    if (r.c == l_max) {
        uint64_t wk;
        uint32_t wh;
        res_at(r, l_max - 1u, wk, wh);
        pass = v && ent_less(ck, ch, wk, wh);
    }
    uint64_t pm = ballot64(pass);
    if (pm == 0) return;
    if (r.c == 0 && (uint32_t)__popcll(pm) >= kBatchMin) {
        uint32_t h[1] = {pass ? ch : 0xffffffffu};
        uint64_t k[1] = {pass ? ck : ~0ull};
        r.c = (uint32_t)__builtin_amdgcn_readfirstlane((int)select_sorted<1>(h, k, l_max, lane));
        r.k[0] = k[0];
        r.h[0] = h[0];
        return;
    }
    while (pm) {
        const uint32_t j = (uint32_t)__builtin_ctzll(pm);
        pm &= pm - 1ull;
        res_insert(r, readlane64(ck, j), readlane32(ch, j), l_max, lane);
    }
}

// What a wave loads for one active source before merging it: its segment
// descriptors (lane s: the run's segment s, for s < 64) and its slots.
template <int ER>
struct SourceLoad {
    uint32_t src, start, len;  // run: sorted segments [start, start + len)
    uint32_t cnt;              // lane's segment: record count and first record
    uint64_t first;
    uint32_t c;
    uint64_t k[ER];
    uint32_t h[ER];
};

template <int ER>
__device__ __forceinline__ void load_source(SourceLoad<ER> &L, uint32_t src, uint32_t start, uint32_t len,
                                            const uint4 *sorted, uint32_t num_points, uint32_t l_max,
                                            const uint64_t *slot_keys, const uint16_t *slot_hash,
                                            const uint32_t *slot_count, uint32_t lane) {
    L.src = src;
    L.start = start;
    L.len = len;
    L.cnt = 0;
    L.first = 0;
    L.c = 0;
    const bool real = src < num_points;  // the run of empty / bad segments sorts last
    if (real && lane < len) {
        const uint4 g = sorted[(uint64_t)start + lane];
        L.cnt = g.w;
        L.first = ((uint64_t)g.z << 32) | g.y;
    }
    const uint64_t sbase = (uint64_t)(real ? src : 0u) * l_max;
    if (real) L.c = slot_count[src];
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        // every slot position is read (not only the live ones), so these loads
        // do not wait for the count
        const uint32_t e = (uint32_t)q * 64u + lane;
        const bool in = real && e < l_max;
        L.k[q] = in ? slot_keys[sbase + e] : ~0ull;
        L.h[q] = in ? (uint32_t)slot_hash[sbase + e] : 0xffffffffu;
    }
}

// Streams the records of a group of up to 64 segments (lane s: segment s, cnt
// records from first) 64 at a time across segment boundaries into
// chunk(key, hash, valid).
template <typename Chunk>
__device__ __forceinline__ void stream_group(const uint4 *records, uint32_t ng, uint32_t cnt, uint64_t first,
                                             uint32_t lane, Chunk &&chunk) {
    uint32_t total;
    const uint32_t pre = wave_excl_scan(cnt, lane, total);
    uint32_t sg = 0;  // first segment not yet wholly read
    for (uint32_t c0 = 0; c0 < total; c0 += 64) {
        const uint32_t p = c0 + lane;
        uint64_t addr = 0;
        for (uint32_t s = sg; s < ng; ++s) {
            const uint32_t ps = readlane32(pre, s);
            if (ps >= c0 + 64u) break;
            const uint32_t cs = readlane32(cnt, s);
            const uint64_t fs = readlane64(first, s);
            addr = (p >= ps && p < ps + cs) ? fs + (p - ps) : addr;
            if (ps + cs <= c0 + 64u) sg = s + 1;
        }
        const bool v = p < total;
        uint64_t ck = ~0ull;
        uint32_t ch = 0xffffffffu;
        if (v) {
            const uint4 rec = records[addr];
            ck = ((uint64_t)total_key(__uint_as_float(rec.w)) << 32) | rec.y;
            ch = rec.z & 0xffffu;
        }
        chunk(ck, ch, v);
    }
}

template <int ER>
__device__ __forceinline__ void merge_group(Reservoir<ER> &r, const uint4 *records, uint32_t ng, uint32_t cnt,
                                            uint64_t first, uint32_t l_max, uint32_t lane) {
    stream_group(records, ng, cnt, first, lane,
                 [&](uint64_t ck, uint32_t ch, bool v) { res_chunk(r, ck, ch, v, l_max, lane); });
}

// Active sources in ascending source order (run-length encoding of the sorted
// segment keys).  Each wave walks its sources with the next source's
// segments and slots, and the one after's run, already in flight.
template <int ER>
__global__ __launch_bounds__(kHpThreads) void hp_merge_stream_kernel(const uint4 *records, const uint4 *sorted,
                                                                     const uint32_t *run_src,
                                                                     const uint32_t *run_start,
                                                                     const uint32_t *run_len,
                                                                     const uint32_t *num_runs, uint32_t num_points,
                                                                     uint32_t l_max, uint64_t *slot_keys,
                                                                     uint16_t *slot_hash, uint32_t *slot_count) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t waves = gridDim.x * kHpWaves;
    const uint32_t na = *num_runs;
    uint32_t a = blockIdx.x * kHpWaves + wave;
    if (a >= na) return;
    SourceLoad<ER> cur;
    load_source(cur, run_src[a], run_start[a], run_len[a], sorted, num_points, l_max, slot_keys, slot_hash,
                slot_count, lane);
    uint32_t d_src = num_points, d_start = 0, d_len = 0;  // run of the next source
    if (a + waves < na) {
        d_src = run_src[a + waves];
        d_start = run_start[a + waves];
        d_len = run_len[a + waves];
    }
    for (; a < na; a += waves) {
        SourceLoad<ER> nxt;
        load_source(nxt, d_src, d_start, d_len, sorted, num_points, l_max, slot_keys, slot_hash, slot_count, lane);
        const uint32_t a2 = a + 2u * waves;
        d_src = num_points;
        d_len = 0;
        if (a2 < na) {
            d_src = run_src[a2];
            d_start = run_start[a2];
            d_len = run_len[a2];
        }
        const uint32_t src = cur.src;
        if (src < num_points) {
            Reservoir<ER> r;
            r.c = (uint32_t)__builtin_amdgcn_readfirstlane((int)cur.c);
#pragma unroll
            for (int q = 0; q < ER; ++q) {
                const bool live = (uint32_t)q * 64u + lane < r.c;
                r.k[q] = live ? cur.k[q] : ~0ull;
                r.h[q] = live ? cur.h[q] : 0xffffffffu;
            }
            merge_group(r, records, cur.len < 64u ? cur.len : 64u, cur.cnt, cur.first, l_max, lane);
            for (uint32_t g0 = 64; g0 < cur.len; g0 += 64) {
                // a source with more than 64 segments in the batch: the rest, 64 at a time
                const uint32_t ng = cur.len - g0 < 64u ? cur.len - g0 : 64u;
                uint32_t cnt = 0;
                uint64_t first = 0;
                if (lane < ng) {
                    const uint4 g = sorted[(uint64_t)cur.start + g0 + lane];
                    cnt = g.w;
                    first = ((uint64_t)g.z << 32) | g.y;
                }
                merge_group(r, records, ng, cnt, first, l_max, lane);
            }
            const uint64_t sbase = (uint64_t)src * l_max;
#pragma unroll
            for (int q = 0; q < ER; ++q) {
                const uint32_t e = (uint32_t)q * 64u + lane;
                if (e < r.c) {
                    slot_keys[sbase + e] = r.k[q];
                    slot_hash[sbase + e] = (uint16_t)r.h[q];
                }
            }
            if (lane == 0) slot_count[src] = r.c;
        }
        cur = nxt;
    }
}

// Segment workspace layout (nseg entries each unless noted): sort keys and
// values in / out (u32), run sources, lengths and starts (u32), the run count
// (one u32), the segment descriptors in sorted order (uint4), then the
// temporary of the radix sort / run-length encoding / scan.
struct SegWs {
    uint32_t *keys_in, *keys_out, *vals_in, *vals_out, *run_src, *run_len, *run_start, *num_runs;
    uint4 *sorted;
    void *temp;
    size_t temp_bytes;
};
size_t seg_align(size_t x) { return (x + 255) & ~(size_t)255; }
int key_bits(uint32_t num_points) {
    int b = 1;
    while (b < 32 && ((uint64_t)1 << b) <= num_points) ++b;  // keys go up to num_points (unused segments)
    return b;
}
size_t seg_temp(uint64_t nseg, uint32_t num_points) {
    size_t sort = 0, rle = 0, scan = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, sort, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                       (const uint32_t *)nullptr, (uint32_t *)nullptr, (int)nseg, 0,
                                       key_bits(num_points));
    (void)hipcub::DeviceRunLengthEncode::Encode(nullptr, rle, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                          (uint32_t *)nullptr, (uint32_t *)nullptr, (int)nseg);
    (void)hipcub::DeviceScan::ExclusiveSum(nullptr, scan, (const uint32_t *)nullptr, (uint32_t *)nullptr, (int)nseg);
    return sort > rle ? (sort > scan ? sort : scan) : (rle > scan ? rle : scan);
}
SegWs seg_ws_layout(void *base, uint64_t nseg, uint32_t num_points) {
    SegWs w{};
    char *p = static_cast<char *>(base);
    const size_t a = seg_align(nseg * 4);
    uint32_t **arr[7] = {&w.keys_in, &w.keys_out, &w.vals_in, &w.vals_out, &w.run_src, &w.run_len, &w.run_start};
    for (int i = 0; i < 7; ++i) *arr[i] = reinterpret_cast<uint32_t *>(p + i * a);
    w.num_runs = reinterpret_cast<uint32_t *>(p + 7 * a);
    w.sorted = reinterpret_cast<uint4 *>(p + 7 * a + 256);
    w.temp = p + 7 * a + 256 + seg_align(nseg * 16);
    w.temp_bytes = seg_temp(nseg, num_points);
    return w;
}

// One wave per point: its slots sorted by hash (a reservoir's hashes are
// distinct, so the order is the reference's emit order, ascending hash).
template <int ER>
__global__ __launch_bounds__(kHpThreads) void hp_export_kernel(const uint64_t *slot_keys, const uint16_t *slot_hash,
                                                               const uint32_t *slot_count, uint32_t num_points,
                                                               uint32_t l_max, uint32_t *targets, uint16_t *hashes,
                                                               float *dists, uint32_t *counts) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t waves = gridDim.x * kHpWaves;
    for (uint32_t p = blockIdx.x * kHpWaves + (threadIdx.x >> 6); p < num_points; p += waves) {
        const uint32_t c = slot_count[p];
        const uint64_t base = (uint64_t)p * l_max;
        uint32_t h[ER];
        uint64_t k[ER];
#pragma unroll
        for (int q = 0; q < ER; ++q) {
            const uint32_t e = (uint32_t)q * 64u + lane;
            h[q] = e < c ? (uint32_t)slot_hash[base + e] : 0xffffffffu;
            k[q] = e < c ? slot_keys[base + e] : ~0ull;
        }
        reg_bitonic<ER, true>(h, k, lane);
#pragma unroll
        for (int q = 0; q < ER; ++q) {
            const uint32_t e = (uint32_t)q * 64u + lane;
            if (e >= l_max) continue;
            const bool live = e < c;
            if (targets) targets[base + e] = live ? (uint32_t)k[q] : 0xffffffffu;
            if (hashes) hashes[base + e] = live ? (uint16_t)h[q] : (uint16_t)0;
            if (dists) dists[base + e] = live ? key_dist((uint32_t)(k[q] >> 32)) : 0.0f;
        }
        if (counts && lane == 0) counts[p] = c;
    }
}

// ---- named R-half backfill ----------------------------------------------------
// The reference's order-independent characterization of its R-half streaming
// reservoir (shear-core/src/algorithm/pipnn/hash_prune.rs:2601-2682
// reference_tiered_rhalf_slots; ranking :655-685, capacities
// hash_prune_backfill.rs:299-336, SoftTier score :375-386): a row with some
// but fewer than l_max primaries is completed with up to `capacity` backups,
// chosen by the mode's priority among each primary hash's next `quota`
// distinct targets (each at its best key, the primary's own target
// excluded; a member's hit layer is its rank in its group).
//
// Each slot keeps its hash's best quota + 1 distinct targets: the slot key and
// a group of quota keys.  That set does not depend on the order of the
// candidates (a target dropped from it had quota + 1 better distinct targets
// of the hash, whose keys only improve), so batches still merge in any
// order.  A reservoir that has filled never frees a slot and a full row takes
// no backups, so groups are kept only while a slot is free; nothing is
// evicted then either, so those slots are kept unsorted (a candidate is one
// hash ballot and an append or an in-place update).  The insert that fills
// the reservoir sorts it in total order, the plain insert takes over, and the
// groups are neither read nor written again.

template <int ER>
struct GroupReservoir {
    Reservoir<ER> b;
    uint64_t g[ER][kRhalfGroup];  // the lane's slot's group, ascending keys, ~0 = none
};

// The hash's best quota + 1 distinct targets (s[0] the slot key, s[1..] its
// group, ascending, ~0 = none) with candidate bk added: its target keeps its
// better key; a new target takes position quota when better than what is
// there; one backward pass restores the order.
static_assert(kRhalfGroup == 3, "a group is three keys");
__device__ __forceinline__ void group_update(uint64_t (&s)[kRhalfGroup + 1], uint64_t bk, uint32_t quota) {
    const uint32_t bt = (uint32_t)bk;
    bool present = false;
#pragma unroll
    for (uint32_t j = 0; j <= kRhalfGroup; ++j) {
        const bool m = j <= quota && s[j] != ~0ull && (uint32_t)s[j] == bt;
        present = present || m;
        s[j] = m && bk < s[j] ? bk : s[j];
    }
#pragma unroll
    for (uint32_t j = 0; j <= kRhalfGroup; ++j) s[j] = !present && j == quota && bk < s[j] ? bk : s[j];
#pragma unroll
    for (int j = kRhalfGroup; j >= 1; --j) {
        const uint64_t lo = s[j] < s[j - 1] ? s[j] : s[j - 1];
        const uint64_t hi = s[j] < s[j - 1] ? s[j - 1] : s[j];
        s[j - 1] = lo;
        s[j] = hi;
    }
}

// Inserts candidate (bk, bh) into a reservoir with a free slot.  While a slot
// is free the slots are kept in no particular order (nothing is evicted, so no
// rank is needed): a new hash is appended with an empty group, a repeat of a
// slot's own (target, distance) (a pair seen forward and reverse) changes
// nothing, and any other candidate of a slot's hash updates that slot's best
// quota + 1 distinct targets in the owner lane (the slot key is the best of
// them, the group the rest).  The first two are selects; only the third
// branches.
template <int ER>
__device__ __forceinline__ void gres_fill_insert(GroupReservoir<ER> &r, uint64_t bk, uint32_t bh, uint32_t quota,
                                                 uint32_t lane) {
    uint32_t hit = 0xffffffffu;
    uint64_t ek = 0;
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        const bool live = (uint32_t)q * 64u + lane < r.b.c;
        const uint64_t m = ballot64(live && r.b.h[q] == bh);
        if (m) {
            const uint32_t l = (uint32_t)__builtin_ctzll(m);
            hit = (uint32_t)q * 64u + l;
            ek = readlane64(r.b.k[q], l);
        }
    }
    const bool is_new = hit == 0xffffffffu;
    const uint32_t e = r.b.c, eq = e >> 6;
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        const bool at = is_new && eq == (uint32_t)q && lane == (e & 63u);
        r.b.k[q] = at ? bk : r.b.k[q];
        r.b.h[q] = at ? bh : r.b.h[q];
#pragma unroll
        for (uint32_t j = 0; j < kRhalfGroup; ++j) r.g[q][j] = at ? ~0ull : r.g[q][j];
    }
    r.b.c = e + (is_new ? 1u : 0u);
    if (is_new || ek == bk) return;
    const uint32_t hq = hit >> 6, hl = hit & 63u;
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        if (hq != (uint32_t)q) continue;
        uint64_t s[kRhalfGroup + 1] = {r.b.k[q], r.g[q][0], r.g[q][1], r.g[q][2]};
        group_update(s, bk, quota);
        const bool own = lane == hl;
        r.b.k[q] = own ? s[0] : r.b.k[q];
#pragma unroll
        for (uint32_t j = 0; j < kRhalfGroup; ++j) r.g[q][j] = own ? s[j + 1] : r.g[q][j];
    }
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_up64(uint64_t v) {
    const uint32_t lo = __shfl_up((uint32_t)v, 1);
    const uint32_t hi = __shfl_up((uint32_t)(v >> 32), 1);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_down64(uint64_t v, uint32_t d) {
    const uint32_t lo = __shfl_down((uint32_t)v, d);
    const uint32_t hi = __shfl_down((uint32_t)(v >> 32), d);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t permute64(uint32_t dest, uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_permute((int)(dest * 4u), (int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_permute((int)(dest * 4u), (int)(uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Ascending bitonic sort of one (a, b) pair per lane across the wave,
// lexicographic.
__device__ __forceinline__ void wave_sort_pair(uint64_t &a, uint64_t &b, uint32_t lane) {
#pragma unroll
    for (uint32_t kk = 2; kk <= 64u; kk <<= 1) {
#pragma unroll
        for (uint32_t j = kk >> 1; j > 0; j >>= 1) {
            const uint64_t pa = shfl_xor64(a, (int)j), pb = shfl_xor64(b, (int)j);
            const bool want_min = ((lane & j) == 0) == ((lane & kk) == 0);
            const bool p_less = pa < a || (pa == a && pb < b);
            const bool p_more = a < pa || (a == pa && b < pb);
            const bool take = want_min ? p_less : p_more;
            a = take ? pa : a;
            b = take ? pb : b;
        }
    }
}

// A chunk (candidate (ck, ch) in each lane where v) into an empty reservoir,
// by sorting instead of one insert per candidate: the candidates sorted by
// (hash, target, key) drop repeats of a (hash, target); sorted by (hash,
// key), each hash's first is its slot and the next `quota` its group.  With
// l_max hashes or more the reservoir fills: each hash's best, the l_max best
// of those, sorted in total order (select_sorted).  Otherwise the slots are
// moved to positions [0, hashes) (one push permute per word).
template <int ER>
__device__ __forceinline__ void gres_batch_fill(GroupReservoir<ER> &r, uint64_t ck, uint32_t ch, bool v, uint32_t l_max,
                                uint32_t quota, uint32_t lane) {
    uint64_t a = v ? ((uint64_t)ch << 32) | (uint32_t)ck : ~0ull;  // (hash, target)
    uint64_t b = v ? (ck >> 32) : ~0ull;                             // distance key
    wave_sort_pair(a, b, lane);
    const uint64_t ap = shfl_up64(a);
    const bool keep = a != ~0ull && (lane == 0 || ap != a);  // a target's best within its hash
    uint64_t hs = keep ? (a >> 32) : ~0ull;
    uint64_t k = keep ? ((b << 32) | (uint32_t)a) : ~0ull;
    wave_sort_pair(hs, k, lane);
    const uint32_t h = (uint32_t)hs;  // 0xffffffff for the empty entries after the real ones
    const uint32_t hp = __shfl_up(h, 1);
    const bool start = h != 0xffffffffu && (lane == 0 || hp != h);
    const uint64_t S = ballot64(start);
    const uint32_t m = (uint32_t)__popcll(S);
    if (m >= l_max) {
        uint32_t rh[ER];
        uint64_t rk[ER];
#pragma unroll
        for (int q = 0; q < ER; ++q) {
            rh[q] = q == 0 ? h : 0xffffffffu;
            rk[q] = q == 0 ? k : ~0ull;
        }
        r.b.c = (uint32_t)__builtin_amdgcn_readfirstlane((int)select_sorted<ER>(rh, rk, l_max, lane));
#pragma unroll
        for (int q = 0; q < ER; ++q) {
            r.b.h[q] = rh[q];
            r.b.k[q] = rk[q];
        }
        return;
    }
    // rank of each entry within its hash: lanes since the last start at or before it
    const uint64_t upto = lane == 63u ? ~0ull : ((2ull << lane) - 1ull);
    const uint32_t rank = lane - (63u - (uint32_t)__builtin_clzll(S & upto));
    uint64_t g[kRhalfGroup];
#pragma unroll
    for (uint32_t j = 1; j <= kRhalfGroup; ++j) {
        const uint64_t kd = shfl_down64(k, j);
        const uint32_t rd = __shfl_down(rank, j);
        const uint32_t hd = __shfl_down(h, j);
        g[j - 1] = lane + j < 64u && j <= quota && hd == h && rd == j ? kd : ~0ull;
    }
    // slots to [0, m), the other entries after them
    const uint32_t below = (uint32_t)__popcll(S & ((1ull << lane) - 1ull));
    const uint32_t dest = start ? below : m + (lane - below);
    const uint64_t sk = permute64(dest, k);
    const uint32_t sh = (uint32_t)__builtin_amdgcn_ds_permute((int)(dest * 4u), (int)h);
    uint64_t sg[kRhalfGroup];
#pragma unroll
    for (uint32_t j = 0; j < kRhalfGroup; ++j) sg[j] = permute64(dest, g[j]);
    const bool live = lane < m;
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        r.b.k[q] = q == 0 && live ? sk : ~0ull;
        r.b.h[q] = q == 0 && live ? sh : 0xffffffffu;
#pragma unroll
        for (uint32_t j = 0; j < kRhalfGroup; ++j) r.g[q][j] = q == 0 && live ? sg[j] : ~0ull;
    }
    r.b.c = m;
}

// Merges one chunk.  A full reservoir takes the plain path (res_chunk: slots
// sorted in total order, the one-compare bound); a first chunk of at least
// kBatchMin candidates into an empty one is sorted in (gres_batch_fill).
// Otherwise the candidates go in one at a time; the insert that fills the
// reservoir sorts its slots in total order (the plain path's invariant) and
// the rest of the chunk takes the plain path.
template <int ER>
__device__ __forceinline__ void gres_chunk(GroupReservoir<ER> &r, uint64_t ck, uint32_t ch, bool v, uint32_t l_max, uint32_t quota,
                           uint32_t lane) {
    if (r.b.c == l_max) {
        res_chunk(r.b, ck, ch, v, l_max, lane);
        return;
    }
    uint64_t pm = ballot64(v);
    if (r.b.c == 0 && (uint32_t)__popcll(pm) >= kBatchMin) {
        gres_batch_fill(r, ck, ch, v, l_max, quota, lane);
        return;
    }
    while (pm) {
        const uint32_t j = (uint32_t)__builtin_ctzll(pm);
        pm &= pm - 1ull;
        gres_fill_insert(r, readlane64(ck, j), readlane32(ch, j), quota, lane);
        if (r.b.c == l_max) {
            reg_bitonic<ER, false>(r.b.h, r.b.k, lane);
            res_chunk(r.b, ck, ch, v && lane > j, l_max, lane);
            return;
        }
    }
}

// A source's run as the merge needs it: source (num_points: nothing to
// merge), its sorted segments [start, start + len), the lane's segment
// (records cnt from first), and its slot count.
struct RunInfo {
    uint32_t src, start, len, cnt, c;
    uint64_t first;
};

template <bool kGrouped>
__device__ __forceinline__ RunInfo run_info(uint32_t a, uint32_t na, const uint4 *sorted, const uint32_t *run_src,
                                            const uint32_t *run_start, const uint32_t *run_len,
                                            const uint32_t *offsets, uint32_t num_points,
                                            const uint32_t *slot_count, uint32_t lane) {
    RunInfo ri{num_points, 0u, 1u, 0u, 0u, 0ull};
    if (a >= na) return ri;
    if (kGrouped) {
        const uint32_t o0 = offsets[a], o1 = offsets[a + 1];
        if (o1 == o0) return ri;
        ri.src = a;
        ri.cnt = lane == 0 ? o1 - o0 : 0u;
        ri.first = o0;
    } else {
        const uint32_t src = run_src[a];
        if (src >= num_points) return ri;  // the run of empty / bad segments
        ri.src = src;
        ri.start = run_start[a];
        ri.len = run_len[a];
        if (lane < ri.len) {
            const uint4 g = sorted[(uint64_t)ri.start + lane];
            ri.cnt = g.w;
            ri.first = ((uint64_t)g.z << 32) | g.y;
        }
    }
    ri.c = slot_count[ri.src];
    return ri;
}

// A source's live slots (prefetched one source ahead).
template <int ER>
__device__ __forceinline__ void load_slots(Reservoir<ER> &r, const RunInfo &ri, uint32_t num_points,
                                           uint32_t l_max, const uint64_t *slot_keys, const uint16_t *slot_hash,
                                           uint32_t lane) {
    const bool real = ri.src < num_points;
    const uint32_t c = real ? ri.c : 0u;
    const uint64_t sbase = (uint64_t)(real ? ri.src : 0u) * l_max;
#pragma unroll
    for (int q = 0; q < ER; ++q) {
        const uint32_t e = (uint32_t)q * 64u + lane;
        const bool live = e < c;
        r.k[q] = live ? slot_keys[sbase + e] : ~0ull;
        r.h[q] = live ? (uint32_t)slot_hash[sbase + e] : 0xffffffffu;
    }
}

// One wave per source with new records: its slots (and, while a slot is free,
// their groups) in registers, its records streamed through them.  Sources
// come from segment runs (as hp_merge_stream_kernel) or, kGrouped, from the
// record batch grouped by source (offsets[src] .. offsets[src + 1]).  Each
// wave walks its sources with the next source's slots, and the one after's
// run and slot count, already in flight.  Five waves per SIMD (a few
// registers of the rarely taken paths spill) beat the four that fit without
// spilling: the kernel is bound by latency more than by its instructions.
template <int ER, bool kGrouped>
__global__ __launch_bounds__(kHpThreads) __attribute__((amdgpu_waves_per_eu(5))) void hp_merge_rhalf_kernel(
    const uint4 *records, const uint4 *sorted, const uint32_t *run_src, const uint32_t *run_start,
    const uint32_t *run_len, const uint32_t *num_runs, const uint32_t *offsets, uint32_t num_points, uint32_t l_max,
    uint32_t quota, uint64_t *slot_keys, uint16_t *slot_hash, uint32_t *slot_count, uint64_t *grp_keys) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t waves = gridDim.x * kHpWaves;
    const uint32_t na = kGrouped ? num_points : *num_runs;
    uint32_t a = blockIdx.x * kHpWaves + (threadIdx.x >> 6);
    if (a >= na) return;
    auto info = [&](uint32_t i) {
        return run_info<kGrouped>(i, na, sorted, run_src, run_start, run_len, offsets, num_points, slot_count,
                                  lane);
    };
    RunInfo cur_ri = info(a);
    Reservoir<ER> cur;
    load_slots(cur, cur_ri, num_points, l_max, slot_keys, slot_hash, lane);
    RunInfo nxt_ri = info(a + waves);
    for (; a < na; a += waves) {
        Reservoir<ER> nxt;
        load_slots(nxt, nxt_ri, num_points, l_max, slot_keys, slot_hash, lane);
        const RunInfo far_ri = info(a + 2u * waves);
        const uint32_t src = cur_ri.src;
        if (src < num_points) {
            GroupReservoir<ER> r;
            r.b = cur;
            r.b.c = (uint32_t)__builtin_amdgcn_readfirstlane((int)cur_ri.c);
            const uint64_t sbase = (uint64_t)src * l_max;
            // the groups of a reservoir with a free slot (its slots' only)
            const bool groups = r.b.c > 0u && r.b.c < l_max;
#pragma unroll
            for (int q = 0; q < ER; ++q) {
                const uint32_t e = (uint32_t)q * 64u + lane;
#pragma unroll
                for (uint32_t j = 0; j < kRhalfGroup; ++j)
                    r.g[q][j] = groups && e < r.b.c ? grp_keys[(sbase + e) * kRhalfGroup + j] : ~0ull;
            }
            const uint32_t len = cur_ri.len;
            auto chunk = [&](uint64_t ck, uint32_t ch, bool v) { gres_chunk(r, ck, ch, v, l_max, quota, lane); };
            stream_group(records, len < 64u ? len : 64u, cur_ri.cnt, cur_ri.first, lane, chunk);
            for (uint32_t g0 = 64; g0 < len; g0 += 64) {
                // a source with more than 64 segments in the batch: the rest, 64 at a time
                const uint32_t ng = len - g0 < 64u ? len - g0 : 64u;
                uint32_t c2 = 0;
                uint64_t f2 = 0;
                if (lane < ng) {
                    const uint4 g = sorted[(uint64_t)cur_ri.start + g0 + lane];
                    c2 = g.w;
                    f2 = ((uint64_t)g.z << 32) | g.y;
                }
                stream_group(records, ng, c2, f2, lane, chunk);
            }
            const bool keep_groups = r.b.c < l_max;
#pragma unroll
            for (int q = 0; q < ER; ++q) {
                const uint32_t e = (uint32_t)q * 64u + lane;
                if (e < r.b.c) {
                    slot_keys[sbase + e] = r.b.k[q];
                    slot_hash[sbase + e] = (uint16_t)r.b.h[q];
                    if (keep_groups) {
#pragma unroll
                        for (uint32_t j = 0; j < kRhalfGroup; ++j)
                            grp_keys[(sbase + e) * kRhalfGroup + j] = r.g[q][j];
                    }
                }
            }
            if (lane == 0) slot_count[src] = r.b.c;
        }
        cur = nxt;
        cur_ri = nxt_ri;
        nxt_ri = far_ri;
    }
}

__device__ __forceinline__ uint64_t total_key64(double d) {
    const uint64_t b = (uint64_t)__double_as_longlong(d);
    return (b & 0x8000000000000000ull) ? ~b : (b | 0x8000000000000000ull);
}

// A group member's rank under the mode's priority (hash_prune.rs:655-685) as
// a 128-bit key (hi, lo); members are distinct (hash, target) pairs, so keys
// are distinct.  SoftTier: (score, layer, target, hash), the score the f64
// distance times alpha^2 per layer past the first (hash_prune_backfill.rs:
// 375-386); HardTier: (layer, distance, target, hash); the others:
// (distance, layer, target, hash).
__device__ __forceinline__ void member_rank(uint32_t mode, double alpha_sq, uint64_t key, uint32_t hash,
                                            uint32_t layer, uint64_t &hi, uint64_t &lo) {
    const uint32_t dk = (uint32_t)(key >> 32);
    const uint64_t th = ((uint64_t)(uint32_t)key << 16) | hash;
    if (mode == kRhalfSoftTierQ3) {
        double s = (double)key_dist(dk);
        if (layer >= 2) s = s * alpha_sq;
        if (layer >= 3) s = s * alpha_sq;
        hi = total_key64(s);
        lo = ((uint64_t)layer << 48) | th;
    } else if (mode == kRhalfHardTierQ3) {
        hi = ((uint64_t)layer << 32) | dk;
        lo = th;
    } else {
        hi = dk;
        lo = ((uint64_t)layer << 48) | th;
    }
}

// hp_export_kernel followed, for a row with some but fewer than l_max
// primaries, by min(capacity, l_max - c) backups: the best group members by
// the mode's priority, one wave-wide arg-min per backup, written after the
// primaries in priority order.
template <int ER>
__global__ __launch_bounds__(kHpThreads) void hp_export_rhalf_kernel(
    const uint64_t *slot_keys, const uint16_t *slot_hash, const uint32_t *slot_count, const uint64_t *grp_keys,
    uint32_t num_points, uint32_t l_max, uint32_t mode, uint32_t quota, uint32_t capacity, double alpha_sq,
    uint32_t *targets, uint16_t *hashes, float *dists, uint32_t *counts) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t waves = gridDim.x * kHpWaves;
    for (uint32_t p = blockIdx.x * kHpWaves + (threadIdx.x >> 6); p < num_points; p += waves) {
        const uint32_t c = slot_count[p];
        const uint64_t base = (uint64_t)p * l_max;
        uint32_t h[ER];
        uint64_t k[ER];
#pragma unroll
        for (int q = 0; q < ER; ++q) {
            const uint32_t e = (uint32_t)q * 64u + lane;
            h[q] = e < c ? (uint32_t)slot_hash[base + e] : 0xffffffffu;
            k[q] = e < c ? slot_keys[base + e] : ~0ull;
        }
        uint32_t take = 0;
        if (c > 0 && c < l_max) {
            const uint32_t cap = capacity < l_max - c ? capacity : l_max - c;
            uint64_t mh[ER][kRhalfGroup], ml[ER][kRhalfGroup];
#pragma unroll
            for (int q = 0; q < ER; ++q) {
                const uint32_t e = (uint32_t)q * 64u + lane;
#pragma unroll
                for (uint32_t j = 0; j < kRhalfGroup; ++j) {
                    const uint64_t g = e < c && j < quota ? grp_keys[(base + e) * kRhalfGroup + j] : ~0ull;
                    mh[q][j] = ~0ull;
                    ml[q][j] = ~0ull;
                    if (g != ~0ull) member_rank(mode, alpha_sq, g, h[q], j + 1u, mh[q][j], ml[q][j]);
                }
            }
            for (; take < cap; ++take) {
                uint64_t bh = ~0ull, bl = ~0ull;
                uint32_t bi = 0;
#pragma unroll
                for (int q = 0; q < ER; ++q) {
#pragma unroll
                    for (uint32_t j = 0; j < kRhalfGroup; ++j) {
                        const bool lt = mh[q][j] < bh || (mh[q][j] == bh && ml[q][j] < bl);
                        bh = lt ? mh[q][j] : bh;
                        bl = lt ? ml[q][j] : bl;
                        bi = lt ? (uint32_t)q * kRhalfGroup + j : bi;
                    }
                }
                uint64_t wh = bh, wl = bl;
#pragma unroll
                for (int m = 1; m < 64; m <<= 1) {
                    const uint64_t oh = shfl_xor64(wh, m), ol = shfl_xor64(wl, m);
                    const bool lt = oh < wh || (oh == wh && ol < wl);
                    wh = lt ? oh : wh;
                    wl = lt ? ol : wl;
                }
                if (wl == ~0ull) break;  // no member left (valid ranks never have lo = ~0)
                if (bh == wh && bl == wl) {
                    const uint64_t o = base + c + take;
#pragma unroll
                    for (int q = 0; q < ER; ++q) {
#pragma unroll
                        for (uint32_t j = 0; j < kRhalfGroup; ++j) {
                            if (bi != (uint32_t)q * kRhalfGroup + j) continue;
                            const uint64_t g = grp_keys[(base + (uint32_t)q * 64u + lane) * kRhalfGroup + j];
                            if (targets) targets[o] = (uint32_t)g;
                            if (hashes) hashes[o] = (uint16_t)h[q];
                            if (dists) dists[o] = key_dist((uint32_t)(g >> 32));
                            mh[q][j] = ~0ull;
                            ml[q][j] = ~0ull;
                        }
                    }
                }
            }
        }
        reg_bitonic<ER, true>(h, k, lane);
#pragma unroll
        for (int q = 0; q < ER; ++q) {
            const uint32_t e = (uint32_t)q * 64u + lane;
            if (e >= l_max || (e >= c && e < c + take)) continue;  // the backups' positions
            const bool live = e < c;
            if (targets) targets[base + e] = live ? (uint32_t)k[q] : 0xffffffffu;
            if (hashes) hashes[base + e] = live ? (uint16_t)h[q] : (uint16_t)0;
            if (dists) dists[base + e] = live ? key_dist((uint32_t)(k[q] >> 32)) : 0.0f;
        }
        if (counts && lane == 0) counts[p] = c + take;
    }
}

uint32_t grid_for(uint64_t n, uint32_t threads, uint32_t cap) {
    const uint64_t g = (n + threads - 1) / threads;
    return (uint32_t)(g < 1 ? 1 : (g > cap ? cap : g));
}

}  // namespace

uint64_t hashprune_scan_blocks(uint32_t num_points) { return (num_points + kScanBlock - 1) / kScanBlock + 1; }

int launch_hashprune_clear(HashPruneState &s, hipStream_t stream) {
    hipLaunchKernelGGL(hp_fill_u32, dim3(grid_for(s.num_points, 256, 4096)), dim3(256), 0, stream, s.slot_count,
                       (uint64_t)s.num_points, 0u);
    hipLaunchKernelGGL(hp_fill_u32, dim3(grid_for(s.num_points, 256, 4096)), dim3(256), 0, stream, s.bucket,
                       (uint64_t)s.num_points, 0u);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_hashprune_insert(HashPruneState &s, const uint4 *records, uint64_t count, hipStream_t stream) {
    const uint32_t n = s.num_points;
    hipLaunchKernelGGL(hp_status_init, dim3(1), dim3(1), 0, stream, s.status);
    if (count == 0 || n == 0) return hipGetLastError() == hipSuccess ? 0 : -1;
    hipLaunchKernelGGL(hp_count_kernel, dim3(grid_for(count, 256, 16384)), dim3(256), 0, stream, records, count, n,
                       s.bucket, s.status);
    const uint32_t nb = (n + kScanBlock - 1) / kScanBlock;
    hipLaunchKernelGGL(hp_scan_reduce, dim3(nb), dim3(kScanThreads), 0, stream, s.bucket, n, s.block_sums);
    hipLaunchKernelGGL(hp_scan_partials, dim3(1), dim3(kScanThreads), 0, stream, s.block_sums, nb, s.offsets, n);
    hipLaunchKernelGGL(hp_scan_apply, dim3(nb), dim3(kScanThreads), 0, stream, s.bucket, n, s.block_sums, s.offsets);
    hipLaunchKernelGGL(hp_scatter_kernel, dim3(grid_for(count, 256, 16384)), dim3(256), 0, stream, records, count, n,
                       s.bucket, s.offsets, s.grouped);
    if (s.rhalf_mode) {
        const uint32_t grid = grid_for(n, kHpWaves, 8192);
        if (s.l_max <= 64)
            hipLaunchKernelGGL((hp_merge_rhalf_kernel<1, true>), dim3(grid), dim3(kHpThreads), 0, stream, s.grouped,
                               nullptr, nullptr, nullptr, nullptr, nullptr, s.offsets, n, s.l_max, s.rhalf_quota,
                               s.slot_keys, s.slot_hash, s.slot_count, s.grp_keys);
        else if (s.l_max <= 128)
            hipLaunchKernelGGL((hp_merge_rhalf_kernel<2, true>), dim3(grid), dim3(kHpThreads), 0, stream, s.grouped,
                               nullptr, nullptr, nullptr, nullptr, nullptr, s.offsets, n, s.l_max, s.rhalf_quota,
                               s.slot_keys, s.slot_hash, s.slot_count, s.grp_keys);
        else
            hipLaunchKernelGGL((hp_merge_rhalf_kernel<4, true>), dim3(grid), dim3(kHpThreads), 0, stream, s.grouped,
                               nullptr, nullptr, nullptr, nullptr, nullptr, s.offsets, n, s.l_max, s.rhalf_quota,
                               s.slot_keys, s.slot_hash, s.slot_count, s.grp_keys);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    // Both kernels decide from slots + new records; a merge never shrinks a
    // reservoir, so after the large kernel every source it merged still counts
    // more than kHpRegMax and the small kernel skips it (the reverse order
    // could merge a source twice).
    hipLaunchKernelGGL(hp_merge_large_kernel, dim3(grid_for(n, kHpWaves, 2048)), dim3(kHpThreads), 0, stream,
                       s.grouped, s.offsets, n, s.l_max, s.slot_keys, s.slot_hash, s.slot_count);
    hipLaunchKernelGGL(hp_merge_small_kernel, dim3(grid_for(n, kHpWaves, 8192)), dim3(kHpThreads), 0, stream,
                       s.grouped, s.offsets, n, s.l_max, s.slot_keys, s.slot_hash, s.slot_count);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

uint64_t hashprune_segment_workspace_bytes(uint64_t nseg, uint32_t num_points) {
    const uint64_t n = nseg ? nseg : 1;
    return 7 * seg_align(n * 4) + 256 + seg_align(n * 16) + seg_temp(n, num_points) + 256;
}

int launch_hashprune_insert_segments(HashPruneState &s, const uint4 *records, const uint4 *segs, uint64_t nseg,
                                     hipStream_t stream) {
    const uint32_t n = s.num_points;
    hipLaunchKernelGGL(hp_status_init, dim3(1), dim3(1), 0, stream, s.status);
    if (nseg == 0 || n == 0) return hipGetLastError() == hipSuccess ? 0 : -1;
    SegWs w = seg_ws_layout(s.seg_ws, nseg, n);
    hipLaunchKernelGGL(hp_seg_keys_kernel, dim3(grid_for(nseg, 256, 16384)), dim3(256), 0, stream, segs, nseg, n,
                       w.keys_in, w.vals_in, s.status);
    size_t tb = w.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(w.temp, tb, w.keys_in, w.keys_out, w.vals_in, w.vals_out, (int)nseg, 0,
                                           key_bits(n), stream) != hipSuccess)
        return -1;
    tb = w.temp_bytes;
    if (hipcub::DeviceRunLengthEncode::Encode(w.temp, tb, w.keys_out, w.run_src, w.run_len, w.num_runs, (int)nseg,
                                              stream) != hipSuccess)
        return -1;
    // run starts: exclusive sum of the lengths (entries past the run count
    // are never read)
    tb = w.temp_bytes;
    if (hipcub::DeviceScan::ExclusiveSum(w.temp, tb, w.run_len, w.run_start, (int)nseg, stream) != hipSuccess)
        return -1;
    hipLaunchKernelGGL(hp_seg_gather_kernel, dim3(grid_for(nseg, 256, 16384)), dim3(256), 0, stream, segs,
                       w.vals_out, nseg, w.sorted);
    const uint32_t grid = grid_for(nseg, kHpWaves, 8192);
    const uint32_t l = s.l_max;
    if (s.rhalf_mode) {
        if (l <= 64)
            hipLaunchKernelGGL((hp_merge_rhalf_kernel<1, false>), dim3(grid), dim3(kHpThreads), 0, stream, records,
                               w.sorted, w.run_src, w.run_start, w.run_len, w.num_runs, nullptr, n, l, s.rhalf_quota,
                               s.slot_keys, s.slot_hash, s.slot_count, s.grp_keys);
        else if (l <= 128)
            hipLaunchKernelGGL((hp_merge_rhalf_kernel<2, false>), dim3(grid), dim3(kHpThreads), 0, stream, records,
                               w.sorted, w.run_src, w.run_start, w.run_len, w.num_runs, nullptr, n, l, s.rhalf_quota,
                               s.slot_keys, s.slot_hash, s.slot_count, s.grp_keys);
        else
            hipLaunchKernelGGL((hp_merge_rhalf_kernel<4, false>), dim3(grid), dim3(kHpThreads), 0, stream, records,
                               w.sorted, w.run_src, w.run_start, w.run_len, w.num_runs, nullptr, n, l, s.rhalf_quota,
                               s.slot_keys, s.slot_hash, s.slot_count, s.grp_keys);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (l <= 64)
        hipLaunchKernelGGL(hp_merge_stream_kernel<1>, dim3(grid), dim3(kHpThreads), 0, stream, records, w.sorted,
                           w.run_src, w.run_start, w.run_len, w.num_runs, n, l, s.slot_keys, s.slot_hash,
                           s.slot_count);
    else if (l <= 128)
        hipLaunchKernelGGL(hp_merge_stream_kernel<2>, dim3(grid), dim3(kHpThreads), 0, stream, records, w.sorted,
                           w.run_src, w.run_start, w.run_len, w.num_runs, n, l, s.slot_keys, s.slot_hash,
                           s.slot_count);
    else
        hipLaunchKernelGGL(hp_merge_stream_kernel<4>, dim3(grid), dim3(kHpThreads), 0, stream, records, w.sorted,
                           w.run_src, w.run_start, w.run_len, w.num_runs, n, l, s.slot_keys, s.slot_hash,
                           s.slot_count);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_hashprune_export(const HashPruneState &s, uint32_t *targets, uint16_t *hashes, float *dists,
                            uint32_t *counts, hipStream_t stream) {
    const uint32_t n = s.num_points;
    if (n == 0 || s.l_max == 0) return 0;
    const uint32_t grid = grid_for(n, kHpWaves, 8192);
    if (s.rhalf_mode) {
        if (s.l_max <= 64)
            hipLaunchKernelGGL(hp_export_rhalf_kernel<1>, dim3(grid), dim3(kHpThreads), 0, stream, s.slot_keys,
                               s.slot_hash, s.slot_count, s.grp_keys, n, s.l_max, s.rhalf_mode, s.rhalf_quota,
                               s.rhalf_capacity, s.rhalf_alpha_sq, targets, hashes, dists, counts);
        else if (s.l_max <= 128)
            hipLaunchKernelGGL(hp_export_rhalf_kernel<2>, dim3(grid), dim3(kHpThreads), 0, stream, s.slot_keys,
                               s.slot_hash, s.slot_count, s.grp_keys, n, s.l_max, s.rhalf_mode, s.rhalf_quota,
                               s.rhalf_capacity, s.rhalf_alpha_sq, targets, hashes, dists, counts);
        else
            hipLaunchKernelGGL(hp_export_rhalf_kernel<4>, dim3(grid), dim3(kHpThreads), 0, stream, s.slot_keys,
                               s.slot_hash, s.slot_count, s.grp_keys, n, s.l_max, s.rhalf_mode, s.rhalf_quota,
                               s.rhalf_capacity, s.rhalf_alpha_sq, targets, hashes, dists, counts);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (s.l_max <= 64)
        hipLaunchKernelGGL(hp_export_kernel<1>, dim3(grid), dim3(kHpThreads), 0, stream, s.slot_keys, s.slot_hash,
                           s.slot_count, n, s.l_max, targets, hashes, dists, counts);
    else if (s.l_max <= 128)
        hipLaunchKernelGGL(hp_export_kernel<2>, dim3(grid), dim3(kHpThreads), 0, stream, s.slot_keys, s.slot_hash,
                           s.slot_count, n, s.l_max, targets, hashes, dists, counts);
    else
        hipLaunchKernelGGL(hp_export_kernel<4>, dim3(grid), dim3(kHpThreads), 0, stream, s.slot_keys, s.slot_hash,
                           s.slot_count, n, s.l_max, targets, hashes, dists, counts);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
