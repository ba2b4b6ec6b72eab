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
// reduction:
//   1. count records per source (atomics), exclusive scan, scatter the records
//      grouped by source (the per-source counters return to zero);
//   2. one wave per source with new records merges its current slots with them
//      (in registers up to 256 candidates, else in LDS up to kHpMergeCap at a
//      time): a bitonic sort by (hash, total order: dist key, target) puts
//      each hash's best first; when more than l_max hashes remain, a sort of
//      those by the total order gives the l_max-th as a threshold; the
//      survivors, in ascending hash order, are the new slots.
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
    reg_bitonic<E, true>(h, k, lane);
    // kept = first of its hash (the predecessor of element 64*q is lane 63 of slot q-1)
    bool kept[E];
    uint32_t n_kept = 0;
#pragma unroll
    for (int q = 0; q < E; ++q) {
        uint32_t prev = __shfl_up(h[q], 1);
        if (q > 0) {
            const uint32_t last = __shfl(h[q - 1], 63);
            prev = lane == 0 ? last : prev;
        }
        const uint32_t e = (uint32_t)q * 64u + lane;
        kept[q] = e < N && (e == 0 || prev != h[q]);
        n_kept += (uint32_t)__popcll(__ballot(kept[q]));
    }
    bool sel[E];
#pragma unroll
    for (int q = 0; q < E; ++q) sel[q] = kept[q];
    if (n_kept > l_max) {
        // threshold: the l_max-th kept candidate in total order
        uint32_t h2[E];
        uint64_t k2[E];
#pragma unroll
        for (int q = 0; q < E; ++q) {
            h2[q] = kept[q] ? h[q] : 0xffffffffu;
            k2[q] = kept[q] ? k[q] : ~0ull;
        }
        reg_bitonic<E, false>(h2, k2, lane);
        const uint32_t tq = (l_max - 1u) / 64u, tl = (l_max - 1u) % 64u;
        uint64_t tk = k2[0];
        uint32_t th = h2[0];
#pragma unroll
        for (int q = 1; q < E; ++q) {
            tk = tq == (uint32_t)q ? k2[q] : tk;
            th = tq == (uint32_t)q ? h2[q] : th;
        }
        const uint64_t tkey = ((uint64_t)__shfl((uint32_t)(tk >> 32), (int)tl) << 32) | __shfl((uint32_t)tk, (int)tl);
        const uint32_t thash = __shfl(th, (int)tl);
#pragma unroll
        for (int q = 0; q < E; ++q) sel[q] = kept[q] && (k[q] < tkey || (k[q] == tkey && h[q] <= thash));
    }
    uint32_t base = 0;
#pragma unroll
    for (int q = 0; q < E; ++q) {
        const uint64_t m = __ballot(sel[q]);
        if (sel[q]) {
            const uint32_t pos = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
            slot_keys_out[pos] = k[q];
            slot_hash_out[pos] = (uint16_t)h[q];
        }
        base += (uint32_t)__popcll(m);
    }
    return base;
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
    uint64_t tkey[kHpMergeCap];     // kept candidates, when more than l_max, by total order;
    uint32_t thash[kHpMergeCap];    // then the merged reservoir (once the threshold is read)
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
// w.tkey/w.thash[0, result); returns its size.
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
    // kept = first of its hash; kpos = its place among the kept
    uint32_t kcount = 0;
    for (uint32_t q = 0; q < E; ++q) {
        const uint32_t e = eb + q;
        kcount += (e < N && (e == 0 || w.val[e - 1] != w.val[e])) ? 1u : 0u;
    }
    uint32_t n_kept;
    const uint32_t kbase = wave_excl_scan(kcount, lane, n_kept);
    if (n_kept <= l_max) {
        // every hash's best stays, already in ascending hash order
        uint32_t run = kbase;
        for (uint32_t q = 0; q < E; ++q) {
            const uint32_t e = eb + q;
            if (e < N && (e == 0 || w.val[e - 1] != w.val[e])) {
                w.tkey[run] = w.key[e];
                w.thash[run] = w.val[e];
                ++run;
            }
        }
        n_old = n_kept;
    } else {
        // the l_max best of the kept by (key, hash): threshold from a sort of the kept
        uint32_t run = kbase;
        for (uint32_t q = 0; q < E; ++q) {
            const uint32_t e = eb + q;
            if (e < N && (e == 0 || w.val[e - 1] != w.val[e])) {
                w.tkey[run] = w.key[e];
                w.thash[run] = w.val[e];
                ++run;
            }
        }
        uint32_t P2 = 64;
        while (P2 < n_kept) P2 <<= 1;
        for (uint32_t e = n_kept + lane; e < P2; e += 64) {
            w.tkey[e] = ~0ull;
            w.thash[e] = 0xffffffffu;
        }
        __builtin_amdgcn_wave_barrier();
        wave_bitonic<uint64_t>(w.tkey, w.thash, P2, lane);
        const uint64_t tk = w.tkey[l_max - 1];
        const uint32_t th = w.thash[l_max - 1];
        uint32_t scount = 0;
        for (uint32_t q = 0; q < E; ++q) {
            const uint32_t e = eb + q;
            const bool kept = e < N && (e == 0 || w.val[e - 1] != w.val[e]);
            const uint64_t k = w.key[e];
            scount += (kept && (k < tk || (k == tk && w.val[e] <= th))) ? 1u : 0u;
        }
        uint32_t n_sel;
        uint32_t srun = wave_excl_scan(scount, lane, n_sel);
        for (uint32_t q = 0; q < E; ++q) {
            const uint32_t e = eb + q;
            const bool kept = e < N && (e == 0 || w.val[e - 1] != w.val[e]);
            const uint64_t k = w.key[e];
            if (kept && (k < tk || (k == tk && w.val[e] <= th))) {
                w.tkey[srun] = k;
                w.thash[srun] = w.val[e];
                ++srun;
            }
        }
        n_old = n_sel;
    }
    __builtin_amdgcn_wave_barrier();
    return n_old;
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

// Run heads of the sorted keys -> the active sources (src, first position);
// their order is not fixed (each source is merged independently).
__global__ void hp_seg_runs_kernel(const uint32_t *keys, uint64_t nseg, uint32_t num_points, uint32_t *run_src,
                                   uint32_t *run_start, uint32_t *run_count) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nseg; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t k = keys[i];
        if (k < num_points && (i == 0 || keys[i - 1] != k)) {
            const uint32_t a = atomicAdd(run_count, 1u);
            run_src[a] = k;
            run_start[a] = (uint32_t)i;
        }
    }
}

// Register merge of one source's reservoir and its segments' records.  Lane
// s < ns holds segment s (exclusive prefix `pre`, `cnt` records from
// `first`).  The record of each register slot is located first, with every
// lane active (the lanes' segment values are read by shuffles), then the
// merge reads it.
template <int E>
__device__ uint32_t seg_merge(const uint4 *records, uint64_t *slot_keys, uint16_t *slot_hash, uint32_t n_old,
                              uint32_t n_new, uint32_t ns, uint32_t pre, uint32_t cnt, uint64_t first, uint32_t l_max,
                              uint32_t lane) {
    uint64_t addr[E];
#pragma unroll
    for (int q = 0; q < E; ++q) addr[q] = 0;
    for (uint32_t sg = 0; sg < ns; ++sg) {
        const uint32_t ps = __shfl(pre, (int)sg), cs = __shfl(cnt, (int)sg);
        const uint64_t fs = ((uint64_t)__shfl((uint32_t)(first >> 32), (int)sg) << 32) | __shfl((uint32_t)first, (int)sg);
#pragma unroll
        for (int q = 0; q < E; ++q) {
            const uint32_t e = (uint32_t)q * 64u + lane;
            if (e >= n_old && e - n_old >= ps && e - n_old < ps + cs) addr[q] = fs + (e - n_old - ps);
        }
    }
    auto fetch = [&](int q, uint32_t) -> uint4 {
        uint64_t a = addr[0];
#pragma unroll
        for (int i = 1; i < E; ++i) a = i == q ? addr[i] : a;
        return records[a];
    };
    return reg_merge_f<E>(slot_keys, slot_hash, n_old, n_new, fetch, l_max, lane, slot_keys, slot_hash);
}

// The segments of active source a: sorted positions [start, start + ns);
// lanes read the keys after `start` and count the leading run equal to src
// (ns > 64 means "more than 64").
__device__ __forceinline__ uint32_t run_length64(const uint32_t *keys, uint64_t nseg, uint32_t start, uint32_t src,
                                                 uint32_t lane) {
    const uint64_t at = (uint64_t)start + lane;
    const bool eq = at < nseg && keys[at] == src;
    const uint64_t m = ~__ballot(eq);
    return m ? (uint32_t)__builtin_ctzll(m) : 65u;
}

// Register merges of active sources with at most 64 segments and kHpRegMax
// candidates.
__global__ __launch_bounds__(kHpThreads) void hp_merge_small_seg_kernel(const uint4 *records, const uint4 *segs,
                                                                        const uint32_t *keys, const uint32_t *vals,
                                                                        uint64_t nseg, const uint32_t *run_src,
                                                                        const uint32_t *run_start,
                                                                        const uint32_t *run_count, uint32_t l_max,
                                                                        uint64_t *slot_keys, uint16_t *slot_hash,
                                                                        uint32_t *slot_count) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t waves = gridDim.x * kHpWaves;
    const uint32_t na = *run_count;
    for (uint32_t a = blockIdx.x * kHpWaves + (threadIdx.x >> 6); a < na; a += waves) {
        const uint32_t src = run_src[a];
        const uint32_t s0 = run_start[a];
        const uint32_t ns = run_length64(keys, nseg, s0, src, lane);
        if (ns > 64u) continue;  // hp_merge_large_seg_kernel
        uint32_t cnt = 0;
        uint64_t first = 0;
        if (lane < ns) {
            const uint4 g = segs[vals[s0 + lane]];
            cnt = g.w;
            first = ((uint64_t)g.z << 32) | g.y;
        }
        uint32_t n_new;
        const uint32_t pre = wave_excl_scan(cnt, lane, n_new);
        const uint32_t n_old = slot_count[src];
        if (n_old + n_new > kHpRegMax) continue;
        const uint64_t sbase = (uint64_t)src * l_max;
        uint32_t c;
        if (n_old + n_new <= 64u)
            c = seg_merge<1>(records, slot_keys + sbase, slot_hash + sbase, n_old, n_new, ns, pre, cnt, first, l_max,
                             lane);
        else if (n_old + n_new <= 128u)
            c = seg_merge<2>(records, slot_keys + sbase, slot_hash + sbase, n_old, n_new, ns, pre, cnt, first, l_max,
                             lane);
        else
            c = seg_merge<4>(records, slot_keys + sbase, slot_hash + sbase, n_old, n_new, ns, pre, cnt, first, l_max,
                             lane);
        if (lane == 0) slot_count[src] = c;
    }
}

// The other active sources: their segments' records staged in LDS, merged
// kHpMergeCap candidates at a time.
__global__ __launch_bounds__(kHpThreads) void hp_merge_large_seg_kernel(const uint4 *records, const uint4 *segs,
                                                                        const uint32_t *keys, const uint32_t *vals,
                                                                        uint64_t nseg, const uint32_t *run_src,
                                                                        const uint32_t *run_start,
                                                                        const uint32_t *run_count, uint32_t l_max,
                                                                        uint64_t *slot_keys, uint16_t *slot_hash,
                                                                        uint32_t *slot_count) {
    __shared__ HpWaveLds lds[kHpWaves];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    HpWaveLds &w = lds[wave];
    const uint32_t waves = gridDim.x * kHpWaves;
    const uint32_t na = *run_count;
    for (uint32_t a = blockIdx.x * kHpWaves + wave; a < na; a += waves) {
        const uint32_t src = run_src[a];
        const uint32_t s0 = run_start[a];
        const uint32_t ns64 = run_length64(keys, nseg, s0, src, lane);
        uint32_t n_old = slot_count[src];
        if (ns64 <= 64u) {
            // the small kernel's case unless it holds more than kHpRegMax candidates
            const uint32_t cnt = lane < ns64 ? segs[vals[s0 + lane]].w : 0u;
            uint32_t n_new;
            (void)wave_excl_scan(cnt, lane, n_new);
            if (n_old + n_new <= kHpRegMax) continue;
        }
        const uint64_t sbase = (uint64_t)src * l_max;
        for (uint32_t e = lane; e < n_old; e += 64) {
            w.key[e] = slot_keys[sbase + e];
            w.val[e] = slot_hash[sbase + e];
        }
        __builtin_amdgcn_wave_barrier();
        uint32_t fill = 0;  // candidates staged after the reservoir
        bool merged = false;
        for (uint64_t si = s0; si < nseg && keys[si] == src; ++si) {
            const uint4 g = segs[vals[si]];
            const uint64_t first = ((uint64_t)g.z << 32) | g.y;
            uint32_t used = 0;
            while (used < g.w) {
                const uint32_t room = kHpMergeCap - n_old - fill;
                const uint32_t take = (g.w - used < room) ? g.w - used : room;
                for (uint32_t e = lane; e < take; e += 64) {
                    const uint4 r = records[first + used + e];
                    w.key[n_old + fill + e] = ((uint64_t)total_key(__uint_as_float(r.w)) << 32) | r.y;
                    w.val[n_old + fill + e] = r.z & 0xffffu;
                }
                fill += take;
                used += take;
                if (n_old + fill == kHpMergeCap) {
                    __builtin_amdgcn_wave_barrier();
                    n_old = lds_merge_round(w, n_old, n_old + fill, l_max, lane);
                    fill = 0;
                    for (uint32_t e = lane; e < n_old; e += 64) {
                        w.key[e] = w.tkey[e];
                        w.val[e] = w.thash[e];
                    }
                    __builtin_amdgcn_wave_barrier();
                    merged = true;
                }
            }
        }
        if (fill > 0 || !merged) {
            __builtin_amdgcn_wave_barrier();
            n_old = lds_merge_round(w, n_old, n_old + fill, l_max, lane);
        }
        for (uint32_t e = lane; e < n_old; e += 64) {
            slot_keys[sbase + e] = w.tkey[e];
            slot_hash[sbase + e] = (uint16_t)w.thash[e];
        }
        if (lane == 0) slot_count[src] = n_old;
        __builtin_amdgcn_wave_barrier();
    }
}

// Segment workspace layout: keys in/out, values in/out, run sources and
// starts (nseg each, u32), the run count, then the radix sort's temporary.
struct SegWs {
    uint32_t *keys_in, *keys_out, *vals_in, *vals_out, *run_src, *run_start, *run_count;
    void *temp;
    size_t temp_bytes;
};
size_t seg_align(size_t x) { return (x + 255) & ~(size_t)255; }
int key_bits(uint32_t num_points) {
    int b = 1;
    while (b < 32 && ((uint64_t)1 << b) <= num_points) ++b;  // keys go up to num_points (unused segments)
    return b;
}
size_t seg_sort_temp(uint64_t nseg, uint32_t num_points) {
    size_t bytes = 0;
    hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                       (const uint32_t *)nullptr, (uint32_t *)nullptr, (int)nseg, 0,
                                       key_bits(num_points));
    return bytes;
}
SegWs seg_ws_layout(void *base, uint64_t nseg, uint32_t num_points) {
    SegWs w{};
    char *p = static_cast<char *>(base);
    const size_t a = seg_align(nseg * 4);
    w.keys_in = reinterpret_cast<uint32_t *>(p);
    w.keys_out = reinterpret_cast<uint32_t *>(p + a);
    w.vals_in = reinterpret_cast<uint32_t *>(p + 2 * a);
    w.vals_out = reinterpret_cast<uint32_t *>(p + 3 * a);
    w.run_src = reinterpret_cast<uint32_t *>(p + 4 * a);
    w.run_start = reinterpret_cast<uint32_t *>(p + 5 * a);
    w.run_count = reinterpret_cast<uint32_t *>(p + 6 * a);
    w.temp = p + 6 * a + 256;
    w.temp_bytes = seg_sort_temp(nseg, num_points);
    return w;
}

__global__ void hp_export_kernel(const uint64_t *slot_keys, const uint16_t *slot_hash, const uint32_t *slot_count,
                                 uint32_t num_points, uint32_t l_max, uint32_t *targets, uint16_t *hashes,
                                 float *dists, uint32_t *counts) {
    const uint64_t total = (uint64_t)num_points * l_max;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t p = (uint32_t)(i / l_max), s = (uint32_t)(i % l_max);
        const uint32_t c = slot_count[p];
        const bool live = s < c;
        const uint64_t k = live ? slot_keys[i] : 0ull;
        if (targets) targets[i] = live ? (uint32_t)k : 0xffffffffu;
        if (hashes) hashes[i] = live ? slot_hash[i] : (uint16_t)0;
        if (dists) dists[i] = live ? key_dist((uint32_t)(k >> 32)) : 0.0f;
        if (counts && s == 0) counts[p] = c;
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
    return 6 * seg_align((nseg ? nseg : 1) * 4) + 256 + seg_sort_temp(nseg ? nseg : 1, num_points) + 256;
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
    hipLaunchKernelGGL(hp_fill_u32, dim3(1), dim3(64), 0, stream, w.run_count, (uint64_t)1, 0u);
    hipLaunchKernelGGL(hp_seg_runs_kernel, dim3(grid_for(nseg, 256, 16384)), dim3(256), 0, stream, w.keys_out, nseg,
                       n, w.run_src, w.run_start, w.run_count);
    // large first (a merge never shrinks a reservoir, so the small kernel then
    // skips what the large kernel merged)
    const uint32_t ga = grid_for(nseg, kHpWaves, 8192);
    hipLaunchKernelGGL(hp_merge_large_seg_kernel, dim3(grid_for(nseg, kHpWaves, 2048)), dim3(kHpThreads), 0, stream,
                       records, segs, w.keys_out, w.vals_out, nseg, w.run_src, w.run_start, w.run_count, s.l_max,
                       s.slot_keys, s.slot_hash, s.slot_count);
    hipLaunchKernelGGL(hp_merge_small_seg_kernel, dim3(ga), dim3(kHpThreads), 0, stream, records, segs, w.keys_out,
                       w.vals_out, nseg, w.run_src, w.run_start, w.run_count, s.l_max, s.slot_keys, s.slot_hash,
                       s.slot_count);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_hashprune_export(const HashPruneState &s, uint32_t *targets, uint16_t *hashes, float *dists,
                            uint32_t *counts, hipStream_t stream) {
    const uint64_t total = (uint64_t)s.num_points * s.l_max;
    if (total == 0) return 0;
    hipLaunchKernelGGL(hp_export_kernel, dim3(grid_for(total, 256, 16384)), dim3(256), 0, stream, s.slot_keys,
                       s.slot_hash, s.slot_count, s.num_points, s.l_max, targets, hashes, dists, counts);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
