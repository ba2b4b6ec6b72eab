// edge_records.hip -- candidate records -> HashPrune edge records.
//
// The reference converts every leaf's CompactTopKBatch on the host
// (flush_compact_topk_batch_into_edges, leaf_build.rs:1679-1829): for member
// row i and rank q, a slot (j, d) with j != u32::MAX and finite d becomes the
// two PendingEdges (i -> j, compute_hash(s_i, s_j), d) and (j -> i,
// compute_hash(s_j, s_i), d) (hash_prune.rs:2239-2251: bit b set when
// s_c[b] - s_p[b] >= 0), in (row, rank) order.  Here the same record stream
// is produced on the device, as 16-byte SpillRecord16 records
// (spill_hashprune.rs:137-145), straight from the top-k slots in HBM.
//
// Three launches, all byte-moving work (HBM-bound):
//   count  one workgroup per leaf: valid slots per row (half-wave ballots),
//          leaf total;
//   scan   one workgroup: exclusive scan of the leaf totals -> first record
//          of every leaf (2 per valid slot) and the record count;
//   emit   one workgroup per leaf: the per-row counts again, an exclusive
//          scan in LDS, a membership table of the leaf's global ids in LDS
//          (the reference's compact_local_index lookup, leaf_build.rs:330-346,
//          which rejects ids outside the leaf), then each half-wave writes its
//          row's records: a lane writes the forward and reverse record of its
//          slot as two adjacent 16-byte stores, so a row's records are one
//          contiguous run.
#include <hip/hip_runtime.h>

#include "edge_kernels.h"
#include "kernel_attr.h"

namespace tessa {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kCountUnroll = 4;  // rows per half-wave in flight (count pass)
constexpr int kEmitUnroll = 4;   // rows per half-wave in flight (emit pass)
constexpr uint32_t kNoKey = 0xffffffffu;
constexpr uint32_t kLeafRegular = 0x80000000u;  // leaf_totals flag: every row has k_eff valid slots
// The leaf's sketch rows are staged in LDS whenever everything fits one CU
// (two workgroups per CU for 1,024-row leaves, one for 2,048-row leaves: the
// hashes' reads from L2 instead made 2,048-row leaves 2.6x slower).
constexpr size_t kEmitLdsBudget = 160 * 1024;

__device__ __forceinline__ bool slot_valid(uint32_t id, float d) {
    // j != u32::MAX && d.is_finite()
    return id != 0xffffffffu && (__float_as_uint(d) & 0x7f800000u) != 0x7f800000u;
}

// Records in the reference's order are written once, in runs from
// consecutive lanes, and never read back by these kernels: they stream past
// the caches (nontemporal stores).  Source-grouped records land all over the
// leaf's range (reverse records fill their targets' segments from the end),
// so they are written through L2, which joins a line's 16-byte pieces before
// it goes to HBM (C2 grouped emission 7.6 -> 2.9 ms).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <bool kTemporal = false>
__device__ __forceinline__ void store_record(uint4 *out, uint64_t i, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 v = {a, b, c, d};
    if constexpr (kTemporal)
        *reinterpret_cast<u32x4 *>(out + i) = v;
    else
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out + i));
}

__device__ __forceinline__ uint32_t table_hash(uint32_t g, uint32_t bits) { return (g * 0x9E3779B1u) >> (32 - bits); }

__device__ __forceinline__ uint32_t leaf_k(const EdgeParams &p, uint32_t n) {
    return n > 1u ? (p.k < n - 1u ? p.k : n - 1u) : 0u;
}

// Rows of a leaf, 1 + largest-leaf flag when a leaf exceeds max_leaf_rows
// (its records are not emitted; the host reports LEAF_ROW).
__device__ __forceinline__ uint32_t leaf_rows(const EdgeParams &p, uint32_t leaf, bool report) {
    const uint32_t n = p.member_counts[leaf];
    if (n <= p.max_leaf_rows) return n;
    if (report && threadIdx.x == 0) atomicMax((unsigned long long *)&p.status[kEdgeLeafTooLarge], 1ull + n);
    return 0u;
}

// Valid-slot count of every row of leaf `leaf` into cnt[0..n), then an
// exclusive scan in place; returns the leaf total and whether every row has
// all of its k_eff slots valid (then row r's records start at 2*r*k_eff).
// All threads call it.
// Each half-wave owns a row (lane q = rank); kCountUnroll rows per half-wave
// have their loads in flight together.
__device__ uint32_t row_counts_scan(const EdgeParams &p, uint32_t leaf, uint32_t n, uint32_t kl, uint32_t *cnt,
                                    uint32_t *wsum, bool &regular) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t q = lane & 31u;
    const uint32_t h = lane >> 5;
    const uint64_t out0 = p.output_offsets[leaf];
    constexpr uint32_t kStep = 2u * kWaves;
    int irregular = 0;
    for (uint32_t r0 = 2u * wave + h; r0 < n + h; r0 += kStep * kCountUnroll) {
        uint32_t id[kCountUnroll];
        float d[kCountUnroll];
#pragma unroll
        for (int u = 0; u < kCountUnroll; ++u) {
            const uint32_t r = r0 + u * kStep;
            id[u] = kNoKey;
            d[u] = 0.0f;
            if (r < n && q < kl) {
                const uint64_t s = out0 + (uint64_t)r * p.k + q;
                id[u] = p.topk_ids[s];
                d[u] = p.topk_dists[s];
            }
        }
#pragma unroll
        for (int u = 0; u < kCountUnroll; ++u) {
            const uint32_t r = r0 + u * kStep;
            const uint64_t m = __ballot(slot_valid(id[u], d[u]));
            const uint32_t c = __popcll(h ? (m >> 32) : (m & 0xffffffffull));
            if (r < n && q == 0u) {
                cnt[r] = c;
                irregular |= c != kl ? 1 : 0;
            }
        }
    }
    regular = __syncthreads_or(irregular) == 0;
    const uint32_t per = (n + kThreads - 1) / kThreads;
    const uint32_t b = tid * per;
    const uint32_t e = b + per < n ? b + per : n;
    uint32_t sum = 0;
    for (uint32_t i = b; i < e; ++i) sum += cnt[i];
    uint32_t x = sum;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63u) wsum[wave] = x;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        base += (uint32_t)w < wave ? wsum[w] : 0u;
        total += wsum[w];
    }
    uint32_t run = base + x - sum;
    for (uint32_t i = b; i < e; ++i) {
        const uint32_t c = cnt[i];
        cnt[i] = run;
        run += c;
    }
    __syncthreads();
    return total;
}

__global__ __launch_bounds__(kThreads) void edge_count_kernel(EdgeParams p) {
    extern __shared__ uint32_t lds[];
    uint32_t *wsum = lds;
    uint32_t *cnt = lds + kWaves;
    for (uint32_t leaf = blockIdx.x; leaf < p.leaf_count; leaf += gridDim.x) {
        const uint32_t n = leaf_rows(p, leaf, true);
        bool regular;
        const uint32_t total = row_counts_scan(p, leaf, n, leaf_k(p, n), cnt, wsum, regular);
        // total <= 4096 * 32: bit 31 is free for the regular-leaf flag
        if (threadIdx.x == 0) p.leaf_totals[leaf] = total | (regular ? kLeafRegular : 0u);
    }
}

// Exclusive scan over the leaves of v(leaf) into out[0..leaf_count], the
// total last (one 1024-thread workgroup).
template <typename F>
__device__ uint64_t leaf_scan(const EdgeParams &p, F v_of, uint64_t *out, uint64_t scale) {
    __shared__ uint64_t wsum[16];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    uint64_t carry = 0;
    for (uint32_t base = 0; base < p.leaf_count; base += 1024u) {
        const uint32_t i = base + tid;
        const uint64_t v = i < p.leaf_count ? v_of(i) : 0ull;
        uint64_t x = v;
#pragma unroll
        for (uint32_t off = 1; off < 64; off <<= 1) {
            const uint64_t y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        if (lane == 63u) wsum[wave] = x;
        __syncthreads();
        uint64_t before = 0, total = 0;
        for (uint32_t w = 0; w < 16u; ++w) {
            before += w < wave ? wsum[w] : 0ull;
            total += wsum[w];
        }
        if (i < p.leaf_count) out[i] = scale * (carry + before + x - v);
        carry += total;
        __syncthreads();
    }
    if (tid == 0) out[p.leaf_count] = scale * carry;
    return scale * carry;
}

__global__ __launch_bounds__(1024) void edge_scan_kernel(EdgeParams p) {
    // records: 2 per valid slot
    const uint64_t total = leaf_scan(p, [&](uint32_t i) { return (uint64_t)(p.leaf_totals[i] & ~kLeafRegular); },
                                     p.leaf_base, 2ull);
    if (threadIdx.x == 0) p.status[kEdgeRecordCount] = total;
    // segments: one per member row of a leaf within max_leaf_rows
    if (p.segments)
        leaf_scan(p, [&](uint32_t i) {
            const uint32_t n = p.member_counts[i];
            return (uint64_t)(n <= p.max_leaf_rows ? n : 0u);
        }, p.leaf_seg_base, 1ull);
}

// compute_hash(s_i, s_j) and compute_hash(s_j, s_i) over m_bits coordinates.
// kVec4: both rows are 16-byte aligned with at least ceil(m_bits/4)*4 floats.
template <bool kVec4>
__device__ __forceinline__ void pair_hashes(const float *si, const float *sj, uint32_t m_bits, uint32_t &hf,
                                            uint32_t &hr) {
    hf = 0u;
    hr = 0u;
    if (kVec4) {
        const float4 *a4 = reinterpret_cast<const float4 *>(si);
        const float4 *c4 = reinterpret_cast<const float4 *>(sj);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (4u * v >= m_bits) break;
            const float4 a = a4[v], c = c4[v];
            const float av[4] = {a.x, a.y, a.z, a.w};
            const float cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t bit = 4u * v + e;
                if (bit < m_bits) {
                    hf |= (cv[e] - av[e] >= 0.0f ? 1u : 0u) << bit;
                    hr |= (av[e] - cv[e] >= 0.0f ? 1u : 0u) << bit;
                }
            }
        }
    } else {
        for (uint32_t bit = 0; bit < m_bits; ++bit) {
            const float a = si[bit], c = sj[bit];
            hf |= (c - a >= 0.0f ? 1u : 0u) << bit;
            hr |= (a - c >= 0.0f ? 1u : 0u) << bit;
        }
    }
}

// Sketch access modes of the emit kernel.
enum SketchMode : int {
    kSketchGlobal = 0,    // scalar loads from the sketch rows in HBM
    kSketchGlobalV4 = 1,  // float4 loads (width % 4 == 0, 16-byte aligned base)
    kSketchLds = 2        // the leaf's sketch rows staged in LDS (float4 reads)
};

// LDS words of the emit kernel: wave sums and the leaf's record base (two
// words) | row counts | member ids | table keys | table values (u16) |
// (16-byte aligned) staged sketches.  Grouped order adds two arrays of
// max_rows words: per row its record count (then a cursor over its reverse
// records) and the mask of its slots whose reverse record is left out.
__host__ __device__ inline uint32_t emit_sketch_offset(uint32_t max_rows, uint32_t table_bits, bool grouped) {
    const uint32_t words = kWaves + 2u + 2u * max_rows + (1u << table_bits) + (1u << table_bits) / 2u +
                           (grouped ? 2u * max_rows : 0u);
    return (words + 3u) & ~3u;
}

// Largest finite distance among the kl <= k <= 32 slots of a top-k list from
// slot index `slot0`; -1 when there is none.  An entry of the list lies at or
// below it, so a slot whose distance exceeds it cannot be repeated there.
__device__ __forceinline__ float list_max_dist(const EdgeParams &p, uint64_t slot0, uint32_t kl) {
    const float *ds = p.topk_dists + slot0;
    float m = -1.0f;
    if ((p.k & 3u) == 0u && (reinterpret_cast<uintptr_t>(ds) & 15u) == 0u) {
        const float4 *v = reinterpret_cast<const float4 *>(ds);
        float4 x[8];
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c) {
            x[c] = make_float4(-1.0f, -1.0f, -1.0f, -1.0f);
            if (4u * c < kl) x[c] = v[c];
        }
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c) {
            const uint32_t t = 4u * c;
            const float e[4] = {x[c].x, x[c].y, x[c].z, x[c].w};
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i)
                if (t + i < kl && (__float_as_uint(e[i]) & 0x7f800000u) != 0x7f800000u) m = fmaxf(m, e[i]);
        }
    } else {
        for (uint32_t t = 0; t < kl; ++t)
            if ((__float_as_uint(ds[t]) & 0x7f800000u) != 0x7f800000u) m = fmaxf(m, ds[t]);
    }
    return m;
}

// Whether the top-k list of a leaf row (kl <= k <= 32 slots from slot index
// `slot0`) names target g at distance bits db.  Then that row's forward
// record is the record (row's id -> g, compute_hash(s_row, s_g), d) -- the
// reverse record of g's slot naming the row, bit for bit (the distance of a
// pair is symmetric: (rn + cn) and rs * cs commute exactly).  Ids are read
// 16 bytes at a time when the list is aligned and k is a multiple of 4 (the
// last 16 bytes then stay inside the row's k slots); only a matching id's
// distance is read.
__device__ __forceinline__ bool slot_listed(const EdgeParams &p, uint64_t slot0, uint32_t kl, uint32_t g,
                                            uint32_t db) {
    const uint32_t *ids = p.topk_ids + slot0;
    uint32_t pos = kNoKey;
    if ((p.k & 3u) == 0u && (reinterpret_cast<uintptr_t>(ids) & 15u) == 0u) {
        const uint4 *v = reinterpret_cast<const uint4 *>(ids);
        uint4 x[8];
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c) {
            x[c] = make_uint4(kNoKey, kNoKey, kNoKey, kNoKey);
            if (4u * c < kl) x[c] = v[c];
        }
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c) {
            const uint32_t t = 4u * c;
            if (x[c].x == g && t < kl) pos = t;
            if (x[c].y == g && t + 1u < kl) pos = t + 1u;
            if (x[c].z == g && t + 2u < kl) pos = t + 2u;
            if (x[c].w == g && t + 3u < kl) pos = t + 3u;
        }
    } else {
        for (uint32_t t = 0; t < kl; ++t)
            if (ids[t] == g) pos = t;
    }
    return pos != kNoKey && __float_as_uint(p.topk_dists[slot0 + pos]) == db;
}

template <int kMode, bool kGrouped>
__global__ __launch_bounds__(kThreads) void edge_emit_kernel(EdgeParams p) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const uint32_t tbits = p.table_bits;
    const uint32_t tmask = (1u << tbits) - 1u;
    uint32_t *wsum = lds;  // kWaves sums, then the leaf's record base (lo, hi)
    uint32_t *cnt = lds + kWaves + 2u;
    uint32_t *gid = cnt + p.max_leaf_rows;
    uint32_t *tkey = gid + p.max_leaf_rows;
    uint16_t *tval = reinterpret_cast<uint16_t *>(tkey + (1u << tbits));
    uint32_t *tot = tkey + (1u << tbits) + (1u << tbits) / 2u;  // grouped order only
    uint32_t *dup = tot + p.max_leaf_rows;
    float *sk_lds = reinterpret_cast<float *>(lds + emit_sketch_offset(p.max_leaf_rows, tbits, kGrouped));
    const uint32_t mw = (p.m_bits + 3u) & ~3u;  // staged row stride (floats)
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t q = lane & 31u;
    const uint32_t h = lane >> 5;
    if (p.leaf_base[p.leaf_count] > p.out_capacity ||
        (kGrouped && p.leaf_seg_base[p.leaf_count] > p.segment_capacity)) {
        if (blockIdx.x == 0 && tid == 0) p.status[kEdgeCapacityHit] = 1ull;
        return;  // uniform over the grid: nothing is written
    }
    for (uint32_t leaf = blockIdx.x; leaf < p.leaf_count; leaf += gridDim.x) {
        const uint32_t n = leaf_rows(p, leaf, false);
        const uint32_t kl = leaf_k(p, n);
        const uint32_t *mem = p.members + p.member_offsets[leaf];
        for (uint32_t i = tid; i <= tmask; i += kThreads) tkey[i] = kNoKey;
        // Row record offsets: r * k_eff for a regular leaf (every slot valid),
        // else counted again and scanned into cnt.
        const bool regular = (p.leaf_totals[leaf] & kLeafRegular) != 0u;
        if (kGrouped) {
            // with p.unique, cnt holds each row's largest listed distance
            // until the segment scan below overwrites it
            const uint64_t o0 = p.output_offsets[leaf];
            for (uint32_t c = tid; c < n; c += kThreads) {
                tot[c] = 0u;
                if (p.unique) cnt[c] = __float_as_uint(list_max_dist(p, o0 + (uint64_t)c * p.k, kl));
            }
            __syncthreads();
        } else if (regular) {
            __syncthreads();
        } else {
            bool unused;
            row_counts_scan(p, leaf, n, kl, cnt, wsum, unused);  // ends with a barrier
        }
        // Member ids, the membership table (global id -> member position) and,
        // in LDS mode, the m_bits leading coordinates of every member's sketch
        // row (independent loads, all in flight together).  A point without a
        // resident row or sketch row is an error (the reference's sketch
        // prefetch of the batch, leaf_build.rs:1758-1763) and is left out of
        // the table.
        for (uint32_t c = tid; c < n; c += kThreads) {
            const uint32_t mr = mem[c];
            const uint32_t g = mr < p.resident_rows ? p.gids[mr] : kNoKey;
            const bool ok = mr < p.resident_rows && g < p.sketch_rows;
            gid[c] = ok ? g : kNoKey;
            if (kMode == kSketchLds) {
                float v[16];
                const float *row = p.sketches + (uint64_t)(ok ? g : 0u) * p.width;
#pragma unroll
                for (uint32_t bit = 0; bit < 16u; ++bit) v[bit] = (ok && bit < p.m_bits) ? row[bit] : 0.0f;
#pragma unroll
                for (uint32_t bit = 0; bit < 16u; ++bit)
                    if (bit < mw) sk_lds[c * mw + bit] = v[bit];
            }
            if (!ok) {
                atomicMin((unsigned long long *)&p.status[kEdgeFirstError],
                          (unsigned long long)edge_error_key(leaf, kEdgeErrSketch, c, 0));
                continue;
            }
            uint32_t slot = table_hash(g, tbits);
            while (true) {
                const uint32_t prev = atomicCAS(&tkey[slot], kNoKey, g);
                if (prev == kNoKey) {
                    tval[slot] = (uint16_t)c;
                    break;
                }
                if (prev == g) break;  // repeated id: the first position holds it
                slot = (slot + 1u) & tmask;
            }
        }
        __syncthreads();
        const uint64_t out0 = p.output_offsets[leaf];
        uint64_t rec0 = p.leaf_base[leaf];
        constexpr uint32_t kStep = 2u * kWaves;
        if (kGrouped) {
            // Per member: its forward records (its valid slots) and its
            // reverse records (valid slots of other rows naming it); the
            // member's segment holds the forward ones, then the reverse ones.
            // With p.unique a slot whose reverse record another row's forward
            // record repeats (slot_listed) gets a bit in dup[row] and its
            // reverse record is neither counted nor written.
            for (uint32_t r0 = 2u * wave + h; r0 < n + h; r0 += kStep * kEmitUnroll) {
                uint32_t j[kEmitUnroll];
                float d[kEmitUnroll];
#pragma unroll
                for (int u = 0; u < kEmitUnroll; ++u) {
                    const uint32_t r = r0 + u * kStep;
                    j[u] = kNoKey;
                    d[u] = 0.0f;
                    if (r < n && q < kl) {
                        const uint64_t sl = out0 + (uint64_t)r * p.k + q;
                        j[u] = p.topk_ids[sl];
                        d[u] = p.topk_dists[sl];
                    }
                }
#pragma unroll
                for (int u = 0; u < kEmitUnroll; ++u) {
                    const uint32_t r = r0 + u * kStep;
                    const bool valid = slot_valid(j[u], d[u]);
                    const uint64_t m = __ballot(valid);
                    uint32_t cj = kNoKey;
                    if (valid) {
                        for (uint32_t slot = table_hash(j[u], tbits);; slot = (slot + 1u) & tmask) {
                            const uint32_t t = tkey[slot];
                            if (t == j[u]) {
                                cj = tval[slot];
                                break;
                            }
                            if (t == kNoKey) break;
                        }
                    }
                    bool same = false;
                    if (p.unique && cj != kNoKey && d[u] <= __uint_as_float(cnt[cj])) {
                        const uint32_t gi = gid[r];  // r < n: the slot is valid
                        if (gi != kNoKey) same = slot_listed(p, out0 + (uint64_t)cj * p.k, kl, gi, __float_as_uint(d[u]));
                    }
                    if (cj != kNoKey && !same) atomicAdd(&tot[cj], 1u);
                    const uint64_t sm = __ballot(same);
                    if (r < n && q == 0u) {
                        atomicAdd(&tot[r], (uint32_t)__popc((uint32_t)(h ? (m >> 32) : m)));
                        dup[r] = (uint32_t)(h ? (sm >> 32) : sm);
                    }
                }
            }
            __syncthreads();
            // exclusive scan of tot into cnt (segment offsets in the leaf)
            const uint32_t per = (n + kThreads - 1) / kThreads;
            const uint32_t b = tid * per;
            const uint32_t e = b + per < n ? b + per : n;
            uint32_t sum = 0;
            for (uint32_t i = b; i < e; ++i) sum += tot[i];
            uint32_t x = sum;
#pragma unroll
            for (uint32_t off = 1; off < 64; off <<= 1) {
                const uint32_t y = __shfl_up(x, off);
                if (lane >= off) x += y;
            }
            if (lane == 63u) wsum[wave] = x;
            __syncthreads();
            uint32_t base = 0, leaf_total = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                base += (uint32_t)w < wave ? wsum[w] : 0u;
                leaf_total += wsum[w];
            }
            if (p.unique) {
                // the leaf's place in the output: its records once the
                // repeats are left out, taken from the batch's cursor
                if (tid == 0) {
                    const uint64_t at = atomicAdd((unsigned long long *)&p.status[kEdgeKept],
                                                  (unsigned long long)leaf_total);
                    wsum[kWaves] = (uint32_t)at;
                    wsum[kWaves + 1] = (uint32_t)(at >> 32);
                }
                __syncthreads();
                rec0 = (uint64_t)wsum[kWaves] | ((uint64_t)wsum[kWaves + 1] << 32);
            }
            uint32_t run = base + x - sum;
            const uint64_t sbase = p.leaf_seg_base[leaf];
            for (uint32_t i = b; i < e; ++i) {
                const uint32_t c = tot[i];
                cnt[i] = run;
                const uint64_t first = rec0 + run;
                p.segments[sbase + i] = make_uint4(gid[i], (uint32_t)first, (uint32_t)(first >> 32), c);
                run += c;
                tot[i] = run;  // cursor: reverse records fill the segment from its end
            }
            __syncthreads();
        }
        for (uint32_t r0 = 2u * wave + h; r0 < n + h; r0 += kStep * kEmitUnroll) {
            uint32_t j[kEmitUnroll];
            float d[kEmitUnroll];
#pragma unroll
            for (int u = 0; u < kEmitUnroll; ++u) {
                const uint32_t r = r0 + u * kStep;
                j[u] = kNoKey;
                d[u] = 0.0f;
                if (r < n && q < kl) {
                    const uint64_t s = out0 + (uint64_t)r * p.k + q;
                    j[u] = p.topk_ids[s];
                    d[u] = p.topk_dists[s];
                }
            }
#pragma unroll
            for (int u = 0; u < kEmitUnroll; ++u) {
                const uint32_t r = r0 + u * kStep;
                const bool valid = slot_valid(j[u], d[u]);
                const uint64_t m = __ballot(valid);
                const uint32_t half = (uint32_t)(h ? (m >> 32) : m);
                const uint32_t gi = r < n ? gid[r] : kNoKey;
                // valid slots of the leaf before row r
                const uint32_t row_rec = r < n ? (regular ? r * kl : cnt[r]) : 0u;
                uint32_t hf = 0, hr = 0;
                bool ok = false;
                uint32_t cj = kNoKey;
                if (valid) {
                    // membership of j (leaf_build.rs:1783-1801)
                    for (uint32_t slot = table_hash(j[u], tbits);; slot = (slot + 1u) & tmask) {
                        const uint32_t t = tkey[slot];
                        if (t == j[u]) {
                            cj = tval[slot];
                            break;
                        }
                        if (t == kNoKey) break;
                    }
                    if (cj == kNoKey)
                        atomicMin((unsigned long long *)&p.status[kEdgeFirstError],
                                  (unsigned long long)edge_error_key(leaf, kEdgeErrOutside, r, q));
                    ok = cj != kNoKey && gi != kNoKey;  // a missing sketch row is reported by the table build
                    if (ok) {
                        if (kMode == kSketchLds)
                            pair_hashes<true>(sk_lds + r * mw, sk_lds + cj * mw, p.m_bits, hf, hr);
                        else
                            pair_hashes<kMode == kSketchGlobalV4>(p.sketches + (uint64_t)gi * p.width,
                                                                  p.sketches + (uint64_t)j[u] * p.width, p.m_bits,
                                                                  hf, hr);
                    }
                }
                const uint32_t db = __float_as_uint(d[u]);
                // Records of row r: 2 per valid slot, forward then reverse, from
                // record rec0 + 2*row_rec.  When every row of the wave has its
                // valid slots as a prefix of its ranks (always, for leaf top-k
                // output), lane q of a half writes records q and 32 + q of its
                // row, taking the slot's values by shuffle: 16-byte stores from
                // consecutive lanes to consecutive addresses.
                const uint64_t ok_mask = __ballot(ok);
                if (kGrouped) {
                    if (ok) {
                        // forward: its place among the row's valid slots; reverse:
                        // the last free place of j's segment
                        const uint32_t fpos = cnt[r] + (uint32_t)__popc(half & ((1u << q) - 1u));
                        store_record<true>(p.out, rec0 + fpos, gi, j[u], hf, db);
                        if (((dup[r] >> q) & 1u) == 0u) {
                            const uint32_t rpos = atomicSub(&tot[cj], 1u) - 1u;
                            store_record<true>(p.out, rec0 + rpos, j[u], gi, hr, db);
                        }
                    }
                    (void)ok_mask;
                    (void)row_rec;
                } else if (__ballot((half & (half + 1u)) != 0u) == 0ull) {
                    const uint32_t row_slots = (uint32_t)__popc(half);
                    const uint64_t base = rec0 + 2ull * row_rec;
#pragma unroll
                    for (uint32_t pass = 0; pass < 2u; ++pass) {
                        const uint32_t sidx = 16u * pass + (q >> 1);
                        const uint32_t src = (h << 5) + sidx;
                        const uint32_t js = __shfl(j[u], (int)src);
                        const uint32_t ds = __shfl(db, (int)src);
                        const uint32_t hfs = __shfl(hf, (int)src);
                        const uint32_t hrs = __shfl(hr, (int)src);
                        const bool oks = ((ok_mask >> src) & 1ull) != 0ull;
                        if (sidx < row_slots && oks) {
                            if (q & 1u)
                                store_record(p.out, base + 32u * pass + q, js, gi, hrs, ds);
                            else
                                store_record(p.out, base + 32u * pass + q, gi, js, hfs, ds);
                        }
                    }
                } else if (ok) {
                    const uint64_t pos = rec0 + 2ull * (row_rec + (uint32_t)__popc(half & ((1u << q) - 1u)));
                    store_record(p.out, pos, gi, j[u], hf, db);  // flags 0: evidence annotation off
                    store_record(p.out, pos + 1, j[u], gi, hr, db);
                }
            }
        }
        __syncthreads();  // the next leaf clears the table
    }
}

__global__ void edge_status_init_kernel(uint64_t *status) {
    if (threadIdx.x < kEdgeStatusWords) status[threadIdx.x] = threadIdx.x == kEdgeFirstError ? ~0ull : 0ull;
}

}  // namespace

uint32_t edge_table_bits(uint32_t max_leaf_rows) {
    uint32_t bits = 6;
    while ((1u << bits) < 2u * max_leaf_rows) ++bits;
    return bits;
}

int launch_edge_records(const EdgeParams &p, hipStream_t stream) {
    hipLaunchKernelGGL(edge_status_init_kernel, dim3(1), dim3(64), 0, stream, p.status);
    if (p.leaf_count == 0) return hipGetLastError() == hipSuccess ? 0 : -1;
    const uint32_t grid = p.leaf_count < 8192u ? p.leaf_count : 8192u;
    const size_t count_lds = (kWaves + (size_t)p.max_leaf_rows) * sizeof(uint32_t);
    hipLaunchKernelGGL(edge_count_kernel, dim3(grid), dim3(kThreads), count_lds, stream, p);
    hipLaunchKernelGGL(edge_scan_kernel, dim3(1), dim3(1024), 0, stream, p);
    // Stage the leaf's sketch rows in LDS when they fit; else read them from
    // HBM (float4 loads when rows are 16-byte aligned).
    const bool grouped = p.segments != nullptr;
    const size_t base_lds = (size_t)emit_sketch_offset(p.max_leaf_rows, p.table_bits, grouped) * sizeof(uint32_t);
    const size_t staged = (size_t)p.max_leaf_rows * ((p.m_bits + 3u) & ~3u) * sizeof(float);
    const bool vec4 = p.width % 4u == 0u && (reinterpret_cast<uintptr_t>(p.sketches) & 15u) == 0u;
    const bool in_lds = base_lds + staged <= kEmitLdsBudget;
    const size_t lds = in_lds ? base_lds + staged : base_lds;
    const void *emit_fn = grouped ? (in_lds ? reinterpret_cast<const void *>(edge_emit_kernel<kSketchLds, true>)
                                            : vec4 ? reinterpret_cast<const void *>(edge_emit_kernel<kSketchGlobalV4, true>)
                                                   : reinterpret_cast<const void *>(edge_emit_kernel<kSketchGlobal, true>))
                                  : (in_lds ? reinterpret_cast<const void *>(edge_emit_kernel<kSketchLds, false>)
                                            : vec4 ? reinterpret_cast<const void *>(edge_emit_kernel<kSketchGlobalV4, false>)
                                                   : reinterpret_cast<const void *>(edge_emit_kernel<kSketchGlobal, false>));
    if (ensure_lds_limit(emit_fn, (int)lds)) return -1;
    if (grouped) {
        if (in_lds)
            hipLaunchKernelGGL((edge_emit_kernel<kSketchLds, true>), dim3(grid), dim3(kThreads), lds, stream, p);
        else if (vec4)
            hipLaunchKernelGGL((edge_emit_kernel<kSketchGlobalV4, true>), dim3(grid), dim3(kThreads), lds, stream, p);
        else
            hipLaunchKernelGGL((edge_emit_kernel<kSketchGlobal, true>), dim3(grid), dim3(kThreads), lds, stream, p);
    } else {
        if (in_lds)
            hipLaunchKernelGGL((edge_emit_kernel<kSketchLds, false>), dim3(grid), dim3(kThreads), lds, stream, p);
        else if (vec4)
            hipLaunchKernelGGL((edge_emit_kernel<kSketchGlobalV4, false>), dim3(grid), dim3(kThreads), lds, stream, p);
        else
            hipLaunchKernelGGL((edge_emit_kernel<kSketchGlobal, false>), dim3(grid), dim3(kThreads), lds, stream, p);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
