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

namespace tessa {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kTableBits = 13;  // 8192 slots >= 2 x kEdgeMaxLeafRows
constexpr uint32_t kTableSize = 1u << kTableBits;
constexpr uint32_t kNoKey = 0xffffffffu;

__device__ __forceinline__ bool slot_valid(uint32_t id, float d) {
    // j != u32::MAX && d.is_finite()
    return id != 0xffffffffu && (__float_as_uint(d) & 0x7f800000u) != 0x7f800000u;
}

__device__ __forceinline__ uint32_t table_hash(uint32_t g) { return (g * 0x9E3779B1u) >> (32 - kTableBits); }

__device__ __forceinline__ uint32_t leaf_k(const EdgeParams &p, uint32_t n) {
    return n > 1u ? (p.k < n - 1u ? p.k : n - 1u) : 0u;
}

// Valid-slot count of every row of leaf `leaf` into cnt[0..n), then an
// exclusive scan in place; returns the leaf total.  All threads call it.
__device__ uint32_t row_counts_scan(const EdgeParams &p, uint32_t leaf, uint32_t n, uint32_t kl, uint32_t *cnt,
                                    uint32_t *wsum) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t q = lane & 31u;
    const uint32_t h = lane >> 5;
    const uint64_t out0 = p.output_offsets[leaf];
    for (uint32_t r0 = 2u * wave; r0 < n; r0 += 2u * kWaves) {
        const uint32_t r = r0 + h;
        bool valid = false;
        if (r < n && q < kl) {
            const uint64_t s = out0 + (uint64_t)r * p.k + q;
            valid = slot_valid(p.topk_ids[s], p.topk_dists[s]);
        }
        const uint64_t m = __ballot(valid);
        if (r < n && q == 0u) cnt[r] = __popcll(h ? (m >> 32) : (m & 0xffffffffull));
    }
    __syncthreads();
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
    __shared__ uint32_t cnt[kEdgeMaxLeafRows];
    __shared__ uint32_t wsum[kWaves];
    for (uint32_t leaf = blockIdx.x; leaf < p.leaf_count; leaf += gridDim.x) {
        uint32_t n = p.member_counts[leaf];
        if (n > kEdgeMaxLeafRows) {
            if (threadIdx.x == 0) atomicMax((unsigned long long *)&p.status[kEdgeLeafTooLarge], 1ull + n);
            n = 0;
        }
        const uint32_t total = row_counts_scan(p, leaf, n, leaf_k(p, n), cnt, wsum);
        if (threadIdx.x == 0) p.leaf_totals[leaf] = total;
    }
}

__global__ __launch_bounds__(1024) void edge_scan_kernel(EdgeParams p) {
    __shared__ uint64_t wsum[16];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    uint64_t carry = 0;
    for (uint32_t base = 0; base < p.leaf_count; base += 1024u) {
        const uint32_t i = base + tid;
        const uint64_t v = i < p.leaf_count ? p.leaf_totals[i] : 0ull;
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
        if (i < p.leaf_count) p.leaf_base[i] = 2ull * (carry + before + x - v);  // records
        carry += total;
        __syncthreads();
    }
    if (tid == 0) {
        p.leaf_base[p.leaf_count] = 2ull * carry;
        p.status[kEdgeRecordCount] = 2ull * carry;
    }
}

__global__ __launch_bounds__(kThreads) void edge_emit_kernel(EdgeParams p) {
    __shared__ uint32_t cnt[kEdgeMaxLeafRows];
    __shared__ uint32_t table[kTableSize];
    __shared__ uint32_t wsum[kWaves];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t q = lane & 31u;
    const uint32_t h = lane >> 5;
    if (p.leaf_base[p.leaf_count] > p.out_capacity) {
        if (blockIdx.x == 0 && tid == 0) p.status[kEdgeCapacityHit] = 1ull;
        return;  // uniform over the grid: nothing is written
    }
    for (uint32_t leaf = blockIdx.x; leaf < p.leaf_count; leaf += gridDim.x) {
        uint32_t n = p.member_counts[leaf];
        n = n <= kEdgeMaxLeafRows ? n : 0u;  // reported by the count kernel
        const uint32_t kl = leaf_k(p, n);
        const uint32_t *mem = p.members + p.member_offsets[leaf];
        for (uint32_t i = tid; i < kTableSize; i += kThreads) table[i] = kNoKey;
        row_counts_scan(p, leaf, n, kl, cnt, wsum);  // ends with a barrier (table cleared)
        // Membership table of the leaf's global ids.  A point without a
        // resident row or sketch row is an error (the reference's sketch
        // prefetch of the batch, leaf_build.rs:1758-1763) and is left out.
        for (uint32_t c = tid; c < n; c += kThreads) {
            const uint32_t mr = mem[c];
            const uint32_t g = mr < p.resident_rows ? p.gids[mr] : kNoKey;
            if (mr >= p.resident_rows || g >= p.sketch_rows) {
                atomicMin((unsigned long long *)&p.status[kEdgeFirstError],
                          (unsigned long long)edge_error_key(leaf, kEdgeErrSketch, c, 0));
                continue;
            }
            uint32_t slot = table_hash(g);
            while (true) {
                const uint32_t prev = atomicCAS(&table[slot], kNoKey, g);
                if (prev == kNoKey || prev == g) break;
                slot = (slot + 1u) & (kTableSize - 1u);
            }
        }
        __syncthreads();
        const uint64_t out0 = p.output_offsets[leaf];
        const uint64_t rec0 = p.leaf_base[leaf];
        for (uint32_t r0 = 2u * wave; r0 < n; r0 += 2u * kWaves) {
            const uint32_t r = r0 + h;
            bool valid = false;
            uint32_t j = kNoKey;
            float d = 0.0f;
            if (r < n && q < kl) {
                const uint64_t s = out0 + (uint64_t)r * p.k + q;
                j = p.topk_ids[s];
                d = p.topk_dists[s];
                valid = slot_valid(j, d);
            }
            const uint64_t m = __ballot(valid);
            if (!valid) continue;
            const uint32_t half = (uint32_t)(h ? (m >> 32) : m);
            const uint64_t pos = rec0 + 2ull * (cnt[r] + (uint32_t)__popc(half & ((1u << q) - 1u)));
            const uint32_t mr = mem[r];
            const uint32_t gi = mr < p.resident_rows ? p.gids[mr] : kNoKey;
            // membership of j (leaf_build.rs:1783-1801)
            bool member = false;
            for (uint32_t slot = table_hash(j);; slot = (slot + 1u) & (kTableSize - 1u)) {
                const uint32_t t = table[slot];
                if (t == j) {
                    member = true;
                    break;
                }
                if (t == kNoKey) break;
            }
            if (!member) {
                atomicMin((unsigned long long *)&p.status[kEdgeFirstError],
                          (unsigned long long)edge_error_key(leaf, kEdgeErrOutside, r, q));
                continue;
            }
            if (gi >= p.sketch_rows) continue;  // reported by the table build
            const float *si = p.sketches + (uint64_t)gi * p.width;
            const float *sj = p.sketches + (uint64_t)j * p.width;
            uint32_t hf = 0, hr = 0;
            for (uint32_t bit = 0; bit < p.m_bits; ++bit) {
                const float a = si[bit], c = sj[bit];
                hf |= (c - a >= 0.0f ? 1u : 0u) << bit;  // compute_hash(s_i, s_j)
                hr |= (a - c >= 0.0f ? 1u : 0u) << bit;  // compute_hash(s_j, s_i)
            }
            const uint32_t db = __float_as_uint(d);
            p.out[pos] = make_uint4(gi, j, hf, db);  // flags 0: evidence annotation off
            p.out[pos + 1] = make_uint4(j, gi, hr, db);
        }
        __syncthreads();  // the next leaf clears the table
    }
}

__global__ void edge_status_init_kernel(uint64_t *status) {
    if (threadIdx.x < kEdgeStatusWords) status[threadIdx.x] = threadIdx.x == kEdgeFirstError ? ~0ull : 0ull;
}

}  // namespace

int launch_edge_records(const EdgeParams &p, hipStream_t stream) {
    hipLaunchKernelGGL(edge_status_init_kernel, dim3(1), dim3(64), 0, stream, p.status);
    if (p.leaf_count == 0) return hipGetLastError() == hipSuccess ? 0 : -1;
    const uint32_t grid = p.leaf_count < 4096u ? p.leaf_count : 4096u;
    hipLaunchKernelGGL(edge_count_kernel, dim3(grid), dim3(kThreads), 0, stream, p);
    hipLaunchKernelGGL(edge_scan_kernel, dim3(1), dim3(1024), 0, stream, p);
    hipLaunchKernelGGL(edge_emit_kernel, dim3(grid), dim3(kThreads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
