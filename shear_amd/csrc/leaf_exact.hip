// leaf_exact.hip -- exact scalar leaf top-k (the reference's DP4A role).
//
// One wavefront per (leaf, row).  Lanes compute 64 candidate distances at a
// time with packed int8 dot4; the candidates are then inserted, in member
// order, into the row's k-slot buffer with the reference rule
// (compute_backend.rs:7229-7259 / leaf_build.rs:887-957).  The buffer lives
// in lanes 0..k-1 (slot j in lane j).  A candidate that does not beat the
// buffer's tail is dropped, so one ballot finds the next candidate that can
// enter; its insertion position is one past the highest slot it does not beat
// (the reference's scan from the tail stops there) and the slots above shift
// up by one lane.  This kernel is the semantic baseline on the GPU; the rows
// the MFMA executor cannot certify are re-run with the same insertion by a
// workgroup per row (exact_row_wg), and rows with eps-tie chains are replayed
// by the chain kernel at the end of this file.
#include "leaf_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

constexpr int kExactThreads = 64;

// Lane i receives lane i-1's value (DPP wave shift; lane 0 keeps its own).
__device__ __forceinline__ uint32_t wave_shr1(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x138, 0xf, 0xf, false);
}
__device__ __forceinline__ float wave_shr1(float v) {
    return __uint_as_float(wave_shr1(__float_as_uint(v)));
}
// Broadcast of lane `i` (wave-uniform index).
__device__ __forceinline__ uint32_t lane_bcast(uint32_t v, uint32_t i) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)i);
}
__device__ __forceinline__ float lane_bcast(float v, uint32_t i) {
    return __uint_as_float(lane_bcast(__float_as_uint(v), i));
}

// Insert candidate (cd, cg) into the lane-distributed buffer (bd, bg) of
// length `len` <= keff; returns the new length.  Wave-uniform arguments.
__device__ __forceinline__ uint32_t wave_insert(float cd, uint32_t cg, float &bd, uint32_t &bg, uint32_t len,
                                                uint32_t keff) {
    const uint32_t lane = threadIdx.x & 63u;
    const bool b = lane < len && beats(cd, cg, bd, bg);
    uint32_t new_len = len;
    uint64_t stop;
    if (len < keff) {
        new_len = len + 1u;
        stop = __ballot(lane < len && !b);
    } else {
        const uint64_t bm = __ballot(b);
        if (((bm >> (keff - 1u)) & 1ull) == 0ull) return len;  // does not beat the tail
        stop = __ballot(lane + 1u < keff && !b);
    }
    const uint32_t pos = stop ? (uint32_t)(64 - __clzll((long long)stop)) : 0u;
    const float ud = wave_shr1(bd);
    const uint32_t ug = wave_shr1(bg);
    if (lane > pos && lane < new_len) {
        bd = ud;
        bg = ug;
    }
    if (lane == pos) {
        bd = cd;
        bg = cg;
    }
    return new_len;
}

__device__ void exact_row(const LeafParams &p, uint32_t leaf, uint32_t row) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n = p.member_counts[leaf];
    if (row >= n) return;
    const uint32_t *mem = p.members + p.member_offsets[leaf];
    const uint32_t keff = (p.k < n - 1u) ? p.k : (n - 1u);
    const uint32_t self = mem[row];
    if (self >= p.rows) {
        if (lane == 0) flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_ROW_ID);
        return;
    }
    const int8_t *rc = p.codes + (uint64_t)self * p.padded_dim;
    const float rs = p.scales[self];
    const float rn = p.norms[self];
    float bd = kEmptyDist;
    uint32_t bg = kEmptyId;
    uint32_t len = 0;
    for (uint32_t base = 0; base < n && keff > 0u; base += kExactThreads) {
        const uint32_t c = base + lane;
        float d = kEmptyDist;
        uint32_t g = kEmptyId;
        bool ok = c < n && c != row;
        if (ok) {
            const uint32_t cj = mem[c];
            if (cj >= p.rows) {
                flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_COL_ID);
                ok = false;
            } else {
                const int dot = dot_i8_rows(rc, p.codes + (uint64_t)cj * p.padded_dim, p.padded_dim);
                d = leaf_l2(dot, rs, rn, p.scales[cj], p.norms[cj]);
                g = p.gids[cj];
            }
        }
        // candidates in member order; skip those that cannot enter the full buffer
        uint32_t next = 0;
        while (true) {
            bool cand = ok && lane >= next;
            if (len == keff) {
                const float td = lane_bcast(bd, keff - 1u);
                const uint32_t tg = lane_bcast(bg, keff - 1u);
                cand = cand && beats(d, g, td, tg);
            }
            const uint64_t m = __ballot(cand);
            if (m == 0ull) break;
            const uint32_t i = (uint32_t)(__ffsll((long long)m) - 1);
            len = wave_insert(lane_bcast(d, i), lane_bcast(g, i), bd, bg, len, keff);
            next = i + 1u;
        }
    }
    const uint64_t out = p.output_offsets[leaf] + (uint64_t)row * p.k;
    if (lane < p.k) {
        p.out_ids[out + lane] = lane < len ? bg : kEmptyId;
        p.out_dists[out + lane] = lane < len ? bd : kEmptyDist;
    }
}

__global__ __launch_bounds__(kExactThreads) void leaf_exact_all_kernel(LeafParams p) {
    const uint64_t total = (uint64_t)p.leaf_count * p.max_leaf_rows;
    uint64_t done = 0;
    for (uint64_t w = blockIdx.x; w < total; w += gridDim.x) {
        const uint32_t leaf = (uint32_t)(w / p.max_leaf_rows);
        const uint32_t row = (uint32_t)(w % p.max_leaf_rows);
        if (row < p.member_counts[leaf]) {
            exact_row(p, leaf, row);
            ++done;
        }
    }
    if (threadIdx.x == 0) {
        counter_add(p.counters, TESSA_C_LEAF_EXACT_ROWS, done);
        counter_add(p.counters, TESSA_C_LEAF_ROWS, done);
    }
}

// Re-run of the rows the MFMA executor could not certify: one 512-thread
// workgroup per row.  The row's distances to a chunk of 1,024 member columns
// are computed four lanes per column (a quarter of the dims each, summed over
// the quad) into LDS; then wave 0 inserts them in member order with the rule
// of exact_row.  Few rows (often a few hundred) are re-run per call, so the
// latency of one row is what counts; a grid of 512 workgroups strides over
// the device-side row count.  The workgroup size trades that latency against
// scheduling beside other streams' kernels (the build runs the leaf operator
// beside record emission and reservoir merges): 1,024-thread workgroups,
// which need 16 free wave slots on one CU, took 14-62 ms per C3 build there
// against 2-17 ms at 512 threads, and C2 alone 0.091 against 0.104 ms.
#ifndef TESSA_FALLBACK_THREADS
#define TESSA_FALLBACK_THREADS 512
#endif
#ifndef TESSA_FALLBACK_GRID
#define TESSA_FALLBACK_GRID 512
#endif
constexpr int kFallbackThreads = TESSA_FALLBACK_THREADS;
constexpr uint32_t kFallbackChunk = 1024;

__device__ void exact_row_wg(const LeafParams &p, uint32_t leaf, uint32_t row, float *sd, uint32_t *sg,
                             uint8_t *sv) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n = p.member_counts[leaf];
    if (row >= n) return;
    const uint32_t *mem = p.members + p.member_offsets[leaf];
    const uint32_t keff = (p.k < n - 1u) ? p.k : (n - 1u);
    const uint32_t self = mem[row];
    if (self >= p.rows) {
        if (tid == 0) flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_ROW_ID);
        return;
    }
    const int4 *rc = reinterpret_cast<const int4 *>(p.codes + (uint64_t)self * p.padded_dim);
    const float rs = p.scales[self];
    const float rn = p.norms[self];
    const uint32_t pieces = p.padded_dim / 16u;
    float bd = kEmptyDist;
    uint32_t bg = kEmptyId;
    uint32_t len = 0;
    for (uint32_t cb = 0; cb < n && keff > 0u; cb += kFallbackChunk) {
        const uint32_t cn = (n - cb < kFallbackChunk) ? n - cb : kFallbackChunk;
        __syncthreads();  // the previous chunk's insertion is done with sd/sg/sv
        for (uint32_t j = tid >> 2; j < cn; j += kFallbackThreads / 4) {
            const uint32_t c = cb + j, q = tid & 3u;
            const uint32_t cj = mem[c];
            const bool ok = c != row && cj < p.rows;
            int acc = 0;
            if (ok) {
                const int4 *cc = reinterpret_cast<const int4 *>(p.codes + (uint64_t)cj * p.padded_dim);
                for (uint32_t i = q; i < pieces; i += 4u) {
                    const int4 x = rc[i], y = cc[i];
                    acc = __builtin_amdgcn_sdot4(x.x, y.x, acc, false);
                    acc = __builtin_amdgcn_sdot4(x.y, y.y, acc, false);
                    acc = __builtin_amdgcn_sdot4(x.z, y.z, acc, false);
                    acc = __builtin_amdgcn_sdot4(x.w, y.w, acc, false);
                }
            }
            acc += __shfl_xor(acc, 1);
            acc += __shfl_xor(acc, 2);
            if (q == 0u) {
                if (c != row && cj >= p.rows) flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_COL_ID);
                sd[j] = ok ? leaf_l2(acc, rs, rn, p.scales[cj], p.norms[cj]) : kEmptyDist;
                sg[j] = ok ? p.gids[cj] : kEmptyId;
                sv[j] = ok ? 1u : 0u;
            }
        }
        __syncthreads();
        if (wave == 0u) {
            for (uint32_t base = 0; base < cn; base += 64u) {
                const uint32_t j = base + lane;
                const bool ok = j < cn && sv[j] != 0u;
                const float d = ok ? sd[j] : kEmptyDist;
                const uint32_t g = ok ? sg[j] : kEmptyId;
                uint32_t next = 0;
                while (true) {
                    bool cand = ok && lane >= next;
                    if (len == keff) {
                        const float td = lane_bcast(bd, keff - 1u);
                        const uint32_t tg = lane_bcast(bg, keff - 1u);
                        cand = cand && beats(d, g, td, tg);
                    }
                    const uint64_t m = __ballot(cand);
                    if (m == 0ull) break;
                    const uint32_t i = (uint32_t)(__ffsll((long long)m) - 1);
                    len = wave_insert(lane_bcast(d, i), lane_bcast(g, i), bd, bg, len, keff);
                    next = i + 1u;
                }
            }
        }
    }
    if (wave == 0u) {
        const uint64_t out = p.output_offsets[leaf] + (uint64_t)row * p.k;
        if (lane < p.k) {
            p.out_ids[out + lane] = lane < len ? bg : kEmptyId;
            p.out_dists[out + lane] = lane < len ? bd : kEmptyDist;
        }
    }
}

__global__ __launch_bounds__(kFallbackThreads) void leaf_exact_fallback_kernel(LeafParams p) {
    __shared__ float sd[kFallbackChunk];
    __shared__ uint32_t sg[kFallbackChunk];
    __shared__ uint8_t sv[kFallbackChunk];
    uint32_t count = *p.fallback_count;
    if (count > p.fallback_capacity) count = p.fallback_capacity;
    uint64_t done = 0;
    for (uint32_t w = blockIdx.x; w < count; w += gridDim.x) {
        exact_row_wg(p, p.fallback[2 * w], p.fallback[2 * w + 1], sd, sg, sv);
        __syncthreads();  // the next row's first chunk overwrites sd/sg/sv
        ++done;
    }
    if (threadIdx.x == 0) {
        counter_add(p.counters, TESSA_C_LEAF_EXACT_ROWS, done);
        counter_add(p.counters, TESSA_C_LEAF_ROWS, done);
    }
}

// ---- chain replay -----------------------------------------------------------
// For a row whose certified candidate set G (every candidate outside G is more
// than 2e-5 above all of G) contains an eps-tie chain, the reference result is
// the bounded insertion over G's members in column order; other candidates can
// neither enter in front of G's nor stay in the buffer.
//
// One lane per queued row (|G| <= 40).  The lane sorts (column, index) keys of
// G in registers, keeps the sorted indices in LDS, reads G's (distance, global
// id) back from the pool in column order two steps ahead (scattered 16-byte
// reads: most miss L2 and fetch a whole sector from HBM, which at four waves
// per SIMD still beats holding G in LDS at 1.5), and replays the bounded
// insertion of leaf_build.rs:913-951 over
// a 32-slot list in registers: slot s is visited from the back, and a
// candidate moves forward while it beats the slot before it.  Blocks of 8
// slots that no lane of the wave can touch are skipped.  With 5 KB of LDS per
// workgroup the kernel runs four waves per SIMD (at most 128 VGPRs); rows
// whose output is 16-byte aligned are written with vector stores.
constexpr int kChainSeq = (int)kLeafChainSetEntries;  // G holds at most kMaxK + 8 entries
constexpr int kChainSlots = kMaxK; // the row's top-k list
constexpr int kChainThreads = 128;

__global__ __launch_bounds__(kChainThreads) __attribute__((amdgpu_waves_per_eu(4))) void leaf_chain_kernel(LeafParams p) {
    __shared__ uint8_t order[kChainSeq][kChainThreads];  // G's entry indices in column order
    const uint32_t tid = threadIdx.x;
    uint32_t count = *p.chain_count;
    if (count > p.chain_capacity) count = p.chain_capacity;
    uint64_t done = 0;
    for (uint32_t base = blockIdx.x * kChainThreads; base < count; base += gridDim.x * kChainThreads) {
        const uint32_t w = base + tid;
        const bool live = w < count;
        const uint4 hdr = live ? p.chain_rows[w] : make_uint4(0u, 0u, 0u, 0u);
        uint32_t m = hdr.w & 0xffu;
        m = m < (uint32_t)kChainSeq ? m : (uint32_t)kChainSeq;
        const uint32_t keff = (hdr.w >> 8) & 0xffu;
        // keys: column << 6 | index, padding sorts last
        uint32_t key[64];
#pragma unroll
        for (int i = 0; i < 64; ++i) key[i] = 0xffffffffu;
#pragma unroll
        for (int i = 0; i < kChainSeq; ++i) {
            if ((uint32_t)i < m) {
                const uint4 e = p.chain_pool[(uint64_t)hdr.z + (uint64_t)i * 64u];  // 64 rows interleaved
                key[i] = (e.y << 6) | (uint32_t)i;
            }
        }
#pragma unroll
        for (int kk = 2; kk <= 64; kk <<= 1) {
#pragma unroll
            for (int jj = kk >> 1; jj > 0; jj >>= 1) {
#pragma unroll
                for (int i = 0; i < 64; ++i) {
                    const int l = i ^ jj;
                    if (l > i) {
                        const uint32_t lo = min(key[i], key[l]), hi = max(key[i], key[l]);
                        const bool up = (i & kk) == 0;
                        key[i] = up ? lo : hi;
                        key[l] = up ? hi : lo;
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kChainSeq; ++i) order[i][tid] = (uint8_t)(key[i] & 63u);
        // bounded insertion in column order
        float bd[kChainSlots];
        uint32_t bg[kChainSlots];
#pragma unroll
        for (int s = 0; s < kChainSlots; ++s) {
            bd[s] = kEmptyDist;
            bg[s] = kEmptyId;
        }
        uint32_t len = 0;
        // G's entries in column order, read back from the pool two steps ahead
        const uint4 *gp = p.chain_pool + hdr.z;
        auto fetch = [&](int t) {
            uint2 v = make_uint2(0u, 0u);
            if ((uint32_t)t < m && keff > 0u) {
                const uint4 e = gp[(uint64_t)order[t][tid] * 64u];
                v = make_uint2(e.x, e.z);
            }
            return v;
        };
        uint2 x0 = fetch(0), x1 = fetch(1);
        for (int t = 0; t < kChainSeq; ++t) {
            if (!__any((uint32_t)t < m && keff > 0u)) break;
            const bool act = (uint32_t)t < m && keff > 0u;
            const uint2 x = x0;
            x0 = x1;
            x1 = fetch(t + 2);
            const float dc = __uint_as_float(x.x);
            const uint32_t gc = x.y;
            const bool full = len >= keff;
            // start: the slot the candidate takes first (the empty slot, or the
            // last one, which it must beat to enter at all)
            const int start = act ? (int)(full ? keff - 1u : len) : -1;
            bool moving = false;
#pragma unroll
            for (int blk = kChainSlots / 8 - 1; blk >= 0; --blk) {
                // a lane works in this block while its candidate moves through it
                // or enters here (start in the block)
                if (!__any(moving || (start >= 8 * blk && start < 8 * blk + 8))) continue;
                // beats(c, slot s) for the block's first slot; later slots carry it down
                bool b_next = beats(dc, gc, bd[8 * blk + 7], bg[8 * blk + 7]);
#pragma unroll
                for (int u = 7; u >= 0; --u) {
                    const int s = 8 * blk + u;
                    const bool b_here = b_next;  // beats(c, slot s), before any change to slot s
                    if (s == start) moving = full ? b_here : true;
                    const bool b_prev = s > 0 ? beats(dc, gc, bd[s > 0 ? s - 1 : 0], bg[s > 0 ? s - 1 : 0]) : false;
                    const bool shift = moving && b_prev;
                    const float nd = moving ? (shift ? bd[s > 0 ? s - 1 : 0] : dc) : bd[s];
                    const uint32_t ng = moving ? (shift ? bg[s > 0 ? s - 1 : 0] : gc) : bg[s];
                    bd[s] = nd;
                    bg[s] = ng;
                    moving = shift;
                    b_next = b_prev;
                }
            }
            len += (act && !full) ? 1u : 0u;
        }
        if (live) {
            const uint64_t out = (uint64_t)hdr.x | ((uint64_t)hdr.y << 32);
            if (((p.k | (uint32_t)out) & 3u) == 0u) {
#pragma unroll
                for (int s = 0; s < kChainSlots; s += 4) {
                    if ((uint32_t)s >= p.k) continue;
                    uint4 vi, vd;
                    vi.x = (uint32_t)s + 0u < len ? bg[s + 0] : kEmptyId;
                    vi.y = (uint32_t)s + 1u < len ? bg[s + 1] : kEmptyId;
                    vi.z = (uint32_t)s + 2u < len ? bg[s + 2] : kEmptyId;
                    vi.w = (uint32_t)s + 3u < len ? bg[s + 3] : kEmptyId;
                    vd.x = __float_as_uint((uint32_t)s + 0u < len ? bd[s + 0] : kEmptyDist);
                    vd.y = __float_as_uint((uint32_t)s + 1u < len ? bd[s + 1] : kEmptyDist);
                    vd.z = __float_as_uint((uint32_t)s + 2u < len ? bd[s + 2] : kEmptyDist);
                    vd.w = __float_as_uint((uint32_t)s + 3u < len ? bd[s + 3] : kEmptyDist);
                    *reinterpret_cast<uint4 *>(p.out_ids + out + s) = vi;
                    *reinterpret_cast<uint4 *>(p.out_dists + out + s) = vd;
                }
                done += 1;
                continue;
            }
#pragma unroll
            for (int s = 0; s < kChainSlots; ++s) {
                if ((uint32_t)s >= p.k) continue;
                const bool keep = (uint32_t)s < len;
                p.out_ids[out + s] = keep ? bg[s] : kEmptyId;
                p.out_dists[out + s] = keep ? bd[s] : kEmptyDist;
            }
            done += 1;
        }
    }
    // one atomic per wave
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) done += __shfl_xor(done, off);
    if ((tid & 63u) == 0u) counter_add(p.counters, TESSA_C_LEAF_ROWS, done);
}

}  // namespace

int launch_leaf_chain(const LeafParams &p, hipStream_t stream) {
    // grid-stride over the device-side queue count: no host round trip
    hipLaunchKernelGGL(leaf_chain_kernel, dim3(4096), dim3(kChainThreads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_leaf_exact_all(const LeafParams &p, hipStream_t stream) {
    const uint64_t total = (uint64_t)p.leaf_count * p.max_leaf_rows;
    if (total == 0) return 0;
    const uint32_t grid = (uint32_t)(total < 65536 ? total : 65536);
    hipLaunchKernelGGL(leaf_exact_all_kernel, dim3(grid), dim3(kExactThreads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_leaf_exact_fallback(const LeafParams &p, hipStream_t stream) {
    // Grid-stride over the device-side count: no host round trip.
    hipLaunchKernelGGL(leaf_exact_fallback_kernel, dim3(TESSA_FALLBACK_GRID), dim3(kFallbackThreads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
