// d0_assign.hip -- global D0 assignment on gfx950 int8 MFMA: every SQ8 row
// to its fanout_top (<= 32) nearest global D0 leaders, then the fragments
// grouped into the D0 children.
//
// Reference (shear-core/src/algorithm/pipnn/compute_backend.rs): the GPU-D0
// kernels sq8_global_d0_tiled_partial_kernel / sq8_global_d0_wmma_partial_kernel
// (:18016-18275, per leader tile the best partial_r leaders of each row) and
// the merge rabitq_residual_global_d0_tiled_merge_kernel (:18446-18511, the
// best fanout_top over the tiles), both ordered by (dist, leader global id)
// strictly, the distance sq_int8_approx_l2 (dco_sq_int8.rs:2950-2965):
// (norm_r + norm_l) - ((2 * scale_r) * scale_l) * dot, clamped at 0.  Output
// fragments row-major (child = leader index, point = global id, :18503-18510).
//
// Here one pass replaces partial + merge: a wave holds 32 rows' codes in VGPRs
// as the MFMA B operand and streams the leaders 32 at a time as A.  The eight
// waves of a workgroup (256 rows) share each leader tile through LDS (double
// buffered; the next tile's codes, scales, norms and ranks are loaded into
// registers while the current one is used), so a tile crosses L2 once per
// 256 rows instead of once per 32; each lane owns one row and
// half of a tile's leaders and keeps its best F >= fanout (distance bits << 32
// | leader rank) keys sorted in registers, inserting a candidate only when it
// beats the current F-th.  The two halves of a row merge at the end.  A
// leader's rank is its position in (leader id, index) order, so the key's
// integer order is the reference's order (distances are >= 0).
//
// Grouping: an LSD radix sort of (child, point) pairs by child, stable, so a
// child's points keep ascending row order; offsets from a child histogram.
#include <hipcub/hipcub.hpp>

#include "kernel_attr.h"
#include "d0_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8;  // 256 rows per workgroup share each leader tile
constexpr int kThreads = kWaves * 64;
constexpr uint64_t kNoKey = ~0ull;

// rank of each leader in (id, index) order; O(leaders^2) compares, leaders are few
__global__ void d0_rank_kernel(const uint32_t *ids, uint32_t n, uint32_t *rank, uint32_t *inv) {
    const uint32_t l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= n) return;
    const uint32_t me = ids[l];
    uint32_t r = 0;
    for (uint32_t o = 0; o < n; ++o) {
        const uint32_t v = ids[o];
        r += (v < me || (v == me && o < l)) ? 1u : 0u;
    }
    rank[l] = r;
    inv[r] = l;
}

template <int F>
__device__ __forceinline__ void insert_key(uint64_t (&best)[F], uint64_t key) {
#pragma unroll
    for (int s = 0; s < F; ++s) {
        const uint64_t b = best[s];
        const bool lt = key < b;
        best[s] = lt ? key : b;
        key = lt ? b : key;
    }
}

template <int KS>
struct D0Tile {
    static constexpr int kStride = KS * 32 + 16;          // bytes per leader row (16-byte pad: no bank aliasing)
    static constexpr int kCodeBytes = 32 * kStride;
    static constexpr int kChunks = 32 * KS * 2;           // 16-byte chunks of the tile's codes
    static constexpr int kPerThread = (kChunks + kThreads - 1) / kThreads;
    static constexpr int kBytes = kCodeBytes + 32 * 12;  // + scales, norms, ranks
};

template <int KS, int F>
__global__ __launch_bounds__(kThreads) void d0_assign_kernel(D0AssignParams p) {
    using T = D0Tile<KS>;
    extern __shared__ __attribute__((aligned(16))) int8_t tiles[];  // 2 x T::kBytes
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t j = lane & 31u, h = lane >> 5;
    const uint64_t row = (uint64_t)blockIdx.x * (kWaves * 32) + wave * 32u + j;
    const bool ok = row < p.rows;
    const uint32_t pd = p.padded_dim;
    const uint32_t nl = p.leaders;

    v4i bfrag[KS];
    const int8_t *rc = p.codes + (ok ? row : 0ull) * pd;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const uint32_t off = 32u * s + 16u * h;
        v4i z = {0, 0, 0, 0};
        if (ok && off < pd) z = *reinterpret_cast<const v4i *>(rc + off);
        bfrag[s] = z;
    }
    const float rs = ok ? p.scales[row] : 0.0f;
    const float rn = ok ? p.norms[row] : 0.0f;

    uint64_t best[F];
#pragma unroll
    for (int s = 0; s < F; ++s) best[s] = kNoKey;

    // the next tile in registers: this thread's code chunks and one meta word
    v4i pre[T::kPerThread];
    uint32_t pmeta = 0u;
    auto issue = [&](uint32_t t) {
#pragma unroll
        for (int q = 0; q < T::kPerThread; ++q) {
            const uint32_t c = tid + (uint32_t)q * kThreads;
            const uint32_t li = c / (KS * 2), off = (c % (KS * 2)) * 16u;
            const uint32_t l = 32u * t + li;
            v4i z = {0, 0, 0, 0};
            if (c < (uint32_t)T::kChunks && l < nl && off < pd)
                z = *reinterpret_cast<const v4i *>(p.leader_codes + (uint64_t)l * pd + off);
            pre[q] = z;
        }
        if (tid < 96u) {
            const uint32_t l = 32u * t + (tid & 31u);
            const uint32_t li = l < nl ? l : 0u;
            pmeta = tid < 32u ? __float_as_uint(p.leader_scales[li])
                              : tid < 64u ? __float_as_uint(p.leader_norms[li]) : p.leader_rank[li];
        }
    };
    auto store = [&](int8_t *dst) {
#pragma unroll
        for (int q = 0; q < T::kPerThread; ++q) {
            const uint32_t c = tid + (uint32_t)q * kThreads;
            if (c < (uint32_t)T::kChunks) {
                const uint32_t li = c / (KS * 2), off = (c % (KS * 2)) * 16u;
                *reinterpret_cast<v4i *>(dst + li * T::kStride + off) = pre[q];
            }
        }
        if (tid < 96u) reinterpret_cast<uint32_t *>(dst + T::kCodeBytes)[tid] = pmeta;
    };

    const uint32_t ntiles = (nl + 31u) / 32u;
    issue(0);
    store(tiles);
    if (ntiles > 1u) issue(1);
    for (uint32_t t = 0; t < ntiles; ++t) {
        // tile t is in buffer t & 1; the other buffer was last read at t - 1
        __syncthreads();
        int8_t *cur = tiles + (t & 1u) * T::kBytes;
        if (t + 1u < ntiles) {
            store(tiles + ((t + 1u) & 1u) * T::kBytes);
            if (t + 2u < ntiles) issue(t + 2u);
        }
        const int8_t *arow = cur + j * T::kStride + 16u * h;
        v16i acc = {};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const v4i a = *reinterpret_cast<const v4i *>(arow + 32 * s);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bfrag[s], acc, 0, 0, 0);
        }
        // lane value v is leader 8*(v/4) + 4h + v%4 of the tile: four consecutive
        // leaders per group, their scales / norms / ranks read as 16-byte vectors
        const float4 *tsc = reinterpret_cast<const float4 *>(cur + T::kCodeBytes);
        const float4 *tno = tsc + 8;
        const uint4 *trk = reinterpret_cast<const uint4 *>(tno + 8);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 sc4 = tsc[2 * g + h], no4 = tno[2 * g + h];
            const uint4 rk4 = trk[2 * g + h];
            const float scv[4] = {sc4.x, sc4.y, sc4.z, sc4.w}, nov[4] = {no4.x, no4.y, no4.z, no4.w};
            const uint32_t rkv[4] = {rk4.x, rk4.y, rk4.z, rk4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = 4 * g + e;
                const uint32_t l = 32u * t + 8u * g + 4u * h + e;
                const bool live = ok && l < nl;
                const float d = assign_l2(acc[v], rs, rn, scv[e], nov[e]);
                const uint64_t key = live ? (((uint64_t)__float_as_uint(d) << 32) | rkv[e]) : kNoKey;
                if (key < best[F - 1]) insert_key<F>(best, key);
            }
        }
    }
    // merge the other half-wave's list into lanes 0..31
#pragma unroll
    for (int s = 0; s < F; ++s) {
        const uint64_t o = ((uint64_t)__shfl((uint32_t)(best[s] >> 32), j + 32u) << 32) |
                           __shfl((uint32_t)best[s], j + 32u);
        if (h == 0u && o < best[F - 1]) insert_key<F>(best, o);
    }
    if (h == 0u && ok) {
        const uint32_t g = p.global_ids[row];
#pragma unroll
        for (int s = 0; s < F; ++s) {
            if ((uint32_t)s < p.fanout) {
                const uint32_t r = (uint32_t)best[s];  // always a real leader: fanout <= leaders
                p.out_child[row * p.fanout + s] = r < p.leaders ? p.rank_leader[r] : kEmptyId;
                p.out_point[row * p.fanout + s] = g;
            }
        }
    }
}

template <int KS, int F>
int launch_kf(const D0AssignParams &p, dim3 grid, hipStream_t stream) {
    constexpr int lds = 2 * D0Tile<KS>::kBytes;
    if (ensure_lds_limit(reinterpret_cast<const void *>(&d0_assign_kernel<KS, F>), (int)lds)) return -1;
    hipLaunchKernelGGL((d0_assign_kernel<KS, F>), grid, dim3(kThreads), lds, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int KS>
int launch_ks(const D0AssignParams &p, hipStream_t stream) {
    const uint64_t blocks = (p.rows + kWaves * 32 - 1) / (kWaves * 32);
    if (blocks > 0x7fffffffull) return -2;
    const dim3 grid((uint32_t)blocks);
    if (p.fanout <= 2) return launch_kf<KS, 2>(p, grid, stream);  // the builds' replication fanout
    if (p.fanout <= 4) return launch_kf<KS, 4>(p, grid, stream);
    if (p.fanout <= 8) return launch_kf<KS, 8>(p, grid, stream);
    if (p.fanout <= 16) return launch_kf<KS, 16>(p, grid, stream);
    return launch_kf<KS, 32>(p, grid, stream);
}

// Child histogram with per-workgroup counts in LDS (bins = leaders + 1 words,
// dynamic LDS), added to the global counts once per workgroup and bin: the
// ~1,000 global counters would otherwise take one atomic per fragment.
__global__ __launch_bounds__(256) void d0_hist_lds_kernel(const uint32_t *child, uint64_t n, uint32_t bins,
                                                          uint64_t *counts) {
    extern __shared__ uint32_t hist[];
    for (uint32_t b = threadIdx.x; b < bins; b += blockDim.x) hist[b] = 0u;
    __syncthreads();
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t b = child[i] + 1u;
        if (b < bins) atomicAdd(&hist[b], 1u);
        else atomicAdd(reinterpret_cast<unsigned long long *>(&counts[b]), 1ull);  // not a leader index
    }
    __syncthreads();
    for (uint32_t b = threadIdx.x; b < bins; b += blockDim.x)
        if (hist[b]) atomicAdd(reinterpret_cast<unsigned long long *>(&counts[b]), (unsigned long long)hist[b]);
}

__global__ void d0_hist_kernel(const uint32_t *child, uint64_t n, uint64_t *counts) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        atomicAdd(reinterpret_cast<unsigned long long *>(&counts[child[i] + 1]), 1ull);
}

__global__ void d0_fill_zero(uint64_t *a, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        a[i] = 0ull;
}

// inclusive scan of counts[1..n] in place (one workgroup; n = leaders is small)
__global__ __launch_bounds__(1024) void d0_scan_kernel(uint64_t *counts, uint32_t n) {
    __shared__ uint64_t part[1024];
    __shared__ uint64_t carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (uint32_t b = 0; b < n; b += 1024) {
        const uint32_t i = b + threadIdx.x;
        part[threadIdx.x] = i < n ? counts[i + 1] : 0ull;
        __syncthreads();
        for (uint32_t off = 1; off < 1024; off <<= 1) {
            const uint64_t v = threadIdx.x >= off ? part[threadIdx.x - off] : 0ull;
            __syncthreads();
            part[threadIdx.x] += v;
            __syncthreads();
        }
        if (i < n) counts[i + 1] = carry + part[threadIdx.x];
        __syncthreads();
        if (threadIdx.x == 0) carry += part[1023];
        __syncthreads();
    }
}

uint32_t key_bits(uint32_t leaders) {
    uint32_t b = 1;
    while (b < 32 && (1ull << b) < leaders) ++b;
    return b;
}

}  // namespace

int launch_d0_assign(const D0AssignParams &p, hipStream_t stream) {
    if (p.fanout == 0 || p.fanout > kD0MaxFanout || p.fanout > p.leaders || p.padded_dim % 16 != 0) return -3;
    hipLaunchKernelGGL(d0_rank_kernel, dim3((p.leaders + 255) / 256), dim3(256), 0, stream, p.leader_ids, p.leaders,
                       p.leader_rank, p.rank_leader);
    if (hipGetLastError() != hipSuccess) return -1;
    if (p.rows == 0) return 0;
    const uint32_t ks = (p.padded_dim + 31) / 32;
    if (ks <= 4) return launch_ks<4>(p, stream);
    if (ks <= 8) return launch_ks<8>(p, stream);
    if (ks <= 16) return launch_ks<16>(p, stream);
    if (ks <= 24) return launch_ks<24>(p, stream);
    if (ks <= 32) return launch_ks<32>(p, stream);
    return -3;
}

size_t d0_group_temp_bytes(uint64_t items, uint32_t leaders) {
    size_t sort_bytes = 0;
    hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                       (const uint32_t *)nullptr, (uint32_t *)nullptr, (int)items, 0,
                                       (int)key_bits(leaders));
    // sorted keys, then the sort's own storage (256-byte aligned)
    return ((items * 4 + 255) / 256) * 256 + sort_bytes;
}

int launch_d0_group(const D0AssignParams &p, uint64_t *child_offsets, uint32_t *child_points, void *temp,
                    size_t temp_bytes, hipStream_t stream) {
    const uint64_t items = p.rows * p.fanout;
    hipLaunchKernelGGL(d0_fill_zero, dim3(((uint64_t)p.leaders + 256) / 256), dim3(256), 0, stream, child_offsets,
                       (uint64_t)p.leaders + 1);
    if (items == 0) return hipGetLastError() == hipSuccess ? 0 : -1;
    uint64_t hg = (items + 255) / 256;
    const uint32_t bins = p.leaders + 1u;
    if (bins <= 16384u) {
        hg = hg > 512 ? 512 : hg;
        hipLaunchKernelGGL(d0_hist_lds_kernel, dim3((uint32_t)hg), dim3(256), bins * 4u, stream, p.out_child, items,
                           bins, child_offsets);
    } else {
        hg = hg > 8192 ? 8192 : hg;
        hipLaunchKernelGGL(d0_hist_kernel, dim3((uint32_t)hg), dim3(256), 0, stream, p.out_child, items,
                           child_offsets);
    }
    hipLaunchKernelGGL(d0_scan_kernel, dim3(1), dim3(1024), 0, stream, child_offsets, p.leaders);
    const size_t keys_bytes = ((items * 4 + 255) / 256) * 256;
    uint32_t *keys_out = reinterpret_cast<uint32_t *>(temp);
    size_t sort_bytes = temp_bytes - keys_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(reinterpret_cast<char *>(temp) + keys_bytes, sort_bytes, p.out_child,
                                           keys_out, p.out_point, child_points, (int)items, 0,
                                           (int)key_bits(p.leaders), stream) != hipSuccess)
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
