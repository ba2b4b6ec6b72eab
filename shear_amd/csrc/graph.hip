// graph.hip -- graph emission: the `_mem.index` byte image of a neighbour
// table, built on the GPU.
//
// Reference (shear-core/src/index/inmem_index/pipnn_oom_writer.rs:23-72,
// DirectMemGraphWriter): a 24-byte header (index_size u64, max_degree u32,
// start u32, num_frozen_pts u64; rewritten by finish() once the rows are
// in), then per point in id order its degree (u32) and its neighbour ids
// (u32), little-endian.  index_size is the file size; max_degree the largest
// degree.  Here the rows come from a [points x row_stride] table with a count
// per point (the HashPrune reservoirs' slot targets, in slot order).
//
// Kernels: a u64 exclusive scan of (1 + count) over the points (per-block
// sums, one workgroup over the sums, per-block apply) gives each row's word
// offset; the max degree is an atomicMax reduction; one pass writes the
// header and every row's words (consecutive threads on consecutive words).
#include "graph_kernels.h"

namespace tessa {

namespace {

constexpr int kGThreads = 1024;
constexpr int kGPer = 4;
constexpr uint32_t kGBlock = kGThreads * kGPer;

__device__ __forceinline__ uint64_t wave_excl_scan64(uint64_t v, uint32_t lane, uint64_t &total) {
    uint64_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t y = __shfl_up(x, off);
        if (lane >= (uint32_t)off) x += y;
    }
    total = __shfl(x, 63);
    return x - v;
}

// words of point p's row: its degree and its neighbours
__device__ __forceinline__ uint64_t row_words(const uint32_t *counts, uint32_t p, uint32_t stride) {
    const uint32_t c = counts[p];
    return 1ull + (c < stride ? c : stride);
}

__global__ __launch_bounds__(kGThreads) void g_block_sums(const uint32_t *counts, uint32_t n, uint32_t stride,
                                                         uint64_t *sums, uint32_t *max_degree) {
    __shared__ uint64_t ws[kGThreads / 64];
    const uint32_t base = blockIdx.x * kGBlock + threadIdx.x * kGPer;
    uint64_t v = 0;
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < kGPer; ++e) {
        if (base + e < n) {
            const uint64_t w = row_words(counts, base + e, stride);
            v += w;
            m = m > (uint32_t)(w - 1) ? m : (uint32_t)(w - 1);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_xor(v, off);
        const uint32_t o = __shfl_xor(m, off);
        m = m > o ? m : o;
    }
    if ((threadIdx.x & 63u) == 0) {
        ws[threadIdx.x >> 6] = v;
        atomicMax(max_degree, m);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t t = 0;
        for (int w = 0; w < kGThreads / 64; ++w) t += ws[w];
        sums[blockIdx.x] = t;
    }
}

__global__ __launch_bounds__(kGThreads) void g_scan_sums(uint64_t *sums, uint32_t nb, uint64_t *total_words) {
    __shared__ uint64_t ws[kGThreads / 64];
    __shared__ uint64_t carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (uint32_t b0 = 0; b0 < nb; b0 += kGThreads) {
        const uint32_t i = b0 + threadIdx.x;
        const uint64_t v = i < nb ? sums[i] : 0ull;
        uint64_t wt;
        const uint64_t ex = wave_excl_scan64(v, lane, wt);
        if (lane == 0) ws[wave] = wt;
        __syncthreads();
        uint64_t before = 0, all = 0;
        for (uint32_t w = 0; w < kGThreads / 64; ++w) {
            before += w < wave ? ws[w] : 0ull;
            all += ws[w];
        }
        if (i < nb) sums[i] = carry + before + ex;
        __syncthreads();
        if (threadIdx.x == 0) carry += all;
        __syncthreads();
    }
    if (threadIdx.x == 0) *total_words = carry;
}

__global__ __launch_bounds__(kGThreads) void g_apply(const uint32_t *counts, uint32_t n, uint32_t stride,
                                                    const uint64_t *sums, uint64_t *row_off) {
    __shared__ uint64_t ws[kGThreads / 64];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t base = blockIdx.x * kGBlock + threadIdx.x * kGPer;
    uint64_t v[kGPer], t = 0;
#pragma unroll
    for (int e = 0; e < kGPer; ++e) {
        v[e] = base + e < n ? row_words(counts, base + e, stride) : 0ull;
        t += v[e];
    }
    uint64_t wt;
    const uint64_t ex = wave_excl_scan64(t, lane, wt);
    if (lane == 0) ws[wave] = wt;
    __syncthreads();
    uint64_t run = sums[blockIdx.x] + ex;
    for (uint32_t w = 0; w < wave; ++w) run += ws[w];
#pragma unroll
    for (int e = 0; e < kGPer; ++e) {
        if (base + e < n) row_off[base + e] = run;
        run += v[e];
    }
}

// One thread per (point, word): word 0 is the degree, word 1 + s neighbour s.
__global__ void g_pack(const uint32_t *targets, const uint32_t *counts, uint32_t n, uint32_t stride,
                       const uint64_t *row_off, const uint64_t *total_words, const uint32_t *max_degree,
                       uint32_t start, uint64_t num_frozen, uint32_t *out_words) {
    const uint64_t per = (uint64_t)stride + 1u;
    const uint64_t total = (uint64_t)n * per;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t p = (uint32_t)(i / per), s = (uint32_t)(i % per);
        const uint32_t c = counts[p] < stride ? counts[p] : stride;
        if (s > c) continue;
        // the header is 6 words; rows follow
        out_words[6 + row_off[p] + s] = s == 0 ? c : targets[(uint64_t)p * stride + (s - 1)];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const uint64_t size = 24ull + 4ull * *total_words;
        out_words[0] = (uint32_t)size;
        out_words[1] = (uint32_t)(size >> 32);
        out_words[2] = *max_degree;
        out_words[3] = start;
        out_words[4] = (uint32_t)num_frozen;
        out_words[5] = (uint32_t)(num_frozen >> 32);
    }
}

__global__ void g_init(uint32_t *max_degree) { *max_degree = 0u; }

uint32_t g_grid(uint64_t n, uint32_t threads, uint32_t cap) {
    const uint64_t g = (n + threads - 1) / threads;
    return (uint32_t)(g < 1 ? 1 : (g > cap ? cap : g));
}

}  // namespace

uint64_t graph_scan_blocks(uint32_t num_points) { return (num_points + kGBlock - 1) / kGBlock + 1; }

int launch_graph_size(const GraphPackParams &p, hipStream_t stream) {
    const uint32_t nb = (p.num_points + kGBlock - 1) / kGBlock;
    hipLaunchKernelGGL(g_init, dim3(1), dim3(1), 0, stream, p.max_degree);
    if (p.num_points) {
        hipLaunchKernelGGL(g_block_sums, dim3(nb), dim3(kGThreads), 0, stream, p.counts, p.num_points, p.row_stride,
                           p.block_sums, p.max_degree);
    }
    hipLaunchKernelGGL(g_scan_sums, dim3(1), dim3(kGThreads), 0, stream, p.block_sums, nb, p.total_words);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_graph_pack(const GraphPackParams &p, hipStream_t stream) {
    const uint32_t nb = (p.num_points + kGBlock - 1) / kGBlock;
    if (p.num_points) {
        hipLaunchKernelGGL(g_apply, dim3(nb), dim3(kGThreads), 0, stream, p.counts, p.num_points, p.row_stride,
                           p.block_sums, p.row_off);
    }
    const uint64_t total = (uint64_t)p.num_points * ((uint64_t)p.row_stride + 1u);
    hipLaunchKernelGGL(g_pack, dim3(g_grid(total, 256, 16384)), dim3(256), 0, stream, p.targets, p.counts,
                       p.num_points, p.row_stride, p.row_off, p.total_words, p.max_degree, p.start, p.num_frozen,
                       p.out_words);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
