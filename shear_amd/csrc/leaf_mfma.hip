// leaf_mfma.hip -- SQ8 leaf all-pairs filter on gfx950 int8 MFMA (the
// first of the two kernels of the leaf operator; leaf_select.hip is the
// second).
//
// Reference role: the WMMA leaf filter of gpu_persistent_subtree_topk_only
// (compute_backend.rs:10389-10950 tile evaluation, :11841-12295 drain); the
// operator's result must equal RowTopK insertion over the columns in member
// order (leaf_build.rs:887-957 with dco_sq_int8.rs:2950-2965 distances).
//
// Work item = (leaf, block of 256 member rows); a workgroup is 8 waves (one
// workgroup per CU, two waves per SIMD), wave w owns 32 rows of the block.
// The wave keeps its 32 rows' codes in VGPRs for the whole K range as the
// MFMA "B" operand (N = rows); 32-candidate column tiles are staged in LDS
// as the "A" operand (M = candidates) and shared by the 8 waves.  With
// v_mfma_i32_32x32x32_i8 output lane l holds row l%32 and candidates
// 8*(v/4) + 4*(l/32) + v%4 of the tile: each row is served by a lane pair
// (l, l+32), each lane seeing half of the row's candidates.  The grid is
// persistent (one workgroup per CU); the 8 XCDs each work through a
// contiguous range of work items, so a leaf's items share one L2.
//
// The column tiles of a block form one stream (phase A's sampled tiles, then
// every tile for phase B), double buffered in LDS with one barrier per tile;
// each tile's epilogue runs interleaved with the next tile's MFMAs.
//
//  * phase A: every 3rd (4th for wide leaves) column tile is evaluated and
//    each lane keeps its 16 smallest of the minima of adjacent candidate
//    pairs, ranked by cn - 2*rs*cs*dot (the distance less the row's norm, up
//    to rounding); the row threshold F is the pair's 24th (18th) smallest
//    kept value plus rn and 3*eps.  F only steers the filter: whatever its
//    value, the select kernel certifies each row against it and re-runs the
//    rows it cannot certify;
//  * phase B: every column tile; a candidate passes a bound on cs*dot and its
//    column's norm derived from F (a necessary condition for d <= F, with a
//    rounding margin; filter_bound) and is appended (raw dot, column) to the
//    row's survivor log in global memory (log_capacity entries per lane, the
//    pair's entries interleaved);
//  * end of item: F and both lanes' entry counts go to the row's row_meta
//    words.  The select kernel folds the two logs, certifies the row and
//    writes it, or queues it for the chain replay or the exact re-run; every
//    candidate it does not see lies above F.
#include <type_traits>
#include <utility>

#include "kernel_attr.h"
#include "leaf_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#ifndef TESSA_LEAF_WAVES
#define TESSA_LEAF_WAVES 8
#endif
constexpr int kWaves = TESSA_LEAF_WAVES;  // waves per workgroup, 32 rows each
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerBlock = kWaves * 32;
constexpr int kTileCols = 32;
constexpr uint32_t kMaxLeafRows = 4096;
constexpr float kFilterMargin = 3.0f * kTieEps;
// Phase A samples every kSampleStride-th column tile; F is the pair's
// kSampleRank-th smallest sampled distance plus the margin.  Every third
// tile with rank 24 leaves ~72 survivors per 1024-row leaf row (C2 data).
// Leaves of at least kSampleWideTiles column tiles sample every
// kSampleStrideWide-th tile with rank kSampleRankWide instead (a quarter of
// a 1024-row leaf is still 256 candidates per row): fewer sampled tiles, a
// few more rows sent to the exact kernel (~6 in 100,000 on C2 data).
#ifndef TESSA_LEAF_SAMPLE_STRIDE
#define TESSA_LEAF_SAMPLE_STRIDE 3
#endif
#ifndef TESSA_LEAF_SAMPLE_RANK
#define TESSA_LEAF_SAMPLE_RANK 24
#endif
#ifndef TESSA_LEAF_SAMPLE_WIDE_TILES
#define TESSA_LEAF_SAMPLE_WIDE_TILES 32
#endif
// Survivor-log drain steps run inside each phase B MFMA block (the rest of
// a lane's bits are drained by a loop at the next position's start).
#ifndef TESSA_LEAF_DRAIN_STEPS
#define TESSA_LEAF_DRAIN_STEPS 3
#endif
constexpr uint32_t kSampleStride = TESSA_LEAF_SAMPLE_STRIDE;
constexpr int kSampleRank = TESSA_LEAF_SAMPLE_RANK;
constexpr uint32_t kSampleWideTiles = TESSA_LEAF_SAMPLE_WIDE_TILES;
#ifndef TESSA_LEAF_SAMPLE_STRIDE_WIDE
#define TESSA_LEAF_SAMPLE_STRIDE_WIDE 4
#endif
#ifndef TESSA_LEAF_SAMPLE_RANK_WIDE
#define TESSA_LEAF_SAMPLE_RANK_WIDE 18
#endif
constexpr uint32_t kSampleStrideWide = TESSA_LEAF_SAMPLE_STRIDE_WIDE;
constexpr int kSampleRankWide = TESSA_LEAF_SAMPLE_RANK_WIDE;

template <int KS>
struct Layout {
    static constexpr int kTileStride = KS * 32 + 16;  // bytes per LDS tile row (16 B pad: no bank aliasing)
    static constexpr int kTileBytes = kTileCols * kTileStride;
    static constexpr int kChunks = kTileCols * KS * 2;            // 16-byte chunks per tile
    static constexpr int kChunksPerThread = (kChunks + kThreads - 1) / kThreads;
};

// Dynamic LDS limit (the whole CU).  One 8-wave workgroup per CU gives two
// waves per SIMD (256 VGPRs each); its 256 rows share every LDS column tile,
// so a leaf's tiles cross L2 -> LDS n/256 times.
#ifndef TESSA_LEAF_MIN_BLOCKS
#define TESSA_LEAF_MIN_BLOCKS 1
#endif
constexpr uint32_t kLdsBudget = 160u * 1024u;

// LDS: two column tiles and each wave's 4 KB accumulator scratch, then the
// leaf's member ids, scales and norms, and 128 bytes of scalars (each wave's
// norm range, the workgroup's next item).
__host__ __device__ constexpr uint32_t union_bytes(uint32_t tile_bytes, uint32_t nbuf) {
    return nbuf * tile_bytes + kWaves * 16u * 64u * 4u;
}
__host__ __device__ constexpr uint32_t lds_bytes(uint32_t tile_bytes, uint32_t nbuf, uint32_t cols_cap) {
    return union_bytes(tile_bytes, nbuf) + cols_cap * 12u + 128u;
}

// Compile-time loops: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, B + I>{}), ...);
}
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (E > B) static_for_impl<B>(f, std::make_integer_sequence<int, E - B>{});
}

// One column tile's MFMAs (A = the tile row read from LDS at `arow`, B = the
// row codes) with an epilogue spread over the k-steps: step s runs epilogue
// units [s*kUnits/KS, (s+1)*kUnits/KS) after its MFMA.  The units belong to
// the previous position and do not depend on these MFMAs, so they issue
// while the matrix pipe runs.  A operands are read two steps ahead; a
// scheduling fence after each step keeps this order (the default schedule
// puts every LDS read first and the whole epilogue after the last MFMA).
template <int KS, int kUnits, typename Epi>
__device__ __forceinline__ v16i mfma_block(const int8_t *arow, const v4i (&bfrag)[KS], Epi &&epi) {
    v16i acc = {};
    v4i ring[3];
    ring[0] = *reinterpret_cast<const v4i *>(arow);
    if constexpr (KS > 1) ring[1] = *reinterpret_cast<const v4i *>(arow + 32);
    static_for<0, KS>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        if constexpr (s + 2 < KS) ring[(s + 2) % 3] = *reinterpret_cast<const v4i *>(arow + 32 * (s + 2));
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ring[s % 3], bfrag[s], acc, 0, 0, 0);
        static_for<s * kUnits / KS, (s + 1) * kUnits / KS>(epi);
        __builtin_amdgcn_sched_barrier(0);
    });
    return acc;
}

// Compare-exchange c of a bitonic merge stage over 16 values (8 per stage,
// distance j): the (c%8)-th index i with i&j == 0 pairs with i+j.
__host__ __device__ constexpr int ce_low(int c, int jj) {
    return ((c % 8) / jj) * 2 * jj + (c % 8) % jj;
}
// Compare-exchange number c (0..23) of the bitonic sort of 8 values: stage
// c/4 of (k, j) = (2,1) (4,2) (4,1) (8,4) (8,2) (8,1); within a stage the
// (c%4)-th index i with i&j == 0 pairs with i+j.
__host__ __device__ constexpr int sort8_k(int c) { return c < 4 ? 2 : c < 12 ? 4 : 8; }
__host__ __device__ constexpr int sort8_j(int c) {
    return c < 4 ? 1 : c < 12 ? (2 >> ((c - 4) / 4)) : (4 >> ((c - 12) / 4));
}
__host__ __device__ constexpr int ce_low8(int c, int jj) { return ((c % 4) / jj) * 2 * jj + (c % 4) % jj; }

// x unchanged, but opaque to the optimizer: conditions derived from it are
// evaluated where they are used, inside the work-item loop, instead of being
// hoisted out of it as loop invariants (every hoisted lane mask would hold two
// scalar registers for the kernel's lifetime and spill).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t x) {
    asm volatile("" : "+s"(x));
    return x;
}

// Barrier for LDS hand-offs only: waits for this wave's LDS operations, not
// for its global loads and stores (prefetches stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Necessary condition for a candidate to pass d <= F, per column: d <= F
// implies cs*dot >= (rn - F)/(2 rs) + cn/(2 rs) - err, so the filter passes a
// candidate when t = fma(cn, B, fma(-cs, dot, A)) < 0 with B = 1/(2 rs) and A
// below (rn - F)/(2 rs) by a margin (1e-5 of the terms' scale) that covers
// the f32 roundings of d, of B and of t.  F = +inf (or a row scale that is
// not positive) passes everything; A = +inf passes nothing.
// With the leaf's smallest norm in place of cn the bound needs no per-column
// term: d <= F implies 2*rs*cs*dot >= rn + cn - F - err >= rn + cn_min - F -
// err, with err covering the f32 roundings of d (computed in double, lowered),
// so a candidate passes when fma(-cs, dot, A) < 0.  The per-column bound
// below is tighter when the leaf's norms differ (unnormalised data).
__device__ __forceinline__ void filter_bound_leaf(float F, float rs, float rn, float cn_min, float cn_max,
                                                  float &A) {
    if (!(F < __builtin_inff()) || !(rs > 0.0f)) {
        A = -__builtin_inff();
        return;
    }
    const double err = 1.0e-6 * ((double)fabsf(rn) + (double)cn_max + (double)F) + 1.0e-30;
    const double tau = ((double)rn + (double)cn_min - (double)F - err) / (2.0 * (double)rs);
    A = (float)(tau - fabs(tau) * 2.0e-6 - 1.0e-30);
}
__device__ __forceinline__ void filter_bound(float F, float rs, float rn, float cn_max, float &A, float &B) {
    if (!(F < __builtin_inff()) || !(rs > 0.0f)) {
        A = -__builtin_inff();
        B = 0.0f;
        return;
    }
    const double s2 = 2.0 * (double)rs;
    const double scale = ((double)fabsf(rn) + (double)cn_max + fabs((double)F)) / s2;
    A = (float)(((double)rn - (double)F) / s2 - 1.0e-5 * scale - 1.0e-30);
    B = (float)(1.0 / s2);
}


// Values-only compare-exchange (ascending).
__device__ __forceinline__ void cexv(float &a, float &b) {
    const float lo = fminf(a, b), hi = fmaxf(a, b);
    a = lo;
    b = hi;
}

template <int N>
__device__ __forceinline__ void bitonic_sort_v(float (&v)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    if ((i & k) == 0) cexv(v[i], v[l]);
                    else cexv(v[l], v[i]);
                }
            }
        }
    }
}

template <int N>
__device__ __forceinline__ void bitonic_merge_v(float (&v)[N]) {
#pragma unroll
    for (int j = N >> 1; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int l = i ^ j;
            if (l > i) cexv(v[i], v[l]);
        }
    }
}

// rsel-th smallest (1-based, rsel <= 2N) of the union of this lane's and its
// partner's ascending N-lists: ascending ++ descending is bitonic, one merge
// sorts it, and a static select picks the element.
template <int N>
__device__ __forceinline__ float pair_kth(const float (&a)[N], int rsel) {
    float m[2 * N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        m[i] = a[i];
        m[2 * N - 1 - i] = __shfl_xor(a[i], 32);
    }
    bitonic_merge_v<2 * N>(m);
    float res = __builtin_inff();
#pragma unroll
    for (int i = 0; i < 2 * N; ++i) res = (i == rsel - 1) ? m[i] : res;
    return res;
}

// NB column-tile buffers in LDS (2 or 4); a barrier every NB/2 positions.
template <int KS, int NB>
__global__ __launch_bounds__(kThreads, TESSA_LEAF_MIN_BLOCKS) void leaf_mfma_kernel(LeafParams p) {
    using L = Layout<KS>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // Runtime layout: tiles x2 | scratch | members | scales | norms | misc.
    const uint32_t cols_cap = (p.max_leaf_rows + 31u) & ~31u;
    int8_t *tile = reinterpret_cast<int8_t *>(smem);
    uint32_t *mem_lds = reinterpret_cast<uint32_t *>(smem + union_bytes(L::kTileBytes, NB));
    float *cs_lds = reinterpret_cast<float *>(mem_lds + cols_cap);
    float *cn_lds = cs_lds + cols_cap;
    uint32_t *misc = reinterpret_cast<uint32_t *>(cn_lds + cols_cap);

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t j = lane & 31u;
    const uint32_t h = lane >> 5;
    const uint32_t cap = p.log_capacity;

    // Work items are (leaf, 256-row block).  Workgroups are dispatched
    // round-robin over the 8 XCDs: XCD x walks its own contiguous item range,
    // so the row blocks of a leaf run at the same time on one XCD and share
    // its L2 for the leaf's column tiles.  The grid is one workgroup per CU;
    // a workgroup's first item is fixed (its rank on the XCD), the rest come
    // from the XCD's ticket counter (ragged leaves balance themselves).  The
    // ticket for the next item is taken as an item starts and published to
    // the workgroup through LDS at the item's second barrier, so its latency
    // is hidden behind the item's first loads.
    const uint32_t total = *p.item_total;
    const uint32_t items = total > p.item_begin ? (total - p.item_begin < p.item_count ? total - p.item_begin
                                                                                      : p.item_count)
                                                : 0u;
    const uint32_t per_xcd = (items + 7u) / 8u;
    const uint32_t xcd = blockIdx.x % 8u;
    const uint32_t lane_in_xcd = blockIdx.x / 8u;
    const uint32_t wgs_per_xcd = gridDim.x / 8u;
    uint32_t s_surv = 0, s_tiles = 0;
    uint32_t *const s_next = misc + 2 * kWaves;  // the next item, from thread 0
    uint32_t it = lane_in_xcd, it_next = per_xcd;

    while (it < per_xcd) {
        const uint32_t work = xcd * per_xcd + it;  // item of the batch
        if (work >= items) break;
        uint32_t ticket = 0u;
        if (tid == 0) ticket = wgs_per_xcd + atomicAdd(p.item_tickets + xcd, 1u);
        const uint2 li = p.item_list[p.item_begin + work];
        const uint32_t leaf = li.x;
        const uint32_t blk = li.y;
        // The row's two lanes share one log region of 2*cap entries: lane h
        // writes its e-th entry at 2e + h, so the select kernel reads a row's
        // entries as one contiguous run.
        const uint32_t brow = wave * 32u + j;  // row within the block
        uint2 *slog = p.survivor_log + ((uint64_t)work * kRowsPerBlock + brow) * 2u * cap + h;
        const uint32_t n = p.member_counts[leaf];
        const uint32_t row_base = blk * kRowsPerBlock;
        // an item without rows (or an oversized leaf) only passes its ticket
        // on; the first barrier orders the write after every read of the
        // previous value
        if (row_base >= n || n > p.max_leaf_rows || n > kMaxLeafRows) {
            if (tid == 0 && row_base < n) flag_overflow(p.counters, TESSA_OVF_LEAF_ROW);
            __syncthreads();
            if (tid == 0) *s_next = ticket;
            __syncthreads();
            it = *s_next;
            continue;
        }
        const uint32_t *mem = p.members + p.member_offsets[leaf];
        const uint32_t pd = opaque_u32(p.padded_dim);
        const uint32_t pk = opaque_u32(p.k);

        // The lane's row: its member id straight from the member list, and its
        // codes (the B operand, zero past padded_dim) requested before the
        // staging below, so both sets of loads are in flight together.
        const uint32_t r = row_base + wave * 32u + j;  // leaf-local row position
        const bool row_ok = r < n;
        uint32_t mr = row_ok ? mem[r] : 0u;
        mr = mr < p.rows ? mr : 0u;  // the staging flags an invalid id
        const uint32_t keff = n > 1u ? ((pk < n - 1u) ? pk : (n - 1u)) : 0u;
        v4i bfrag[KS];
        {
            const int8_t *rc = p.codes + (uint64_t)mr * pd;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const uint32_t off = 32u * s + 16u * h;
                const bool ok = row_ok && off < pd;
                const v4i z = *reinterpret_cast<const v4i *>(rc + (ok ? off : 0u));
                const v4i zero = {0, 0, 0, 0};
                bfrag[s] = ok ? z : zero;
            }
        }

        // previous item's readers of the LDS arrays are done; an LDS-only
        // barrier, so the row codes above stay in flight through the staging
        lds_barrier();
        {
            // four columns per thread per step (a 2,048-row leaf in one step),
            // every load of a step issued before its results are used
            float lo = __builtin_inff(), hi = 0.0f;
            for (uint32_t c0 = tid; c0 < n; c0 += 4u * kThreads) {
                uint32_t m[4];
                bool bad = false;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t c = c0 + (uint32_t)i * kThreads;
                    m[i] = mem[c < n ? c : c0];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bad |= m[i] >= p.rows;
                    m[i] = m[i] < p.rows ? m[i] : 0u;
                }
                if (bad) flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_COL_ID);
                float sv[4], nv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sv[i] = p.scales[m[i]];
                    nv[i] = p.norms[m[i]];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t c = c0 + (uint32_t)i * kThreads;
                    if (c < n) {
                        mem_lds[c] = m[i];
                        cs_lds[c] = sv[i];
                        cn_lds[c] = nv[i];
                        lo = fminf(lo, nv[i]);
                        hi = fmaxf(hi, nv[i]);
                    }
                }
            }
            // the last column tile's columns past n: zero scale, infinite norm
            // (their codes are zero, so their sampled distance is +inf)
            for (uint32_t c = n + tid; c < ((n + 31u) & ~31u); c += kThreads) {
                cs_lds[c] = 0.0f;
                cn_lds[c] = __builtin_inff();
            }
            // per-wave norm range into misc; combined after the barrier
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                lo = fminf(lo, __shfl_xor(lo, off));
                hi = fmaxf(hi, __shfl_xor(hi, off));
            }
            if (lane == 0u) {
                misc[2u * wave] = __float_as_uint(lo);
                misc[2u * wave + 1u] = __float_as_uint(hi);
            }
        }
        if (tid == 0) *s_next = ticket;
        lds_barrier();
        it_next = *s_next;
        float cn_min = __uint_as_float(misc[0]), cn_max = __uint_as_float(misc[1]);
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            cn_min = fminf(cn_min, __uint_as_float(misc[2 * w]));
            cn_max = fmaxf(cn_max, __uint_as_float(misc[2 * w + 1]));
        }
        // the per-column test when the leaf's norms differ by more than 1 %
        // (unnormalised data); else the cheaper leaf-wide one
        const bool per_column = __fsub_rn(cn_max, cn_min) > 0.01f * cn_max;

        const float rs = row_ok ? cs_lds[r] : 1.0f;
        const float rn = row_ok ? cn_lds[r] : 0.0f;
        const float rs_m2 = -2.0f * rs;

        const uint32_t ntiles = (n + kTileCols - 1) / kTileCols;
        v4i pre[L::kChunksPerThread];

        // Tile loads are branch-free and split in two: prep_tile reads the
        // member ids of a tile's chunks from LDS (it runs as a unit of the
        // previous MFMA block, so its LDS wait is hidden there), issue_tile
        // starts the global loads.  A chunk past the tile, the leaf or the
        // padded row loads from a valid address (member 0, offset 0) and is
        // zeroed when stored to LDS, a position later, so nothing waits for
        // the loads when they are issued.
        uint32_t pre_ok = 0u;  // bit q: chunk q of `pre` is real data
        // a tile inside the leaf, rows without padding: every chunk is real
        // data (a uniform flag, so stores of such tiles skip the selects)
        const bool pd_full = pd == (uint32_t)(KS * 32);
        bool nx_full = false, pre_full = false;
        uint32_t nx_mc[L::kChunksPerThread];
        uint32_t nx_ok = 0u;
        auto chunk_off = [&](int q) { return ((tid + q * kThreads) % (KS * 2)) * 16u; };
        auto prep_tile = [&](uint32_t t) {
            nx_full = ((t + 1u) * kTileCols <= n) & pd_full;
            nx_ok = 0u;
#pragma unroll
            for (int q = 0; q < L::kChunksPerThread; ++q) {
                const uint32_t chunk = tid + q * kThreads;
                const uint32_t c = t * kTileCols + chunk / (KS * 2);
                const bool ok = (chunk < (uint32_t)L::kChunks) & (c < n) & (chunk_off(q) < pd);
                nx_ok |= ok ? (1u << q) : 0u;
                nx_mc[q] = mem_lds[ok ? c : 0u];
            }
        };
        auto issue_to = [&](v4i (&dst)[L::kChunksPerThread]) {
#pragma unroll
            for (int q = 0; q < L::kChunksPerThread; ++q) {
                const uint32_t off = ((nx_ok >> q) & 1u) ? chunk_off(q) : 0u;
                dst[q] = *reinterpret_cast<const v4i *>(p.codes + (uint64_t)nx_mc[q] * pd + off);
            }
        };
        auto issue_tile = [&]() {
            pre_full = nx_full;
            pre_ok = nx_ok;
            issue_to(pre);
        };
        auto store_from = [&](const v4i (&src)[L::kChunksPerThread], bool full, uint32_t ok, int8_t *dst) {
            if (full) {  // every chunk is real data: no selects
#pragma unroll
                for (int q = 0; q < L::kChunksPerThread; ++q) {
                    const uint32_t chunk = tid + q * kThreads;
                    if (chunk < (uint32_t)L::kChunks) {
                        const uint32_t row = chunk / (KS * 2);
                        const uint32_t off = (chunk % (KS * 2)) * 16u;
                        *reinterpret_cast<v4i *>(dst + row * L::kTileStride + off) = src[q];
                    }
                }
                return;
            }
#pragma unroll
            for (int q = 0; q < L::kChunksPerThread; ++q) {
                const uint32_t chunk = tid + q * kThreads;
                if (chunk < (uint32_t)L::kChunks) {
                    const uint32_t row = chunk / (KS * 2);
                    const uint32_t off = (chunk % (KS * 2)) * 16u;
                    const v4i zero = {0, 0, 0, 0};
                    *reinterpret_cast<v4i *>(dst + row * L::kTileStride + off) = ((ok >> q) & 1u) ? src[q] : zero;
                }
            }
        };
        auto store_tile = [&](int8_t *dst) { store_from(pre, pre_full, pre_ok, dst); };

        // ---- the tile stream ----------------------------------------------------
        // Stream position i < nA is phase A's sampled tile i*sstride,
        // position nA + t is phase B's tile t.  Column tiles are double
        // buffered in LDS with one barrier per position: position i's MFMAs
        // read buffer i&1 while the tile of position i+1 goes to the other
        // buffer and position i+2's codes are in flight in registers.  The
        // epilogue of position i-1 (its accumulators held over) runs in the
        // same straight-line block as position i's MFMAs, so the VALU work
        // overlaps the matrix pipe.
        //  * phase A epilogue: of each sampled tile a lane takes the minimum of
        //    each adjacent pair of its 16 ranking values (cn - 2*rs*cs*dot)
        //    and keeps the 16 smallest of those minima (values only); F is the
        //    pair's kSel-th smallest kept value plus rn and 3 eps;
        //  * phase B epilogue: a 16-bit mask of the lane's candidates that
        //    pass filter_bound's test, and the raw dots parked in the wave's
        //    LDS scratch;
        //    the next position drains the mask (set bits only) into the lane's
        //    survivor log.  Column validity (c < n, c != r) is checked there.
        constexpr int kSample = 16;
        const bool wide = ntiles >= kSampleWideTiles;
        const uint32_t sstride = wide ? kSampleStrideWide : kSampleStride;
        const uint32_t srank = wide ? (uint32_t)kSampleRankWide : (uint32_t)kSampleRank;
        const int rsel = (int)(keff < srank ? keff : srank);
        float samp[kSample];
#pragma unroll
        for (int i = 0; i < kSample; ++i) samp[i] = __builtin_inff();
        float F = -__builtin_inff();
        float tauA = __builtin_inff(), tauB = 0.0f;
        const uint32_t nA = (ntiles + sstride - 1u) / sstride;
        const uint32_t S = nA + ntiles;
        auto tile_of = [&](uint32_t i) { return i < nA ? i * sstride : i - nA; };
        constexpr uint32_t kAhead = NB / 2;  // positions between a tile's store and its use
        int *const scr = reinterpret_cast<int *>(tile + NB * L::kTileBytes) + wave * (16u * 64u);

        // Phase A epilogue units (92): per group of 4 candidates one LDS read
        // of their scales and norms and 4 ranking values (20), 8 pair
        // minima, the 24 compare-exchanges of their bitonic sort, 8 minima
        // against the kept samples and the 32 of their bitonic merge.
        constexpr int kSampleUnits = 20 + 8 + 24 + 8 + 32;
        float4 ep_cs[4], ep_cn[4];
        // scale and norm arrays start 16-byte aligned; each group of 4 is a float4
        const float *cs_al = static_cast<const float *>(__builtin_assume_aligned(cs_lds, 16));
        const float *cn_al = static_cast<const float *>(__builtin_assume_aligned(cn_lds, 16));
        float ep_v[16];
        const v16i *ep_acc = nullptr;
        uint32_t ep_cbase = 0u;
        // Columns past n carry norm +inf (distance +inf); the row's own column
        // lies in the wave's diagonal tile only, whose epilogue variant
        // (kDiag) excludes it.  Rows past n get samples but pass nothing.
        auto sample_unit_impl = [&](auto wc, auto diag_tag) {
            constexpr int W = decltype(wc)::value;
            constexpr bool kDiag = decltype(diag_tag)::value;
            if constexpr (W < 20) {
                constexpr int q = W / 5, u = W % 5;
                if constexpr (u == 0) {
                    ep_cs[q] = *reinterpret_cast<const float4 *>(cs_al + ep_cbase + 8 * q + 4 * h);
                    ep_cn[q] = *reinterpret_cast<const float4 *>(cn_al + ep_cbase + 8 * q + 4 * h);
                } else {
                    constexpr int e = u - 1, vi = 4 * q + e;
                    const float csv = e == 0 ? ep_cs[q].x : e == 1 ? ep_cs[q].y : e == 2 ? ep_cs[q].z : ep_cs[q].w;
                    const float cnv = e == 0 ? ep_cn[q].x : e == 1 ? ep_cn[q].y : e == 2 ? ep_cn[q].z : ep_cn[q].w;
                    const float d = __builtin_fmaf(rs_m2, __fmul_rn(csv, (float)(*ep_acc)[vi]), cnv);
                    if constexpr (kDiag) {
                        const uint32_t c = ep_cbase + 4u * h + (uint32_t)(8 * q + e);
                        ep_v[vi] = c != r ? d : __builtin_inff();
                    } else {
                        ep_v[vi] = d;
                    }
                }
            } else if constexpr (W < 28) {
                constexpr int i = W - 20;  // pair minima, in place (ep_v[2i], ep_v[2i+1] are still unread)
                ep_v[i] = fminf(ep_v[2 * i], ep_v[2 * i + 1]);
            } else if constexpr (W < 52) {
                constexpr int c = W - 28, k = sort8_k(c), jj = sort8_j(c), lo = ce_low8(c, jj);
                if constexpr ((lo & k) == 0) cexv(ep_v[lo], ep_v[lo + jj]);
                else cexv(ep_v[lo + jj], ep_v[lo]);
            } else if constexpr (W < 60) {
                // the kept 16 against the 8 sorted minima followed by 8 x +inf,
                // reversed: the upper half takes min(samp[8+i], min[7-i]) and the
                // whole is bitonic with the 16 smallest of both
                constexpr int i = W - 52;
                samp[8 + i] = fminf(samp[8 + i], ep_v[7 - i]);
            } else {
                constexpr int c = W - 60, jj = 8 >> (c / 8), lo = ce_low(c, jj);
                cexv(samp[lo], samp[lo + jj]);
            }
        };
        auto sample_unit = [&](auto wc) { sample_unit_impl(wc, std::false_type{}); };
        auto sample_unit_diag = [&](auto wc) { sample_unit_impl(wc, std::true_type{}); };
        const uint32_t diag_tile = (row_base + wave * 32u) / kTileCols;
        // Phase B epilogue units (24): per group of 4 candidates (groups
        // taken from 3 down to 0) one LDS read of their scales, 4 filter
        // tests, one LDS write of the raw dots.
        // The mask block adds kDrainSteps drain steps (each takes the lane's
        // lowest set bit: an LDS read of its dot, then a store to the survivor
        // log through a buffer store whose offset is out of range, so dropped,
        // for lanes with nothing to store) and the next tile's prep.  Bits left
        // after them are drained by the loop at the next position's start.
        constexpr int kMaskUnits = 24;
        constexpr int kDrainSteps = TESSA_LEAF_DRAIN_STEPS;
        constexpr int kMaskBlockUnits = kMaskUnits + 2 * kDrainSteps + 1;
        uint32_t ep_m = 0u;
        uint32_t prep_t = 0u;
        int dr_dot[kDrainSteps > 0 ? kDrainSteps : 1];
        uint32_t dr_c[kDrainSteps > 0 ? kDrainSteps : 1];
        uint32_t dr_has = 0u;
        uint32_t cnt = 0;
        // survivor log as a buffer: this thread's entries start at slog_off bytes
        const __amdgpu_buffer_rsrc_t log_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            p.survivor_log, (short)0, (int)(p.item_count * (uint32_t)kThreads * cap * 8u), 0x00020000);
        const uint32_t slog_off = ((work * (uint32_t)kRowsPerBlock + brow) * 2u * cap + h) * 8u;
        auto mask_unit_impl = [&](auto wc, auto pc_tag) {
            constexpr int W = decltype(wc)::value, G = 3 - W / 6, u = W % 6;
            constexpr bool kPC = decltype(pc_tag)::value;
            if constexpr (W >= kMaskUnits + 2 * kDrainSteps) {
                prep_tile(prep_t);
            } else if constexpr (W >= kMaskUnits + kDrainSteps) {
                constexpr int d = W - kMaskUnits - kDrainSteps;
                const bool ok = ((dr_has >> d) & 1u) & (dr_c[d] < n) & (dr_c[d] != r);
                const uint32_t off = (ok & (cnt < cap)) ? slog_off + cnt * 16u : 0x80000000u;
                const int2 rec = make_int2(dr_dot[d], (int)dr_c[d]);
                __builtin_amdgcn_raw_buffer_store_b64(*reinterpret_cast<const v2i *>(&rec), log_rsrc, off, 0, 0);
                cnt += ok ? 1u : 0u;
            } else if constexpr (W >= kMaskUnits) {
                constexpr int d = W - kMaskUnits;
                const uint32_t m = ep_m;
                const uint32_t vi = m != 0u ? (uint32_t)__builtin_ctz(m) : 0u;
                dr_has |= (m != 0u) ? (1u << d) : 0u;
                ep_m = m & (m - 1u);
                dr_c[d] = ep_cbase + 4u * h + 8u * (vi >> 2) + (vi & 3u);
                dr_dot[d] = scr[((vi >> 2) * 64u + lane) * 4u + (vi & 3u)];
            } else if constexpr (u == 0) {
                ep_cs[G] = *reinterpret_cast<const float4 *>(cs_al + ep_cbase + 8 * G + 4 * h);
                if constexpr (kPC) ep_cn[G] = *reinterpret_cast<const float4 *>(cn_al + ep_cbase + 8 * G + 4 * h);
            } else if constexpr (u < 5) {
                // t < 0 is the filter test (filter_bound / filter_bound_leaf),
                // t rounded once per FMA; its sign bit is shifted into the
                // mask, so the candidates taken from 15 down to 0 land on bits
                // 15..0
                constexpr int e = 4 - u, vi = 4 * G + e;
                const float csv = e == 0 ? ep_cs[G].x : e == 1 ? ep_cs[G].y : e == 2 ? ep_cs[G].z : ep_cs[G].w;
                float t = __builtin_fmaf(-csv, (float)(*ep_acc)[vi], tauA);
                if constexpr (kPC) {
                    const float cnv = e == 0 ? ep_cn[G].x : e == 1 ? ep_cn[G].y : e == 2 ? ep_cn[G].z : ep_cn[G].w;
                    t = __builtin_fmaf(cnv, tauB, t);
                }
                ep_m = __builtin_amdgcn_alignbit(ep_m, __float_as_uint(t), 31u);
            } else {
                const v4i d = {(*ep_acc)[4 * G], (*ep_acc)[4 * G + 1], (*ep_acc)[4 * G + 2], (*ep_acc)[4 * G + 3]};
                *reinterpret_cast<v4i *>(scr + (G * 64 + lane) * 4) = d;
            }
        };
        auto mask_unit = [&](auto wc) { mask_unit_impl(wc, std::false_type{}); };
        auto mask_unit_pc = [&](auto wc) { mask_unit_impl(wc, std::true_type{}); };
        auto prep_unit = [&](auto) { prep_tile(prep_t); };
        auto sample_prep_unit = [&](auto wc) {
            if constexpr (decltype(wc)::value == kSampleUnits) prep_tile(prep_t);
            else sample_unit(wc);
        };
        auto sample_prep_unit_diag = [&](auto wc) {
            if constexpr (decltype(wc)::value == kSampleUnits) prep_tile(prep_t);
            else sample_unit_diag(wc);
        };
        const uint32_t arow_off = j * L::kTileStride + 16u * h;
        auto drain = [&](uint32_t m, uint32_t tp) {
            const uint32_t cbase = tp * kTileCols + 4u * h;
            while (m != 0u) {
                const uint32_t vi = (uint32_t)__builtin_ctz(m);
                m &= m - 1u;
                const uint32_t c = cbase + 8u * (vi >> 2) + (vi & 3u);
                const int dot = scr[((vi >> 2) * 64u + lane) * 4u + (vi & 3u)];
                const bool ok = (c < n) & (c != r);
                if (ok & (cnt < cap)) slog[2u * cnt] = make_uint2((uint32_t)dot, c);
                cnt += ok ? 1u : 0u;
            }
        };

        uint32_t pend_mask = 0u, pend_tile = 0u;
        // Position i reads buffer i % NB.  Start of position i: a barrier
        // when i % (NB/2) == 0, the tile of position i + NB/2 from registers
        // to its buffer, the held mask's drain, then the prefetch of position
        // i + NB/2 + 1.  A tile stored at position j is read at j + NB/2,
        // after the next barrier; the buffer it overwrites was last read at
        // j - NB/2, before the barrier every wave has passed.
        auto bufp = [&](uint32_t i) -> int8_t * { return tile + (i % NB) * L::kTileBytes; };
        auto head = [&](uint32_t i) {
            if (i % kAhead == 0u) lds_barrier();
            if (i + kAhead < S) store_tile(bufp(i + kAhead));
            drain(pend_mask, pend_tile);
            pend_mask = 0u;
            if (i + kAhead + 1u < S) issue_tile();  // prepared by the previous block
        };
        auto src_of = [&](uint32_t i) -> const int8_t * { return bufp(i); };

        // prologue: positions 0 .. NB/2-1 in their LDS buffers, position
        // NB/2 in registers, the ids of position NB/2 + 1 prepared (S >= 2:
        // nA >= 1 and ntiles >= 1)
        if constexpr (kAhead == 2u) {
            // both buffered tiles' loads in flight together: one round trip
            // before the first MFMA instead of two
            v4i pre0[L::kChunksPerThread];
            prep_tile(tile_of(0));
            const bool full0 = nx_full;
            const uint32_t ok0 = nx_ok;
            issue_to(pre0);
            prep_tile(tile_of(1));
            issue_tile();
            store_from(pre0, full0, ok0, bufp(0));
            store_tile(bufp(1));
        } else {
            for (uint32_t t0 = 0; t0 < kAhead && t0 < S; ++t0) {
                prep_tile(tile_of(t0));
                issue_tile();
                store_tile(bufp(t0));
            }
        }
        prep_tile(tile_of(kAhead < S ? kAhead : S - 1u));
        issue_tile();
        prep_tile(tile_of(kAhead + 1u < S ? kAhead + 1u : S - 1u));
        // each block prepares the ids of the tile NB/2 + 2 positions ahead
        auto prep_for = [&](uint32_t i) { prep_t = tile_of(i + kAhead + 2u < S ? i + kAhead + 2u : S - 1u); };
        // accP holds the accumulators of the latest position; each block
        // computes position i into accQ/accP alternately while the epilogue
        // of position i-1 runs on the other.
        v16i accP, accQ;
        auto sample_block = [&](uint32_t i, const v16i &prev) {
            ep_acc = &prev;
            const uint32_t tp = tile_of(i - 1u);
            ep_cbase = tp * kTileCols;
            prep_for(i);
            if (tp == diag_tile)
                return mfma_block<KS, kSampleUnits + 1>(src_of(i) + arow_off, bfrag, sample_prep_unit_diag);
            return mfma_block<KS, kSampleUnits + 1>(src_of(i) + arow_off, bfrag, sample_prep_unit);
        };
        auto mask_block = [&](uint32_t i, const v16i &prev, auto &unit) {
            ep_acc = &prev;
            ep_cbase = (i - 1u - nA) * kTileCols;
            ep_m = 0u;
            dr_has = 0u;
            prep_for(i);
            const v16i acc = mfma_block<KS, kMaskBlockUnits>(src_of(i) + arow_off, bfrag, unit);
            // the residual mask is needed here, not only by the next position's
            // drain: its tests stay interleaved with the MFMAs instead of sinking
            asm volatile("" : "+v"(ep_m));
            pend_mask = ep_m;
            pend_tile = i - 1u - nA;
            return acc;
        };
        head(0);
        prep_for(0);
        accP = mfma_block<KS, 1>(src_of(0) + arow_off, bfrag, prep_unit);
        uint32_t i = 1;
        // positions 1..nA: epilogues of the sampled tiles
        for (; i + 1u <= nA; i += 2u) {
            head(i);
            accQ = sample_block(i, accP);
            head(i + 1u);
            accP = sample_block(i + 1u, accQ);
        }
        if (i <= nA) {
            head(i);
            accQ = sample_block(i, accP);
            accP = accQ;
            ++i;
        }
        if (rsel > 0) F = __fadd_rn(__fadd_rn(pair_kth<kSample>(samp, rsel), rn), kFilterMargin);
        // the row's filter test (rows past n pass nothing)
        if (row_ok && F != -__builtin_inff()) {
            if (per_column) filter_bound(F, rs, rn, cn_max, tauA, tauB);
            else filter_bound_leaf(F, rs, rn, cn_min, cn_max, tauA);
        }
        // positions nA+1..S-1: filter epilogues of phase B tiles, then the
        // tail: drain the held mask, then the last position (phase B's last
        // tile); one copy of the loop per form of the test
        auto phase_b = [&](auto &unit) {
            for (; i + 1u < S; i += 2u) {
                head(i);
                accQ = mask_block(i, accP, unit);
                head(i + 1u);
                accP = mask_block(i + 1u, accQ, unit);
            }
            if (i < S) {
                head(i);
                accQ = mask_block(i, accP, unit);
                accP = accQ;
            }
            drain(pend_mask, pend_tile);
            ep_acc = &accP;
            ep_cbase = (ntiles - 1u) * kTileCols;
            ep_m = 0u;
            static_for<0, kMaskUnits>(unit);
            drain(ep_m, ntiles - 1u);
        };
        if (per_column) phase_b(mask_unit_pc);
        else phase_b(mask_unit);
        s_tiles += S;
        s_surv += cnt < cap ? cnt : cap;

        // ---- end of item: the row's threshold and each lane's entry count ----
        // (the select kernel folds the logs, certifies and writes the rows;
        // a count above the capacity marks a log that overflowed)
        if (row_ok) {
            uint32_t *rm = reinterpret_cast<uint32_t *>(p.row_meta + (uint64_t)work * kRowsPerBlock + brow);
            if (h == 0u) {
                rm[0] = __float_as_uint(F);
                rm[1] = cnt;
            } else {
                rm[2] = cnt;
            }
        }
        it = it_next;
    }

    // The last workgroup to finish (every other one has taken its final
    // ticket) resets the tickets for the next launch on the stream.
    if (tid == 0 && atomicAdd(p.item_tickets + 8, 1u) == gridDim.x - 1u) {
#pragma unroll
        for (int x = 0; x < 9; ++x) atomicExch(p.item_tickets + x, 0u);
    }

    // One atomic per counter per wave.
    uint64_t a_surv = s_surv;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) a_surv += __shfl_xor(a_surv, off);
    if (lane == 0) {
        counter_add(p.counters, TESSA_C_LEAF_SURVIVORS, a_surv);
        if (wave == 0) counter_add(p.counters, TESSA_C_LEAF_MFMA_TILES, s_tiles);
    }
}

// CUs of the current device (cached per device).
uint32_t cu_count() {
    static uint32_t cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256u;
    if (cached[dev] == 0u) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cached[dev] = (uint32_t)v;
    }
    return cached[dev];
}

template <int KS>
int launch_ks(const LeafParams &p, hipStream_t stream) {
    using L = Layout<KS>;
    if (ensure_lds_limit(reinterpret_cast<const void *>(leaf_mfma_kernel<KS, 2>), (int)kLdsBudget) ||
        ensure_lds_limit(reinterpret_cast<const void *>(leaf_mfma_kernel<KS, 4>), (int)kLdsBudget))
        return -1;
    const uint32_t cols_cap = (p.max_leaf_rows + 31u) & ~31u;
    // four tile buffers (a barrier every second position) when they fit
    const bool four = lds_bytes(L::kTileBytes, 4, cols_cap) <= kLdsBudget;
    const uint32_t lds = lds_bytes(L::kTileBytes, four ? 4 : 2, cols_cap);
    if (lds > kLdsBudget) return -4;
    if (p.item_count == 0) return 0;
    // a batch's log offsets stay below 2^31 (the out-of-range store marker)
    if ((uint64_t)p.item_count * kThreads * p.log_capacity * 8u > 0x80000000ull) return -2;
    // persistent grid: one workgroup per CU (a multiple of the 8 XCDs); with
    // the batch's listed items (count read on the device) split in 8 equal
    // ranges, XCD x works through range x
    const uint32_t per_xcd = (p.item_count + 7u) / 8u;
    uint32_t grid = cu_count() & ~7u;
    if (grid < 8u) grid = 8u;
    if (per_xcd * 8u < grid) grid = per_xcd * 8u;
    if (four)
        hipLaunchKernelGGL((leaf_mfma_kernel<KS, 4>), dim3(grid), dim3(kThreads), lds, stream, p);
    else
        hipLaunchKernelGGL((leaf_mfma_kernel<KS, 2>), dim3(grid), dim3(kThreads), lds, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int leaf_mfma_supported(uint32_t padded_dim, uint32_t max_leaf_rows) {
    return padded_dim > 0 && padded_dim <= 1024 && padded_dim % 16 == 0 && max_leaf_rows <= kMaxLeafRows;
}

int launch_leaf_mfma(const LeafParams &p, hipStream_t stream) {
    const uint32_t ks = (p.padded_dim + 31) / 32;
    if (ks <= 4) return launch_ks<4>(p, stream);
    if (ks <= 8) return launch_ks<8>(p, stream);
    if (ks <= 12) return launch_ks<12>(p, stream);
    if (ks <= 16) return launch_ks<16>(p, stream);
    if (ks <= 24) return launch_ks<24>(p, stream);
    if (ks <= 32) return launch_ks<32>(p, stream);
    return -3;
}

}  // namespace tessa
