// leaf_mfma.hip -- SQ8 leaf all-pairs + per-row top-k on gfx950 int8 MFMA.
//
// Reference role: the WMMA leaf filter of gpu_persistent_subtree_topk_only
// (compute_backend.rs:10389-10950 tile evaluation, :11841-12295 drain); the
// result must equal RowTopK insertion over the columns in member order
// (leaf_build.rs:887-957 with dco_sq_int8.rs:2950-2965 distances).
//
// Work item = (leaf, block of 128 member rows); a workgroup is 4 waves, wave w
// owns 32 rows.  The wave keeps its 32 rows' codes in VGPRs for the whole K
// range and is the MFMA "B" operand (N = rows); 32-candidate column tiles are
// staged in LDS and are the "A" operand (M = candidates).  With
// v_mfma_i32_32x32x32_i8 the output lane l holds row l%32 and the 16
// candidates 8*(v/4) + 4*(l/32) + v%4 of the tile, so each lane owns half of
// one row's candidates and walks them in increasing column order.
//
// Selection is exact by construction:
//  * each lane keeps every candidate with d <= F in a list (F is the running
//    threshold of the row, shared by its two lanes, never increasing);
//  * F is the larger of the two lanes' 16th-smallest distance seen so far, so
//    at least 32 >= k candidates of the row are <= F at all times;
//  * at the end, the row's listed candidates with d <= F are pushed in column
//    order through the reference insertion rule.  Let M be the largest kept
//    distance and theta the smallest value >= M with no candidate in
//    (theta, theta + 2e-5].  Every candidate <= theta is listed (theta <= F is
//    checked), every candidate above it is > theta + 2e-5 away from all of
//    them, and for such a split the bounded insertion over the whole row and
//    over the listed part give the same buffer (candidates more than eps
//    above every kept one can never enter in front of them or stay).  Rows
//    where the check fails, or whose list overflowed, are queued and re-run
//    by the exact scalar kernel.
#include "leaf_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerBlock = kWaves * 32;
constexpr int kTileCols = 32;
constexpr int kCap = 56;       // per-lane candidate list capacity
constexpr int kKeepPerLane = 16;
constexpr uint32_t kMaxLeafRows = 4096;

template <int KS>
struct Layout {
    static constexpr int kTileStride = KS * 32 + 16;                 // bytes per LDS tile row
    static constexpr int kTileBytes = kTileCols * kTileStride;
    // The tile area also stages the leaf's global ids for the final phase.
    static constexpr int kTileRegion =
        kTileBytes > (int)kMaxLeafRows * 4 ? kTileBytes : (int)kMaxLeafRows * 4;
    static constexpr int kMetaOff = kTileRegion;                     // scales[32], norms[32]
    static constexpr int kListDOff = kMetaOff + 2 * kTileCols * 4;
    static constexpr int kListCOff = kListDOff + (kCap + 1) * kThreads * 4;
    static constexpr int kFinDOff = kListCOff + (kCap + 1) * kThreads * 2;
    static constexpr int kFinGOff = kFinDOff + kMaxK * kRowsPerBlock * 4;
    static constexpr int kBytes = kFinGOff + kMaxK * kRowsPerBlock * 4;
    static constexpr int kChunks = kTileCols * KS * 2;               // 16-byte chunks per tile
    static constexpr int kChunksPerThread = (kChunks + kThreads - 1) / kThreads;
    static_assert(kBytes <= 160 * 1024, "LDS budget");
};

template <int N>
__device__ __forceinline__ void bitonic_sort(float (&v)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const float a = v[i], b = v[l];
                    const float lo = fminf(a, b), hi = fmaxf(a, b);
                    if ((i & k) == 0) { v[i] = lo; v[l] = hi; }
                    else { v[i] = hi; v[l] = lo; }
                }
            }
        }
    }
}

template <int N>
__device__ __forceinline__ void bitonic_merge(float (&v)[N]) {
#pragma unroll
    for (int j = N >> 1; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int l = i ^ j;
            if (l > i) {
                const float a = v[i], b = v[l];
                v[i] = fminf(a, b);
                v[l] = fmaxf(a, b);
            }
        }
    }
}

__device__ __forceinline__ int wave_max_i(int x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = max(x, __shfl_xor(x, off));
    return x;
}

template <int KS>
__global__ __launch_bounds__(kThreads, 1) void leaf_mfma_kernel(LeafParams p, uint32_t blocks_per_leaf,
                                                              uint32_t total_work, uint32_t padded_grid) {
    using L = Layout<KS>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    int8_t *tile = reinterpret_cast<int8_t *>(smem);
    float *meta_s = reinterpret_cast<float *>(smem + L::kMetaOff);
    float *meta_n = meta_s + kTileCols;
    float *list_d = reinterpret_cast<float *>(smem + L::kListDOff);
    uint16_t *list_c = reinterpret_cast<uint16_t *>(smem + L::kListCOff);
    float *fin_d = reinterpret_cast<float *>(smem + L::kFinDOff);
    uint32_t *fin_g = reinterpret_cast<uint32_t *>(smem + L::kFinGOff);
    uint32_t *gid_lds = reinterpret_cast<uint32_t *>(smem);  // reuses the tile area at the end

    // XCD-aware order: blocks are dispatched round-robin over the 8 XCDs, so
    // give each XCD a contiguous range of work items (the row blocks of one
    // leaf then share that XCD's L2).
    const uint32_t per_xcd = padded_grid / 8u;
    const uint32_t work = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    if (work >= total_work) return;
    const uint32_t leaf = work / blocks_per_leaf;
    const uint32_t blk = work % blocks_per_leaf;
    const uint32_t n = p.member_counts[leaf];
    const uint32_t row_base = blk * kRowsPerBlock;
    if (row_base >= n) return;
    if (n > p.max_leaf_rows || n > kMaxLeafRows) {
        if (threadIdx.x == 0) flag_overflow(p.counters, TESSA_OVF_LEAF_ROW);
        return;
    }
    const uint32_t *mem = p.members + p.member_offsets[leaf];
    const uint32_t pd = p.padded_dim;
    const uint32_t cap = (p.list_cap_override != 0u && p.list_cap_override < (uint32_t)kCap)
                             ? p.list_cap_override : (uint32_t)kCap;

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t j = lane & 31u;
    const uint32_t h = lane >> 5;
    const uint32_t r = row_base + wave * 32u + j;  // leaf-local row position
    bool row_ok = r < n;
    uint32_t mr = row_ok ? mem[r] : 0u;
    if (row_ok && mr >= p.rows) {
        flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_ROW_ID);
        row_ok = false;
        mr = 0u;
    }

    // Row codes for the whole K range (B operand), zero past padded_dim.
    v4i bfrag[KS];
    {
        const int8_t *rc = p.codes + (uint64_t)mr * pd;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const uint32_t off = 32u * s + 16u * h;
            v4i z = {0, 0, 0, 0};
            if (row_ok && off < pd) z = *reinterpret_cast<const v4i *>(rc + off);
            bfrag[s] = z;
        }
    }
    const float rs = row_ok ? p.scales[mr] : 0.0f;
    const float rn = row_ok ? p.norms[mr] : 0.0f;

    float top[kKeepPerLane];
#pragma unroll
    for (int i = 0; i < kKeepPerLane; ++i) top[i] = __builtin_inff();
    float F = __builtin_inff();
    int cnt = 0;
    int merged = 0;      // list entries already folded into `top`
    bool ovf = false;
    uint32_t survivors = 0, refines = 0;

    const uint32_t ntiles = (n + kTileCols - 1) / kTileCols;
    v4i pre[L::kChunksPerThread];
    float pre_meta = 0.0f;

    auto load_tile = [&](uint32_t t) {
#pragma unroll
        for (int q = 0; q < L::kChunksPerThread; ++q) {
            const uint32_t chunk = tid + q * kThreads;
            v4i z = {0, 0, 0, 0};
            if (chunk < (uint32_t)L::kChunks) {
                const uint32_t row = chunk / (KS * 2);
                const uint32_t off = (chunk % (KS * 2)) * 16u;
                const uint32_t c = t * kTileCols + row;
                if (c < n && off < pd) {
                    const uint32_t mc = mem[c];
                    if (mc < p.rows) z = *reinterpret_cast<const v4i *>(p.codes + (uint64_t)mc * pd + off);
                }
            }
            pre[q] = z;
        }
        // threads 0..31 carry scales, 32..63 norms of the tile's columns
        if (tid < 2u * kTileCols) {
            const uint32_t c = t * kTileCols + (tid & 31u);
            float v = 0.0f;
            if (c < n) {
                const uint32_t mc = mem[c];
                if (mc < p.rows) v = (tid < 32u) ? p.scales[mc] : p.norms[mc];
                else flag_overflow(p.counters, TESSA_OVF_INVALID_TOPK_COL_ID);
            }
            pre_meta = v;
        }
    };

    load_tile(0);
    for (uint32_t t = 0; t < ntiles; ++t) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < L::kChunksPerThread; ++q) {
            const uint32_t chunk = tid + q * kThreads;
            if (chunk < (uint32_t)L::kChunks) {
                const uint32_t row = chunk / (KS * 2);
                const uint32_t off = (chunk % (KS * 2)) * 16u;
                *reinterpret_cast<v4i *>(tile + row * L::kTileStride + off) = pre[q];
            }
        }
        if (tid < 2u * kTileCols) meta_s[tid] = pre_meta;  // meta_n follows meta_s
        __syncthreads();
        if (t + 1 < ntiles) load_tile(t + 1);

        v16i acc = {};
        const int8_t *arow = tile + j * L::kTileStride + 16u * h;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const v4i a = *reinterpret_cast<const v4i *>(arow + 32 * s);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bfrag[s], acc, 0, 0, 0);
        }

        // Epilogue: exact distances, running-threshold filter, list append.
        const uint32_t cbase = t * kTileCols;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 cs4 = *reinterpret_cast<const float4 *>(meta_s + 8 * q + 4 * h);
            const float4 cn4 = *reinterpret_cast<const float4 *>(meta_n + 8 * q + 4 * h);
            const float csv[4] = {cs4.x, cs4.y, cs4.z, cs4.w};
            const float cnv[4] = {cn4.x, cn4.y, cn4.z, cn4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = 4 * q + e;
                const uint32_t c = cbase + 8u * q + 4u * h + e;
                const float d = leaf_l2(acc[v], rs, rn, csv[e], cnv[e]);
                const bool cand = row_ok && c < n && c != r && d <= F;
                const bool room = cnt < (int)cap;
                ovf |= cand && !room;
                const bool take = cand && room;
                const int slot = take ? cnt : kCap;  // slot kCap is a scratch sink
                list_d[slot * kThreads + tid] = d;
                list_c[slot * kThreads + tid] = (uint16_t)c;
                cnt += take ? 1 : 0;
                survivors += take ? 1u : 0u;
            }
        }

        // Refine before the next tile can overflow a list (up to 16 appends).
        if (__any(cnt > (int)cap - 16)) {
            ++refines;
            const int fresh = wave_max_i(cnt - merged);
            for (int base = 0; base < fresh; base += 16) {
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int e = merged + base + i;
                    v[i] = (e < cnt) ? list_d[e * kThreads + tid] : __builtin_inff();
                }
                bitonic_sort<16>(v);
                float m[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) m[i] = fminf(top[i], v[15 - i]);
                bitonic_merge<16>(m);
#pragma unroll
                for (int i = 0; i < 16; ++i) top[i] = m[i];
            }
            const float own = top[kKeepPerLane - 1];
            F = fmaxf(own, __shfl_xor(own, 32));
            const int cmax = wave_max_i(cnt);
            int kept = 0;
            for (int e = 0; e < cmax; ++e) {
                if (e < cnt) {
                    const float d = list_d[e * kThreads + tid];
                    const uint16_t c = list_c[e * kThreads + tid];
                    const bool keep = d <= F;
                    const int slot = keep ? kept : kCap;
                    list_d[slot * kThreads + tid] = d;
                    list_c[slot * kThreads + tid] = c;
                    kept += keep ? 1 : 0;
                }
            }
            cnt = kept;
            merged = kept;
        }
    }

    // ---- final ordered insertion -------------------------------------------
    __syncthreads();  // tile area is free: stage the leaf's global ids
    for (uint32_t c = tid; c < n; c += kThreads) {
        const uint32_t mc = mem[c];
        gid_lds[c] = mc < p.rows ? p.gids[mc] : kEmptyId;
    }
    __syncthreads();

    const int cnt_b = __shfl_xor(cnt, 32);
    const bool ovf_b = __shfl_xor((int)ovf, 32) != 0;
    uint32_t final_cands = 0, fallbacks = 0, gap_fallbacks = 0, list_ovf = 0, done_rows = 0;
    if (h == 0u && row_ok) {
        const uint32_t keff = (p.k < n - 1u) ? p.k : (n - 1u);
        const uint32_t slot_row = wave * 32u + j;
        const uint32_t tid_b = tid + 32u;
        bool ok = !(ovf || ovf_b);
        if (!ok) ++list_ovf;
        uint32_t len = 0;
        if (ok && keff > 0u) {
            int ia = 0, ib = 0;
            while (ia < cnt || ib < cnt_b) {
                float d;
                uint32_t c;
                const uint32_t ca = ia < cnt ? list_c[ia * kThreads + tid] : 0xffffu;
                const uint32_t cb = ib < cnt_b ? list_c[ib * kThreads + tid_b] : 0xffffu;
                if (ia < cnt && (ib >= cnt_b || ca < cb)) {
                    d = list_d[ia * kThreads + tid];
                    c = ca;
                    ++ia;
                } else {
                    d = list_d[ib * kThreads + tid_b];
                    c = cb;
                    ++ib;
                }
                if (!(d <= F)) continue;
                ++final_cands;
                const uint32_t g = gid_lds[c];
                // compute_backend.rs:7229-7259 insertion into keff slots.
                if (len < keff) {
                    uint32_t pos = len;
                    while (pos > 0 && beats(d, g, fin_d[(pos - 1) * kRowsPerBlock + slot_row],
                                            fin_g[(pos - 1) * kRowsPerBlock + slot_row])) {
                        fin_d[pos * kRowsPerBlock + slot_row] = fin_d[(pos - 1) * kRowsPerBlock + slot_row];
                        fin_g[pos * kRowsPerBlock + slot_row] = fin_g[(pos - 1) * kRowsPerBlock + slot_row];
                        --pos;
                    }
                    fin_d[pos * kRowsPerBlock + slot_row] = d;
                    fin_g[pos * kRowsPerBlock + slot_row] = g;
                    ++len;
                } else {
                    const uint32_t last = keff - 1;
                    if (!beats(d, g, fin_d[last * kRowsPerBlock + slot_row], fin_g[last * kRowsPerBlock + slot_row]))
                        continue;
                    uint32_t pos = last;
                    while (pos > 0 && beats(d, g, fin_d[(pos - 1) * kRowsPerBlock + slot_row],
                                            fin_g[(pos - 1) * kRowsPerBlock + slot_row])) {
                        fin_d[pos * kRowsPerBlock + slot_row] = fin_d[(pos - 1) * kRowsPerBlock + slot_row];
                        fin_g[pos * kRowsPerBlock + slot_row] = fin_g[(pos - 1) * kRowsPerBlock + slot_row];
                        --pos;
                    }
                    fin_d[pos * kRowsPerBlock + slot_row] = d;
                    fin_g[pos * kRowsPerBlock + slot_row] = g;
                }
            }
            if (len < keff) ok = false;  // cannot happen when F is finite; be strict
            if (ok) {
                // Gap certificate: theta >= max kept distance, no candidate in
                // (theta, theta + eps], and theta + eps < F (list completeness).
                float theta = 0.0f;
                for (uint32_t s = 0; s < keff; ++s) theta = fmaxf(theta, fin_d[s * kRowsPerBlock + slot_row]);
                for (int guard = 0; guard < 2 * kCap + 2; ++guard) {
                    float next = __builtin_inff();
                    for (int e = 0; e < cnt; ++e) {
                        const float d = list_d[e * kThreads + tid];
                        if (d <= F && d > theta) next = fminf(next, d);
                    }
                    for (int e = 0; e < cnt_b; ++e) {
                        const float d = list_d[e * kThreads + tid_b];
                        if (d <= F && d > theta) next = fminf(next, d);
                    }
                    if (next == __builtin_inff()) {
                        ok = __fsub_rn(F, theta) > kTieEps;
                        break;
                    }
                    if (__fsub_rn(next, theta) > kTieEps) break;
                    theta = next;
                    if (guard == 2 * kCap + 1) ok = false;
                }
                if (!ok) ++gap_fallbacks;
            }
        }
        if (ok) {
            const uint64_t out = p.output_offsets[leaf] + (uint64_t)r * p.k;
            for (uint32_t s = 0; s < p.k; ++s) {
                const bool live = s < keff;
                p.out_ids[out + s] = live ? fin_g[s * kRowsPerBlock + slot_row] : kEmptyId;
                p.out_dists[out + s] = live ? fin_d[s * kRowsPerBlock + slot_row] : kEmptyDist;
            }
            ++done_rows;
        } else {
            ++fallbacks;
            const uint32_t idx = atomicAdd(p.fallback_count, 1u);
            if (idx < p.fallback_capacity) {
                p.fallback[2 * idx] = leaf;
                p.fallback[2 * idx + 1] = r;
            } else {
                flag_overflow(p.counters, TESSA_OVF_LEAF_ROW);
            }
        }
    }

    // One atomic per counter per wave.
    uint64_t s_surv = survivors, s_fc = final_cands, s_fb = fallbacks, s_gap = gap_fallbacks,
             s_lo = list_ovf, s_done = done_rows;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        s_surv += __shfl_xor(s_surv, off);
        s_fc += __shfl_xor(s_fc, off);
        s_fb += __shfl_xor(s_fb, off);
        s_gap += __shfl_xor(s_gap, off);
        s_lo += __shfl_xor(s_lo, off);
        s_done += __shfl_xor(s_done, off);
    }
    if (lane == 0) {
        counter_add(p.counters, TESSA_C_LEAF_SURVIVORS, s_surv);
        counter_add(p.counters, TESSA_C_LEAF_FINAL_CANDIDATES, s_fc);
        counter_add(p.counters, TESSA_C_LEAF_FALLBACK_ROWS, s_fb);
        counter_add(p.counters, TESSA_C_LEAF_GAP_FALLBACK_ROWS, s_gap);
        counter_add(p.counters, TESSA_C_LEAF_LIST_OVERFLOW_ROWS, s_lo);
        counter_add(p.counters, TESSA_C_LEAF_ROWS, s_done);
        counter_add(p.counters, TESSA_C_LEAF_REFINES, refines);
        counter_add(p.counters, TESSA_C_LEAF_MFMA_TILES, ntiles);
    }
}

template <int KS>
int launch_ks(const LeafParams &p, hipStream_t stream) {
    using L = Layout<KS>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void *)leaf_mfma_kernel<KS>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes) != hipSuccess)
            return -1;
        attr_set = true;
    }
    const uint32_t blocks_per_leaf = (p.max_leaf_rows + kRowsPerBlock - 1) / kRowsPerBlock;
    const uint64_t total = (uint64_t)blocks_per_leaf * p.leaf_count;
    if (total == 0) return 0;
    if (total > 0x7fffff00ull) return -2;
    const uint32_t padded = (uint32_t)((total + 7) / 8 * 8);
    hipLaunchKernelGGL(leaf_mfma_kernel<KS>, dim3(padded), dim3(kThreads), L::kBytes, stream, p,
                       blocks_per_leaf, (uint32_t)total, padded);
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
