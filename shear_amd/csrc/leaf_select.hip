// leaf_select.hip -- second kernel of the SQ8 leaf operator: per row, the
// fold of the filter kernel's survivor logs, the exactness certificate and
// the row's output (or its hand-off to the chain replay / exact re-run).
//
// Reference role: the per-row RowTopK result of the leaf filter
// (leaf_build.rs:887-957 insertion with the mod.rs:417-428 comparator;
// compute_backend.rs:7229-7259 on the GPU), written at the persistent output
// slice (compute_backend.rs:10924-10944 layout: slot (row, rank) at
// output_offsets[leaf] + row * k + rank).
//
// One workgroup per work item (leaf, 256-row block) of the batch, one thread
// per block row.  The leaf's scales, norms and global ids are staged in LDS.
// A thread reads its row's survivor log (the filter's lane pair, entries
// interleaved), turns each (raw dot, column) entry into the exact distance
// and folds the entries 16 at a time into the sorted 32 smallest plus the sorted next 8 (bitonic
// networks with the column as payload); `disc` is the smallest distance that
// left the 40.  Every candidate the row has not seen lies above F (the
// filter's threshold), every dropped one at or above disc.
//
// Certificate over the known sequence s_0 <= ... <= s_39 (consecutive
// elements within 2e-5 form tie clusters; G = s_0..s_q is the prefix closed
// at the cluster holding s_{k-1}):
//  * the next distance after s_q, known or not, lies more than 2e-5 above
//    s_q: every candidate outside G is then eps-separated from all of G, so
//    the reference's bounded insertion over the whole row keeps exactly G's
//    k best (such candidates can neither enter in front of G's nor stay);
//  * every cluster inside G spans <= 2e-5: the tie relation is then an
//    equivalence on G and the comparator a total order (distance order,
//    clusters by global id), so the row is written directly;
//  * a cluster wider than 2e-5 (an eps-chain, whose result depends on the
//    arrival order) sends the row with G to the chain replay, which inserts
//    G's members in column order;
//  * anything else (no gap, an overflowed log) sends the row to the exact
//    re-run.
// Queue slots are reserved with one atomic per wave.
#include "kernel_attr.h"
#include "leaf_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

constexpr int kSelThreads = (int)kLeafBlockRows;  // one thread per block row
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kTop = 32;
constexpr int kNext = 8;
constexpr int kSeq = kTop + kNext;
static_assert(kSeq == (int)kLeafChainSetEntries, "a chain row's pool set holds the 40 known positions");

// Sort keys: (distance, column) as one double.  The high word holds the
// distance's bits plus 2^20 (distances are >= 0, so their bit patterns order
// like their values; the offset keeps every key a normal double), the low
// word the column.  Non-negative doubles order like their bit patterns, so
// f64 min / max order the keys by (distance, column), and a compare-exchange
// is two instructions with no mask registers.
constexpr uint32_t kKeyBias = 0x00100000u;
__device__ __forceinline__ double dkey(float d, uint32_t col) {
    return __hiloint2double((int)(__float_as_uint(d) + kKeyBias), (int)col);
}
__device__ __forceinline__ float key_dist(double k) {
    return __uint_as_float((uint32_t)__double2hiint(k) - kKeyBias);
}
__device__ __forceinline__ uint32_t key_col(double k) { return (uint32_t)__double2loint(k); }
#define kInfKey (__hiloint2double((int)(0x7f800000u + kKeyBias), 0xffff))

template <int N>
__device__ __forceinline__ void sort_keys(double (&v)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const double lo = fmin(v[i], v[l]), hi = fmax(v[i], v[l]);
                    const bool up = (i & k) == 0;
                    v[i] = up ? lo : hi;
                    v[l] = up ? hi : lo;
                }
            }
        }
    }
}

// Sorts a bitonic sequence ascending.
template <int N>
__device__ __forceinline__ void merge_keys(double (&v)[N]) {
#pragma unroll
    for (int j = N >> 1; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int l = i ^ j;
            if (l > i) {
                const double lo = fmin(v[i], v[l]), hi = fmax(v[i], v[l]);
                v[i] = lo;
                v[l] = hi;
            }
        }
    }
}

// Wave-wide exclusive prefix sum of x; *total gets the wave's sum.
__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t x, uint32_t *total) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(inc, off);
        inc += lane >= (uint32_t)off ? y : 0u;
    }
    *total = __shfl(inc, 63);
    return inc - x;
}

// One thread of the workgroup: turns the per-wave totals red[w][q] of up to
// two queues into exclusive per-wave offsets and reserves the workgroup's
// total of queue q with one atomic on counter q; the base goes to
// red[kSelWaves][q].
__device__ __forceinline__ void wg_reserve(uint32_t (*red)[2], int queues, uint32_t *c0, uint32_t *c1) {
    for (int q = 0; q < queues; ++q) {
        uint32_t run = 0;
        for (int w = 0; w < kSelWaves; ++w) {
            const uint32_t t = red[w][q];
            red[w][q] = run;
            run += t;
        }
        uint32_t *ctr = q == 0 ? c0 : c1;
        red[kSelWaves][q] = run ? atomicAdd(ctr, run) : 0u;
    }
}

__global__ __launch_bounds__(kSelThreads, 2) void leaf_select_kernel(LeafParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const uint32_t cols_cap = (p.max_leaf_rows + 31u) & ~31u;
    float *cs_lds = reinterpret_cast<float *>(smem);
    float *cn_lds = cs_lds + cols_cap;
    uint32_t *gid_lds = reinterpret_cast<uint32_t *>(cn_lds + cols_cap);

    __shared__ uint32_t red[kSelWaves + 1][2];  // per-wave totals, then (row kSelWaves) the bases
    __shared__ uint32_t stat[kSelWaves][5];
    const uint32_t tid = threadIdx.x;
    const uint32_t work = blockIdx.x;
    const uint32_t g = p.item_begin + work;
    if (g >= *p.item_total) return;  // past the listed items
    const uint2 li = p.item_list[g];
    const uint32_t leaf = li.x;
    const uint32_t blk = li.y;
    const uint32_t n = p.member_counts[leaf];
    const uint32_t row_base = blk * kLeafBlockRows;
    // whole-workgroup exits only (the filter kernel flagged oversized leaves)
    if (row_base >= n || n > p.max_leaf_rows) return;
    const uint32_t *mem = p.members + p.member_offsets[leaf];
    // staged 8 columns per thread at a time: every member id of a step is
    // requested before any of them is used, then every scale, norm and id
    // (two memory round trips per step instead of two per column)
    for (uint32_t c0 = tid; c0 < n; c0 += 8u * kSelThreads) {
        uint32_t mc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = c0 + (uint32_t)i * kSelThreads;
            mc[i] = mem[c < n ? c : c0];
        }
        float sv[8], nv[8];
        uint32_t gv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t m = mc[i] < p.rows ? mc[i] : 0u;
            sv[i] = p.scales[m];
            nv[i] = p.norms[m];
            gv[i] = p.gids[m];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = c0 + (uint32_t)i * kSelThreads;
            if (c < n) {
                cs_lds[c] = sv[i];
                cn_lds[c] = nv[i];
                gid_lds[c] = gv[i];
            }
        }
    }
    __syncthreads();

    const uint32_t r = row_base + tid;
    const bool row_ok = r < n;
    const uint32_t pk = p.k;
    const uint32_t keff = n > 1u ? ((pk < n - 1u) ? pk : (n - 1u)) : 0u;
    const uint32_t cap = p.log_capacity;
    const uint4 meta = row_ok ? p.row_meta[(uint64_t)work * kLeafBlockRows + tid] : make_uint4(0u, 0u, 0u, 0u);
    const float F = __uint_as_float(meta.x);
    const uint32_t cnt0 = meta.y, cnt1 = meta.z;
    const bool log_ovf = cnt0 > cap || cnt1 > cap;
    const uint32_t lim0 = cnt0 < cap ? cnt0 : cap;
    const uint32_t lim1 = cnt1 < cap ? cnt1 : cap;
    // the row's log: entry e of the filter lane h at 2e + h
    const uint4 *rlog = reinterpret_cast<const uint4 *>(p.survivor_log +
                                                         ((uint64_t)work * kLeafBlockRows + tid) * 2ull * cap);
    const uint32_t span = row_ok ? 2u * (lim0 > lim1 ? lim0 : lim1) : 0u;  // entries to read (holes included)
    const float rs = row_ok ? cs_lds[r] : 1.0f;
    const float rn = row_ok ? cn_lds[r] : 0.0f;

    // ---- fold: the 40 smallest (distance, column) in two sorted runs --------
    // Keys are (distance, column) packed into one double (see dkey): the
    // networks below are plain f64 min / max.
    double td[kTop], nd[kNext];
#pragma unroll
    for (int i = 0; i < kTop; ++i) td[i] = kInfKey;
#pragma unroll
    for (int i = 0; i < kNext; ++i) nd[i] = kInfKey;
    double disc = kInfKey;
    // 16 entries per step as 8 aligned 16-byte loads (inside the row's region:
    // span <= 2 * cap, a multiple of 16); the next step's loads are issued
    // before this step's entries are folded
    uint4 qn[8];
    if (span > 0u) {
#pragma unroll
        for (int i = 0; i < 8; ++i) qn[i] = rlog[(uint32_t)i];
    }
    for (uint32_t base = 0; base < span; base += 16u) {
        uint4 q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = qn[i];
        if (base + 16u < span) {
#pragma unroll
            for (int i = 0; i < 8; ++i) qn[i] = rlog[(base + 16u) / 2u + (uint32_t)i];
        }
        double v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t e = base + (uint32_t)i;
            const uint32_t dot = (i & 1) ? q[i / 2].z : q[i / 2].x;
            const uint32_t cc = (i & 1) ? q[i / 2].w : q[i / 2].y;
            const bool valid = (e >> 1) < ((i & 1) ? lim1 : lim0);
            const uint32_t col = cc < n ? cc : 0u;
            const float d = leaf_l2((int)dot, rs, rn, cs_lds[col], cn_lds[col]);
            v[i] = valid ? dkey(d, cc) : kInfKey;
        }
        sort_keys<16>(v);
        // lower 32 of (top ascending) ++ (chunk descending, padded): positions
        // 16..31 meet the chunk; the larger of each pair forms the spill
        double sp[16];
#pragma unroll
        for (int i = 16; i < kTop; ++i) {
            const double a = td[i], b = v[kTop - 1 - i];
            sp[i - 16] = fmax(a, b);
            td[i] = fmin(a, b);
        }
        merge_keys<kTop>(td);
        merge_keys<16>(sp);  // the upper half of a half-cleaner is bitonic
        // next 8 = lower 8 of (next ascending) ++ (spill ascending): only the
        // spill's 8 smallest can enter
        double dmin = sp[8];
#pragma unroll
        for (int i = 0; i < kNext; ++i) {
            const double a = nd[i], b = sp[kNext - 1 - i];
            dmin = fmin(dmin, fmax(a, b));
            nd[i] = fmin(a, b);
        }
        merge_keys<kNext>(nd);
        disc = fmin(disc, dmin);
    }
    float sd[kSeq];
    uint32_t sc[kSeq];
#pragma unroll
    for (int i = 0; i < kTop; ++i) {
        sd[i] = key_dist(td[i]);
        sc[i] = key_col(td[i]);
    }
#pragma unroll
    for (int i = 0; i < kNext; ++i) {
        sd[kTop + i] = key_dist(nd[i]);
        sc[kTop + i] = key_col(nd[i]);
    }
    // not known: filtered (d > F) or dropped from the 40 (>= disc)
    const float disc_all = fminf(key_dist(disc), F);

    // ---- certificate -----------------------------------------------------------
    // bit i of `same`: positions i and i+1 are in one cluster; bit i of
    // `bad`: position i is tied to its predecessor but lies more than eps
    // past its cluster's first element (the cluster is not a clique).  Both
    // are built as bit masks in one pass, so no per-position condition stays
    // live across the passes below.
    uint64_t same = 0ull, bad = 0ull;
    {
        float cstart = sd[0];
#pragma unroll
        for (int i = 1; i < kSeq; ++i) {
            const bool tie = __fsub_rn(sd[i], sd[i - 1]) <= kTieEps;  // false on INF/NaN
            same |= tie ? (1ull << (i - 1)) : 0ull;
            bad |= (tie && (__fsub_rn(sd[i], cstart) > kTieEps)) ? (1ull << i) : 0ull;
            cstart = tie ? cstart : sd[i];
        }
    }
    // G = positions [0, q_end]: from keff - 1 on, every position tied to
    // the next extends it; `extending` when the ties run to the end of the
    // known sequence (the gap after G is then not known)
    int q_end = (int)keff - 1;  // last index of G
    bool extending = false;
    if (keff > 0u) {
        const uint32_t k0 = keff - 1u;                 // the first tie that could extend G
        const uint32_t room = (uint32_t)kSeq - 1u - k0;  // ties that exist after it
        const uint64_t t = ~(same >> k0);
        const uint32_t run = t ? (uint32_t)__builtin_ctzll(t) : 64u;
        extending = run >= room;
        q_end = (int)(k0 + (run < room ? run : room));
    }
    const uint64_t in_q = q_end >= 1 ? ((2ull << q_end) - 2ull) : 0ull;  // positions 1..q_end
    const bool clique_bad = (bad & in_q) != 0ull;
    bool gap_ok = (keff == 0u || !extending) && !log_ovf;
    if (keff > 0u && gap_ok) {
        float theta = sd[0];
        float next = disc_all;
#pragma unroll
        for (int i = 1; i < kSeq; ++i) {
            theta = (i == q_end) ? sd[i] : theta;
            next = (i == q_end + 1) ? fminf(next, sd[i]) : next;
        }
        gap_ok = next == __builtin_inff() || __fsub_rn(next, theta) > kTieEps;
    }
    // Test knob: re-run every `debug_rerun_every`-th row through the exact kernel.
    if (p.debug_rerun_every != 0u && (r % p.debug_rerun_every) == 0u) gap_ok = false;
    const bool direct = row_ok && gap_ok && !clique_bad;
    const bool chain = row_ok && gap_ok && clique_bad;

    // Direct rows: global ids of G's positions, then each cluster ordered by
    // global id (odd-even transposition; sorted once an even and an odd phase
    // in a row swap nothing).
#pragma unroll
    for (int i = 0; i < kSeq; ++i) {
        const uint32_t col = sc[i] < n ? sc[i] : 0u;
        sc[i] = (direct && i <= q_end && sc[i] < n) ? gid_lds[col] : sc[i];
    }
    const uint64_t in_g = q_end >= 1 ? ((q_end >= 64 ? ~0ull : ((1ull << q_end) - 1ull))) : 0ull;
    if (__any(direct && (same & in_g) != 0ull)) {
        const uint64_t mask = direct ? (same & in_g) : 0ull;
        for (int pass = 0; pass < kSeq + 2; pass += 2) {
            bool swapped = false;
#pragma unroll
            for (int i = 0; i + 1 < kSeq; i += 2) {
                const bool sw = ((mask >> i) & 1ull) && sc[i] > sc[i + 1];
                const uint32_t ga = sc[i], gb = sc[i + 1];
                const float da = sd[i], db = sd[i + 1];
                sc[i] = sw ? gb : ga;
                sc[i + 1] = sw ? ga : gb;
                sd[i] = sw ? db : da;
                sd[i + 1] = sw ? da : db;
                swapped |= sw;
            }
#pragma unroll
            for (int i = 1; i + 1 < kSeq; i += 2) {
                const bool sw = ((mask >> i) & 1ull) && sc[i] > sc[i + 1];
                const uint32_t ga = sc[i], gb = sc[i + 1];
                const float da = sd[i], db = sd[i + 1];
                sc[i] = sw ? gb : ga;
                sc[i + 1] = sw ? ga : gb;
                sd[i] = sw ? db : da;
                sd[i + 1] = sw ? da : db;
                swapped |= sw;
            }
            if (!__any(swapped)) break;
        }
    }

    // ---- output ----------------------------------------------------------------
    const uint64_t out = p.output_offsets[leaf] + (uint64_t)r * pk;
    if (direct) {
        if ((pk & 3u) == 0u && (out & 3u) == 0u) {
#pragma unroll
            for (int i = 0; i < kTop; i += 4) {
                if ((uint32_t)i >= pk) continue;
                uint4 gi, gd;
                gi.x = (uint32_t)(i + 0) < keff ? sc[i + 0] : kEmptyId;
                gi.y = (uint32_t)(i + 1) < keff ? sc[i + 1] : kEmptyId;
                gi.z = (uint32_t)(i + 2) < keff ? sc[i + 2] : kEmptyId;
                gi.w = (uint32_t)(i + 3) < keff ? sc[i + 3] : kEmptyId;
                gd.x = __float_as_uint((uint32_t)(i + 0) < keff ? sd[i + 0] : kEmptyDist);
                gd.y = __float_as_uint((uint32_t)(i + 1) < keff ? sd[i + 1] : kEmptyDist);
                gd.z = __float_as_uint((uint32_t)(i + 2) < keff ? sd[i + 2] : kEmptyDist);
                gd.w = __float_as_uint((uint32_t)(i + 3) < keff ? sd[i + 3] : kEmptyDist);
                *reinterpret_cast<uint4 *>(p.out_ids + out + i) = gi;
                *reinterpret_cast<uint4 *>(p.out_dists + out + i) = gd;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kTop; ++i) {
                if ((uint32_t)i >= pk) continue;
                const bool live = (uint32_t)i < keff;
                p.out_ids[out + i] = live ? sc[i] : kEmptyId;
                p.out_dists[out + i] = live ? sd[i] : kEmptyDist;
            }
        }
    }

    // chain rows: header (output offset, pool offset, |G| | keff << 8) and
    // |G| pool entries (distance bits, column, global id).  The pool keeps the
    // candidate sets of 64 consecutive queue entries interleaved: entry i of
    // queue index x at (x / 64 * kSeq + i) * 64 + x % 64, so the chain kernel
    // (one lane per queue entry) reads entry i of 64 rows as one 1 KB run.
    const uint32_t m = chain ? (uint32_t)q_end + 1u : 0u;
    const uint32_t wave = tid >> 6, lane = tid & 63u;
    // queue slots: a wave prefix sum, then one atomic per workgroup
    uint32_t tot_c = 0;
    const uint32_t pre_c = wave_excl_scan(chain ? 1u : 0u, &tot_c);
    if (lane == 0u) red[wave][0] = tot_c;
    __syncthreads();
    if (tid == 0u) wg_reserve(red, 1, p.chain_count, nullptr);
    __syncthreads();
    const uint32_t idx = red[kSelWaves][0] + red[wave][0] + pre_c;
    const uint64_t pbase = (uint64_t)(idx >> 6) * (uint64_t)(kSeq * 64) + (idx & 63u);
    const bool queued = chain && idx < p.chain_capacity &&
                        ((uint64_t)(idx >> 6) + 1u) * (uint64_t)(kSeq * 64) <= p.chain_pool_capacity;
    if (queued) {
#pragma unroll
        for (int i = 0; i < kSeq; ++i)
            if ((uint32_t)i < m)
                p.chain_pool[pbase + (uint64_t)i * 64u] =
                    make_uint4(__float_as_uint(sd[i]), sc[i], gid_lds[sc[i] < n ? sc[i] : 0u], 0u);
        p.chain_rows[idx] = make_uint4((uint32_t)out, (uint32_t)(out >> 32), (uint32_t)pbase, m | (keff << 8));
    }
    const bool rerun = row_ok && !direct && !queued;
    uint32_t tot_f = 0;
    const uint32_t pre_f = wave_excl_scan(rerun ? 1u : 0u, &tot_f);
    __syncthreads();  // the slot words above are read
    if (lane == 0u) red[wave][0] = tot_f;
    __syncthreads();
    if (tid == 0u) wg_reserve(red, 1, p.fallback_count, nullptr);
    __syncthreads();
    if (rerun) {
        const uint32_t fidx = red[kSelWaves][0] + red[wave][0] + pre_f;
        if (fidx < p.fallback_capacity) {
            p.fallback[2 * fidx] = leaf;
            p.fallback[2 * fidx + 1] = r;
        } else {
            flag_overflow(p.counters, TESSA_OVF_LEAF_ROW);
        }
    }

    // statistics: one atomic per counter and workgroup
    uint32_t v5[5] = {direct ? 1u : 0u, queued ? 1u : 0u, queued ? m : 0u, rerun ? 1u : 0u,
                      (row_ok && log_ovf) ? 1u : 0u};
#pragma unroll
    for (int c = 0; c < 5; ++c) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v5[c] += __shfl_xor(v5[c], o);
    }
    __syncthreads();
    if (lane == 0u)
        for (int c = 0; c < 5; ++c) stat[wave][c] = v5[c];
    __syncthreads();
    if (tid < 5u) {
        uint64_t t = 0;
        for (int w = 0; w < kSelWaves; ++w) t += stat[w][tid];
        const int idx5[5] = {TESSA_C_LEAF_ROWS, TESSA_C_LEAF_CHAIN_ROWS, TESSA_C_LEAF_FINAL_CANDIDATES,
                             TESSA_C_LEAF_FALLBACK_ROWS, TESSA_C_LEAF_LIST_OVERFLOW_ROWS};
        if (t) {
            counter_add(p.counters, idx5[tid], t);
            if (tid == 3u) counter_add(p.counters, TESSA_C_LEAF_GAP_FALLBACK_ROWS, t);
        }
    }
}

}  // namespace

int launch_leaf_select(const LeafParams &p, hipStream_t stream) {
    if (p.item_count == 0) return 0;
    const uint32_t cols_cap = (p.max_leaf_rows + 31u) & ~31u;
    const uint32_t lds = cols_cap * 12u;
    if (ensure_lds_limit(reinterpret_cast<const void *>(leaf_select_kernel), 64 * 1024)) return -1;
    if (lds > 64u * 1024u) return -4;
    hipLaunchKernelGGL(leaf_select_kernel, dim3(p.item_count), dim3(kSelThreads), lds, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
