// prune.hip -- the final RobustPrune pass over a neighbour table, one
// wavefront per point.
//
// Reference (paths relative to shear-core/src/): final_prune_pipnn,
// index/inmem_index/pipnn_builder.rs:287-330 (the pool is the point's current
// neighbours with their distance to it; an empty row stays empty), then
// robust_prune / occlude_list, algorithm/prune/prune.rs:17-214: the pool sorted
// by (distance, id) and cut to max_occlusion; alpha passes 1.0, x1.2, .. while
// <= alpha and the result is short of max_degree; in pool order a candidate
// whose occlusion factor is <= the pass's alpha is taken (factor := f32::MAX,
// added unless it is the point itself) and every later candidate whose factor
// is <= alpha gets max(factor, d_j / d(j, taken)), f32::MAX when that
// distance is 0; with saturate and alpha > 1 the result is then filled from
// the pool in order.
//
// The scan over the pool is sequential by definition; the wave runs it with
// uniform control and spreads each taken candidate's factor updates over the
// lanes (one later candidate per lane, its distance to the taken one summed in
// coordinate order).  Pool keys (distance bits << 32 | id) are sorted in LDS by
// a wave bitonic network; the factors and the result list live in LDS.
#include "prune_kernels.h"
#include "tessa_device.h"

namespace tessa {

namespace {

constexpr uint32_t kWaves = 4;
constexpr uint32_t kThreads = kWaves * 64;
constexpr uint64_t kNoKey = ~0ull;

struct alignas(16) PruneLds {
    uint64_t key[kPruneMaxPool];
    float occ[kPruneMaxPool];
    uint32_t res[kPruneMaxPool];
};

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ void wave_sort_lds(uint64_t *key, uint32_t n2, uint32_t lane) {
    for (uint32_t k = 2; k <= n2; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t c = lane; c < n2 / 2; c += 64) {
                const uint32_t i = ((c & ~(j - 1u)) << 1) | (c & (j - 1u));
                const uint32_t l = i + j;
                const bool up = (i & k) == 0;
                const uint64_t a = key[i], b = key[l];
                if (up ? b < a : a < b) {
                    key[i] = b;
                    key[l] = a;
                }
            }
            wave_lds_sync();
        }
    }
}

template <bool kVec4>
__global__ __launch_bounds__(kThreads) void robust_prune_kernel(RobustPruneParams p) {
    __shared__ PruneLds lds[kWaves];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t v = blockIdx.x * kWaves + wave;
    if (v >= p.num_points) return;  // whole wave
    PruneLds &w = lds[wave];
    const float *xv = p.data + (uint64_t)v * p.dim;
    const uint32_t cnt = p.counts[v];
    const uint32_t deg = cnt < p.row_stride ? cnt : p.row_stride;
    uint32_t n2 = 1;
    while (n2 < deg) n2 <<= 1;
    uint32_t n = 0;
    for (uint32_t s0 = 0; s0 < n2; s0 += 64) {
        const uint32_t s = s0 + lane;
        const uint32_t id = s < deg ? p.targets[(uint64_t)v * p.row_stride + s] : 0xFFFFFFFFu;
        const bool ok = id < p.num_points;
        uint64_t key = kNoKey;
        if (ok) key = ((uint64_t)__float_as_uint(l2_ordered<kVec4>(xv, p.data + (uint64_t)id * p.dim, p.dim)) << 32) | id;
        if (s < n2) w.key[s] = key;
        n += (uint32_t)__popcll(__ballot(ok));
    }
    wave_lds_sync();
    wave_sort_lds(w.key, n2, lane);
    if (n > p.max_occlusion) n = p.max_occlusion;
    for (uint32_t i = lane; i < n; i += 64) w.occ[i] = 0.0f;
    wave_lds_sync();

    uint32_t rl = 0;
    if (n > 0) {
        float cur = 1.0f;
        while (cur <= p.alpha && rl < p.max_degree) {
            for (uint32_t i = 0; i < n; ++i) {
                if (rl >= p.max_degree) break;
                if (w.occ[i] > cur) continue;
                const uint64_t ki = w.key[i];
                const uint32_t idi = (uint32_t)ki;
                wave_lds_sync();
                if (lane == 0) {
                    w.occ[i] = kEmptyDist;  // f32::MAX
                    if (idi != v) w.res[rl] = idi;
                }
                if (idi != v) ++rl;
                const float *xi = p.data + (uint64_t)idi * p.dim;
                for (uint32_t j = i + 1 + lane; j < n; j += 64) {
                    const float oj = w.occ[j];
                    if (oj > p.alpha) continue;
                    const uint64_t kj = w.key[j];
                    const float djk = l2_ordered<kVec4>(p.data + (uint64_t)(uint32_t)kj * p.dim, xi, p.dim);
                    float nf;
                    if (djk == 0.0f) {
                        nf = kEmptyDist;
                    } else {
                        const float q = __fdiv_rn(__uint_as_float((uint32_t)(kj >> 32)), djk);
                        nf = oj > q ? oj : q;
                    }
                    w.occ[j] = nf;
                }
                wave_lds_sync();
            }
            cur = __fmul_rn(cur, 1.2f);
        }
        if (p.saturate && p.alpha > 1.0f) {
            for (uint32_t i = 0; i < n && rl < p.max_degree; ++i) {
                const uint32_t idi = (uint32_t)w.key[i];
                bool seen = false;
                for (uint32_t r = lane; r < rl; r += 64) seen = seen || (w.res[r] == idi);
                seen = __ballot(seen) != 0ull || idi == v;
                wave_lds_sync();
                if (!seen) {
                    if (lane == 0) w.res[rl] = idi;
                    ++rl;
                }
                wave_lds_sync();
            }
        }
    }
    wave_lds_sync();
    uint32_t *out = p.out_targets + (uint64_t)v * p.max_degree;
    for (uint32_t r = lane; r < p.max_degree; r += 64) out[r] = r < rl ? w.res[r] : 0xFFFFFFFFu;
    if (lane == 0) p.out_counts[v] = rl;
}

}  // namespace

int launch_robust_prune(const RobustPruneParams &p, hipStream_t stream) {
    if (p.num_points == 0) return 0;
    const dim3 grid((p.num_points + kWaves - 1) / kWaves), block(kThreads);
    const bool vec4 = p.dim % 4 == 0 && reinterpret_cast<uintptr_t>(p.data) % 16 == 0;
    if (vec4) hipLaunchKernelGGL(robust_prune_kernel<true>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(robust_prune_kernel<false>, grid, block, 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
