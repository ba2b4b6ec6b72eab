// assign_replay.hip -- leader assignment replay on gfx950 int8 MFMA.
//
// Reference: gpu_tessa_assignment_replay (compute_backend.rs:15729-15943) with
// gpu_persistent_assignment_best_slots4_no_dco (:6618-6699) and the insertion
// rule gpu_persistent_assignment_insert_candidate (:6524-6580).  For each
// member, leaders are visited in slot order and kept in 4 slots; a candidate
// within 2e-5 of a slot is ordered by the SplitMix64 tie key of
// (member, leader) and then by leader id.
//
// A workgroup takes one task and a run of 128-member chunks; the task's
// leaders (<= 128) are staged once in LDS as the MFMA "A" operand and each
// wave keeps 32 members' codes in VGPRs as "B".  Per 32-leader tile the
// distances go through LDS so that one lane per member can apply the
// order-dependent insertion in leader-slot order.  Member codes are read once
// from HBM; leader codes come from L2 after the first workgroup of the task.
#include "kernel_attr.h"
#include "assign_kernels.h"
#include "tessa_device.h"

namespace tessa {



namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kThreads = 256;
constexpr int kChunkMembers = kWaves * 32;
constexpr int kMaxLeaders = 128;
constexpr int kChunksPerBlock = 4;  // 512 members per workgroup amortise the leader stage

template <int KS>
struct ALayout {
    static constexpr int kStride = KS * 32 + 16;
    static constexpr int kLeaderBytes = kMaxLeaders * kStride;
    static constexpr int kMetaOff = kLeaderBytes;  // scales, norms, local ids [128] each
    static constexpr int kDistOff = kMetaOff + 3 * kMaxLeaders * 4;
    static constexpr int kBytes = kDistOff + kWaves * 32 * 33 * 4;
    static_assert(kBytes <= 160 * 1024, "LDS budget");
};

__device__ __forceinline__ bool assign_before(float d, uint32_t point, uint32_t leader, float od,
                                              uint32_t oleader, uint32_t &ties) {
    // compute_backend.rs:6541-6568
    if (fabsf(__fsub_rn(d, od)) <= kTieEps) {
        ++ties;
        const uint64_t ck = assign_tie_key(point, leader);
        const uint64_t ok = assign_tie_key(point, oleader);
        return ck < ok || (ck == ok && leader < oleader);
    }
    return d < od;
}

template <int KS>
__global__ __launch_bounds__(kThreads, 1) void assign_mfma_kernel(AssignParams p, uint32_t blocks_per_task) {
    using L = ALayout<KS>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    int8_t *lcodes = reinterpret_cast<int8_t *>(smem);
    float *ls = reinterpret_cast<float *>(smem + L::kMetaOff);
    float *ln = ls + kMaxLeaders;
    uint32_t *lid = reinterpret_cast<uint32_t *>(ln + kMaxLeaders);
    float *dbuf = reinterpret_cast<float *>(smem + L::kDistOff);

    const uint32_t task = blockIdx.x / blocks_per_task;
    const uint32_t bt = blockIdx.x % blocks_per_task;
    if (task >= p.task_count) return;
    const uint32_t nm = p.member_counts[task];
    const uint32_t nl = p.leader_counts[task];
    const uint32_t rh = p.r_h[task];
    const uint32_t first = bt * kChunkMembers * kChunksPerBlock;
    if (first >= nm) return;
    if (nl > (uint32_t)kMaxLeaders || rh == 0 || rh > 4 || nl < rh) {
        if (threadIdx.x == 0) flag_overflow(p.counters, TESSA_OVF_UNSUPPORTED_EXPLICIT_KERNEL);
        return;
    }
    const uint32_t pd = p.padded_dim;
    const uint32_t *tm = p.members + p.member_offsets[task];
    const uint32_t *tl = p.leaders + p.leader_offsets[task];
    const uint32_t tid = threadIdx.x;

    // Stage the task's leaders (A operand) and their scales/norms/ids.
    for (uint32_t q = tid; q < (uint32_t)kMaxLeaders * KS * 2; q += kThreads) {
        const uint32_t li = q / (KS * 2);
        const uint32_t off = (q % (KS * 2)) * 16u;
        v4i z = {0, 0, 0, 0};
        if (li < nl && off < pd) {
            const uint32_t g = tl[li];
            if (g < p.rows) z = *reinterpret_cast<const v4i *>(p.codes + (uint64_t)g * pd + off);
        }
        *reinterpret_cast<v4i *>(lcodes + li * L::kStride + off) = z;
    }
    for (uint32_t li = tid; li < (uint32_t)kMaxLeaders; li += kThreads) {
        uint32_t g = li < nl ? tl[li] : 0u;
        if (li < nl && g >= p.rows) {
            flag_overflow(p.counters, TESSA_OVF_INVALID_ASSIGN_LEADER_ID);
            g = 0u;
        }
        ls[li] = li < nl ? p.scales[g] : 0.0f;
        ln[li] = li < nl ? p.norms[g] : 0.0f;
        lid[li] = g;
    }
    __syncthreads();

    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t j = lane & 31u;
    const uint32_t h = lane >> 5;
    const uint32_t ntiles = (nl + 31) / 32;
    uint32_t pairs = 0, rows_done = 0, ties = 0;

    for (int ch = 0; ch < kChunksPerBlock; ++ch) {
        const uint32_t m = first + ch * kChunkMembers + wave * 32u + j;
        if (first + ch * kChunkMembers >= nm) break;  // uniform across the block
        bool ok = m < nm;
        uint32_t pt = ok ? tm[m] : 0u;
        if (ok && pt >= p.rows) {
            flag_overflow(p.counters, TESSA_OVF_INVALID_ASSIGN_POINT_ID);
            ok = false;
            pt = 0u;
        }
        v4i bfrag[KS];
        const int8_t *mc = p.codes + (uint64_t)pt * pd;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const uint32_t off = 32u * s + 16u * h;
            v4i z = {0, 0, 0, 0};
            if (ok && off < pd) z = *reinterpret_cast<const v4i *>(mc + off);
            bfrag[s] = z;
        }
        const float ps = ok ? p.scales[pt] : 0.0f;
        const float pn = ok ? p.norms[pt] : 0.0f;

        // compute_backend.rs:6357-6368 reset: 4 slots of (FLT_MAX, empty)
        float bd[4] = {kEmptyDist, kEmptyDist, kEmptyDist, kEmptyDist};
        uint32_t bs[4] = {kEmptyId, kEmptyId, kEmptyId, kEmptyId};
        uint32_t bl[4] = {kEmptyId, kEmptyId, kEmptyId, kEmptyId};

        for (uint32_t t = 0; t < ntiles; ++t) {
            v16i acc = {};
            const int8_t *arow = lcodes + (32u * t + j) * L::kStride + 16u * h;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const v4i a = *reinterpret_cast<const v4i *>(arow + 32 * s);
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bfrag[s], acc, 0, 0, 0);
            }
            float *wb = dbuf + wave * 32 * 33;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t li = 8u * (v / 4) + 4u * h + (v % 4);  // leader within tile
                const uint32_t gl = 32u * t + li;
                const float d = gl < nl ? assign_l2(acc[v], ps, pn, ls[gl], ln[gl]) : kEmptyDist;
                wb[li * 33 + j] = d;
            }
            __syncthreads();
            if (h == 0u && ok) {
                const uint32_t lim = (nl - 32u * t) < 32u ? (nl - 32u * t) : 32u;
                for (uint32_t li = 0; li < lim; ++li) {
                    const uint32_t slot = 32u * t + li;
                    const uint32_t leader = lid[slot];
                    const float d = wb[li * 33 + j];
                    if (!assign_before(d, pt, leader, bd[3], bl[3], ties)) continue;
                    int pos = 3;
                    while (pos > 0 && assign_before(d, pt, leader, bd[pos - 1], bl[pos - 1], ties)) {
                        bd[pos] = bd[pos - 1];
                        bs[pos] = bs[pos - 1];
                        bl[pos] = bl[pos - 1];
                        --pos;
                    }
                    bd[pos] = d;
                    bs[pos] = slot;
                    bl[pos] = leader;
                }
            }
            __syncthreads();
        }
        if (h == 0u && ok) {
            const uint64_t out = p.output_offsets[task] + (uint64_t)m * rh;
            for (uint32_t q = 0; q < rh; ++q) {
                const uint32_t slot = bs[q];
                if (slot >= nl) {
                    flag_overflow(p.counters, TESSA_OVF_QUEUE_ROW);
                    continue;
                }
                p.out_ids[out + q] = p.gids[lid[slot]];
                p.out_dists[out + q] = bd[q];
            }
            pairs += nl;
            ++rows_done;
        }
    }
    uint64_t a = pairs, b = rows_done, c = ties;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        a += __shfl_xor(a, off);
        b += __shfl_xor(b, off);
        c += __shfl_xor(c, off);
    }
    if (lane == 0) {
        counter_add(p.counters, TESSA_C_ASSIGN_PAIRS, a);
        counter_add(p.counters, TESSA_C_ASSIGN_ROWS, b);
        counter_add(p.counters, TESSA_C_ASSIGN_TIE_EVENTS, c);
    }
}

template <int KS>
int launch_assign_ks(const AssignParams &p, hipStream_t stream) {
    using L = ALayout<KS>;
    if (ensure_lds_limit(reinterpret_cast<const void *>(assign_mfma_kernel<KS>), L::kBytes)) return -1;
    const uint32_t per_block = kChunkMembers * kChunksPerBlock;
    const uint32_t blocks_per_task = (p.max_members + per_block - 1) / per_block;
    const uint64_t total = (uint64_t)blocks_per_task * p.task_count;
    if (total == 0) return 0;
    if (total > 0x7fffffffull) return -2;
    hipLaunchKernelGGL(assign_mfma_kernel<KS>, dim3((uint32_t)total), dim3(kThreads), L::kBytes, stream, p,
                       blocks_per_task);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_assign_replay(const AssignParams &p, hipStream_t stream) {
    const uint32_t ks = (p.padded_dim + 31) / 32;
    if (ks <= 4) return launch_assign_ks<4>(p, stream);
    if (ks <= 8) return launch_assign_ks<8>(p, stream);
    if (ks <= 12) return launch_assign_ks<12>(p, stream);
    if (ks <= 16) return launch_assign_ks<16>(p, stream);
    if (ks <= 24) return launch_assign_ks<24>(p, stream);
    if (ks <= 32) return launch_assign_ks<32>(p, stream);
    return -3;
}

}  // namespace tessa
