// capacity.hip -- GPU-memory-aware task formation: resident admission of a
// subtree task and the D0 capacity thresholds (host code, no device work).
//
// Reference (shear-core/src/algorithm/pipnn/):
//   tessa_plan_subtree_resident_admission  compute_backend.rs:1490-1522 with the
//       resident estimates :898-930 (f32 rows, or SQ8 codes padded to 16 bytes /
//       packed int4, plus a u32 id and two f32 per row)
//   tessa_find_max_admissible_rows         d0_capacity.rs:55-102 (doubling, then
//       bisection, of the largest admitted row count below 2^31)
//   tessa_d0_thresholds                    d0_capacity.rs:201-223
//   tessa_d0_plan_root_leaders             d0_capacity.rs:225-258
//   tessa_d0_split_leader_count            d0_capacity.rs:260-265
//   tessa_d0_observe_child_sizes           d0_capacity.rs:267-299
#include <algorithm>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/tessa_hip.h"

namespace {

uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
uint64_t sat_mul(uint64_t a, uint64_t b) { return (b && a > UINT64_MAX / b) ? UINT64_MAX : a * b; }

uint64_t resident_bytes(uint64_t rows, uint32_t dim, uint32_t format) {
    if (format == TESSA_RESIDENT_F32)  // estimate_gpu_resident_subtree_device_bytes
        return sat_add(sat_mul(rows, sat_mul(dim, 4)), sat_add(sat_mul(rows, 4), sat_mul(rows, 4)));
    const uint64_t padded = ((uint64_t)dim + 15) / 16 * 16;
    const uint64_t code = format == TESSA_RESIDENT_SQ4 ? (padded + 1) / 2 : padded;
    return sat_mul(rows, code + 4 + 4 + 4);
}

uint64_t div_ceil(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }

}  // namespace

extern "C" {

tessa_status tessa_plan_subtree_resident_admission(uint64_t resident_rows, uint32_t dim, uint32_t leaf_knn,
                                                   uint32_t max_leaders_per_node, uint32_t max_fanout,
                                                   uint64_t workspace_budget_bytes, uint64_t device_budget_bytes,
                                                   uint32_t c_max, uint32_t resident_format,
                                                   tessa_resident_admission *out) {
    tessa_status st{};
    if (!out) {
        st.code = TESSA_ERR_INVALID_ARGUMENT;
        std::snprintf(st.msg, sizeof(st.msg), "resident admission output is null");
        return st;
    }
    std::memset(out, 0, sizeof(*out));
    st = tessa_plan_subtree(resident_rows, leaf_knn, max_leaders_per_node, max_fanout, workspace_budget_bytes, c_max,
                            &out->plan);
    if (st.code) return st;
    out->resident_device_bytes = resident_bytes(resident_rows, dim, resident_format);
    out->device_admission_required_bytes = sat_add(out->resident_device_bytes, out->plan.required_bytes);
    out->device_admission_budget_bytes = device_budget_bytes ? device_budget_bytes : UINT64_MAX;
    if (resident_rows != 0 && device_budget_bytes && out->device_admission_required_bytes > device_budget_bytes) {
        out->plan.fallback_reason_flags |= TESSA_PLAN_FALLBACK_WORKSPACE;
        out->plan.overflow_flags |= TESSA_OVF_WORKSPACE_BUDGET;
        out->plan.supported = 0;
    }
    return st;
}

uint64_t tessa_find_max_admissible_rows(uint32_t dim, uint32_t leaf_knn, uint32_t max_leaders_per_node,
                                        uint32_t max_fanout, uint64_t workspace_budget_bytes,
                                        uint64_t device_budget_bytes, uint32_t c_max, uint32_t resident_format) {
    if (dim == 0) return 0;
    auto supported = [&](uint64_t rows) {
        tessa_resident_admission a;
        const tessa_status st = tessa_plan_subtree_resident_admission(
            rows, dim, leaf_knn, max_leaders_per_node, max_fanout, workspace_budget_bytes, device_budget_bytes, c_max,
            resident_format, &a);
        return st.code == 0 && a.plan.supported != 0;
    };
    if (!supported(1)) return 0;
    uint64_t lo = 1, hi = 2;
    while (supported(hi) && hi < (1ull << 31)) {
        lo = hi;
        hi *= 2;
    }
    while (lo + 1 < hi) {
        const uint64_t mid = lo + (hi - lo) / 2;
        if (supported(mid)) lo = mid;
        else hi = mid;
    }
    return lo;
}

tessa_d0_thresholds tessa_d0_compute_thresholds(uint64_t c_gpu, double high_ratio, double target_ratio,
                                                double low_ratio, uint64_t min_efficient_rows) {
    tessa_d0_thresholds t{};
    if (c_gpu == 0) return t;
    const double hi = std::min(std::max(high_ratio, 0.01), 1.0);
    const double tg = std::min(std::max(target_ratio, 0.01), hi);
    const double lo = std::min(std::max(low_ratio, 0.0), tg);
    auto cut = [&](double r) { return (uint64_t)std::max(std::floor((double)c_gpu * r), 1.0); };
    t.c_gpu = c_gpu;
    t.c_high = cut(hi);
    t.c_target = cut(tg);
    t.c_low = std::min(std::max(cut(lo), min_efficient_rows), t.c_target);
    return t;
}

tessa_d0_leader_plan tessa_d0_plan_root_leaders(uint64_t total_points, uint64_t root_fanout,
                                                const tessa_d0_thresholds *t, uint64_t quality_min_root_leaders,
                                                uint64_t root_leader_cap) {
    tessa_d0_leader_plan p{};
    if (total_points == 0 || root_fanout == 0 || !t) return p;
    const uint64_t assignments = sat_mul(total_points, root_fanout);
    p.k_capacity = t->c_target == 0 ? 0 : std::max<uint64_t>(div_ceil(assignments, t->c_target), 1);
    const uint64_t np = std::max<uint64_t>(total_points, 1);
    p.root_leader_cap = std::min(std::max<uint64_t>(root_leader_cap, 1), np);
    const uint64_t capacity_target = std::max<uint64_t>(p.k_capacity, 1);
    const uint64_t quality_floor = std::min(std::max<uint64_t>(quality_min_root_leaders, 1), np);
    const uint64_t desired = std::max(capacity_target, quality_floor);
    p.source = desired > p.root_leader_cap ? TESSA_D0_LEADERS_ROOT_CAP
               : quality_floor > capacity_target ? TESSA_D0_LEADERS_QUALITY_FLOOR
                                                 : TESSA_D0_LEADERS_CAPACITY;
    p.k_initial = std::min(std::max<uint64_t>(desired, 1), p.root_leader_cap);
    return p;
}

uint64_t tessa_d0_split_leader_count(uint64_t rows, const tessa_d0_thresholds *t) {
    if (!t || rows <= t->c_high || t->c_target == 0) return 1;
    return std::max<uint64_t>(div_ceil(rows, t->c_target), 2);
}

tessa_d0_child_summary tessa_d0_observe_child_sizes(const uint64_t *sizes, uint64_t count,
                                                    const tessa_d0_thresholds *t) {
    tessa_d0_child_summary s{};
    if (!sizes || count == 0 || !t) return s;
    std::vector<uint64_t> v(sizes, sizes + count);
    std::sort(v.begin(), v.end());
    auto pct = [&](uint64_t p) {  // nearest rank
        const uint64_t rank = div_ceil(sat_mul(v.size(), p), 100);
        return v[std::min<uint64_t>(rank ? rank - 1 : 0, v.size() - 1)];
    };
    s.max_rows = v.back();
    s.p50_rows = pct(50);
    s.p95_rows = pct(95);
    s.p99_rows = pct(99);
    for (uint64_t x : v) {
        if (x > t->c_high) ++s.oversized_count;
        if (x < t->c_low) {
            ++s.small_count;
            s.small_rows += x;
        }
    }
    return s;
}

}  // extern "C"
