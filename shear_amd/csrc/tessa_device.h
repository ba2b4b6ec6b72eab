// tessa_device.h -- device helpers shared by the gfx950 TESSA kernels.
//
// Distances are computed with explicit round-to-nearest intrinsics in the
// reference's operation order; the library is also compiled with
// -ffp-contract=off, so no multiply-add is fused behind our back.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tessa_hip.h"

namespace tessa {

constexpr float kTieEps = 2.0e-5f;        // mod.rs:74 STABLE_DISTANCE_TIE_EPS
constexpr uint32_t kEmptyId = 0xffffffffu;
constexpr float kEmptyDist = 3.402823466e+38f;  // FLT_MAX, compute_backend.rs:16531
constexpr int kMaxK = 32;

// compute_backend.rs:8987-9002 gpu_persistent_sq_int8_l2_from_dot:
// (rn + cn) + (-2 * ((rs * cs) * (float)dot)), clamped at 0.
__device__ __forceinline__ float leaf_l2(int dot, float rs, float rn, float cs, float cn) {
    float sc = __fmul_rn(rs, cs);
    float u = __fmul_rn(sc, (float)dot);
    float w = __fmul_rn(-2.0f, u);
    float d = __fadd_rn(__fadd_rn(rn, cn), w);
    return d <= 0.0f ? 0.0f : d;
}

// rbc_partition.rs:17630-17639 (compute_backend.rs:6400-6411 without the FMA
// contraction NVRTC may apply): (pn + ln) - ((2 * ps) * ls) * (float)dot.
__device__ __forceinline__ float assign_l2(int dot, float ps, float pn, float ls, float ln) {
    float a = __fmul_rn(2.0f, ps);
    float b = __fmul_rn(a, ls);
    float c = __fmul_rn(b, (float)dot);
    float d = __fsub_rn(__fadd_rn(pn, ln), c);
    return d <= 0.0f ? 0.0f : d;
}

// Squared L2 of two f32 rows summed over the coordinates in order, each
// product rounded before the add (the order the graph search and the final
// prune are pinned to).  kVec4: 16-byte aligned rows, dim a multiple of 4.
template <bool kVec4>
__device__ float l2_ordered(const float *__restrict__ x, const float *__restrict__ q, uint32_t dim) {
    float s = 0.0f;
    if constexpr (kVec4) {
        const float4 *xv = reinterpret_cast<const float4 *>(x);
        const float4 *qv = reinterpret_cast<const float4 *>(q);
        for (uint32_t i = 0; i < dim / 4; ++i) {
            const float4 a = xv[i], b = qv[i];
            float t = __fsub_rn(a.x, b.x);
            s = __fadd_rn(s, __fmul_rn(t, t));
            t = __fsub_rn(a.y, b.y);
            s = __fadd_rn(s, __fmul_rn(t, t));
            t = __fsub_rn(a.z, b.z);
            s = __fadd_rn(s, __fmul_rn(t, t));
            t = __fsub_rn(a.w, b.w);
            s = __fadd_rn(s, __fmul_rn(t, t));
        }
    } else {
        for (uint32_t i = 0; i < dim; ++i) {
            const float t = __fsub_rn(x[i], q[i]);
            s = __fadd_rn(s, __fmul_rn(t, t));
        }
    }
    return s;
}

// mod.rs:417-428 stable_distance_order(..).is_lt(): does candidate c beat s?
__device__ __forceinline__ bool beats(float dc, uint32_t idc, float ds, uint32_t ids) {
    float delta = __fsub_rn(dc, ds);
    return fabsf(delta) <= kTieEps ? (idc < ids) : (dc < ds);
}

// compute_backend.rs:5983-5989 (SplitMix64 finalizer).
__device__ __forceinline__ uint64_t hash64(uint64_t v) {
    v ^= v >> 30;
    v *= 0xbf58476d1ce4e5b9ull;
    v ^= v >> 27;
    v *= 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

// compute_backend.rs:6513-6522.
__device__ __forceinline__ uint64_t assign_tie_key(uint32_t point, uint32_t leader) {
    return hash64((((uint64_t)point) << 32) ^ (uint64_t)leader ^ 0x9e3779b97f4a7c15ull);
}

__device__ __forceinline__ void counter_add(uint64_t *counters, int idx, uint64_t v) {
    if (counters != nullptr && v != 0)
        atomicAdd((unsigned long long *)&counters[idx], (unsigned long long)v);
}

__device__ __forceinline__ void flag_overflow(uint64_t *counters, uint64_t bits) {
    if (counters != nullptr)
        atomicOr((unsigned long long *)&counters[TESSA_C_OVERFLOW_FLAGS], (unsigned long long)bits);
}

// Exact int8 dot of two code rows of `n` bytes (n % 16 == 0, 16-byte aligned
// rows) using the packed signed dot4 instruction; integer, so order-free.
__device__ __forceinline__ int dot_i8_rows(const int8_t *a, const int8_t *b, uint32_t n) {
    const int4 *pa = reinterpret_cast<const int4 *>(a);
    const int4 *pb = reinterpret_cast<const int4 *>(b);
    int acc = 0;
    for (uint32_t i = 0; i < n / 16; ++i) {
        int4 x = pa[i];
        int4 y = pb[i];
        acc = __builtin_amdgcn_sdot4(x.x, y.x, acc, false);
        acc = __builtin_amdgcn_sdot4(x.y, y.y, acc, false);
        acc = __builtin_amdgcn_sdot4(x.z, y.z, acc, false);
        acc = __builtin_amdgcn_sdot4(x.w, y.w, acc, false);
    }
    return acc;
}

}  // namespace tessa
