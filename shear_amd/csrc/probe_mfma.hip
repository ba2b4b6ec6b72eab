// probe_mfma.hip -- diagnostic: the sustained int8 MFMA rate of this GPU.
//
// No counterpart in the reference.  It measures the ceiling the leaf
// filter's roofline is read against in practice: every wave of the grid
// issues independent v_mfma_i32_32x32x32_i8 chains whose A/B operands cycle
// through eight registers of random bytes (constant operands barely toggle
// the multipliers and let the clock stay high), with no memory traffic in
// the loop, for long enough that the power management settles.  It reports
// the int8 rate and the shader clock (s_memtime cycles over the 100 MHz
// wall clock) of the fastest of three runs.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/tessa_hip.h"

namespace tessa {
namespace {

tessa_status probe_status(int32_t code, const char *what, const char *why) {
    tessa_status s;
    std::memset(&s, 0, sizeof(s));
    s.code = code;
    if (what) std::snprintf(s.msg, sizeof(s.msg), "probe: %s%s%s", what, why ? " failed: " : "", why ? why : "");
    return s;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kProbeThreads = 256;
constexpr int kProbeRegs = 8;

template <int CH>
__global__ __launch_bounds__(kProbeThreads) void mfma_rate_kernel(const v4i *rnd, uint64_t iters, int *sink,
                                                                  unsigned long long *clk) {
    const uint64_t t = (uint64_t)blockIdx.x * kProbeThreads + threadIdx.x;
    v4i ra[kProbeRegs], rb[kProbeRegs];
#pragma unroll
    for (int i = 0; i < kProbeRegs; ++i) {
        ra[i] = rnd[t * 2 * kProbeRegs + i];
        rb[i] = rnd[t * 2 * kProbeRegs + kProbeRegs + i];
    }
    v16i acc[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[c] = v16i{};
    const unsigned long long c0 = __builtin_readcyclecounter(), r0 = wall_clock64();
    for (uint64_t it = 0; it < iters; it += kProbeRegs) {
#pragma unroll
        for (int u = 0; u < kProbeRegs; ++u)
#pragma unroll
            for (int c = 0; c < CH; ++c)
                acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ra[(u + c) % kProbeRegs], rb[(3 * u + c) % kProbeRegs],
                                                               acc[c], 0, 0, 0);
    }
    const unsigned long long c1 = __builtin_readcyclecounter(), r1 = wall_clock64();
    int s = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) s += acc[c][v];
    sink[t] = s;  // keeps the MFMAs live
    if (t == 0) {
        clk[0] = c1 - c0;
        clk[1] = r1 - r0;
    }
}

}  // namespace
}  // namespace tessa

extern "C" tessa_status tessa_probe_mfma_rate(uint32_t workgroups, uint32_t chains, uint64_t iters, double *tops,
                                              double *mhz) {
    using namespace tessa;
    if (!tops || !mhz || workgroups == 0 || iters == 0 || (chains != 2 && chains != 4 && chains != 8))
        return probe_status(TESSA_ERR_INVALID_ARGUMENT, "workgroups, iters > 0 and chains in {2, 4, 8}", nullptr);
    iters = (iters + kProbeRegs - 1) / kProbeRegs * kProbeRegs;
    const size_t nthreads = (size_t)workgroups * kProbeThreads;
    std::vector<uint32_t> h(nthreads * 2 * kProbeRegs * 4);
    uint32_t x = 2463534242u;
    for (auto &w : h) {  // xorshift32
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        w = x;
    }
    v4i *rnd = nullptr;
    int *sink = nullptr;
    unsigned long long *clk = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    tessa_status st = probe_status(TESSA_OK, nullptr, nullptr);
    auto fail = [&](hipError_t e, const char *what) { st = probe_status(TESSA_ERR_HIP, what, hipGetErrorString(e)); };
    hipError_t e;
    if ((e = hipMalloc(&rnd, h.size() * 4)) != hipSuccess || (e = hipMalloc(&sink, nthreads * 4)) != hipSuccess ||
        (e = hipMalloc(&clk, 16)) != hipSuccess || (e = hipEventCreate(&e0)) != hipSuccess ||
        (e = hipEventCreate(&e1)) != hipSuccess ||
        (e = hipMemcpy(rnd, h.data(), h.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) {
        fail(e, "set-up");
    } else {
        float best = 1e30f;
        for (int rep = 0; rep < 3 && st.code == TESSA_OK; ++rep) {
            hipEventRecord(e0, nullptr);
            if (chains == 2)
                hipLaunchKernelGGL(mfma_rate_kernel<2>, dim3(workgroups), dim3(kProbeThreads), 0, nullptr, rnd, iters,
                                   sink, clk);
            else if (chains == 4)
                hipLaunchKernelGGL(mfma_rate_kernel<4>, dim3(workgroups), dim3(kProbeThreads), 0, nullptr, rnd, iters,
                                   sink, clk);
            else
                hipLaunchKernelGGL(mfma_rate_kernel<8>, dim3(workgroups), dim3(kProbeThreads), 0, nullptr, rnd, iters,
                                   sink, clk);
            hipEventRecord(e1, nullptr);
            if ((e = hipEventSynchronize(e1)) != hipSuccess) {
                fail(e, "run");
                break;
            }
            float ms = 0.0f;
            unsigned long long c[2] = {0, 0};
            if ((e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess ||
                (e = hipMemcpy(c, clk, 16, hipMemcpyDeviceToHost)) != hipSuccess) {
                fail(e, "read-back");
                break;
            }
            if (ms < best && c[1] > 0) {
                best = ms;
                const double ops = (double)nthreads / 64.0 * chains * (double)iters * 65536.0;
                *tops = ops / (ms * 1e-3) / 1e12;
                *mhz = (double)c[0] / (double)c[1] * 100.0;
            }
        }
    }
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (rnd) hipFree(rnd);
    if (sink) hipFree(sink);
    if (clk) hipFree(clk);
    return st;
}
