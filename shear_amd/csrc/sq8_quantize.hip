// sq8_quantize.hip -- per-vector symmetric SQ8 quantizer on the GPU.
//
// Restates dco_sq_int8.rs:1431-1467 bit for bit: max|x| and a *sequential*
// f32 sum of squares in dimension order (the reference's own GPU twin,
// compute_backend.rs:17955-18014, tree-reduces the norm and can differ in the
// last bits; this kernel does not), scale = max|x| / max_code (correctly
// rounded division), code = clamp(round_half_away(x / scale)).  One thread
// per row; rows with a non-finite value are zeroed and reported.
#include "tessa_device.h"

namespace tessa {

namespace {

__global__ __launch_bounds__(256) void sq8_quantize_kernel(const float *x, uint64_t rows, uint32_t dim,
                                                           uint32_t padded_dim, float max_code,
                                                           int8_t *codes, float *scales, float *norms,
                                                           unsigned long long *bad_row) {
    const uint64_t row = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const float *in = x + row * dim;
    int8_t *out = codes + row * padded_dim;
    float max_abs = 0.0f;
    float norm = 0.0f;
    bool finite = true;
    for (uint32_t d = 0; d < dim; ++d) {
        const float v = in[d];
        finite &= isfinite(v);
        max_abs = fmaxf(max_abs, fabsf(v));
        norm = __fadd_rn(norm, __fmul_rn(v, v));
    }
    if (!finite) {
        for (uint32_t d = 0; d < padded_dim; ++d) out[d] = 0;
        scales[row] = 1.0f;
        norms[row] = 0.0f;
        if (bad_row) atomicMin(bad_row, (unsigned long long)row);
        return;
    }
    if (max_abs == 0.0f) {
        for (uint32_t d = 0; d < padded_dim; ++d) out[d] = 0;
        scales[row] = 1.0f;
        norms[row] = norm;
        return;
    }
    const float scale = __fdiv_rn(max_abs, max_code);
    for (uint32_t d = 0; d < dim; ++d) {
        float q = roundf(__fdiv_rn(in[d], scale));
        q = fminf(fmaxf(q, -max_code), max_code);
        out[d] = (int8_t)(int)q;
    }
    for (uint32_t d = dim; d < padded_dim; ++d) out[d] = 0;
    scales[row] = scale;
    norms[row] = norm;
}

__global__ void init_bad_row(unsigned long long *bad_row) { *bad_row = ~0ull; }

}  // namespace

int launch_sq8_quantize(const float *x, uint64_t rows, uint32_t dim, uint32_t padded_dim, uint32_t bits,
                        int8_t *codes, float *scales, float *norms, uint64_t *bad_row, hipStream_t stream) {
    const float max_code = (float)((1u << (bits - 1)) - 1u);
    if (bad_row) {
        hipLaunchKernelGGL(init_bad_row, dim3(1), dim3(1), 0, stream, (unsigned long long *)bad_row);
    }
    if (rows == 0) return 0;
    const uint64_t blocks = (rows + 255) / 256;
    if (blocks > 0x7fffffffull) return -2;
    hipLaunchKernelGGL(sq8_quantize_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, x, rows, dim,
                       padded_dim, max_code, codes, scales, norms, (unsigned long long *)bad_row);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
