// sq8_quantize.hip -- per-vector symmetric SQ8 quantizer on the GPU.
//
// Restates dco_sq_int8.rs:1431-1467 bit for bit: max|x| and a *sequential*
// f32 sum of squares in dimension order (the reference's own GPU twin,
// compute_backend.rs:17955-18014, tree-reduces the norm and can differ in the
// last bits; this kernel does not), scale = max|x| / max_code (correctly
// rounded division), code = clamp(round_half_away(x / scale)).  Rows with a
// non-finite value are zeroed and reported.
//
// The sums are sequential per row, so one thread owns one row; the row data
// reaches it through LDS.  A workgroup takes 256 rows and walks them in
// 64-column chunks: the waves load a chunk with consecutive lanes on
// consecutive addresses (float4 per lane when rows are 16-byte aligned) into a
// row-major LDS tile padded to 65 floats per row, so the owner threads then
// read their rows without bank conflicts.  Pass 1 accumulates max|x| and the
// norm; pass 2 reloads each chunk, quantizes it and writes the codes through a
// second LDS tile as 4-byte words from consecutive lanes.  HBM traffic per row:
// 2 * 4 * dim read + padded_dim + 8 written.
#include "tessa_device.h"

namespace tessa {

namespace {

constexpr int kQRows = 256;              // rows per workgroup, one per thread
constexpr int kQCols = 64;               // columns per chunk
constexpr int kQStride = kQCols + 1;     // floats per LDS row
constexpr int kQCodeWords = kQCols / 4 + 1;  // u32 code words per LDS row

// One chunk of columns [c0, c0 + w) of rows row0.. into the LDS tile.
template <bool kVec4>
__device__ __forceinline__ void load_chunk(const float *x, uint64_t row0, uint32_t nrows, uint32_t dim, uint32_t c0,
                                           uint32_t w, float *tile) {
    const uint32_t t = threadIdx.x;
    if (kVec4 && (w & 3u) == 0u) {
        // 16 lanes per row, 4 floats each: a wave instruction reads 4 rows
        const uint32_t q = t & 15u;
        for (uint32_t r = t >> 4; r < nrows; r += kQRows / 16) {
            if (4u * q < w) {
                const float4 v = *reinterpret_cast<const float4 *>(x + (row0 + r) * dim + c0 + 4u * q);
                float *o = tile + r * kQStride + 4u * q;
                o[0] = v.x;
                o[1] = v.y;
                o[2] = v.z;
                o[3] = v.w;
            }
        }
    } else {
        const uint32_t c = t & 63u;
        for (uint32_t r = t >> 6; r < nrows; r += kQRows / 64)
            if (c < w) tile[r * kQStride + c] = x[(row0 + r) * dim + c0 + c];
    }
}

template <bool kVec4>
__global__ __launch_bounds__(kQRows) void sq8_quantize_kernel(const float *x, uint64_t rows, uint32_t dim,
                                                              uint32_t padded_dim, float max_code, int8_t *codes,
                                                              float *scales, float *norms,
                                                              unsigned long long *bad_row) {
    __shared__ float tile[kQRows * kQStride];
    __shared__ uint32_t ctile[kQRows * kQCodeWords];
    const uint64_t row0 = (uint64_t)blockIdx.x * kQRows;
    const uint32_t nrows = rows - row0 < (uint64_t)kQRows ? (uint32_t)(rows - row0) : (uint32_t)kQRows;
    const uint32_t t = threadIdx.x;
    const bool mine = t < nrows;
    float max_abs = 0.0f;
    float norm = 0.0f;
    bool finite = true;
    // pass 1: max|x| and the sequential sum of squares
    for (uint32_t c0 = 0; c0 < dim; c0 += kQCols) {
        const uint32_t w = dim - c0 < (uint32_t)kQCols ? dim - c0 : (uint32_t)kQCols;
        __syncthreads();  // the previous chunk has been read
        load_chunk<kVec4>(x, row0, nrows, dim, c0, w, tile);
        __syncthreads();
        if (mine) {
            const float *rowp = tile + t * kQStride;
            for (uint32_t c = 0; c < w; ++c) {
                const float v = rowp[c];
                finite &= isfinite(v);
                max_abs = fmaxf(max_abs, fabsf(v));
                norm = __fadd_rn(norm, __fmul_rn(v, v));
            }
        }
    }
    // zero codes for a non-finite row (reported) or an all-zero row
    const bool zero = !finite || max_abs == 0.0f;
    const float scale = zero ? 1.0f : __fdiv_rn(max_abs, max_code);
    if (mine) {
        scales[row0 + t] = scale;
        norms[row0 + t] = finite ? norm : 0.0f;
        if (!finite && bad_row) atomicMin(bad_row, (unsigned long long)(row0 + t));
    }
    // pass 2: codes, chunk by chunk, through the code tile
    for (uint32_t c0 = 0; c0 < padded_dim; c0 += kQCols) {
        const uint32_t w_in = dim > c0 ? (dim - c0 < (uint32_t)kQCols ? dim - c0 : (uint32_t)kQCols) : 0u;
        const uint32_t w_out = padded_dim - c0 < (uint32_t)kQCols ? padded_dim - c0 : (uint32_t)kQCols;
        __syncthreads();  // the previous chunk's tiles have been read
        if (w_in) load_chunk<kVec4>(x, row0, nrows, dim, c0, w_in, tile);
        __syncthreads();
        if (mine) {
            const float *rowp = tile + t * kQStride;
            for (uint32_t c = 0; c < w_out; c += 4) {
                uint32_t word = 0u;
#pragma unroll
                for (uint32_t e = 0; e < 4; ++e) {
                    int8_t code = 0;
                    if (!zero && c + e < w_in) {
                        float qv = roundf(__fdiv_rn(rowp[c + e], scale));
                        qv = fminf(fmaxf(qv, -max_code), max_code);
                        code = (int8_t)(int)qv;
                    }
                    word |= (uint32_t)(uint8_t)code << (8u * e);
                }
                ctile[t * kQCodeWords + c / 4] = word;
            }
        }
        __syncthreads();
        // rows of codes: w_out / 4 words each, consecutive lanes on consecutive words
        const uint32_t words = w_out / 4u;
        for (uint32_t e = t; e < nrows * words; e += kQRows) {
            const uint32_t r = e / words, qw = e - r * words;
            *reinterpret_cast<uint32_t *>(codes + (row0 + r) * padded_dim + c0 + 4u * qw) = ctile[r * kQCodeWords + qw];
        }
    }
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
    const uint64_t blocks = (rows + kQRows - 1) / kQRows;
    if (blocks > 0x7fffffffull) return -2;
    const bool vec4 = dim % 4u == 0u && (reinterpret_cast<uintptr_t>(x) & 15u) == 0u;
    if (vec4)
        hipLaunchKernelGGL(sq8_quantize_kernel<true>, dim3((uint32_t)blocks), dim3(kQRows), 0, stream, x, rows, dim,
                           padded_dim, max_code, codes, scales, norms, (unsigned long long *)bad_row);
    else
        hipLaunchKernelGGL(sq8_quantize_kernel<false>, dim3((uint32_t)blocks), dim3(kQRows), 0, stream, x, rows,
                           dim, padded_dim, max_code, codes, scales, norms, (unsigned long long *)bad_row);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tessa
