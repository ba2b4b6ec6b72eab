// sq8_quantize.hip -- per-vector symmetric SQ8 quantizer on the GPU.
//
// Restates dco_sq_int8.rs:1431-1467 bit for bit: max|x| and a *sequential*
// f32 sum of squares in dimension order (the reference's own GPU twin,
// compute_backend.rs:17955-18014, tree-reduces the norm and can differ in the
// last bits; this kernel does not), scale = max|x| / max_code (correctly
// rounded division), code = clamp(round_half_away(x / scale)).  Rows with a
// non-finite value are zeroed and reported.
//
// The sums are sequential per row, so one lane owns one row's sum.  Rows of
// a width that is a multiple of 4 go through sq8_quantize_block_kernel (one
// wave per 4 rows, each row read from HBM once; see there).  Other rows go
// through sq8_quantize_kernel: a workgroup takes 256 rows and walks them in
// 64-column chunks through a padded LDS tile, one thread per row, pass 1 for
// max|x| and the norm, pass 2 reloading each chunk for the codes (HBM traffic
// per row: 2 * 4 * dim read + padded_dim + 8 written).
#include "kernel_attr.h"
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

// ---- one wave per block of rows, the block read once --------------------------
// The default path (dim % 4 == 0, 16-byte aligned rows, dim <= kBlockMaxDim).
// The wave copies its kBlockRows rows to LDS with 16-byte LDS-DMA loads
// (global_load_lds_dwordx4: no VGPR round trip), one run of instructions per
// row so each row starts 16 bytes past a multiple of its width (row stride
// dim + 4 floats, 4 dwords past a multiple of the 32 banks when dim % 32 == 0:
// the row lanes below read disjoint banks), then works from LDS only:
//  * max|x| of each row: every lane over its quads (4 columns) of the row,
//    then a wave max (exact in any order);
//  * lane r < rows forms row r's sequential sum of squares in dimension
//    order, one quad per step;
//  * all 64 lanes form the codes, one quad each per step, and store them as
//    4-byte words from consecutive lanes.
// Few rows per wave keep the LDS block small, so many waves share a CU and
// hide each other's DMA and LDS latency (10M x 768: 4 rows per wave 11.3 ms,
// 8 rows 16.7 ms, 16 rows 33 ms; the one-thread-per-row kernel below 46 ms).
// Codes: q = x * (1/scale) lies within 3 * 2^-24 * |x/scale| < 2.3e-5 of the
// correctly rounded quotient fl(x/scale) (|x/scale| <= max_code < 128), so
// round-half-away of q and of fl(x/scale) agree unless a half-integer lies
// within that distance of q; those elements (|frac(q) - 0.5| <= 4e-5), and
// rows whose scale is not a normal float with a finite reciprocal, take the
// correctly rounded division instead.  Codes equal the per-element division's
// bit for bit.
#ifndef TESSA_Q_BLOCK_ROWS
#define TESSA_Q_BLOCK_ROWS 4
#endif
constexpr uint32_t kBlockRows = TESSA_Q_BLOCK_ROWS;
constexpr uint32_t kBlockMaxDim = 8192;  // 128 KB of LDS per block of 4 rows
constexpr float kHalfMargin = 4.0e-5f;

enum : uint32_t { kRowFast = 0u, kRowExact = 1u, kRowZero = 2u };

// Fast path: no tie can occur (the quotient is more than the margin away from
// every half-integer), so round-half-away equals round-to-nearest-even.
__device__ __forceinline__ uint32_t quant_code(float v, float inv, float scale, uint32_t mode, float max_code) {
    const float q = __fmul_rn(v, inv);
    float r;
    if (mode == kRowFast && fabsf(__fsub_rn(__builtin_amdgcn_fractf(q), 0.5f)) > kHalfMargin)
        r = __builtin_rintf(q);
    else
        r = roundf(__fdiv_rn(v, scale));
    r = fminf(fmaxf(r, -max_code), max_code);
    return mode == kRowZero ? 0u : (uint32_t)(uint8_t)(int8_t)(int)r;
}

__global__ __launch_bounds__(64) void sq8_quantize_block_kernel(const float *x, uint64_t rows, uint32_t dim,
                                                                uint32_t padded_dim, float max_code, int8_t *codes,
                                                                float *scales, float *norms,
                                                                unsigned long long *bad_row) {
    extern __shared__ __attribute__((aligned(16))) float blk[];  // kBlockRows rows of dim + 4 floats
    __shared__ float inv_s[kBlockRows], scale_s[kBlockRows];
    __shared__ uint32_t mode_s[kBlockRows];
    const uint32_t lane = threadIdx.x;
    const uint64_t row0 = (uint64_t)blockIdx.x * kBlockRows;
    const uint32_t nrows = rows - row0 < (uint64_t)kBlockRows ? (uint32_t)(rows - row0) : kBlockRows;
    const uint32_t nq = dim / 4u;       // quads per row
    const uint32_t rstride = dim + 4u;  // floats per LDS row
    for (uint32_t r = 0; r < nrows; ++r) {
        const float *src = x + (row0 + r) * dim;
        for (uint32_t q0 = 0; q0 < nq; q0 += 64u) {
            if (q0 + lane < nq)
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(src + 4u * (q0 + lane)),
                                                 (__attribute__((address_space(3))) void *)(blk + r * rstride + 4u * q0),
                                                 16, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // max|x| per row: every lane over its quads of the row, then a wave max
    float mx = 0.0f;
    for (uint32_t r = 0; r < nrows; ++r) {
        float m = 0.0f;
        for (uint32_t q = lane; q < nq; q += 64u) {
            const float4 v = *reinterpret_cast<const float4 *>(blk + r * rstride + 4u * q);
            m = fmaxf(fmaxf(m, fabsf(v.x)), fmaxf(fabsf(v.y), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        mx = lane == r ? m : mx;
    }

    // rows: sequential sum of squares in dimension order
    if (lane < nrows) {
        const float4 *rowp = reinterpret_cast<const float4 *>(blk + lane * rstride);
        float norm = 0.0f;
        for (uint32_t t = 0; t < nq; ++t) {
            const float4 v = rowp[t];
            norm = __fadd_rn(norm, __fmul_rn(v.x, v.x));
            norm = __fadd_rn(norm, __fmul_rn(v.y, v.y));
            norm = __fadd_rn(norm, __fmul_rn(v.z, v.z));
            norm = __fadd_rn(norm, __fmul_rn(v.w, v.w));
        }
        // a non-finite value makes the sum non-finite; a non-finite sum of
        // finite values (overflow) is told apart by looking at the values
        bool finite = isfinite(norm);
        if (!finite) {
            finite = true;
            const float *rp = blk + lane * rstride;
            for (uint32_t c = 0; c < dim; ++c) finite &= isfinite(rp[c]);
        }
        const bool zero = !finite || mx == 0.0f;
        const float scale = zero ? 1.0f : __fdiv_rn(mx, max_code);
        const float inv = __fdiv_rn(1.0f, scale);
        scale_s[lane] = scale;
        inv_s[lane] = inv;
        mode_s[lane] = zero ? kRowZero : ((scale >= 1.17549435e-38f && isfinite(inv)) ? kRowFast : kRowExact);
        scales[row0 + lane] = scale;
        norms[row0 + lane] = finite ? norm : 0.0f;
        if (!finite && bad_row) atomicMin(bad_row, (unsigned long long)(row0 + lane));
    }
    __syncthreads();

    // codes: row by row, consecutive lanes on consecutive quads
    for (uint32_t r = 0; r < nrows; ++r) {
        const float inv = inv_s[r], scale = scale_s[r];
        const uint32_t mode = mode_s[r];
        for (uint32_t q = lane; q < nq; q += 64u) {
            const float4 v = *reinterpret_cast<const float4 *>(blk + r * rstride + 4u * q);
            const uint32_t word = quant_code(v.x, inv, scale, mode, max_code) |
                                  (quant_code(v.y, inv, scale, mode, max_code) << 8) |
                                  (quant_code(v.z, inv, scale, mode, max_code) << 16) |
                                  (quant_code(v.w, inv, scale, mode, max_code) << 24);
            *reinterpret_cast<uint32_t *>(codes + (row0 + r) * padded_dim + 4u * q) = word;
        }
    }
    // the rows' padding bytes [dim, padded_dim) are zero
    const uint32_t pad_words = (padded_dim - dim) / 4u;
    for (uint32_t e = lane; e < nrows * pad_words; e += 64u) {
        const uint32_t r = e / pad_words, w = e - r * pad_words;
        *reinterpret_cast<uint32_t *>(codes + (row0 + r) * padded_dim + dim + 4u * w) = 0u;
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
    // rows of 4-aligned width whose block fits LDS: the one-read block kernel
    if (dim % 4u == 0u && dim <= kBlockMaxDim && (reinterpret_cast<uintptr_t>(x) & 15u) == 0u) {
        const uint64_t nblk = (rows + kBlockRows - 1) / kBlockRows;
        if (nblk > 0x7fffffffull) return -2;
        const int lds = (int)(kBlockRows * (dim + 4u) * sizeof(float));
        if (ensure_lds_limit(reinterpret_cast<const void *>(sq8_quantize_block_kernel), lds)) return -1;
        hipLaunchKernelGGL(sq8_quantize_block_kernel, dim3((uint32_t)nblk), dim3(64), lds, stream, x, rows, dim,
                           padded_dim, max_code, codes, scales, norms, (unsigned long long *)bad_row);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
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
