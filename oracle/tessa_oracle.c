/*
 * tessa_oracle.c -- CPU restatement of the reference TESSA operator semantics.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
 * Nothing in the product path (shear_amd/) links or calls this file.
 *
 * Build with -ffp-contract=off and without -ffast-math: every float operation
 * below is one IEEE-754 binary32 operation in the order the reference writes
 * it (Rust never contracts a*b+c into an FMA, and the reference CUDA pins the
 * leaf epilogue with __fadd_rn/__fmul_rn).
 */
#include "tessa_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- SQ8 --- */

size_t orc_sq8_padded_dim(size_t dim, size_t k_align) {
    /* dco_sq_int8.rs:1216-1224: dim.div_ceil(max(k_align,1)) * k_align */
    if (dim == 0) return 0;
    if (k_align == 0) k_align = 1;
    return (dim + k_align - 1) / k_align * k_align;
}

int orc_sq8_quantize(const float *x, size_t rows, size_t dim, size_t padded_dim,
                     unsigned bits, int8_t *codes, float *scales, float *norms,
                     size_t *bad_row) {
    /* dco_sq_int8.rs:1325-1329 sq_int8_max_code_for_bits, bits in [4, 8] */
    if (bits < 4 || bits > 8 || dim == 0 || padded_dim < dim) return -2;
    const float max_code = (float)((1u << (bits - 1)) - 1u);
    for (size_t row = 0; row < rows; ++row) {
        const float *in = x + row * dim;
        int8_t *out = codes + row * padded_dim;
        memset(out, 0, padded_dim);
        /* dco_sq_int8.rs:1446-1456: one pass, max |x| and a sequential f32
         * sum of squares; any non-finite value is an error. */
        float max_abs = 0.0f;
        float norm = 0.0f;
        for (size_t d = 0; d < dim; ++d) {
            float v = in[d];
            if (!isfinite(v)) {
                if (bad_row) *bad_row = row;
                return -1;
            }
            float a = fabsf(v);
            if (a > max_abs) max_abs = a;
            float sq = v * v;
            norm = norm + sq;
        }
        /* :1458-1460 all-zero row: scale 1, codes 0 */
        if (max_abs == 0.0f) {
            scales[row] = 1.0f;
            norms[row] = norm;
            continue;
        }
        /* :1462-1466 scale = max_abs / max_code; code = clamp(round(v/scale)) */
        float scale = max_abs / max_code;
        for (size_t d = 0; d < dim; ++d) {
            float q = roundf(in[d] / scale); /* half away from zero, as Rust */
            if (q < -max_code) q = -max_code;
            if (q > max_code) q = max_code;
            out[d] = (int8_t)q;
        }
        scales[row] = scale;
        norms[row] = norm;
    }
    return 0;
}

/* ---------------------------------------------------------------- dots --- */

int32_t orc_sq8_dot_scalar(const int8_t *a, const int8_t *b, size_t n) {
    /* dco_sq_int8.rs:2685-2691 */
    int32_t s = 0;
    for (size_t i = 0; i < n; ++i) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

#if defined(__x86_64__)
__attribute__((target("avx2"))) static int32_t dot_avx2(const int8_t *a,
                                                        const int8_t *b,
                                                        size_t n) {
    __m256i acc = _mm256_setzero_si256();
    size_t i = 0;
    for (; i + 16 <= n; i += 16) {
        __m256i va = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + i)));
        __m256i vb = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + i)));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(va, vb));
    }
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(acc), _mm256_extracti128_si256(acc, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    int32_t r = _mm_cvtsi128_si32(s);
    for (; i < n; ++i) r += (int32_t)a[i] * (int32_t)b[i];
    return r;
}

/* u8 x s8 VNNI with the +128 bias on the left operand: sum((a^0x80)*b) is
 * sum(a*b) + 128*sum(b); vpdpbusd accumulates without saturation. */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static int32_t
dot_vnni(const int8_t *a, const int8_t *b, size_t n) {
    const __m512i bias = _mm512_set1_epi8((char)0x80);
    const __m512i ones = _mm512_set1_epi8(1);
    __m512i acc = _mm512_setzero_si512();
    __m512i sb = _mm512_setzero_si512();
    size_t i = 0;
    for (; i + 64 <= n; i += 64) {
        __m512i va = _mm512_xor_si512(_mm512_loadu_si512((const void *)(a + i)), bias);
        __m512i vb = _mm512_loadu_si512((const void *)(b + i));
        acc = _mm512_dpbusd_epi32(acc, va, vb);
        sb = _mm512_dpbusd_epi32(sb, ones, vb);
    }
    if (i < n) {
        __mmask64 m = (n - i >= 64) ? ~(__mmask64)0 : (((__mmask64)1 << (n - i)) - 1);
        __m512i va = _mm512_xor_si512(_mm512_maskz_loadu_epi8(m, a + i), bias);
        __m512i vb = _mm512_maskz_loadu_epi8(m, b + i);
        acc = _mm512_dpbusd_epi32(acc, va, vb); /* masked-off b bytes are 0 */
        sb = _mm512_dpbusd_epi32(sb, ones, vb);
    }
    return _mm512_reduce_add_epi32(acc) - 128 * _mm512_reduce_add_epi32(sb);
}
#endif

static int g_dot_kernel = -1;

static int detect_dot_kernel(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw"))
        return 2;
    if (__builtin_cpu_supports("avx2")) return 1;
#endif
    return 0;
}

int orc_sq8_dot_kernel(void) {
    if (g_dot_kernel < 0) g_dot_kernel = detect_dot_kernel();
    return g_dot_kernel;
}

int orc_sq8_set_dot_kernel(int kernel) {
    int prev = orc_sq8_dot_kernel();
    int best = detect_dot_kernel();
    if (kernel < 0 || kernel > best) kernel = best;
    g_dot_kernel = kernel;
    return prev;
}

int32_t orc_sq8_dot(const int8_t *a, const int8_t *b, size_t n) {
#if defined(__x86_64__)
    switch (orc_sq8_dot_kernel()) {
    case 2: return dot_vnni(a, b, n);
    case 1: return dot_avx2(a, b, n);
    default: break;
    }
#endif
    return orc_sq8_dot_scalar(a, b, n);
}

/* ------------------------------------------------------------ distances --- */

float orc_sq8_leaf_l2(int32_t dot, float row_scale, float row_norm,
                      float col_scale, float col_norm) {
    /* compute_backend.rs:8994-8997:
     * __fadd_rn(__fadd_rn(rn, cn), __fmul_rn(-2, __fmul_rn(__fmul_rn(rs, cs), dot))) */
    float sc = row_scale * col_scale;
    float prod = sc * (float)dot;
    float twice = -2.0f * prod;
    float nsum = row_norm + col_norm;
    float d = nsum + twice;
    if (d <= 0.0f) d = 0.0f;
    return d;
}

float orc_sq8_assign_l2(int32_t dot, float point_scale, float point_norm,
                        float leader_scale, float leader_norm) {
    /* rbc_partition.rs:17637: left_norm + right_norm - 2.0*ls*rs*dot, Rust
     * evaluates the product chain left to right and never contracts. */
    float a = 2.0f * point_scale;
    float b = a * leader_scale;
    float c = b * (float)dot;
    float nsum = point_norm + leader_norm;
    float d = nsum - c;
    if (d <= 0.0f) d = 0.0f;
    return d;
}

/* ------------------------------------------------------------- top-k --- */

int orc_beats(float dc, uint32_t idc, float ds, uint32_t ids) {
    /* mod.rs:417-428: |dc-ds| <= eps ? idc < ids : dc.total_cmp(ds) == Less.
     * Distances here are finite and >= 0 (or the FLT_MAX/INF empty marker),
     * where total_cmp's Less is plain '<'. */
    float delta = dc - ds;
    if (fabsf(delta) <= ORC_TIE_EPS) return idc < ids;
    return dc < ds;
}

void orc_rowtopk_push(uint32_t k, float d, uint32_t id, float *best_d,
                      uint32_t *best_id, uint32_t *len) {
    /* leaf_build.rs:913-951 */
    if (k == 0) return;
    if (*len < k) {
        uint32_t i = *len;
        while (i > 0 && orc_beats(d, id, best_d[i - 1], best_id[i - 1])) {
            best_d[i] = best_d[i - 1];
            best_id[i] = best_id[i - 1];
            --i;
        }
        best_d[i] = d;
        best_id[i] = id;
        *len += 1;
        return;
    }
    if (!orc_beats(d, id, best_d[k - 1], best_id[k - 1])) return;
    uint32_t i = k - 1;
    while (i > 0 && orc_beats(d, id, best_d[i - 1], best_id[i - 1])) {
        best_d[i] = best_d[i - 1];
        best_id[i] = best_id[i - 1];
        --i;
    }
    best_d[i] = d;
    best_id[i] = id;
}

static int set_threads(int threads) {
#ifdef _OPENMP
    int n = threads > 0 ? threads : omp_get_max_threads();
    return n < 1 ? 1 : n;
#else
    (void)threads;
    return 1;
#endif
}

int orc_leaf_topk_batch(const int8_t *codes, const float *scales,
                        const float *norms, const uint32_t *global_ids,
                        size_t resident_rows, size_t padded_dim,
                        const uint32_t *members, const uint64_t *member_offsets,
                        const uint32_t *member_counts,
                        const uint64_t *output_offsets, size_t leaf_count,
                        uint32_t k, uint32_t *out_ids, float *out_dists,
                        int threads) {
    if (k == 0 || k > 32 || padded_dim == 0) return -2;
    for (size_t leaf = 0; leaf < leaf_count; ++leaf) {
        const uint32_t *m = members + member_offsets[leaf];
        for (uint32_t r = 0; r < member_counts[leaf]; ++r)
            if (m[r] >= resident_rows) return -3;
    }
    int nt = set_threads(threads);
    int err = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
    for (long long leaf = 0; leaf < (long long)leaf_count; ++leaf) {
        const uint32_t *m = members + member_offsets[leaf];
        const uint32_t n = member_counts[leaf];
        const uint32_t keff = n > 0 ? (k < n - 1 ? k : n - 1) : 0;
        for (uint32_t row = 0; row < n; ++row) {
            float bd[32];
            uint32_t bid[32];
            uint32_t len = 0;
            const uint32_t ri = m[row];
            const int8_t *rc = codes + (size_t)ri * padded_dim;
            /* leaf_build.rs:1573-1590: every other member in member order */
            for (uint32_t col = 0; col < n; ++col) {
                if (col == row) continue;
                const uint32_t cj = m[col];
                int32_t dot = orc_sq8_dot(rc, codes + (size_t)cj * padded_dim, padded_dim);
                float d = orc_sq8_leaf_l2(dot, scales[ri], norms[ri], scales[cj], norms[cj]);
                orc_rowtopk_push(keff, d, global_ids[cj], bd, bid, &len);
            }
            uint64_t out = output_offsets[leaf] + (uint64_t)row * k;
            for (uint32_t s = 0; s < k; ++s) {
                out_ids[out + s] = s < len ? bid[s] : ORC_EMPTY_ID;
                out_dists[out + s] = s < len ? bd[s] : FLT_MAX;
            }
        }
    }
    return err;
}

/* ---------------------------------------------------------- assignment --- */

uint64_t orc_hash64(uint64_t v) {
    /* compute_backend.rs:5983-5989 */
    v ^= v >> 30;
    v *= 0xbf58476d1ce4e5b9ull;
    v ^= v >> 27;
    v *= 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

uint64_t orc_assign_tie_key(uint32_t point, uint32_t leader) {
    /* compute_backend.rs:6513-6522 */
    return orc_hash64((((uint64_t)point) << 32) ^ (uint64_t)leader ^ 0x9e3779b97f4a7c15ull);
}

int orc_assign_before(float d, uint32_t point, uint32_t leader, float od,
                         uint32_t oleader) {
    /* compute_backend.rs:6541-6568: eps tie -> (tie key, leader) order */
    if (fabsf(d - od) <= ORC_TIE_EPS) {
        uint64_t ck = orc_assign_tie_key(point, leader);
        uint64_t ok = orc_assign_tie_key(point, oleader);
        return ck < ok || (ck == ok && leader < oleader);
    }
    return d < od;
}

static int check_assign_tasks(size_t resident_rows, const uint32_t *members,
                              const uint32_t *leaders,
                              const uint32_t *member_offsets,
                              const uint32_t *member_counts,
                              const uint32_t *leader_offsets,
                              const uint32_t *leader_counts,
                              const uint32_t *r_h, size_t task_count) {
    for (size_t t = 0; t < task_count; ++t) {
        if (r_h[t] == 0 || r_h[t] > 4 || leader_counts[t] < r_h[t]) return -2;
        for (uint32_t i = 0; i < member_counts[t]; ++i)
            if (members[member_offsets[t] + i] >= resident_rows) return -3;
        for (uint32_t i = 0; i < leader_counts[t]; ++i)
            if (leaders[leader_offsets[t] + i] >= resident_rows) return -3;
    }
    return 0;
}

int orc_assign_replay(const int8_t *codes, const float *scales,
                      const float *norms, const uint32_t *global_ids,
                      size_t resident_rows, size_t padded_dim,
                      const uint32_t *members, const uint32_t *leaders,
                      const uint32_t *member_offsets,
                      const uint32_t *member_counts,
                      const uint32_t *leader_offsets,
                      const uint32_t *leader_counts, const uint32_t *r_h,
                      const uint64_t *output_offsets, size_t task_count,
                      uint32_t *out_ids, float *out_dists, int threads) {
    int rc = check_assign_tasks(resident_rows, members, leaders, member_offsets,
                                member_counts, leader_offsets, leader_counts, r_h,
                                task_count);
    if (rc) return rc;
    int nt = set_threads(threads);
    for (size_t t = 0; t < task_count; ++t) {
        const uint32_t *tm = members + member_offsets[t];
        const uint32_t *tl = leaders + leader_offsets[t];
        const uint32_t L = leader_counts[t];
#pragma omp parallel for schedule(static) num_threads(nt)
        for (long long row = 0; row < (long long)member_counts[t]; ++row) {
            const uint32_t p = tm[row];
            /* :6357-6368 reset: FLT_MAX / 0xffffffff; local fanout 4 (:15805) */
            float bd[4] = {FLT_MAX, FLT_MAX, FLT_MAX, FLT_MAX};
            uint32_t bs[4] = {ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID};
            uint32_t bl[4] = {ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID, ORC_EMPTY_ID};
            for (uint32_t s = 0; s < L; ++s) {
                const uint32_t l = tl[s];
                int32_t dot = orc_sq8_dot(codes + (size_t)p * padded_dim,
                                          codes + (size_t)l * padded_dim, padded_dim);
                float d = orc_sq8_assign_l2(dot, scales[p], norms[p], scales[l], norms[l]);
                if (!orc_assign_before(d, p, l, bd[3], bl[3])) continue;
                uint32_t pos = 3;
                while (pos > 0 && orc_assign_before(d, p, l, bd[pos - 1], bl[pos - 1])) {
                    bd[pos] = bd[pos - 1];
                    bs[pos] = bs[pos - 1];
                    bl[pos] = bl[pos - 1];
                    --pos;
                }
                bd[pos] = d;
                bs[pos] = s;
                bl[pos] = l;
            }
            /* :15912-15940 output: leader global id and recomputed distance */
            for (uint32_t r = 0; r < r_h[t]; ++r) {
                uint64_t o = output_offsets[t] + (uint64_t)row * r_h[t] + r;
                const uint32_t l = tl[bs[r]];
                int32_t dot = orc_sq8_dot(codes + (size_t)p * padded_dim,
                                          codes + (size_t)l * padded_dim, padded_dim);
                out_ids[o] = global_ids[l];
                out_dists[o] = orc_sq8_assign_l2(dot, scales[p], norms[p], scales[l], norms[l]);
            }
        }
    }
    return 0;
}

int orc_assign_strict(const int8_t *codes, const float *scales,
                      const float *norms, const uint32_t *global_ids,
                      size_t resident_rows, size_t padded_dim,
                      const uint32_t *members, const uint32_t *leaders,
                      const uint32_t *member_offsets,
                      const uint32_t *member_counts,
                      const uint32_t *leader_offsets,
                      const uint32_t *leader_counts, const uint32_t *r_h,
                      const uint64_t *output_offsets, size_t task_count,
                      uint32_t *out_ids, float *out_dists, int threads) {
    int rc = check_assign_tasks(resident_rows, members, leaders, member_offsets,
                                member_counts, leader_offsets, leader_counts, r_h,
                                task_count);
    if (rc) return rc;
    int nt = set_threads(threads);
    for (size_t t = 0; t < task_count; ++t) {
        const uint32_t *tm = members + member_offsets[t];
        const uint32_t *tl = leaders + leader_offsets[t];
        const uint32_t L = leader_counts[t];
        const uint32_t R = r_h[t];
#pragma omp parallel for schedule(static) num_threads(nt)
        for (long long row = 0; row < (long long)member_counts[t]; ++row) {
            const uint32_t p = tm[row];
            float bd[4];
            uint32_t bg[4];
            uint32_t len = 0;
            for (uint32_t s = 0; s < L; ++s) {
                const uint32_t l = tl[s];
                int32_t dot = orc_sq8_dot(codes + (size_t)p * padded_dim,
                                          codes + (size_t)l * padded_dim, padded_dim);
                float d = orc_sq8_assign_l2(dot, scales[p], norms[p], scales[l], norms[l]);
                uint32_t g = global_ids[l];
                /* rbc_partition.rs:17714-17733: (dist total order, global id) */
                uint32_t i = len < R ? len : R;
                if (len >= R && !(d < bd[R - 1] || (d == bd[R - 1] && g < bg[R - 1])))
                    continue;
                if (len >= R) i = R - 1;
                while (i > 0 && (d < bd[i - 1] || (d == bd[i - 1] && g < bg[i - 1]))) {
                    bd[i] = bd[i - 1];
                    bg[i] = bg[i - 1];
                    --i;
                }
                bd[i] = d;
                bg[i] = g;
                if (len < R) ++len;
            }
            for (uint32_t r = 0; r < R; ++r) {
                uint64_t o = output_offsets[t] + (uint64_t)row * R + r;
                out_ids[o] = r < len ? bg[r] : ORC_EMPTY_ID;
                out_dists[o] = r < len ? bd[r] : FLT_MAX;
            }
        }
    }
    return 0;
}
