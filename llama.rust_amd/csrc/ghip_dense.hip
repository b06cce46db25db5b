// ghip_dense.hip -- MUL_MAT with F32, F16 and BF16 weights (decode kernel,
// any number of activation rows in groups of at most 8).
//
// Reference (compute.rs:1680-1745; vec_dot.rs:1700-1727): F16 / BF16 weights
// take the f32 activation row rounded to the weight type (round to nearest
// even), so every product of two f16 (two bf16) values is exact in f32; F32
// weights multiply the f32 activation as it is.  Products are accumulated in
// f32 here (lane chains, then the workgroup's tree), the reference in its own
// f32 / f64 order: the results agree to fp32 summation rounding.
//
// Workgroup: 256 threads, 8 weight rows.  Thread j walks the row in chunks of
// 8 elements (j, j + 256, ...), loads each chunk of the 8 rows once (16 bytes
// per row for F16 / BF16, 32 for F32) and the matching activation chunk of
// every column, and keeps 8 x NC f32 partial sums.
#include "ghip_common.h"

namespace {

constexpr int WT_F32 = 0, WT_F16 = 1, WT_BF16 = 30;
constexpr int DRB = 8;  // weight rows per workgroup

DEV float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
// f32 -> bf16 -> f32, round to nearest even (NaN stays NaN)
DEV float round_bf16(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float((u | 0x00400000u) & 0xffff0000u);
    return __uint_as_float((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
}
DEV float round_f16(float x) { return (float)(_Float16)x; }

template <int WT> DEV float round_act(float x) {
    if constexpr (WT == WT_F16) return round_f16(x);
    else if constexpr (WT == WT_BF16) return round_bf16(x);
    else return x;
}
// element e of a weight row
template <int WT> DEV float wval(const uint8_t *row, int e) {
    if constexpr (WT == WT_F32) return __uint_as_float(ld4(row + 4 * e));
    else if constexpr (WT == WT_F16) return h2f(ld2(row + 2 * e));
    else return bf16_to_f32(ld2(row + 2 * e));
}
// the 8 elements of chunk c of a row (VEC: the row's chunks are 16-byte aligned)
template <int WT, bool VEC> DEV void wchunk(const uint8_t *row, int c, float *w) {
    if constexpr (VEC && WT != WT_F32) {
        const uint4 v = ld16(row + 16 * c);
        const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if constexpr (WT == WT_F16) {
                w[2 * k] = h2f(x[k] & 0xffffu);
                w[2 * k + 1] = h2f(x[k] >> 16);
            } else {
                w[2 * k] = bf16_to_f32(x[k] & 0xffffu);
                w[2 * k + 1] = bf16_to_f32(x[k] >> 16);
            }
        }
    } else if constexpr (VEC) {
        const uint4 a = ld16(row + 32 * c), b = ld16(row + 32 * c + 16);
        const uint32_t x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 8; k++) w[k] = __uint_as_float(x[k]);
    } else {
#pragma unroll
        for (int k = 0; k < 8; k++) w[k] = wval<WT>(row, 8 * c + k);
    }
}

template <int WT, int NC, bool VEC>
__device__ __forceinline__ void gemv_dense_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int K,
                                                const float *__restrict__ x, int64_t x_stride, int ncols,
                                                float *__restrict__ dst, int64_t ldd) {
    __shared__ float red[4][DRB * NC];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = (int)blockIdx.x * DRB;
    const int nrow = min(DRB, rows - r0);
    float acc[DRB][NC];
#pragma unroll
    for (int r = 0; r < DRB; r++)
#pragma unroll
        for (int c = 0; c < NC; c++) acc[r][c] = 0.0f;
    const int nch = K / 8;
    for (int ch = tid; ch < nch; ch += 256) {
        float xv[NC][8];
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float *xc = x + (int64_t)min(c, ncols - 1) * x_stride + 8 * ch;
            const uint4 a = ld16(reinterpret_cast<const uint8_t *>(xc)), b = ld16(reinterpret_cast<const uint8_t *>(xc + 4));
            const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int k = 0; k < 8; k++) xv[c][k] = round_act<WT>(__uint_as_float(u[k]));
        }
#pragma unroll
        for (int r = 0; r < DRB; r++) {
            float w[8];
            wchunk<WT, VEC>(W + (int64_t)(r0 + min(r, nrow - 1)) * w_row_bytes, ch, w);
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int k = 0; k < 8; k++) acc[r][c] = fmaf(w[k], xv[c][k], acc[r][c]);
        }
    }
    // the K % 8 tail, one element per thread
    for (int e = 8 * nch + tid; e < K; e += 256) {
#pragma unroll
        for (int r = 0; r < DRB; r++) {
            const float w = wval<WT>(W + (int64_t)(r0 + min(r, nrow - 1)) * w_row_bytes, e);
#pragma unroll
            for (int c = 0; c < NC; c++)
                acc[r][c] = fmaf(w, round_act<WT>(x[(int64_t)min(c, ncols - 1) * x_stride + e]), acc[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < DRB; r++)
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float s = wave_sum_dpp(acc[r][c]);
            if (lane == 0) red[wave][r * NC + c] = s;
        }
    __syncthreads();
    if (tid < DRB * NC) {
        const int r = tid / NC, c = tid - r * NC;
        if (r < nrow && c < ncols)
            dst[(int64_t)c * ldd + r0 + r] = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
    }
}

}  // namespace

#define DENSE_INST(TN, WT, NC)                                                                                      \
    extern "C" __global__ void __launch_bounds__(256)                                                               \
        ghip_gemv_dense_##TN##_c##NC(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int K,            \
                                     const float *__restrict__ x, int64_t x_stride, int ncols,                      \
                                     float *__restrict__ dst, int64_t ldd, int vec) {                               \
        if (vec) gemv_dense_impl<WT, NC, true>(W, w_row_bytes, rows, K, x, x_stride, ncols, dst, ldd);              \
        else gemv_dense_impl<WT, NC, false>(W, w_row_bytes, rows, K, x, x_stride, ncols, dst, ldd);                 \
    }
#define DENSE_TYPE(TN, WT) DENSE_INST(TN, WT, 1) DENSE_INST(TN, WT, 2) DENSE_INST(TN, WT, 4) DENSE_INST(TN, WT, 8)
DENSE_TYPE(f32, WT_F32)
DENSE_TYPE(f16, WT_F16)
DENSE_TYPE(bf16, WT_BF16)
