// ghip_gemv.hip -- decode MUL_MAT (batch 1..8 activation rows) for Q4_K, Q6_K
// and Q4_0 weights, dequantizing in registers from 16-byte HBM loads.
//
// Work layout (all three kernels):
//  * A workgroup is one "K-team": W_K wavefronts whose 64*W_K lanes tile the
//    reduction dimension once (8 lanes per 256-block for the K-quants, one
//    lane per pair of 32-blocks for Q4_0).  A lane's K position never changes,
//    so its activation codes are loaded once into registers and reused for
//    every weight row the team visits.
//  * The team walks a tile of rows_per_wg consecutive weight rows; each row is
//    a contiguous span, so a wavefront's loads are fully coalesced.
//  * Per row and activation column a lane forms an exact int32 partial
//    (v_dot4_i32_i8 on unpacked nibbles), scales it in fp32, and the
//    wavefront reduces; the W_K wave partials meet in LDS at the end.
//
// The exact integer sums of the reference (per row, column and block) are
// available through the SUBSUMS instantiations, which reduce the 8 lanes of
// a block in int32 and store them:
//   Q4_K: {iacc, imin} per super-block  (repack.rs:1664-1680)
//   Q6_K: sum_s scale_s * sum (q6-32) q8 per super-block (vec_dot.rs:1000-1036)
//   Q4_0: sum (nib-8) q8 per 32-block   (repack.rs:3351-3378)
#include "ghip_common.h"

constexpr int MAXC = 8;  // activation columns per launch

// ---------------------------------------------------------------- Q4_K x Q8_K
template <int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q4K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                              int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                              int ncols, float *__restrict__ dst, int64_t ldd,
                                              int rows_per_wg, int32_t *__restrict__ sub) {
    extern __shared__ float red[];  // [rows_per_wg][W_K][NC]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int b = 8 * w + (lane >> 3), j = lane & 7, g = j >> 1, h = j & 1;
    const bool valid = b < nb;

    uint4 alo[NC], ahi[NC];
    int bp[NC];
    float da[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if (valid && c < ncols) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b * Q8K_BYTES;
            alo[c] = ld16(A + 4 + 64 * g + 16 * h);
            ahi[c] = ld16(A + 4 + 64 * g + 32 + 16 * h);
            const uint32_t bs = ld4(A + 260 + 4 * j);
            bp[c] = (int)(int16_t)(bs & 0xffff) + (int)(int16_t)(bs >> 16);
            da[c] = __uint_as_float(ld4(A));
        } else {
            alo[c] = ahi[c] = make_uint4(0, 0, 0, 0);
            bp[c] = 0;
            da[c] = 0.0f;
        }
    }

    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = min(rows, r0 + rows_per_wg);
    const uint8_t *wb = W + (int64_t)b * Q4K_BYTES;

    auto row_body = [&](int r, uint4 hdr, uint4 q) {
        const float dw = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
        int slo, shi, sj, mj, mdummy;
        scale_min_k4(hdr.y, hdr.z, hdr.w, 2 * g, slo, mdummy);
        scale_min_k4(hdr.y, hdr.z, hdr.w, 2 * g + 1, shi, mdummy);
        scale_min_k4(hdr.y, hdr.z, hdr.w, j, sj, mj);
        const uint32_t l0 = q.x & 0x0f0f0f0f, l1 = q.y & 0x0f0f0f0f, l2 = q.z & 0x0f0f0f0f, l3 = q.w & 0x0f0f0f0f;
        const uint32_t h0 = (q.x >> 4) & 0x0f0f0f0f, h1 = (q.y >> 4) & 0x0f0f0f0f;
        const uint32_t h2 = (q.z >> 4) & 0x0f0f0f0f, h3 = (q.w >> 4) & 0x0f0f0f0f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int dl = dot4(l3, alo[c].w, dot4(l2, alo[c].z, dot4(l1, alo[c].y, dot4(l0, alo[c].x, 0))));
            const int dh = dot4(h3, ahi[c].w, dot4(h2, ahi[c].z, dot4(h1, ahi[c].y, dot4(h0, ahi[c].x, 0))));
            const int ia = slo * dl + shi * dh;
            const int im = mj * bp[c];
            if (SUBSUMS) {
                const int iab = group8_sum(ia), imb = group8_sum(im);
                if (j == 0 && valid && c < ncols) {
                    int32_t *s = sub + (((int64_t)c * rows + r) * nb + b) * 2;
                    s[0] = iab;
                    s[1] = imb;
                }
            }
            float part = valid ? da[c] * fmaf(dw, (float)ia, -(dmin * (float)im)) : 0.0f;
            part = wave_sum(part);
            if (lane == 0) red[((r - r0) * nw + w) * NC + c] = part;
        }
    };

    int r = r0;
    for (; r + 1 < r1; r += 2) {
        uint4 hA = make_uint4(0, 0, 0, 0), qA = hA, hB = hA, qB = hA;
        if (valid) {
            const uint8_t *pA = wb + (int64_t)r * w_row_bytes;
            const uint8_t *pB = pA + w_row_bytes;
            hA = ld16(pA);
            qA = ld16(pA + 16 + 16 * j);
            hB = ld16(pB);
            qB = ld16(pB + 16 + 16 * j);
        }
        row_body(r, hA, qA);
        row_body(r + 1, hB, qB);
    }
    if (r < r1) {
        uint4 hA = make_uint4(0, 0, 0, 0), qA = hA;
        if (valid) {
            const uint8_t *pA = wb + (int64_t)r * w_row_bytes;
            hA = ld16(pA);
            qA = ld16(pA + 16 + 16 * j);
        }
        row_body(r, hA, qA);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < (r1 - r0) * ncols; idx += blockDim.x) {
        const int rr = idx / ncols, c = idx - rr * ncols;
        float s = 0.0f;
        for (int ww = 0; ww < nw; ww++) s += red[(rr * nw + ww) * NC + c];
        dst[(int64_t)c * ldd + r0 + rr] = s;
    }
}

// ---------------------------------------------------------------- Q6_K x Q8_K
template <int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q6K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                              int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                              int ncols, float *__restrict__ dst, int64_t ldd,
                                              int rows_per_wg, int32_t *__restrict__ sub) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int b = 8 * w + (lane >> 3), j = lane & 7;
    const int jj = j >> 2, p = (j >> 1) & 1, t = j & 1;
    const bool valid = b < nb;
    const int ea = 128 * jj + 32 * p + 16 * t;  // first element of the low-nibble stream
    const int si = 8 * jj + 2 * p + t;          // its scale / bsum index; high stream is si+4

    uint4 ya[NC], yb[NC];
    int bsa[NC], bsb[NC];
    float da[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if (valid && c < ncols) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b * Q8K_BYTES;
            ya[c] = ld16(A + 4 + ea);
            yb[c] = ld16(A + 4 + ea + 64);
            bsa[c] = 32 * (int)(int16_t)ld2(A + 260 + 2 * si);
            bsb[c] = 32 * (int)(int16_t)ld2(A + 260 + 2 * (si + 4));
            da[c] = __uint_as_float(ld4(A));
        } else {
            ya[c] = yb[c] = make_uint4(0, 0, 0, 0);
            bsa[c] = bsb[c] = 0;
            da[c] = 0.0f;
        }
    }
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = min(rows, r0 + rows_per_wg);
    const uint8_t *wb = W + (int64_t)b * Q6K_BYTES;
    const int sh = 2 * p;

    auto row_body = [&](int r, uint4 ql, uint4 qh, int sca, int scb, float dw) {
        uint32_t va[4], vb[4];
        const uint32_t qlv[4] = {ql.x, ql.y, ql.z, ql.w}, qhv[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            va[k] = (qlv[k] & 0x0f0f0f0f) | (((qhv[k] >> sh) & 0x03030303) << 4);
            vb[k] = ((qlv[k] >> 4) & 0x0f0f0f0f) | (((qhv[k] >> (sh + 4)) & 0x03030303) << 4);
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int dA = dot4(va[3], ya[c].w, dot4(va[2], ya[c].z, dot4(va[1], ya[c].y, dot4(va[0], ya[c].x, 0))));
            const int dB = dot4(vb[3], yb[c].w, dot4(vb[2], yb[c].z, dot4(vb[1], yb[c].y, dot4(vb[0], yb[c].x, 0))));
            const int is = sca * (dA - bsa[c]) + scb * (dB - bsb[c]);
            if (SUBSUMS) {
                const int isb = group8_sum(is);
                if (j == 0 && valid && c < ncols) sub[((int64_t)c * rows + r) * nb + b] = isb;
            }
            float part = valid ? (dw * (float)is) * da[c] : 0.0f;
            part = wave_sum(part);
            if (lane == 0) red[((r - r0) * nw + w) * NC + c] = part;
        }
    };
    auto load = [&](int r, uint4 &ql, uint4 &qh, int &sca, int &scb, float &dw) {
        if (valid) {
            const uint8_t *blk = wb + (int64_t)r * w_row_bytes;
            ql = ld16(blk + 64 * jj + 32 * p + 16 * t);
            qh = ld16(blk + 128 + 32 * jj + 16 * t);
            sca = (int)(int8_t)blk[192 + si];
            scb = (int)(int8_t)blk[196 + si];
            dw = h2f(ld2(blk + 208));
        } else {
            ql = qh = make_uint4(0, 0, 0, 0);
            sca = scb = 0;
            dw = 0.0f;
        }
    };
    int r = r0;
    for (; r + 1 < r1; r += 2) {
        uint4 qlA, qhA, qlB, qhB;
        int saA, sbA, saB, sbB;
        float dA, dB;
        load(r, qlA, qhA, saA, sbA, dA);
        load(r + 1, qlB, qhB, saB, sbB, dB);
        row_body(r, qlA, qhA, saA, sbA, dA);
        row_body(r + 1, qlB, qhB, saB, sbB, dB);
    }
    if (r < r1) {
        uint4 qlA, qhA;
        int saA, sbA;
        float dA;
        load(r, qlA, qhA, saA, sbA, dA);
        row_body(r, qlA, qhA, saA, sbA, dA);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < (r1 - r0) * ncols; idx += blockDim.x) {
        const int rr = idx / ncols, c = idx - rr * ncols;
        float s = 0.0f;
        for (int ww = 0; ww < nw; ww++) s += red[(rr * nw + ww) * NC + c];
        dst[(int64_t)c * ldd + r0 + rr] = s;
    }
}

// ---------------------------------------------------------------- Q4_0 x Q8_0
// One lane per pair of 32-blocks (36 bytes, 64 elements).
template <int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q4_0_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                               int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                               int ncols, float *__restrict__ dst, int64_t ldd,
                                               int rows_per_wg, int32_t *__restrict__ sub) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int pr = 64 * w + lane;  // pair index
    const int b0 = 2 * pr, b1 = 2 * pr + 1;
    const bool v0 = b0 < nb, v1 = b1 < nb;

    uint4 y0l[NC], y0h[NC], y1l[NC], y1h[NC];
    int sy0[NC], sy1[NC];
    float d0[NC], d1[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        y0l[c] = y0h[c] = y1l[c] = y1h[c] = make_uint4(0, 0, 0, 0);
        sy0[c] = sy1[c] = 0;
        d0[c] = d1[c] = 0.0f;
        if (c < ncols && v0) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b0 * Q8_0_BYTES;
            d0[c] = h2f(ld2(A));
            y0l[c] = ld16(A + 2);
            y0h[c] = ld16(A + 18);
            const uint32_t one = 0x01010101u;
            sy0[c] = 8 * dot4(y0l[c].x, one, dot4(y0l[c].y, one, dot4(y0l[c].z, one, dot4(y0l[c].w, one,
                     dot4(y0h[c].x, one, dot4(y0h[c].y, one, dot4(y0h[c].z, one, dot4(y0h[c].w, one, 0))))))));
        }
        if (c < ncols && v1) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b1 * Q8_0_BYTES;
            d1[c] = h2f(ld2(A));
            y1l[c] = ld16(A + 2);
            y1h[c] = ld16(A + 18);
            const uint32_t one = 0x01010101u;
            sy1[c] = 8 * dot4(y1l[c].x, one, dot4(y1l[c].y, one, dot4(y1l[c].z, one, dot4(y1l[c].w, one,
                     dot4(y1h[c].x, one, dot4(y1h[c].y, one, dot4(y1h[c].z, one, dot4(y1h[c].w, one, 0))))))));
        }
    }
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = min(rows, r0 + rows_per_wg);
    const uint8_t *wb = W + (int64_t)pr * 36;

    auto load = [&](int r, uint4 &a, uint4 &bq, uint32_t &c8) {
        const uint8_t *p = wb + (int64_t)r * w_row_bytes;
        if (v1) {
            a = ld16(p);
            bq = ld16(p + 16);
            c8 = ld4(p + 32);
        } else if (v0) {
            a = ld16(p);
            const uint16_t t = ld2(p + 16);
            bq = make_uint4(t, 0, 0, 0);
            c8 = 0;
        } else {
            a = bq = make_uint4(0, 0, 0, 0);
            c8 = 0;
        }
    };
    auto row_body = [&](int r, uint4 a, uint4 bq, uint32_t c8) {
        const float dw0 = h2f(a.x), dw1 = h2f(bq.x >> 16);
        const uint32_t q0[4] = {__builtin_amdgcn_alignbyte(a.y, a.x, 2), __builtin_amdgcn_alignbyte(a.z, a.y, 2),
                                __builtin_amdgcn_alignbyte(a.w, a.z, 2), __builtin_amdgcn_alignbyte(bq.x, a.w, 2)};
        const uint32_t q1[4] = {bq.y, bq.z, bq.w, c8};
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int s0 = dot4(q0[3] & 0x0f0f0f0f, y0l[c].w, dot4(q0[2] & 0x0f0f0f0f, y0l[c].z,
                           dot4(q0[1] & 0x0f0f0f0f, y0l[c].y, dot4(q0[0] & 0x0f0f0f0f, y0l[c].x,
                           dot4((q0[3] >> 4) & 0x0f0f0f0f, y0h[c].w, dot4((q0[2] >> 4) & 0x0f0f0f0f, y0h[c].z,
                           dot4((q0[1] >> 4) & 0x0f0f0f0f, y0h[c].y, dot4((q0[0] >> 4) & 0x0f0f0f0f, y0h[c].x,
                           -sy0[c]))))))));
            const int s1 = dot4(q1[3] & 0x0f0f0f0f, y1l[c].w, dot4(q1[2] & 0x0f0f0f0f, y1l[c].z,
                           dot4(q1[1] & 0x0f0f0f0f, y1l[c].y, dot4(q1[0] & 0x0f0f0f0f, y1l[c].x,
                           dot4((q1[3] >> 4) & 0x0f0f0f0f, y1h[c].w, dot4((q1[2] >> 4) & 0x0f0f0f0f, y1h[c].z,
                           dot4((q1[1] >> 4) & 0x0f0f0f0f, y1h[c].y, dot4((q1[0] >> 4) & 0x0f0f0f0f, y1h[c].x,
                           -sy1[c]))))))));
            if (SUBSUMS && c < ncols) {
                int32_t *s = sub + ((int64_t)c * rows + r) * nb;
                if (v0) s[b0] = s0;
                if (v1) s[b1] = s1;
            }
            float part = v0 ? (float)s0 * (dw0 * d0[c]) : 0.0f;
            if (v1) part = fmaf((float)s1, dw1 * d1[c], part);
            part = wave_sum(part);
            if (lane == 0) red[((r - r0) * nw + w) * NC + c] = part;
        }
    };
    int r = r0;
    for (; r + 1 < r1; r += 2) {
        uint4 aA, bA, aB, bB;
        uint32_t cA, cB;
        load(r, aA, bA, cA);
        load(r + 1, aB, bB, cB);
        row_body(r, aA, bA, cA);
        row_body(r + 1, aB, bB, cB);
    }
    if (r < r1) {
        uint4 aA, bA;
        uint32_t cA;
        load(r, aA, bA, cA);
        row_body(r, aA, bA, cA);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < (r1 - r0) * ncols; idx += blockDim.x) {
        const int rr = idx / ncols, c = idx - rr * ncols;
        float s = 0.0f;
        for (int ww = 0; ww < nw; ww++) s += red[(rr * nw + ww) * NC + c];
        dst[(int64_t)c * ldd + r0 + rr] = s;
    }
}

#define GEMV_ARGS                                                                                     \
    const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act, \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int rows_per_wg,          \
        int32_t *__restrict__ sub
#define GEMV_PASS W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, rows_per_wg, sub

#define GEMV_INST(name, impl, NC)                                                                  \
    extern "C" __global__ void __launch_bounds__(512) name##_c##NC(GEMV_ARGS) {                  \
        impl<NC, false>(GEMV_PASS);                                                                \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) name##_sub_c##NC(GEMV_ARGS) {              \
        impl<NC, true>(GEMV_PASS);                                                                 \
    }
#define GEMV_ALL(name, impl) \
    GEMV_INST(name, impl, 1) GEMV_INST(name, impl, 2) GEMV_INST(name, impl, 4) GEMV_INST(name, impl, 8)

GEMV_ALL(ghip_gemv_q4_K, gemv_q4K_impl)
GEMV_ALL(ghip_gemv_q6_K, gemv_q6K_impl)
GEMV_ALL(ghip_gemv_q4_0, gemv_q4_0_impl)
