// ghip_wquant.hip -- weight quantizers on the GPU (the no-imatrix path of
// ggml_quantize_chunk: tools/quantize/src/rows.rs:63 -> quantize_row_*_ref).
//
// One thread per block; each runs the reference's serial per-block search, so
// the bytes equal the CPU quantizers':
//   Q4_0   quants.rs:124-152
//   Q4_K   quants_k.rs:1861-1950 (make_qkx2_quants :1396)
//   Q6_K   quants_k.rs:2058-2133 (make_qx_quants :1170)
//   MXFP4  upstream ggml quantize_row_mxfp4_ref (the reference has none)
// Compiled with -ffp-contract=off and using only correctly rounded +,-,*,/,
// sqrt, so every float op rounds exactly as on the CPU.
#include "ghip_common.h"

DEV int nearest_int(float f) { return (int)rintf(f); }  // quants.rs:13 (RNE, |f| < 2^22)
DEV uint16_t f2h(float f) { return f2h_rn(f); }
// Correctly rounded fp32 sqrt (the CPU's sqrtss): the hardware estimate is
// within an ulp, so pick among its neighbours the one whose exact square (in
// double, 48 significant bits) is closest to x.  A tie is impossible: the
// midpoint of two floats squared needs more than 24 bits.
DEV float sqrt_crt(float x) {
    if (!(x > 0.0f) || x == __builtin_inff()) return sqrtf(x);
    const float r = sqrtf(x);
    const float c[3] = {__uint_as_float(__float_as_uint(r) - 1), r, __uint_as_float(__float_as_uint(r) + 1)};
    float best = r;
    double be = 1e300;
    for (int i = 0; i < 3; i++) {
        const double e = fabs((double)c[i] * (double)c[i] - (double)x);
        if (e < be) { be = e; best = c[i]; }
    }
    return best;
}
DEV int imin(int a, int b) { return a < b ? a : b; }
DEV int imax(int a, int b) { return a > b ? a : b; }

extern "C" __global__ void __launch_bounds__(256)
ghip_wquant_q4_0(const float *__restrict__ x, int64_t nblocks, uint8_t *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float *xb = x + i * 32;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float v = xb[j];
        if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
    }
    const float d = __fdiv_rn(max, -8.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint8_t out[18];
    const uint16_t dh = f2h(d);
    __builtin_memcpy(out, &dh, 2);
    for (int j = 0; j < 16; j++) {
        const float x0 = __fmul_rn(xb[j], id), x1 = __fmul_rn(xb[16 + j], id);
        const int xi0 = imin((int)(int8_t)(int)__fadd_rn(x0, 8.5f), 15);
        const int xi1 = imin((int)(int8_t)(int)__fadd_rn(x1, 8.5f), 15);
        out[2 + j] = (uint8_t)((xi0 & 0xf) | ((xi1 & 0xf) << 4));
    }
    __builtin_memcpy(y + i * 18, out, 18);
}

// quants_k.rs:1396-1490
DEV float make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *the_min,
                           uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0.0f) min = 0.0f;
    if (max == min) {
        for (int i = 0; i < n; i++) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = __fdiv_rn((float)nmax, max - min);
    float scale = __fdiv_rn(1.0f, iscale);
    float best_error = 0.0f;
    for (int i = 0; i < n; i++) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)imax(0, imin(nmax, l));
        float diff = scale * (float)L[i] + min - x[i];
        diff = diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) { *the_min = -min; return scale; }
    for (int is = 0; is <= nstep; is++) {
        iscale = __fdiv_rn(rmin + rdelta * (float)is + (float)nmax, max - min);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; i++) {
            const int l = imax(0, imin(nmax, nearest_int(iscale * (x[i] - min))));
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * (float)l;
            sum_l2 += w * (float)l * (float)l;
            sum_xl += w * (float)l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0.0f) {
            float this_scale = __fdiv_rn(sum_w * sum_xl - sum_x * sum_l, D);
            float this_min = __fdiv_rn(sum_l2 * sum_x - sum_l * sum_xl, D);
            if (this_min > 0.0f) { this_min = 0.0f; this_scale = __fdiv_rn(sum_xl, sum_l2); }
            float cur_error = 0.0f;
            for (int i = 0; i < n; i++) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; i++) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

DEV void get_scale_min_k4_b(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

extern "C" __global__ void __launch_bounds__(64)
ghip_wquant_q4_K(const float *__restrict__ x, int64_t nblocks, uint8_t *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float *xb = x + i * 256;
    uint8_t L[256], Laux[32];
    float weights[32], mins[8], scales[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float sum_x2 = 0.0f;
        for (int l = 0; l < 32; l++) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
        const float av_x = sqrt_crt(__fdiv_rn(sum_x2, 32.0f));
        for (int l = 0; l < 32; l++) weights[l] = av_x + fabsf(xb[32 * j + l]);
        scales[j] = make_qkx2_quants(32, 15, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.0f, 0.1f, 20);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0.0f ? __fdiv_rn(63.0f, max_scale) : 0.0f;
    const float inv_min = max_min > 0.0f ? __fdiv_rn(63.0f, max_min) : 0.0f;
    uint8_t out[144];
    uint8_t *sc = out + 4;
    for (int j = 0; j < 12; j++) sc[j] = 0;
    for (int j = 0; j < 8; j++) {
        uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
        if (ls > 63) ls = 63;
        if (lm > 63) lm = 63;
        if (j < 4) {
            sc[j] = ls;
            sc[j + 4] = lm;
        } else {
            sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t dh = f2h(__fdiv_rn(max_scale, 63.0f));
    const uint16_t dminh = f2h(__fdiv_rn(max_min, 63.0f));
    const float dhf = h2f(dh), dminf = h2f(dminh);
    for (int j = 0; j < 8; j++) {
        uint8_t s, m;
        get_scale_min_k4_b(j, sc, &s, &m);
        const float d = dhf * (float)s;
        if (d == 0.0f) continue;
        const float dm = dminf * (float)m;
        for (int ii = 0; ii < 32; ii++) {
            const int l = nearest_int(__fdiv_rn(xb[32 * j + ii] + dm, d));
            L[32 * j + ii] = (uint8_t)imax(0, imin(15, l));
        }
    }
    __builtin_memcpy(out, &dh, 2);
    __builtin_memcpy(out + 2, &dminh, 2);
    uint8_t *q = out + 16;
    for (int j = 0; j < 256; j += 64) {
        for (int l = 0; l < 32; l++) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
        q += 32;
    }
    __builtin_memcpy(y + i * 144, out, 144);
}

// quants_k.rs:1170-1260 with rmse_type = 1 and no quant weights
DEV float make_qx_quants_rmse1(int n, int nmax, const float *x, int8_t *L) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; i++) L[i] = 0;
        return 0.0f;
    }
    float iscale = __fdiv_rn(-(float)nmax, max);
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        int l = nearest_int(iscale * x[i]);
        l = imax(-nmax, imin(nmax - 1, l));
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.0f ? __fdiv_rn(sumlx, suml2) : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = __fdiv_rn(-((float)nmax + 0.1f * (float)is), max);
        sumlx = suml2 = 0.0f;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * x[i]);
            l = imax(-nmax, imin(nmax - 1, l));
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; i++) {
                const int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + imax(-nmax, imin(nmax - 1, l)));
            }
            scale = __fdiv_rn(sumlx, suml2);
            best = scale * sumlx;
        }
    }
    return scale;
}

extern "C" __global__ void __launch_bounds__(64)
ghip_wquant_q6_K(const float *__restrict__ x, int64_t nblocks, uint8_t *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float *xb = x + i * 256;
    int8_t L[256];
    float scales[16];
    uint8_t out[210];
    float max_scale = 0.0f, max_abs_scale = 0.0f;
    for (int ib = 0; ib < 16; ib++) {
        const float scale = make_qx_quants_rmse1(16, 32, xb + 16 * ib, L + 16 * ib);
        scales[ib] = scale;
        const float abs_scale = fabsf(scale);
        if (abs_scale > max_abs_scale) { max_abs_scale = abs_scale; max_scale = scale; }
    }
    if (max_abs_scale < 1e-15f) {
        for (int k = 0; k < 210; k++) out[k] = 0;
        __builtin_memcpy(y + i * 210, out, 210);
        return;
    }
    const float iscale = __fdiv_rn(-128.0f, max_scale);
    const uint16_t dh = f2h(__fdiv_rn(1.0f, iscale));
    const float dhf = h2f(dh);
    int8_t *sc = (int8_t *)(out + 192);
    for (int ib = 0; ib < 16; ib++) sc[ib] = (int8_t)imin(127, nearest_int(iscale * scales[ib]));
    for (int j = 0; j < 16; j++) {
        const float d = dhf * (float)sc[j];
        if (d == 0.0f) continue;
        for (int ii = 0; ii < 16; ii++) {
            int l = nearest_int(__fdiv_rn(xb[16 * j + ii], d));
            l = imax(-32, imin(31, l));
            L[16 * j + ii] = (int8_t)(l + 32);
        }
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int j = 0; j < 256; j += 128) {
        for (int l = 0; l < 32; l++) {
            const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF;
            const uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
            ql[l] = (uint8_t)(q1 | (q3 << 4));
            ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
            qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                              ((L[j + l + 96] >> 4) << 6));
        }
        ql += 64;
        qh += 32;
    }
    __builtin_memcpy(out + 208, &dh, 2);
    __builtin_memcpy(y + i * 210, out, 210);
}

// floor(log2f(a)) as the CPU's correctly rounded log2f yields it: log2 in
// double, rounded to float, then floored (log2 of a float just below 2^k
// rounds up to k in float precision).
DEV float floor_log2f_crt(float a) { return floorf((float)log2((double)a)); }

extern "C" __global__ void __launch_bounds__(256)
ghip_wquant_mxfp4(const float *__restrict__ x, int64_t nblocks, uint8_t *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float *xb = x + i * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++)
        if (amax < fabsf(xb[j])) amax = fabsf(xb[j]);
    const uint8_t e = amax > 0.0f ? (uint8_t)(int)(floor_log2f_crt(amax) - 2.0f + 127.0f) : 0;
    const float d = e8m0_half(e);
    uint8_t out[17];
    out[0] = e;
    for (int j = 0; j < 16; j++) {
        int best[2];
        for (int h = 0; h < 2; h++) {
            const float v = xb[16 * h + j];
            int bi = 0;
            float be = fabsf((float)kvalues_mxfp4_dev[0] * d - v);
            for (int k = 1; k < 16; k++) {
                const float err = fabsf((float)kvalues_mxfp4_dev[k] * d - v);
                if (err < be) { bi = k; be = err; }
            }
            best[h] = bi;
        }
        out[1 + j] = (uint8_t)(best[0] | (best[1] << 4));
    }
    __builtin_memcpy(y + i * 17, out, 17);
}
