/*
 * ggml_oracle.c -- TEST INFRASTRUCTURE ONLY (see ggml_oracle.h).
 *
 * Plain-C restatement of llama.rust's CPU kernels for the quantized ggml hot
 * path.  Compiled with -ffp-contract=off so that every fused multiply-add is an
 * explicit fmaf() where the reference uses f32::mul_add, and every other float
 * operation rounds on its own, exactly as Rust evaluates it.
 */
#include "ggml_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#define GHIP_GRID_QUAL static const
#include "../llama.rust_amd/csrc/ghip_iq_grids.h"
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK4_0 32
#define QK8_0 32
#define QK_K 256
#define QK_MXFP4 32

/* byte layouts: crates/ggml/src/blocks.rs:33-168 */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;                       /* 18 B  */
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;                        /* 34 B  */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4_K; /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } blk_q8_K;       /* 292 B */
typedef struct { uint8_t e; uint8_t qs[16]; } blk_mxfp4;                        /* 17 B  */
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_0;        /* 22 B  */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } blk_q5_K; /* 176 B */
typedef struct { uint16_t d, m; uint8_t qs[16]; } blk_q4_1;                    /* 20 B  */
typedef struct { uint8_t scales[16]; uint8_t qs[64]; uint16_t d, dmin; } blk_q2_K;   /* 84 B  */
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } blk_q3_K; /* 110 B */
typedef struct { uint16_t d, m; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_1;     /* 24 B  */
typedef struct { uint16_t d, s; int8_t qs[32]; } blk_q8_1;                     /* 36 B  */

_Static_assert(sizeof(blk_q4_0) == 18, "q4_0");
_Static_assert(sizeof(blk_q8_0) == 34, "q8_0");
_Static_assert(sizeof(blk_q4_K) == 144, "q4_K");
_Static_assert(sizeof(blk_q6_K) == 210, "q6_K");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K");
_Static_assert(sizeof(blk_mxfp4) == 17, "mxfp4");
_Static_assert(sizeof(blk_q5_0) == 22, "q5_0");
_Static_assert(sizeof(blk_q5_K) == 176, "q5_K");
_Static_assert(sizeof(blk_q4_1) == 20, "q4_1");
_Static_assert(sizeof(blk_q2_K) == 84, "q2_K");
_Static_assert(sizeof(blk_q3_K) == 110, "q3_K");
_Static_assert(sizeof(blk_q5_1) == 24, "q5_1");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1");

double oracle_wtime(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

/* ------------------------------------------------------------------ fp16 */

static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even (half 2.7.1 `f16::from_f32`). */
uint16_t oracle_fp32_to_fp16(float f) {
    uint32_t x = fbits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {                              /* inf / NaN (quiet bit kept) */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u); /* overflow */
    if (e <= 0) {                                   /* subnormal half or zero */
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_m = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++; /* carries into exp correctly */
    return (uint16_t)h;
}

float oracle_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return bitsf(sign);
        /* subnormal: man * 2^-24, exact */
        float v = (float)man * bitsf(0x33800000u);
        return sign ? -v : v;
    }
    if (exp == 0x1f) return bitsf(sign | 0x7f800000u | (man << 13));
    return bitsf(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

#define H2F(h) oracle_fp16_to_fp32(h)
#define F2H(f) oracle_fp32_to_fp16(f)

/* quants.rs:13 nearest_int -- magic-number round-to-nearest-even */
int32_t oracle_nearest_int(float fval) {
    float val = fval + 12582912.0f;
    int32_t i;
    memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}
#define nearest_int oracle_nearest_int

static inline int imin_(int a, int b) { return a < b ? a : b; }
static inline int imax_(int a, int b) { return a > b ? a : b; }

/* quants.rs:660 KVALUES_MXFP4 */
static const int8_t kvalues_mxfp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* quants.rs:682 e8m0_to_fp32_half: 2^(x-128) built from bits */
float oracle_e8m0_to_fp32_half(uint8_t x) {
    uint32_t bits = x < 2 ? (0x00200000u << x) : ((uint32_t)(x - 1) << 23);
    return bitsf(bits);
}

/* ------------------------------------------------------------ quantizers */

/* quants.rs:124-152 quantize_row_q4_0_ref */
void oracle_quantize_row_q4_0_ref(const float *x, void *vy, int64_t k) {
    blk_q4_0 *y = (blk_q4_0 *)vy;
    const int64_t nb = k / QK4_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK4_0; j++) {
            const float v = x[i * QK4_0 + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        for (int j = 0; j < QK4_0 / 2; j++) {
            const float x0 = x[i * QK4_0 + j] * id;
            const float x1 = x[i * QK4_0 + QK4_0 / 2 + j] * id;
            const int8_t xi0 = (int8_t)imin_((int8_t)(x0 + 8.5f), 15);
            const int8_t xi1 = (int8_t)imin_((int8_t)(x1 + 8.5f), 15);
            y[i].qs[j] = (uint8_t)((xi0 & 0x0f) | ((xi1 & 0x0f) << 4));
        }
    }
}

/* quants.rs:207-240 quantize_row_q5_0_ref */
void oracle_quantize_row_q5_0_ref(const float *x, void *vy, int64_t k) {
    blk_q5_0 *y = (blk_q5_0 *)vy;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -16.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            const float x0 = x[i * 32 + j] * id;
            const float x1 = x[i * 32 + 16 + j] * id;
            const uint8_t xi0 = (uint8_t)imin_((int8_t)(x0 + 16.5f), 31) & 0x1F;
            const uint8_t xi1 = (uint8_t)imin_((int8_t)(x1 + 16.5f), 31) & 0x1F;
            y[i].qs[j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
            qh |= (uint32_t)((xi0 & 0x10) >> 4) << j;
            qh |= (uint32_t)((xi1 & 0x10) >> 4) << (j + 16);
        }
        y[i].d = F2H(d);
        for (int b = 0; b < 4; b++) y[i].qh[b] = (uint8_t)(qh >> (8 * b));
    }
}

/* quants.rs:302 quantize_row_q8_0_ref (roundf: half away from zero) */
void oracle_quantize_row_q8_0_ref(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        for (int j = 0; j < QK8_0; j++) y[i].qs[j] = (int8_t)roundf(x[i * QK8_0 + j] * id);
    }
}

/* Rust `f as i32` / `f as u8`: truncation toward zero, saturating, NaN -> 0 */
static inline int32_t sat_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483647.0f) return 2147483647;
    if (f <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)f;
}
static inline uint8_t sat_u8(float f) {
    if (f != f || f <= 0.0f) return 0;
    if (f >= 255.0f) return 255;
    return (uint8_t)f;
}
static inline int8_t sat_i8(float f) {
    if (f != f) return 0;
    if (f >= 127.0f) return 127;
    if (f <= -128.0f) return -128;
    return (int8_t)f;
}

/* quants.rs:29-41 minmax: NaN never replaces either bound */
static void minmax32(const float *x, float *mn, float *mx) {
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (int j = 0; j < 32; j++) {
        if (x[j] < lo) lo = x[j];
        if (x[j] > hi) hi = x[j];
    }
    *mn = lo;
    *mx = hi;
}

/* quants.rs:169-187 quantize_row_q4_1_ref */
void oracle_quantize_row_q4_1_ref(const float *x, void *vy, int64_t k) {
    blk_q4_1 *y = (blk_q4_1 *)vy;
    for (int64_t i = 0; i < k / 32; i++) {
        float mn, mx;
        minmax32(x + i * 32, &mn, &mx);
        const float d = (mx - mn) / 15.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        for (int j = 0; j < 16; j++) {
            const float x0 = (x[i * 32 + j] - mn) * id, x1 = (x[i * 32 + 16 + j] - mn) * id;
            int32_t a = sat_i32(x0 + 0.5f), b = sat_i32(x1 + 0.5f);
            a = a < 15 ? a : 15;
            a = a > 0 ? a : 0;
            b = b < 15 ? b : 15;
            b = b > 0 ? b : 0;
            y[i].qs[j] = (uint8_t)(a | (b << 4));
        }
        y[i].d = F2H(d);
        y[i].m = F2H(mn);
    }
}

/* quants.rs:260-286 quantize_row_q5_1_ref */
void oracle_quantize_row_q5_1_ref(const float *x, void *vy, int64_t k) {
    blk_q5_1 *y = (blk_q5_1 *)vy;
    for (int64_t i = 0; i < k / 32; i++) {
        float mn, mx;
        minmax32(x + i * 32, &mn, &mx);
        const float d = (mx - mn) / 31.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            const float x0 = (x[i * 32 + j] - mn) * id, x1 = (x[i * 32 + 16 + j] - mn) * id;
            const uint8_t a = sat_u8(x0 + 0.5f), b = sat_u8(x1 + 0.5f);
            y[i].qs[j] = (uint8_t)((a & 0x0F) | ((b & 0x0F) << 4));
            qh |= (uint32_t)((a & 0x10) >> 4) << j;
            qh |= (uint32_t)((b & 0x10) >> 4) << (j + 16);
        }
        memcpy(y[i].qh, &qh, 4);
        y[i].d = F2H(d);
        y[i].m = F2H(mn);
    }
}

/* quants.rs:375-397 quantize_row_q8_1_ref (= quantize_row_q8_1): d = amax / 127,
 * id = 1 / d, q = round-half-even(x * id) saturated to i8 (NaN -> 0),
 * s = f16(sum(q) * d) */
void oracle_quantize_row_q8_1(const float *x, void *vy, int64_t k) {
    blk_q8_1 *y = (blk_q8_1 *)vy;
    for (int64_t i = 0; i < k / 32; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[i * 32 + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int32_t sum = 0;
        for (int j = 0; j < 32; j++) {
            y[i].qs[j] = sat_i8(rintf(x[i * 32 + j] * id));
            sum += y[i].qs[j];
        }
        y[i].d = F2H(d);
        y[i].s = F2H((float)sum * d);
    }
}

/* quants.rs:331-362 quantize_row_q8_0 (runtime AVX2 arithmetic): id = 127/amax,
 * round-half-even, NaN/overflow -> -128. */
void oracle_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        y[i].d = F2H(d);
        for (int j = 0; j < QK8_0; j++) {
            const float r = nearbyintf(x[i * QK8_0 + j] * id);
            y[i].qs[j] = (isnan(r) || fabsf(r) >= 2147483648.0f) ? (int8_t)-128 : (int8_t)(int)r;
        }
    }
}

/* quants.rs:615-650 quantize_row_q8_K_ref */
void oracle_quantize_row_q8_K_ref(const float *x, void *vy, int64_t k) {
    blk_q8_K *y = (blk_q8_K *)vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(blk_q8_K));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; j++) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t)imin_(127, v);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int sum = 0;
            for (int ii = 0; ii < 16; ii++) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* repack.rs:1561-1620 quantize_mat_q8_K_4x8, per-row values: iscale = 127/amax,
 * round-half-even, clamp to i8, d = 1/iscale; bsums over the stored values.
 * Written as plain block_q8_K rows (the interleave only moves bytes). */
void oracle_quantize_row_q8_K_mat(const float *x, void *vy, int64_t k) {
    blk_q8_K *y = (blk_q8_K *)vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * QK_K;
        float max_abs = 0.0f;
        for (int j = 0; j < QK_K; j++) { const float a = fabsf(xb[j]); if (a > max_abs) max_abs = a; }
        const float iscale = max_abs != 0.0f ? 127.0f / max_abs : 0.0f;
        y[i].d = max_abs != 0.0f ? 1.0f / iscale : 0.0f;
        for (int j = 0; j < QK_K; j++) {
            float r = nearbyintf(iscale * xb[j]);
            if (r < -128.0f) r = -128.0f;
            if (r > 127.0f) r = 127.0f;
            y[i].qs[j] = (int8_t)(int)r;
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int sum = 0;
            for (int ii = 0; ii < 16; ii++) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
    }
}

/* quants_k.rs:1396-1490 make_qkx2_quants */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights,
                              uint8_t *L, float *the_min, uint8_t *Laux,
                              float rmin, float rdelta, int nstep, int use_mad) {
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
    float iscale = (float)nmax / (max - min);
    float scale = 1.0f / iscale;
    float best_error = 0.0f;
    for (int i = 0; i < n; i++) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)imax_(0, imin_(nmax, l));
        float diff = scale * (float)L[i] + min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) { *the_min = -min; return scale; }
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (max - min);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; i++) {
            const int l = imax_(0, imin_(nmax, nearest_int(iscale * (x[i] - min))));
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * (float)l;
            sum_l2 += w * (float)l * (float)l;
            sum_xl += w * (float)l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0.0f) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0.0f) { this_min = 0.0f; this_scale = sum_xl / sum_l2; }
            float cur_error = 0.0f;
            for (int i = 0; i < n; i++) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = use_mad ? fabsf(diff) : diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                memcpy(L, Laux, (size_t)n);
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* quants_k.rs:1672 get_scale_min_k4 */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* The scale/min selection shared by quantize_row_q4_K_ref (quants_k.rs:1861-1950,
 * nmax 15, rmin -1, 20 steps) and quantize_row_q5_K_ref (quants_k.rs:1952-2040,
 * nmax 31, rmin -0.5, 15 steps): per super-block the 6-bit scales and mins,
 * d, dmin and the levels L[256] in 0..nmax. */
static void k_quant_levels(const float *xb, int nmax, float rmin, int nstep, uint8_t L[QK_K], uint8_t sc[12],
                           uint16_t *dh_out, uint16_t *dminh_out) {
    uint8_t Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < QK_K / 32; j++) {
        float sum_x2 = 0.0f;
        for (int l = 0; l < 32; l++) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32.0f);
        for (int l = 0; l < 32; l++) weights[l] = av_x + fabsf(xb[32 * j + l]);
        scales[j] = make_qkx2_quants(32, nmax, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux,
                                     rmin, 0.1f, nstep, 0);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    memset(sc, 0, 12);
    for (int j = 0; j < QK_K / 32; j++) {
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
    const uint16_t dh = F2H(max_scale / 63.0f);
    const uint16_t dminh = F2H(max_min / 63.0f);
    for (int j = 0; j < QK_K / 32; j++) {
        uint8_t s, m;
        get_scale_min_k4(j, sc, &s, &m);
        const float d = H2F(dh) * (float)s;
        if (d == 0.0f) continue;
        const float dm = H2F(dminh) * (float)m;
        for (int ii = 0; ii < 32; ii++) {
            const int l = nearest_int((xb[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t)imax_(0, imin_(nmax, l));
        }
    }
    *dh_out = dh;
    *dminh_out = dminh;
}

/* quants_k.rs:1861-1950 quantize_row_q4_K_ref */
void oracle_quantize_row_q4_K_ref(const float *x, void *vy, int64_t k) {
    blk_q4_K *y = (blk_q4_K *)vy;
    const int64_t nb = k / QK_K;
    uint8_t L[QK_K], sc[12];
    for (int64_t i = 0; i < nb; i++) {
        uint16_t dh, dminh;
        k_quant_levels(x + i * QK_K, 15, -1.0f, 20, L, sc, &dh, &dminh);
        y[i].d = dh;
        y[i].dmin = dminh;
        memcpy(y[i].scales, sc, 12);
        uint8_t *q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; l++) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
    }
}

/* quants_k.rs:1952-2056 quantize_row_q5_K_ref: levels 0..31, the fifth bit
 * of sub-block 2j / 2j+1 element e in bit 2j / 2j+1 of qh[e] */
void oracle_quantize_row_q5_K_ref(const float *x, void *vy, int64_t k) {
    blk_q5_K *y = (blk_q5_K *)vy;
    const int64_t nb = k / QK_K;
    uint8_t L[QK_K], sc[12];
    for (int64_t i = 0; i < nb; i++) {
        uint16_t dh, dminh;
        k_quant_levels(x + i * QK_K, 31, -0.5f, 15, L, sc, &dh, &dminh);
        y[i].d = dh;
        y[i].dmin = dminh;
        memcpy(y[i].scales, sc, 12);
        memset(y[i].qh, 0, 32);
        for (int j = 0; j < 4; j++)
            for (int e = 0; e < 32; e++) {
                int l1 = L[64 * j + e], l2 = L[64 * j + 32 + e];
                if (l1 > 15) { l1 -= 16; y[i].qh[e] |= (uint8_t)(1u << (2 * j)); }
                if (l2 > 15) { l2 -= 16; y[i].qh[e] |= (uint8_t)(2u << (2 * j)); }
                y[i].qs[32 * j + e] = (uint8_t)(l1 | (l2 << 4));
            }
    }
}

/* quants_k.rs:1170-1260 make_qx_quants (qw == NULL) */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *L, int rmse_type) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; i++) L[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; i++) {
            const int l = nearest_int(iscale * x[i]);
            L[i] = (int8_t)(nmax + imax_(-nmax, imin_(nmax - 1, l)));
        }
        return 1.0f / iscale;
    }
    int return_early = 0;
    if (rmse_type < 0) { rmse_type = -rmse_type; return_early = 1; }
#define WEIGHT(i) (rmse_type == 1 ? x[i] * x[i] : rmse_type == 2 ? 1.0f : rmse_type == 3 ? fabsf(x[i]) : sqrtf(fabsf(x[i])))
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        int l = nearest_int(iscale * x[i]);
        l = imax_(-nmax, imin_(nmax - 1, l));
        L[i] = (int8_t)(l + nmax);
        const float w = WEIGHT(i);
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    if (return_early) return suml2 > 0.0f ? 0.5f * (scale + 1.0f / iscale) : 1.0f / iscale;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        sumlx = suml2 = 0.0f;
        for (int i = 0; i < n; i++) {
            int l = nearest_int(iscale * x[i]);
            l = imax_(-nmax, imin_(nmax - 1, l));
            const float w = WEIGHT(i);
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; i++) {
                const int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + imax_(-nmax, imin_(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
#undef WEIGHT
    return scale;
}

/* quants_k.rs:2058-2133 quantize_row_q6_K_ref */
void oracle_quantize_row_q6_K_ref(const float *x, void *vy, int64_t k) {
    blk_q6_K *y = (blk_q6_K *)vy;
    const int64_t nb = k / QK_K;
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * QK_K;
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int ib = 0; ib < QK_K / 16; ib++) {
            const float scale = make_qx_quants(16, 32, xb + 16 * ib, L + 16 * ib, 1);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) { max_abs_scale = abs_scale; max_scale = scale; }
        }
        if (max_abs_scale < 1e-15f) {
            memset(&y[i], 0, sizeof(blk_q6_K));
            y[i].d = F2H(0.0f);
            continue;
        }
        const float iscale = -128.0f / max_scale;
        const uint16_t dh = F2H(1.0f / iscale);
        int8_t sc[16];
        for (int ib = 0; ib < QK_K / 16; ib++) sc[ib] = (int8_t)imin_(127, nearest_int(iscale * scales[ib]));
        for (int j = 0; j < QK_K / 16; j++) {
            const float d = H2F(dh) * (float)sc[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                int l = nearest_int(xb[16 * j + ii] / d);
                l = imax_(-32, imin_(31, l));
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = y[i].ql, *qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; l++) {
                const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
                ql[l] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                  ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        memcpy(y[i].scales, sc, 16);
        y[i].d = dh;
    }
}

/* MXFP4 quantizer.  The reference has none (compute.rs:9861-9863); this is the
 * published upstream ggml quantize_row_mxfp4_ref algorithm (ggml-quants.c),
 * pinned by the SECT sections of parity/quants_ref_fp4.bin:
 *   e = amax > 0 ? (u8)(floor(log2(amax)) - 2 + 127) : 0, d = e8m0_half(e),
 *   nibble = argmin_i |kvalues[i]*d - x| (first minimum wins). */
static int best_index_mxfp4(float x, float e) {
    int best = 0;
    float best_err = fabsf((float)kvalues_mxfp4[0] * e - x);
    for (int i = 1; i < 16; i++) {
        const float err = fabsf((float)kvalues_mxfp4[i] * e - x);
        if (err < best_err) { best = i; best_err = err; }
    }
    return best;
}

void oracle_quantize_row_mxfp4_ref(const float *x, void *vy, int64_t k) {
    blk_mxfp4 *y = (blk_mxfp4 *)vy;
    const int64_t nb = k / QK_MXFP4;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK_MXFP4; j++) {
            const float v = x[i * QK_MXFP4 + j];
            if (amax < fabsf(v)) amax = fabsf(v);
        }
        const uint8_t e = amax > 0.0f ? (uint8_t)(floorf(log2f(amax)) - 2 + 127) : 0;
        const float d = oracle_e8m0_to_fp32_half(e);
        y[i].e = e;
        for (int j = 0; j < QK_MXFP4 / 2; j++) {
            const int x0 = best_index_mxfp4(x[i * QK_MXFP4 + j], d);
            const int x1 = best_index_mxfp4(x[i * QK_MXFP4 + QK_MXFP4 / 2 + j], d);
            y[i].qs[j] = (uint8_t)(x0 | (x1 << 4));
        }
    }
}

/* ---------------------------------------------------------- dequantizers */

/* quants.rs:142 / :363 / quants_k.rs via quants.rs:540,584 / quants.rs:732 */
/* q5_0 value e of a 32-block: nibble | bit e of qh << 4, minus 16
 * (vec_dot.rs:661-686) */
static inline int q5_0_val(const blk_q5_0 *x, int e) {
    const uint32_t qh = (uint32_t)x->qh[0] | ((uint32_t)x->qh[1] << 8) | ((uint32_t)x->qh[2] << 16) |
                        ((uint32_t)x->qh[3] << 24);
    const int lo = e < 16 ? (x->qs[e] & 0x0F) : (x->qs[e - 16] >> 4);
    return (lo | (int)(((qh >> e) & 1u) << 4)) - 16;
}

/* q5_0 x q8_0 and q8_0 x q8_0, one 32-block: the exact block sum */
static inline int32_t isum_q5_0(const blk_q5_0 *x, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += q5_0_val(x, e) * y->qs[e];
    return s;
}
static inline int32_t isum_q8_0(const blk_q8_0 *x, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += x->qs[e] * y->qs[e];
    return s;
}

/* q5_K 5-bit values of sub-blocks 2j (low nibbles, qh bit 2j) and 2j+1 (high
 * nibbles, qh bit 2j+1), element e of 32 (vec_dot.rs:954-962) */
static inline int q5k_lo(const blk_q5_K *x, int j, int e) {
    return (x->qs[32 * j + e] & 0x0F) | (((x->qh[e] >> (2 * j)) & 1) << 4);
}
static inline int q5k_hi(const blk_q5_K *x, int j, int e) {
    return (x->qs[32 * j + e] >> 4) | (((x->qh[e] >> (2 * j + 1)) & 1) << 4);
}

/* q5_K x q8_K, whole super-block: {iacc, imin} as for q4_K
 * (iacc = sum_s sc_s * sum q5*q8, imin = sum_s m_s * bsum32_s) */
static inline void isum_q5_K(const blk_q5_K *x, const blk_q8_K *y, int32_t *iacc, int32_t *imin) {
    int32_t ia = 0, im = 0;
    for (int j = 0; j < 4; j++) {
        uint8_t s0, m0, s1, m1;
        get_scale_min_k4(2 * j, x->scales, &s0, &m0);
        get_scale_min_k4(2 * j + 1, x->scales, &s1, &m1);
        int32_t a = 0, b = 0;
        for (int e = 0; e < 32; e++) {
            a += q5k_lo(x, j, e) * y->qs[64 * j + e];
            b += q5k_hi(x, j, e) * y->qs[64 * j + 32 + e];
        }
        ia += s0 * a + s1 * b;
        im += m0 * (y->bsums[4 * j] + y->bsums[4 * j + 1]) + m1 * (y->bsums[4 * j + 2] + y->bsums[4 * j + 3]);
    }
    *iacc = ia;
    *imin = im;
}

/* q5_1 value e of a 32-block: nibble | bit e of qh << 4 (unsigned) */
static inline int q5_1_val(const blk_q5_1 *x, int e) {
    uint32_t qh;
    memcpy(&qh, x->qh, 4);
    const int lo = e < 16 ? (x->qs[e] & 0x0F) : (x->qs[e - 16] >> 4);
    return lo | (int)(((qh >> e) & 1) << 4);
}
static inline int q4_1_val(const blk_q4_1 *x, int e) { return e < 16 ? (x->qs[e] & 0x0F) : (x->qs[e - 16] >> 4); }
/* the exact integer sums of one 32-block (unsigned codes x q8_1 codes) */
static inline int32_t isum_q4_1(const blk_q4_1 *x, const blk_q8_1 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += q4_1_val(x, e) * y->qs[e];
    return s;
}
static inline int32_t isum_q5_1(const blk_q5_1 *x, const blk_q8_1 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += q5_1_val(x, e) * y->qs[e];
    return s;
}

/* Q2_K / Q3_K element e of 128-group j at shift k (e < 32): element
 * 128j + 32k + e, byte qs[32j + e] >> 2k, scale index 8j + 2k + (e >= 16)
 * (quants.rs:431-465, :467-520). */
static inline int q2k_val(const blk_q2_K *x, int j, int k, int e) { return (x->qs[32 * j + e] >> (2 * k)) & 3; }
static inline int q3k_val(const blk_q3_K *x, int j, int k, int e) {
    const int lo = (x->qs[32 * j + e] >> (2 * k)) & 3;
    return (x->hmask[e] >> (4 * j + k)) & 1 ? lo : lo - 4;
}
/* the 16 6-bit Q3_K scales from the 12 packed bytes, as unsigned 0..63
 * (quants.rs:475-484: aux[] de-packing) */
static void q3k_scales_u(const uint8_t *packed, int sc[16]) {
    const uint32_t km1 = 0x03030303u, km2 = 0x0f0f0f0fu;
    uint32_t a0, a1, a2;
    memcpy(&a0, packed, 4);
    memcpy(&a1, packed + 4, 4);
    memcpy(&a2, packed + 8, 4);
    const uint32_t w[4] = {(a0 & km2) | ((a2 & km1) << 4), (a1 & km2) | (((a2 >> 2) & km1) << 4),
                           ((a0 >> 4) & km2) | (((a2 >> 4) & km1) << 4), ((a1 >> 4) & km2) | (((a2 >> 6) & km1) << 4)};
    for (int i = 0; i < 16; i++) sc[i] = (int)((w[i >> 2] >> (8 * (i & 3))) & 0xff);
}
/* exact per-super-block sums: Q2_K isum = sum_g (sc_g & 15) * sum q2*q8,
 * summs = sum_g (sc_g >> 4) * bsums_g; Q3_K isum = sum_g (sc_g - 32) * sum v*q8 */
static inline void isum_q2_K(const blk_q2_K *x, const blk_q8_K *y, int32_t *isum, int32_t *summs) {
    int32_t is = 0, sm = 0;
    for (int g = 0; g < 16; g++) sm += (x->scales[g] >> 4) * y->bsums[g];
    for (int j = 0; j < 2; j++)
        for (int k = 0; k < 4; k++)
            for (int h = 0; h < 2; h++) {
                int32_t s = 0;
                for (int e = 16 * h; e < 16 * h + 16; e++) s += q2k_val(x, j, k, e) * y->qs[128 * j + 32 * k + e];
                is += (x->scales[8 * j + 2 * k + h] & 0xF) * s;
            }
    *isum = is;
    *summs = sm;
}
static inline int32_t isum_q3_K(const blk_q3_K *x, const blk_q8_K *y) {
    int sc[16];
    q3k_scales_u(x->scales, sc);
    int32_t is = 0;
    for (int j = 0; j < 2; j++)
        for (int k = 0; k < 4; k++)
            for (int h = 0; h < 2; h++) {
                int32_t s = 0;
                for (int e = 16 * h; e < 16 * h + 16; e++) s += q3k_val(x, j, k, e) * y->qs[128 * j + 32 * k + e];
                is += (sc[8 * j + 2 * k + h] - 32) * s;
            }
    return is;
}

/* ---- Q1_0, Q2_0 (blocks.rs:14-28) ---- */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q1_0;  /* 18 B per 128 */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q2_0;  /* 18 B per 64 */
/* element j of a Q1_0 block: +1 where bit j is set, else -1 (quants.rs:66-78) */
static inline int q1_0_val(const blk_q1_0 *x, int j) { return ((x->qs[j / 8] >> (j % 8)) & 1) ? 1 : -1; }
/* element j of a Q2_0 block: 2-bit field j minus 1 (quants.rs:108-120) */
static inline int q2_0_val(const blk_q2_0 *x, int j) { return (int)((x->qs[j / 4] >> ((j % 4) * 2)) & 3) - 1; }

/* quants.rs:44-63: d = sum |x| / 128 (summed in order), bit = x >= 0 */
void oracle_quantize_row_q1_0_ref(const float *x, void *vy, int64_t k) {
    blk_q1_0 *y = (blk_q1_0 *)vy;
    for (int64_t i = 0; i < k / 128; i++) {
        float sum_abs = 0.0f;
        for (int j = 0; j < 128; j++) sum_abs += fabsf(x[i * 128 + j]);
        const float d = sum_abs / 128.0f;
        memset(y[i].qs, 0, 16);
        for (int j = 0; j < 128; j++) y[i].qs[j / 8] |= (uint8_t)((x[i * 128 + j] >= 0.0f) << (j % 8));
        y[i].d = oracle_fp32_to_fp16(d);
    }
}
/* quants.rs:82-106: d = max |x|, q = clamp(round(x / d) + 1, 0, 3), round half away from zero */
void oracle_quantize_row_q2_0_ref(const float *x, void *vy, int64_t k) {
    blk_q2_0 *y = (blk_q2_0 *)vy;
    for (int64_t i = 0; i < k / 64; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 64; j++) {
            const float a = fabsf(x[i * 64 + j]);
            if (a > amax) amax = a;
        }
        const float d = amax, id = d > 0.0f ? 1.0f / d : 0.0f;
        memset(y[i].qs, 0, 16);
        for (int j = 0; j < 64; j++) {
            int q = (int)roundf(x[i * 64 + j] * id) + 1;
            q = q < 0 ? 0 : q > 3 ? 3 : q;
            y[i].qs[j / 4] |= (uint8_t)(q << ((j % 4) * 2));
        }
        y[i].d = oracle_fp32_to_fp16(d);
    }
}
/* exact sums per Q8_0 block: group g (32 elements) of the weight row */
static inline int32_t isum_q1_0(const blk_q1_0 *x, int k, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += q1_0_val(x, 32 * k + e) * y->qs[e];
    return s;
}
static inline int32_t isum_q2_0(const blk_q2_0 *x, int k, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += q2_0_val(x, 32 * k + e) * y->qs[e];
    return s;
}

/* ---- IQ4_NL, IQ4_XS, NVFP4 (blocks.rs:55-62, :234-249) ---- */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_iq4_nl;                               /* 18 B  */
typedef struct { uint16_t d, scales_h; uint8_t scales_l[4]; uint8_t qs[128]; } blk_iq4_xs; /* 136 B */
typedef struct { uint8_t d[4]; uint8_t qs[32]; } blk_nvfp4;                                /* 36 B  */
_Static_assert(sizeof(blk_iq4_nl) == 18, "iq4_nl");
_Static_assert(sizeof(blk_iq4_xs) == 136, "iq4_xs");
_Static_assert(sizeof(blk_nvfp4) == 36, "nvfp4");
/* KVALUES_IQ4NL (quants_k.rs:647) */
static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* ue4m3_to_fp32 (quants.rs:699-712): 0 for 0x00 / 0x7F, subnormals man * 2^-9,
 * else (1 + man/8) * 2^(exp-7); then halved.  Every step is exact. */
float oracle_ue4m3_to_fp32(uint8_t x) {
    if (x == 0 || x == 0x7F) return 0.0f;
    const int ex = (x >> 3) & 0xF, man = x & 7;
    const float raw = ex == 0 ? ldexpf((float)man, -9) : ldexpf(1.0f + (float)man / 8.0f, ex - 7);
    return raw * 0.5f;
}
/* element e (0..31) of an IQ4_NL / IQ4_XS 32-group: low nibbles of qs[0..15]
 * are elements 0..15, high nibbles 16..31 (dequantize_row_iq4_nl, quants_k.rs:2379) */
static inline int iq4_val(const uint8_t *qs16, int e) {
    return kvalues_iq4nl[e < 16 ? (qs16[e] & 0x0F) : (qs16[e - 16] >> 4)];
}
/* the 6-bit scale of 32-group ib, minus 32 (quants_k.rs:2401-2403) */
static inline int iq4xs_ls(const blk_iq4_xs *x, int ib) {
    return (int)(((x->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((x->scales_h >> (2 * ib)) & 3) << 4)) - 32;
}
/* element e (0..63) of an NVFP4 block: sub-block s = e / 16, within it the low
 * nibbles of qs[8s .. 8s+7] are elements 0..7 and the high nibbles 8..15
 * (dequantize_row_nvfp4, quants.rs:749-767) */
static inline int nvfp4_val(const blk_nvfp4 *x, int e) {
    const int s = e / 16, j = e % 16;
    const uint8_t b = x->qs[8 * s + j % 8];
    return kvalues_mxfp4[j < 8 ? (b & 0x0F) : (b >> 4)];
}
/* exact sums: IQ4_NL per 32-block, NVFP4 per 16-sub-block (element e of the
 * 64-block meets code e % 32 of Q8_0 block e / 32), IQ4_XS per super-block
 * sum_ib (ls_ib - 32) * sum kvalue * q8 */
static inline int32_t isum_iq4_nl(const blk_iq4_nl *x, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += iq4_val(x->qs, e) * y->qs[e];
    return s;
}
static inline int32_t isum_nvfp4_sub(const blk_nvfp4 *x, const blk_q8_0 *y2, int s) {
    int32_t r = 0;
    for (int e = 16 * s; e < 16 * s + 16; e++) r += nvfp4_val(x, e) * y2[e / 32].qs[e % 32];
    return r;
}
static inline int32_t isum_iq4_xs(const blk_iq4_xs *x, const blk_q8_K *y) {
    int32_t is = 0;
    for (int ib = 0; ib < 8; ib++) {
        int32_t s = 0;
        for (int e = 0; e < 32; e++) s += iq4_val(x->qs + 16 * ib, e) * y->qs[32 * ib + e];
        is += iq4xs_ls(x, ib) * s;
    }
    return is;
}

void oracle_dequantize_row(int type, const void *vx, float *y, int64_t k) {
    if (type == OR_Q1_0) { /* quants.rs:66-78 */
        const blk_q1_0 *x = (const blk_q1_0 *)vx;
        for (int64_t i = 0; i < k / 128; i++) {
            const float d = H2F(x[i].d), neg = -d;
            for (int j = 0; j < 128; j++) y[i * 128 + j] = q1_0_val(&x[i], j) > 0 ? d : neg;
        }
        return;
    }
    if (type == OR_Q2_0) { /* quants.rs:108-120 */
        const blk_q2_0 *x = (const blk_q2_0 *)vx;
        for (int64_t i = 0; i < k / 64; i++) {
            const float d = H2F(x[i].d);
            for (int j = 0; j < 64; j++) y[i * 64 + j] = (float)q2_0_val(&x[i], j) * d;
        }
        return;
    }
    if (type == OR_IQ4_NL) { /* quants_k.rs:2379-2390 */
        const blk_iq4_nl *x = (const blk_iq4_nl *)vx;
        for (int64_t i = 0; i < k / 32; i++) {
            const float d = H2F(x[i].d);
            for (int e = 0; e < 32; e++) y[i * 32 + e] = d * (float)iq4_val(x[i].qs, e);
        }
        return;
    }
    if (type == OR_IQ4_XS) { /* quants_k.rs:2393-2412 */
        const blk_iq4_xs *x = (const blk_iq4_xs *)vx;
        for (int64_t i = 0; i < k / QK_K; i++) {
            const float d = H2F(x[i].d);
            for (int ib = 0; ib < 8; ib++) {
                const float dl = d * (float)iq4xs_ls(&x[i], ib);
                for (int e = 0; e < 32; e++) y[i * QK_K + 32 * ib + e] = dl * (float)iq4_val(x[i].qs + 16 * ib, e);
            }
        }
        return;
    }
    if (type == OR_NVFP4) { /* quants.rs:749-767 */
        const blk_nvfp4 *x = (const blk_nvfp4 *)vx;
        for (int64_t i = 0; i < k / 64; i++)
            for (int s = 0; s < 4; s++) {
                const float d = oracle_ue4m3_to_fp32(x[i].d[s]);
                for (int j = 0; j < 16; j++) y[i * 64 + 16 * s + j] = (float)nvfp4_val(&x[i], 16 * s + j) * d;
            }
        return;
    }
    if (type == OR_Q2_K) { /* quants.rs:431-465 */
        const blk_q2_K *x = (const blk_q2_K *)vx;
        for (int64_t i = 0; i < k / QK_K; i++) {
            const float d = H2F(x[i].d), mn = H2F(x[i].dmin);
            for (int j = 0; j < 2; j++)
                for (int kk = 0; kk < 4; kk++)
                    for (int h = 0; h < 2; h++) {
                        const uint8_t sc = x[i].scales[8 * j + 2 * kk + h];
                        const float dl = d * (float)(sc & 0xF), ml = mn * (float)(sc >> 4);
                        for (int e = 16 * h; e < 16 * h + 16; e++)
                            y[i * QK_K + 128 * j + 32 * kk + e] = dl * (float)q2k_val(&x[i], j, kk, e) - ml;
                    }
        }
        return;
    }
    if (type == OR_Q3_K) { /* quants.rs:467-520 */
        const blk_q3_K *x = (const blk_q3_K *)vx;
        for (int64_t i = 0; i < k / QK_K; i++) {
            const float d = H2F(x[i].d);
            int sc[16];
            q3k_scales_u(x[i].scales, sc);
            for (int j = 0; j < 2; j++)
                for (int kk = 0; kk < 4; kk++)
                    for (int h = 0; h < 2; h++) {
                        const float dl = d * ((float)(int8_t)sc[8 * j + 2 * kk + h] - 32.0f);
                        for (int e = 16 * h; e < 16 * h + 16; e++)
                            y[i * QK_K + 128 * j + 32 * kk + e] = dl * (float)q3k_val(&x[i], j, kk, e);
                    }
        }
        return;
    }
    if (type == OR_Q4_1 || type == OR_Q5_1) { /* quants.rs:189-202, :288-304: x * d + m */
        for (int64_t i = 0; i < k / 32; i++) {
            const blk_q4_1 *a = (const blk_q4_1 *)vx + i;
            const blk_q5_1 *b = (const blk_q5_1 *)vx + i;
            const float d = H2F(type == OR_Q4_1 ? a->d : b->d), m = H2F(type == OR_Q4_1 ? a->m : b->m);
            for (int e = 0; e < 32; e++)
                y[i * 32 + e] = (float)(type == OR_Q4_1 ? q4_1_val(a, e) : q5_1_val(b, e)) * d + m;
        }
        return;
    }
    if (type == OR_Q8_1) { /* qs * d */
        const blk_q8_1 *x = (const blk_q8_1 *)vx;
        for (int64_t i = 0; i < k / 32; i++)
            for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)x[i].qs[j] * H2F(x[i].d);
        return;
    }
    if (type == OR_Q4_0) {
        const blk_q4_0 *x = (const blk_q4_0 *)vx;
        for (int64_t i = 0; i < k / QK4_0; i++) {
            const float d = H2F(x[i].d);
            for (int j = 0; j < 16; j++) {
                y[i * 32 + j] = (float)((x[i].qs[j] & 0x0F) - 8) * d;
                y[i * 32 + 16 + j] = (float)((x[i].qs[j] >> 4) - 8) * d;
            }
        }
    } else if (type == OR_Q5_0) { /* quants.rs:242-258 */
        const blk_q5_0 *x = (const blk_q5_0 *)vx;
        for (int64_t i = 0; i < k / QK8_0; i++) {
            const float d = H2F(x[i].d);
            for (int e = 0; e < 32; e++) y[i * 32 + e] = (float)q5_0_val(&x[i], e) * d;
        }
    } else if (type == OR_Q5_K) { /* quants.rs:549-585 */
        const blk_q5_K *x = (const blk_q5_K *)vx;
        for (int64_t i = 0; i < k / QK_K; i++) {
            const float d = H2F(x[i].d), mn = H2F(x[i].dmin);
            for (int j = 0; j < 4; j++) {
                uint8_t s0, m0, s1, m1;
                get_scale_min_k4(2 * j, x[i].scales, &s0, &m0);
                get_scale_min_k4(2 * j + 1, x[i].scales, &s1, &m1);
                const float d1 = d * (float)s0, mm1 = mn * (float)m0, d2 = d * (float)s1, mm2 = mn * (float)m1;
                for (int e = 0; e < 32; e++) {
                    y[i * QK_K + 64 * j + e] = d1 * (float)q5k_lo(&x[i], j, e) - mm1;
                    y[i * QK_K + 64 * j + 32 + e] = d2 * (float)q5k_hi(&x[i], j, e) - mm2;
                }
            }
        }
    } else if (type == OR_Q8_0) {
        const blk_q8_0 *x = (const blk_q8_0 *)vx;
        for (int64_t i = 0; i < k / QK8_0; i++) {
            const float d = H2F(x[i].d);
            for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)x[i].qs[j] * d;
        }
    } else if (type == OR_Q4_K) {
        const blk_q4_K *x = (const blk_q4_K *)vx;
        for (int64_t i = 0; i < k / QK_K; i++) {
            const float d = H2F(x[i].d), min = H2F(x[i].dmin);
            const uint8_t *q = x[i].qs;
            float *yy = y + i * QK_K;
            int is = 0;
            for (int j = 0; j < QK_K; j += 64) {
                uint8_t sc, m;
                get_scale_min_k4(is, x[i].scales, &sc, &m);
                const float d1 = d * sc, m1 = min * m;
                get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
                const float d2 = d * sc, m2 = min * m;
                for (int l = 0; l < 32; l++) *yy++ = d1 * (float)(q[l] & 0xF) - m1;
                for (int l = 0; l < 32; l++) *yy++ = d2 * (float)(q[l] >> 4) - m2;
                q += 32;
                is += 2;
            }
        }
    } else if (type == OR_Q6_K) {
        const blk_q6_K *x = (const blk_q6_K *)vx;
        for (int64_t i = 0; i < k / QK_K; i++) {
            const float d = H2F(x[i].d);
            const uint8_t *ql = x[i].ql, *qh = x[i].qh;
            const int8_t *sc = x[i].scales;
            float *yy = y + i * QK_K;
            for (int n = 0; n < QK_K; n += 128) {
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int8_t q1 = (int8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int8_t q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    yy[l] = d * (float)sc[is + 0] * (float)q1;
                    yy[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    yy[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    yy[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
                yy += 128;
                ql += 64;
                qh += 32;
                sc += 8;
            }
        }
    } else if (type == OR_MXFP4) {
        const blk_mxfp4 *x = (const blk_mxfp4 *)vx;
        for (int64_t i = 0; i < k / QK_MXFP4; i++) {
            const float d = oracle_e8m0_to_fp32_half(x[i].e);
            for (int j = 0; j < 16; j++) {
                y[i * 32 + j] = (float)kvalues_mxfp4[x[i].qs[j] & 0x0F] * d;
                y[i * 32 + 16 + j] = (float)kvalues_mxfp4[x[i].qs[j] >> 4] * d;
            }
        }
    } else if (type == OR_Q8_K) {
        const blk_q8_K *x = (const blk_q8_K *)vx;
        for (int64_t i = 0; i < k / QK_K; i++)
            for (int j = 0; j < QK_K; j++) y[i * QK_K + j] = x[i].d * (float)x[i].qs[j];
    }
}

/* ------------------------------------------------------ integer partials */

/* Exact integer partials of one (weight row, activation row, block).  These
 * are what every route of the reference computes before any float op. */

/* q4_0 x q8_0, one 32-block: sum (nib-8)*q8 (repack.rs:3351 / vec_dot.rs:599) */
static inline int32_t isum_q4_0(const blk_q4_0 *x, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        s += ((x->qs[j] & 0x0F) - 8) * y->qs[j];
        s += ((x->qs[j] >> 4) - 8) * y->qs[16 + j];
    }
    return s;
}

/* unpacked 6-bit scales/mins of a q4_K block (same values as
 * unpack_q4k_scales_bytes, repack.rs:1323) */
static inline void q4k_scales(const blk_q4_K *x, uint8_t s[8], uint8_t m[8]) {
    for (int j = 0; j < 8; j++) get_scale_min_k4(j, x->scales, &s[j], &m[j]);
}

/* q4_K x q8_K, sub-block pair g (elements 64g..64g+63):
 * iacc_g = s_2g*sum(lo*q8) + s_2g+1*sum(hi*q8); imin_g = m_2g*b_lo + m_2g+1*b_hi
 * (repack.rs:1664-1680). */
static inline void isum_q4_K_pair(const blk_q4_K *x, const blk_q8_K *y, int g,
                                  const uint8_t s[8], const uint8_t m[8],
                                  int32_t *iacc, int32_t *imin) {
    int32_t lo = 0, hi = 0;
    for (int e = 0; e < 32; e++) {
        lo += (x->qs[32 * g + e] & 0x0F) * y->qs[64 * g + e];
        hi += (x->qs[32 * g + e] >> 4) * y->qs[64 * g + 32 + e];
    }
    const int32_t b_lo = y->bsums[4 * g] + y->bsums[4 * g + 1];
    const int32_t b_hi = y->bsums[4 * g + 2] + y->bsums[4 * g + 3];
    *iacc = lo * s[2 * g] + hi * s[2 * g + 1];
    *imin = m[2 * g] * b_lo + m[2 * g + 1] * b_hi;
}

/* q6_K value e of a super-block (0..63, unbiased) */
static inline int q6_val(const blk_q6_K *x, int e) {
    const int j = e / 128, k = (e % 128) / 32, ii = e % 32;
    const uint8_t *ql = x->ql + 64 * j, *qh = x->qh + 32 * j;
    switch (k) {
    case 0: return (ql[ii] & 0x0F) | ((qh[ii] & 0x03) << 4);
    case 1: return (ql[32 + ii] & 0x0F) | (((qh[ii] >> 2) & 0x03) << 4);
    case 2: return (ql[ii] >> 4) | (qh[ii] & 0x30);
    default: return (ql[32 + ii] >> 4) | ((qh[ii] & 0xC0) >> 2);
    }
}

/* q6_K x q8_K, whole super-block: sum_s scale_s * sum (q6-32)*q8 */
static inline int32_t isum_q6_K(const blk_q6_K *x, const blk_q8_K *y) {
    int32_t s = 0;
    for (int sb = 0; sb < 16; sb++) {
        int32_t t = 0;
        for (int e = 16 * sb; e < 16 * sb + 16; e++) t += (q6_val(x, e) - 32) * y->qs[e];
        s += t * x->scales[sb];
    }
    return s;
}

/* mxfp4 x q8_0, one 32-block (repack.rs:1048-1075) */
static inline int32_t isum_mxfp4(const blk_mxfp4 *x, const blk_q8_0 *y) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        s += kvalues_mxfp4[x->qs[j] & 0x0F] * y->qs[j];
        s += kvalues_mxfp4[x->qs[j] >> 4] * y->qs[16 + j];
    }
    return s;
}

/* ------------------------------------------- dots in the reference order */

/* vec_dot.rs:564 hsum8 */
static inline float hsum8(const float a[8]) {
    float r[4];
    for (int i = 0; i < 4; i++) r[i] = a[i + 4] + a[i];
    const float s0 = r[0] + r[2], s1 = r[1] + r[3];
    return s0 + s1;
}

/* vec_dot.rs:599-618 */
float oracle_vec_dot_q4_0_q8_0(int n, const void *vx, const void *vy) {
    const blk_q4_0 *x = (const blk_q4_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float acc[8] = {0};
    for (int ib = 0; ib < n / QK8_0; ib++) {
        const float d = H2F(x[ib].d) * H2F(y[ib].d);
        for (int l = 0; l < 8; l++) {
            int32_t q = 0;
            for (int i = 0; i < 4; i++) {
                const int e = 4 * l + i;
                const int v = e < 16 ? (x[ib].qs[e] & 0x0F) : (x[ib].qs[e - 16] >> 4);
                q += (v - 8) * y[ib].qs[e];
            }
            acc[l] = fmaf(d, (float)q, acc[l]);
        }
    }
    return hsum8(acc);
}

/* vec_dot.rs:872-918 */
float oracle_vec_dot_q4_K_q8_K(int n, const void *vx, const void *vy) {
    const blk_q4_K *x = (const blk_q4_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0}, acc_m[4] = {0};
    for (int i = 0; i < n / QK_K; i++) {
        const float d = y[i].d * H2F(x[i].d);
        const float dmin = -y[i].d * H2F(x[i].dmin);
        uint8_t sc[8], mn[8];
        q4k_scales(&x[i], sc, mn);
        for (int l = 0; l < 4; l++) {
            const int32_t lo = y[i].bsums[4 * l] + y[i].bsums[4 * l + 1];
            const int32_t hi = y[i].bsums[4 * l + 2] + y[i].bsums[4 * l + 3];
            const int32_t prod = mn[2 * l] * lo + mn[2 * l + 1] * hi;
            acc_m[l] = fmaf(dmin, (float)prod, acc_m[l]);
        }
        int32_t sumi[8] = {0};
        for (int j = 0; j < QK_K / 64; j++) {
            for (int l = 0; l < 8; l++) {
                int32_t a = 0, b = 0;
                for (int ii = 0; ii < 4; ii++) {
                    const int e = 4 * l + ii;
                    a += (x[i].qs[32 * j + e] & 0x0F) * y[i].qs[64 * j + e];
                    b += (x[i].qs[32 * j + e] >> 4) * y[i].qs[64 * j + 32 + e];
                }
                sumi[l] += sc[2 * j] * a + sc[2 * j + 1] * b;
            }
        }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    const float m0 = acc_m[0] + acc_m[2], m1 = acc_m[1] + acc_m[3];
    return hsum8(acc) + (m0 + m1);
}

/* vec_dot.rs:990-1040 */
float oracle_vec_dot_q6_K_q8_K(int n, const void *vx, const void *vy) {
    const blk_q6_K *x = (const blk_q6_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0};
    for (int i = 0; i < n / QK_K; i++) {
        const float d = y[i].d * H2F(x[i].d);
        const int8_t *sc = x[i].scales;
        int32_t sumi[8] = {0};
        for (int j = 0; j < 2; j++)
            for (int k = 0; k < 4; k++)
                for (int ii = 0; ii < 32; ii++) {
                    const int e = 128 * j + 32 * k + ii;
                    const int val = q6_val(&x[i], e);
                    const int s = sc[8 * j + 2 * k + (ii >= 16)];
                    sumi[ii / 4] += s * y[i].qs[e] * val;
                }
        for (int l = 0; l < 8; l++) {
            const int32_t sub = (y[i].bsums[2 * l] * sc[2 * l] + y[i].bsums[2 * l + 1] * sc[2 * l + 1]) << 5;
            sumi[l] -= sub;
            acc[l] = fmaf(d, (float)sumi[l], acc[l]);
        }
    }
    return hsum8(acc);
}

/* vec_dot.rs:661-686: lane l holds elements 4l..4l+3, one fma per block */
/* vec_dot.rs:620-650 vec_dot_q4_1_q8_1 (the AVX2 kernel's order, as its
 * scalar twin): 8 lane accumulators acc[l] = fma(dx*dy, q_l, acc[l]) over the
 * 4-element lanes, summs = fma(m, s, summs), result hsum8(acc) + summs */
float oracle_vec_dot_q4_1_q8_1(int n, const void *vx, const void *vy) {
    const blk_q4_1 *x = (const blk_q4_1 *)vx;
    const blk_q8_1 *y = (const blk_q8_1 *)vy;
    float acc[8] = {0}, summs = 0.0f;
    for (int ib = 0; ib < n / 32; ib++) {
        const float d0d1 = H2F(x[ib].d) * H2F(y[ib].d);
        summs = fmaf(H2F(x[ib].m), H2F(y[ib].s), summs);
        for (int l = 0; l < 8; l++) {
            int32_t q = 0;
            for (int i = 0; i < 4; i++) q += q4_1_val(&x[ib], 4 * l + i) * y[ib].qs[4 * l + i];
            acc[l] = fmaf(d0d1, (float)q, acc[l]);
        }
    }
    return hsum8(acc) + summs;
}

/* vec_dot.rs:687-720 vec_dot_q5_1_q8_1: as q4_1 with the fifth bit */
float oracle_vec_dot_q5_1_q8_1(int n, const void *vx, const void *vy) {
    const blk_q5_1 *x = (const blk_q5_1 *)vx;
    const blk_q8_1 *y = (const blk_q8_1 *)vy;
    float acc[8] = {0}, summs = 0.0f;
    for (int ib = 0; ib < n / 32; ib++) {
        const float dxdy = H2F(x[ib].d) * H2F(y[ib].d);
        summs = fmaf(H2F(x[ib].m), H2F(y[ib].s), summs);
        for (int l = 0; l < 8; l++) {
            int32_t q = 0;
            for (int i = 0; i < 4; i++) q += q5_1_val(&x[ib], 4 * l + i) * y[ib].qs[4 * l + i];
            acc[l] = fmaf(dxdy, (float)q, acc[l]);
        }
    }
    return hsum8(acc) + summs;
}

/* vec_dot.rs:758-797 vec_dot_q2_K_q8_K (the AVX2 kernel's order): per block
 * the min term first, acc[l] = fma(-d8*dmin, (sc>>4)[2l]*bsums[2l] +
 * (sc>>4)[2l+1]*bsums[2l+1], acc[l]); then sumi[l] over the 4-element lanes
 * e = 4l .. 4l+3 of every 32-value shift group scaled by sc[8j+2k+(l>=4)] & 15,
 * acc[l] = fma(d8*d, sumi[l], acc[l]); result hsum8(acc) */
float oracle_vec_dot_q2_K_q8_K(int n, const void *vx, const void *vy) {
    const blk_q2_K *x = (const blk_q2_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0};
    for (int i = 0; i < n / QK_K; i++) {
        const float d = y[i].d * H2F(x[i].d);
        const float dmin = -y[i].d * H2F(x[i].dmin);
        for (int l = 0; l < 8; l++) {
            const int32_t prod = (x[i].scales[2 * l] >> 4) * y[i].bsums[2 * l] +
                                 (x[i].scales[2 * l + 1] >> 4) * y[i].bsums[2 * l + 1];
            acc[l] = fmaf(dmin, (float)prod, acc[l]);
        }
        int32_t sumi[8] = {0};
        for (int j = 0; j < 2; j++)
            for (int k = 0; k < 4; k++)
                for (int l = 0; l < 8; l++) {
                    const int sc = x[i].scales[8 * j + 2 * k + (l >= 4)] & 0x0F;
                    int32_t s = 0;
                    for (int ii = 0; ii < 4; ii++)
                        s += q2k_val(&x[i], j, k, 4 * l + ii) * y[i].qs[128 * j + 32 * k + 4 * l + ii];
                    sumi[l] += sc * s;
                }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    return hsum8(acc);
}

/* vec_dot.rs:801-834 vec_dot_q3_K_q8_K (the AVX2 kernel's order): scales
 * sc - 32, values lo - 4 * (hmask bit clear), sumi[l] as for Q2_K,
 * acc[l] = fma(d8*d, sumi[l], acc[l]); result hsum8(acc) */
float oracle_vec_dot_q3_K_q8_K(int n, const void *vx, const void *vy) {
    const blk_q3_K *x = (const blk_q3_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0};
    for (int i = 0; i < n / QK_K; i++) {
        const float d = y[i].d * H2F(x[i].d);
        int sc[16];
        q3k_scales_u(x[i].scales, sc);
        int32_t sumi[8] = {0};
        for (int j = 0; j < 2; j++)
            for (int k = 0; k < 4; k++)
                for (int l = 0; l < 8; l++) {
                    const int s6 = sc[8 * j + 2 * k + (l >= 4)] - 32;
                    int32_t s = 0;
                    for (int ii = 0; ii < 4; ii++)
                        s += q3k_val(&x[i], j, k, 4 * l + ii) * y[i].qs[128 * j + 32 * k + 4 * l + ii];
                    sumi[l] += s6 * s;
                }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    return hsum8(acc);
}

float oracle_vec_dot_q5_0_q8_0(int n, const void *vx, const void *vy) {
    const blk_q5_0 *x = (const blk_q5_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float acc[8] = {0};
    for (int ib = 0; ib < n / QK8_0; ib++) {
        const float d = H2F(x[ib].d) * H2F(y[ib].d);
        for (int l = 0; l < 8; l++) {
            int32_t q = 0;
            for (int i = 0; i < 4; i++) q += q5_0_val(&x[ib], 4 * l + i) * y[ib].qs[4 * l + i];
            acc[l] = fmaf(d, (float)q, acc[l]);
        }
    }
    return hsum8(acc);
}

/* vec_dot.rs:732-756 */
float oracle_vec_dot_q8_0_q8_0(int n, const void *vx, const void *vy) {
    const blk_q8_0 *x = (const blk_q8_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float acc[8] = {0};
    for (int ib = 0; ib < n / QK8_0; ib++) {
        const float d = H2F(x[ib].d) * H2F(y[ib].d);
        for (int l = 0; l < 8; l++) {
            int32_t q = 0;
            for (int i = 0; i < 4; i++) q += x[ib].qs[4 * l + i] * y[ib].qs[4 * l + i];
            acc[l] = fmaf(d, (float)q, acc[l]);
        }
    }
    return hsum8(acc);
}

/* vec_dot.rs:928-980: the min term folds into one scalar per super-block
 * first (summs), then eight lanes of scaled 5-bit sums */
float oracle_vec_dot_q5_K_q8_K(int n, const void *vx, const void *vy) {
    const blk_q5_K *x = (const blk_q5_K *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0}, summs = 0.0f;
    for (int i = 0; i < n / QK_K; i++) {
        const float d = y[i].d * H2F(x[i].d);
        const float dmin = -y[i].d * H2F(x[i].dmin);
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) get_scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        int32_t m = 0;
        for (int l = 0; l < 4; l++) {
            const int32_t lo = y[i].bsums[4 * l] + y[i].bsums[4 * l + 1];
            const int32_t hi = y[i].bsums[4 * l + 2] + y[i].bsums[4 * l + 3];
            m += mn[2 * l] * lo + mn[2 * l + 1] * hi;
        }
        summs = fmaf((float)m, dmin, summs);
        int32_t sumi[8] = {0};
        for (int j = 0; j < QK_K / 64; j++)
            for (int l = 0; l < 8; l++) {
                int32_t a = 0, b = 0;
                for (int ii = 0; ii < 4; ii++) {
                    const int e = 4 * l + ii;
                    a += q5k_lo(&x[i], j, e) * y[i].qs[64 * j + e];
                    b += q5k_hi(&x[i], j, e) * y[i].qs[64 * j + 32 + e];
                }
                sumi[l] += sc[2 * j] * a + sc[2 * j + 1] * b;
            }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    return hsum8(acc) + summs;
}

/* ------------------------------------------------------- routed MUL_MAT */

/* vec_dot.rs:1597-1650 vec_dot_iq4_nl_q8_0: block pairs into two 8-lane
 * accumulators (lane l = elements 4l..4l+3), fma(y.d * x.d, lane sum, acc),
 * added lane-wise before one hsum8; an odd last block adds d * (sumi1 + sumi2) */
float oracle_vec_dot_iq4_nl_q8_0(int n, const void *vx, const void *vy) {
    const blk_iq4_nl *x = (const blk_iq4_nl *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    const int nb = n / 32;
    float acc1[8] = {0}, acc2[8] = {0};
    int ib = 0;
    for (; ib + 1 < nb; ib += 2) {
        const float d0 = H2F(y[ib].d) * H2F(x[ib].d), d1 = H2F(y[ib + 1].d) * H2F(x[ib + 1].d);
        for (int l = 0; l < 8; l++) {
            int32_t s0 = 0, s1 = 0;
            for (int t = 0; t < 4; t++) {
                s0 += iq4_val(x[ib].qs, 4 * l + t) * y[ib].qs[4 * l + t];
                s1 += iq4_val(x[ib + 1].qs, 4 * l + t) * y[ib + 1].qs[4 * l + t];
            }
            acc1[l] = fmaf(d0, (float)s0, acc1[l]);
            acc2[l] = fmaf(d1, (float)s1, acc2[l]);
        }
    }
    float a[8];
    for (int l = 0; l < 8; l++) a[l] = acc1[l] + acc2[l];
    float sumf = hsum8(a);
    for (; ib < nb; ib++) {
        const float d = H2F(y[ib].d) * H2F(x[ib].d);
        int32_t s1 = 0, s2 = 0;
        for (int j = 0; j < 16; j++) {
            s1 += y[ib].qs[j] * kvalues_iq4nl[x[ib].qs[j] & 0xF];
            s2 += y[ib].qs[j + 16] * kvalues_iq4nl[x[ib].qs[j] >> 4];
        }
        sumf += d * (float)(s1 + s2);
    }
    return sumf;
}

/* vec_dot.rs:1655-1700 vec_dot_iq4_xs_q8_K: per super-block d = x.d * y.d,
 * sumi[l] += (ls - 32) * (lane l's 4-element sum) over the 8 groups,
 * acc[l] = fma(d, sumi[l], acc[l]); hsum8 */
float oracle_vec_dot_iq4_xs_q8_K(int n, const void *vx, const void *vy) {
    const blk_iq4_xs *x = (const blk_iq4_xs *)vx;
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0};
    for (int i = 0; i < n / QK_K; i++) {
        const float d = H2F(x[i].d) * y[i].d;
        int32_t sumi[8] = {0};
        for (int ib = 0; ib < 8; ib++) {
            const int ls = iq4xs_ls(&x[i], ib);
            for (int l = 0; l < 8; l++) {
                int32_t s = 0;
                for (int t = 0; t < 4; t++) s += iq4_val(x[i].qs + 16 * ib, 4 * l + t) * y[i].qs[32 * ib + 4 * l + t];
                sumi[l] += ls * s;
            }
        }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
    }
    return hsum8(acc);
}

/* vec_dot.rs:1154-1210 vec_dot_nvfp4_q8_0: per 64-block the sub-block scales
 * s_k = ue4m3(d_k) * y.d of the Q8_0 block holding them; lane l of half h
 * sums elements 4l..4l+3 of that half (lanes 0-3 sub-block 2h, 4-7 sub-block
 * 2h+1); acc[l] = fma(s, p1[l], acc[l]) for half 0, then half 1; hsum8 */
float oracle_vec_dot_nvfp4_q8_0(int n, const void *vx, const void *vy) {
    const blk_nvfp4 *x = (const blk_nvfp4 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float acc[8] = {0};
    for (int ib = 0; ib < n / 64; ib++) {
        const float dy0 = H2F(y[2 * ib].d), dy1 = H2F(y[2 * ib + 1].d);
        const float sc[4] = {oracle_ue4m3_to_fp32(x[ib].d[0]) * dy0, oracle_ue4m3_to_fp32(x[ib].d[1]) * dy0,
                             oracle_ue4m3_to_fp32(x[ib].d[2]) * dy1, oracle_ue4m3_to_fp32(x[ib].d[3]) * dy1};
        int32_t p[2][8];
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 8; l++) {
                int32_t s = 0;
                for (int t = 0; t < 4; t++) {
                    const int e = 4 * l + t;
                    s += nvfp4_val(&x[ib], 32 * h + e) * y[2 * ib + h].qs[e];
                }
                p[h][l] = s;
            }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(sc[l < 4 ? 0 : 1], (float)p[0][l], acc[l]);
        for (int l = 0; l < 8; l++) acc[l] = fmaf(sc[l < 4 ? 2 : 3], (float)p[1][l], acc[l]);
    }
    return hsum8(acc);
}

/* vec_dot.rs:1074-1116 vec_dot_q1_0_q8_0: per 128-block, per Q8_0 block k the
 * 8 lane sums of +-q8 (lane l = elements 4l..4l+3); acc_block = dy0 * s (k = 0,
 * a plain product), then fma(dy_k, s, acc_block); acc = fma(d, acc_block, acc) */
float oracle_vec_dot_q1_0_q8_0(int n, const void *vx, const void *vy) {
    const blk_q1_0 *x = (const blk_q1_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float acc[8] = {0};
    for (int ib = 0; ib < n / 128; ib++) {
        const float d0 = H2F(x[ib].d);
        float ab[8] = {0};
        for (int k = 0; k < 4; k++) {
            const blk_q8_0 *yk = &y[ib * 4 + k];
            const float dy = H2F(yk->d);
            for (int l = 0; l < 8; l++) {
                int32_t s = 0;
                for (int i = 0; i < 4; i++) s += q1_0_val(&x[ib], 32 * k + 4 * l + i) * yk->qs[4 * l + i];
                ab[l] = k == 0 ? dy * (float)s : fmaf(dy, (float)s, ab[l]);
            }
        }
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d0, ab[l], acc[l]);
    }
    return hsum8(acc);
}

/* vec_dot.rs:1120-1148 vec_dot_q2_0_q8_0 (the generic kernel): per 64-block
 * sumi = sum_k dy_k * sumi_block_k (in order), sumf += d * sumi */
float oracle_vec_dot_q2_0_q8_0(int n, const void *vx, const void *vy) {
    const blk_q2_0 *x = (const blk_q2_0 *)vx;
    const blk_q8_0 *y = (const blk_q8_0 *)vy;
    float sumf = 0.0f;
    for (int i = 0; i < n / 64; i++) {
        const float d0 = H2F(x[i].d);
        float sumi = 0.0f;
        for (int k = 0; k < 2; k++) {
            const blk_q8_0 *yk = &y[i * 2 + k];
            int32_t sb = 0;
            for (int b = 0; b < 8; b++) {
                const uint8_t byte = x[i].qs[8 * k + b];
                sb += ((byte & 3) - 1) * yk->qs[4 * b];
                sb += (((byte >> 2) & 3) - 1) * yk->qs[4 * b + 1];
                sb += (((byte >> 4) & 3) - 1) * yk->qs[4 * b + 2];
                sb += (((byte >> 6) & 3) - 1) * yk->qs[4 * b + 3];
            }
            sumi += H2F(yk->d) * (float)sb;
        }
        sumf += d0 * sumi;
    }
    return sumf;
}


/* ---------------------------------------------------------------- IQ1 / IQ2 / IQ3
 * Block layouts (blocks.rs:178-232) and the row dots of vec_dot.rs:1215-1590.
 * Each *_lanes function forms the reference's eight lane sums sumi[l] of one
 * super-block (lane l: elements 4l..4l+3 of every 32-element block, times the
 * block's scale) exactly; the IQ1 types also their delta sums. */
typedef struct { uint16_t d; uint16_t qs[32]; } blk_iq2_xxs;                                   /* 66 B */
typedef struct { uint16_t d; uint16_t qs[32]; uint8_t scales[8]; } blk_iq2_xs;                  /* 74 B */
typedef struct { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t scales[8]; } blk_iq2_s;     /* 82 B */
typedef struct { uint16_t d; uint8_t qs[96]; } blk_iq3_xxs;                                    /* 98 B */
typedef struct { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t signs[32]; uint8_t scales[4]; } blk_iq3_s; /* 110 B */
typedef struct { uint16_t d; uint8_t qs[32]; uint16_t qh[8]; } blk_iq1_s;                      /* 50 B */
typedef struct { uint8_t qs[32]; uint8_t qh[16]; uint8_t scales[8]; } blk_iq1_m;               /* 56 B */

/* KSIGNS_IQ2XS (quants_k.rs:42): the 7 stored sign bits and their odd-parity bit */
static inline int iq_sign(uint32_t s7, int e) {
    const uint32_t s8 = s7 | ((uint32_t)__builtin_parity(s7) << 7);
    return (s8 >> e) & 1 ? -1 : 1;
}
static inline int grid8(const uint64_t *g, uint32_t idx, int e) { return (int)((g[idx] >> (8 * e)) & 0xFF); }
static inline int grid4(const uint32_t *g, uint32_t idx, int e) { return (int)((g[idx] >> (8 * e)) & 0xFF); }

/* vec_dot.rs:1215-1255 */
static void iq2_xxs_lanes(const blk_iq2_xxs *x, const blk_q8_K *y, int32_t sumi[8]) {
    for (int l = 0; l < 8; l++) sumi[l] = 0;
    int q8i = 0;
    for (int it = 0; it < 4; it++) {
        /* the 8 u16 of this 64-element group (qs[8 it .. 8 it + 7]) as 4 words */
        uint32_t aux32[4];
        for (int k = 0; k < 4; k++) aux32[k] = (uint32_t)x->qs[8 * it + 2 * k] | ((uint32_t)x->qs[8 * it + 2 * k + 1] << 16);
        for (int h = 0; h < 2; h++) {
            const uint32_t signs_word = aux32[1 + 2 * h];
            const int ls = 2 * (int)(signs_word >> 28) + 1;
            for (int l = 0; l < 8; l++) {
                int s = 0;
                for (int t = 0; t < 4; t++) {
                    const int e = 4 * l + t;
                    const int j = 8 * h + e / 8;
                    const uint32_t idx = (aux32[j / 4] >> (8 * (j % 4))) & 0xFF;
                    const int g = grid8(ghip_iq2xxs_grid, idx, e % 8);
                    s += g * iq_sign((signs_word >> (7 * (e / 8))) & 127, e % 8) * y->qs[q8i + e];
                }
                sumi[l] += ls * s;
            }
            q8i += 32;
        }
    }
}
/* vec_dot.rs:1266-1305 */
static void iq2_xs_lanes(const blk_iq2_xs *x, const blk_q8_K *y, int32_t sumi[8]) {
    for (int l = 0; l < 8; l++) sumi[l] = 0;
    int q8i = 0;
    for (int it = 0; it < 2; it++)
        for (int c = 0; c < 4; c++) {
            const int b = 4 * it + c;
            const int sc_lo = 2 * (x->scales[b] & 0x0F) + 1, sc_hi = 2 * (x->scales[b] >> 4) + 1;
            for (int l = 0; l < 8; l++) {
                const int sc = l < 4 ? sc_lo : sc_hi;
                int s = 0;
                for (int t = 0; t < 4; t++) {
                    const int e = 4 * l + t;
                    const uint32_t q2 = x->qs[16 * it + 4 * c + e / 8];
                    s += grid8(ghip_iq2xs_grid, q2 & 511, e % 8) * iq_sign((q2 >> 9) & 127, e % 8) * y->qs[q8i + e];
                }
                sumi[l] += sc * s;
            }
            q8i += 32;
        }
}
/* vec_dot.rs:1312-1352 */
static void iq2_s_lanes(const blk_iq2_s *x, const blk_q8_K *y, int32_t sumi[8]) {
    for (int l = 0; l < 8; l++) sumi[l] = 0;
    int q8i = 0;
    for (int t = 0; t < 4; t++)
        for (int h = 0; h < 2; h++) {
            const int v = 2 * t + h;
            const int sc_lo = 2 * (x->scales[v] & 0x0F) + 1, sc_hi = 2 * (x->scales[v] >> 4) + 1;
            for (int l = 0; l < 8; l++) {
                const int sc = l < 4 ? sc_lo : sc_hi;
                int s = 0;
                for (int tt = 0; tt < 4; tt++) {
                    const int e = 4 * l + tt, k = e / 8;
                    const uint32_t idx = (uint32_t)x->qs[8 * t + 4 * h + k] | (((uint32_t)x->qh[v] << (8 - 2 * k)) & 0x300);
                    const int sgn = (x->qs[32 + 8 * t + 4 * h + k] >> (e % 8)) & 1 ? -1 : 1;
                    s += grid8(ghip_iq2s_grid, idx, e % 8) * sgn * y->qs[q8i + e];
                }
                sumi[l] += sc * s;
            }
            q8i += 32;
        }
}
/* vec_dot.rs:1358-1397 */
static void iq3_xxs_lanes(const blk_iq3_xxs *x, const blk_q8_K *y, int32_t sumi[8]) {
    for (int l = 0; l < 8; l++) sumi[l] = 0;
    int q8i = 0;
    for (int it = 0; it < 4; it++)
        for (int h = 0; h < 2; h++) {
            const int gas = 64 + 8 * it + 4 * h;
            uint32_t signs_word;
            memcpy(&signs_word, x->qs + gas, 4);
            const int ls = 2 * (int)(signs_word >> 28) + 1;
            for (int l = 0; l < 8; l++) {
                int s = 0;
                for (int t = 0; t < 4; t++) {
                    const int e = 4 * l + t;
                    const uint32_t idx = x->qs[16 * it + 8 * h + e / 4];
                    s += grid4(ghip_iq3xxs_grid, idx, e % 4) * iq_sign((signs_word >> (7 * (e / 8))) & 127, e % 8) *
                         y->qs[q8i + e];
                }
                sumi[l] += ls * s;
            }
            q8i += 32;
        }
}
/* vec_dot.rs:1403-1450 */
static void iq3_s_lanes(const blk_iq3_s *x, const blk_q8_K *y, int32_t sumi[8]) {
    for (int l = 0; l < 8; l++) sumi[l] = 0;
    int q8i = 0, qsi = 0;
    for (int t = 0; t < 4; t++) {
        for (int h = 0; h < 2; h++) {
            const int v = 2 * t + h;
            const uint32_t qhv = x->qh[v];
            const int ls = h == 0 ? 2 * (x->scales[t] & 0x0F) + 1 : 2 * (x->scales[t] >> 4) + 1;
            for (int l = 0; l < 8; l++) {
                int s = 0;
                for (int tt = 0; tt < 4; tt++) {
                    const int e = 4 * l + tt, k = e / 4;
                    const uint32_t idx = (uint32_t)x->qs[qsi + 8 * h + k] | ((qhv << (8 - k)) & 256);
                    const int sgn = (x->signs[8 * t + 4 * h + e / 8] >> (e % 8)) & 1 ? -1 : 1;
                    s += grid4(ghip_iq3s_grid, idx, e % 4) * sgn * y->qs[q8i + e];
                }
                sumi[l] += ls * s;
            }
            q8i += 32;
        }
        qsi += 16;
    }
}
/* vec_dot.rs:1460-1510; *sumi1: the delta sum (bsum pairs * sign * ls) */
static void iq1_s_lanes(const blk_iq1_s *x, const blk_q8_K *y, int32_t sumi[8], int32_t *sumi1) {
    for (int l = 0; l < 8; l++) sumi[l] = 0;
    *sumi1 = 0;
    int q8i = 0, qsi = 0;
    for (int t = 0; t < 4; t++) {
        for (int j = 0; j < 2; j++) {
            const uint32_t qhw = x->qh[2 * t + j];
            const int ls = 2 * (int)((qhw >> 12) & 7) + 1;
            for (int l = 0; l < 8; l++) {
                int s = 0;
                for (int tt = 0; tt < 4; tt++) {
                    const int e = 4 * l + tt, k = e / 8;
                    const int shift = 8 - 3 * k;
                    const uint32_t qhi = shift >= 0 ? qhw << shift : qhw >> 1;
                    const uint32_t idx = (uint32_t)x->qs[qsi + 4 * j + k] | (qhi & 0x700);
                    const int v = (int)(int8_t)(uint8_t)((ghip_iq1s_grid[idx] >> (8 * (e % 8))) & 0xFF);
                    s += v * y->qs[q8i + e];
                }
                sumi[l] += ls * s;
            }
            const int sg = qhw & 0x8000 ? -1 : 1;
            *sumi1 += ((int)y->bsums[4 * t + 2 * j] + (int)y->bsums[4 * t + 2 * j + 1]) * sg * ls;
            q8i += 32;
        }
        qsi += 8;
    }
}
static inline float iq1m_d(const blk_iq1_m *x) {
    uint16_t sc[4];
    for (int m = 0; m < 4; m++) sc[m] = (uint16_t)(x->scales[2 * m] | (x->scales[2 * m + 1] << 8));
    const uint16_t u = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000));
    return H2F(u);
}
/* vec_dot.rs:1525-1590; sumi2: the delta lane sums */
static void iq1_m_lanes(const blk_iq1_m *x, const blk_q8_K *y, int32_t sumi1[8], int32_t sumi2[8]) {
    for (int l = 0; l < 8; l++) sumi1[l] = sumi2[l] = 0;
    int q8i = 0, qsi = 0, qhi = 0;
    for (int t = 0; t < 4; t++) {
        const uint32_t sct = (uint32_t)(x->scales[2 * t] | (x->scales[2 * t + 1] << 8));
        const int scv[2][2] = {{2 * (int)(sct & 7) + 1, 2 * (int)((sct >> 3) & 7) + 1},
                               {2 * (int)((sct >> 6) & 7) + 1, 2 * (int)((sct >> 9) & 7) + 1}};
        for (int j = 0; j < 2; j++) {
            for (int l = 0; l < 8; l++) {
                const int scl = scv[j][l >= 4];
                int s = 0, sd = 0;
                for (int tt = 0; tt < 4; tt++) {
                    const int e = 4 * l + tt, k = e / 8;
                    const uint32_t qhb = x->qh[qhi + 2 * j + k / 2];
                    const uint32_t idx = (uint32_t)x->qs[qsi + 4 * j + k] | ((qhb << (8 - 4 * (k % 2))) & 0x700);
                    const int v = (int)(int8_t)(uint8_t)((ghip_iq1s_grid[idx] >> (8 * (e % 8))) & 0xFF);
                    s += v * y->qs[q8i + e];
                    const int dsgn = qhb & (k % 2 == 0 ? 0x08 : 0x80) ? -1 : 1;
                    sd += dsgn * y->qs[q8i + e];
                }
                sumi1[l] += scl * s;
                sumi2[l] += scl * sd;
            }
            q8i += 32;
        }
        qsi += 8;
        qhi += 4;
    }
}

int oracle_iq_block_bytes(int type) {
    switch (type) {
    case OR_IQ2_XXS: return 66;
    case OR_IQ2_XS: return 74;
    case OR_IQ2_S: return 82;
    case OR_IQ3_XXS: return 98;
    case OR_IQ3_S: return 110;
    case OR_IQ1_S: return 50;
    case OR_IQ1_M: return 56;
    default: return 0;
    }
}
/* one super-block: the eight lane sums (the reference's accumulator input),
 * the delta lane sums (IQ1, else zero), the weight scale d (f32) and the
 * exact integer the tiled kernel forms (tiled.rs:440-640: the weights as
 * grid * sign, IQ1 as 8 * grid + delta, times the sub-block scales) */
static void iq_super_block(int type, const uint8_t *xb, const blk_q8_K *y, int32_t s[8], int32_t s2[8], float *d,
                           int32_t *is) {
    int32_t one = 0;
    for (int l = 0; l < 8; l++) s2[l] = 0;
    switch (type) {
    case OR_IQ2_XXS: iq2_xxs_lanes((const blk_iq2_xxs *)xb, y, s); *d = H2F(((const blk_iq2_xxs *)xb)->d); break;
    case OR_IQ2_XS: iq2_xs_lanes((const blk_iq2_xs *)xb, y, s); *d = H2F(((const blk_iq2_xs *)xb)->d); break;
    case OR_IQ2_S: iq2_s_lanes((const blk_iq2_s *)xb, y, s); *d = H2F(((const blk_iq2_s *)xb)->d); break;
    case OR_IQ3_XXS: iq3_xxs_lanes((const blk_iq3_xxs *)xb, y, s); *d = H2F(((const blk_iq3_xxs *)xb)->d); break;
    case OR_IQ3_S: iq3_s_lanes((const blk_iq3_s *)xb, y, s); *d = H2F(((const blk_iq3_s *)xb)->d); break;
    case OR_IQ1_S: iq1_s_lanes((const blk_iq1_s *)xb, y, s, &one); *d = H2F(((const blk_iq1_s *)xb)->d); break;
    default: iq1_m_lanes((const blk_iq1_m *)xb, y, s, s2); *d = iq1m_d((const blk_iq1_m *)xb); break;
    }
    int32_t a = 0, b = 0;
    for (int l = 0; l < 8; l++) a += s[l], b += s2[l];
    *is = type == OR_IQ1_S ? 8 * a + one : type == OR_IQ1_M ? 8 * a + b : a;
    if (type == OR_IQ1_S) s2[0] = one; /* the caller reads IQ1_S's delta sum from s2[0] */
}
/* the vec_dot final scale: 0.125 (IQ2), 0.25 (IQ3_XXS), 1 (IQ3_S) -- and for
 * the tiled kernel the factor folded into its d (tiled.rs:454-618) */
static float iq_scale(int type) {
    return type == OR_IQ3_XXS ? 0.25f : type == OR_IQ3_S ? 1.0f : 0.125f;
}

/* the row dot of vec_dot.rs:1215-1590: per super-block d = d_w * d8 (IQ1_S:
 * d8 * d_w), acc[l] = fma(d, sumi[l], acc[l]); IQ1_S adds the delta chain
 * accum1 = fma(d, sumi1, accum1) and IQ1_M a second accumulator set */
float oracle_vec_dot_iq(int type, int n, const void *vx, const void *vy) {
    const int bs = oracle_iq_block_bytes(type);
    const blk_q8_K *y = (const blk_q8_K *)vy;
    float acc[8] = {0}, acc2[8] = {0}, accum1 = 0.0f;
    for (int i = 0; i < n / QK_K; i++) {
        int32_t s[8], s2[8], is;
        float dw;
        iq_super_block(type, (const uint8_t *)vx + (size_t)i * bs, &y[i], s, s2, &dw, &is);
        const float d = (type == OR_IQ1_S || type == OR_IQ1_M) ? y[i].d * dw : dw * y[i].d;
        for (int l = 0; l < 8; l++) acc[l] = fmaf(d, (float)s[l], acc[l]);
        if (type == OR_IQ1_S) accum1 = fmaf(d, (float)s2[0], accum1);
        if (type == OR_IQ1_M)
            for (int l = 0; l < 8; l++) acc2[l] = fmaf(d, (float)s2[l], acc2[l]);
    }
    if (type == OR_IQ1_S) return hsum8(acc) + 0.125f * accum1;
    if (type == OR_IQ1_M) return hsum8(acc) + 0.125f * hsum8(acc2);
    return iq_scale(type) * hsum8(acc);
}

static int omp_threads(int nthreads) {
#ifdef _OPENMP
    return nthreads > 0 ? nthreads : omp_get_max_threads();
#else
    (void)nthreads;
    return 1;
#endif
}

static int route_of(int type, int64_t rows, int64_t cols) {
    if ((type == OR_Q4_0 || type == OR_Q4_K) && rows % 8 == 0) return ORACLE_ROUTE_REPACK;
    /* tiled.rs:203-242 formats, from 8 columns (tiled.rs:1300) */
    if ((type == OR_Q4_K || type == OR_Q5_K || type == OR_Q6_K || type == OR_Q2_K || type == OR_Q3_K ||
         type == OR_IQ4_XS || oracle_iq_block_bytes(type)) && cols >= 8)
        return ORACLE_ROUTE_TILED;
    if (type == OR_Q4_0 && cols >= 2) return -1; /* tinyBLAS: out of scope */
    return ORACLE_ROUTE_VECDOT;
}

/* vec_dot_type Q8_0 (vec_dot.rs:1727) */
static int q8_0_dot(int type) {
    return type == OR_Q4_0 || type == OR_Q5_0 || type == OR_Q8_0 || type == OR_IQ4_NL || type == OR_NVFP4 ||
           type == OR_Q1_0 || type == OR_Q2_0;
}
static size_t act_row_size(int type, int64_t n) {
    if (type == OR_Q4_1 || type == OR_Q5_1) return (size_t)(n / 32) * sizeof(blk_q8_1);
    return q8_0_dot(type) ? (size_t)(n / 32) * sizeof(blk_q8_0) : (size_t)(n / QK_K) * sizeof(blk_q8_K);
}

/* compute.rs:1504-1549 (wdata pass) and compute.rs:5350-5398 (repack wdata) */
int oracle_mul_mat_act(int type, int64_t n, int64_t rows, const float *x, int64_t cols, void *act) {
    const int route = route_of(type, rows, cols);
    if (route < 0) return -1;
    const size_t rs = act_row_size(type, n);
    const int64_t nr4 = cols - cols % 4;
    for (int64_t c = 0; c < cols; c++) {
        uint8_t *dst = (uint8_t *)act + (size_t)c * rs;
        if (q8_0_dot(type))
            oracle_quantize_row_q8_0(x + c * n, dst, n);
        else if (type == OR_Q4_1 || type == OR_Q5_1)  /* vec_dot_type Q8_1 */
            oracle_quantize_row_q8_1(x + c * n, dst, n);
        else if (type == OR_Q4_K && route == ORACLE_ROUTE_REPACK && c < nr4)
            oracle_quantize_row_q8_K_mat(x + c * n, dst, n);
        else
            oracle_quantize_row_q8_K_ref(x + c * n, dst, n);
    }
    return route;
}

int oracle_mul_mat(int type, const void *w, int64_t n, int64_t rows, const float *x, int64_t cols,
                   float *out, int32_t *subsums, int *route_out, int nthreads) {
    const int route = route_of(type, rows, cols);
    if (route_out) *route_out = route;
    if (route < 0) return -1;
    if (type != OR_Q4_0 && type != OR_Q4_K && type != OR_Q6_K && type != OR_Q5_0 && type != OR_Q8_0 &&
        type != OR_Q5_K && type != OR_Q4_1 && type != OR_Q5_1 && type != OR_Q2_K && type != OR_Q3_K &&
        type != OR_IQ4_NL && type != OR_IQ4_XS && type != OR_NVFP4 && type != OR_Q1_0 && type != OR_Q2_0 &&
        !oracle_iq_block_bytes(type))
        return -2;
    const size_t rs = act_row_size(type, n);
    uint8_t *act = (uint8_t *)malloc(rs * (size_t)cols);
    if (!act) return -3;
    oracle_mul_mat_act(type, n, rows, x, cols, act);
    const int64_t nr4 = cols - cols % 4;
    const int nth = omp_threads(nthreads);

    if (type == OR_Q4_0) {
        const int64_t nb = n / 32;
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const blk_q4_0 *wr = (const blk_q4_0 *)((const uint8_t *)w + (size_t)r * nb * 18);
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_0 *a = (const blk_q8_0 *)(act + (size_t)c * rs);
                float v;
                if (route == ORACLE_ROUTE_REPACK) {
                    /* repack.rs:3351-3378 / :3380-3420: one fma per block */
                    float acc = 0.0f;
                    for (int64_t b = 0; b < nb; b++) {
                        const int32_t is = isum_q4_0(&wr[b], &a[b]);
                        if (subsums) subsums[((size_t)c * rows + r) * nb + b] = is;
                        acc = fmaf((float)is, H2F(wr[b].d) * H2F(a[b].d), acc);
                    }
                    v = acc;
                } else {
                    if (subsums)
                        for (int64_t b = 0; b < nb; b++)
                            subsums[((size_t)c * rows + r) * nb + b] = isum_q4_0(&wr[b], &a[b]);
                    v = oracle_vec_dot_q4_0_q8_0((int)n, wr, a);
                }
                out[c * rows + r] = v;
            }
        }
    } else if (type == OR_Q4_K) {
        const int64_t nb = n / QK_K;
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const blk_q4_K *wr = (const blk_q4_K *)((const uint8_t *)w + (size_t)r * nb * 144);
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_K *a = (const blk_q8_K *)(act + (size_t)c * rs);
                float v = 0.0f;
                float acc = 0.0f, accmin = 0.0f;
                for (int64_t b = 0; b < nb; b++) {
                    uint8_t s[8], m[8];
                    q4k_scales(&wr[b], s, m);
                    int32_t ia = 0, im = 0;
                    const float d_col = H2F(wr[b].d), dmin_col = H2F(wr[b].dmin), d_row = a[b].d;
                    for (int g = 0; g < 4; g++) {
                        int32_t iag, img;
                        isum_q4_K_pair(&wr[b], &a[b], g, s, m, &iag, &img);
                        ia += iag;
                        im += img;
                        if (route == ORACLE_ROUTE_REPACK && c < nr4) {
                            /* gemm: one fma per (super-block, pair), repack.rs:1742-1754 */
                            acc = fmaf((float)iag, d_col * d_row, acc);
                            accmin = fmaf((float)img, dmin_col * d_row, accmin);
                        }
                    }
                    if (subsums) {
                        subsums[(((size_t)c * rows + r) * nb + b) * 2 + 0] = ia;
                        subsums[(((size_t)c * rows + r) * nb + b) * 2 + 1] = im;
                    }
                    if (route == ORACLE_ROUTE_REPACK && c >= nr4) {
                        /* gemv: one fma per super-block, repack.rs:1681-1684 */
                        acc = fmaf((float)ia, d_col * d_row, acc);
                        accmin = fmaf((float)im, dmin_col * d_row, accmin);
                    } else if (route == ORACLE_ROUTE_TILED) {
                        /* tiled.rs:826-838: result = d0*f1; fnmadd(dmin, f2); fma(result, d1, buf) */
                        float res = d_col * (float)ia;
                        res = fmaf(-dmin_col, (float)im, res);
                        acc = fmaf(res, d_row, acc);
                    }
                }
                if (route == ORACLE_ROUTE_REPACK) v = acc - accmin;
                else if (route == ORACLE_ROUTE_TILED) v = acc;
                else v = oracle_vec_dot_q4_K_q8_K((int)n, wr, a);
                out[c * rows + r] = v;
            }
        }
    } else if (type == OR_Q2_K || type == OR_Q3_K) {
        /* the row vec_dot below 8 columns, the tiled kernel's fold from 8
         * (tiled.rs:363-411: the same integer sums, another fp32 order) */
        const int64_t nb = n / QK_K;
        const size_t wbs = type == OR_Q2_K ? sizeof(blk_q2_K) : sizeof(blk_q3_K);
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const uint8_t *wr = (const uint8_t *)w + (size_t)r * nb * wbs;
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_K *a = (const blk_q8_K *)(act + (size_t)c * rs);
                if (subsums)
                    for (int64_t b = 0; b < nb; b++) {
                        if (type == OR_Q2_K) {
                            int32_t is, sm;
                            isum_q2_K((const blk_q2_K *)wr + b, &a[b], &is, &sm);
                            subsums[(((size_t)c * rows + r) * nb + b) * 2 + 0] = is;
                            subsums[(((size_t)c * rows + r) * nb + b) * 2 + 1] = sm;
                        } else {
                            subsums[((size_t)c * rows + r) * nb + b] = isum_q3_K((const blk_q3_K *)wr + b, &a[b]);
                        }
                    }
                if (route == ORACLE_ROUTE_TILED) {
                    /* tiled.rs:822-836 epilogue per super-block (Q2_K: HAS_MIN) */
                    float acc = 0.0f;
                    for (int64_t b = 0; b < nb; b++) {
                        float res;
                        if (type == OR_Q2_K) {
                            const blk_q2_K *xb = (const blk_q2_K *)wr + b;
                            int32_t is, sm;
                            isum_q2_K(xb, &a[b], &is, &sm);
                            res = H2F(xb->d) * (float)is;
                            res = fmaf(-H2F(xb->dmin), (float)sm, res);
                        } else {
                            const blk_q3_K *xb = (const blk_q3_K *)wr + b;
                            res = H2F(xb->d) * (float)isum_q3_K(xb, &a[b]);
                        }
                        acc = fmaf(res, a[b].d, acc);
                    }
                    out[c * rows + r] = acc;
                } else {
                    out[c * rows + r] = type == OR_Q2_K ? oracle_vec_dot_q2_K_q8_K((int)n, wr, a)
                                                        : oracle_vec_dot_q3_K_q8_K((int)n, wr, a);
                }
            }
        }
    } else if (type == OR_Q4_1 || type == OR_Q5_1) {
        /* the row vec_dot at every column count: tinyBLAS does not take Q4_1 /
         * Q5_1 (tinyblas.rs:1327-1328) and no repack exists for them */
        const int64_t nb = n / 32;
        const size_t wbs = type == OR_Q4_1 ? sizeof(blk_q4_1) : sizeof(blk_q5_1);
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const uint8_t *wr = (const uint8_t *)w + (size_t)r * nb * wbs;
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_1 *a = (const blk_q8_1 *)(act + (size_t)c * rs);
                if (subsums)
                    for (int64_t b = 0; b < nb; b++)
                        subsums[((size_t)c * rows + r) * nb + b] =
                            type == OR_Q4_1 ? isum_q4_1((const blk_q4_1 *)wr + b, &a[b])
                                            : isum_q5_1((const blk_q5_1 *)wr + b, &a[b]);
                out[c * rows + r] = type == OR_Q4_1 ? oracle_vec_dot_q4_1_q8_1((int)n, wr, a)
                                                    : oracle_vec_dot_q5_1_q8_1((int)n, wr, a);
            }
        }
    } else if (type == OR_Q5_0 || type == OR_Q8_0) {
        /* the row vec_dot; tinyBLAS_Q0 (cols >= 2) keeps one accumulator per
         * output with the same lanes and fma order (tinyblas.rs:55-75) */
        const int64_t nb = n / 32;
        const size_t wbs = type == OR_Q5_0 ? sizeof(blk_q5_0) : sizeof(blk_q8_0);
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const uint8_t *wr = (const uint8_t *)w + (size_t)r * nb * wbs;
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_0 *a = (const blk_q8_0 *)(act + (size_t)c * rs);
                if (subsums)
                    for (int64_t b = 0; b < nb; b++)
                        subsums[((size_t)c * rows + r) * nb + b] =
                            type == OR_Q5_0 ? isum_q5_0((const blk_q5_0 *)wr + b, &a[b])
                                            : isum_q8_0((const blk_q8_0 *)wr + b, &a[b]);
                out[c * rows + r] = type == OR_Q5_0 ? oracle_vec_dot_q5_0_q8_0((int)n, wr, a)
                                                    : oracle_vec_dot_q8_0_q8_0((int)n, wr, a);
            }
        }
    } else if (type == OR_Q5_K) {
        const int64_t nb = n / QK_K;
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const blk_q5_K *wr = (const blk_q5_K *)((const uint8_t *)w + (size_t)r * nb * sizeof(blk_q5_K));
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_K *a = (const blk_q8_K *)(act + (size_t)c * rs);
                float acc = 0.0f;
                for (int64_t b = 0; b < nb; b++) {
                    int32_t ia, im;
                    isum_q5_K(&wr[b], &a[b], &ia, &im);
                    if (subsums) {
                        subsums[(((size_t)c * rows + r) * nb + b) * 2 + 0] = ia;
                        subsums[(((size_t)c * rows + r) * nb + b) * 2 + 1] = im;
                    }
                    if (route == ORACLE_ROUTE_TILED) {
                        /* tiled.rs:826-838 with the q5_K constants (tiled.rs:238) */
                        float res = H2F(wr[b].d) * (float)ia;
                        res = fmaf(-H2F(wr[b].dmin), (float)im, res);
                        acc = fmaf(res, a[b].d, acc);
                    }
                }
                out[c * rows + r] = route == ORACLE_ROUTE_TILED ? acc : oracle_vec_dot_q5_K_q8_K((int)n, wr, a);
            }
        }
    } else if (type == OR_IQ4_NL || type == OR_NVFP4) {
        /* the row vec_dot (IQ4_NL from 2 columns would take tinyBLAS_Q0,
         * tinyblas.rs:1334: the same integer block sums in another fp32 order);
         * sub-sums per 32-block (IQ4_NL) or 16-element sub-block (NVFP4) */
        const int64_t nbw = type == OR_IQ4_NL ? n / 32 : n / 64;
        const size_t wbs = type == OR_IQ4_NL ? sizeof(blk_iq4_nl) : sizeof(blk_nvfp4);
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const uint8_t *wr = (const uint8_t *)w + (size_t)r * nbw * wbs;
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_0 *a = (const blk_q8_0 *)(act + (size_t)c * rs);
                if (subsums) {
                    if (type == OR_IQ4_NL)
                        for (int64_t b = 0; b < nbw; b++)
                            subsums[((size_t)c * rows + r) * nbw + b] = isum_iq4_nl((const blk_iq4_nl *)wr + b, &a[b]);
                    else
                        for (int64_t b = 0; b < nbw; b++)
                            for (int sb = 0; sb < 4; sb++)
                                subsums[(((size_t)c * rows + r) * nbw + b) * 4 + sb] =
                                    isum_nvfp4_sub((const blk_nvfp4 *)wr + b, &a[2 * b], sb);
                }
                out[c * rows + r] = type == OR_IQ4_NL ? oracle_vec_dot_iq4_nl_q8_0((int)n, wr, a)
                                                      : oracle_vec_dot_nvfp4_q8_0((int)n, wr, a);
            }
        }
    } else if (type == OR_Q1_0 || type == OR_Q2_0) {
        /* the row vec_dot; sub-sums per 32-element group (one Q8_0 block) */
        const int qk = type == OR_Q1_0 ? 128 : 64, gpb = qk / 32;
        const int64_t nbw = n / qk;
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const uint8_t *wr = (const uint8_t *)w + (size_t)r * nbw * 18;
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_0 *a = (const blk_q8_0 *)(act + (size_t)c * rs);
                if (subsums)
                    for (int64_t b = 0; b < nbw; b++)
                        for (int k = 0; k < gpb; k++)
                            subsums[(((size_t)c * rows + r) * nbw + b) * gpb + k] =
                                type == OR_Q1_0 ? isum_q1_0((const blk_q1_0 *)wr + b, k, &a[b * gpb + k])
                                                : isum_q2_0((const blk_q2_0 *)wr + b, k, &a[b * gpb + k]);
                out[c * rows + r] = type == OR_Q1_0 ? oracle_vec_dot_q1_0_q8_0((int)n, wr, a)
                                                    : oracle_vec_dot_q2_0_q8_0((int)n, wr, a);
            }
        }
    } else if (oracle_iq_block_bytes(type)) {
        /* IQ1 / IQ2 / IQ3: the row dot, or from 8 columns the tiled kernel's
         * fold per super-block, res = (d * scale) * is, acc = fma(res, d8, acc)
         * (tiled.rs:454-618, :822-836); sub-sum: that integer is */
        const int64_t nb = n / QK_K;
        const int bs = oracle_iq_block_bytes(type);
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const uint8_t *wr = (const uint8_t *)w + (size_t)r * nb * bs;
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_K *a = (const blk_q8_K *)(act + (size_t)c * rs);
                float acc = 0.0f;
                for (int64_t b = 0; b < nb; b++) {
                    int32_t s8[8], s2[8], is;
                    float dw;
                    iq_super_block(type, wr + (size_t)b * bs, &a[b], s8, s2, &dw, &is);
                    if (subsums) subsums[((size_t)c * rows + r) * nb + b] = is;
                    const float td = dw * iq_scale(type);
                    acc = fmaf(td * (float)is, a[b].d, acc);
                }
                out[c * rows + r] = route == ORACLE_ROUTE_TILED ? acc : oracle_vec_dot_iq(type, (int)n, wr, a);
            }
        }
    } else if (type == OR_IQ4_XS) {
        const int64_t nb = n / QK_K;
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const blk_iq4_xs *wr = (const blk_iq4_xs *)((const uint8_t *)w + (size_t)r * nb * sizeof(blk_iq4_xs));
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_K *a = (const blk_q8_K *)(act + (size_t)c * rs);
                float acc = 0.0f;
                for (int64_t b = 0; b < nb; b++) {
                    const int32_t is = isum_iq4_xs(&wr[b], &a[b]);
                    if (subsums) subsums[((size_t)c * rows + r) * nb + b] = is;
                    /* tiled.rs:822-836 epilogue (no min term) */
                    acc = fmaf(H2F(wr[b].d) * (float)is, a[b].d, acc);
                }
                out[c * rows + r] = route == ORACLE_ROUTE_TILED ? acc : oracle_vec_dot_iq4_xs_q8_K((int)n, wr, a);
            }
        }
    } else { /* Q6_K */
        const int64_t nb = n / QK_K;
#pragma omp parallel for num_threads(nth) schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const blk_q6_K *wr = (const blk_q6_K *)((const uint8_t *)w + (size_t)r * nb * 210);
            for (int64_t c = 0; c < cols; c++) {
                const blk_q8_K *a = (const blk_q8_K *)(act + (size_t)c * rs);
                float v;
                if (route == ORACLE_ROUTE_TILED) {
                    float acc = 0.0f;
                    for (int64_t b = 0; b < nb; b++) {
                        const int32_t is = isum_q6_K(&wr[b], &a[b]);
                        if (subsums) subsums[((size_t)c * rows + r) * nb + b] = is;
                        const float res = H2F(wr[b].d) * (float)is;
                        acc = fmaf(res, a[b].d, acc);
                    }
                    v = acc;
                } else {
                    if (subsums)
                        for (int64_t b = 0; b < nb; b++)
                            subsums[((size_t)c * rows + r) * nb + b] = isum_q6_K(&wr[b], &a[b]);
                    v = oracle_vec_dot_q6_K_q8_K((int)n, wr, a);
                }
                out[c * rows + r] = v;
            }
        }
    }
    free(act);
    return route;
}

/* ---------------------------------------------------- MUL_MAT_ID (MXFP4) */

int oracle_mul_mat_id_mxfp4(const void *as, int64_t n, int64_t rows, int64_t n_as,
                            const float *b, int64_t ne11, int64_t n_tokens,
                            const int32_t *ids, int64_t n_ids, float *dst, int nthreads) {
    const int64_t nb = n / 32;
    const size_t rs = (size_t)nb * sizeof(blk_q8_0);
    const size_t wrow = (size_t)nb * sizeof(blk_mxfp4);
    uint8_t *act = (uint8_t *)malloc(rs * (size_t)(ne11 * n_tokens));
    if (!act) return -3;
    for (int64_t i = 0; i < ne11 * n_tokens; i++) oracle_quantize_row_q8_0(b + i * n, act + i * rs, n);
    for (int64_t i = 0; i < n_ids * n_tokens; i++)
        if (ids[i] < 0 || ids[i] >= n_as) { free(act); return -4; }
    const int repack = rows % 8 == 0;
    const int nth = omp_threads(nthreads);
#pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t ir = 0; ir < n_ids * n_tokens; ir++) {
        const int64_t i1 = ir % n_ids, i2 = ir / n_ids;
        const int64_t id = ids[i2 * n_ids + i1];
        const int64_t i11 = i1 % ne11;
        const blk_q8_0 *y = (const blk_q8_0 *)(act + (size_t)(i11 + i2 * ne11) * rs);
        for (int64_t r = 0; r < rows; r++) {
            const blk_mxfp4 *x = (const blk_mxfp4 *)((const uint8_t *)as + ((size_t)id * rows + r) * wrow);
            float acc = 0.0f;
            for (int64_t ib = 0; ib < nb; ib++) {
                const int32_t dot = isum_mxfp4(&x[ib], &y[ib]);
                if (repack) {
                    /* repack.rs:1071-1073 */
                    const float scale = oracle_e8m0_to_fp32_half(x[ib].e) * H2F(y[ib].d);
                    acc = fmaf((float)dot, scale, acc);
                } else {
                    /* compute.rs:7140-7150 (non-fused) */
                    const float d = H2F(y[ib].d) * oracle_e8m0_to_fp32_half(x[ib].e);
                    acc += d * (float)dot;
                }
            }
            dst[(i2 * n_ids + i1) * rows + r] = acc;
        }
    }
    free(act);
    return 0;
}

/* FLASH_ATTN_EXT lives in ggml_oracle_fa.c */

/* half 2.7.1 bf16::from_f32 (RNE on the top 16 bits; NaN stays a quiet NaN) */
uint16_t oracle_fp32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    const uint32_t round = 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)((u + round) >> 16);
}
float oracle_bf16_to_fp32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* compute.rs:1700-1745 (F16 / BF16 weights: the activation row converted to
 * the weight type, then the row dot) and :1680-1698 (F32 weights); the dots are
 * ggml_vec_dot_f16 / _bf16 / _f32's scalar forms (vec_dot.rs:1700-1727): each
 * product in f32 (exact for f16 and bf16 operands), summed in double */
int oracle_mul_mat_dense(int type, const void *w, int64_t n, int64_t rows, const float *x, int64_t cols, float *out,
                         int nthreads) {
    if (type != OR_F32 && type != OR_F16 && type != OR_BF16) return -1;
    float *xc = (float *)malloc(sizeof(float) * (size_t)(n * cols));
    if (!xc) return -3;
    for (int64_t i = 0; i < n * cols; i++)
        xc[i] = type == OR_F16 ? H2F(F2H(x[i])) : type == OR_BF16 ? oracle_bf16_to_fp32(oracle_fp32_to_bf16(x[i])) : x[i];
    const int nth = omp_threads(nthreads);
#pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t c = 0; c < cols; c++) {
            const float *y = xc + c * n;
            double s = 0.0;
            for (int64_t i = 0; i < n; i++) {
                float wv;
                if (type == OR_F32) wv = ((const float *)w)[r * n + i];
                else if (type == OR_F16) wv = H2F(((const uint16_t *)w)[r * n + i]);
                else wv = oracle_bf16_to_fp32(((const uint16_t *)w)[r * n + i]);
                s += (double)(wv * y[i]);
            }
            out[c * rows + r] = (float)s;
        }
    }
    free(xc);
    return 0;
}
