/*
 * ggml_oracle_fa.c -- TEST INFRASTRUCTURE ONLY: restatement of llama.rust's
 * GGML_OP_FLASH_ATTN_EXT CPU kernels (crates/ggml/src/flash_attn.rs), used as
 * the checker of the HIP kernels and as the timed CPU baseline.
 *
 * Dispatch (flash_attn.rs:907-935): split-KV for a single query row with
 * S_kv >= 512 and n_chunks chunks (the reference's thread count), else the
 * 64x64 tiled kernel for >= 64 query rows, else one_chunk.  Each path keeps
 * the reference's float evaluation order (fused multiply-adds exactly where
 * the reference fuses; -ffp-contract=off elsewhere).
 */
#include "ggml_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define Q_TILE 64
#define KV_TILE 64

static inline float h2f(uint16_t h) { return oracle_fp16_to_fp32(h); }
static inline uint16_t f2h(float f) { return oracle_fp32_to_fp16(f); }

/* vec_dot.rs:1893 reduce_add16 */
static float reduce_add16(const float x[16]) {
    float t[16];
    memcpy(t, x, sizeof t);
    for (int half = 8; half >= 1; half >>= 1)
        for (int i = 0; i < half; i++) t[i] += t[i + half];
    return t[0];
}

/* vec_dot.rs:1982 vec_dot_f16_c (x: K row f16, y: Q row f16) */
static float vec_dot_f16(int n, const uint16_t *x, const uint16_t *y) {
    const int np = n & ~63;
    float sum[4][16];
    memset(sum, 0, sizeof sum);
    int i = 0;
    for (; i < np; i += 64)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 16; l++) {
                const int k = i + j * 16 + l;
                sum[j][l] = fmaf(h2f(y[k]), h2f(x[k]), sum[j][l]);
            }
    float a[16], b[16];
    for (int l = 0; l < 16; l++) a[l] = sum[0][l] + sum[2][l];
    for (int l = 0; l < 16; l++) b[l] = sum[1][l] + sum[3][l];
    for (int l = 0; l < 16; l++) a[l] += b[l];
    double res = reduce_add16(a);
    for (; i < n; i++) res += (double)(h2f(x[i]) * h2f(y[i]));
    return (float)res;
}

/* vec_dot.rs:1921 vec_dot_f32_c */
static float vec_dot_f32(int n, const float *x, const float *y) {
    const int np = n & ~63;
    float sum[4][16];
    memset(sum, 0, sizeof sum);
    int i = 0;
    for (; i < np; i += 64)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 16; l++) {
                const int k = i + j * 16 + l;
                sum[j][l] = fmaf(y[k], x[k], sum[j][l]);
            }
    float a[16], b[16];
    for (int l = 0; l < 16; l++) a[l] = sum[0][l] + sum[2][l];
    for (int l = 0; l < 16; l++) b[l] = sum[1][l] + sum[3][l];
    for (int l = 0; l < 16; l++) a[l] += b[l];
    float res = reduce_add16(a);
    int left = n - i;
    while (left >= 16) { for (int j = 0; j < 16; j++) { const float p = x[i + j] * y[i + j]; res += p; } i += 16; left -= 16; }
    if (left >= 8) { for (int j = 0; j < 8; j++) { const float p = x[i + j] * y[i + j]; res += p; } i += 8; left -= 8; }
    while (left > 0) { res = fmaf(x[i], y[i], res); i++; left--; }
    return res;
}

/* compiler-rt __powisf2 (what Rust's f32::powi lowers to for a runtime exponent) */
static float powi_f(float a, int b) {
    const int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* flash_attn.rs:395-409 */
static float alibi_slope(const oracle_fa_args *a, int h) {
    if (a->max_bias <= 0.0f) return 1.0f;
    const unsigned nl2 = 1u << (unsigned)floor(log2((double)a->H));
    const float m0 = powf(2.0f, -a->max_bias / (float)nl2);
    const float m1 = powf(2.0f, -(a->max_bias / 2.0f) / (float)nl2);
    return (unsigned)h < nl2 ? powi_f(m0, h + 1) : powi_f(m1, 2 * (h - (int)nl2) + 1);
}

static float kq_scale(const oracle_fa_args *a) {
    return a->softcap != 0.0f ? a->scale / a->softcap : a->scale;
}

static const float *q_row(const oracle_fa_args *a, int t, int h) { return a->q + (int64_t)h * a->q_nb2 + (int64_t)t * a->q_nb1; }
static int kv_head(const oracle_fa_args *a, int h) { return h / (a->H / a->H_kv); }
static float k_elem(const oracle_fa_args *a, int hk, int s, int d) {
    const int64_t o = (int64_t)hk * a->k_nb2 + (int64_t)s * a->k_nb1 + d;
    return a->kv_f16 ? h2f(((const uint16_t *)a->k)[o]) : ((const float *)a->k)[o];
}
static float v_elem(const oracle_fa_args *a, int hv, int s, int d) {
    const int64_t o = (int64_t)hv * a->v_nb2 + (int64_t)s * a->v_nb1 + d;
    return a->kv_f16 ? h2f(((const uint16_t *)a->v)[o]) : ((const float *)a->v)[o];
}
static float mask_at(const oracle_fa_args *a, int t, int s) {
    return h2f(a->mask[(int64_t)t * a->mask_nb1 + s]);
}
static float *dst_row(const oracle_fa_args *a, int t, int h) { return a->dst + ((int64_t)t * a->H + h) * a->DV; }

/* flash_attn.rs:482-703 attn_row: one query row over [ic0, ic1); writes the
 * unnormalized accumulator into vkq (DV) and returns M, S. */
static void attn_row(const oracle_fa_args *a, int t, int h, int ic0, int ic1, float *vkq, float *M_out, float *S_out) {
    const int DK = a->DK, DV = a->DV;
    const float slope = alibi_slope(a, h);
    const float scale = kq_scale(a);
    const int hk = kv_head(a, h);
    float S = 0.0f, M = -INFINITY;
    for (int d = 0; d < DV; d++) vkq[d] = 0.0f;
    uint16_t *vkq16 = (uint16_t *)calloc((size_t)DV, 2);
    uint16_t *q16 = (uint16_t *)malloc((size_t)DK * 2);
    const float *qr = q_row(a, t, h);
    for (int d = 0; d < DK; d++) q16[d] = f2h(qr[d]);
    for (int ic = ic0; ic < ic1; ic++) {
        const float mv = a->mask ? slope * mask_at(a, t, ic) : 0.0f;
        if (mv == -INFINITY) continue;
        float s;
        if (a->kv_f16) s = vec_dot_f16(DK, (const uint16_t *)a->k + (int64_t)hk * a->k_nb2 + (int64_t)ic * a->k_nb1, q16);
        else s = vec_dot_f32(DK, (const float *)a->k + (int64_t)hk * a->k_nb2 + (int64_t)ic * a->k_nb1, qr);
        s = s * scale;
        if (a->softcap != 0.0f) s = a->softcap * tanhf(s);
        s += mv;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        if (a->kv_f16) {
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                for (int d = 0; d < DV; d++) vkq16[d] = f2h(h2f(vkq16[d]) * ms);
            } else {
                vs = expf(s - M);
            }
            for (int d = 0; d < DV; d++) vkq16[d] = f2h(fmaf(v_elem(a, hk, ic, d), vs, h2f(vkq16[d])));
        } else {
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                for (int d = 0; d < DV; d++) vkq[d] *= ms;
            } else {
                vs = expf(s - M);
            }
            for (int d = 0; d < DV; d++) vkq[d] = fmaf(v_elem(a, hk, ic, d), vs, vkq[d]);
        }
        S = fmaf(S, ms, vs);
    }
    if (a->kv_f16)
        for (int d = 0; d < DV; d++) vkq[d] = h2f(vkq16[d]);
    if (a->sinks && ic0 == 0) {
        const float sh = a->sinks[h];
        float ms = 1.0f, vs = 1.0f;
        if (sh > M) {
            ms = expf(M - sh);
            M = sh;
            for (int d = 0; d < DV; d++) vkq[d] *= ms;
        } else {
            vs = expf(sh - M);
        }
        S = S * ms + vs; /* unfused in the reference (flash_attn.rs:684-697) */
    }
    free(vkq16);
    free(q16);
    *M_out = M;
    *S_out = S;
}

static void one_chunk(const oracle_fa_args *a, int t0, int t1) {
    float *vkq = (float *)malloc((size_t)a->DV * 4);
    for (int h = 0; h < a->H; h++)
        for (int t = t0; t < t1; t++) {
            float M, S;
            attn_row(a, t, h, 0, a->S, vkq, &M, &S);
            const float sinv = S == 0.0f ? 0.0f : 1.0f / S;
            float *o = dst_row(a, t, h);
            for (int d = 0; d < a->DV; d++) o[d] = vkq[d] * sinv;
        }
    free(vkq);
}

/* flash_attn.rs:779-862 split_kv + reduce_partials (one query row) */
static void split_kv(const oracle_fa_args *a, int n_chunks) {
    const int DV = a->DV;
    const int chunk = (a->S + n_chunks - 1) / n_chunks;
    float *part = (float *)malloc((size_t)n_chunks * (2 + DV) * 4);
    float *fin = (float *)malloc((size_t)DV * 4);
    for (int h = 0; h < a->H; h++) {
        for (int c = 0; c < n_chunks; c++) {
            float *p = part + (size_t)c * (2 + DV);
            const int ic0 = c * chunk;
            if (ic0 >= a->S) { p[0] = -INFINITY; p[1] = 0.0f; continue; }
            const int ic1 = ic0 + chunk < a->S ? ic0 + chunk : a->S;
            attn_row(a, 0, h, ic0, ic1, p + 2, &p[0], &p[1]);
        }
        float Mf = -INFINITY, Sf = 0.0f;
        for (int d = 0; d < DV; d++) fin[d] = 0.0f;
        for (int c = 0; c < n_chunks; c++) {
            if ((int64_t)c * chunk >= a->S) continue;
            const float *p = part + (size_t)c * (2 + DV);
            if (p[1] == 0.0f) continue;
            const float Mn = fmaxf(Mf, p[0]);
            const float so = expf(Mf - Mn), sn = expf(p[0] - Mn);
            for (int d = 0; d < DV; d++) fin[d] = fmaf(fin[d], so, p[2 + d] * sn);
            Sf = fmaf(Sf, so, p[1] * sn);
            Mf = Mn;
        }
        if (Sf != 0.0f) {
            const float sinv = 1.0f / Sf;
            for (int d = 0; d < DV; d++) fin[d] *= sinv;
        }
        memcpy(dst_row(a, 0, h), fin, (size_t)DV * 4);
    }
    free(part);
    free(fin);
}

/* flash_attn.rs:948-977 v_expf (ggml's AVX512 expf polynomial, elementwise) */
static float v_expf(float x) {
    const float R = 12582912.0f;                 /* 0x1.8p23 */
    const float LOG2E = 1.44269502162933349609f; /* 0x1.715476p+0 */
    union { uint32_t u; float f; } c1 = {0x35bfbe8eu}, c2 = {0x3f317200u}, p1 = {0x3c072010u},
        p2 = {0x3d2b9f17u}, p3 = {0x3e2aaf33u}, p4 = {0x3efffedbu}, p5 = {0x3f7ffff6u}, lg = {0x3fb8aa3bu};
    (void)LOG2E;
    const float z = fmaf(x, lg.f, R);
    const float n = z - R;
    const float b = fmaf(n, -c1.f, fmaf(n, -c2.f, x));
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(b, p1.f, p2.f), u, fmaf(b, p3.f, p4.f)), u, fmaf(b, p5.f, 1.0f));
    if (fabsf(n) > 192.0f) return n <= 0.0f ? 0.0f : INFINITY;
    return (float)((double)j * ldexp(1.0, (int)n));
}

/* flash_attn.rs:996-1005 _mm512_reduce_add_ps fold */
static float reduce_add_ps(const float v[16]) {
    float t3[8], t6[4];
    for (int j = 0; j < 8; j++) t3[j] = v[8 + j] + v[j];
    for (int j = 0; j < 4; j++) t6[j] = t3[4 + j] + t3[j];
    return (t6[0] + t6[2]) + (t6[1] + t6[3]);
}

/* flash_attn.rs:1020-1043 vec_soft_max_f32, in place; returns the f64 sum */
static double soft_max_inplace(float *y, int n, float max) {
    int i = 0;
    double sum = 0.0;
    for (; i + 15 < n; i += 16) {
        float v[16];
        for (int j = 0; j < 16; j++) v[j] = v_expf(y[i + j] - max);
        memcpy(y + i, v, sizeof v);
        sum += (double)reduce_add_ps(v);
    }
    for (; i < n; i++) {
        const float val = expf(y[i] - max);
        sum += (double)val;
        y[i] = val;
    }
    return sum;
}

/* simd_gemm (flash_attn.rs:1065-1076): C[m x n] += A[m x k] B[k x n], one fma chain per element */
static void simd_gemm(float *c, const float *a, const float *b, int m, int k, int n) {
    for (int i = 0; i < m; i++)
        for (int kk = 0; kk < k; kk++) {
            const float av = a[i * k + kk];
            const float *brow = b + kk * n;
            float *crow = c + i * n;
            for (int x = 0; x < n; x++) crow[x] = fmaf(av, brow[x], crow[x]);
        }
}

/* flash_attn.rs:1111-1366 tiled_impl over query rows [t0, t1) of every head */
static void tiled(const oracle_fa_args *a, int t0, int t1) {
    const int DK = a->DK, DV = a->DV;
    const float scale = kq_scale(a);
    float *qf = (float *)malloc((size_t)Q_TILE * DK * 4);
    float *kq = (float *)malloc((size_t)Q_TILE * KV_TILE * 4);
    float *m32 = (float *)malloc((size_t)Q_TILE * KV_TILE * 4);
    float *vkq = (float *)malloc((size_t)Q_TILE * DV * 4);
    float *v32 = (float *)malloc((size_t)KV_TILE * DV * 4);
    float *kf = (float *)malloc((size_t)KV_TILE * DK * 4);
    for (int h = 0; h < a->H; h++) {
        const int hk = kv_head(a, h);
        const float slope = alibi_slope(a, h);
        for (int tq0 = t0; tq0 < t1; tq0 += Q_TILE) {
            const int rows = (t1 - tq0) < Q_TILE ? (t1 - tq0) : Q_TILE;
            float S[Q_TILE], M[Q_TILE];
            for (int i = 0; i < Q_TILE; i++) { S[i] = 0.0f; M[i] = -INFINITY; }
            memset(vkq, 0, (size_t)Q_TILE * DV * 4);
            memset(m32, 0, (size_t)Q_TILE * KV_TILE * 4);
            for (int tq = 0; tq < Q_TILE; tq++)
                for (int d = 0; d < DK; d++) qf[tq * DK + d] = tq < rows ? q_row(a, tq0 + tq, h)[d] : 0.0f;
            memset(kf, 0, (size_t)KV_TILE * DK * 4);
            memset(v32, 0, (size_t)KV_TILE * DV * 4);
            for (int ic = 0; ic < a->S; ic += KV_TILE) {
                const int kvt = (a->S - ic) < KV_TILE ? (a->S - ic) : KV_TILE;
                if (a->mask) {
                    int can_skip = 1;
                    for (int tq = 0; tq < rows; tq++) {
                        for (int tk = 0; tk < kvt; tk++) {
                            const float mv = slope * mask_at(a, tq0 + tq, ic + tk);
                            m32[tq * KV_TILE + tk] = mv;
                            if (mv != -INFINITY) can_skip = 0;
                        }
                        for (int tk = kvt; tk < KV_TILE; tk++) m32[tq * KV_TILE + tk] = -INFINITY;
                    }
                    if (can_skip) continue;
                }
                for (int tk = 0; tk < kvt; tk++)
                    for (int d = 0; d < DK; d++) kf[d * KV_TILE + tk] = k_elem(a, hk, ic + tk, d);
                memset(kq, 0, (size_t)Q_TILE * KV_TILE * 4);
                simd_gemm(kq, qf, kf, Q_TILE, DK, KV_TILE);
                for (int i = 0; i < Q_TILE * KV_TILE; i++) kq[i] *= scale;
                if (a->softcap != 0.0f)
                    for (int i = 0; i < Q_TILE * KV_TILE; i++) kq[i] = a->softcap * tanhf(kq[i]);
                if (kvt < KV_TILE)
                    for (int tq = 0; tq < Q_TILE; tq++)
                        for (int tk = kvt; tk < KV_TILE; tk++) kq[tq * KV_TILE + tk] = -INFINITY;
                if (a->mask)
                    for (int i = 0; i < rows * KV_TILE; i++) kq[i] += m32[i];
                int skip[Q_TILE];
                for (int tq = 0; tq < Q_TILE; tq++) {
                    float *row = kq + tq * KV_TILE;
                    float tmax = -INFINITY;
                    for (int x = 0; x < KV_TILE; x++) tmax = tmax > row[x] ? tmax : row[x];
                    skip[tq] = tmax == -INFINITY;
                    if (skip[tq]) continue;
                    const float mold = M[tq];
                    const float mnew = mold > tmax ? mold : tmax;
                    if (mnew > mold) {
                        const float ms = expf(mold - mnew);
                        for (int d = 0; d < DV; d++) vkq[tq * DV + d] *= ms;
                        S[tq] *= ms;
                    }
                    M[tq] = mnew;
                    const double sum = soft_max_inplace(row, KV_TILE, mnew);
                    S[tq] = (float)((double)S[tq] + sum);
                }
                for (int tk = 0; tk < kvt; tk++)
                    for (int d = 0; d < DV; d++) v32[tk * DV + d] = v_elem(a, hk, ic + tk, d);
                for (int tq = 0; tq < Q_TILE; tq++)
                    if (skip[tq]) memset(kq + tq * KV_TILE, 0, KV_TILE * 4);
                simd_gemm(vkq, kq, v32, Q_TILE, KV_TILE, DV);
            }
            if (a->sinks) {
                const float sv = a->sinks[h];
                for (int tq = 0; tq < rows; tq++) {
                    float ms = 1.0f, vs = 1.0f;
                    if (sv > M[tq]) {
                        ms = expf(M[tq] - sv);
                        for (int d = 0; d < DV; d++) vkq[tq * DV + d] *= ms;
                    } else {
                        vs = expf(sv - M[tq]);
                    }
                    S[tq] = fmaf(S[tq], ms, vs);
                }
            }
            for (int tq = 0; tq < rows; tq++) {
                const float sinv = S[tq] == 0.0f ? 0.0f : 1.0f / S[tq];
                float *o = dst_row(a, tq0 + tq, h);
                for (int d = 0; d < DV; d++) o[d] = vkq[tq * DV + d] * sinv;
            }
        }
    }
    free(qf); free(kq); free(m32); free(vkq); free(v32); free(kf);
}

int oracle_flash_attn_ext(const oracle_fa_args *a) {
    if (a->H % a->H_kv) return -1;
    if (a->T == 1 && a->S >= 512) {
        split_kv(a, a->n_chunks > 0 ? a->n_chunks : 1);
        return 1;
    }
    if (a->T >= Q_TILE) {
        /* rows are independent: split the query range over threads, tiles of 64
         * start at multiples of 64 exactly as the single-threaded reference */
        const int ntiles = (a->T + Q_TILE - 1) / Q_TILE;
#pragma omp parallel for schedule(dynamic) num_threads(a->nthreads > 0 ? a->nthreads : 1)
        for (int i = 0; i < ntiles; i++) {
            const int t0 = i * Q_TILE, t1 = t0 + Q_TILE < a->T ? t0 + Q_TILE : a->T;
            tiled(a, t0, t1);
        }
        return 2;
    }
    one_chunk(a, 0, a->T);
    return 3;
}
