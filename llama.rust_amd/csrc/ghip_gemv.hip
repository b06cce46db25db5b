// ghip_gemv.hip -- decode MUL_MAT (batch 1..8 activation rows) for Q4_K, Q6_K
// and Q4_0 weights, dequantizing in registers from 16-byte HBM loads.
//
// Work layout (all three kernels):
//  * A workgroup is one "K-team": W_K wavefronts whose 64*W_K lanes tile the
//    reduction dimension once (8 lanes per 256-block for the K-quants, one
//    lane per pair of 32-blocks for Q4_0).  A lane's K position never changes,
//    so its activation codes are loaded once into registers.
//  * The team owns RB = 8 consecutive weight rows.  Every lane issues the loads
//    of all 8 rows before it consumes any (8 x 16 B per stream in flight per
//    lane), which is what keeps enough HBM traffic in flight on a ~5 us
//    kernel.  A wavefront's loads of one row are contiguous, so they coalesce.
//  * Per row and activation column a lane forms an exact int32 partial
//    (v_dot4_i32_i8 on unpacked nibbles) and scales it in fp32; the 8 rows are
//    reduced across the wavefront together (reduce8_rows), and the W_K
//    wavefront partials meet in LDS.
//
// The exact integer sums of the reference (per row, column and block) are
// available through the SUBSUMS instantiations, which reduce the 8 lanes of
// a block in int32 and store them:
//   Q4_K: {iacc, imin} per super-block  (repack.rs:1664-1680)
//   Q6_K: sum_s scale_s * sum (q6-32) q8 per super-block (vec_dot.rs:1000-1036)
//   Q4_0: sum (nib-8) q8 per 32-block   (repack.rs:3351-3378)
#include "ghip_common.h"

constexpr int RB = 8;  // weight rows per workgroup

// write the 8 row totals of column c (lanes with lane%8 == 0 hold them)
DEV void stash_rows(float *red, float part[RB], int lane, int w, int nw, int c, int NC) {
    const float t = reduce8_rows(part, lane);
    if ((lane & 7) == 0) red[((lane >> 3) * nw + w) * NC + c] = t;
}

DEV void finish_rows(const float *red, int r0, int nrows, int ncols, int NC, int nw, float *dst, int64_t ldd) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < nrows * ncols; idx += blockDim.x) {
        const int rr = idx / ncols, c = idx - rr * ncols;
        float s = 0.0f;
        for (int ww = 0; ww < nw; ww++) s += red[(rr * nw + ww) * NC + c];
        dst[(int64_t)c * ldd + r0 + rr] = s;
    }
}

// ---------------------------------------------------------------- Q4_K x Q8_K
// Activation codes of one lane: the 32 elements 64g+16h+[0,16) (low stream)
// and 64g+32+16h+[0,16) (high stream) of super-block b, the pair sum of
// subblock j for the min term, and the block scale.
struct Q4KAct {
    uint4 lo, hi;
    int bp;
    float d;
};

// Quantize this lane's share of activation row xr (f32) to Q8_K inside the
// kernel, bit-identical to ghip_quantize_q8_K: the 8 lanes of a super-block
// reduce its signed max-abs (first occurrence wins), then each lane codes its
// 32 elements.  mat selects the quantize_mat_q8_K_4x8 values.
struct XLane {
    float l[16], h[16];
};

DEV XLane load_x_lane(const float *__restrict__ xr, int b, int g, int h, bool valid) {
    XLane x;
    if (valid) {
        __builtin_memcpy(x.l, xr + (int64_t)b * QK_K + 64 * g + 16 * h, 64);
        __builtin_memcpy(x.h, xr + (int64_t)b * QK_K + 64 * g + 32 + 16 * h, 64);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) x.l[i] = x.h[i] = 0.0f;
    }
    return x;
}

DEV Q4KAct quant_q8K_lane(const XLane &x, int g, int h, int j, bool mat) {
    const float *xl = x.l, *xh = x.h;
    // element index inside the block, for the first-occurrence tie break
    const int base_l = 64 * g + 16 * h, base_h = base_l + 32;
    float bax = 0.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float a = fabsf(xl[i]);
        if (a > bax) { bax = a; bval = xl[i]; bidx = base_l + i; }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float a = fabsf(xh[i]);
        if (a > bax || (a == bax && a > 0.0f && base_h + i < bidx)) { bax = a; bval = xh[i]; bidx = base_h + i; }
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        const float oax = __shfl_xor(bax, o, 64);
        const float oval = __shfl_xor(bval, o, 64);
        const int oidx = __shfl_xor(bidx, o, 64);
        if (oax > bax || (oax == bax && oidx < bidx)) { bax = oax; bval = oval; bidx = oidx; }
    }
    Q4KAct r;
    int ql[16], qh[16];
    if (bax == 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; i++) ql[i] = qh[i] = 0;
        r.d = 0.0f;
    } else if (!mat) {
        const float iscale = __fdiv_rn(-127.0f, bval);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            ql[i] = min(127, (int)rintf(__fmul_rn(iscale, xl[i])));
            qh[i] = min(127, (int)rintf(__fmul_rn(iscale, xh[i])));
        }
        r.d = __fdiv_rn(1.0f, iscale);
    } else {
        const float iscale = __fdiv_rn(127.0f, bax);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            ql[i] = (int)fminf(fmaxf(rintf(__fmul_rn(iscale, xl[i])), -128.0f), 127.0f);
            qh[i] = (int)fminf(fmaxf(rintf(__fmul_rn(iscale, xh[i])), -128.0f), 127.0f);
        }
        r.d = __fdiv_rn(1.0f, iscale);
    }
    uint32_t pl[4], ph[4];
    int sl = 0, sh = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        pl[k] = (uint32_t)(ql[4 * k] & 0xff) | ((uint32_t)(ql[4 * k + 1] & 0xff) << 8) |
                ((uint32_t)(ql[4 * k + 2] & 0xff) << 16) | ((uint32_t)(ql[4 * k + 3] & 0xff) << 24);
        ph[k] = (uint32_t)(qh[4 * k] & 0xff) | ((uint32_t)(qh[4 * k + 1] & 0xff) << 8) |
                ((uint32_t)(qh[4 * k + 2] & 0xff) << 16) | ((uint32_t)(qh[4 * k + 3] & 0xff) << 24);
        sl += ql[4 * k] + ql[4 * k + 1] + ql[4 * k + 2] + ql[4 * k + 3];
        sh += qh[4 * k] + qh[4 * k + 1] + qh[4 * k + 2] + qh[4 * k + 3];
    }
    r.lo = make_uint4(pl[0], pl[1], pl[2], pl[3]);
    r.hi = make_uint4(ph[0], ph[1], ph[2], ph[3]);
    // subblock j = 2g' collects the low streams of lanes 2g', 2g'+1; 2g'+1 their high streams
    const int ol = __shfl_xor(sl, 1, 64), oh = __shfl_xor(sh, 1, 64);
    r.bp = (j & 1) ? (sh + oh) : (sl + ol);
    return r;
}

DEV Q4KAct load_q8K_lane(const uint8_t *__restrict__ A, int g, int h, int j) {
    Q4KAct r;
    r.lo = ld16(A + 4 + 64 * g + 16 * h);
    r.hi = ld16(A + 4 + 64 * g + 32 + 16 * h);
    const uint32_t bs = ld4(A + 260 + 4 * j);
    r.bp = (int)(int16_t)(bs & 0xffff) + (int)(int16_t)(bs >> 16);
    r.d = __uint_as_float(ld4(A));
    return r;
}

// One launch per MUL_MAT: FUSEQ kernels read the f32 activations and quantize
// them in registers; the others read ready Q8_K rows.  Each workgroup walks
// rows_per_wg rows in groups of RB, loading group i+1 while computing group i.
template <int NC, bool SUBSUMS, bool FUSEQ>
__device__ __forceinline__ void gemv_q4K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                              int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                              int ncols, float *__restrict__ dst, int64_t ldd,
                                              int32_t *__restrict__ sub, int rows_per_wg, int n_mat) {
    extern __shared__ float red[];  // [rows_per_wg][W_K][NC]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int b = 8 * w + (lane >> 3), j = lane & 7, g = j >> 1, h = j & 1;
    const bool valid = b < nb;
    const int r0 = blockIdx.x * rows_per_wg;
    const int r1 = min(rows, r0 + rows_per_wg);
    const uint8_t *wb = W + (int64_t)b * Q4K_BYTES;

    // Branch-free weight loads: rows past the tile and lanes past the row
    // re-read a valid block (clamped index) and contribute zero (their
    // activation codes and scale are zero).
    const uint8_t *wbc = W + (int64_t)min(b, nb - 1) * Q4K_BYTES;
    uint4 hdr[RB], q[RB];
    auto load_group = [&](int rg, uint4 *hd, uint4 *qq) {
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const uint8_t *p = wbc + (int64_t)min(rg + rr, r1 - 1) * w_row_bytes;
            hd[rr] = ld16(p);
            qq[rr] = ld16(p + 16 + 16 * j);
        }
    };
    // Order of issue: the f32 activations of up to two columns, then the first
    // weight group, then the activation quantization -- which waits on the
    // activation loads only, with the weight loads still in flight.
    constexpr int NX = FUSEQ ? (NC < 2 ? NC : 2) : 0;
    XLane xs[NX > 0 ? NX : 1];
#pragma unroll
    for (int c = 0; c < NX; c++)
        xs[c] = load_x_lane(reinterpret_cast<const float *>(act + c * act_row_bytes), b, g, h,
                            valid && c < ncols);
    load_group(r0, hdr, q);
    Q4KAct a[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if (c < ncols) {
            if (FUSEQ) {
                const XLane xv = c < NX ? xs[c]
                                        : load_x_lane(reinterpret_cast<const float *>(act + c * act_row_bytes), b,
                                                      g, h, valid);
                a[c] = quant_q8K_lane(xv, g, h, j, c < n_mat);
            } else if (valid) {
                a[c] = load_q8K_lane(act + c * act_row_bytes + (int64_t)b * Q8K_BYTES, g, h, j);
            } else {
                a[c] = Q4KAct{make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), 0, 0.0f};
            }
        } else {
            a[c] = Q4KAct{make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), 0, 0.0f};
        }
    }

    auto compute_group = [&](int rg, const uint4 *hdr_, const uint4 *q_) {
        float part[NC][RB];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const uint4 hd = hdr_[rr], qq = q_[rr];
            const float dw = h2f(hd.x), dmin = h2f(hd.x >> 16);
            int slo, shi, mj, mdummy, sdummy;
            scale_min_k4(hd.y, hd.z, hd.w, 2 * g, slo, mdummy);
            scale_min_k4(hd.y, hd.z, hd.w, 2 * g + 1, shi, mdummy);
            scale_min_k4(hd.y, hd.z, hd.w, j, sdummy, mj);
            const uint32_t l0 = qq.x & 0x0f0f0f0f, l1 = qq.y & 0x0f0f0f0f, l2 = qq.z & 0x0f0f0f0f, l3 = qq.w & 0x0f0f0f0f;
            const uint32_t h0 = (qq.x >> 4) & 0x0f0f0f0f, h1 = (qq.y >> 4) & 0x0f0f0f0f;
            const uint32_t h2 = (qq.z >> 4) & 0x0f0f0f0f, h3 = (qq.w >> 4) & 0x0f0f0f0f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int dl = dot4(l3, a[c].lo.w, dot4(l2, a[c].lo.z, dot4(l1, a[c].lo.y, dot4(l0, a[c].lo.x, 0))));
                const int dh = dot4(h3, a[c].hi.w, dot4(h2, a[c].hi.z, dot4(h1, a[c].hi.y, dot4(h0, a[c].hi.x, 0))));
                const int ia = slo * dl + shi * dh;
                const int im = mj * a[c].bp;
                if (SUBSUMS) {
                    const int iab = group8_sum(ia), imb = group8_sum(im);
                    if (j == 0 && valid && c < ncols && rg + rr < r1) {
                        int32_t *s = sub + (((int64_t)c * rows + rg + rr) * nb + b) * 2;
                        s[0] = iab;
                        s[1] = imb;
                    }
                }
                part[c][rr] = a[c].d * fmaf(dw, (float)ia, -(dmin * (float)im));
            }
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float t = reduce8_rows(part[c], lane);
            if ((lane & 7) == 0 && rg + (lane >> 3) < r1) red[((rg - r0 + (lane >> 3)) * nw + w) * NC + c] = t;
        }
    };
    // Ping-pong over two register buffers (no copies, so the next group's
    // loads stay in flight while this group is computed).
    uint4 hdr2[RB], q2[RB];
    for (int rg = r0; rg < r1; rg += 2 * RB) {
        if (rg + RB < r1) load_group(rg + RB, hdr2, q2);
        compute_group(rg, hdr, q);
        if (rg + RB >= r1) break;
        if (rg + 2 * RB < r1) load_group(rg + 2 * RB, hdr, q);
        compute_group(rg + RB, hdr2, q2);
    }
    finish_rows(red, r0, r1 - r0, ncols, NC, nw, dst, ldd);
}

// ---------------------------------------------------------------- Q6_K x Q8_K
template <int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q6K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                              int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                              int ncols, float *__restrict__ dst, int64_t ldd,
                                              int32_t *__restrict__ sub) {
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int b = 8 * w + (lane >> 3), j = lane & 7;
    const int jj = j >> 2, p = (j >> 1) & 1, t = j & 1;
    const bool valid = b < nb;
    const int ea = 128 * jj + 32 * p + 16 * t;  // first element of the low-nibble stream
    const int si = 8 * jj + 2 * p + t;          // its scale / bsum index; high stream is si+4
    const int r0 = blockIdx.x * RB;
    const int nr = min(RB, rows - r0);

    uint4 ql[RB], qh[RB];
    uint2 scv[RB];
    uint32_t dv[RB];
    const uint8_t *wb = W + (int64_t)r0 * w_row_bytes + (int64_t)b * Q6K_BYTES;
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        if (valid && rr < nr) {
            const uint8_t *blk = wb + rr * w_row_bytes;
            ql[rr] = ld16(blk + 64 * jj + 32 * p + 16 * t);
            qh[rr] = ld16(blk + 128 + 32 * jj + 16 * t);
            scv[rr] = ld8(blk + 192 + 8 * jj);
            dv[rr] = ld2(blk + 208);
        } else {
            ql[rr] = qh[rr] = make_uint4(0, 0, 0, 0);
            scv[rr] = make_uint2(0, 0);
            dv[rr] = 0;
        }
    }
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
    const int sh = 2 * p;
    const int sa_shift = 8 * ((2 * p + t) & 3);  // byte of sc[si] inside the 8-byte scale load
    float part[NC][RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        uint32_t va[4], vb[4];
        const uint32_t qlv[4] = {ql[rr].x, ql[rr].y, ql[rr].z, ql[rr].w};
        const uint32_t qhv[4] = {qh[rr].x, qh[rr].y, qh[rr].z, qh[rr].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            va[k] = (qlv[k] & 0x0f0f0f0f) | (((qhv[k] >> sh) & 0x03030303) << 4);
            vb[k] = ((qlv[k] >> 4) & 0x0f0f0f0f) | (((qhv[k] >> (sh + 4)) & 0x03030303) << 4);
        }
        // sc[si] is byte (2p+t) of the low word, sc[si+4] the same byte of the high word
        const int sca = (int)(int8_t)((scv[rr].x >> sa_shift) & 0xff);
        const int scb = (int)(int8_t)((scv[rr].y >> sa_shift) & 0xff);
        const float dw = h2f(dv[rr]);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int dA = dot4(va[3], ya[c].w, dot4(va[2], ya[c].z, dot4(va[1], ya[c].y, dot4(va[0], ya[c].x, 0))));
            const int dB = dot4(vb[3], yb[c].w, dot4(vb[2], yb[c].z, dot4(vb[1], yb[c].y, dot4(vb[0], yb[c].x, 0))));
            const int is = sca * (dA - bsa[c]) + scb * (dB - bsb[c]);
            if (SUBSUMS) {
                const int isb = group8_sum(is);
                if (j == 0 && valid && c < ncols && rr < nr) sub[((int64_t)c * rows + r0 + rr) * nb + b] = isb;
            }
            part[c][rr] = (dw * (float)is) * da[c];
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, nr, ncols, NC, nw, dst, ldd);
}

// ---------------------------------------------------------------- Q4_0 x Q8_0
// One lane per pair of 32-blocks (36 bytes, 64 elements).
template <int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q4_0_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                               int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                               int ncols, float *__restrict__ dst, int64_t ldd,
                                               int32_t *__restrict__ sub) {
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int pr = 64 * w + lane;  // pair index
    const int b0 = 2 * pr, b1 = 2 * pr + 1;
    const bool v0 = b0 < nb, v1 = b1 < nb;
    const int r0 = blockIdx.x * RB;
    const int nr = min(RB, rows - r0);

    uint4 wa[RB], wbq[RB];
    uint32_t wc[RB];
    const uint8_t *wb = W + (int64_t)r0 * w_row_bytes + (int64_t)pr * 36;
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint8_t *p = wb + rr * w_row_bytes;
        wa[rr] = wbq[rr] = make_uint4(0, 0, 0, 0);
        wc[rr] = 0;
        if (rr < nr) {
            if (v1) {
                wa[rr] = ld16(p);
                wbq[rr] = ld16(p + 16);
                wc[rr] = ld4(p + 32);
            } else if (v0) {
                wa[rr] = ld16(p);
                wbq[rr] = make_uint4(ld2(p + 16), 0, 0, 0);
            }
        }
    }
    uint4 y0l[NC], y0h[NC], y1l[NC], y1h[NC];
    int sy0[NC], sy1[NC];
    float d0[NC], d1[NC];
    const uint32_t one = 0x01010101u;
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
            sy0[c] = 8 * dot4(y0l[c].x, one, dot4(y0l[c].y, one, dot4(y0l[c].z, one, dot4(y0l[c].w, one,
                     dot4(y0h[c].x, one, dot4(y0h[c].y, one, dot4(y0h[c].z, one, dot4(y0h[c].w, one, 0))))))));
        }
        if (c < ncols && v1) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b1 * Q8_0_BYTES;
            d1[c] = h2f(ld2(A));
            y1l[c] = ld16(A + 2);
            y1h[c] = ld16(A + 18);
            sy1[c] = 8 * dot4(y1l[c].x, one, dot4(y1l[c].y, one, dot4(y1l[c].z, one, dot4(y1l[c].w, one,
                     dot4(y1h[c].x, one, dot4(y1h[c].y, one, dot4(y1h[c].z, one, dot4(y1h[c].w, one, 0))))))));
        }
    }
    float part[NC][RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint4 a = wa[rr], bq = wbq[rr];
        const float dw0 = h2f(a.x), dw1 = h2f(bq.x >> 16);
        const uint32_t q0[4] = {__builtin_amdgcn_alignbyte(a.y, a.x, 2), __builtin_amdgcn_alignbyte(a.z, a.y, 2),
                                __builtin_amdgcn_alignbyte(a.w, a.z, 2), __builtin_amdgcn_alignbyte(bq.x, a.w, 2)};
        const uint32_t q1[4] = {bq.y, bq.z, bq.w, wc[rr]};
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
            if (SUBSUMS && c < ncols && rr < nr) {
                int32_t *s = sub + ((int64_t)c * rows + r0 + rr) * nb;
                if (v0) s[b0] = s0;
                if (v1) s[b1] = s1;
            }
            float pp = v0 ? (float)s0 * (dw0 * d0[c]) : 0.0f;
            if (v1) pp = fmaf((float)s1, dw1 * d1[c], pp);
            part[c][rr] = pp;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, nr, ncols, NC, nw, dst, ldd);
}

#define GEMV_ARGS                                                                                     \
    const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act, \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub
#define GEMV_PASS W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub

#define GEMV_INST(name, impl, NC)                                                                  \
    extern "C" __global__ void __launch_bounds__(512) name##_c##NC(GEMV_ARGS) {                   \
        impl<NC, false>(GEMV_PASS);                                                                \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) name##_sub_c##NC(GEMV_ARGS) {               \
        impl<NC, true>(GEMV_PASS);                                                                 \
    }
#define GEMV_ALL(name, impl) \
    GEMV_INST(name, impl, 1) GEMV_INST(name, impl, 2) GEMV_INST(name, impl, 4) GEMV_INST(name, impl, 8)

GEMV_ALL(ghip_gemv_q6_K, gemv_q6K_impl)
GEMV_ALL(ghip_gemv_q4_0, gemv_q4_0_impl)

// Q4_K: "_f" kernels take f32 activations (fused Q8_K quantization), the
// others ready Q8_K rows; "_sub" kernels also store the integer partials.
#define Q4K_ARGS GEMV_ARGS, int rows_per_wg, int n_mat
#define Q4K_PASS GEMV_PASS, rows_per_wg, n_mat
#define Q4K_INST(NC)                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_c##NC(Q4K_ARGS) {                           \
        gemv_q4K_impl<NC, false, false>(Q4K_PASS);                                                              \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_sub_c##NC(Q4K_ARGS) {                       \
        gemv_q4K_impl<NC, true, false>(Q4K_PASS);                                                               \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_f_c##NC(Q4K_ARGS) {                         \
        gemv_q4K_impl<NC, false, true>(Q4K_PASS);                                                               \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_f_sub_c##NC(Q4K_ARGS) {                     \
        gemv_q4K_impl<NC, true, true>(Q4K_PASS);                                                                \
    }
Q4K_INST(1) Q4K_INST(2) Q4K_INST(4) Q4K_INST(8)
