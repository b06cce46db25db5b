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

constexpr int RB = 8;  // weight rows per workgroup (Q6_K, Q4_0; Q4_K takes it as a parameter)

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
// Q4_K workgroup = T row teams x W_K wavefronts (the K-team tiles the row
// once, 8 lanes per super-block).  The activation columns are quantized to
// Q8_K ONCE per workgroup, by all its lanes, into LDS; each lane then reads
// the codes of its fixed K position from there.
//
// LDS (dynamic): codes [NC][K] int8 | d [NC][nb] f32 | 16-element sums
// [NC][nb][16] int32 | row partials [T*rows_per_team][W_K][NC] f32.
#include "ghip_actq.h"

// Activation codes of one lane: elements 64i..64i+31 (low nibbles, sub-block
// 2i) and 64i+32..64i+63 (high nibbles, sub-block 2i+1) of super-block b, the
// two sub-block sums and the block scale.
struct Q4KAct {
    uint4 lo0, lo1, hi0, hi1;
    int bs0, bs1;
    float d;
};

// Q4_K workgroup = T row teams x W_K wavefronts; a wavefront covers 16
// super-blocks of a row with 4 lanes per super-block (lane i of a block owns
// qs bytes 32i..32i+31), so K <= 4096 is one wavefront and a row's partials
// never leave it.  Rows are processed in register groups of RB, two groups
// in flight (ping-pong buffers).
// Q5 = true reads Q5_K blocks (176 B: the Q4_K header, qh[32], qs[128]): the
// same scales, mins and integer sums with each nibble's fifth bit taken from
// qh -- bit 2i of qh[e] for sub-block 2i (low nibbles), bit 2i+1 for 2i+1
// (vec_dot.rs:928-980).
template <int NC, bool SUBSUMS, bool FUSEQ, int RB, int NG, bool Q5 = false, int NSLOT = 2>
__device__ __forceinline__ void gemv_q4K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                              int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                              int ncols, float *__restrict__ dst, int64_t ldd,
                                              int32_t *__restrict__ sub, int n_mat, int wg = -1) {
    // Q5_K: n_mat < 0 asks for the tiled kernel's fold (the reference's route
    // from 8 activation rows, tiled.rs: per super-block d * is - dmin * im, then
    // times d8), otherwise the row vec_dot's (main and min sums apart,
    // vec_dot.rs:934-978); its activations never take the 4x8 values
    const bool tiled_fold = Q5 && n_mat < 0;
    if (Q5) n_mat = 0;
    // NG == 0: persistent grid (one row per group, K in one wavefront): each
    // team takes ceil(rows / (teams in the grid)) consecutive rows, streamed
    // through the two register slots, so every wavefront of the grid carries
    // the same number of rows and the activation row is quantized once per
    // workgroup
    constexpr bool PERSIST = NG == 0;
    static_assert(!PERSIST || RB == 1, "persistent teams stream one row per group");
    constexpr int RPT = RB * NG;  // rows per team
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwk = (nb + 15) >> 4;                // wavefronts per K-team
    const int T = (blockDim.x >> 6) / nwk;         // row teams
    const int rpt = PERSIST ? (rows + (int)gridDim.x * T - 1) / ((int)gridDim.x * T) : RPT;
    const int team = wave / nwk, w = wave - team * nwk;
    const int K = nb * QK_K;
    int8_t *codes = reinterpret_cast<int8_t *>(smem);
    float *dq = reinterpret_cast<float *>(smem + NC * K);
    int *bsum = reinterpret_cast<int *>(dq + NC * nb);
    float *red = reinterpret_cast<float *>(bsum + NC * nb * 16);  // [T*RPT][nwk][NC], K-teams of > 1 wave

    const int b = 16 * w + (lane >> 2), i = lane & 3;
    const bool valid = b < nb;
    // wg: this workgroup's index within the matrix (-1: blockIdx.x)
    const int rw0 = (wg < 0 ? (int)blockIdx.x : wg) * T * rpt;  // first row of the workgroup (uniform)
    const int r0 = rw0 + team * rpt;       // first row of the team (uniform)
    const int r1 = min(rows, r0 + rpt);

    // Branch-free weight loads from a uniform row base: rows past the tile and
    // lanes past the row re-read a valid block (clamped index) and contribute
    // zero (their activation codes and scale are zero); a team past the last
    // row loads row rows-1 and computes nothing.
    constexpr uint32_t BBYTES = Q5 ? 176 : Q4K_BYTES;
    const uint32_t boff = (uint32_t)min(b, nb - 1) * BBYTES;
    const uint32_t qoff = boff + (Q5 ? 48 : 16) + 32 * i;
    const int rlast = min(max(r0, r1 - 1), rows - 1);
    // Row groups stream through two register slots: group g + 2 is loaded
    // into g's slot as soon as g is computed, so each wavefront keeps two
    // groups in flight and computes its early rows while its later rows are
    // still on the way (with every group loaded up front, most data would
    // land at the end and all of the arithmetic would follow the last byte).
    constexpr int NS = PERSIST ? 2 : NG < NSLOT ? NG : NSLOT;  // register slots
    uint4 hdr[NS][RB], qa[NS][RB], qb[NS][RB];
    uint4 xh0[NS][Q5 ? RB : 1], xh1[NS][Q5 ? RB : 1];  // Q5_K qh[0..15], qh[16..31]
    auto load_group = [&](int gi, int slot) {
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const uint8_t *rowp = W + (int64_t)min(r0 + gi * RB + rr, rlast) * w_row_bytes;
            hdr[slot][rr] = ld16(rowp + boff);
            qa[slot][rr] = ld16(rowp + qoff);
            qb[slot][rr] = ld16(rowp + qoff + 16);
            if constexpr (Q5) {
                xh0[slot][rr] = ld16(rowp + boff + 16);
                xh1[slot][rr] = ld16(rowp + boff + 32);
            }
        }
    };
    auto load_all = [&]() {
#pragma unroll
        for (int gi = 0; gi < NS; gi++) load_group(gi, gi);
    };
    // Activations first (their wait then does not cover the weight loads),
    // then ALL of the team's weight rows (NG groups of RB rows in flight at
    // once), then the activation image in LDS.  Quantization tasks are 16
    // elements; wavefronts without a task skip it.
    const int total = NC * nb * 16;
    const bool qwave = wave * 64 < total;
    if (FUSEQ) {
        const float *x = reinterpret_cast<const float *>(act);
        const int64_t xs = act_row_bytes / 4;
        // the first two rounds of tasks are loaded before the weights, so
        // their latencies overlap (a 14336-wide activation row is two rounds)
        XTask t0, t1;
        const bool qwave1 = (int)blockDim.x + wave * 64 < total;
        if (qwave) t0 = quant_q8K_load(x, xs, ncols, nb, total, threadIdx.x);
        if (qwave1) t1 = quant_q8K_load(x, xs, ncols, nb, total, blockDim.x + threadIdx.x);
        load_all();
        if (qwave) quant_q8K_store(t0, nb, n_mat, total, threadIdx.x, codes, dq, bsum);
        if (qwave1) quant_q8K_store(t1, nb, n_mat, total, blockDim.x + threadIdx.x, codes, dq, bsum);
        for (int base = 2 * blockDim.x; base < total; base += blockDim.x) {
            if (base + wave * 64 >= total) break;
            const XTask t = quant_q8K_load(x, xs, ncols, nb, total, base + threadIdx.x);
            quant_q8K_store(t, nb, n_mat, total, base + threadIdx.x, codes, dq, bsum);
        }
    } else {
        Q8KTask t0;
        if (qwave) t0 = q8K_load(act, act_row_bytes, ncols, nb, total, threadIdx.x);
        load_all();
        if (qwave) q8K_store(t0, nb, total, threadIdx.x, codes, dq, bsum);
        for (int base = blockDim.x; base < total; base += blockDim.x) {
            const Q8KTask t = q8K_load(act, act_row_bytes, ncols, nb, total, base + threadIdx.x);
            q8K_store(t, nb, total, base + threadIdx.x, codes, dq, bsum);
        }
    }
    __syncthreads();
    // Few columns: the lane's activation codes live in registers.  Four or
    // more: they are re-read from LDS per row group (register pressure).
    constexpr bool ACT_LDS = NC >= 4;
    constexpr int NCR = ACT_LDS ? 1 : NC;
    auto act_of = [&](int c) {
        Q4KAct r;
        if (valid) {
            const int8_t *cb = codes + (int64_t)c * K + b * QK_K + 64 * i;
            if (ACT_LDS) asm volatile("" : "+v"(cb));  // keep the loads inside the row loop
            r.lo0 = *reinterpret_cast<const uint4 *>(cb);
            r.lo1 = *reinterpret_cast<const uint4 *>(cb + 16);
            r.hi0 = *reinterpret_cast<const uint4 *>(cb + 32);
            r.hi1 = *reinterpret_cast<const uint4 *>(cb + 48);
            const int *bs16 = bsum + (c * nb + b) * 16 + 4 * i;  // sub-blocks 2i, 2i+1 = 16-groups 4i .. 4i+3
            r.bs0 = bs16[0] + bs16[1];
            r.bs1 = bs16[2] + bs16[3];
            r.d = dq[c * nb + b];
        } else {
            const uint4 z = make_uint4(0, 0, 0, 0);
            r = Q4KAct{z, z, z, z, 0, 0, 0.0f};
        }
        return r;
    };
    Q4KAct areg[NCR];
#pragma unroll
    for (int c = 0; c < NCR; c++) areg[c] = act_of(c);
    const ScaleSel sel = scale_sel(i);

    // A row group: decode the RB rows' nibbles and scales once, then one
    // pass per activation column (dots, scaling, wave reduction per row).
    auto compute_group = [&](int rg, const uint4 *hdr_, const uint4 *q0_, const uint4 *q1_, const uint4 *h0_,
                             const uint4 *h1_) {
        uint32_t lo[RB][8], hi[RB][8];
        int sc0[RB], sc1[RB], m0[RB], m1[RB];
        float dw[RB], dmin[RB];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const uint4 hd = hdr_[rr], x0 = q0_[rr], x1 = q1_[rr];
            dw[rr] = h2f(hd.x);
            dmin[rr] = h2f(hd.x >> 16);
            k4_scales(hd.y, hd.z, hd.w, sel, sc0[rr], sc1[rr], m0[rr], m1[rr]);
            const uint32_t qv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                lo[rr][k] = qv[k] & 0x0f0f0f0f;
                hi[rr][k] = (qv[k] >> 4) & 0x0f0f0f0f;
            }
            if constexpr (Q5) {
                // qh dword k covers elements 4k..4k+3; after >> 2i, bit 0 of a
                // byte is sub-block 2i's fifth bit and bit 1 sub-block 2i+1's
                const uint4 g0 = h0_[rr], g1 = h1_[rr];
                const uint32_t hv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t q2 = hv[k] >> (2 * i);
                    lo[rr][k] |= (q2 & 0x01010101u) << 4;
                    hi[rr][k] |= (q2 << 3) & 0x10101010u;
                }
            }
        }
#pragma unroll(ACT_LDS ? 1 : NC)
        for (int c = 0; c < NC; c++) {
            const Q4KAct ac = ACT_LDS ? act_of(c) : areg[ACT_LDS ? 0 : c];
            const uint32_t al[8] = {ac.lo0.x, ac.lo0.y, ac.lo0.z, ac.lo0.w, ac.lo1.x, ac.lo1.y, ac.lo1.z, ac.lo1.w};
            const uint32_t ah[8] = {ac.hi0.x, ac.hi0.y, ac.hi0.z, ac.hi0.w, ac.hi1.x, ac.hi1.y, ac.hi1.z, ac.hi1.w};
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                int dl = 0, dh = 0;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    dl = dot4(lo[rr][k], al[k], dl);
                    dh = dot4(hi[rr][k], ah[k], dh);
                }
                // |dl|, |dh| < 2^16 and scales < 64: 24-bit multiplies are exact
                const int ia = __mul24(sc0[rr], dl) + __mul24(sc1[rr], dh);
                const int im = __mul24(m0[rr], ac.bs0) + __mul24(m1[rr], ac.bs1);
                if (SUBSUMS) {
                    const int iab = quad_sum_dpp(ia), imb = quad_sum_dpp(im);
                    if (i == 0 && valid && c < ncols && rg + rr < r1) {
                        int32_t *s = sub + (((int64_t)c * rows + rg + rr) * nb + b) * 2;
                        s[0] = iab;
                        s[1] = imb;
                    }
                }
                float tot;
                if (tiled_fold) {
                    const int iab = quad_sum_dpp(ia), imb = quad_sum_dpp(im);
                    tot = wave_sum_dpp(i == 0 ? ac.d * fmaf(dw[rr], (float)iab, -(dmin[rr] * (float)imb)) : 0.0f);
                } else if constexpr (Q5) {
                    // the reference's two sums (vec_dot.rs:934-978): d * sumi
                    // with d = d8 * dw, and the mins' integer sum times
                    // -d8 * dmin, added at the end -- Q5_K's mins cancel main
                    // terms of the same size, so the two are kept apart, each
                    // from the super-block's exact integer sum
                    const int iab = quad_sum_dpp(ia), imb = quad_sum_dpp(im);
                    const float pm = i == 0 ? (ac.d * dw[rr]) * (float)iab : 0.0f;
                    const float pn = i == 0 ? (-ac.d * dmin[rr]) * (float)imb : 0.0f;
                    tot = wave_sum_dpp(pm) + wave_sum_dpp(pn);
                } else {
                    tot = wave_sum_dpp(ac.d * fmaf(dw[rr], (float)ia, -(dmin[rr] * (float)im)));
                }
                // columns past ncols (the NC - ncols padding columns) are not stored
                if (lane == 0 && c < ncols && rg + rr < r1) {
                    if (nwk == 1) dst[(int64_t)c * ldd + rg + rr] = tot;
                    else red[((rg + rr - rw0) * nwk + w) * NC + c] = tot;
                }
            }
        }
    };
    if constexpr (PERSIST) {
        const int nrow = max(0, r1 - r0);
        for (int gi = 0; gi < nrow; gi += 2) {
            // loads outside run-time branches (clamped rows past the end)
            compute_group(r0 + gi, hdr[0], qa[0], qb[0], xh0[0], xh1[0]);
            load_group(gi + 2, 0);
            if (gi + 1 < nrow) compute_group(r0 + gi + 1, hdr[1], qa[1], qb[1], xh0[1], xh1[1]);
            load_group(gi + 3, 1);
        }
        return;  // (the host launches it with K in one wavefront)
    } else {
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            const int sl = gi % NS;
            if (r0 + gi * RB < r1) compute_group(r0 + gi * RB, hdr[sl], qa[sl], qb[sl], xh0[sl], xh1[sl]);
            // unconditional (rows past the team's end re-read a clamped valid
            // row): a load under a run-time branch makes the compiler wait
            // for every outstanding load before the next group's arithmetic
            if (gi + NS < NG) load_group(gi + NS, sl);
        }
    }
    if (nwk == 1) return;
    __syncthreads();
    const int nrows = max(0, min(rows, rw0 + T * RPT) - rw0);
    for (int idx = threadIdx.x; idx < nrows * ncols; idx += blockDim.x) {
        const int rr = idx / ncols, c = idx - rr * ncols;
        float s = 0.0f;
        for (int ww = 0; ww < nwk; ww++) s += red[(rr * nwk + ww) * NC + c];
        dst[(int64_t)c * ldd + rw0 + rr] = s;
    }
}

// ---------------------------------------------------------------- Q6_K x Q8_K (v2)
// Same workgroup shape, activation image and reductions as the Q4_K kernel.
// Lane i of a super-block takes half j = i/2 (elements 128j ..) and the
// 16-element column hh = i%2 of each of its four quarters q:
// elements 128j + 32q + 16hh + [0, 16), from ql bytes 64j + 32(q&1) + 16hh
// (low nibbles for q < 2, high for q >= 2), qh bytes 32j + 16hh (bits 2q,
// 2q+1) and scale 8j + 2q + hh.  vec_dot_q6_K_q8_K (vec_dot.rs:982-1040):
// is = sum_g sc_g * (sum q6*q8 - 32 * bsum16_g), out += (d * is) * d8.
template <int NC, bool SUBSUMS, bool FUSEQ, int RB, int NG>
__device__ __forceinline__ void gemv_q6K_v2_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                                 int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                                 int ncols, float *__restrict__ dst, int64_t ldd,
                                                 int32_t *__restrict__ sub, int n_mat, int wg = -1) {
    constexpr int RPT = RB * NG;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwk = (nb + 15) >> 4;
    const int T = (blockDim.x >> 6) / nwk;
    const int team = wave / nwk, w = wave - team * nwk;
    const int K = nb * QK_K;
    int8_t *codes = reinterpret_cast<int8_t *>(smem);
    float *dq = reinterpret_cast<float *>(smem + NC * K);
    int *bsum = reinterpret_cast<int *>(dq + NC * nb);
    float *red = reinterpret_cast<float *>(bsum + NC * nb * 16);

    const int b = 16 * w + (lane >> 2), i = lane & 3;
    const int j = i >> 1, hh = i & 1;
    const bool valid = b < nb;
    const int rw0 = (wg < 0 ? (int)blockIdx.x : wg) * T * RPT;
    const int r0 = rw0 + team * RPT;
    const int r1 = min(rows, r0 + RPT);
    const uint32_t boff = (uint32_t)min(b, nb - 1) * Q6K_BYTES;
    const uint32_t o_ql = boff + 64 * j + 16 * hh, o_qh = boff + 128 + 32 * j + 16 * hh;
    const uint32_t o_sc = boff + 192 + 8 * j, o_d = boff + 208;
    const int rlast = min(max(r0, r1 - 1), rows - 1);
    // two register slots of row groups in flight, as in gemv_q4K_impl
    constexpr int NS = NG < 2 ? NG : 2;
    uint4 ql0[NS][RB], ql1[NS][RB], qhv[NS][RB];
    uint2 scv[NS][RB];
    uint32_t dv[NS][RB];
    auto load_group = [&](int gi, int slot) {
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const uint8_t *rowp = W + (int64_t)min(r0 + gi * RB + rr, rlast) * w_row_bytes;
            ql0[slot][rr] = ld16(rowp + o_ql);
            ql1[slot][rr] = ld16(rowp + o_ql + 32);
            qhv[slot][rr] = ld16(rowp + o_qh);
            scv[slot][rr] = ld8(rowp + o_sc);
            dv[slot][rr] = ld2(rowp + o_d);
        }
    };
    auto load_all = [&]() {
#pragma unroll
        for (int gi = 0; gi < NS; gi++) load_group(gi, gi);
    };
    const int total = NC * nb * 16;
    const bool qwave = wave * 64 < total;
    if (FUSEQ) {
        const float *x = reinterpret_cast<const float *>(act);
        const int64_t xs = act_row_bytes / 4;
        // the first two rounds of tasks are loaded before the weights, so
        // their latencies overlap (a 14336-wide activation row is two rounds)
        XTask t0, t1;
        const bool qwave1 = (int)blockDim.x + wave * 64 < total;
        if (qwave) t0 = quant_q8K_load(x, xs, ncols, nb, total, threadIdx.x);
        if (qwave1) t1 = quant_q8K_load(x, xs, ncols, nb, total, blockDim.x + threadIdx.x);
        load_all();
        if (qwave) quant_q8K_store(t0, nb, n_mat, total, threadIdx.x, codes, dq, bsum);
        if (qwave1) quant_q8K_store(t1, nb, n_mat, total, blockDim.x + threadIdx.x, codes, dq, bsum);
        for (int base = 2 * blockDim.x; base < total; base += blockDim.x) {
            if (base + wave * 64 >= total) break;
            const XTask t = quant_q8K_load(x, xs, ncols, nb, total, base + threadIdx.x);
            quant_q8K_store(t, nb, n_mat, total, base + threadIdx.x, codes, dq, bsum);
        }
    } else {
        Q8KTask t0;
        if (qwave) t0 = q8K_load(act, act_row_bytes, ncols, nb, total, threadIdx.x);
        load_all();
        if (qwave) q8K_store(t0, nb, total, threadIdx.x, codes, dq, bsum);
        for (int base = blockDim.x; base < total; base += blockDim.x) {
            const Q8KTask t = q8K_load(act, act_row_bytes, ncols, nb, total, base + threadIdx.x);
            q8K_store(t, nb, total, base + threadIdx.x, codes, dq, bsum);
        }
    }
    __syncthreads();
    // activation codes of this lane (4 quarters x 16) and its four 16-sums x 32
    struct Q6Act {
        uint4 y[4];
        int bs32[4];
        float d;
    };
    constexpr bool ACT_LDS = NC >= 4;
    constexpr int NCR = ACT_LDS ? 1 : NC;
    auto act_of = [&](int c) {
        Q6Act r;
        if (valid) {
            const int8_t *cb = codes + (int64_t)c * K + b * QK_K + 128 * j + 16 * hh;
            if (ACT_LDS) asm volatile("" : "+v"(cb));
            const int *bs16 = bsum + (c * nb + b) * 16 + 8 * j + hh;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                r.y[q] = *reinterpret_cast<const uint4 *>(cb + 32 * q);
                r.bs32[q] = 32 * bs16[2 * q];
            }
            r.d = dq[c * nb + b];
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                r.y[q] = make_uint4(0, 0, 0, 0);
                r.bs32[q] = 0;
            }
            r.d = 0.0f;
        }
        return r;
    };
    Q6Act areg[NCR];
#pragma unroll
    for (int c = 0; c < NCR; c++) areg[c] = act_of(c);

    auto compute_group = [&](int rg, const uint4 *l0_, const uint4 *l1_, const uint4 *qh_, const uint2 *sc_,
                             const uint32_t *d_) {
        uint32_t q6[RB][4][4];
        int sc[RB][4];
        float dw[RB];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const uint32_t la[4] = {l0_[rr].x, l0_[rr].y, l0_[rr].z, l0_[rr].w};
            const uint32_t lb[4] = {l1_[rr].x, l1_[rr].y, l1_[rr].z, l1_[rr].w};
            const uint32_t hv[4] = {qh_[rr].x, qh_[rr].y, qh_[rr].z, qh_[rr].w};
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t src = (q & 1) ? lb[k] : la[k];
                    const uint32_t nib = (q & 2) ? ((src >> 4) & 0x0f0f0f0f) : (src & 0x0f0f0f0f);
                    q6[rr][q][k] = nib | (((hv[k] >> (2 * q)) & 0x03030303) << 4);
                }
            // scales 8j + 2q + hh: bytes hh, 2+hh, 4+hh, 6+hh of the 8 loaded
            const uint32_t s0 = sc_[rr].x, s1 = sc_[rr].y;
            sc[rr][0] = (int)(int8_t)(s0 >> (8 * hh));
            sc[rr][1] = (int)(int8_t)(s0 >> (8 * hh + 16));
            sc[rr][2] = (int)(int8_t)(s1 >> (8 * hh));
            sc[rr][3] = (int)(int8_t)(s1 >> (8 * hh + 16));
            dw[rr] = h2f(d_[rr]);
        }
#pragma unroll(ACT_LDS ? 1 : NC)
        for (int c = 0; c < NC; c++) {
            const Q6Act ac = ACT_LDS ? act_of(c) : areg[ACT_LDS ? 0 : c];
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                int is = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint4 y = ac.y[q];
                    int dqv = dot4(q6[rr][q][0], y.x, 0);
                    dqv = dot4(q6[rr][q][1], y.y, dqv);
                    dqv = dot4(q6[rr][q][2], y.z, dqv);
                    dqv = dot4(q6[rr][q][3], y.w, dqv);
                    is += sc[rr][q] * (dqv - ac.bs32[q]);
                }
                if (SUBSUMS) {
                    const int isb = quad_sum_dpp(is);
                    if (i == 0 && valid && c < ncols && rg + rr < r1) sub[((int64_t)c * rows + rg + rr) * nb + b] = isb;
                }
                const float part = (dw[rr] * (float)is) * ac.d;
                const float tot = wave_sum_dpp(part);
                // columns past ncols (the NC - ncols padding columns) are not stored
                if (lane == 0 && c < ncols && rg + rr < r1) {
                    if (nwk == 1) dst[(int64_t)c * ldd + rg + rr] = tot;
                    else red[((rg + rr - rw0) * nwk + w) * NC + c] = tot;
                }
            }
        }
    };
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        const int sl = gi % NS;
        if (r0 + gi * RB < r1) compute_group(r0 + gi * RB, ql0[sl], ql1[sl], qhv[sl], scv[sl], dv[sl]);
        if (gi + NS < NG) load_group(gi + NS, sl);  // unconditional, as in gemv_q4K_impl
    }
    if (nwk == 1) return;
    __syncthreads();
    const int nrows = max(0, min(rows, rw0 + T * RPT) - rw0);
    for (int idx = threadIdx.x; idx < nrows * ncols; idx += blockDim.x) {
        const int rr = idx / ncols, c = idx - rr * ncols;
        float sacc = 0.0f;
        for (int ww = 0; ww < nwk; ww++) sacc += red[(rr * nwk + ww) * NC + c];
        dst[(int64_t)c * ldd + rw0 + rr] = sacc;
    }
}

// ---------------------------------------------------------------- Q6_K x Q8_K
template <int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q6K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                              int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                              int ncols, float *__restrict__ dst, int64_t ldd,
                                              int32_t *__restrict__ sub, int wg = -1) {
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int b = 8 * w + (lane >> 3), j = lane & 7;
    const int jj = j >> 2, p = (j >> 1) & 1, t = j & 1;
    const bool valid = b < nb;
    const int ea = 128 * jj + 32 * p + 16 * t;  // first element of the low-nibble stream
    const int si = 8 * jj + 2 * p + t;          // its scale / bsum index; high stream is si+4
    const int r0 = (wg < 0 ? (int)blockIdx.x : wg) * RB;  // wg: index within the matrix
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
// One 32-block of quantize_row_q8_0 (quants.rs:331-362) quantized by the lane
// that consumes it, with the arithmetic of ghip_quantize_q8_0: amax over the
// block, d = f16(amax / 127), q = rne(x * 127 / amax), NaN or out of range ->
// -128.  Codes of elements 0..15 in lo, 16..31 in hi; d as the f32 value of
// its f16.
DEV void q8_0_quant_vals(const float *v, uint4 &lo, uint4 &hi, float &d);
DEV void q8_0_quant_block(const float *__restrict__ xb, uint4 &lo, uint4 &hi, float &d) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint4 t = ld16(reinterpret_cast<const uint8_t *>(xb + 4 * i));
        v[4 * i] = __uint_as_float(t.x);
        v[4 * i + 1] = __uint_as_float(t.y);
        v[4 * i + 2] = __uint_as_float(t.z);
        v[4 * i + 3] = __uint_as_float(t.w);
    }
    q8_0_quant_vals(v, lo, hi, d);
}
// the quantize_row_q8_0 arithmetic on 32 values already in registers
DEV void q8_0_quant_vals(const float *v, uint4 &lo, uint4 &hi, float &d) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float dd = __fdiv_rn(amax, 127.0f);
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    uint32_t pk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float r = rintf(__fmul_rn(v[4 * k + i], id));
            const int q = (r != r || fabsf(r) >= 2147483648.0f) ? -128 : (int)r;
            w |= (uint32_t)(q & 0xff) << (8 * i);
        }
        pk[k] = w;
    }
    lo = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    hi = make_uint4(pk[4], pk[5], pk[6], pk[7]);
    d = h2f(f2h_rn(dd));
}

// FUSEQ: act is the f32 activation rows (act_row_bytes apart) and each lane
// quantizes its own two blocks per column (q8_0_quant_block); otherwise act
// holds ready Q8_0 rows.
template <int NC, bool SUBSUMS, bool FUSEQ>
__device__ __forceinline__ void gemv_q4_0_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                               int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                               int ncols, float *__restrict__ dst, int64_t ldd,
                                               int32_t *__restrict__ sub, int wg = -1) {
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int pr = 64 * w + lane;  // pair index
    const int b0 = 2 * pr, b1 = 2 * pr + 1;
    const bool v0 = b0 < nb, v1 = b1 < nb;
    const int r0 = (wg < 0 ? (int)blockIdx.x : wg) * RB;  // wg: index within the matrix
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
        if (c < ncols && v0 && FUSEQ) {
            const float *xr = reinterpret_cast<const float *>(act + c * act_row_bytes) + (int64_t)b0 * 32;
            q8_0_quant_block(xr, y0l[c], y0h[c], d0[c]);
            if (v1) q8_0_quant_block(xr + 32, y1l[c], y1h[c], d1[c]);
        }
        if (c < ncols && v0 && !FUSEQ) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b0 * Q8_0_BYTES;
            d0[c] = h2f(ld2(A));
            y0l[c] = ld16(A + 2);
            y0h[c] = ld16(A + 18);
        }
        if (c < ncols && v1 && !FUSEQ) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b1 * Q8_0_BYTES;
            d1[c] = h2f(ld2(A));
            y1l[c] = ld16(A + 2);
            y1h[c] = ld16(A + 18);
        }
        // the -8 of every nibble as -8 * sum(q8) (zero for absent blocks)
        sy0[c] = 8 * dot4(y0l[c].x, one, dot4(y0l[c].y, one, dot4(y0l[c].z, one, dot4(y0l[c].w, one,
                 dot4(y0h[c].x, one, dot4(y0h[c].y, one, dot4(y0h[c].z, one, dot4(y0h[c].w, one, 0))))))));
        sy1[c] = 8 * dot4(y1l[c].x, one, dot4(y1l[c].y, one, dot4(y1l[c].z, one, dot4(y1l[c].w, one,
                 dot4(y1h[c].x, one, dot4(y1h[c].y, one, dot4(y1h[c].z, one, dot4(y1h[c].w, one, 0))))))));
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

// Q4_0, whole row groups and pairs (rows % RB == 0, even nb): the same
// arithmetic as gemv_q4_0_impl with every load unconditional (lanes past the
// row's pairs re-read its last pair and contribute zero), the activation
// loads issued before the weights.  A load under a run-time branch, or
// activations loaded after the weights, made the quantization wait for every
// weight byte (loads complete in order).
template <int NC, bool SUBSUMS, bool FUSEQ>
__device__ __forceinline__ void gemv_q4_0_full_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                                    int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                                    int ncols, float *__restrict__ dst, int64_t ldd,
                                                    int32_t *__restrict__ sub, int wg = -1) {
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int pr = 64 * w + lane, np = nb >> 1;
    const bool v = pr < np;
    const int b0 = 2 * min(pr, np - 1), b1 = b0 + 1;
    const int r0 = (wg < 0 ? (int)blockIdx.x : wg) * RB;

    // activations first: f32 values (FUSEQ) or the Q8_0 blocks of columns
    // c < ncols (columns past ncols re-read column 0 and are zeroed below)
    float xv[FUSEQ ? NC : 1][64];
    uint4 y0l[NC], y0h[NC], y1l[NC], y1h[NC];
    uint32_t dh[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int cc = c < ncols ? c : 0;
        if constexpr (FUSEQ) {
            const uint8_t *xr = act + cc * act_row_bytes + (int64_t)b0 * 128;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint4 t = ld16(xr + 16 * i);
                xv[c][4 * i] = __uint_as_float(t.x);
                xv[c][4 * i + 1] = __uint_as_float(t.y);
                xv[c][4 * i + 2] = __uint_as_float(t.z);
                xv[c][4 * i + 3] = __uint_as_float(t.w);
            }
        } else {
            const uint8_t *A = act + cc * act_row_bytes + (int64_t)b0 * Q8_0_BYTES;
            dh[c] = ld2(A) | ((uint32_t)ld2(A + Q8_0_BYTES) << 16);
            y0l[c] = ld16(A + 2);
            y0h[c] = ld16(A + 18);
            y1l[c] = ld16(A + Q8_0_BYTES + 2);
            y1h[c] = ld16(A + Q8_0_BYTES + 18);
        }
    }
    uint4 wa[RB], wbq[RB];
    uint32_t wc[RB];
    const uint8_t *wb = W + (int64_t)r0 * w_row_bytes + (int64_t)(b0 >> 1) * 36;
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint8_t *p = wb + rr * w_row_bytes;
        wa[rr] = ld16(p);
        wbq[rr] = ld16(p + 16);
        wc[rr] = ld4(p + 32);
    }
    // every weight load is issued before the activations are consumed: the
    // values pass through an empty asm that no load can move across
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if constexpr (FUSEQ) {
#pragma unroll
            for (int i = 0; i < 64; i++) asm volatile("" : "+v"(xv[c][i]) : : "memory");
        } else {
            uint4 *ys[4] = {&y0l[c], &y0h[c], &y1l[c], &y1h[c]};
#pragma unroll
            for (int k = 0; k < 4; k++)
                asm volatile("" : "+v"(ys[k]->x), "+v"(ys[k]->y), "+v"(ys[k]->z), "+v"(ys[k]->w) : : "memory");
            asm volatile("" : "+v"(dh[c]) : : "memory");
        }
    }
    int sy0[NC], sy1[NC];
    float d0[NC], d1[NC];
    const uint32_t one = 0x01010101u;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if constexpr (FUSEQ) {
            q8_0_quant_vals(&xv[c][0], y0l[c], y0h[c], d0[c]);
            q8_0_quant_vals(&xv[c][32], y1l[c], y1h[c], d1[c]);
        } else {
            d0[c] = h2f(dh[c] & 0xffffu);
            d1[c] = h2f(dh[c] >> 16);
        }
        if (c >= ncols) d0[c] = d1[c] = 0.0f;
        sy0[c] = 8 * dot4(y0l[c].x, one, dot4(y0l[c].y, one, dot4(y0l[c].z, one, dot4(y0l[c].w, one,
                 dot4(y0h[c].x, one, dot4(y0h[c].y, one, dot4(y0h[c].z, one, dot4(y0h[c].w, one, 0))))))));
        sy1[c] = 8 * dot4(y1l[c].x, one, dot4(y1l[c].y, one, dot4(y1l[c].z, one, dot4(y1l[c].w, one,
                 dot4(y1h[c].x, one, dot4(y1h[c].y, one, dot4(y1h[c].z, one, dot4(y1h[c].w, one, 0))))))));
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
            if (SUBSUMS && c < ncols && v) {
                int32_t *s = sub + ((int64_t)c * rows + r0 + rr) * nb;
                s[b0] = s0;
                s[b1] = s1;
            }
            // exactly 0 from lanes past the row (as in gemv_q4_0_impl)
            part[c][rr] = v ? fmaf((float)s1, dw1 * d1[c], (float)s0 * (dw0 * d0[c])) : 0.0f;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, RB, ncols, NC, nw, dst, ldd);
}

// ---------------------------------------------------------------- Q5_0 / Q8_0 x Q8_0
// The Q4_0 work layout: one lane per pair of 32-blocks, RB rows per
// workgroup, all rows' loads issued before any is consumed.  Block values:
//   Q8_0: the int8 codes                                  (vec_dot.rs:732-756)
//   Q5_0: (nibble | bit e of qh << 4) - 16, the -16 folded in as
//         -16 * sum(q8) per block, as Q4_0 folds its -8   (vec_dot.rs:661-686)
// The integer block sums are the reference's exactly; they are scaled by
// d_w * d_x in fp32 per block.
constexpr int WT_Q5_0 = 6, WT_Q8_0 = 8;

// bit j (< 4) of t moved to bit 4 of byte j: t * (2^4 + 2^11) puts bit j at
// j+4 and j+11, the copy shifted by 14 adds j+18 and j+25; of these only
// 4, 12, 20 and 28 survive the mask (one per j, no carries)
DEV uint32_t spread4_bit4(uint32_t t) {
    const uint32_t m = __mul24(t, 0x810u);
    return ((m << 14) | m) & 0x10101010u;
}

template <int WT>
DEV void pair_block_codes(const uint32_t *w, int blk, uint32_t (&q)[8], float &d) {
    if constexpr (WT == WT_Q8_0) {
        // block 0: d = bytes 0-1, codes 2..33; block 1: d = bytes 34-35, codes 36..67
        if (blk == 0) {
            d = h2f(w[0] & 0xffffu);
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
        } else {
            d = h2f(w[8] >> 16);
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] = w[9 + k];
        }
    } else {
        // block 0: d = bytes 0-1, qh 2..5, qs 6..21; block 1: d = 22-23, qh 24..27, qs 28..43
        uint32_t qh, qs[4];
        if (blk == 0) {
            d = h2f(w[0] & 0xffffu);
            qh = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
#pragma unroll
            for (int k = 0; k < 4; k++) qs[k] = __builtin_amdgcn_alignbyte(w[k + 2], w[k + 1], 2);
        } else {
            d = h2f(w[5] >> 16);
            qh = w[6];
#pragma unroll
            for (int k = 0; k < 4; k++) qs[k] = w[7 + k];
        }
        // elements 4k..4k+3 (low nibbles, qh bits 4k..) and 16+4k.. (high nibbles)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q[k] = (qs[k] & 0x0f0f0f0fu) | spread4_bit4(__builtin_amdgcn_ubfe(qh, 4 * k, 4));
            q[4 + k] = ((qs[k] >> 4) & 0x0f0f0f0fu) | spread4_bit4(__builtin_amdgcn_ubfe(qh, 16 + 4 * k, 4));
        }
    }
}

// FULL (pre-quantized activations, rows % RB == 0, even nb): the activation
// blocks are loaded first and every weight load is unconditional (lanes past
// the row's pairs re-read its last pair and add exactly 0), as in
// gemv_q4_0_full_impl.
template <int WT, int NC, bool SUBSUMS, bool FUSEQ, bool FULL = false>
__device__ __forceinline__ void gemv_pair_q8_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                                  int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                                  int ncols, float *__restrict__ dst, int64_t ldd,
                                                  int32_t *__restrict__ sub, int wg = -1) {
    static_assert(!FULL || !FUSEQ, "FULL takes ready Q8_0 rows");
    constexpr int PB = WT == WT_Q8_0 ? 68 : 44;  // bytes per block pair
    constexpr int ND = PB / 4;                  // dwords per block pair
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int pr = 64 * w + lane;  // pair index
    const int prl = FULL ? min(pr, (nb >> 1) - 1) : pr;  // the pair loaded
    const int b0 = 2 * prl, b1 = 2 * prl + 1;
    const bool v0 = FULL ? pr < (nb >> 1) : b0 < nb, v1 = FULL ? v0 : b1 < nb;
    const int r0 = (wg < 0 ? (int)blockIdx.x : wg) * RB;  // wg: index within the matrix
    const int nr = FULL ? RB : min(RB, rows - r0);

    uint4 y0l[NC], y0h[NC], y1l[NC], y1h[NC];
    uint32_t dh[NC];
    if constexpr (FULL) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint8_t *A = act + (c < ncols ? c : 0) * act_row_bytes + (int64_t)b0 * Q8_0_BYTES;
            dh[c] = ld2(A) | ((uint32_t)ld2(A + Q8_0_BYTES) << 16);
            y0l[c] = ld16(A + 2);
            y0h[c] = ld16(A + 18);
            y1l[c] = ld16(A + Q8_0_BYTES + 2);
            y1h[c] = ld16(A + Q8_0_BYTES + 18);
        }
    }

    uint32_t wq[RB][ND];
    const uint8_t *wb = W + (int64_t)r0 * w_row_bytes + (int64_t)prl * PB;
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint8_t *p = wb + rr * w_row_bytes;
#pragma unroll
        for (int k = 0; k < ND; k++) wq[rr][k] = 0;
        if (FULL || (rr < nr && v0)) {
            // the first block always; the second only when it exists (a lone
            // last block reads its own 22 / 34 bytes, nothing past the row)
            const uint4 a = ld16(p);
            wq[rr][0] = a.x; wq[rr][1] = a.y; wq[rr][2] = a.z; wq[rr][3] = a.w;
            if constexpr (WT == WT_Q8_0) {
                const uint4 b = ld16(p + 16);
                wq[rr][4] = b.x; wq[rr][5] = b.y; wq[rr][6] = b.z; wq[rr][7] = b.w;
                if (FULL || v1) {
                    const uint4 c = ld16(p + 32), e = ld16(p + 48);
                    wq[rr][8] = c.x; wq[rr][9] = c.y; wq[rr][10] = c.z; wq[rr][11] = c.w;
                    wq[rr][12] = e.x; wq[rr][13] = e.y; wq[rr][14] = e.z; wq[rr][15] = e.w;
                    wq[rr][16] = ld4(p + 64);
                } else {
                    wq[rr][8] = ld2(p + 32);
                }
            } else {
                if (FULL || v1) {
                    const uint4 b = ld16(p + 16);
                    const uint2 c = ld8(p + 32);
                    wq[rr][4] = b.x; wq[rr][5] = b.y; wq[rr][6] = b.z; wq[rr][7] = b.w;
                    wq[rr][8] = c.x; wq[rr][9] = c.y;
                    wq[rr][10] = ld4(p + 40);
                } else {
                    wq[rr][4] = ld4(p + 16);
                    wq[rr][5] = ld2(p + 20);
                }
            }
        }
    }
    if constexpr (FULL) {
        // the activation values pass through an empty asm after the weight
        // loads, so no wait for them moves above a weight load
#pragma unroll
        for (int c = 0; c < NC; c++) {
            uint4 *ys[4] = {&y0l[c], &y0h[c], &y1l[c], &y1h[c]};
#pragma unroll
            for (int k = 0; k < 4; k++)
                asm volatile("" : "+v"(ys[k]->x), "+v"(ys[k]->y), "+v"(ys[k]->z), "+v"(ys[k]->w) : : "memory");
            asm volatile("" : "+v"(dh[c]) : : "memory");
        }
    }
    int sy0[NC], sy1[NC];
    float d0[NC], d1[NC];
    const uint32_t one = 0x01010101u;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if constexpr (FULL) {
            d0[c] = c < ncols ? h2f(dh[c] & 0xffffu) : 0.0f;
            d1[c] = c < ncols ? h2f(dh[c] >> 16) : 0.0f;
        } else {
            y0l[c] = y0h[c] = y1l[c] = y1h[c] = make_uint4(0, 0, 0, 0);
            d0[c] = d1[c] = 0.0f;
        }
        sy0[c] = sy1[c] = 0;
        if (c < ncols && v0 && FUSEQ) {
            const float *xr = reinterpret_cast<const float *>(act + c * act_row_bytes) + (int64_t)b0 * 32;
            q8_0_quant_block(xr, y0l[c], y0h[c], d0[c]);
            if (v1) q8_0_quant_block(xr + 32, y1l[c], y1h[c], d1[c]);
        }
        if (c < ncols && v0 && !FUSEQ && !FULL) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b0 * Q8_0_BYTES;
            d0[c] = h2f(ld2(A));
            y0l[c] = ld16(A + 2);
            y0h[c] = ld16(A + 18);
        }
        if (c < ncols && v1 && !FUSEQ && !FULL) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b1 * Q8_0_BYTES;
            d1[c] = h2f(ld2(A));
            y1l[c] = ld16(A + 2);
            y1h[c] = ld16(A + 18);
        }
        if constexpr (WT == WT_Q5_0) {
            sy0[c] = 16 * dot4(y0l[c].x, one, dot4(y0l[c].y, one, dot4(y0l[c].z, one, dot4(y0l[c].w, one,
                     dot4(y0h[c].x, one, dot4(y0h[c].y, one, dot4(y0h[c].z, one, dot4(y0h[c].w, one, 0))))))));
            sy1[c] = 16 * dot4(y1l[c].x, one, dot4(y1l[c].y, one, dot4(y1l[c].z, one, dot4(y1l[c].w, one,
                     dot4(y1h[c].x, one, dot4(y1h[c].y, one, dot4(y1h[c].z, one, dot4(y1h[c].w, one, 0))))))));
        }
    }
    float part[NC][RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        uint32_t q0[8], q1[8];
        float dw0, dw1;
        pair_block_codes<WT>(wq[rr], 0, q0, dw0);
        pair_block_codes<WT>(wq[rr], 1, q1, dw1);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int s0 = dot4(q0[7], y0h[c].w, dot4(q0[6], y0h[c].z, dot4(q0[5], y0h[c].y, dot4(q0[4], y0h[c].x,
                           dot4(q0[3], y0l[c].w, dot4(q0[2], y0l[c].z, dot4(q0[1], y0l[c].y, dot4(q0[0], y0l[c].x,
                           -sy0[c]))))))));
            const int s1 = dot4(q1[7], y1h[c].w, dot4(q1[6], y1h[c].z, dot4(q1[5], y1h[c].y, dot4(q1[4], y1h[c].x,
                           dot4(q1[3], y1l[c].w, dot4(q1[2], y1l[c].z, dot4(q1[1], y1l[c].y, dot4(q1[0], y1l[c].x,
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

template <int NC, bool SUBSUMS, bool FUSEQ>
__device__ __forceinline__ void gemv_q5_0_full_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                                    int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                                    int ncols, float *__restrict__ dst, int64_t ldd,
                                                    int32_t *__restrict__ sub, int wg = -1) {
    gemv_pair_q8_impl<WT_Q5_0, NC, SUBSUMS, false, true>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst,
                                                         ldd, sub, wg);
}
template <int NC, bool SUBSUMS, bool FUSEQ>
__device__ __forceinline__ void gemv_q5_0_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb,
                                               const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols,
                                               float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub,
                                               int wg = -1) {
    gemv_pair_q8_impl<WT_Q5_0, NC, SUBSUMS, FUSEQ>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub,
                                                   wg);
}
template <int NC, bool SUBSUMS, bool FUSEQ>
__device__ __forceinline__ void gemv_q8_0_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb,
                                               const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols,
                                               float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub,
                                               int wg = -1) {
    gemv_pair_q8_impl<WT_Q8_0, NC, SUBSUMS, FUSEQ>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub,
                                                   wg);
}

// ---------------------------------------------------------------- Q4_1 / Q5_1 x Q8_1
// One lane per 32-block, RB rows per workgroup (all rows' loads issued before
// any is consumed), Q8_1 activation rows quantized by ghip_quantize_q8_1.
// vec_dot_q4_1_q8_1 / vec_dot_q5_1_q8_1 (vec_dot.rs:620-720): per block the
// exact integer sum of the unsigned codes (nibble, | bit e of qh << 4 for
// Q5_1) times the Q8_1 codes, scaled as (d_w * d_x) * sumi + m_w * s_x.
constexpr int WT_Q4_1 = 3, WT_Q5_1 = 7;
template <int WT, int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_q41_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb,
                                              const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols,
                                              float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    constexpr int BB = WT == WT_Q4_1 ? 20 : 24;  // block bytes: d, m, (qh), qs[16]
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int b = 64 * w + lane;
    const bool valid = b < nb;
    const int r0 = (int)blockIdx.x * RB;
    const int nr = min(RB, rows - r0);
    uint32_t wq[RB][6];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
#pragma unroll
        for (int k = 0; k < 6; k++) wq[rr][k] = 0;
        if (rr < nr && valid) {
            const uint8_t *p = W + (int64_t)(r0 + rr) * w_row_bytes + (int64_t)b * BB;
            const uint4 a = ld16(p);
            wq[rr][0] = a.x; wq[rr][1] = a.y; wq[rr][2] = a.z; wq[rr][3] = a.w;
            if constexpr (WT == WT_Q4_1) {
                wq[rr][4] = ld4(p + 16);
            } else {
                const uint2 c = ld8(p + 16);
                wq[rr][4] = c.x; wq[rr][5] = c.y;
            }
        }
    }
    uint4 yl[NC], yh[NC];
    float dx[NC], sx[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        yl[c] = yh[c] = make_uint4(0, 0, 0, 0);
        dx[c] = sx[c] = 0.0f;
        if (c < ncols && valid) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b * 36;
            const uint32_t ds = ld4(A);
            dx[c] = h2f(ds);
            sx[c] = h2f(ds >> 16);
            yl[c] = ld16(A + 4);
            yh[c] = ld16(A + 20);
        }
    }
    float part[NC][RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const float dw = h2f(wq[rr][0]), mw = h2f(wq[rr][0] >> 16);
        uint32_t qs[4], qh = 0;
        if constexpr (WT == WT_Q4_1) {
#pragma unroll
            for (int k = 0; k < 4; k++) qs[k] = wq[rr][1 + k];
        } else {
            qh = wq[rr][1];
#pragma unroll
            for (int k = 0; k < 4; k++) qs[k] = wq[rr][2 + k];
        }
        // elements 4k..4k+3 (low nibbles) and 16+4k.. (high nibbles)
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q[k] = qs[k] & 0x0f0f0f0fu;
            q[4 + k] = (qs[k] >> 4) & 0x0f0f0f0fu;
            if constexpr (WT == WT_Q5_1) {
                q[k] |= spread4_bit4(__builtin_amdgcn_ubfe(qh, 4 * k, 4));
                q[4 + k] |= spread4_bit4(__builtin_amdgcn_ubfe(qh, 16 + 4 * k, 4));
            }
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int si = dot4(q[7], yh[c].w, dot4(q[6], yh[c].z, dot4(q[5], yh[c].y, dot4(q[4], yh[c].x,
                           dot4(q[3], yl[c].w, dot4(q[2], yl[c].z, dot4(q[1], yl[c].y, dot4(q[0], yl[c].x, 0))))))));
            if (SUBSUMS && c < ncols && rr < nr && valid) sub[((int64_t)c * rows + r0 + rr) * nb + b] = si;
            part[c][rr] = valid ? fmaf(dw * dx[c], (float)si, mw * sx[c]) : 0.0f;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, nr, ncols, NC, nw, dst, ldd);
}
#define GEMV_Q41_INST(TN, WT, NC)                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_c##NC(                                    \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_q41_impl<WT, NC, false>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);       \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_sub_c##NC(                                \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_q41_impl<WT, NC, true>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);        \
    }
GEMV_Q41_INST(q4_1, WT_Q4_1, 1) GEMV_Q41_INST(q4_1, WT_Q4_1, 2) GEMV_Q41_INST(q4_1, WT_Q4_1, 4)
GEMV_Q41_INST(q4_1, WT_Q4_1, 8)
GEMV_Q41_INST(q5_1, WT_Q5_1, 1) GEMV_Q41_INST(q5_1, WT_Q5_1, 2) GEMV_Q41_INST(q5_1, WT_Q5_1, 4)
GEMV_Q41_INST(q5_1, WT_Q5_1, 8)

// ---------------------------------------------------------------- Q2_K / Q3_K x Q8_K
// Four lanes per super-block: lane quarter qq takes 128-group j = qq / 2 and
// shift groups k = 2(qq & 1), 2(qq & 1) + 1, i.e. elements 128j + 32k + e
// (e < 32) with codes (qs[32j + e] >> 2k) & 3 and scales 8j + 2k + (e >= 16)
// (dequantize_row_q2_K / _q3_K, quants.rs:431-520).  Per super-block
// (vec_dot_q2_K_q8_K / _q3_K_q8_K, vec_dot.rs:758-834):
//   Q2_K: isum = sum_g (sc_g & 15) * sum q * q8,  summs = sum_g (sc_g >> 4) * bsum16_g,
//         d8 * d * isum - d8 * dmin * summs;
//   Q3_K: values lo - 4 where the hmask bit 4j + k is clear, scales sc_g - 32,
//         isum = sum_g (sc_g - 32) * sum v * q8,  d8 * d * isum.
// RB rows per workgroup, each row's bytes loaded one row ahead; the integer
// sums are exact and (_sub kernels) exported per super-block.
constexpr int WT_Q2_K = 10, WT_Q3_K = 11;
template <int WT, int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_k23_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb,
                                              const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols,
                                              float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    constexpr bool Q2 = WT == WT_Q2_K;
    constexpr int BB = Q2 ? 84 : 110;
    constexpr int NWD = Q2 ? 10 : 20;  // dwords of weight data per lane and row
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int qq = lane & 3, j = qq >> 1, kp = qq & 1;  // k = 2kp, 2kp + 1
    const int b = 16 * w + (lane >> 2);
    const bool valid = b < nb;
    const int r0 = (int)blockIdx.x * RB;
    const int nr = min(RB, rows - r0);
    const uint8_t *base = W + (int64_t)min(b, nb - 1) * BB;
    // Q2_K: scales 8j+4kp .. +3 | qs 32j .. +31 (8 dwords) | d, dmin
    // Q3_K: hmask (8 dwords) | qs 32j .. +31 (8 dwords) | scales 12 bytes | d
    auto load_row = [&](int rr, uint32_t (&v)[NWD]) {
        const uint8_t *p = base + (int64_t)min(r0 + rr, rows - 1) * w_row_bytes;
        if constexpr (Q2) {
            v[0] = ld4(p + 8 * j + 4 * kp);
            const uint4 a = ld16(p + 16 + 32 * j), c = ld16(p + 32 + 32 * j);
            v[1] = a.x; v[2] = a.y; v[3] = a.z; v[4] = a.w;
            v[5] = c.x; v[6] = c.y; v[7] = c.z; v[8] = c.w;
            v[9] = ld4(p + 80);
        } else {
            const uint4 h0 = ld16(p), h1 = ld16(p + 16), a = ld16(p + 32 + 32 * j), c = ld16(p + 48 + 32 * j);
            v[0] = h0.x; v[1] = h0.y; v[2] = h0.z; v[3] = h0.w;
            v[4] = h1.x; v[5] = h1.y; v[6] = h1.z; v[7] = h1.w;
            v[8] = a.x; v[9] = a.y; v[10] = a.z; v[11] = a.w;
            v[12] = c.x; v[13] = c.y; v[14] = c.z; v[15] = c.w;
            const uint2 s01 = ld8(p + 96);
            v[16] = s01.x;
            v[17] = s01.y;
            v[18] = ld4(p + 104);
            v[19] = ld2(p + 108);
        }
    };
    // activations: codes of elements 128j + 32k + e for the lane's two k, bsum16
    // of its four groups (Q2_K), d
    uint4 ya[NC][4];
    int bs[NC][4];
    float dy[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        dy[c] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            ya[c][i] = make_uint4(0, 0, 0, 0);
            bs[c][i] = 0;
        }
        if (c < ncols && valid) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)b * Q8K_BYTES;
            dy[c] = __uint_as_float(ld4(A));
#pragma unroll
            for (int i = 0; i < 4; i++) ya[c][i] = ld16(A + 4 + 128 * j + 64 * kp + 16 * i);
            if constexpr (Q2) {
                const uint2 g = ld8(A + 260 + 2 * (8 * j + 4 * kp));
                bs[c][0] = (int)(int16_t)(g.x & 0xffff);
                bs[c][1] = (int)(int16_t)(g.x >> 16);
                bs[c][2] = (int)(int16_t)(g.y & 0xffff);
                bs[c][3] = (int)(int16_t)(g.y >> 16);
            }
        }
    }
    float part[NC][RB];
    uint32_t wv[2][NWD];
    load_row(0, wv[0]);
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        if (rr + 1 < RB) load_row(rr + 1, wv[(rr + 1) & 1]);
        const uint32_t *v = wv[rr & 1];
        int sc4[4];  // scales of groups (k0, h0), (k0, h1), (k1, h0), (k1, h1)
        float dw, dmw = 0.0f;
        uint32_t q[2][8];  // codes of e = 4i .. 4i+3 per k, as bytes
        if constexpr (Q2) {
#pragma unroll
            for (int g = 0; g < 4; g++) sc4[g] = (int)((v[0] >> (8 * g)) & 0xff);
            dw = h2f(v[9]);
            dmw = h2f(v[9] >> 16);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 8; i++) q[t][i] = (v[1 + i] >> (2 * (2 * kp + t))) & 0x03030303u;
        } else {
            // the scale word 2j + kp of the de-packed 16 (quants.rs:475-484)
            const uint32_t a0 = v[16], a1 = v[17], a2 = v[18];
            const uint32_t km1 = 0x03030303u, km2 = 0x0f0f0f0fu;
            const int wi = 2 * j + kp;
            const uint32_t sw = wi == 0   ? (a0 & km2) | ((a2 & km1) << 4)
                                : wi == 1 ? (a1 & km2) | (((a2 >> 2) & km1) << 4)
                                : wi == 2 ? ((a0 >> 4) & km2) | (((a2 >> 4) & km1) << 4)
                                          : ((a1 >> 4) & km2) | (((a2 >> 6) & km1) << 4);
#pragma unroll
            for (int g = 0; g < 4; g++) sc4[g] = (int)((sw >> (8 * g)) & 0xff) - 32;
            dw = h2f(v[19]);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int k = 2 * kp + t, bit = 4 * j + k;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t lo = (v[8 + i] >> (2 * k)) & 0x03030303u;
                    const uint32_t hb = (v[i] >> bit) & 0x01010101u;
                    q[t][i] = lo | ((hb ^ 0x01010101u) * 0xfcu);  // lo - 4 where the bit is clear
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            int is = 0, sm = 0;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t yv[8] = {ya[c][2 * t].x, ya[c][2 * t].y, ya[c][2 * t].z, ya[c][2 * t].w,
                                        ya[c][2 * t + 1].x, ya[c][2 * t + 1].y, ya[c][2 * t + 1].z, ya[c][2 * t + 1].w};
                int s0 = 0, s1 = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    s0 = dot4(q[t][i], yv[i], s0);
                    s1 = dot4(q[t][4 + i], yv[4 + i], s1);
                }
                if constexpr (Q2) {
                    is += __mul24(sc4[2 * t] & 15, s0) + __mul24(sc4[2 * t + 1] & 15, s1);
                    sm += __mul24(sc4[2 * t] >> 4, bs[c][2 * t]) + __mul24(sc4[2 * t + 1] >> 4, bs[c][2 * t + 1]);
                } else {
                    is += __mul24(sc4[2 * t], s0) + __mul24(sc4[2 * t + 1], s1);
                }
            }
            // the super-block's exact sums over its four lanes, folded once
            const int isb = quad_sum_dpp(is), smb = Q2 ? quad_sum_dpp(sm) : 0;
            if (SUBSUMS && qq == 0 && valid && c < ncols && rr < nr) {
                if constexpr (Q2) {
                    int32_t *sp = sub + (((int64_t)c * rows + r0 + rr) * nb + b) * 2;
                    sp[0] = isb;
                    sp[1] = smb;
                } else {
                    sub[((int64_t)c * rows + r0 + rr) * nb + b] = isb;
                }
            }
            float pp = 0.0f;
            if (valid && qq == 0) {
                pp = (dy[c] * dw) * (float)isb;
                if constexpr (Q2) pp = fmaf(-(dy[c] * dmw), (float)smb, pp);
            }
            part[c][rr] = pp;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, nr, ncols, NC, nw, dst, ldd);
}
#define GEMV_K23_INST(TN, WT, NC)                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_c##NC(                                    \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_k23_impl<WT, NC, false>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);       \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_sub_c##NC(                                \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_k23_impl<WT, NC, true>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);        \
    }
GEMV_K23_INST(q2_K, WT_Q2_K, 1) GEMV_K23_INST(q2_K, WT_Q2_K, 2) GEMV_K23_INST(q2_K, WT_Q2_K, 4)
GEMV_K23_INST(q3_K, WT_Q3_K, 1) GEMV_K23_INST(q3_K, WT_Q3_K, 2) GEMV_K23_INST(q3_K, WT_Q3_K, 4)

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

// 32-element blocks with Q8_0 activations: "_f" kernels take f32 activations
// (quantization fused), the others ready Q8_0 rows
#define GEMV_PAIR_INST(name, impl, NC)                                                             \
    extern "C" __global__ void __launch_bounds__(512) name##_c##NC(GEMV_ARGS) {                   \
        impl<NC, false, false>(GEMV_PASS);                                                         \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) name##_sub_c##NC(GEMV_ARGS) {               \
        impl<NC, true, false>(GEMV_PASS);                                                          \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) name##_f_c##NC(GEMV_ARGS) {                 \
        impl<NC, false, true>(GEMV_PASS);                                                          \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) name##_f_sub_c##NC(GEMV_ARGS) {             \
        impl<NC, true, true>(GEMV_PASS);                                                           \
    }
#define GEMV_PAIR_ALL(name, impl)                                                      \
    GEMV_PAIR_INST(name, impl, 1) GEMV_PAIR_INST(name, impl, 2) GEMV_PAIR_INST(name, impl, 4) \
        GEMV_PAIR_INST(name, impl, 8)
GEMV_PAIR_ALL(ghip_gemv_q4_0, gemv_q4_0_impl)
GEMV_PAIR_INST(ghip_gemv_q4_0_full, gemv_q4_0_full_impl, 1) GEMV_PAIR_INST(ghip_gemv_q4_0_full, gemv_q4_0_full_impl, 2)
GEMV_PAIR_ALL(ghip_gemv_q5_0, gemv_q5_0_impl)
GEMV_PAIR_ALL(ghip_gemv_q8_0, gemv_q8_0_impl)
// whole-group variant of the ready-Q8_0 Q5_0 kernel (no fused quantization;
// for Q8_0 it measured slower, 17.8 -> 20.1 us on 4096 -> 14336)
#define GEMV_PAIR_FULL_INST(name, impl, NC)                                                        \
    extern "C" __global__ void __launch_bounds__(512) name##_c##NC(GEMV_ARGS) {                   \
        impl<NC, false, false>(GEMV_PASS);                                                         \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) name##_sub_c##NC(GEMV_ARGS) {               \
        impl<NC, true, false>(GEMV_PASS);                                                          \
    }
GEMV_PAIR_FULL_INST(ghip_gemv_q5_0_full, gemv_q5_0_full_impl, 1) GEMV_PAIR_FULL_INST(ghip_gemv_q5_0_full, gemv_q5_0_full_impl, 2)

// Q4_K: "_f" kernels take f32 activations (fused Q8_K quantization), the
// others ready Q8_K rows; "_sub" kernels also store the integer partials.
#define Q4K_ARGS GEMV_ARGS, int n_mat
#define Q4K_PASS GEMV_PASS, n_mat
#define QK45_INST(TN, Q5, NC, RB, NG)                                                                             \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_c##NC##_r##RB##x##NG(Q4K_ARGS) {          \
        gemv_q4K_impl<NC, false, false, RB, NG, Q5>(Q4K_PASS);                                                  \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_sub_c##NC##_r##RB##x##NG(Q4K_ARGS) {      \
        gemv_q4K_impl<NC, true, false, RB, NG, Q5>(Q4K_PASS);                                                   \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_f_c##NC##_r##RB##x##NG(Q4K_ARGS) {        \
        gemv_q4K_impl<NC, false, true, RB, NG, Q5>(Q4K_PASS);                                                   \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_f_sub_c##NC##_r##RB##x##NG(Q4K_ARGS) {    \
        gemv_q4K_impl<NC, true, true, RB, NG, Q5>(Q4K_PASS);                                                    \
    }
#define Q4K_INST(NC, RB, NG) QK45_INST(q4_K, false, NC, RB, NG)
// NS register slots (row groups loaded before the activation is quantized)
#define Q4K_INST_S(NC, RB, NG, NS)                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_c##NC##_r##RB##x##NG##s##NS(Q4K_ARGS) {      \
        gemv_q4K_impl<NC, false, false, RB, NG, false, NS>(Q4K_PASS);                                           \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_sub_c##NC##_r##RB##x##NG##s##NS(Q4K_ARGS) {  \
        gemv_q4K_impl<NC, true, false, RB, NG, false, NS>(Q4K_PASS);                                            \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_f_c##NC##_r##RB##x##NG##s##NS(Q4K_ARGS) {    \
        gemv_q4K_impl<NC, false, true, RB, NG, false, NS>(Q4K_PASS);                                            \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q4_K_f_sub_c##NC##_r##RB##x##NG##s##NS(Q4K_ARGS) { \
        gemv_q4K_impl<NC, true, true, RB, NG, false, NS>(Q4K_PASS);                                             \
    }
Q4K_INST_S(1, 1, 4, 3) Q4K_INST_S(1, 1, 7, 3) Q4K_INST_S(1, 1, 8, 3)
Q4K_INST_S(2, 1, 4, 3) Q4K_INST_S(2, 1, 7, 3) Q4K_INST_S(2, 1, 8, 3) Q4K_INST(2, 1, 2)
Q4K_INST(4, 1, 2)
// register row groups (RB rows) x groups in flight (NG)
#define Q4K_INST_RB(NC) Q4K_INST(NC, 2, 2) Q4K_INST(NC, 2, 4) Q4K_INST(NC, 4, 2) Q4K_INST(NC, 2, 8) Q4K_INST(NC, 4, 4)
Q4K_INST_RB(1) Q4K_INST_RB(2) Q4K_INST_RB(4) Q4K_INST_RB(8)
Q4K_INST(1, 1, 4) Q4K_INST(1, 1, 8) Q4K_INST(1, 1, 2) Q4K_INST(1, 1, 0) Q4K_INST(1, 1, 7)
// Q5_K: the same shapes and naming as Q4_K
#define Q5K_INST_RB(NC) QK45_INST(q5_K, true, NC, 2, 2) QK45_INST(q5_K, true, NC, 2, 4) \
    QK45_INST(q5_K, true, NC, 4, 2) QK45_INST(q5_K, true, NC, 2, 8) QK45_INST(q5_K, true, NC, 4, 4)
Q5K_INST_RB(1) Q5K_INST_RB(2) Q5K_INST_RB(4) Q5K_INST_RB(8)
// Q5_K one-row groups with NS register slots (the Q4_K batch-1 shapes)
#define Q5K_INST_S(NC, NG, NS)                                                                                     \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q5_K_f_c##NC##_r1x##NG##s##NS(Q4K_ARGS) {         \
        gemv_q4K_impl<NC, false, true, 1, NG, true, NS>(Q4K_PASS);                                             \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q5_K_f_sub_c##NC##_r1x##NG##s##NS(Q4K_ARGS) {     \
        gemv_q4K_impl<NC, true, true, 1, NG, true, NS>(Q4K_PASS);                                              \
    }
Q5K_INST_S(1, 2, 2) Q5K_INST_S(1, 4, 3) Q5K_INST_S(1, 7, 3) Q5K_INST_S(1, 8, 3)

// Q6_K (v2): same shapes and naming, "_f" = fused Q8_K quantization
#define Q6K_INST(NC, RB, NG)                                                                                      \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q6_K_v2_c##NC##_r##RB##x##NG(Q4K_ARGS) {         \
        gemv_q6K_v2_impl<NC, false, false, RB, NG>(Q4K_PASS);                                                   \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q6_K_v2_sub_c##NC##_r##RB##x##NG(Q4K_ARGS) {     \
        gemv_q6K_v2_impl<NC, true, false, RB, NG>(Q4K_PASS);                                                    \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q6_K_v2_f_c##NC##_r##RB##x##NG(Q4K_ARGS) {       \
        gemv_q6K_v2_impl<NC, false, true, RB, NG>(Q4K_PASS);                                                    \
    }                                                                                                           \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_q6_K_v2_f_sub_c##NC##_r##RB##x##NG(Q4K_ARGS) {   \
        gemv_q6K_v2_impl<NC, true, true, RB, NG>(Q4K_PASS);                                                     \
    }
#define Q6K_INST_RB(NC) Q6K_INST(NC, 2, 2) Q6K_INST(NC, 2, 4) Q6K_INST(NC, 4, 2)
Q6K_INST_RB(1) Q6K_INST_RB(2) Q6K_INST_RB(4) Q6K_INST_RB(8)
Q6K_INST(1, 2, 8) Q6K_INST(1, 1, 4) Q6K_INST(1, 1, 8)

// Sibling MUL_MATs in one launch (ghip_graph_compute): up to four weight
// matrices of one type and K that read the same f32 activation rows, each
// quantized per workgroup exactly as in the one-matrix kernels; workgroups
// [wg0[i], wg0[i+1]) compute matrix i into dst[i] (row stride ldd[i]).
// Passed by value; the host mirror in ghip.cpp has the same layout.
struct GemvMulti {
    const uint8_t *W[4];
    float *dst[4];
    int64_t ldd[4];
    int rows[4];
    int wg0[4];
    int n;
};
#define GEMV_MULTI_RN(TN, NC, RB, NG, IMPL, ...)                                                                 \
    extern "C" __global__ void __launch_bounds__(512)                                                            \
        ghip_gemv_##TN##_f_c##NC##_r##RB##x##NG##_multi(GemvMulti g, int64_t w_row_bytes, int nb,               \
                                                        const uint8_t *__restrict__ act, int64_t act_row_bytes, \
                                                        int ncols, int n_mat) {                                  \
        const int bx = blockIdx.x;                                                                               \
        int i = 0;                                                                                               \
        _Pragma("unroll") for (int k = 1; k < 4; k++) if (k < g.n && bx >= g.wg0[k]) i = k;                     \
        IMPL<NC, false, true, RB, NG, ##__VA_ARGS__>(g.W[i], w_row_bytes, g.rows[i], nb, act, act_row_bytes,     \
                                                     ncols, g.dst[i], g.ldd[i], nullptr, n_mat, bx - g.wg0[i]);  \
    }
#define GEMV_MULTI(TN, NC, IMPL, ...) GEMV_MULTI_RN(TN, NC, 2, 2, IMPL, ##__VA_ARGS__)
GEMV_MULTI(q4_K, 1, gemv_q4K_impl, false) GEMV_MULTI(q4_K, 2, gemv_q4K_impl, false)
GEMV_MULTI(q4_K, 4, gemv_q4K_impl, false) GEMV_MULTI(q4_K, 8, gemv_q4K_impl, false)
GEMV_MULTI(q5_K, 1, gemv_q4K_impl, true) GEMV_MULTI(q5_K, 2, gemv_q4K_impl, true)
GEMV_MULTI(q5_K, 4, gemv_q4K_impl, true) GEMV_MULTI(q5_K, 8, gemv_q4K_impl, true)
GEMV_MULTI(q6_K_v2, 1, gemv_q6K_v2_impl)
// one-row groups streamed four (Q4_K) or eight (Q6_K) deep: the batch-1 shapes of large matrices
GEMV_MULTI_RN(q4_K, 1, 1, 4, gemv_q4K_impl, false)
GEMV_MULTI_RN(q4_K, 1, 1, 2, gemv_q4K_impl, false)
#define GEMV_MULTI_RNS(TN, NC, RB, NG, NS, IMPL)                                                                 \
    extern "C" __global__ void __launch_bounds__(512)                                                            \
        ghip_gemv_##TN##_f_c##NC##_r##RB##x##NG##s##NS##_multi(GemvMulti g, int64_t w_row_bytes, int nb,        \
                                                               const uint8_t *__restrict__ act,                  \
                                                               int64_t act_row_bytes, int ncols, int n_mat) {    \
        const int bx = blockIdx.x;                                                                               \
        int i = 0;                                                                                               \
        _Pragma("unroll") for (int k = 1; k < 4; k++) if (k < g.n && bx >= g.wg0[k]) i = k;                     \
        IMPL<NC, false, true, RB, NG, false, NS>(g.W[i], w_row_bytes, g.rows[i], nb, act, act_row_bytes, ncols,   \
                                                 g.dst[i], g.ldd[i], nullptr, n_mat, bx - g.wg0[i]);             \
    }
GEMV_MULTI_RNS(q4_K, 1, 1, 4, 3, gemv_q4K_impl) GEMV_MULTI_RNS(q4_K, 1, 1, 7, 3, gemv_q4K_impl)
GEMV_MULTI_RNS(q4_K, 1, 1, 8, 3, gemv_q4K_impl)
GEMV_MULTI_RN(q4_K, 2, 1, 2, gemv_q4K_impl, false) GEMV_MULTI_RN(q4_K, 4, 1, 2, gemv_q4K_impl, false) GEMV_MULTI_RNS(q4_K, 2, 1, 4, 3, gemv_q4K_impl)
GEMV_MULTI_RNS(q4_K, 2, 1, 7, 3, gemv_q4K_impl) GEMV_MULTI_RNS(q4_K, 2, 1, 8, 3, gemv_q4K_impl)
GEMV_MULTI_RN(q6_K_v2, 1, 1, 8, gemv_q6K_v2_impl)

// Q4_0 / Q5_0 / Q8_0 siblings: ready Q8_0 rows (one quantize launch for the
// group), 8 weight rows per workgroup
#define GEMV_PAIR_MULTI(TN, NC, IMPL)                                                                            \
    extern "C" __global__ void __launch_bounds__(512)                                                            \
        ghip_gemv_##TN##_c##NC##_multi(GemvMulti g, int64_t w_row_bytes, int nb, const uint8_t *__restrict__ act, \
                                       int64_t act_row_bytes, int ncols) {                                       \
        const int bx = blockIdx.x;                                                                               \
        int i = 0;                                                                                               \
        _Pragma("unroll") for (int k = 1; k < 4; k++) if (k < g.n && bx >= g.wg0[k]) i = k;                     \
        IMPL<NC, false, false>(g.W[i], w_row_bytes, g.rows[i], nb, act, act_row_bytes, ncols, g.dst[i], g.ldd[i], \
                               nullptr, bx - g.wg0[i]);                                                          \
    }
#define GEMV_PAIR_MULTI_ALL(TN, IMPL) \
    GEMV_PAIR_MULTI(TN, 1, IMPL) GEMV_PAIR_MULTI(TN, 2, IMPL) GEMV_PAIR_MULTI(TN, 4, IMPL) GEMV_PAIR_MULTI(TN, 8, IMPL)
GEMV_PAIR_MULTI_ALL(q4_0, gemv_q4_0_impl)
GEMV_PAIR_MULTI_ALL(q5_0, gemv_q5_0_impl)
GEMV_PAIR_MULTI_ALL(q8_0, gemv_q8_0_impl)

// ------------------------------------------------ MUL_MAT_ID, further types
// forward_mul_mat_id for experts other than MXFP4 / Q4_K / Q5_K / Q6_K: every
// (token, slot) pair runs the decode kernel of its expert on its ready Q8
// activation row (the reference's row vec_dot, or the Q4_0 8x8 gemv for
// rows % 8 == 0 experts, compute.rs:2012-2024, 2166-2174), grid (row blocks,
// pairs).
#define MMID_GEMV(TN, CALL_FALSE, CALL_TRUE)                                                                        \
    extern "C" __global__ void __launch_bounds__(512) ghip_mmid_gemv_##TN(MMID_ARGS) {                              \
        MMID_PAIR(q) CALL_FALSE(q.W, as_nb1, rows, nb, q.act, act_rb, 1, q.dst, 0, nullptr);                       \
    }                                                                                                               \
    extern "C" __global__ void __launch_bounds__(512) ghip_mmid_gemv_##TN##_sub(MMID_ARGS) {                        \
        MMID_PAIR(q) CALL_TRUE(q.W, as_nb1, rows, nb, q.act, act_rb, 1, q.dst, 0, q.sub);                          \
    }
MMID_GEMV(q4_0, (gemv_q4_0_impl<1, false, false>), (gemv_q4_0_impl<1, true, false>))
MMID_GEMV(q5_0, (gemv_q5_0_impl<1, false, false>), (gemv_q5_0_impl<1, true, false>))
MMID_GEMV(q8_0, (gemv_q8_0_impl<1, false, false>), (gemv_q8_0_impl<1, true, false>))
MMID_GEMV(q4_1, (gemv_q41_impl<WT_Q4_1, 1, false>), (gemv_q41_impl<WT_Q4_1, 1, true>))
MMID_GEMV(q5_1, (gemv_q41_impl<WT_Q5_1, 1, false>), (gemv_q41_impl<WT_Q5_1, 1, true>))
MMID_GEMV(q2_K, (gemv_k23_impl<WT_Q2_K, 1, false>), (gemv_k23_impl<WT_Q2_K, 1, true>))
MMID_GEMV(q3_K, (gemv_k23_impl<WT_Q3_K, 1, false>), (gemv_k23_impl<WT_Q3_K, 1, true>))
