// ghip_iq.hip -- MUL_MAT for the lookup-table 4-bit weight types:
//   IQ4_NL  18 B / 32  {f16 d; u8 qs[16]}                 x Q8_0 (vec_dot.rs:1597)
//   IQ4_XS  136 B / 256 {f16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128]} x Q8_K (vec_dot.rs:1655)
//   NVFP4   36 B / 64  {u8 d[4] (UE4M3 per 16); u8 qs[32]} x Q8_0 (vec_dot.rs:1154)
// and the 1- and 2-bit codes of the same family of kernels:
//   Q1_0    18 B / 128 {f16 d; u8 qs[16]} sign bits, +-d   x Q8_0 (vec_dot.rs:1074)
//   Q2_0    18 B / 64  {f16 d; u8 qs[16]} (q - 1) * d      x Q8_0 (vec_dot.rs:1120)
// (block layouts blocks.rs:14-28, :55-62, :234-249).  A nibble is an index into a
// 16-entry int8 table: KVALUES_IQ4NL (quants_k.rs:647) or the E2M1 values
// doubled, KVALUES_MXFP4 (quants.rs:660).
//
// Decode (1..8 activation rows): one lane per 32 weight elements, which is
// one Q8_0 activation block (IQ4_NL, NVFP4) or one 32-group of a Q8_K block
// (IQ4_XS); RB weight rows per workgroup, all of a lane's loads issued
// before any is consumed.  Per lane and row the integer dot of the 32
// elements is exact (v_dot4_i32_i8 on the looked-up int8 values) and scaled
// once: IQ4_NL d_w * d_a, NVFP4 ue4m3(d_s) * d_a per 16-element sub-block,
// IQ4_XS d_w * d8 * (ls - 32).  Rows are reduced over the wavefront and the
// workgroup as in the other decode kernels.
//
// Prefill: IQ4_NL and IQ4_XS weights become int8 codes (the table values)
// with one f32 scale per 32 elements (IQ4_NL: d; IQ4_XS: the integer ls - 32,
// with d per super-block beside it), the operands of the int8-MFMA GEMM of
// ghip_gemm.hip; IQ4_XS activations are Q8_K rows written in that GEMM's
// layout (ghip_gemm_act_q8K_q8).
#include "ghip_common.h"
#define GHIP_GRID_QUAL static __device__ const
#include "ghip_iq_grids.h"
#include "ghip_q8k.h"

namespace {

constexpr int RB = 8;  // weight rows per decode workgroup
constexpr int WT_IQ4_NL = 20, WT_IQ4_XS = 23, WT_NVFP4 = 40, WT_Q1_0 = 41, WT_Q2_0 = 42;

// 16-entry int8 tables as four little-endian dwords (entries 4i .. 4i+3 in T[i])
struct Lut {
    uint32_t t0, t1, t2, t3;
};
// KVALUES_IQ4NL: -127 -104 -83 -65 | -49 -35 -22 -10 | 1 13 25 38 | 53 69 89 113
constexpr Lut kIq4nl = {0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u};
// KVALUES_MXFP4: 0 1 2 3 | 4 6 8 12 | 0 -1 -2 -3 | -4 -6 -8 -12
constexpr Lut kMxfp4 = {0x03020100u, 0x0C080604u, 0xFDFEFF00u, 0xF4F8FAFCu};

// Table values of four nibbles, one in bits 0-3 of each byte of x (higher bits
// of a byte are ignored): v_perm_b32 picks from entries 0-7 and 8-15 by the
// low three bits, and a third v_perm_b32 picks, per byte, the half that bit 3
// names.
DEV uint32_t lut4(const Lut &L, uint32_t x) {
    const uint32_t idx = x & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(L.t1, L.t0, idx);
    const uint32_t hi = __builtin_amdgcn_perm(L.t3, L.t2, idx);
    const uint32_t sel = 0x03020100u | ((x >> 1) & 0x04040404u);  // byte i: i, or 4 + i where bit 3 is set
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// ue4m3_to_fp32 (quants.rs:699-712): exp 0 -> man * 2^-10, 0x7F -> 0, else
// (8 + man) * 2^(exp - 11) (the halving included); built from bits, exact
DEV float ue4m3(uint32_t x) {
    x &= 0xffu;
    const uint32_t e = (x >> 3) & 15u, m = x & 7u;
    if (x == 0x7Fu) return 0.0f;
    if (e == 0) return (float)m * 0x1p-10f;
    return __uint_as_float(((e + 119u) << 23) | (m << 20));
}

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

// nb: weight blocks per row (K / 32, K / 256, K / 64 or K / 128).  Sub-sums
// (the ghip_mul_mat_subsums layout): IQ4_NL, Q1_0 and Q2_0 the exact dot per
// 32-element group (one Q8_0 block); NVFP4 per 16-element sub-block (4 per
// block); IQ4_XS sum (ls - 32) * dot per super-block.
template <int WT, int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_lut_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb,
                                              const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols,
                                              float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    // 32-element groups per row
    const int ng = WT == WT_IQ4_NL ? nb : WT == WT_NVFP4 || WT == WT_Q2_0 ? 2 * nb : WT == WT_Q1_0 ? 4 * nb : 8 * nb;
    constexpr bool BITS = WT == WT_Q1_0 || WT == WT_Q2_0;  // 1- and 2-bit codes, no table
    const int g = 64 * w + lane;
    const bool valid = g < ng;
    const int gc = valid ? g : ng - 1;  // loads of invalid lanes re-read a valid group
    const int r0 = (int)blockIdx.x * RB;
    const int nr = min(RB, rows - r0);
    const Lut L = WT == WT_NVFP4 ? kMxfp4 : kIq4nl;

    // this lane's weight bytes: the 16 qs bytes of its 32 elements and the
    // scale word (IQ4_NL: d; NVFP4: the two UE4M3 bytes; IQ4_XS: d, scales_h,
    // scales_l)
    uint32_t boff, qoff;
    if (WT == WT_IQ4_NL) {
        boff = (uint32_t)gc * 18u;
        qoff = boff + 2u;
    } else if (WT == WT_NVFP4) {
        boff = (uint32_t)(gc >> 1) * 36u + 2u * (uint32_t)(gc & 1);
        qoff = (uint32_t)(gc >> 1) * 36u + 4u + 16u * (uint32_t)(gc & 1);
    } else if (WT == WT_Q1_0) {  // 4 bytes of sign bits per group
        boff = (uint32_t)(gc >> 2) * 18u;
        qoff = boff + 2u + 4u * (uint32_t)(gc & 3);
    } else if (WT == WT_Q2_0) {  // 8 bytes of 2-bit codes per group
        boff = (uint32_t)(gc >> 1) * 18u;
        qoff = boff + 2u + 8u * (uint32_t)(gc & 1);
    } else {
        boff = (uint32_t)(gc >> 3) * 136u;
        qoff = boff + 8u + 16u * (uint32_t)(gc & 7);
    }
    uint4 qv[RB];
    uint2 hv[RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint8_t *p = W + (int64_t)min(r0 + rr, rows - 1) * w_row_bytes;
        // (exact-size loads: a group's bytes may end the matrix)
        if (WT == WT_Q1_0) qv[rr] = make_uint4(ld4(p + qoff), 0u, 0u, 0u);
        else if (WT == WT_Q2_0) {
            const uint2 t = ld8(p + qoff);
            qv[rr] = make_uint4(t.x, t.y, 0u, 0u);
        } else qv[rr] = ld16(p + qoff);
        if (WT == WT_IQ4_XS) hv[rr] = ld8(p + boff);
        else hv[rr] = make_uint2(ld2(p + boff), 0u);
    }
    // activations: the 32 codes and the scale of this lane's block or group
    uint4 ya[NC], yb[NC];
    float dy[NC];
    int ysum[NC];  // Q1_0 / Q2_0: sum of the block's 32 codes
#pragma unroll
    for (int c = 0; c < NC; c++) {
        ya[c] = yb[c] = make_uint4(0, 0, 0, 0);
        dy[c] = 0.0f;
        if (c < ncols && valid) {
            if (WT == WT_IQ4_XS) {
                const uint8_t *A = act + c * act_row_bytes + (int64_t)(g >> 3) * Q8K_BYTES;
                dy[c] = __uint_as_float(ld4(A));
                ya[c] = ld16(A + 4 + 32 * (g & 7));
                yb[c] = ld16(A + 20 + 32 * (g & 7));
            } else {
                const uint8_t *A = act + c * act_row_bytes + (int64_t)g * Q8_0_BYTES;
                dy[c] = h2f(ld2(A));
                ya[c] = ld16(A + 2);
                yb[c] = ld16(A + 18);
            }
        }
        ysum[c] = 0;
        if (BITS) {
            const uint32_t y[8] = {ya[c].x, ya[c].y, ya[c].z, ya[c].w, yb[c].x, yb[c].y, yb[c].z, yb[c].w};
#pragma unroll
            for (int k = 0; k < 8; k++) ysum[c] = dot4(y[k], 0x01010101u, ysum[c]);
        }
    }
    float part[NC][RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint32_t q[4] = {qv[rr].x, qv[rr].y, qv[rr].z, qv[rr].w};
        // v[i]: table values of elements 4i .. 4i+3 of the lane's 32
        uint32_t v[8];
        if (WT == WT_Q1_0) {
            // bit e of the group's dword is element e: bits 4k..4k+3 spread to
            // the four bytes as 0 / 1 (the value is 2 * bit - 1)
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = __umul24((q[0] >> (4 * k)) & 0xFu, 0x00204081u) & 0x01010101u;
        } else if (WT == WT_Q2_0) {
            // byte j holds elements 4j..4j+3 as 2-bit fields (the value is
            // field - 1); the copies are ORed, not added, so nothing carries
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t B = (q[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                const uint32_t u = B | (B << 6);
                v[j] = (u | (u << 12)) & 0x03030303u;
            }
        } else if (WT == WT_NVFP4) {
            // sub-block 2h: qs bytes 0..7, low nibbles elements 0..7, high 8..15;
            // sub-block 2h+1: bytes 8..15 -> elements 16..23 and 24..31
            v[0] = lut4(L, q[0]);
            v[1] = lut4(L, q[1]);
            v[2] = lut4(L, q[0] >> 4);
            v[3] = lut4(L, q[1] >> 4);
            v[4] = lut4(L, q[2]);
            v[5] = lut4(L, q[3]);
            v[6] = lut4(L, q[2] >> 4);
            v[7] = lut4(L, q[3] >> 4);
        } else {
            // low nibbles of qs[0..15] are elements 0..15, high nibbles 16..31
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v[k] = lut4(L, q[k]);
                v[4 + k] = lut4(L, q[k] >> 4);
            }
        }
        const uint32_t hw = hv[rr].x;
        int ls = 0;
        if (WT == WT_IQ4_XS) {
            // 6-bit scale of group ib: nibble ib of scales_l, bits 2ib.. of scales_h
            const int ib = g & 7;
            const uint32_t sl = (hv[rr].y >> (4 * ib)) & 0xFu;
            const uint32_t sh = ((hw >> 16) >> (2 * ib)) & 3u;
            ls = (int)(sl | (sh << 4)) - 32;
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint32_t y[8] = {ya[c].x, ya[c].y, ya[c].z, ya[c].w, yb[c].x, yb[c].y, yb[c].z, yb[c].w};
            float pp = 0.0f;
            if (WT == WT_NVFP4) {
                const int s0 = dot4(v[3], y[3], dot4(v[2], y[2], dot4(v[1], y[1], dot4(v[0], y[0], 0))));
                const int s1 = dot4(v[7], y[7], dot4(v[6], y[6], dot4(v[5], y[5], dot4(v[4], y[4], 0))));
                if (SUBSUMS && valid && c < ncols && rr < nr) {
                    int32_t *sp = sub + ((int64_t)c * rows + r0 + rr) * (int64_t)(4 * nb) + 2 * g;
                    sp[0] = s0;
                    sp[1] = s1;
                }
                pp = (ue4m3(hw) * dy[c]) * (float)s0 + (ue4m3(hw >> 8) * dy[c]) * (float)s1;
            } else {
                int s = 0;
#pragma unroll
                for (int k = 0; k < 8; k++) s = dot4(v[k], y[k], s);
                if (WT == WT_Q1_0) s = 2 * s - ysum[c];
                if (WT == WT_Q2_0) s -= ysum[c];
                if (WT != WT_IQ4_XS) {
                    if (SUBSUMS && valid && c < ncols && rr < nr) sub[((int64_t)c * rows + r0 + rr) * ng + g] = s;
                    pp = (h2f(hw) * dy[c]) * (float)s;
                } else {
                    // the super-block's exact sum (its 8 groups sit in 8
                    // consecutive lanes), scaled once by d * d8 as the
                    // reference scales each super-block (vec_dot.rs:1665-1696)
                    int t = ls * s;  // |.| <= 32 * 32 * 127 * 128
                    t += __shfl_xor(t, 1, 64);
                    t += __shfl_xor(t, 2, 64);
                    t += __shfl_xor(t, 4, 64);
                    if (SUBSUMS && (g & 7) == 0 && valid && c < ncols && rr < nr)
                        sub[((int64_t)c * rows + r0 + rr) * nb + (g >> 3)] = t;
                    pp = (g & 7) == 0 ? (h2f(hw) * dy[c]) * (float)t : 0.0f;
                }
            }
            part[c][rr] = valid ? pp : 0.0f;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, nr, ncols, NC, nw, dst, ldd);
}

// weights -> int8 codes [Npad][Kpad] and one f32 scale per 32 elements at
// dw[b][row], zero past N and K (the operands of ghip_gemm_q8); one thread per
// (row, 32-group)
// IQ4_XS: dw holds the group's integer scale ls - 32 and dsb[super-block][row]
// the block's d (the XS mode of the GEMM sums the groups per super-block)
template <int WT>
__device__ __forceinline__ void q8w_repack_lut(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb, int Kpad,
                                               int Npad, int8_t *__restrict__ codes, float *__restrict__ dw,
                                               float *__restrict__ dsb = nullptr) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int nbp = Kpad / 32;
    if (i >= (int64_t)Npad * nbp) return;
    const int row = (int)(i / nbp), g = (int)(i % nbp);
    const int ng = WT == WT_IQ4_NL ? nb : WT == WT_Q1_0 ? 4 * nb : WT == WT_Q2_0 ? 2 * nb : 8 * nb;
    uint32_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float d = 0.0f;
    if (row < N && g < ng && (WT == WT_Q1_0 || WT == WT_Q2_0)) {
        // sign bits -> +-1, 2-bit fields -> field - 1, as int8
        const uint8_t *r = W + (int64_t)row * row_bytes;
        const int per = WT == WT_Q1_0 ? 4 : 2;
        const uint8_t *blk = r + (int64_t)(g / per) * 18;
        d = h2f(ld2(blk));
        const uint8_t *q = blk + 2 + (WT == WT_Q1_0 ? 4 : 8) * (g % per);
#pragma unroll
        for (int e = 0; e < 32; e++) {
            const int val = WT == WT_Q1_0 ? (((q[e >> 3] >> (e & 7)) & 1) ? 1 : -1) : (int)((q[e >> 2] >> (2 * (e & 3))) & 3) - 1;
            v[e >> 2] |= (uint32_t)(val & 0xff) << (8 * (e & 3));
        }
    } else if (row < N && g < ng) {
        const uint8_t *r = W + (int64_t)row * row_bytes;
        const uint8_t *qs;
        if (WT == WT_IQ4_NL) {
            d = h2f(ld2(r + (int64_t)g * 18));
            qs = r + (int64_t)g * 18 + 2;
        } else {
            const uint8_t *blk = r + (int64_t)(g >> 3) * 136;
            const int ib = g & 7;
            const uint32_t sh = ((uint32_t)ld2(blk + 2) >> (2 * ib)) & 3u;
            const uint32_t sl = ((uint32_t)blk[4 + ib / 2] >> (4 * (ib % 2))) & 0xFu;
            d = (float)((int)(sl | (sh << 4)) - 32);
            if (ib == 0) dsb[(int64_t)(g >> 3) * Npad + row] = h2f(ld2(blk));
            qs = blk + 8 + 16 * ib;
        }
        const uint4 q = ld16(qs);
        const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = lut4(kIq4nl, qq[k]);
            v[4 + k] = lut4(kIq4nl, qq[k] >> 4);
        }
    }
    int8_t *o = codes + q8w_piece(row, g, Kpad);
    *reinterpret_cast<uint4 *>(o) = make_uint4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<uint4 *>(o + 512) = make_uint4(v[4], v[5], v[6], v[7]);
    dw[(int64_t)g * Npad + row] = d;
}

}  // namespace

#define GEMV_LUT_INST(TN, WT, NC)                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_c##NC(                                    \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_lut_impl<WT, NC, false>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);       \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_sub_c##NC(                                \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_lut_impl<WT, NC, true>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);        \
    }
GEMV_LUT_INST(iq4_nl, WT_IQ4_NL, 1) GEMV_LUT_INST(iq4_nl, WT_IQ4_NL, 2) GEMV_LUT_INST(iq4_nl, WT_IQ4_NL, 4)
GEMV_LUT_INST(iq4_nl, WT_IQ4_NL, 8)
GEMV_LUT_INST(nvfp4, WT_NVFP4, 1) GEMV_LUT_INST(nvfp4, WT_NVFP4, 2) GEMV_LUT_INST(nvfp4, WT_NVFP4, 4)
GEMV_LUT_INST(nvfp4, WT_NVFP4, 8)
GEMV_LUT_INST(iq4_xs, WT_IQ4_XS, 1) GEMV_LUT_INST(iq4_xs, WT_IQ4_XS, 2) GEMV_LUT_INST(iq4_xs, WT_IQ4_XS, 4)
GEMV_LUT_INST(iq4_xs, WT_IQ4_XS, 8)
GEMV_LUT_INST(q1_0, WT_Q1_0, 1) GEMV_LUT_INST(q1_0, WT_Q1_0, 2) GEMV_LUT_INST(q1_0, WT_Q1_0, 4)
GEMV_LUT_INST(q1_0, WT_Q1_0, 8)
GEMV_LUT_INST(q2_0, WT_Q2_0, 1) GEMV_LUT_INST(q2_0, WT_Q2_0, 2) GEMV_LUT_INST(q2_0, WT_Q2_0, 4)
GEMV_LUT_INST(q2_0, WT_Q2_0, 8)

extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8w_repack_iq4_nl(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb, int Kpad, int Npad,
                                int8_t *__restrict__ codes, float *__restrict__ dw) {
    q8w_repack_lut<WT_IQ4_NL>(W, row_bytes, N, nb, Kpad, Npad, codes, dw);
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8w_repack_q1_0(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb, int Kpad, int Npad,
                              int8_t *__restrict__ codes, float *__restrict__ dw) {
    q8w_repack_lut<WT_Q1_0>(W, row_bytes, N, nb, Kpad, Npad, codes, dw);
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8w_repack_q2_0(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb, int Kpad, int Npad,
                              int8_t *__restrict__ codes, float *__restrict__ dw) {
    q8w_repack_lut<WT_Q2_0>(W, row_bytes, N, nb, Kpad, Npad, codes, dw);
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8w_repack_iq4_xs(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb, int Kpad, int Npad,
                                int8_t *__restrict__ codes, float *__restrict__ dw, float *__restrict__ dsb) {
    q8w_repack_lut<WT_IQ4_XS>(W, row_bytes, N, nb, Kpad, Npad, codes, dw, dsb);
}

// f32 rows -> Q8_K (quantize_row_q8_K_ref, quants.rs:615-650, the arithmetic of
// ghip_quantize_q8_K) in the int8 GEMM's layout: codes [Mpad][Kpad] and the
// block scale d repeated for each of the super-block's 8 groups at
// da[g][row]; one wavefront per (row, super-block), padding rows zero
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_act_q8K_q8(const float *__restrict__ x, int64_t x_stride, int M, int Mpad, int nb, int Kpad,
                         int8_t *__restrict__ codes, float *__restrict__ da) {
    const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (task >= (int64_t)Mpad * nb) return;  // whole wavefronts
    const int row = (int)(task / nb), b = (int)(task % nb);
    float xs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row < M) __builtin_memcpy(xs, x + (int64_t)row * x_stride + (int64_t)b * QK_K + 4 * lane, 16);
    int q[4];
    float d;
    q8K_block(xs, lane, false, q, d);
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    *reinterpret_cast<uint32_t *>(codes + (int64_t)row * Kpad + (int64_t)b * QK_K + 4 * lane) = packed;
    if (lane < 8) da[(int64_t)(8 * b + lane) * Mpad + row] = d;
}

// MUL_MAT_ID with these experts: the decode kernel per (token, slot) pair
// (MMID_PAIR in ghip_common.h), grid (row blocks, pairs)
#define MMID_LUT(TN, WT)                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) ghip_mmid_gemv_##TN(MMID_ARGS) {                              \
        MMID_PAIR(q) gemv_lut_impl<WT, 1, false>(q.W, as_nb1, rows, nb, q.act, act_rb, 1, q.dst, 0, nullptr);      \
    }                                                                                                               \
    extern "C" __global__ void __launch_bounds__(512) ghip_mmid_gemv_##TN##_sub(MMID_ARGS) {                        \
        MMID_PAIR(q) gemv_lut_impl<WT, 1, true>(q.W, as_nb1, rows, nb, q.act, act_rb, 1, q.dst, 0, q.sub);         \
    }
MMID_LUT(iq4_nl, WT_IQ4_NL)
MMID_LUT(iq4_xs, WT_IQ4_XS)
MMID_LUT(nvfp4, WT_NVFP4)
MMID_LUT(q1_0, WT_Q1_0)
MMID_LUT(q2_0, WT_Q2_0)

// ------------------------------------------------ IQ1 / IQ2 / IQ3 weights
// vec_dot.rs:1215-1590 (the reference's tiled kernel, tiled.rs:440-640, forms
// the same integers).  One lane per 32-element block, its super-block's 8
// blocks in 8 consecutive lanes.  The lane decodes its 32 weights from the
// codebook (ghip_iq_grids.h) into signed int8 -- magnitudes from the grid
// entry, signs from 7 stored bits and their parity (IQ2_XXS, IQ2_XS, IQ3_XXS)
// or stored sign bytes (IQ2_S, IQ3_S), IQ1 values -1 / 0 / 1 -- and forms
//   t = sum over its 8-element groups k of sc_k * (F * dot_k + delta_k * sum_k q8)
// (sc_k: the block's or 16-element half's odd scale; F = 8 and delta_k = +-1 for
// the IQ1 types, else F = 1, delta 0), the exact integer the reference's lanes
// sum.  The super-block's 8 lanes add their t exactly; that integer is
// scaled once by d * f (f = 1/8 for IQ2 / IQ1, 1/4 for IQ3_XXS, 1 for IQ3_S)
// and the block scale d8 of the activation row.  Sub-sums: that integer per
// super-block.
constexpr int WT_IQ2_XXS = 16, WT_IQ2_XS = 17, WT_IQ3_XXS = 18, WT_IQ1_S = 19, WT_IQ3_S = 21, WT_IQ2_S = 22,
              WT_IQ1_M = 29;
template <int WT> constexpr int grid_block_bytes() {
    return WT == WT_IQ2_XXS ? 66 : WT == WT_IQ2_XS ? 74 : WT == WT_IQ2_S ? 82 : WT == WT_IQ3_XXS ? 98
           : WT == WT_IQ3_S ? 110 : WT == WT_IQ1_S ? 50 : 56;
}
template <int WT> constexpr float grid_scale() { return WT == WT_IQ3_XXS ? 0.25f : WT == WT_IQ3_S ? 1.0f : 0.125f; }
// 8 grid magnitudes (bytes) with the sign bits s8 (bit i: byte i negative)
DEV uint2 signed8(uint64_t gv, uint32_t s8) {
    const uint32_t lo = (uint32_t)gv, hi = (uint32_t)(gv >> 32);
    const uint32_t mlo = ((s8 & 0xFu) * 0x00204081u) & 0x01010101u, mhi = (((s8 >> 4) & 0xFu) * 0x00204081u) & 0x01010101u;
    // -g per marked byte: (g ^ 0xFF) + 1, no carry out of a byte since g >= 1
    return make_uint2((lo ^ (mlo * 0xFFu)) + mlo, (hi ^ (mhi * 0xFFu)) + mhi);
}
DEV uint32_t signed4(uint32_t gv, uint32_t s4) {
    const uint32_t m = ((s4 & 0xFu) * 0x00204081u) & 0x01010101u;
    return (gv ^ (m * 0xFFu)) + m;
}
DEV uint32_t parity7(uint32_t s7) { return s7 | ((__popc(s7) & 1u) << 7); }

// block ib of the super-block at blk: its 32 signed values v[0..7] (elements
// 4i..4i+3 in v[i]), the scales of its halves and the IQ1 deltas of its 8-element groups
template <int WT>
DEV void grid_block(const uint8_t *__restrict__ blk, int ib, uint32_t v[8], int &sc0, int &sc1, int dl[4]) {
    dl[0] = dl[1] = dl[2] = dl[3] = 0;
    if constexpr (WT == WT_IQ2_XXS) {
        const uint2 a = ld8(blk + 2 + 8 * ib);  // 4 index bytes | signs word (ls in its top 4 bits)
        sc0 = sc1 = 2 * (int)(a.y >> 28) + 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint2 t = signed8(ghip_iq2xxs_grid[(a.x >> (8 * k)) & 0xFF], parity7((a.y >> (7 * k)) & 127));
            v[2 * k] = t.x;
            v[2 * k + 1] = t.y;
        }
    } else if constexpr (WT == WT_IQ2_XS) {
        const uint2 a = ld8(blk + 2 + 8 * ib);  // 4 u16: 9-bit index, 7 sign bits
        const uint32_t sc = blk[66 + ib];
        sc0 = 2 * (int)(sc & 15) + 1;
        sc1 = 2 * (int)(sc >> 4) + 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q2 = ((k < 2 ? a.x : a.y) >> (16 * (k & 1))) & 0xFFFF;
            const uint2 t = signed8(ghip_iq2xs_grid[q2 & 511], parity7(q2 >> 9));
            v[2 * k] = t.x;
            v[2 * k + 1] = t.y;
        }
    } else if constexpr (WT == WT_IQ2_S) {
        const uint32_t idx = ld4(blk + 2 + 4 * ib), sg = ld4(blk + 34 + 4 * ib);
        const uint32_t qh = blk[66 + ib], sc = blk[74 + ib];
        sc0 = 2 * (int)(sc & 15) + 1;
        sc1 = 2 * (int)(sc >> 4) + 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t i = ((idx >> (8 * k)) & 0xFF) | ((qh << (8 - 2 * k)) & 0x300);
            const uint2 t = signed8(ghip_iq2s_grid[i], (sg >> (8 * k)) & 0xFF);
            v[2 * k] = t.x;
            v[2 * k + 1] = t.y;
        }
    } else if constexpr (WT == WT_IQ3_XXS) {
        const uint2 a = ld8(blk + 2 + 8 * ib);    // 8 index bytes (4 values each)
        const uint32_t sw = ld4(blk + 66 + 4 * ib);  // signs word, ls in its top 4 bits
        sc0 = sc1 = 2 * (int)(sw >> 28) + 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t s8 = parity7((sw >> (7 * k)) & 127);
            const uint32_t w = k < 2 ? a.x : a.y;
            v[2 * k] = signed4(ghip_iq3xxs_grid[(w >> (16 * (k & 1))) & 0xFF], s8);
            v[2 * k + 1] = signed4(ghip_iq3xxs_grid[(w >> (16 * (k & 1) + 8)) & 0xFF], s8 >> 4);
        }
    } else if constexpr (WT == WT_IQ3_S) {
        const uint2 a = ld8(blk + 2 + 8 * ib);  // 8 index bytes
        const uint32_t qh = blk[66 + ib], sg = ld4(blk + 74 + 4 * ib);
        const uint32_t sc = (blk[106 + (ib >> 1)] >> (4 * (ib & 1))) & 15;
        sc0 = sc1 = 2 * (int)sc + 1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t i = (((k < 4 ? a.x : a.y) >> (8 * (k & 3))) & 0xFF) | ((qh << (8 - k)) & 256);
            v[k] = signed4(ghip_iq3s_grid[i], (sg >> (4 * k)) & 0xF);
        }
    } else if constexpr (WT == WT_IQ1_S) {
        const uint32_t idx = ld4(blk + 2 + 4 * ib), qhw = ld2(blk + 34 + 2 * ib);
        sc0 = sc1 = 2 * (int)((qhw >> 12) & 7) + 1;
        const int d = qhw & 0x8000 ? -1 : 1;
        dl[0] = dl[1] = dl[2] = dl[3] = d;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint64_t gv = ghip_iq1s_grid[((idx >> (8 * k)) & 0xFF) | (((qhw >> (3 * k)) & 7) << 8)];
            v[2 * k] = (uint32_t)gv;
            v[2 * k + 1] = (uint32_t)(gv >> 32);
        }
    } else {  // IQ1_M
        const uint32_t idx = ld4(blk + 4 * ib), qh2 = ld2(blk + 32 + 2 * ib);
        const uint32_t sct = ld2(blk + 48 + 2 * (ib >> 1)), j = ib & 1;
        sc0 = 2 * (int)((sct >> (6 * j)) & 7) + 1;
        sc1 = 2 * (int)((sct >> (6 * j + 3)) & 7) + 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t qhb = (qh2 >> (8 * (k >> 1))) & 0xFF;
            const uint32_t i = ((idx >> (8 * k)) & 0xFF) | ((qhb << (8 - 4 * (k & 1))) & 0x700);
            const uint64_t gv = ghip_iq1s_grid[i];
            v[2 * k] = (uint32_t)gv;
            v[2 * k + 1] = (uint32_t)(gv >> 32);
            dl[k] = qhb & (k & 1 ? 0x80 : 0x08) ? -1 : 1;
        }
    }
}
// the super-block's weight scale d (f16; IQ1_M: assembled from the top
// nibbles of its four scale words)
template <int WT> DEV float grid_d(const uint8_t *__restrict__ blk) {
    if constexpr (WT == WT_IQ1_M) {
        const uint2 s = ld8(blk + 48);
        const uint32_t s0 = s.x & 0xFFFF, s1 = s.x >> 16, s2 = s.y & 0xFFFF, s3 = s.y >> 16;
        return h2f((s0 >> 12) | ((s1 >> 8) & 0x00f0) | ((s2 >> 4) & 0x0f00) | (s3 & 0xf000));
    } else {
        return h2f(ld2(blk));
    }
}

template <int WT, int NC, bool SUBSUMS>
__device__ __forceinline__ void gemv_grid_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb,
                                               const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols,
                                               float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    constexpr int BS = grid_block_bytes<WT>();
    constexpr bool IQ1 = WT == WT_IQ1_S || WT == WT_IQ1_M;
    __shared__ float red[RB * 8 * NC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int ng = 8 * nb;
    const int g = 64 * w + lane;
    const bool valid = g < ng;
    const int gc = valid ? g : ng - 1;
    const int ib = gc & 7;
    const int r0 = (int)blockIdx.x * RB;
    const int nr = min(RB, rows - r0);
    // activations: this block's 32 codes, the per-8 sums (IQ1) and d8
    uint4 ya[NC], yb[NC];
    float dy[NC];
    int ys[NC][4];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        ya[c] = yb[c] = make_uint4(0, 0, 0, 0);
        dy[c] = 0.0f;
        if (c < ncols && valid) {
            const uint8_t *A = act + c * act_row_bytes + (int64_t)(g >> 3) * Q8K_BYTES;
            dy[c] = __uint_as_float(ld4(A));
            ya[c] = ld16(A + 4 + 32 * ib);
            yb[c] = ld16(A + 20 + 32 * ib);
        }
        const uint32_t y[8] = {ya[c].x, ya[c].y, ya[c].z, ya[c].w, yb[c].x, yb[c].y, yb[c].z, yb[c].w};
#pragma unroll
        for (int k = 0; k < 4; k++) ys[c][k] = IQ1 ? dot4(y[2 * k + 1], 0x01010101u, dot4(y[2 * k], 0x01010101u, 0)) : 0;
    }
    float part[NC][RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const uint8_t *blk = W + (int64_t)min(r0 + rr, rows - 1) * w_row_bytes + (int64_t)(gc >> 3) * BS;
        uint32_t v[8];
        int sc0, sc1, dl[4];
        grid_block<WT>(blk, ib, v, sc0, sc1, dl);
        const float td = grid_d<WT>(blk) * grid_scale<WT>();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint32_t y[8] = {ya[c].x, ya[c].y, ya[c].z, ya[c].w, yb[c].x, yb[c].y, yb[c].z, yb[c].w};
            int t = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int s = dot4(v[2 * k + 1], y[2 * k + 1], dot4(v[2 * k], y[2 * k], 0));
                if (IQ1) s = 8 * s + dl[k] * ys[c][k];
                t += (k < 2 ? sc0 : sc1) * s;
            }
            // the super-block's exact integer (its 8 blocks in 8 consecutive lanes)
            t += __shfl_xor(t, 1, 64);
            t += __shfl_xor(t, 2, 64);
            t += __shfl_xor(t, 4, 64);
            if (SUBSUMS && ib == 0 && valid && c < ncols && rr < nr)
                sub[((int64_t)c * rows + r0 + rr) * nb + (g >> 3)] = t;
            part[c][rr] = valid && ib == 0 ? (td * (float)t) * dy[c] : 0.0f;
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) stash_rows(red, part[c], lane, w, nw, c, NC);
    finish_rows(red, r0, nr, ncols, NC, nw, dst, ldd);
}

#define GEMV_GRID_INST(TN, WT, NC)                                                                              \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_c##NC(                                    \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_grid_impl<WT, NC, false>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);       \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) ghip_gemv_##TN##_sub_c##NC(                                \
        const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,   \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {     \
        gemv_grid_impl<WT, NC, true>(W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub);        \
    }
#define GEMV_GRID_TYPE(TN, WT)                                                                                   \
    GEMV_GRID_INST(TN, WT, 1) GEMV_GRID_INST(TN, WT, 2) GEMV_GRID_INST(TN, WT, 4) GEMV_GRID_INST(TN, WT, 8)     \
    extern "C" __global__ void __launch_bounds__(512) ghip_mmid_gemv_##TN(MMID_ARGS) {                           \
        MMID_PAIR(q) gemv_grid_impl<WT, 1, false>(q.W, as_nb1, rows, nb, q.act, act_rb, 1, q.dst, 0, nullptr);  \
    }                                                                                                            \
    extern "C" __global__ void __launch_bounds__(512) ghip_mmid_gemv_##TN##_sub(MMID_ARGS) {                     \
        MMID_PAIR(q) gemv_grid_impl<WT, 1, true>(q.W, as_nb1, rows, nb, q.act, act_rb, 1, q.dst, 0, q.sub);     \
    }
GEMV_GRID_TYPE(iq2_xxs, WT_IQ2_XXS)
GEMV_GRID_TYPE(iq2_xs, WT_IQ2_XS)
GEMV_GRID_TYPE(iq2_s, WT_IQ2_S)
GEMV_GRID_TYPE(iq3_xxs, WT_IQ3_XXS)
GEMV_GRID_TYPE(iq3_s, WT_IQ3_S)
GEMV_GRID_TYPE(iq1_s, WT_IQ1_S)
GEMV_GRID_TYPE(iq1_m, WT_IQ1_M)
