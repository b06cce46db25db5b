// ghip_skinny.hip -- decode MUL_MAT for Q4_K weights at 2-15 activation rows
// on the int8 matrix cores (v_mfma_i32_16x16x64_i8).
//
// The arithmetic is the reference's vec_dot_q4_K_q8_K / gemv_q4_K_8x8_q8_K
// per (token m, weight row n, super-block b) (vec_dot.rs:928-980,
// repack.rs:1692-1770):
//   iacc = sum_e q4[n,e] * sc[n,s(e)] * q8[m,e],  imin = sum_s mn[n,s] * bsum[m,s]
//   out[m,n] = sum_b  d8[m,b] * (dw[n,b] * iacc - dmin[n,b] * imin)
// with the activation rows quantized to Q8_K once per workgroup into LDS, as
// the VALU decode kernels do.  On the matrix cores the 6-bit scale is split
// sc = 8 * hi + lo and each weight nibble enters two int8 planes, q4 * lo and
// q4 * hi (both <= 105): iacc = 8 * (A . W_hi) + (A . W_lo), exact int32.
// The min term is one exact f16 MFMA (mn <= 63 and |bsum16| <= 2032 are exact
// in f16 and every sum stays below 2^24).
//
// Tile: a wavefront owns 16 weight rows (the B columns) and a range of
// super-blocks; the tokens are the A rows, padded to 16 with zeros.  Lane l
// takes row / token l % 16 and the sub-block pair g = l / 16: qs bytes
// 32g .. 32g+31 of its row (sub-blocks 2g and 2g+1, low and high nibbles).
// K-step t of a super-block holds, per lane, bytes 32g + 8t .. +7 as 16
// elements: 8 of sub-block 2g then 8 of sub-block 2g+1 at positions
// 8t .. 8t+7; the activation operand takes the same elements, so both
// operands follow one K order and a lane's scales stay fixed over the four
// K-steps.  A workgroup of RT x KS wavefronts covers RT row tiles with K split
// KS ways; the KS partial sums of a row are added in order through LDS.
#include "ghip_common.h"
#include "ghip_actq.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

DEV uint32_t mul_bytes4(uint32_t nib, uint32_t s) {
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    const us2 a = __builtin_bit_cast(us2, nib);
    const us2 r = a * (us2){(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, r);
}

// NC: activation rows held in LDS (ncols <= NC <= 16).  wg: workgroup index
// within the matrix (-1: blockIdx.x).
template <int NC, bool SUBSUMS, bool FUSEQ, int RT, int KS>
__device__ __forceinline__ void gemv_q4K_mfma_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows,
                                                   int nb, const uint8_t *__restrict__ act, int64_t act_row_bytes,
                                                   int ncols, float *__restrict__ dst, int64_t ldd,
                                                   int32_t *__restrict__ sub, int n_mat, int wg = -1) {
    static_assert(RT * KS == 8, "eight wavefronts per workgroup");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rt = wave % RT, ks = wave / RT;
    const int K = nb * QK_K;
    int8_t *codes = reinterpret_cast<int8_t *>(smem);
    float *dq = reinterpret_cast<float *>(smem + NC * K);
    int *bsum = reinterpret_cast<int *>(dq + NC * nb);
    float *red = reinterpret_cast<float *>(bsum + NC * nb * 16);  // [KS][RT * 16 rows][16 tokens]

    const int n = lane & 15, g = lane >> 4;
    const int tile = (wg < 0 ? (int)blockIdx.x : wg) * RT + rt;
    const int row = tile * 16 + n;
    const int rowc = min(row, rows - 1);  // rows past the matrix re-read the last one (not stored)
    const int nbk = (nb + KS - 1) / KS;
    const int b0 = min(nb, ks * nbk), b1 = min(nb, b0 + nbk);
    const uint8_t *rowp = W + (int64_t)rowc * w_row_bytes;

    // a super-block's weights for this lane: header (d, dmin, scales) and qs
    // bytes 32g .. 32g+31, streamed one super-block ahead
    struct WB {
        uint4 hdr, q0, q1;
    };
    auto wload = [&](int b) {
        WB r;
        const uint8_t *p = rowp + (int64_t)b * Q4K_BYTES;
        r.hdr = ld16(p);
        r.q0 = ld16(p + 16 + 32 * g);
        r.q1 = ld16(p + 32 + 32 * g);
        return r;
    };

    // ---- activation image in LDS (activation loads first, then the first
    // super-blocks' weights, then the quantization)
    const int total = NC * nb * 16;
    const bool qwave = wave * 64 < total;
    WB cur = {}, nxt = {};
    if (FUSEQ) {
        const float *x = reinterpret_cast<const float *>(act);
        const int64_t xs = act_row_bytes / 4;
        XTask t0;
        if (qwave) t0 = quant_q8K_load(x, xs, ncols, nb, total, threadIdx.x);
        if (b0 < b1) cur = wload(b0);
        if (b0 + 1 < b1) nxt = wload(b0 + 1);
        if (qwave) quant_q8K_store(t0, nb, n_mat, total, threadIdx.x, codes, dq, bsum);
        for (int base = blockDim.x; base < total; base += blockDim.x) {
            if (base + wave * 64 >= total) break;
            const XTask t = quant_q8K_load(x, xs, ncols, nb, total, base + threadIdx.x);
            quant_q8K_store(t, nb, n_mat, total, base + threadIdx.x, codes, dq, bsum);
        }
    } else {
        Q8KTask t0;
        if (qwave) t0 = q8K_load(act, act_row_bytes, ncols, nb, total, threadIdx.x);
        if (b0 < b1) cur = wload(b0);
        if (b0 + 1 < b1) nxt = wload(b0 + 1);
        if (qwave) q8K_store(t0, nb, total, threadIdx.x, codes, dq, bsum);
        for (int base = blockDim.x; base < total; base += blockDim.x) {
            const Q8KTask t = q8K_load(act, act_row_bytes, ncols, nb, total, base + threadIdx.x);
            q8K_store(t, nb, total, base + threadIdx.x, codes, dq, bsum);
        }
    }
    __syncthreads();

    const int m = n;            // this lane's token in the A operand
    const bool mlive = m < NC;  // tokens past NC are zero rows
    const int8_t *crow = codes + (int64_t)(mlive ? m : 0) * K + 64 * g;
    const v4i zi = {};
    const v4f zf = {};
    v4f out = zf;
    for (int b = b0; b < b1; b++) {
        const WB w = cur;
        cur = nxt;
        if (b + 2 < b1) nxt = wload(b + 2);
        const float dw = h2f(w.hdr.x), dmin = h2f(w.hdr.x >> 16);
        int sc0, sc1, mn0, mn1;
        k4_scales(w.hdr.y, w.hdr.z, w.hdr.w, scale_sel(g), sc0, sc1, mn0, mn1);
        // min term: A = bsum16 of sub-blocks 2g, 2g+1 (two halves each), B = their mins
        v4h am = {}, bm;
        if (mlive) {
            const int *bs = bsum + (m * nb + b) * 16 + 4 * g;
            am[0] = (_Float16)(float)bs[0];
            am[1] = (_Float16)(float)bs[1];
            am[2] = (_Float16)(float)bs[2];
            am[3] = (_Float16)(float)bs[3];
        }
        bm[0] = bm[1] = (_Float16)(float)mn0;
        bm[2] = bm[3] = (_Float16)(float)mn1;
        const v4f accm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, zf, 0, 0, 0);
        // main term: four K-steps, two planes
        const uint32_t qv[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        const uint32_t l0 = (uint32_t)sc0 & 7u, h0 = (uint32_t)sc0 >> 3, l1 = (uint32_t)sc1 & 7u, h1 = (uint32_t)sc1 >> 3;
        v4i acc_l = zi, acc_h = zi;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            v4i a = zi;
            if (mlive) {
                const uint2 a0 = *reinterpret_cast<const uint2 *>(crow + (int64_t)b * QK_K + 8 * t);
                const uint2 a1 = *reinterpret_cast<const uint2 *>(crow + (int64_t)b * QK_K + 32 + 8 * t);
                a = (v4i){(int)a0.x, (int)a0.y, (int)a1.x, (int)a1.y};
            }
            const uint32_t d0 = qv[2 * t], d1 = qv[2 * t + 1];
            const uint32_t lo0 = d0 & 0x0f0f0f0fu, lo1 = d1 & 0x0f0f0f0fu;
            const uint32_t hi0 = (d0 >> 4) & 0x0f0f0f0fu, hi1 = (d1 >> 4) & 0x0f0f0f0fu;
            const v4i blo = {(int)mul_bytes4(lo0, l0), (int)mul_bytes4(lo1, l0), (int)mul_bytes4(hi0, l1),
                             (int)mul_bytes4(hi1, l1)};
            const v4i bhi = {(int)mul_bytes4(lo0, h0), (int)mul_bytes4(lo1, h0), (int)mul_bytes4(hi0, h1),
                             (int)mul_bytes4(hi1, h1)};
            acc_l = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, blo, acc_l, 0, 0, 0);
            acc_h = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bhi, acc_h, 0, 0, 0);
        }
        // scaling: lane l holds row n = l % 16 and tokens 4g .. 4g+3
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int tok = 4 * g + v;
            const int iacc = (acc_h[v] << 3) + acc_l[v];
            const float im = accm[v];
            const float da = tok < NC ? dq[tok * nb + b] : 0.0f;
            if (SUBSUMS && tok < ncols && row < rows) {
                int32_t *sp = sub + (((int64_t)tok * rows + row) * nb + b) * 2;
                sp[0] = iacc;
                sp[1] = (int)im;
            }
            const float tt = fmaf(dw, (float)iacc, -(dmin * im));
            out[v] = fmaf(da, tt, out[v]);
        }
    }
    if constexpr (KS == 1) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int tok = 4 * g + v;
            if (tok < ncols && row < rows) dst[(int64_t)tok * ldd + row] = out[v];
        }
    } else {
#pragma unroll
        for (int v = 0; v < 4; v++) red[(ks * RT * 16 + rt * 16 + n) * 16 + 4 * g + v] = out[v];
        __syncthreads();
        // row r of the workgroup, token c: the KS partials added in K order
        for (int idx = threadIdx.x; idx < RT * 16 * 16; idx += blockDim.x) {
            const int rr = idx >> 4, c = idx & 15;
            const int grow = (tile - rt) * 16 + rr;
            if (c >= ncols || grow >= rows) continue;
            float s = red[rr * 16 + c];
#pragma unroll
            for (int k = 1; k < KS; k++) s += red[(k * RT * 16 + rr) * 16 + c];
            dst[(int64_t)c * ldd + grow] = s;
        }
    }
}

// LDS: codes [NC][K] | d [NC][nb] | bsum [NC][nb][16] int | partials [KS][RT*16][16] f32
#define SKINNY_ARGS                                                                                                  \
    const uint8_t *__restrict__ W, int64_t w_row_bytes, int rows, int nb, const uint8_t *__restrict__ act,           \
        int64_t act_row_bytes, int ncols, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub, int n_mat
#define SKINNY_PASS W, w_row_bytes, rows, nb, act, act_row_bytes, ncols, dst, ldd, sub, n_mat
#define SKINNY_INST(NC, RT, KS)                                                                                      \
    extern "C" __global__ void __launch_bounds__(512) ghip_mma_q4_K_c##NC##_r##RT##k##KS(SKINNY_ARGS) {              \
        gemv_q4K_mfma_impl<NC, false, false, RT, KS>(SKINNY_PASS);                                                   \
    }                                                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_mma_q4_K_sub_c##NC##_r##RT##k##KS(SKINNY_ARGS) {          \
        gemv_q4K_mfma_impl<NC, true, false, RT, KS>(SKINNY_PASS);                                                    \
    }                                                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_mma_q4_K_f_c##NC##_r##RT##k##KS(SKINNY_ARGS) {            \
        gemv_q4K_mfma_impl<NC, false, true, RT, KS>(SKINNY_PASS);                                                    \
    }                                                                                                                \
    extern "C" __global__ void __launch_bounds__(512) ghip_mma_q4_K_f_sub_c##NC##_r##RT##k##KS(SKINNY_ARGS) {        \
        gemv_q4K_mfma_impl<NC, true, true, RT, KS>(SKINNY_PASS);                                                     \
    }
#define SKINNY_NC(NC) SKINNY_INST(NC, 2, 4) SKINNY_INST(NC, 1, 8) SKINNY_INST(NC, 4, 2)
SKINNY_NC(2) SKINNY_NC(4) SKINNY_NC(8) SKINNY_NC(16)

// Sibling MUL_MATs in one launch (ghip_graph_compute), as the decode GEMVs:
// workgroups [wg0[i], wg0[i+1]) compute matrix i.  Host mirror in ghip.cpp.
struct SkinnyMulti {
    const uint8_t *W[4];
    float *dst[4];
    int64_t ldd[4];
    int rows[4];
    int wg0[4];
    int n;
};
// ready Q8_K rows (quantized once for the group)
#define SKINNY_MULTI(NC, RT, KS)                                                                                     \
    extern "C" __global__ void __launch_bounds__(512)                                                                \
        ghip_mma_q4_K_c##NC##_r##RT##k##KS##_multi(SkinnyMulti g, int64_t w_row_bytes, int nb,                       \
                                                   const uint8_t *__restrict__ act, int64_t act_row_bytes,           \
                                                   int ncols, int n_mat) {                                           \
        const int bx = blockIdx.x;                                                                                   \
        int i = 0;                                                                                                   \
        _Pragma("unroll") for (int k = 1; k < 4; k++) if (k < g.n && bx >= g.wg0[k]) i = k;                         \
        gemv_q4K_mfma_impl<NC, false, false, RT, KS>(g.W[i], w_row_bytes, g.rows[i], nb, act, act_row_bytes, ncols,  \
                                                     g.dst[i], g.ldd[i], nullptr, n_mat, bx - g.wg0[i]);             \
    }
SKINNY_MULTI(4, 2, 4) SKINNY_MULTI(8, 2, 4) SKINNY_MULTI(16, 2, 4)

// ===================================================================== split K
// Decode MUL_MAT at 4..8 activation rows (Q4_K, Q6_K), split over K across
// workgroups.  The K axis is cut into slices of S super-blocks (S depends on
// K only, so a matrix gives the same bits alone and in a grouped launch).  A
// workgroup of 4 wavefronts owns one slice and a set of 64-row tiles:
//  - it quantizes its slice of the f32 activation rows to Q8_K in LDS once
//    (quant_q8K_*, bit-identical to ghip_quantize_q8_K; Q8_K blocks do not
//    cross super-blocks), so no separate quantization launch is needed;
//  - it walks its tiles in steps of 2 super-blocks x 16 rows per wavefront,
//    the next step's weights loaded into registers while the current one
//    runs on the int8 matrix cores.
// Each slice's fp32 partials go to a workspace and ghip_sk_reduce adds them
// in slice order.  (Handing the sum to each tile's last workgroup through a
// counter measured 8-9 us slower on the Llama-3-8B decode layer: every
// workgroup then waits for its partials to reach memory and for the
// counter's round trip.)
//
// Both types put the sub-block in the token dimension of the MFMA: its 16 A
// rows are (token t, parity h) pairs, row 2t+h holding token t's codes at the
// K positions of the step's sub-block h and zeros elsewhere, so C[2t+h][row]
// is the exact integer dot of one sub-block.  Weight codes enter unsigned.
//
// Q4_K (vec_dot_q4_K_q8_K, vec_dot.rs:928-980): v_mfma_i32_16x16x64_i8 per
// 64-element chunk c (sub-blocks 2c: low nibbles of qs 32c..32c+31, 2c+1: high
// nibbles).  Lane group G takes qs 32c + 8G .. +7: its 16 K positions are the
// 8 low nibbles (elements 64c + 8G + i) then the 8 high nibbles (elements
// 64c + 32 + 8G + i).  iacc = sum_s sc[s] C_s; the min term
// sum_s m[s] bsum32[t][s] is one exact f16 MFMA over the 16-element sums.
//
// Q6_K (vec_dot_q6_K_q8_K, vec_dot.rs:1010-1060): v_mfma_i32_16x16x32_i8 per
// 32-element chunk (n, q), elements 128n + 32q + l, l = 0..31 (sub-blocks
// 8n + 2q and 8n + 2q + 1), code
//   (ql[64n + 32(q&1) + l] >> 4(q>>1)) & 15  |  ((qh[32n + l] >> 2q) & 3) << 4
// (dequantize_row_q6_K's element order, quants_k.rs:2096-2115); lane group G
// takes l = 8G .. 8G+7.  The -32 offset is -32 * sum_s sc[s] * bsum16[t][s],
// one exact f16 MFMA per super-block (|sc| <= 128, |bsum16| <= 2032, sums
// < 2^24).
constexpr int SK_WAVES = 4;
constexpr int SK_ROWS = 16 * SK_WAVES;  // weight rows per tile

struct SkMember {
    const uint8_t *W;
    float *dst;
    int64_t ldd;
    float *part;  // [slices][ncols][rows] fp32 partials (more than one slice)
    int rows;
    int tile0;    // first tile of this matrix in the launch
};
struct SkLaunch {
    SkMember m[4];
    int n;        // matrices
    int n_tiles;  // tiles over all matrices
    int nks;      // K-slices
    int tg;       // tile groups: workgroup bx takes slice bx % nks, tiles bx / nks + k * tg
};

typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int sk_nw(int wt) { return wt == 12 ? 12 : 14; }

// The weight dwords lane group G needs of one super-block at p:
// Q4_K: header (d, dmin, 12 scale bytes) | qs 32c + 8G .. +7 for c = 0..3
// Q6_K: ql 32k + 8G .. +7 (k = 0..3) | qh 32k + 8G .. +7 (k = 0, 1) | scales 4G .. 4G+3 | d
template <int WT>
DEV void sk_load(const uint8_t *__restrict__ p, int G, uint32_t (&w)[sk_nw(WT)]) {
    if constexpr (WT == 12) {
        const uint4 h = ld16(p);
        w[0] = h.x;
        w[1] = h.y;
        w[2] = h.z;
        w[3] = h.w;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint2 q = ld8(p + 16 + 32 * c + 8 * G);
            w[4 + 2 * c] = q.x;
            w[5 + 2 * c] = q.y;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 6; k++) {
            const uint2 q = ld8(p + 32 * k + 8 * G);
            w[2 * k] = q.x;
            w[2 * k + 1] = q.y;
        }
        w[12] = ld4(p + 192 + 4 * G);
        w[13] = ld2(p + 208);
    }
}

// One super-block of one 16-row tile: lane (j, G) adds its row j's term for
// tokens 2G and 2G + 1 to out[0..1].  v: the lane's weight dwords (sk_load);
// the activation image holds token t's codes at codes + t * kstride (super-block
// bl at + 256 bl), its scales at dq[t * nbs + bl] and its 16-element sums at
// bsum + t * BS + 16 bl; b is the super-block's index in the row (sub-sums).
template <int WT, bool SUBSUMS>
DEV void sk_block(const uint32_t *v, const int8_t *codes, int kstride, const float *dq, int nbs, const int *bsum,
                  int BS, int bl, int b, int row, int rows, int nb, int ncols, int32_t *__restrict__ sub, int lane,
                  float (&out)[2]) {
    const int j = lane & 15, G = lane >> 4;
    const int t_a = j >> 1, h_a = j & 1;  // this lane's A row: token, parity
    // -32 / min term: A row 4g + u (u < 2) = token 2g + u over the
    // 16-element sums 4G .. 4G+3
    v4h am = {};
    {
        const int gg = j >> 2, u = j & 3;
        if (u < 2) {
            const int *p = bsum + (2 * gg + u) * BS + bl * 16 + 4 * G;
            am[0] = (_Float16)(float)p[0];
            am[1] = (_Float16)(float)p[1];
            am[2] = (_Float16)(float)p[2];
            am[3] = (_Float16)(float)p[3];
        }
    }
    const int8_t *crow = codes + t_a * kstride + bl * QK_K;
    if constexpr (WT == 12) {
        const float dw = h2f(v[0]), dmin = h2f(v[0] >> 16);
        v4h bm;
        {
            int s0, s1, m0, m1;
            k4_scales(v[1], v[2], v[3], scale_sel(G), s0, s1, m0, m1);
            bm[0] = bm[1] = (_Float16)(float)m0;
            bm[2] = bm[3] = (_Float16)(float)m1;
        }
        const v4f accm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, (v4f){}, 0, 0, 0);
        int is0 = 0, is1 = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t d0 = v[4 + 2 * c], d1 = v[5 + 2 * c];
            const v4i bw = {(int)(d0 & 0x0f0f0f0fu), (int)(d1 & 0x0f0f0f0fu), (int)((d0 >> 4) & 0x0f0f0f0fu),
                            (int)((d1 >> 4) & 0x0f0f0f0fu)};
            const uint2 a8 = *reinterpret_cast<const uint2 *>(crow + 64 * c + 32 * h_a + 8 * G);
            const v4i a = h_a ? (v4i){0, 0, (int)a8.x, (int)a8.y} : (v4i){(int)a8.x, (int)a8.y, 0, 0};
            const v4i r = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw, (v4i){}, 0, 0, 0);
            int sc0, sc1, mn0, mn1;
            k4_scales(v[1], v[2], v[3], scale_sel(c), sc0, sc1, mn0, mn1);
            is0 += __mul24(sc0, r[0]) + __mul24(sc1, r[1]);  // |r| < 2^23
            is1 += __mul24(sc0, r[2]) + __mul24(sc1, r[3]);
        }
        const int isv[2] = {is0, is1};
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int tok = 2 * G + u;
            const float im = accm[u];
            if (SUBSUMS && tok < ncols && row < rows) {
                int32_t *sp = sub + (((int64_t)tok * rows + row) * nb + b) * 2;
                sp[0] = isv[u];
                sp[1] = (int)im;
            }
            out[u] = fmaf(dq[tok * nbs + bl], fmaf(dw, (float)isv[u], -(dmin * im)), out[u]);
        }
    } else {
        const float dw = h2f(v[13]);
        const uint32_t sw = v[12];  // scales 4G .. 4G+3 of row j
        v4h bs;
        bs[0] = (_Float16)(float)(int8_t)(sw & 0xff);
        bs[1] = (_Float16)(float)(int8_t)((sw >> 8) & 0xff);
        bs[2] = (_Float16)(float)(int8_t)((sw >> 16) & 0xff);
        bs[3] = (_Float16)(float)(int8_t)(sw >> 24);
        const v4f accm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bs, (v4f){}, 0, 0, 0);
        const bool alive = (G >> 1) == h_a;
        int is0 = 0, is1 = 0;
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const uint32_t qh0 = v[8 + 2 * n], qh1 = v[9 + 2 * n];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int src = 2 * (2 * n + (q & 1));  // ql words of 64n + 32(q&1)
                const int sh = 4 * (q >> 1);
                const uint32_t c0 = ((v[src] >> sh) & 0x0f0f0f0fu) | (((qh0 >> (2 * q)) & 0x03030303u) << 4);
                const uint32_t c1 = ((v[src + 1] >> sh) & 0x0f0f0f0fu) | (((qh1 >> (2 * q)) & 0x03030303u) << 4);
                const long bw = (long)(((uint64_t)c1 << 32) | c0);
                long a = 0;
                if (alive) a = *reinterpret_cast<const long *>(crow + 128 * n + 32 * q + 8 * G);
                const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bw, (v4i){}, 0, 0, 0);
                // scales 8n + 2q, 8n + 2q + 1: dword 2n + (q >> 1), held by lane group 2n + (q >> 1)
                const uint32_t sd = (uint32_t)__shfl((int)sw, j + 16 * (2 * n + (q >> 1)), 64);
                const int sc0 = (int)(int8_t)((sd >> (16 * (q & 1))) & 0xff);
                const int sc1 = (int)(int8_t)((sd >> (16 * (q & 1) + 8)) & 0xff);
                is0 += __mul24(sc0, c[0]) + __mul24(sc1, c[1]);  // |c| < 2^23
                is1 += __mul24(sc0, c[2]) + __mul24(sc1, c[3]);
            }
        }
        const int isv[2] = {is0 - 32 * (int)accm[0], is1 - 32 * (int)accm[1]};
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int tok = 2 * G + u;
            if (SUBSUMS && tok < ncols && row < rows) sub[((int64_t)tok * rows + row) * nb + b] = isv[u];
            out[u] += (dw * (float)isv[u]) * dq[tok * nbs + bl];
        }
    }
}

// Q4_K in 16-byte pieces (the whole-K kernels): lane group G loads the
// header and qs bytes 64p + 16G .. +15 for p = 0, 1, so the 4 lane groups read
// 64 contiguous bytes of a row per load.  qs byte 64p + 16G + x holds element
// 16(G&1) + x of sub-blocks 4p + 2(G>>1) (low nibble) and 4p + 2(G>>1) + 1
// (high nibble), so MFMA (p, n) over the lanes' low (n = 0) or high (n = 1)
// nibbles covers sub-blocks 4p + n (lane groups 0, 1) and 4p + 2 + n (lane
// groups 2, 3).  A row 2t + h holds token t's codes in the lane groups with
// G >> 1 == h and zeros in the others, which read a zeroed region of the
// image instead: C[2t + h][row] is the exact dot of sub-block 4p + 2h + n.
DEV void q4k16_load(const uint8_t *__restrict__ p, int G, uint32_t (&w)[12]) {
    const uint4 h = ld16(p), a = ld16(p + 16 + 16 * G), b = ld16(p + 80 + 16 * G);
    w[0] = h.x;
    w[1] = h.y;
    w[2] = h.z;
    w[3] = h.w;
    w[4] = a.x;
    w[5] = a.y;
    w[6] = a.z;
    w[7] = a.w;
    w[8] = b.x;
    w[9] = b.y;
    w[10] = b.z;
    w[11] = b.w;
}

// One super-block of one 16-row tile, lane (j, G): tokens 2G and 2G + 1 of
// row j added to out[0..1] (the arithmetic of sk_block for Q4_K).  abase: the
// lane's A operand base (token j >> 1's codes + 64 (j & 1) + 16 (G & 1), or
// the zero region); the super-block's codes are at abase + 256 bl.
template <bool SUBSUMS>
DEV void q4k16_block(const uint32_t *v, const int8_t *abase, const float *dq, int nbs, const int *bsum, int BS,
                     int bl, int b, int row, int rows, int nb, int ncols, int32_t *__restrict__ sub, int lane,
                     float (&out)[2]) {
    const int j = lane & 15, G = lane >> 4;
    // min term: A row 4g + u (u < 2) = token 2g + u over the 16-element sums
    // 4G .. 4G+3, B column j = the mins of sub-blocks 2G, 2G + 1 of row j
    v4h am = {};
    {
        const int gg = j >> 2, u = j & 3;
        if (u < 2) {
            const int *p = bsum + (2 * gg + u) * BS + bl * 16 + 4 * G;
            am[0] = (_Float16)(float)p[0];
            am[1] = (_Float16)(float)p[1];
            am[2] = (_Float16)(float)p[2];
            am[3] = (_Float16)(float)p[3];
        }
    }
    const float dw = h2f(v[0]), dmin = h2f(v[0] >> 16);
    v4h bm;
    {
        int s0, s1, m0, m1;
        k4_scales(v[1], v[2], v[3], scale_sel(G), s0, s1, m0, m1);
        bm[0] = bm[1] = (_Float16)(float)m0;
        bm[2] = bm[3] = (_Float16)(float)m1;
    }
    const v4f accm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, (v4f){}, 0, 0, 0);
    int is0 = 0, is1 = 0;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        int sc[4], mn[4];
        k4_scales(v[1], v[2], v[3], scale_sel(2 * p), sc[0], sc[1], mn[0], mn[1]);
        k4_scales(v[1], v[2], v[3], scale_sel(2 * p + 1), sc[2], sc[3], mn[2], mn[3]);
        const uint32_t *q = v + 4 + 4 * p;
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const v4i bw = n == 0 ? (v4i){(int)(q[0] & 0x0f0f0f0fu), (int)(q[1] & 0x0f0f0f0fu), (int)(q[2] & 0x0f0f0f0fu),
                                          (int)(q[3] & 0x0f0f0f0fu)}
                                  : (v4i){(int)((q[0] >> 4) & 0x0f0f0f0fu), (int)((q[1] >> 4) & 0x0f0f0f0fu),
                                          (int)((q[2] >> 4) & 0x0f0f0f0fu), (int)((q[3] >> 4) & 0x0f0f0f0fu)};
            const v4i a = *reinterpret_cast<const v4i *>(abase + bl * QK_K + 128 * p + 32 * n);
            const v4i r = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw, (v4i){}, 0, 0, 0);
            // C rows 4G + v: token 2G + (v >> 1), sub-block 4p + n + 2 (v & 1)
            is0 += __mul24(sc[n], r[0]) + __mul24(sc[n + 2], r[1]);  // |r| < 2^23
            is1 += __mul24(sc[n], r[2]) + __mul24(sc[n + 2], r[3]);
        }
    }
    const int isv[2] = {is0, is1};
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int tok = 2 * G + u;
        const float im = accm[u];
        if (SUBSUMS && tok < ncols && row < rows) {
            int32_t *sp = sub + (((int64_t)tok * rows + row) * nb + b) * 2;
            sp[0] = isv[u];
            sp[1] = (int)im;
        }
        out[u] = fmaf(dq[tok * nbs + bl], fmaf(dw, (float)isv[u], -(dmin * im)), out[u]);
    }
}

template <int WT, int S, int SK_GB, bool SUBSUMS>
__device__ __forceinline__ void sk_impl(const SkLaunch &g, int64_t w_row_bytes, int nb, const float *__restrict__ x,
                                        int64_t x_stride, int ncols, int n_mat, int32_t *__restrict__ sub) {
    static_assert(WT == 12 || WT == 14, "Q4_K or Q6_K");
    static_assert(S % SK_GB == 0, "whole pipeline steps per slice");
    constexpr int NC = 8;  // 16 A rows: 8 tokens x 2 sub-block parities
    constexpr int BB = WT == 12 ? Q4K_BYTES : Q6K_BYTES;
    constexpr int NW = sk_nw(WT);  // weight dwords per lane and super-block
    // image strides per token padded by 16 bytes / 4 ints, so the 8 tokens'
    // operand reads fall in different LDS banks
    constexpr int CS = S * QK_K + 16, BS = S * 16 + 4;
    __shared__ __attribute__((aligned(16))) int8_t codes[NC * CS];
    __shared__ float dq[NC * S];
    __shared__ int bsum[NC * BS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, G = lane >> 4;
    const int ks = (int)blockIdx.x % g.nks, tgi = (int)blockIdx.x / g.nks;
    const int b0 = ks * S, nbs = min(S, nb - b0);
    const int ngrp = (nbs + SK_GB - 1) / SK_GB;
    const int my_tiles = tgi < g.n_tiles ? (g.n_tiles - tgi + g.tg - 1) / g.tg : 0;
    const int items = my_tiles * ngrp;

    // ---- activation slice: the first round's loads go out before any weight
    // load, so the quantization waits only for them
    const float *xs = x + (int64_t)b0 * QK_K;
    const int total = NC * nbs * 16;  // a multiple of 64: whole wavefronts take part or not
    const bool qwave = wave * 64 < total;
    XTask t0;
    if (qwave) t0 = quant_q8K_load(xs, x_stride, ncols, nbs, total, threadIdx.x);

    // the matrix, its row for this lane and the super-blocks of step `it`
    auto member = [&](int tile) {
        int i = 0;
#pragma unroll
        for (int k = 1; k < 4; k++)
            if (k < g.n && tile >= g.m[k].tile0) i = k;
        return i;
    };
    auto load = [&](uint32_t (&w)[SK_GB][NW], int it) {
        const int tile = tgi + (it / ngrp) * g.tg, grp = it % ngrp;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * SK_ROWS + 16 * wave + j;
        const uint8_t *rp = mb.W + (int64_t)min(row, mb.rows - 1) * w_row_bytes + (int64_t)(b0 + SK_GB * grp) * BB;
#pragma unroll
        for (int i = 0; i < SK_GB; i++) {
            if (SK_GB * grp + i >= nbs) break;
            sk_load<WT>(rp + (int64_t)i * BB, G, w[i]);
        }
    };
    uint32_t wa[SK_GB][NW], wb[SK_GB][NW];
    if (items > 0) load(wa, 0);

    if (qwave) quant_q8K_store(t0, nbs, n_mat, total, threadIdx.x, codes, dq, bsum, CS, BS);
    for (int base = blockDim.x; base < total; base += blockDim.x) {
        if (base + wave * 64 >= total) break;
        const XTask t = quant_q8K_load(xs, x_stride, ncols, nbs, total, base + threadIdx.x);
        quant_q8K_store(t, nbs, n_mat, total, base + threadIdx.x, codes, dq, bsum, CS, BS);
    }
    __syncthreads();

    const int kstride = CS;  // one token's codes in the image
    float out[2] = {0.0f, 0.0f};  // tokens 2G, 2G + 1 of row j
    auto compute = [&](const uint32_t (&w)[SK_GB][NW], int it) {
        const int tile = tgi + (it / ngrp) * g.tg, grp = it % ngrp;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * SK_ROWS + 16 * wave + j;
#pragma unroll
        for (int i = 0; i < SK_GB; i++) {
            const int bl = SK_GB * grp + i;
            if (bl >= nbs) break;
            const int b = b0 + bl;
            sk_block<WT, SUBSUMS>(w[i], codes, kstride, dq, nbs, bsum, BS, bl, b, row, mb.rows, nb, ncols, sub, lane,
                                  out);
        }
        if (grp == ngrp - 1) {  // the tile's slice is done: store, or leave the partials for ghip_sk_reduce
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int tok = 2 * G + u;
                if (tok < ncols && row < mb.rows) {
                    if (g.nks == 1) mb.dst[(int64_t)tok * mb.ldd + row] = out[u];
                    else mb.part[((int64_t)ks * ncols + tok) * mb.rows + row] = out[u];
                }
                out[u] = 0.0f;
            }
        }
    };
    for (int it = 0; it < items;) {
        if (it + 1 < items) load(wb, it + 1);
        compute(wa, it);
        if (++it >= items) break;
        if (it + 1 < items) load(wa, it + 1);
        compute(wb, it);
        ++it;
    }
}

// Steps of 2 super-blocks: at most 128 VGPRs, four wavefronts per SIMD (steps
// of 4 measured 27.3 -> 24.6 us on the decode layer's gate/up pair at 8 rows,
// 27.3 -> 24.3 us on Q6_K down)
#define SK_KERNEL(NAME, WT, S, SUBS) SK_KERNELG(NAME, WT, S, 2, SUBS)
#define SK_KERNELG(NAME, WT, S, GB, SUBS)                                                                          \
    extern "C" __global__ void __launch_bounds__(64 * SK_WAVES)                                                    \
        NAME(SkLaunch g, int64_t w_row_bytes, int nb, const float *__restrict__ x, int64_t x_stride, int ncols,   \
             int n_mat, int32_t *__restrict__ sub) {                                                               \
        sk_impl<WT, S, GB, SUBS>(g, w_row_bytes, nb, x, x_stride, ncols, n_mat, sub);                                  \
    }
SK_KERNEL(ghip_sk_q4_K_s4, 12, 4, false)
SK_KERNEL(ghip_sk_q4_K_s8, 12, 8, false)
SK_KERNEL(ghip_sk_q4_K_sub_s4, 12, 4, true)
SK_KERNEL(ghip_sk_q4_K_sub_s8, 12, 8, true)
SK_KERNEL(ghip_sk_q6_K_s4, 14, 4, false)
SK_KERNEL(ghip_sk_q6_K_s8, 14, 8, false)
SK_KERNEL(ghip_sk_q6_K_sub_s4, 14, 4, true)
SK_KERNEL(ghip_sk_q6_K_sub_s8, 14, 8, true)


// ================================================================ whole K
// Decode MUL_MAT at 4..8 activation rows (Q4_K, Q6_K) from ready Q8_K rows
// (ghip_quantize_q8_K's output, or a src1 that is Q8_K already): one launch,
// no reduction launch, and each activation block quantized once per call
// rather than once per workgroup.  A workgroup of W wavefronts owns T tiles
// of 16 weight rows over the whole K axis; wavefront w takes the super-blocks
// [w SW, w SW + SW):
//  - all of its weight loads (T tiles x SW super-blocks, into registers) go
//    out first, then it copies the 8 rows' Q8_K blocks of its super-blocks
//    into an LDS image of its own (no other wavefront reads it: no barrier);
//  - it runs the split-K arithmetic (sk_block) on each tile, the tile's fp32
//    partial kept in registers;
//  - the partials go to LDS over its image, and after one barrier each output
//    is the sum of the W partials in wavefront (K) order.
// SW and W depend on K alone, so a matrix gives the same bits alone and in a
// grouped launch.  The image: codes [8][CS] | d [8][SW] | 16-element sums
// [8][BS] | 256 SW zero bytes (the Q4_K A operand's empty lane groups).  Host
// mirror of its size in ghip.cpp (sq_img_bytes).
constexpr int sq_img_bytes(int sw) { return 8 * (sw * QK_K + 16) + 8 * sw * 4 + 8 * (sw * 16 + 4) * 4 + sw * QK_K; }

template <int WT, int SW, int T, bool SUBSUMS>
__device__ __forceinline__ void sq_impl(const SkLaunch &g, int64_t w_row_bytes, int nb, const uint8_t *__restrict__ act,
                                        int64_t act_rb, int ncols, int32_t *__restrict__ sub) {
    constexpr int NC = 8, NW = sk_nw(WT);
    constexpr int BB = WT == 12 ? Q4K_BYTES : Q6K_BYTES;
    constexpr int CS = SW * QK_K + 16, BS = SW * 16 + 4, IMG = sq_img_bytes(SW);
    static_assert(T * NC * 16 * 4 <= IMG, "the partials fit over the image");
    extern __shared__ __attribute__((aligned(16))) uint8_t sq_smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = (int)(blockDim.x >> 6);
    const int j = lane & 15, G = lane >> 4;
    int8_t *codes = (int8_t *)(sq_smem + wave * IMG);
    float *dq = (float *)(codes + NC * CS);
    int *bsum = (int *)(dq + NC * SW);
    const int b0 = wave * SW, nbs = min(SW, nb - b0);  // >= 1: W = ceil(nb / SW)
    const int tile0 = (int)blockIdx.x * T;

    auto member = [&](int tile) {
        int i = 0;
#pragma unroll
        for (int k = 1; k < 4; k++)
            if (k < g.n && tile >= g.m[k].tile0) i = k;
        return i;
    };
    // activation blocks (token c, super-block b0 + bl), 16 lanes each, 4 per
    // round: block 4r + lane / 16 is c = its index % 8, bl = its index / 8
    constexpr int R = 2 * SW;
    uint4 av[R];
    int as[R];
    float ad[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int blk = 4 * r + G, c = blk & 7, bl = blk >> 3, l = lane & 15;
        av[r] = make_uint4(0, 0, 0, 0);
        as[r] = 0;
        ad[r] = 0.0f;
        if (bl < nbs && c < ncols) {
            const uint8_t *A = act + (int64_t)c * act_rb + (int64_t)(b0 + bl) * Q8K_BYTES;
            av[r] = ld16(A + 4 + 16 * l);
            as[r] = (int)(int16_t)ld2(A + 260 + 2 * l);
            ad[r] = __uint_as_float(ld4(A));
        }
    }
    uint32_t w[T][SW][NW];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int tile = tile0 + t;
        if (tile >= g.n_tiles) break;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * 16 + j;
        const uint8_t *rp = mb.W + (int64_t)min(row, mb.rows - 1) * w_row_bytes + (int64_t)b0 * BB;
#pragma unroll
        for (int bl = 0; bl < SW; bl++) {
            if (bl >= nbs) break;
            if constexpr (WT == 12) q4k16_load(rp + (int64_t)bl * BB, G, w[t][bl]);
            else sk_load<WT>(rp + (int64_t)bl * BB, G, w[t][bl]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int blk = 4 * r + G, c = blk & 7, bl = blk >> 3, l = lane & 15;
        if (bl < nbs) {
            *reinterpret_cast<uint4 *>(codes + c * CS + bl * QK_K + 16 * l) = av[r];
            bsum[c * BS + bl * 16 + l] = as[r];
            if (l == 0) dq[c * SW + bl] = ad[r];
        }
    }
    int8_t *zeros = (int8_t *)(bsum + NC * BS);
    for (int o = 16 * lane; o < SW * QK_K; o += 1024) *reinterpret_cast<uint4 *>(zeros + o) = make_uint4(0, 0, 0, 0);
    // Q4_K A operand base of this lane: token j >> 1 in the lane groups of its
    // parity j & 1, else the zero region
    const int8_t *abase = (G >> 1) == (j & 1) ? codes + (j >> 1) * CS + 64 * (j & 1) + 16 * (G & 1) : zeros;
    (void)abase;
    // the image is written and read by this wavefront only: order its LDS
    // stores before the other lanes' reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float out[T][2];
#pragma unroll
    for (int t = 0; t < T; t++) {
        out[t][0] = out[t][1] = 0.0f;
        const int tile = tile0 + t;
        if (tile >= g.n_tiles) break;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * 16 + j;
#pragma unroll
        for (int bl = 0; bl < SW; bl++) {
            if (bl >= nbs) break;
            if constexpr (WT == 12)
                q4k16_block<SUBSUMS>(w[t][bl], abase, dq, SW, bsum, BS, bl, b0 + bl, row, mb.rows, nb, ncols, sub,
                                     lane, out[t]);
            else
                sk_block<WT, SUBSUMS>(w[t][bl], codes, CS, dq, SW, bsum, BS, bl, b0 + bl, row, mb.rows, nb, ncols, sub,
                                      lane, out[t]);
        }
    }
    // partials [T][8 tokens][16 rows] over this wavefront's image
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float *part = (float *)(sq_smem + wave * IMG);
#pragma unroll
    for (int t = 0; t < T; t++) {
        part[(t * NC + 2 * G) * 16 + j] = out[t][0];
        part[(t * NC + 2 * G + 1) * 16 + j] = out[t][1];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < T * NC * 16; idx += blockDim.x) {
        const int t = idx >> 7, tok = (idx >> 4) & 7, r = idx & 15, tile = tile0 + t;
        if (tile >= g.n_tiles || tok >= ncols) continue;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * 16 + r;
        if (row >= mb.rows) continue;
        float acc = 0.0f;
        for (int k = 0; k < W; k++) {
            const float v = ((const float *)(sq_smem + k * IMG))[idx];
            acc = k == 0 ? v : acc + v;
        }
        mb.dst[(int64_t)tok * mb.ldd + row] = acc;
    }
}

// Streaming form: a workgroup takes tiles [T bx, T bx + T) (T from the
// host), each wavefront with the next tile's weights in flight while it
// computes the current one; tile t's partials go to LDS beside the image
// (partials [T][8 tokens][16 rows] per wavefront), and after one barrier
// every output of the workgroup is summed in wavefront order.
template <int WT, int SW, bool SUBSUMS>
__device__ __forceinline__ void sqs_impl(const SkLaunch &g, int T, int64_t w_row_bytes, int nb,
                                         const uint8_t *__restrict__ act, int64_t act_rb, int ncols,
                                         int32_t *__restrict__ sub) {
    constexpr int NC = 8, NW = sk_nw(WT);
    constexpr int BB = WT == 12 ? Q4K_BYTES : Q6K_BYTES;
    constexpr int CS = SW * QK_K + 16, BS = SW * 16 + 4, IMG = sq_img_bytes(SW);
    extern __shared__ __attribute__((aligned(16))) uint8_t sq_smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = (int)(blockDim.x >> 6);
    const int j = lane & 15, G = lane >> 4;
    const int stride = IMG + T * NC * 16 * 4;  // LDS bytes per wavefront
    int8_t *codes = (int8_t *)(sq_smem + wave * stride);
    float *dq = (float *)(codes + NC * CS);
    int *bsum = (int *)(dq + NC * SW);
    float *part = (float *)(sq_smem + wave * stride + IMG);
    const int b0 = wave * SW, nbs = min(SW, nb - b0);  // >= 1: W = ceil(nb / SW)
    const int tile0 = (int)blockIdx.x * T, cnt = min(T, g.n_tiles - tile0);  // >= 1

    auto member = [&](int tile) {
        int i = 0;
#pragma unroll
        for (int k = 1; k < 4; k++)
            if (k < g.n && tile >= g.m[k].tile0) i = k;
        return i;
    };
    constexpr int R = 2 * SW;
    uint4 av[R];
    int as[R];
    float ad[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int blk = 4 * r + G, c = blk & 7, bl = blk >> 3, l = lane & 15;
        av[r] = make_uint4(0, 0, 0, 0);
        as[r] = 0;
        ad[r] = 0.0f;
        if (bl < nbs && c < ncols) {
            const uint8_t *A = act + (int64_t)c * act_rb + (int64_t)(b0 + bl) * Q8K_BYTES;
            av[r] = ld16(A + 4 + 16 * l);
            as[r] = (int)(int16_t)ld2(A + 260 + 2 * l);
            ad[r] = __uint_as_float(ld4(A));
        }
    }
    auto load = [&](uint32_t (&w)[SW][NW], int t) {
        const int tile = tile0 + t;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * 16 + j;
        const uint8_t *rp = mb.W + (int64_t)min(row, mb.rows - 1) * w_row_bytes + (int64_t)b0 * BB;
#pragma unroll
        for (int bl = 0; bl < SW; bl++) {
            if (bl >= nbs) break;
            if constexpr (WT == 12) q4k16_load(rp + (int64_t)bl * BB, G, w[bl]);
            else sk_load<WT>(rp + (int64_t)bl * BB, G, w[bl]);
        }
    };
    uint32_t wa[SW][NW], wb[SW][NW];
    load(wa, 0);
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int blk = 4 * r + G, c = blk & 7, bl = blk >> 3, l = lane & 15;
        if (bl < nbs) {
            *reinterpret_cast<uint4 *>(codes + c * CS + bl * QK_K + 16 * l) = av[r];
            bsum[c * BS + bl * 16 + l] = as[r];
            if (l == 0) dq[c * SW + bl] = ad[r];
        }
    }
    int8_t *zeros = (int8_t *)(bsum + NC * BS);
    for (int o = 16 * lane; o < SW * QK_K; o += 1024) *reinterpret_cast<uint4 *>(zeros + o) = make_uint4(0, 0, 0, 0);
    // Q4_K A operand base of this lane: token j >> 1 in the lane groups of its
    // parity j & 1, else the zero region
    const int8_t *abase = (G >> 1) == (j & 1) ? codes + (j >> 1) * CS + 64 * (j & 1) + 16 * (G & 1) : zeros;
    (void)abase;
    // the image is written and read by this wavefront only: order its LDS
    // stores before the other lanes' reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    auto compute = [&](const uint32_t (&w)[SW][NW], int t) {
        const int tile = tile0 + t;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * 16 + j;
        float o[2] = {0.0f, 0.0f};
#pragma unroll
        for (int bl = 0; bl < SW; bl++) {
            if (bl >= nbs) break;
            if constexpr (WT == 12)
                q4k16_block<SUBSUMS>(w[bl], abase, dq, SW, bsum, BS, bl, b0 + bl, row, mb.rows, nb, ncols, sub, lane,
                                     o);
            else
                sk_block<WT, SUBSUMS>(w[bl], codes, CS, dq, SW, bsum, BS, bl, b0 + bl, row, mb.rows, nb, ncols, sub,
                                      lane, o);
        }
        part[(t * NC + 2 * G) * 16 + j] = o[0];
        part[(t * NC + 2 * G + 1) * 16 + j] = o[1];
    };
    for (int t = 0; t < cnt;) {
        if (t + 1 < cnt) load(wb, t + 1);
        compute(wa, t);
        if (++t >= cnt) break;
        if (t + 1 < cnt) load(wa, t + 1);
        compute(wb, t);
        ++t;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < cnt * NC * 16; idx += blockDim.x) {
        const int t = idx >> 7, tok = (idx >> 4) & 7, r = idx & 15, tile = tile0 + t;
        if (tok >= ncols) continue;
        const SkMember &mb = g.m[member(tile)];
        const int row = (tile - mb.tile0) * 16 + r;
        if (row >= mb.rows) continue;
        float acc = 0.0f;
        for (int k = 0; k < W; k++) {
            const float v = ((const float *)(sq_smem + k * stride + IMG))[idx];
            acc = k == 0 ? v : acc + v;
        }
        mb.dst[(int64_t)tok * mb.ldd + row] = acc;
    }
}

#define SQS_KERNEL(NAME, WT, SW, SUBS)                                                                             \
    extern "C" __global__ void __launch_bounds__(1024)                                                             \
        NAME(SkLaunch g, int T, int64_t w_row_bytes, int nb, const uint8_t *__restrict__ act, int64_t act_rb,      \
             int ncols, int32_t *__restrict__ sub) {                                                               \
        sqs_impl<WT, SW, SUBS>(g, T, w_row_bytes, nb, act, act_rb, ncols, sub);                                     \
    }
SQS_KERNEL(ghip_sqs_q4_K_w2, 12, 2, false)
SQS_KERNEL(ghip_sqs_q4_K_sub_w2, 12, 2, true)
SQS_KERNEL(ghip_sqs_q6_K_w2, 14, 2, false)
SQS_KERNEL(ghip_sqs_q6_K_sub_w2, 14, 2, true)

#define SQ_KERNEL(NAME, WT, SW, T, SUBS)                                                                           \
    extern "C" __global__ void __launch_bounds__(1024)                                                             \
        NAME(SkLaunch g, int64_t w_row_bytes, int nb, const uint8_t *__restrict__ act, int64_t act_rb, int ncols,  \
             int32_t *__restrict__ sub) {                                                                          \
        sq_impl<WT, SW, T, SUBS>(g, w_row_bytes, nb, act, act_rb, ncols, sub);                                      \
    }
#define SQ_KERNELS(TN, WT, SW, T)                                  \
    SQ_KERNEL(ghip_sq_##TN##_w##SW##_t##T, WT, SW, T, false)       \
    SQ_KERNEL(ghip_sq_##TN##_sub_w##SW##_t##T, WT, SW, T, true)
// (T = 4 at SW = 2 and T = 2 at SW = 4 exceed 128 VGPRs and spill)
SQ_KERNELS(q4_K, 12, 2, 1)
SQ_KERNELS(q4_K, 12, 2, 2)
SQ_KERNELS(q4_K, 12, 4, 1)
SQ_KERNELS(q6_K, 14, 2, 1)
SQ_KERNELS(q6_K, 14, 2, 2)
SQ_KERNELS(q6_K, 14, 4, 1)

// The K-slices' partials of up to 4 matrices added in slice order:
// dst[c][r] = sum_k part[k][c][r]; one lane per (matrix, column, row).  Here
// tile0 of a member is its first row in the launch's concatenated rows.
extern "C" __global__ void __launch_bounds__(256)
    ghip_sk_reduce(SkLaunch g, int ncols, int64_t total) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= total) return;
    int i = 0;
#pragma unroll
    for (int k = 1; k < 4; k++)
        if (k < g.n && id >= (int64_t)g.m[k].tile0 * ncols) i = k;
    const SkMember &mb = g.m[i];
    const int64_t e = id - (int64_t)mb.tile0 * ncols;  // (column, row) in the matrix
    const int c = (int)(e / mb.rows), r = (int)(e - (int64_t)c * mb.rows);
    const int64_t plane = (int64_t)ncols * mb.rows;
    float s = 0.0f;
    for (int k0 = 0; k0 < g.nks; k0 += 8) {  // 8 loads in flight, added in order
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = k0 + k < g.nks ? mb.part[(k0 + k) * plane + e] : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (k0 + k < g.nks) s = k0 + k == 0 ? v[k] : s + v[k];
    }
    mb.dst[(int64_t)c * mb.ldd + r] = s;
}
