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
