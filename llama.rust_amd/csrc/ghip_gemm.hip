// ghip_gemm.hip -- prefill MUL_MAT for Q4_K weights x Q8_K activations on the
// int8 matrix cores (v_mfma_i32_32x32x32_i8).
//
// Per (token m, weight row n, super-block b) the reference forms two exact
// integers (repack.rs:1692-1770, compute.rs:5322):
//   iacc = sum_e  q4[n,e] * sc[n,s(e)] * q8[m,e]      (6-bit sub-block scales sc)
//   imin = sum_s  mn[n,s] * (bsum16[m,2s] + bsum16[m,2s+1])
// and out[m,n] = sum_b  da[m,b] * (dw[n,b] * iacc - dmin[n,b] * imin).
//
// q4*sc reaches 945, too wide for an int8 operand, so the scale is split
// sc = 8*sc_hi + sc_lo (3 bits each) and each weight operand is expanded in
// registers into two int8 planes q4*sc_hi and q4*sc_lo (both <= 105):
//   iacc = 8 * (A . W_hi) + (A . W_lo)      -- two int8 MFMA chains, exact int32.
// imin is a K=16 contraction of mn (<= 63) with bsum16 (|.| <= 2032), both
// exact in fp16, with sums < 2^24: one v_mfma_f32_32x32x16_f16 per tile, exact.
//
// Tiling: a 256-thread workgroup owns a 128-token x 128-row output tile; its
// four wavefronts each own 64 x 64 (2 x 2 MFMA tiles of 32 x 32).  The
// activation codes and the raw Q4_K blocks of one super-block are staged in
// LDS (double-buffered: the global loads of super-block b+1 are in flight
// while b is multiplied).  K-step ks (32 elements) of super-block b is
// qs-chunk c = ks/2, low nibbles for even ks and high for odd, so its 32
// elements share one sub-block scale; lane half h takes bytes 16h..16h+15 of
// the chunk, and the activation operand takes the same 16 elements.
#include "ghip_common.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int BM = 128, BN = 128;
constexpr int AROW = 256 + 16;  // LDS row stride (bytes) of the activation codes
constexpr int QROW = 128 + 16;  // LDS row stride (bytes) of the weight nibbles

struct GemmStage {
    uint8_t a[BM * AROW];    // activation codes            [token][k]
    uint8_t q[BN * QROW];    // Q4_K qs (nibbles)           [row][128]
    _Float16 bs[BM * 16];    // bsum16 as f16               [token][16]
    _Float16 mn[BN * 16];    // mn[s] at k = 2s, 2s+1, f16  [row][16]
    uint8_t sc[BN * 8];      // sub-block scales (6 bits)   [row][8]
    float da[BM];
    float dw[BN];
    float dmin[BN];
};
struct GemmSmem {
    GemmStage st[2];
};

// C layout of a 32x32 MFMA tile: lane l holds column j = l % 32 and rows
// i = 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.
DEV int crow(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// Global prefetch of one super-block for the workgroup, in two register
// batches that are written to the free LDS stage at different points of the
// previous super-block's multiply (fewer live registers).
struct PrefetchA {
    uint4 a[8];  // activation codes: token tid/2, 128-byte half tid%2
    uint4 ab;    // bsum16 [8*half .. 8*half+7] of token tid/2
    uint32_t ad; // activation d
};
struct PrefetchW {
    uint4 w[4];  // weight: row tid/2, qs bytes 64*(tid%2) .. +63
    uint4 wh;    // header of row tid/2
};

DEV void prefetch_a(PrefetchA &P, const uint8_t *__restrict__ act, int64_t act_row_bytes, int M, int m0, int b) {
    const int tid = threadIdx.x;
    const int r = tid >> 1, half = tid & 1;
    // clamped rows re-read a valid token; their codes are never stored
    const int m = min(m0 + r, M - 1);
    const uint8_t *A = act + (int64_t)m * act_row_bytes + (int64_t)b * Q8K_BYTES;
#pragma unroll
    for (int k = 0; k < 8; k++) P.a[k] = ld16(A + 4 + 128 * half + 16 * k);
    P.ab = ld16(A + 260 + 16 * half);
    P.ad = ld4(A);
}

DEV void prefetch_w(PrefetchW &P, const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int n0, int b) {
    const int tid = threadIdx.x;
    const int r = tid >> 1, half = tid & 1;
    const int n = min(n0 + r, N - 1);
    const uint8_t *blk = W + (int64_t)n * w_row_bytes + (int64_t)b * Q4K_BYTES;
#pragma unroll
    for (int k = 0; k < 4; k++) P.w[k] = ld16(blk + 16 + 64 * half + 16 * k);
    P.wh = ld16(blk);
}

// c ? v : 0 on a value (a select between two lvalues would take addresses
// and keep the prefetch arrays out of registers)
DEV uint4 keep_if(bool c, uint4 v) {
    const uint32_t m = c ? 0xffffffffu : 0u;
    return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}

DEV void store_a(GemmStage &S, const PrefetchA &P, int M, int m0) {
    const int tid = threadIdx.x;
    const int r = tid >> 1, half = tid & 1;
    const bool mv = m0 + r < M;
#pragma unroll
    for (int k = 0; k < 8; k++) *reinterpret_cast<uint4 *>(&S.a[r * AROW + 128 * half + 16 * k]) = keep_if(mv, P.a[k]);
    // 8 bsum16 values (int16) of this half -> f16
    const uint4 v = keep_if(mv, P.ab);
    const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
    v8h hv;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        hv[2 * e] = (_Float16)(float)(int16_t)(wv[e] & 0xffff);
        hv[2 * e + 1] = (_Float16)(float)(int16_t)(wv[e] >> 16);
    }
    *reinterpret_cast<v8h *>(&S.bs[r * 16 + 8 * half]) = hv;
    if (half == 0) S.da[r] = mv ? __uint_as_float(P.ad) : 0.0f;
}

DEV void store_w(GemmStage &S, const PrefetchW &P, int N, int n0) {
    const int tid = threadIdx.x;
    const int r = tid >> 1, half = tid & 1;
    const bool nv = n0 + r < N;
#pragma unroll
    for (int k = 0; k < 4; k++) *reinterpret_cast<uint4 *>(&S.q[r * QROW + 64 * half + 16 * k]) = keep_if(nv, P.w[k]);
    // header: this half decodes sub-blocks 4*half .. 4*half+3
    const uint4 hd = keep_if(nv, P.wh);
    uint32_t scb = 0;
    v8h mv8;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        int sc, m;
        scale_min_k4(hd.y, hd.z, hd.w, 4 * half + t, sc, m);
        scb |= (uint32_t)sc << (8 * t);
        mv8[2 * t] = mv8[2 * t + 1] = (_Float16)(float)m;
    }
    *reinterpret_cast<uint32_t *>(&S.sc[r * 8 + 4 * half]) = scb;
    *reinterpret_cast<v8h *>(&S.mn[r * 16 + 8 * half]) = mv8;
    if (half == 0) {
        S.dw[r] = h2f(hd.x);
        S.dmin[r] = h2f(hd.x >> 16);
    }
}

template <bool SUBSUMS>
__device__ __forceinline__ void gemm_q4K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
                                              const uint8_t *__restrict__ act, int64_t act_row_bytes, int M,
                                              float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    GemmSmem &SM = *reinterpret_cast<GemmSmem *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, h = lane >> 5;

    // Tile order: the M-tiles of one N-tile are consecutive, and consecutive
    // tile ids go to the same XCD (workgroups are dealt to the 8 XCDs round
    // robin), so one XCD's L2 serves a weight tile to all its token tiles.
    const int n_tiles_m = (M + BM - 1) / BM, n_tiles_n = (N + BN - 1) / BN;
    const int total = n_tiles_m * n_tiles_n;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int m0 = (id % n_tiles_m) * BM;
    const int n0 = (id / n_tiles_m) * BN;

    v16f out[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int v = 0; v < 16; v++) out[a][c][v] = 0.0f;

    {
        PrefetchA PA;
        PrefetchW PW;
        prefetch_a(PA, act, act_row_bytes, M, m0, 0);
        prefetch_w(PW, W, w_row_bytes, N, n0, 0);
        store_a(SM.st[0], PA, M, m0);
        store_w(SM.st[0], PW, N, n0);
    }
    __syncthreads();

    for (int b = 0; b < nb; b++) {
        const GemmStage &S = SM.st[b & 1];
        GemmStage &Snext = SM.st[(b + 1) & 1];
        const bool more = b + 1 < nb;
        PrefetchA PA;
        PrefetchW PW;
        if (more) prefetch_a(PA, act, act_row_bytes, M, m0, b + 1);

        v16i acc_lo[2][2], acc_hi[2][2];
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc_lo[a][c][v] = acc_hi[a][c][v] = 0;
#pragma unroll
        for (int c4 = 0; c4 < 4; c4++) {  // qs chunk: sub-blocks 2*c4 (low nibbles), 2*c4+1 (high)
            // next super-block: activations land in the free stage after chunk 0,
            // the weight loads are issued then and land after chunk 2
            if (more && c4 == 1) {
                store_a(Snext, PA, M, m0);
                prefetch_w(PW, W, w_row_bytes, N, n0, b + 1);
            }
            if (more && c4 == 3) store_w(Snext, PW, N, n0);
            v4i A[2][2];                 // [nibble half][m tile]
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint8_t *ap = &S.a[(wm * 64 + t * 32 + li) * AROW + 64 * c4 + 16 * h];
                A[0][t] = *reinterpret_cast<const v4i *>(ap);
                A[1][t] = *reinterpret_cast<const v4i *>(ap + 32);
            }
            v4i Blo[2][2], Bhi[2][2];  // [nibble half][n tile]
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int nl = wn * 64 + t * 32 + li;
                const uint4 qv = *reinterpret_cast<const uint4 *>(&S.q[nl * QROW + 32 * c4 + 16 * h]);
                const uint32_t scp = *reinterpret_cast<const uint16_t *>(&S.sc[nl * 8 + 2 * c4]);
                const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
                for (int nh = 0; nh < 2; nh++) {
                    const uint32_t s = (scp >> (8 * nh)) & 0xff;
                    const uint32_t slo = s & 7, shi = s >> 3;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t nib = nh ? ((qw[e] >> 4) & 0x0f0f0f0f) : (qw[e] & 0x0f0f0f0f);
                        Blo[nh][t][e] = (int)(nib * slo);  // bytes stay <= 105: no carries
                        Bhi[nh][t][e] = (int)(nib * shi);
                    }
                }
            }
#pragma unroll
            for (int nh = 0; nh < 2; nh++)
#pragma unroll
                for (int tm = 0; tm < 2; tm++)
#pragma unroll
                    for (int tn = 0; tn < 2; tn++) {
                        acc_lo[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[nh][tm], Blo[nh][tn], acc_lo[tm][tn], 0, 0, 0);
                        acc_hi[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[nh][tm], Bhi[nh][tn], acc_hi[tm][tn], 0, 0, 0);
                    }
        }
        // ---- min term (K = 16 bsum16 slots, one f16 MFMA per tile) and epilogue
        const int kq = 8 * h;
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int nl = wn * 64 + tn * 32 + li;
            const float dw = S.dw[nl], dmin = S.dmin[nl];
            const v8h Bm = *reinterpret_cast<const v8h *>(&S.mn[nl * 16 + kq]);
#pragma unroll
            for (int tm = 0; tm < 2; tm++) {
                const v8h Am = *reinterpret_cast<const v8h *>(&S.bs[(wm * 64 + tm * 32 + li) * 16 + kq]);
                v16f zf;
#pragma unroll
                for (int v = 0; v < 16; v++) zf[v] = 0.0f;
                const v16f accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(Am, Bm, zf, 0, 0, 0);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 da4 = *reinterpret_cast<const float4 *>(&S.da[wm * 64 + tm * 32 + 8 * g + 4 * h]);
                    const float dav[4] = {da4.x, da4.y, da4.z, da4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int v = 4 * g + r;
                        const int iacc = (acc_hi[tm][tn][v] << 3) + acc_lo[tm][tn][v];
                        const float im = accm[v];
                        if (SUBSUMS) {
                            const int ml = wm * 64 + tm * 32 + crow(v, lane);
                            if (m0 + ml < M && n0 + nl < N) {
                                int32_t *sp = sub + (((int64_t)(m0 + ml) * N + (n0 + nl)) * nb + b) * 2;
                                sp[0] = iacc;
                                sp[1] = (int)im;
                            }
                        }
                        const float t = fmaf(dw, (float)iacc, -(dmin * im));
                        out[tm][tn][v] = fmaf(dav[r], t, out[tm][tn][v]);
                    }
                }
            }
        }
        __syncthreads();
    }
    // ---- store
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int n = n0 + wn * 64 + tn * 32 + li;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + wm * 64 + tm * 32 + crow(v, lane);
                if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tm][tn][v];
            }
        }
}

extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_q4_K(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, const uint8_t *__restrict__ act,
               int64_t act_row_bytes, int M, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    gemm_q4K_impl<false>(W, w_row_bytes, N, nb, act, act_row_bytes, M, dst, ldd, sub);
}
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_q4_K_sub(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, const uint8_t *__restrict__ act,
                   int64_t act_row_bytes, int M, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    gemm_q4K_impl<true>(W, w_row_bytes, N, nb, act, act_row_bytes, M, dst, ldd, sub);
}

static_assert(sizeof(GemmSmem) == 2 * (BM * AROW + BN * QROW + BM * 32 + BN * 32 + BN * 8 + 4 * (BM + 2 * BN)),
              "LDS layout");
static_assert(sizeof(GemmSmem) == 128000, "host code launches with this LDS size");
