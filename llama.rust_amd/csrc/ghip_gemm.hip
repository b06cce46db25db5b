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
// sc = 8*sc_hi + sc_lo (3 bits each) and the weights are expanded in LDS into
// two int8 planes W_hi = q4*sc_hi and W_lo = q4*sc_lo (both <= 105):
//   iacc = 8 * (A . W_hi) + (A . W_lo)      -- two int8 MFMA chains, exact int32.
// imin is a K=16 contraction of mn (<= 63) with bsum16 (|.| <= 2032), both
// exact in fp16, with sums < 2^24: one v_mfma_f32_32x32x16_f16 per tile, exact.
//
// Tiling: a 256-thread workgroup owns a 128-token x 128-row output tile; its
// four wavefronts each own 64 x 64 (2 x 2 MFMA tiles of 32 x 32).  Per
// super-block the workgroup stages the activation codes, the two weight planes
// and the per-row/per-token scales in LDS, then runs 8 K-slices of 32.
#include "ghip_common.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int BM = 128, BN = 128;
constexpr int ROWB = 256 + 16;  // LDS row stride (bytes) of the int8 planes

struct GemmSmem {
    uint8_t a[BM * ROWB];     // activation codes  [token][k]
    uint8_t wlo[BN * ROWB];   // q4 * sc_lo         [row][k]
    uint8_t whi[BN * ROWB];   // q4 * sc_hi         [row][k]
    _Float16 bs[BM * 16];     // bsum16 as f16      [token][16]
    _Float16 mn[BN * 16];     // mn[s] at k = 2s,2s+1 as f16 [row][16]
    float da[BM];
    float dw[BN];
    float dmin[BN];
};

// C layout of a 32x32 MFMA tile: lane l holds column j = l % 32 and rows
// i = 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.
DEV int crow(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_q4_K(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
               const uint8_t *__restrict__ act, int64_t act_row_bytes, int M,
               float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    GemmSmem &S = *reinterpret_cast<GemmSmem *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n_tiles_n = (N + BN - 1) / BN;
    const int m0 = (blockIdx.x / n_tiles_n) * BM;
    const int n0 = (blockIdx.x % n_tiles_n) * BN;

    v16f out[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) out[a][b][v] = 0.0f;

    for (int b = 0; b < nb; b++) {
        __syncthreads();  // previous super-block's LDS reads are done
        // ---- activations: 128 tokens x 256 codes, 16 B per load
        for (int c = tid; c < BM * 16; c += 256) {
            const int m = c >> 4, t = c & 15;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (m0 + m < M) v = ld16(act + (int64_t)(m0 + m) * act_row_bytes + (int64_t)b * Q8K_BYTES + 4 + 16 * t);
            *reinterpret_cast<uint4 *>(&S.a[m * ROWB + 16 * t]) = v;
        }
        if (tid < BM) {
            const int m = tid;
            float d = 0.0f;
            int16_t bsv[16];
            for (int k = 0; k < 16; k++) bsv[k] = 0;
            if (m0 + m < M) {
                const uint8_t *A = act + (int64_t)(m0 + m) * act_row_bytes + (int64_t)b * Q8K_BYTES;
                d = __uint_as_float(ld4(A));
                __builtin_memcpy(bsv, A + 260, 32);
            }
            S.da[m] = d;
            for (int k = 0; k < 16; k++) S.bs[m * 16 + k] = (_Float16)(float)bsv[k];
        }
        // ---- weights: (row, pair g) tasks; each expands 64 elements into both planes
        for (int task = tid; task < BN * 4; task += 256) {
            const int r = task >> 2, g = task & 3;
            uint4 hdr = make_uint4(0, 0, 0, 0), q0 = hdr, q1 = hdr;
            if (n0 + r < N) {
                const uint8_t *blk = W + (int64_t)(n0 + r) * w_row_bytes + (int64_t)b * Q4K_BYTES;
                hdr = ld16(blk);
                q0 = ld16(blk + 16 + 32 * g);
                q1 = ld16(blk + 32 + 32 * g);
            }
            int sc0, m0v, sc1, m1v;
            scale_min_k4(hdr.y, hdr.z, hdr.w, 2 * g, sc0, m0v);
            scale_min_k4(hdr.y, hdr.z, hdr.w, 2 * g + 1, sc1, m1v);
            const uint32_t qs[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            uint32_t lo_lo[8], lo_hi[8], hi_lo[8], hi_hi[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t nl = qs[k] & 0x0f0f0f0f, nh = (qs[k] >> 4) & 0x0f0f0f0f;
                lo_lo[k] = nl * (uint32_t)(sc0 & 7);  // bytes stay < 256: no carries
                hi_lo[k] = nl * (uint32_t)(sc0 >> 3);
                lo_hi[k] = nh * (uint32_t)(sc1 & 7);
                hi_hi[k] = nh * (uint32_t)(sc1 >> 3);
            }
            uint8_t *plo = &S.wlo[r * ROWB + 64 * g];
            uint8_t *phi = &S.whi[r * ROWB + 64 * g];
            *reinterpret_cast<uint4 *>(plo + 0) = make_uint4(lo_lo[0], lo_lo[1], lo_lo[2], lo_lo[3]);
            *reinterpret_cast<uint4 *>(plo + 16) = make_uint4(lo_lo[4], lo_lo[5], lo_lo[6], lo_lo[7]);
            *reinterpret_cast<uint4 *>(plo + 32) = make_uint4(lo_hi[0], lo_hi[1], lo_hi[2], lo_hi[3]);
            *reinterpret_cast<uint4 *>(plo + 48) = make_uint4(lo_hi[4], lo_hi[5], lo_hi[6], lo_hi[7]);
            *reinterpret_cast<uint4 *>(phi + 0) = make_uint4(hi_lo[0], hi_lo[1], hi_lo[2], hi_lo[3]);
            *reinterpret_cast<uint4 *>(phi + 16) = make_uint4(hi_lo[4], hi_lo[5], hi_lo[6], hi_lo[7]);
            *reinterpret_cast<uint4 *>(phi + 32) = make_uint4(hi_hi[0], hi_hi[1], hi_hi[2], hi_hi[3]);
            *reinterpret_cast<uint4 *>(phi + 48) = make_uint4(hi_hi[4], hi_hi[5], hi_hi[6], hi_hi[7]);
            S.mn[r * 16 + 4 * g + 0] = (_Float16)(float)m0v;
            S.mn[r * 16 + 4 * g + 1] = (_Float16)(float)m0v;
            S.mn[r * 16 + 4 * g + 2] = (_Float16)(float)m1v;
            S.mn[r * 16 + 4 * g + 3] = (_Float16)(float)m1v;
            if (g == 0) {
                S.dw[r] = h2f(hdr.x);
                S.dmin[r] = h2f(hdr.x >> 16);
            }
        }
        __syncthreads();

        // ---- MFMA: 8 K-slices of 32, two planes
        v16i acc_lo[2][2], acc_hi[2][2];
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc_lo[a][c][v] = acc_hi[a][c][v] = 0;
        const int li = lane & 31, kh = 16 * (lane >> 5);
#pragma unroll 1
        for (int ks = 0; ks < 8; ks++) {
            v4i A[2], Blo[2], Bhi[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                A[t] = *reinterpret_cast<const v4i *>(&S.a[(wm * 64 + t * 32 + li) * ROWB + 32 * ks + kh]);
                Blo[t] = *reinterpret_cast<const v4i *>(&S.wlo[(wn * 64 + t * 32 + li) * ROWB + 32 * ks + kh]);
                Bhi[t] = *reinterpret_cast<const v4i *>(&S.whi[(wn * 64 + t * 32 + li) * ROWB + 32 * ks + kh]);
            }
#pragma unroll
            for (int tm = 0; tm < 2; tm++)
#pragma unroll
                for (int tn = 0; tn < 2; tn++) {
                    acc_lo[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[tm], Blo[tn], acc_lo[tm][tn], 0, 0, 0);
                    acc_hi[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[tm], Bhi[tn], acc_hi[tm][tn], 0, 0, 0);
                }
        }
        // ---- min term (K = 16 bsum16 slots, one f16 MFMA per tile) and epilogue
        const int kq = 8 * (lane >> 5);
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int nl = wn * 64 + tn * 32 + li;
            const float dw = S.dw[nl], dmin = S.dmin[nl];
            const v8h Bm = *reinterpret_cast<const v8h *>(&S.mn[nl * 16 + kq]);
#pragma unroll
            for (int tm = 0; tm < 2; tm++) {
                const v8h Am = *reinterpret_cast<const v8h *>(&S.bs[(wm * 64 + tm * 32 + li) * 16 + kq]);
                v16f z;
#pragma unroll
                for (int v = 0; v < 16; v++) z[v] = 0.0f;
                const v16f accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(Am, Bm, z, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int ml = wm * 64 + tm * 32 + crow(v, lane);
                    const int iacc = (acc_hi[tm][tn][v] << 3) + acc_lo[tm][tn][v];
                    const float im = accm[v];
                    if (sub && m0 + ml < M && n0 + nl < N) {
                        int32_t *sp = sub + (((int64_t)(m0 + ml) * N + (n0 + nl)) * nb + b) * 2;
                        sp[0] = iacc;
                        sp[1] = (int)im;
                    }
                    const float t = fmaf(dw, (float)iacc, -(dmin * im));
                    out[tm][tn][v] = fmaf(S.da[ml], t, out[tm][tn][v]);
                }
            }
        }
    }
    // ---- store
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int n = n0 + wn * 64 + tn * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + wm * 64 + tm * 32 + crow(v, lane);
                if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tm][tn][v];
            }
        }
}

static_assert(sizeof(GemmSmem) == 114176, "host code launches with this LDS size");
