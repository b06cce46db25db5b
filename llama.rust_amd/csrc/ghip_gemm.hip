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
// sc = 8*sc_hi + sc_lo (3 bits each) and the weights are expanded into two
// int8 planes q4*sc_hi and q4*sc_lo (both <= 105):
//   iacc = 8 * (A . W_hi) + (A . W_lo)      -- two int8 MFMA chains, exact int32.
// imin is a K=16 contraction of mn (<= 63) with bsum16 (|.| <= 2032), both
// exact in fp16, with sums < 2^24: one v_mfma_f32_32x32x16_f16 per tile, exact.
//
// Tiling: a 256-thread workgroup owns a 128-token x 64-row output tile; its
// four wavefronts each own 32 tokens x 64 rows (two MFMA tiles of 32 x 32).
// Two workgroups share a CU (78 KB of LDS each, two wavefronts per SIMD) and
// run out of phase, so one's scaling epilogue overlaps the other's MFMAs.  Per super-block the workgroup expands the
// weights ONCE into the two planes in LDS (double-buffered: super-block b+1
// is expanded while b is multiplied); every wavefront streams its own
// activation codes from global memory (L2) straight into registers, one
// super-block ahead.
//
// K order inside a super-block: 16-element piece p = 2*(2*c + nh) + h holds
// elements 64c + 32nh + 16h + [0, 16) -- bytes 32c + 16h + [0,16) of the
// Q4_K qs, low nibbles for nh = 0, high for nh = 1 -- so MFMA K-step
// ks = 2c + nh (32 elements) lies in one sub-block (scale index ks), and lane
// half h of both operands carries piece 2*ks + h.
#include "ghip_common.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int BM = 128, BN = 64;
constexpr int PROW = 256;  // LDS row (bytes) of a weight plane; pieces XOR-swizzled by row

// LDS byte offset of 16-element piece p of plane row r: piece p is stored at
// slot p ^ (r % 16), so the 32 rows a wavefront half reads at one piece index
// fall in 8 distinct 16-byte bank groups per 8 lanes.
DEV int piece_off(int r, int p) { return r * PROW + 16 * (p ^ (r & 15)); }

struct GemmStage {
    uint8_t wlo[BN * PROW];  // q4 * sc_lo  [row][k]  (k in piece order)
    uint8_t whi[BN * PROW];  // q4 * sc_hi  [row][k]
    _Float16 bs[BM * 16];    // bsum16 as f16                [token][16]
    _Float16 mn[BN * 16];    // mn[s] at k = 2s, 2s+1, f16   [row][16]
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

// c ? v : 0 on a value (a select between two lvalues would take addresses
// and keep the prefetch arrays out of registers)
DEV uint4 keep_if(bool c, uint4 v) {
    const uint32_t m = c ? 0xffffffffu : 0u;
    return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}

// Four packed nibbles (one per byte) times a 3-bit scale: each byte product is
// <= 105, so two 16-bit lane multiplies (v_pk_mul_lo_u16) carry nothing
// across bytes.
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
DEV uint32_t mul_bytes(uint32_t nib, uint32_t s) {
    const us2 a = __builtin_bit_cast(us2, nib);
    const us2 r = a * (us2){(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, r);
}

// Weight prefetch of one super-block: thread t owns row t/4 and qs chunk
// t%4 (32 bytes), and decodes the header; the epilogue data of token t/2
// (bsum16[8*(t%2) .. +7] and d) come with it.
struct PrefetchW {
    uint4 q0, q1;  // qs bytes 32c .. 32c+31 of row t/4, c = t%4
    uint4 hd;      // header
    uint4 bsv;     // bsum16[8*(t%2) .. +7] of token t/2
    uint32_t ad;   // the token's d
};

// wrow: this thread's weight row (t/4, clamped); arow: its token row (t/2, clamped)
DEV void prefetch_w(PrefetchW &P, const uint8_t *__restrict__ wrow, const uint8_t *__restrict__ arow, int b) {
    const int c = threadIdx.x & 3;
    const uint8_t *blk = wrow + b * Q4K_BYTES;
    P.q0 = ld16(blk + 16 + 32 * c);
    P.q1 = ld16(blk + 32 + 32 * c);
    P.hd = ld16(blk);
    const uint8_t *A = arow + b * Q8K_BYTES;
    P.bsv = ld16(A + 260 + 16 * (threadIdx.x & 1));
    P.ad = ld4(A);
}

// Expand a prefetched super-block into the planes of stage S.
DEV void store_w(GemmStage &S, const PrefetchW &P, int N, int n0, int M, int m0) {
    const int t = threadIdx.x, r = t >> 2, c = t & 3;
    const int tok = t >> 1, half = t & 1;
    const bool nv = n0 + r < N, mv = m0 + tok < M;
    const uint4 hd = keep_if(nv, P.hd);
    int sc0, mn0, sc1, mn1;
    scale_min_k4(hd.y, hd.z, hd.w, 2 * c, sc0, mn0);
    scale_min_k4(hd.y, hd.z, hd.w, 2 * c + 1, sc1, mn1);
    const uint4 q0 = keep_if(nv, P.q0), q1 = keep_if(nv, P.q1);
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    // pieces of chunk c: (nh, h) -> k offset 64c + 32nh + 16h; bytes 16h.. of the chunk
#pragma unroll
    for (int nh = 0; nh < 2; nh++) {
        const uint32_t slo = nh ? (uint32_t)(sc1 & 7) : (uint32_t)(sc0 & 7);
        const uint32_t shi = nh ? (uint32_t)(sc1 >> 3) : (uint32_t)(sc0 >> 3);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t w = qw[4 * h + e];
                const uint32_t nib = nh ? ((w >> 4) & 0x0f0f0f0f) : (w & 0x0f0f0f0f);
                lo[e] = mul_bytes(nib, slo);
                hi[e] = mul_bytes(nib, shi);
            }
            const int off = piece_off(r, 4 * c + 2 * nh + h);  // elements 64c + 32nh + 16h ..
            *reinterpret_cast<uint4 *>(&S.wlo[off]) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            *reinterpret_cast<uint4 *>(&S.whi[off]) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        }
    }
    // mn of sub-blocks 2c, 2c+1 at k = 4c .. 4c+3
    const uint32_t m01 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)mn0) * 0x10001u;
    const uint32_t m23 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)mn1) * 0x10001u;
    *reinterpret_cast<uint2 *>(&S.mn[r * 16 + 4 * c]) = make_uint2(m01, m23);
    if (c == 0) {
        S.dw[r] = h2f(hd.x);
        S.dmin[r] = h2f(hd.x >> 16);
    }
    // token t/2: bsum16[8*half .. +7] -> f16, and d
    const uint4 bv = keep_if(mv, P.bsv);
    const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
    v8h hv;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        hv[2 * e] = (_Float16)(float)(int16_t)(bw[e] & 0xffff);
        hv[2 * e + 1] = (_Float16)(float)(int16_t)(bw[e] >> 16);
    }
    *reinterpret_cast<v8h *>(&S.bs[tok * 16 + 8 * half]) = hv;
    if (half == 0) S.da[tok] = mv ? __uint_as_float(P.ad) : 0.0f;
}

// Piece 2*ks + h of this lane's token (elements 32ks + 16h .. +15) of
// super-block b; p points at the token's codes + 16h (rows past M re-read a
// valid token; their results are never stored).
DEV v4i load_piece(const uint8_t *__restrict__ p, int b, int ks) {
    const uint4 v = ld16(p + b * Q8K_BYTES + 32 * ks);
    return v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
}

template <bool SUBSUMS>
__device__ __forceinline__ void gemm_q4K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
                                              const uint8_t *__restrict__ act, int64_t act_row_bytes, int M,
                                              float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    GemmSmem &SM = *reinterpret_cast<GemmSmem *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave;  // 4 wavefronts along the tokens
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
    const int mrow = m0 + 32 * wm + li;  // this lane's token for the A operand

    v16f out[2];
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
        for (int v = 0; v < 16; v++) out[c][v] = 0.0f;

    const uint8_t *wrow = W + (int64_t)min(n0 + (tid >> 2), N - 1) * w_row_bytes;
    const uint8_t *arow = act + (int64_t)min(m0 + (tid >> 1), M - 1) * act_row_bytes;
    const uint8_t *apiece = act + (int64_t)min(mrow, M - 1) * act_row_bytes + 4 + 16 * h;

    v4i A[8];
    PrefetchW P;
    prefetch_w(P, wrow, arow, 0);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) A[ks] = load_piece(apiece, 0, ks);
    store_w(SM.st[0], P, N, n0, M, m0);
    __syncthreads();

    for (int b = 0; b < nb; b++) {
        // multiply super-block b from stage b&1; meanwhile super-block b+1's
        // weights go to P (then the other stage) and each activation piece,
        // once its MFMAs are issued, is reloaded with b+1's
        const GemmStage &S = SM.st[b & 1];
        const bool more = b + 1 < nb;
        if (more) prefetch_w(P, wrow, arow, b + 1);
        const v16i zi = {};
        v16i acc_lo[2], acc_hi[2];
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
#pragma unroll
            for (int tn = 0; tn < 2; tn++) {
                const int nl = tn * 32 + li;
                const int off = piece_off(nl, 2 * ks + h);
                const v4i blo = *reinterpret_cast<const v4i *>(&S.wlo[off]);
                const v4i bhi = *reinterpret_cast<const v4i *>(&S.whi[off]);
                acc_lo[tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[ks], blo, ks ? acc_lo[tn] : zi, 0, 0, 0);
                acc_hi[tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[ks], bhi, ks ? acc_hi[tn] : zi, 0, 0, 0);
            }
            if (more) A[ks] = load_piece(apiece, b + 1, ks);
        }
        // ---- min term (K = 16 bsum16 slots, one f16 MFMA per tile) and epilogue
        const int kq = 8 * h;
        const v8h Am = *reinterpret_cast<const v8h *>(&S.bs[(wm * 32 + li) * 16 + kq]);
        float dav[16];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 d4 = *reinterpret_cast<const float4 *>(&S.da[wm * 32 + 8 * g + 4 * h]);
            dav[4 * g] = d4.x;
            dav[4 * g + 1] = d4.y;
            dav[4 * g + 2] = d4.z;
            dav[4 * g + 3] = d4.w;
        }
        const v16f zf = {};
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int nl = tn * 32 + li;
            const float dw = S.dw[nl], dmin = S.dmin[nl];
            const v8h Bm = *reinterpret_cast<const v8h *>(&S.mn[nl * 16 + kq]);
            const v16f accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(Am, Bm, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int iacc = (acc_hi[tn][v] << 3) + acc_lo[tn][v];
                const float im = accm[v];
                if (SUBSUMS) {
                    const int ml = wm * 32 + crow(v, lane);
                    if (m0 + ml < M && n0 + nl < N) {
                        int32_t *sp = sub + (((int64_t)(m0 + ml) * N + (n0 + nl)) * nb + b) * 2;
                        sp[0] = iacc;
                        sp[1] = (int)im;
                    }
                }
                const float t = fmaf(dw, (float)iacc, -(dmin * im));
                out[tn][v] = fmaf(dav[v], t, out[tn][v]);
            }
        }
        if (more) store_w(SM.st[(b + 1) & 1], P, N, n0, M, m0);
        __syncthreads();
    }
    // ---- store: for each v, the 32 lanes of a half write 32 consecutive floats
#pragma unroll
    for (int tn = 0; tn < 2; tn++) {
        const int n = n0 + tn * 32 + li;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + wm * 32 + crow(v, lane);
            if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tn][v];
        }
    }
}

extern "C" __global__ void __launch_bounds__(256, 2)
ghip_gemm_q4_K(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, const uint8_t *__restrict__ act,
               int64_t act_row_bytes, int M, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    gemm_q4K_impl<false>(W, w_row_bytes, N, nb, act, act_row_bytes, M, dst, ldd, sub);
}
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_q4_K_sub(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, const uint8_t *__restrict__ act,
                   int64_t act_row_bytes, int M, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    gemm_q4K_impl<true>(W, w_row_bytes, N, nb, act, act_row_bytes, M, dst, ldd, sub);
}

static_assert(sizeof(GemmSmem) == 2 * (2 * BN * PROW + BM * 32 + BN * 32 + 4 * (BM + 2 * BN)), "LDS layout");
static_assert(sizeof(GemmSmem) == 79872, "host code launches with this LDS size");
