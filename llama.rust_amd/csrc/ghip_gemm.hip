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
#include "ghip_common.h"
#include "ghip_q8k.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// C layout of a 32x32 MFMA tile: lane l holds column j = l % 32 and rows
// i = 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.
DEV int crow(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// Four packed nibbles (one per byte) times a 3-bit scale: each byte product is
// <= 105, so two 16-bit lane multiplies (v_pk_mul_lo_u16) carry nothing
// across bytes.
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
DEV uint32_t mul_bytes(uint32_t nib, uint32_t s) {
    const us2 a = __builtin_bit_cast(us2, nib);
    const us2 r = a * (us2){(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, r);
}

// GEMM activation layout, written by ghip_gemm_act_layout from Q8_K rows
// (tokens padded to a multiple of 128, so every staging load is in bounds):
//   codes [Mpad][K] int8 | bsT [nb][Mpad][16] bsum16 as f16 | dT [nb][Mpad] f32
// One wavefront per (token, super-block): lane l moves codes 4l .. 4l+3,
// lanes 0..15 the sixteen bsum16 and lane 0 the block scale.
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_act_layout(const uint8_t *__restrict__ q8k, int64_t row_bytes, int M, int Mpad, int nb,
                     int8_t *__restrict__ codes, _Float16 *__restrict__ bsT, float *__restrict__ dT) {
    const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (task >= (int64_t)M * nb) return;
    const int m = (int)(task / nb), b = (int)(task % nb);
    const uint8_t *blk = q8k + (int64_t)m * row_bytes + (int64_t)b * Q8K_BYTES;
    const int64_t K = (int64_t)nb * QK_K;
    *reinterpret_cast<uint32_t *>(codes + (int64_t)m * K + b * QK_K + 4 * lane) = ld4(blk + 4 + 4 * lane);
    if (lane < 16) bsT[((int64_t)b * Mpad + m) * 16 + lane] = (_Float16)(float)(int16_t)ld2(blk + 260 + 2 * lane);
    if (lane == 0) dT[(int64_t)b * Mpad + m] = __uint_as_float(ld4(blk));
}

// Prefill GEMM: a 512-thread workgroup (one CU) owns 128 tokens x 128 rows,
// each of its eight wavefronts 64 tokens x 32 rows (two 32 x 32 tiles).  Per
// super-block the workgroup's operands arrive in LDS by direct global->LDS
// loads (no registers, no vector ALU), double-buffered so super-block b+1
// lands while b is multiplied:
//   act   activation codes [token][256], 16-byte slots swizzled by token % 16
//   wraw  raw Q4_K qs [row][128], 16-byte slots swizzled by row % 8
//   hdr   Q4_K header [row][16] (d, dmin, packed 6-bit scales and mins)
//   bs/da bsum16 (f16) and block scale of every token
// Each wavefront decodes its rows' scales from hdr and expands the raw
// nibbles in registers right before the MFMAs: one 16-byte read of qs gives
// the B operands of two K-steps (low and high nibbles) for both planes
// q4*sc_lo and q4*sc_hi (sc = 8*sc_hi + sc_lo, each product <= 105), so
//   iacc = 8*(A.W_hi) + (A.W_lo)   in two exact int32 accumulator sets,
//   imin = sum_s mn_s * (bsum16_2s + bsum16_2s+1)   (one exact f16 MFMA),
//   out += da * (dw * iacc - dmin * imin)           (repack.rs:1692-1770).
namespace g3 {
constexpr int BN = 128;
template <int BM> struct Buf {  // operands of one super-block (two, alternating)
    uint8_t act[BM * 256];
    uint8_t wraw[BN * 128];
    uint8_t hdr[BN * 16];
};
template <int BM> struct Meta {  // per-token scaling data of one super-block (three, in a ring)
    _Float16 bs[BM * 16];
    float da[BM];
};
template <int BM> struct Smem {
    Buf<BM> buf[2];
    Meta<BM> meta[3];
};
}  // namespace g3


// BM = 128 tokens: 8 wavefronts, one workgroup per CU; BM = 64: 4
// wavefronts and half the LDS, two workgroups per CU.
template <int BM, bool SUBSUMS>
__device__ __forceinline__ void gemm_q4K_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
                                               const int8_t *__restrict__ codes, const _Float16 *__restrict__ bsT,
                                               const float *__restrict__ dT, int M, int Mpad,
                                               float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub,
                                               int nbs, int64_t zstride, int tile = -1) {
    constexpr int BN = g3::BN, NW = BM / 16, TPW = BM / 64;
    constexpr int WRI = 16 / NW;                    // wraw pieces per wavefront
    constexpr int DAW = BM == 128 ? 6 : 1;          // wavefront that loads da
    // split K: workgroup row blockIdx.y takes super-blocks [b0, b1) and writes
    // its partial sums to dst + blockIdx.y * zstride
    const int b0 = blockIdx.y * nbs, b1 = min(nb, b0 + nbs);
    dst += blockIdx.y * zstride;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    g3::Smem<BM> &SM = *reinterpret_cast<g3::Smem<BM> *>(smem_raw);
    g3::Buf<BM> *buf = SM.buf;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % TPW, wn = wave / TPW;  // 64-token slice, 32-row quarter
    const int li = lane & 31, h = lane >> 5;
    const int64_t K = (int64_t)nb * QK_K;

    const int n_tiles_m = (M + BM - 1) / BM, n_tiles_n = (N + BN - 1) / BN;
    const int total = n_tiles_m * n_tiles_n;
    // tile: this workgroup's tile of the matrix, tokens fastest (-1: from
    // blockIdx.x, with consecutive ids on one XCD)
    int id = tile;
    if (id < 0) {
        id = blockIdx.x;
        if (total % 8 == 0) id = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    }
    const int m0 = (id % n_tiles_m) * BM;
    const int n0 = (id / n_tiles_m) * BN;

    // ---- direct loads of super-block b into buf[b & 1]; wavefront w issues
    // act pieces 4w..4w+3 (4 tokens each), wraw pieces WRI*w .. (8 rows each),
    // hdr (w = 0, 1), bs (w = 2 .. 2 + BM/32 - 1) and da (w = DAW)
    // (weight rows past N re-read row N-1; tokens past M are padding)
    const uint8_t *wbase[WRI + 1];
    {
        // this lane's rows for the wraw pieces and the hdr piece
#pragma unroll
        for (int i = 0; i < WRI; i++) {
            const int row = 8 * (WRI * wave + i) + (lane >> 3);
            const int slot = (lane & 7) ^ (row & 7);
            wbase[i] = W + (int64_t)min(n0 + row, N - 1) * w_row_bytes + 16 + 16 * slot;
        }
        wbase[WRI] = W + (int64_t)min(n0 + 64 * (wave & 1) + lane, N - 1) * w_row_bytes;
    }
    const int8_t *abase[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int tok = 4 * (4 * wave + i) + (lane >> 4);
        const int slot = (lane & 15) ^ (tok & 15);
        abase[i] = codes + (int64_t)(m0 + tok) * K + 16 * slot;
    }
    auto issue = [&](int b) {
        g3::Buf<BM> &B = buf[b & 1];
        g3::Meta<BM> &Mt = SM.meta[b % 3];
#pragma unroll
        for (int i = 0; i < 4; i++) g2lds(abase[i] + (int64_t)b * QK_K, B.act + 1024 * (4 * wave + i));
#pragma unroll
        for (int i = 0; i < WRI; i++) g2lds(wbase[i] + (int64_t)b * Q4K_BYTES, B.wraw + 1024 * (WRI * wave + i));
        if (wave < 2) g2lds(wbase[WRI] + (int64_t)b * Q4K_BYTES, B.hdr + 1024 * wave);
        if (wave >= 2 && wave < 2 + BM / 32)
            g2lds(bsT + ((int64_t)b * Mpad + m0 + 32 * (wave - 2)) * 16 + 8 * lane,
                  reinterpret_cast<uint8_t *>(Mt.bs) + 1024 * (wave - 2));
        if (wave == DAW && lane < BM / 4) g2lds(dT + (int64_t)b * Mpad + m0 + 4 * lane, Mt.da);
    };

    v16i acc_h[2], acc_l[2];
    v16f out[2];
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) out[tm][v] = 0.0f;

    const int wr = 32 * wn + li;  // this lane's weight row (B operand column)
    const uint32_t raw_off0 = (uint32_t)wr * 128, wsw = (uint32_t)(wr & 7);
    const uint32_t act_off[2] = {(uint32_t)(64 * wm + li) * 256, (uint32_t)(64 * wm + 32 + li) * 256};
    const uint32_t asw = (uint32_t)(li & 15);  // rows 64wm + li and +32 share it

    issue(b0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int b = b0; b < b1; b++) {
        if (b + 1 < b1) issue(b + 1);
        const g3::Buf<BM> &B = buf[b & 1];
        const g3::Meta<BM> &Mt = SM.meta[b % 3];
        // ---- this lane's row: scales of the 8 sub-blocks, d, dmin, and the
        // min-term operand (mins of sub-blocks 4h .. 4h+3 at k = 8h .. 8h+7)
        const uint4 hv = *reinterpret_cast<const uint4 *>(B.hdr + 16 * wr);
        int sc[8], mn[8];
#pragma unroll
        for (int c = 0; c < 4; c++)
            k4_scales(hv.y, hv.z, hv.w, scale_sel(c), sc[2 * c], sc[2 * c + 1], mn[2 * c], mn[2 * c + 1]);
        const float dw = h2f(hv.x), dmin = h2f(hv.x >> 16);
        v8h Bm;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int mlo = mn[j], mhi = mn[4 + j];  // values, not a select of array elements
            const _Float16 m = (_Float16)(float)(h ? mhi : mlo);
            Bm[2 * j] = m;
            Bm[2 * j + 1] = m;
        }
        // ---- MFMAs: chunk c covers K-steps 2c (low nibbles) and 2c+1 (high);
        // chunk c+1's operands are read from LDS while chunk c multiplies
        const v16i zi = {};
        uint4 raw[2];
        v4i av[2][2][2];  // [buffer][nh][tm]
        auto load_chunk = [&](int c, uint4 &rw_, v4i (&a_)[2][2]) {
            rw_ = *reinterpret_cast<const uint4 *>(B.wraw + raw_off0 + 16 * ((2 * c + h) ^ wsw));
#pragma unroll
            for (int nh = 0; nh < 2; nh++)
#pragma unroll
                for (int tm = 0; tm < 2; tm++)
                    a_[nh][tm] = *reinterpret_cast<const v4i *>(B.act + act_off[tm] + 16 * ((2 * (2 * c + nh) + h) ^ asw));
        };
        load_chunk(0, raw[0], av[0]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int cb = c & 1;
            if (c < 3) load_chunk(c + 1, raw[cb ^ 1], av[cb ^ 1]);
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of this chunk's work
            const uint32_t rw[4] = {raw[cb].x, raw[cb].y, raw[cb].z, raw[cb].w};
#pragma unroll
            for (int nh = 0; nh < 2; nh++) {
                const int ks = 2 * c + nh;
                const uint32_t sv = (uint32_t)sc[ks];
                const uint32_t slo = sv & 7u, shi = sv >> 3;
                v4i blo, bhi;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t nib = nh ? ((rw[e] >> 4) & 0x0f0f0f0fu) : (rw[e] & 0x0f0f0f0fu);
                    blo[e] = (int)mul_bytes(nib, slo);
                    bhi[e] = (int)mul_bytes(nib, shi);
                }
#pragma unroll
                for (int tm = 0; tm < 2; tm++) {
                    acc_l[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[cb][nh][tm], blo, ks == 0 ? zi : acc_l[tm], 0, 0, 0);
                    acc_h[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[cb][nh][tm], bhi, ks == 0 ? zi : acc_h[tm], 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- min term and scaling
        const v16f zf = {};
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
            const int tl = 64 * wm + 32 * tm;
            const v8h Am = *reinterpret_cast<const v8h *>(&Mt.bs[(tl + li) * 16 + 8 * h]);
            const v16f accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(Am, Bm, zf, 0, 0, 0);
            float dav[16];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 d4 = *reinterpret_cast<const float4 *>(&Mt.da[tl + 8 * g + 4 * h]);
                dav[4 * g] = d4.x;
                dav[4 * g + 1] = d4.y;
                dav[4 * g + 2] = d4.z;
                dav[4 * g + 3] = d4.w;
            }
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int iacc = (acc_h[tm][v] << 3) + acc_l[tm][v];
                const float im = accm[v];
                if (SUBSUMS) {
                    const int ml = tl + crow(v, lane);
                    if (m0 + ml < M && n0 + wr < N) {
                        int32_t *sp = sub + (((int64_t)(m0 + ml) * N + (n0 + wr)) * nb + b) * 2;
                        sp[0] = iacc;
                        sp[1] = (int)im;
                    }
                }
                const float t = fmaf(dw, (float)iacc, -(dmin * im));
                out[tm][v] = fmaf(dav[v], t, out[tm][v]);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // super-block b+1 is in LDS
        __syncthreads();                                    // ... for every wavefront; buf[b&1] is free
    }
    // ---- store: for each v, the 32 lanes of a half write 32 consecutive floats
    const int n = n0 + wr;
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + 64 * wm + 32 * tm + crow(v, lane);
            if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tm][v];
        }
}

#define GEMM_KERNELS(NAME, BM, NT, LB)                                                                            \
    extern "C" __global__ void __launch_bounds__(NT, LB)                                                            \
        NAME(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, const int8_t *__restrict__ codes,    \
             const _Float16 *__restrict__ bsT, const float *__restrict__ dT, int M, int Mpad,                        \
             float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub, int nbs, int64_t zstride) {            \
        gemm_q4K_impl<BM, false>(W, w_row_bytes, N, nb, codes, bsT, dT, M, Mpad, dst, ldd, sub, nbs, zstride);      \
    }                                                                                                                \
    extern "C" __global__ void __launch_bounds__(NT, LB)                                                            \
        NAME##_sub(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,                               \
                   const int8_t *__restrict__ codes, const _Float16 *__restrict__ bsT, const float *__restrict__ dT, \
                   int M, int Mpad, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub, int nbs,        \
                   int64_t zstride) {                                                                                \
        gemm_q4K_impl<BM, true>(W, w_row_bytes, N, nb, codes, bsT, dT, M, Mpad, dst, ldd, sub, nbs, zstride);       \
    }
GEMM_KERNELS(ghip_gemm_q4_K, 128, 512, 1)
GEMM_KERNELS(ghip_gemm_q4_K_m64, 64, 256, 2)
// Sibling MUL_MATs in one launch (ghip_graph_compute): up to four Q4_K
// matrices of one K that read the same activation rows, so the Q8_K rows and
// their GEMM layout are made once.  Tiles [t0[i], t0[i+1]) belong to matrix i;
// the XCD remap runs over all of them.  Passed by value; the host mirror in
// ghip.cpp has the same layout.
struct GemmMulti {
    const uint8_t *W[4];
    float *dst[4];
    int64_t ldd[4];
    int N[4];
    int t0[4];
    int n, total;
};
extern "C" __global__ void __launch_bounds__(256, 2)
    ghip_gemm_q4_K_m64_multi(GemmMulti g, int64_t w_row_bytes, int nb, const int8_t *__restrict__ codes,
                             const _Float16 *__restrict__ bsT, const float *__restrict__ dT, int M, int Mpad) {
    int id = blockIdx.x;
    if (g.total % 8 == 0) id = (blockIdx.x & 7) * (g.total >> 3) + (blockIdx.x >> 3);
    int i = 0;
#pragma unroll
    for (int k = 1; k < 4; k++)
        if (k < g.n && id >= g.t0[k]) i = k;
    gemm_q4K_impl<64, false>(g.W[i], w_row_bytes, g.N[i], nb, codes, bsT, dT, M, Mpad, g.dst[i], g.ldd[i], nullptr,
                             nb, 0, id - g.t0[i]);
}

// ------------------------------------------------------------ wide Q4_K tiles
// The same arithmetic as gemm_q4K_impl on wider wavefront tiles: every
// wavefront owns 128 tokens x 32 weight rows (four 32 x 32 MFMA tiles per
// plane), so one nibble expansion and one header decode feed four token
// tiles.  A workgroup of NW wavefronts covers 128 tokens x 32*NW rows; its
// operands arrive by buffer loads straight into LDS (addresses are per-lane
// 32-bit offsets fixed for the whole loop plus a scalar per super-block
// offset, so the loop spends no vector instructions on them), two stages.
// Reads past the end of a buffer return zero, so rows past N need no clamp.
namespace g4 {
constexpr int BM = 128;
template <int BN> struct Stage {
    uint8_t act[BM * 256];  // [token][256], 16-byte slots swizzled by token % 16
    uint8_t wraw[BN * 128]; // [row][128] Q4_K qs, 16-byte slots swizzled by row % 8
    uint8_t hdr[BN * 16];   // [row] d, dmin, 12 scale bytes
    _Float16 bs[BM * 16];   // [token][16] bsum16
    float da[BM];           // block scale per token
};
}  // namespace g4
typedef __amdgpu_buffer_rsrc_t brsrc;
DEV brsrc make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
DEV void b2lds(brsrc r, void *lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, voff, soff, 0, 0);
}

// Q5: Q5_K weights (176-byte blocks: d, dmin, 12 scale bytes, qh[32], qs[128];
// vec_dot_q5_K_q8_K, vec_dot.rs:1062-1120, the Q4_K arithmetic with
// q5 = q4 + 16 * (bit s of qh[l]) for element l of sub-block s).  The fifth
// bit enters as a third int8 plane 2 * sc * bit (<= 126) accumulated into the
// high plane, so iacc = 8 * acc_h + acc_l holds 16 * sc * bit * q8 exactly;
// each lane's 16 qh bytes come by a buffer load one super-block ahead.
template <int NW, bool SUBSUMS, bool Q5 = false>
__device__ __forceinline__ void gemm_q4K_wide_impl(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
                                                   const int8_t *__restrict__ codes,
                                                   const _Float16 *__restrict__ bsT, const float *__restrict__ dT,
                                                   int M, int Mpad, float *__restrict__ dst, int64_t ldd,
                                                   int32_t *__restrict__ sub, int nbs, int64_t zstride, int tile) {
    constexpr int BM = g4::BM, BN = 32 * NW;
    constexpr int APW = 32 / NW;  // activation pieces (1 KB) per wavefront
    constexpr uint32_t BB = Q5 ? 176u : 144u, QS_OFF = Q5 ? 48u : 16u;  // block bytes, qs offset
    const int b0 = blockIdx.y * nbs, b1 = min(nb, b0 + nbs);
    dst += blockIdx.y * zstride;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    g4::Stage<BN> *stg = reinterpret_cast<g4::Stage<BN> *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, h = lane >> 5;
    const int K = nb * QK_K;
    const int rb = (int)w_row_bytes;

    const int n_tiles_m = (M + BM - 1) / BM, n_tiles_n = (N + BN - 1) / BN;
    const int total = n_tiles_m * n_tiles_n;
    int id = tile;
    if (id < 0) {
        id = blockIdx.x;
        if (total % 8 == 0) id = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    }
    const int m0 = (id % n_tiles_m) * BM;
    const int n0 = (id / n_tiles_m) * BN;

    // buffer windows: this tile's activation rows, weight rows (to the end
    // of the matrix), bsum16 and block-scale planes
    const brsrc ra = make_rsrc(codes + (int64_t)m0 * K, (uint32_t)BM * (uint32_t)K);
    const brsrc rw = make_rsrc(W + (int64_t)n0 * w_row_bytes, (uint32_t)min(BN, N - n0) * (uint32_t)rb);
    const brsrc rs = make_rsrc(bsT + (int64_t)m0 * 16, (uint32_t)((int64_t)nb * Mpad * 32 - (int64_t)m0 * 32));
    const brsrc rd = make_rsrc(dT + m0, (uint32_t)((int64_t)nb * Mpad * 4 - (int64_t)m0 * 4));
    // per-lane offsets: activation piece p holds tokens 4p .. 4p+3; weight
    // piece q rows 8q .. 8q+7; header piece r rows 64r .. 64r+63
    uint32_t aoff[APW];
#pragma unroll
    for (int i = 0; i < APW; i++) {
        const int tok = 4 * (APW * wave + i) + (lane >> 4);
        aoff[i] = (uint32_t)tok * (uint32_t)K + 16u * (uint32_t)((lane & 15) ^ (tok & 15));
    }
    // (the row goes into the per-lane offset, which the buffer's range check
    // covers, so rows past N read zero)
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        woff[i] = (uint32_t)(32 * wave + 8 * i + (lane >> 3)) * (uint32_t)rb + QS_OFF +
                  16u * (uint32_t)((lane & 7) ^ ((lane >> 3) & 7));
    const uint32_t hoff = (uint32_t)(64 * wave + lane) * (uint32_t)rb;  // header piece `wave`
    // bsum16 pieces wave - NW/2 and wave + NW/2
    const uint32_t soff[2] = {1024u * (uint32_t)(wave - NW / 2) + 16u * (uint32_t)lane,
                              1024u * (uint32_t)(wave + NW / 2) + 16u * (uint32_t)lane};
    const uint32_t doff = 16u * (uint32_t)lane;
    auto issue = [&](int b) {
        g4::Stage<BN> &S = stg[(b - b0) & 1];
#pragma unroll
        for (int i = 0; i < APW; i++) b2lds(ra, S.act + 1024 * (APW * wave + i), aoff[i], (uint32_t)b * 256u);
#pragma unroll
        for (int i = 0; i < 4; i++)
            b2lds(rw, S.wraw + 1024 * (4 * wave + i), woff[i], (uint32_t)b * BB);
        // NW/2 header pieces, then 4 bsum16 pieces: piece e by wavefront e % NW
#pragma unroll
        for (int e = wave; e < NW / 2 + 4; e += NW) {
            if (e < NW / 2) b2lds(rw, S.hdr + 1024 * e, hoff, (uint32_t)b * BB);
            else b2lds(rs, reinterpret_cast<uint8_t *>(S.bs) + 1024 * (e - NW / 2), soff[e >= NW], (uint32_t)b * (uint32_t)Mpad * 32u);
        }
        if (wave == NW - 1 && lane < BM / 4) b2lds(rd, S.da, doff, (uint32_t)b * (uint32_t)Mpad * 4u);
    };

    v16i acc_h[4], acc_l[4];
    v16f out[4];
#pragma unroll
    for (int tm = 0; tm < 4; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) out[tm][v] = 0.0f;

    const int wr = 32 * wave + li;  // this lane's weight row in the tile (B column)
    const uint32_t raw_off0 = (uint32_t)wr * 128, wsw = (uint32_t)(wr & 7);
    const uint32_t asw = (uint32_t)(li & 15);

    // Q5_K: this lane's qh bytes 16h .. 16h+15 (elements 16h + i of every sub-block)
    const uint32_t qhoff = (uint32_t)wr * (uint32_t)rb + 16u + 16u * (uint32_t)h;
    uint4 qh_cur = make_uint4(0, 0, 0, 0), qh_nxt = qh_cur;
    if (Q5 && b0 < b1)
        qh_cur = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, qhoff, (uint32_t)b0 * BB, 0));
    if (b0 < b1) issue(b0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int b = b0; b < b1; b++) {
        if (b + 1 < b1) issue(b + 1);
        if (Q5 && b + 1 < b1)
            qh_nxt = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, qhoff, (uint32_t)(b + 1) * BB, 0));
        const g4::Stage<BN> &S = stg[(b - b0) & 1];
        const uint4 hv = *reinterpret_cast<const uint4 *>(S.hdr + 16 * wr);
        const float dw = h2f(hv.x), dmin = h2f(hv.x >> 16);
        v8h Bm;
        {
            int s0, s1, s2, s3, mA, mB, mC, mD;
            k4_scales(hv.y, hv.z, hv.w, scale_sel(0), s0, s1, mA, mB);
            k4_scales(hv.y, hv.z, hv.w, scale_sel(2), s2, s3, mC, mD);
            int e0, e1, e2, e3, mE, mF, mG, mH;
            k4_scales(hv.y, hv.z, hv.w, scale_sel(1), e0, e1, mE, mF);
            k4_scales(hv.y, hv.z, hv.w, scale_sel(3), e2, e3, mG, mH);
            (void)s0; (void)s1; (void)s2; (void)s3; (void)e0; (void)e1; (void)e2; (void)e3;
            // mins of sub-blocks 4h .. 4h+3 at k = 8h .. 8h+7, each twice
            const int q0 = h ? mC : mA, q1 = h ? mD : mB, q2 = h ? mG : mE, q3 = h ? mH : mF;
            Bm[0] = Bm[1] = (_Float16)(float)q0;
            Bm[2] = Bm[3] = (_Float16)(float)q1;
            Bm[4] = Bm[5] = (_Float16)(float)q2;
            Bm[6] = Bm[7] = (_Float16)(float)q3;
        }
        const v4i zi = {};
        (void)zi;
        const v16i z16 = {};
        // the expansion and MFMAs run at raised wave priority and the epilogue
        // at normal, so the SIMD's other wavefront scales its tiles in the
        // MFMA gaps (measured: 89-91 -> 83-87 us at 512 x 4096 -> 14336)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint4 raw = *reinterpret_cast<const uint4 *>(S.wraw + raw_off0 + 16 * ((2 * c + h) ^ wsw));
            int sa, sb2, mu0, mu1;
            k4_scales(hv.y, hv.z, hv.w, scale_sel(c), sa, sb2, mu0, mu1);
            (void)mu0; (void)mu1;
            const uint32_t rwv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int nh = 0; nh < 2; nh++) {
                const int ks = 2 * c + nh;
                const uint32_t sv = (uint32_t)(nh ? sb2 : sa);
                const uint32_t slo = sv & 7u, shi = sv >> 3;
                v4i blo, bhi, b5;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t nib = nh ? ((rwv[e] >> 4) & 0x0f0f0f0fu) : (rwv[e] & 0x0f0f0f0fu);
                    blo[e] = (int)mul_bytes(nib, slo);
                    bhi[e] = (int)mul_bytes(nib, shi);
                    if (Q5) {
                        const uint32_t qw = e == 0 ? qh_cur.x : e == 1 ? qh_cur.y : e == 2 ? qh_cur.z : qh_cur.w;
                        b5[e] = (int)mul_bytes((qw >> ks) & 0x01010101u, 2u * sv);
                    }
                }
#pragma unroll
                for (int tm = 0; tm < 4; tm++) {
                    const v4i a = *reinterpret_cast<const v4i *>(S.act + (32 * tm + li) * 256 + 16 * ((2 * ks + h) ^ asw));
                    acc_l[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, blo, ks == 0 ? z16 : acc_l[tm], 0, 0, 0);
                    acc_h[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bhi, ks == 0 ? z16 : acc_h[tm], 0, 0, 0);
                    if (Q5) acc_h[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b5, acc_h[tm], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // ---- min term and scaling
        const v16f zf = {};
#pragma unroll
        for (int tm = 0; tm < 4; tm++) {
            const int tl = 32 * tm;
            const v8h Am = *reinterpret_cast<const v8h *>(&S.bs[(tl + li) * 16 + 8 * h]);
            const v16f accm = __builtin_amdgcn_mfma_f32_32x32x16_f16(Am, Bm, zf, 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 d4 = *reinterpret_cast<const float4 *>(&S.da[tl + 8 * g + 4 * h]);
                const float dav[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int v = 4 * g + r;
                    const int iacc = (acc_h[tm][v] << 3) + acc_l[tm][v];
                    const float im = accm[v];
                    if (SUBSUMS) {
                        const int ml = tl + crow(v, lane);
                        if (m0 + ml < M && n0 + wr < N) {
                            int32_t *sp = sub + (((int64_t)(m0 + ml) * N + (n0 + wr)) * nb + b) * 2;
                            sp[0] = iacc;
                            sp[1] = (int)im;
                        }
                    }
                    const float t = fmaf(dw, (float)iacc, -(dmin * im));
                    out[tm][v] = fmaf(dav[r], t, out[tm][v]);
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        qh_cur = qh_nxt;
    }
    const int n = n0 + wr;
#pragma unroll
    for (int tm = 0; tm < 4; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + 32 * tm + crow(v, lane);
            if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tm][v];
        }
}

#define GEMM_WIDE_KERNELS(NAME, NW, LB)                                                                           \
    extern "C" __global__ void __launch_bounds__(64 * NW, LB)                                                     \
        NAME(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, const int8_t *__restrict__ codes,  \
             const _Float16 *__restrict__ bsT, const float *__restrict__ dT, int M, int Mpad,                      \
             float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub, int nbs, int64_t zstride) {          \
        gemm_q4K_wide_impl<NW, false>(W, w_row_bytes, N, nb, codes, bsT, dT, M, Mpad, dst, ldd, sub, nbs, zstride, \
                                      -1);                                                                         \
    }                                                                                                              \
    extern "C" __global__ void __launch_bounds__(64 * NW, LB)                                                     \
        NAME##_sub(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,                             \
                   const int8_t *__restrict__ codes, const _Float16 *__restrict__ bsT,                             \
                   const float *__restrict__ dT, int M, int Mpad, float *__restrict__ dst, int64_t ldd,            \
                   int32_t *__restrict__ sub, int nbs, int64_t zstride) {                                          \
        gemm_q4K_wide_impl<NW, true>(W, w_row_bytes, N, nb, codes, bsT, dT, M, Mpad, dst, ldd, sub, nbs, zstride,  \
                                     -1);                                                                          \
    }
GEMM_WIDE_KERNELS(ghip_gemm_q4_K_w8, 8, 1)
extern "C" __global__ void __launch_bounds__(512, 1)
    ghip_gemm_q5_K_w8(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
                      const int8_t *__restrict__ codes, const _Float16 *__restrict__ bsT, const float *__restrict__ dT,
                      int M, int Mpad, float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub, int nbs,
                      int64_t zstride) {
    gemm_q4K_wide_impl<8, false, true>(W, w_row_bytes, N, nb, codes, bsT, dT, M, Mpad, dst, ldd, sub, nbs, zstride, -1);
}
extern "C" __global__ void __launch_bounds__(512, 1)
    ghip_gemm_q5_K_w8_sub(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb,
                          const int8_t *__restrict__ codes, const _Float16 *__restrict__ bsT,
                          const float *__restrict__ dT, int M, int Mpad, float *__restrict__ dst, int64_t ldd,
                          int32_t *__restrict__ sub, int nbs, int64_t zstride) {
    gemm_q4K_wide_impl<8, true, true>(W, w_row_bytes, N, nb, codes, bsT, dT, M, Mpad, dst, ldd, sub, nbs, zstride, -1);
}




// ---------------------------------------------------------------- Q6_K prefill
// Many activation rows with Q6_K weights (vec_dot_q6_K_q8_K, vec_dot.rs:982-1040,
// per super-block  is = sum_s sc_s * sum_16 (q6 - 32) * q8,  out += (d * is) * d8).
//
// On the f16 matrix cores with exact operands:
//  * activations: the Q8_K codes as f16 (exact), written by ghip_gemm_act_layout_f16;
//  * weights: (q - 32) * sc with the signed scale split sc = 16*sh + sl
//    (sl = sc & 15, sh = sc >> 4), two f16 planes per K-step:
//      (q - 32) * sl        |.| <= 480,  an integer, exact in f16;
//      (q - 32) * 16 * sh   a multiple of 16 with |.| <= 4096, exact in f16.
//    Every product with a code (|q8| <= 128) is exact in fp32; each plane has
//    its own fp32 accumulator per super-block, whose sums stay exact integers
//    (below 2^24, or multiples of 16 below 2^28), and is = lo + hi in int32.
// The 210-byte blocks start at odd 2-byte offsets; ghip_q6K_repack rewrites
// them (per call, or once for a registered weight) into aligned 336-byte
// records:  q[256] (6-bit values 0..63 in element order) | 16 x (f16 sl,
// f16 16*sh) | d f32 | pad.
constexpr int Q6R_BYTES = 336;

// one 64-lane group per block: the block's bytes arrive with coalesced dword
// loads from its 4-byte-aligned base into LDS, then lane u writes elements
// 4u .. 4u+3 (and lanes 0..19 the scale pairs, d and padding)
extern "C" __global__ void __launch_bounds__(256)
ghip_q6K_repack(const uint8_t *__restrict__ W, int64_t w_row_bytes, int N, int nb, uint8_t *__restrict__ out) {
    __shared__ uint32_t stage[4][56];  // 224 bytes per group
    const int grp = threadIdx.x >> 6, u = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + grp;  // row * nb + block
    const bool live = blk < (int64_t)N * nb;
    const int64_t row = live ? blk / nb : 0;
    const int b = live ? (int)(blk - row * nb) : 0;
    const uint8_t *src = W + row * w_row_bytes + (int64_t)b * Q6K_BYTES;
    const uintptr_t base4 = (uintptr_t)src & ~(uintptr_t)3;
    const int sh = (int)((uintptr_t)src - base4);  // 0 or 2
    const uintptr_t end = (uintptr_t)(W + (int64_t)(N - 1) * w_row_bytes + (int64_t)nb * Q6K_BYTES);
    // dwords 0..53 cover the block's 210 bytes plus the shift; none past the matrix
    if (live && u < 54 && base4 + 4 * u + 4 <= end)
        stage[grp][u] = *reinterpret_cast<const uint32_t *>(base4 + 4 * u);
    __syncthreads();
    if (!live) return;
    const uint8_t *blkb = reinterpret_cast<const uint8_t *>(stage[grp]) + sh;
    uint8_t *dst = out + blk * Q6R_BYTES;
    // element i of half j = i / 128, l = i % 128: ql[64j + l % 64] nibble l / 64,
    // qh[32j + l % 32] bits 2 * (l / 32) (dequantize_row_q6_K)
    const int e4 = 4 * u, j = e4 >> 7, l = e4 & 127;
    const uint8_t *ql = blkb + 64 * j + (l & 63);
    const uint8_t *qh = blkb + 128 + 32 * j + (l & 31);
    const int nsh = 4 * (l >> 6), hsh = 2 * (l >> 5);
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) v |= (uint32_t)(((ql[k] >> nsh) & 15) | (((qh[k] >> hsh) & 3) << 4)) << (8 * k);
    *reinterpret_cast<uint32_t *>(dst + e4) = v;
    if (u < 16) {
        // sub-block u's signed scale split 16 * sh + sl, as the f16 pair
        // (sl, 16 * sh) the GEMM multiplies the weight planes by
        const int sc = (int)(int8_t)blkb[192 + u];
        const int sl = sc & 15;
        const _Float16 fl = (_Float16)(float)sl, fh = (_Float16)(float)(sc - sl);
        *reinterpret_cast<uint32_t *>(dst + 256 + 4 * u) =
            (uint32_t)__builtin_bit_cast(uint16_t, fl) | ((uint32_t)__builtin_bit_cast(uint16_t, fh) << 16);
    } else if (u == 16) {
        *reinterpret_cast<float *>(dst + 320) = h2f((uint32_t)blkb[208] | ((uint32_t)blkb[209] << 8));
    } else if (u < 20) {
        *reinterpret_cast<uint32_t *>(dst + 324 + 4 * (u - 17)) = 0u;
    }
}

// Q8_K rows -> f16 codes [Mpad][K] and block scales dT [nb][Mpad] (tokens padded
// to a multiple of 128); one wavefront per (token, super-block)
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_act_layout_f16(const uint8_t *__restrict__ q8k, int64_t row_bytes, int M, int Mpad, int nb,
                         _Float16 *__restrict__ codes, float *__restrict__ dT) {
    const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (task >= (int64_t)M * nb) return;
    const int m = (int)(task / nb), b = (int)(task % nb);
    const uint8_t *blk = q8k + (int64_t)m * row_bytes + (int64_t)b * Q8K_BYTES;
    const uint32_t c4 = ld4(blk + 4 + 4 * lane);
    _Float16 *o = codes + (int64_t)m * nb * QK_K + b * QK_K + 4 * lane;
#pragma unroll
    for (int k = 0; k < 4; k++) o[k] = (_Float16)(float)(int8_t)(c4 >> (8 * k));
    if (lane == 0) dT[(int64_t)b * Mpad + m] = __uint_as_float(ld4(blk));
}

namespace g6 {
constexpr int BM = 64, BN = 128;
struct Smem {
    _Float16 act[2][BM * QK_K];     // [stage][token][256], 16-byte slots swizzled by token % 32
    uint8_t w[2][BN * Q6R_BYTES];   // [stage][row][336]
    float da[3][BM];                // block scales of the tokens, a 3-slot ring
};
}  // namespace g6
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// 64 tokens x 128 rows per 256-thread workgroup; wavefront w owns rows
// 32w .. 32w+31 and both 32-token tiles.  K-step ks (16 elements of
// sub-block ks): lane l takes elements 16ks + 8(l/32) .. +7 of row l % 32 (B)
// and of token l % 32 of each tile (A).
template <bool SUBSUMS>
__device__ __forceinline__ void gemm_q6K_impl(const uint8_t *__restrict__ R, int N, int nb,
                                              const _Float16 *__restrict__ codes, const float *__restrict__ dT,
                                              int M, int Mpad, float *__restrict__ dst, int64_t ldd,
                                              int32_t *__restrict__ sub) {
    constexpr int BM = g6::BM, BN = g6::BN;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    g6::Smem &SM = *reinterpret_cast<g6::Smem *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, h = lane >> 5;
    const int64_t K = (int64_t)nb * QK_K;
    const int n_tiles_m = (M + BM - 1) / BM, n_tiles_n = (N + BN - 1) / BN;
    const int total = n_tiles_m * n_tiles_n;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int m0 = (id % n_tiles_m) * BM;
    const int n0 = (id / n_tiles_m) * BN;

    // buffer descriptors over this tile's activations, weight records and
    // block scales; the per-lane offsets are fixed, super-block b adds a
    // scalar offset.  Weight rows past N read as zeros (range-checked).
    const brsrc ra = make_rsrc(codes + (int64_t)m0 * K, (uint32_t)((int64_t)BM * K * 2));
    const brsrc rw = make_rsrc(R + (int64_t)n0 * nb * Q6R_BYTES, (uint32_t)((int64_t)min(BN, N - n0) * nb * Q6R_BYTES));
    const brsrc rd = make_rsrc(dT + m0, (uint32_t)(((int64_t)nb * Mpad - m0) * 4));
    uint32_t va[8], vw[11];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int tok = 2 * (8 * wave + i) + (lane >> 5);
        const int slot = (lane & 31) ^ (tok & 31);
        va[i] = (uint32_t)tok * (uint32_t)K * 2u + 16u * (uint32_t)slot;
    }
#pragma unroll
    for (int i = 0; i < 11; i++) {
        const int c = 64 * (4 * i + wave) + lane;
        const int row = c / 21, k16 = c - 21 * row;
        vw[i] = (uint32_t)row * (uint32_t)nb * Q6R_BYTES + 16u * (uint32_t)k16;
    }

    // ---- direct loads of super-block b: wavefront w moves act pieces
    // 8w .. 8w+7 (2 tokens each), weight pieces w, w+4, .. (64 16-byte
    // chunks each, 21 per row) and (w = 0) the block scales
    auto issue = [&](int b, int p) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            b2lds(ra, reinterpret_cast<uint8_t *>(SM.act[p]) + 1024 * (8 * wave + i), va[i], (uint32_t)b * 512u);
#pragma unroll
        for (int i = 0; i < 11; i++) {
            const int g = 4 * i + wave;  // 42 groups of 64 chunks
            if (g < BN * (Q6R_BYTES / 16) / 64) b2lds(rw, SM.w[p] + 1024 * g, vw[i], (uint32_t)b * Q6R_BYTES);
        }
        if (wave == 0 && lane < BM / 4) b2lds(rd, SM.da[b % 3], 16u * lane, (uint32_t)b * (uint32_t)Mpad * 4u);
    };

    v16f out[2];
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) out[tm][v] = 0.0f;
    const int wr = 32 * wave + li;  // this lane's weight row (B operand column)
    const uint32_t aoff[2] = {(uint32_t)li * QK_K, (uint32_t)(32 + li) * QK_K};  // halfs
    const uint32_t asw = (uint32_t)(li & 31);
    const v2h bias = {(_Float16)-1056.0f, (_Float16)-1056.0f};  // 1024 + 32

    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        const int p = b & 1;
        if (b + 1 < nb) issue(b + 1, p ^ 1);
        const uint8_t *wrow = SM.w[p] + wr * Q6R_BYTES;
        const float dw = *reinterpret_cast<const float *>(wrow + 320);
        // One accumulator per scale plane: the low plane's sums stay below
        // 256 * 480 * 127 < 2^24 and the high plane's are multiples of 16
        // below 256 * 4096 * 127 < 2^28, so both are exact integers in fp32
        // for any valid block, and so is is = lo + hi added as int32.
        v16f accl[2], acch[2];
        const v16f zf = {};
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
            accl[tm] = zf;
            acch[tm] = zf;
        }
#pragma unroll 16
        for (int ks = 0; ks < 16; ks++) {
            const uint2 qv = *reinterpret_cast<const uint2 *>(wrow + 16 * ks + 8 * h);
            // the sub-block's signed scale split 16 * sh + sl, as f16 pairs
            const uint32_t sp = *reinterpret_cast<const uint32_t *>(wrow + 256 + 4 * ks);
            const v2h pl = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(sp, sp, 0x01000100u));
            const v2h ph = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(sp, sp, 0x03020302u));
            v8h blo, bhi;
            const uint32_t qw[2] = {qv.x, qv.y};
#pragma unroll
            for (int d = 0; d < 2; d++) {
                // bytes q -> f16 (1024 + q) by placing 0x64 above each byte, then - 1056
                const v2h e0 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, qw[d], 0x04010400u)) + bias;
                const v2h e1 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, qw[d], 0x04030402u)) + bias;
                const v2h l0 = e0 * pl, l1 = e1 * pl, h0 = e0 * ph, h1 = e1 * ph;
                blo[4 * d] = l0[0]; blo[4 * d + 1] = l0[1]; blo[4 * d + 2] = l1[0]; blo[4 * d + 3] = l1[1];
                bhi[4 * d] = h0[0]; bhi[4 * d + 1] = h0[1]; bhi[4 * d + 2] = h1[0]; bhi[4 * d + 3] = h1[1];
            }
#pragma unroll
            for (int tm = 0; tm < 2; tm++) {
                const v8h a = *reinterpret_cast<const v8h *>(SM.act[p] + aoff[tm] + 8 * ((uint32_t)(2 * ks + h) ^ asw));
                accl[tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, blo, accl[tm], 0, 0, 0);
                acch[tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bhi, acch[tm], 0, 0, 0);
            }
        }
        // ---- out += (d * is) * d8 (vec_dot_q6_K_q8_K's per-block order)
        const float *dab = SM.da[b % 3];
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int tl = 32 * tm + crow(v, lane);
                const int isi = (int)accl[tm][v] + (int)acch[tm][v];
                if constexpr (SUBSUMS)
                    if (m0 + tl < M && n0 + wr < N) sub[((int64_t)(m0 + tl) * N + (n0 + wr)) * nb + b] = isi;
                out[tm][v] = fmaf(dw * (float)isi, dab[tl], out[tm][v]);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // super-block b+1 is in LDS
        __syncthreads();
    }
    const int n = n0 + wr;
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + 32 * tm + crow(v, lane);
            if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tm][v];
        }
}
extern "C" __global__ void __launch_bounds__(256, 1)
    ghip_gemm_q6_K(const uint8_t *__restrict__ R, int N, int nb, const _Float16 *__restrict__ codes,
                   const float *__restrict__ dT, int M, int Mpad, float *__restrict__ dst, int64_t ldd,
                   int32_t *__restrict__ sub) {
    gemm_q6K_impl<false>(R, N, nb, codes, dT, M, Mpad, dst, ldd, sub);
}
extern "C" __global__ void __launch_bounds__(256, 1)
    ghip_gemm_q6_K_sub(const uint8_t *__restrict__ R, int N, int nb, const _Float16 *__restrict__ codes,
                       const float *__restrict__ dT, int M, int Mpad, float *__restrict__ dst, int64_t ldd,
                       int32_t *__restrict__ sub) {
    gemm_q6K_impl<true>(R, N, nb, codes, dT, M, Mpad, dst, ldd, sub);
}
static_assert(sizeof(g6::Smem) == 152320, "host code launches with this LDS size");

// split-K partial sums [nsplit][M][N] -> dst, slices added in order; four
// consecutive outputs per thread (N % 4 == 0)
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_splitk_reduce(const float *__restrict__ part, int nsplit, int M, int N, float *__restrict__ dst,
                        int64_t ldd) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= (int64_t)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    float4 acc = *reinterpret_cast<const float4 *>(part + i);
    for (int z = 1; z < nsplit; z++) {
        const float4 v = *reinterpret_cast<const float4 *>(part + (int64_t)z * M * N + i);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    float *d = dst + (int64_t)m * ldd + n;
    d[0] = acc.x;
    d[1] = acc.y;
    d[2] = acc.z;
    d[3] = acc.w;
}
static_assert(sizeof(g3::Smem<128>) == 116224 && sizeof(g3::Smem<64>) == 76544, "host code launches with these LDS sizes");
static_assert(2 * sizeof(g4::Stage<256>) == 148480, "host code launches with this LDS size");
// Sibling MUL_MATs in one launch on the wide tiles (see GemmMulti above).
extern "C" __global__ void __launch_bounds__(512, 1)
    ghip_gemm_q4_K_w8_multi(GemmMulti g, int64_t w_row_bytes, int nb, const int8_t *__restrict__ codes,
                            const _Float16 *__restrict__ bsT, const float *__restrict__ dT, int M, int Mpad) {
    int id = blockIdx.x;
    if (g.total % 8 == 0) id = (blockIdx.x & 7) * (g.total >> 3) + (blockIdx.x >> 3);
    int i = 0;
#pragma unroll
    for (int k = 1; k < 4; k++)
        if (k < g.n && id >= g.t0[k]) i = k;
    gemm_q4K_wide_impl<8, false>(g.W[i], w_row_bytes, g.N[i], nb, codes, bsT, dT, M, Mpad, g.dst[i], g.ldd[i],
                                 nullptr, nb, 0, id - g.t0[i]);
}

// Prefill activations straight from f32: the Q8_K quantization of
// ghip_quantize_q8_K (same arithmetic, ghip_q8k.h) written directly in the
// GEMM layouts, so the Q8_K rows never go through HBM.  One wavefront per
// (token, super-block); rows m < n_mat take the quantize_mat_q8_K_4x8 values.
//   F16 = false (Q4_K GEMM): codes [Mpad][K] int8 | bsT [nb][Mpad][16] f16 | dT [nb][Mpad]
//   F16 = true  (Q6_K GEMM): codes [Mpad][K] f16  | dT [nb][Mpad]
template <bool F16>
__device__ __forceinline__ void act_q8K_layout(const float *__restrict__ x, int64_t x_stride, int M, int Mpad, int nb,
                                               int n_mat, void *__restrict__ codes, _Float16 *__restrict__ bsT,
                                               float *__restrict__ dT) {
    const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (task >= (int64_t)M * nb) return;
    const int m = (int)(task / nb), b = (int)(task % nb);
    float xs[4];
    __builtin_memcpy(xs, x + (int64_t)m * x_stride + (int64_t)b * QK_K + 4 * lane, 16);
    int q[4];
    float d;
    q8K_block(xs, lane, m < n_mat, q, d);
    const int64_t e = (int64_t)m * nb * QK_K + (int64_t)b * QK_K + 4 * lane;
    if constexpr (F16) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 v = {(_Float16)(float)q[0], (_Float16)(float)q[1], (_Float16)(float)q[2], (_Float16)(float)q[3]};
        *reinterpret_cast<h4 *>(reinterpret_cast<_Float16 *>(codes) + e) = v;
    } else {
        const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                                ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
        *reinterpret_cast<uint32_t *>(reinterpret_cast<int8_t *>(codes) + e) = packed;
        const int s = q8K_bsum16(q, lane);
        if ((lane & 3) == 0) bsT[((int64_t)b * Mpad + m) * 16 + (lane >> 2)] = (_Float16)(float)s;
    }
    if (lane == 0) dT[(int64_t)b * Mpad + m] = d;
}
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_act_q8K(const float *__restrict__ x, int64_t x_stride, int M, int Mpad, int nb, int n_mat,
                  int8_t *__restrict__ codes, _Float16 *__restrict__ bsT, float *__restrict__ dT) {
    act_q8K_layout<false>(x, x_stride, M, Mpad, nb, n_mat, codes, bsT, dT);
}
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_act_q8K_f16(const float *__restrict__ x, int64_t x_stride, int M, int Mpad, int nb, int n_mat,
                      _Float16 *__restrict__ codes, float *__restrict__ dT) {
    act_q8K_layout<true>(x, x_stride, M, Mpad, nb, n_mat, codes, nullptr, dT);
}

// ------------------------------------------------- Q4_0 / Q5_0 / Q8_0 prefill
// Many activation rows with 32-element-block weights (vec_dot_q4_0_q8_0,
// vec_dot_q5_0_q8_0, vec_dot_q8_0_q8_0, vec_dot.rs:596-700: per block
// dot = sum_32 w * q8 exact, out += (d_w * d_a) * dot).  The weight values
// (q - 8, q - 16, or the Q8_0 codes) are int8, so one v_mfma_i32_32x32x32_i8
// per 32-block gives the exact integer dot of a 32 x 32 tile; the fold is one
// fma per output and block.  Both operands are staged as int8 codes with
// f32 block scales (weights by ghip_gemm_q8w_repack, per call or once for a
// registered weight; activations by ghip_gemm_act_q8_0 with the arithmetic of
// quantize_row_q8_0), K padded to a multiple of 128 with zeros.

// one thread per (row, block): the 32 values as int8 at codes[row][32b..],
// the block scale at dw[b][row] (Npad rows)
template <int TYPE>  // 2 Q4_0, 6 Q5_0, 8 Q8_0
__device__ __forceinline__ void q8w_repack(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb,
                                           int Kpad, int Npad, int8_t *__restrict__ codes, float *__restrict__ dw) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int nbp = Kpad / 32;
    if (i >= (int64_t)Npad * nbp) return;
    const int row = (int)(i / nbp), b = (int)(i % nbp);
    uint32_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float d = 0.0f;
    if (row < N && b < nb) {
        constexpr int BB = TYPE == 2 ? 18 : TYPE == 6 ? 22 : 34;
        const uint8_t *blk = W + (int64_t)row * row_bytes + (int64_t)b * BB;
        d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        if constexpr (TYPE == 8) {
#pragma unroll
            for (int k = 0; k < 32; k++) v[k >> 2] |= (uint32_t)blk[2 + k] << (8 * (k & 3));
        } else {
            const uint8_t *qs = blk + (TYPE == 6 ? 6 : 2);
            const uint32_t qh = TYPE == 6 ? ((uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                                             ((uint32_t)blk[5] << 24))
                                          : 0u;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                int lo = qs[j] & 15, hi = qs[j] >> 4;
                if (TYPE == 6) {
                    lo |= (int)((qh >> j) & 1) << 4;
                    hi |= (int)((qh >> (j + 16)) & 1) << 4;
                }
                const int off = TYPE == 6 ? 16 : 8;
                v[j >> 2] |= (uint32_t)((lo - off) & 0xff) << (8 * (j & 3));
                v[(j + 16) >> 2] |= (uint32_t)((hi - off) & 0xff) << (8 * ((j + 16) & 3));
            }
        }
    }
    int8_t *o = codes + q8w_piece(row, b, Kpad);
    *reinterpret_cast<uint4 *>(o) = make_uint4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<uint4 *>(o + 512) = make_uint4(v[4], v[5], v[6], v[7]);
    dw[(int64_t)b * Npad + row] = d;
}
#define Q8W_REPACK(TN, TYPE)                                                                                       \
    extern "C" __global__ void __launch_bounds__(256)                                                              \
        ghip_gemm_q8w_repack_##TN(const uint8_t *__restrict__ W, int64_t row_bytes, int N, int nb, int Kpad,       \
                                  int Npad, int8_t *__restrict__ codes, float *__restrict__ dw) {                  \
        q8w_repack<TYPE>(W, row_bytes, N, nb, Kpad, Npad, codes, dw);                                              \
    }
Q8W_REPACK(q4_0, 2)
Q8W_REPACK(q5_0, 6)
Q8W_REPACK(q8_0, 8)

// f32 rows -> Q8_0 codes [Mpad][Kpad] int8 and da [nbp][Mpad] f32 (the stored
// f16 scale), the arithmetic of ghip_quantize_q8_0 (quantize_row_q8_0,
// quants.rs:153-180); 8 lanes per block, padding rows and blocks zero
extern "C" __global__ void __launch_bounds__(256)
ghip_gemm_act_q8_0(const float *__restrict__ x, int64_t x_stride, int M, int Mpad, int nb, int Kpad,
                   int8_t *__restrict__ codes, float *__restrict__ da) {
    const int lane = threadIdx.x & 63, sub = lane & 7;
    const int nbp = Kpad / 32;
    const int64_t blk_id = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    if (blk_id >= (int64_t)Mpad * nbp) return;  // whole 8-lane groups exit together
    const int row = (int)(blk_id / nbp), b = (int)(blk_id % nbp);
    const bool live = row < M && b < nb;
    float xs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live) __builtin_memcpy(xs, x + (int64_t)row * x_stride + (int64_t)b * 32 + sub * 4, 16);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(xs[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float r = rintf(__fmul_rn(xs[i], id));
        const int v = (r != r || fabsf(r) >= 2147483648.0f) ? -128 : (int)r;
        packed |= (uint32_t)(v & 0xff) << (8 * i);
    }
    *reinterpret_cast<uint32_t *>(codes + (int64_t)row * Kpad + 32 * b + 4 * sub) = packed;
    if (sub == 0) da[(int64_t)b * Mpad + row] = h2f(f2h_rn(d));
}

namespace g8 {
constexpr int BM = 64, BN = 128, GB = 4;  // tokens, rows, 32-blocks per stage
struct Smem {
    int8_t act[2][BM * GB * 32];   // [stage][token][128 B], 16-byte slots swizzled by token % 8
    float da[2][GB][BM];
    float dw[2][GB][BN];
};
}  // namespace g8

// 64 tokens x 128 rows per 256-thread workgroup; wavefront w owns rows
// 32w .. 32w+31 and both 32-token tiles.  C[token][row]: lane l holds row
// l % 32 and tokens crow(v, l).  Operands: lane l takes K 16(l/32) .. +15 of
// the block (A: token l % 32 of the tile, B: row l % 32).  The activations,
// shared by the four wavefronts, are staged through LDS; each wavefront's
// weights go from memory straight to its registers (q8w_piece layout), one
// group ahead.
//
// XS (IQ4_XS weights, Q8_K activations): dw holds each 32-group's integer
// scale ls - 32 (exact in f32) and dsb[super-block][row] the block's d; the
// groups' exact dots are summed as (ls - 32) * dot in int32 over the
// super-block, and the super-block folds as the reference's tiled kernel does
// (tiled.rs:822-836): res = d * is, out = fma(res, d8, out), in super-block
// order.  Sub-sums are then the super-block sums.
template <bool SUBSUMS, bool XS = false>
__device__ __forceinline__ void gemm_q8_impl(const int8_t *__restrict__ wc, const float *__restrict__ dw, int N,
                                             int Npad, int nb, int Kpad, const int8_t *__restrict__ ac,
                                             const float *__restrict__ da, int M, int Mpad, float *__restrict__ dst,
                                             int64_t ldd, int32_t *__restrict__ sub,
                                             const float *__restrict__ dsb = nullptr) {
    constexpr int BM = g8::BM, BN = g8::BN, GB = g8::GB;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    g8::Smem &SM = *reinterpret_cast<g8::Smem *>(smem_raw);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, h = lane >> 5;
    const int n_tiles_m = (M + BM - 1) / BM, n_tiles_n = (N + BN - 1) / BN;
    const int total = n_tiles_m * n_tiles_n;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int m0 = (id % n_tiles_m) * BM, n0 = (id / n_tiles_m) * BN;
    const int ng = Kpad / (32 * GB);

    // group g into stage p: 2 act chunks, (waves 0-1) the scales
    auto issue = [&](int g, int p) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = 64 * (2 * wave + i) + lane;  // LDS chunk: token c / 8, slot c % 8
            const int t = c >> 3, src = (c & 7) ^ ((t >> 1) & 7);
            g2lds(ac + (int64_t)(m0 + t) * Kpad + (int64_t)g * 128 + 16 * src,
                  SM.act[p] + 1024 * (2 * wave + i));
        }
        if (wave == 0) {  // da: 4 blocks x 64 tokens = 64 chunks
            const int kb = lane >> 4;
            g2lds(da + (int64_t)(g * GB + kb) * Mpad + m0 + 4 * (lane & 15), &SM.da[p][0][0]);
        } else if (wave == 1) {  // dw: 4 blocks x 128 rows = 128 chunks, two per lane
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = 64 * i + lane, kb = c >> 5;
                g2lds(dw + (int64_t)(g * GB + kb) * Npad + min(n0 + 4 * (c & 31), Npad - 4),
                      reinterpret_cast<uint8_t *>(&SM.dw[p][0][0]) + 1024 * i);
            }
        }
    };

    v16f out[2];
    v16i isb[2];  // XS: the super-block's integer sums
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            out[tm][v] = 0.0f;
            isb[tm][v] = 0;
        }
    const int wr = 32 * wave + li;  // this lane's weight row in the tile
    // one 32-block's operands: A for both token tiles and B, plus the scale
    // operands of the outer-product MFMA: lanes of half 0 put the token's
    // (A) and the row's (B) f16 scale at k = 0, every other k is 0, so
    // S[token][row] = da * dw, exact (two f16 values), in the layout of the
    // block's integer dots
    struct Ops {
        v4i a[2];
        v8h sa[2];
        v8h sb;
        float sw;  // XS: the group's integer scale ls - 32
        float da[2][16];  // XS: the 16 token scales of each tile
    };
    auto load = [&](int p, int kb, Ops &o) {
        const int slot = 2 * kb + h;  // this lane's 16 bytes of block kb
        o.sw = SM.dw[p][kb][wr];
        const v8h z8 = {};
        o.sb = z8;
        o.sb[0] = h == 0 ? (_Float16)o.sw : (_Float16)0.0f;
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
            const int ta = 32 * tm + li;
            o.a[tm] = *reinterpret_cast<const v4i *>(SM.act[p] + ta * 128 + 16 * (slot ^ ((ta >> 1) & 7)));
            if constexpr (XS) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 d4 = *reinterpret_cast<const float4 *>(&SM.da[p][kb][32 * tm + 8 * q + 4 * h]);
                    o.da[tm][4 * q] = d4.x;
                    o.da[tm][4 * q + 1] = d4.y;
                    o.da[tm][4 * q + 2] = d4.z;
                    o.da[tm][4 * q + 3] = d4.w;
                }
            } else {
                o.sa[tm] = z8;
                const _Float16 dah = (_Float16)SM.da[p][kb][ta];
                o.sa[tm][0] = h == 0 ? dah : (_Float16)0.0f;
            }
        }
    };
    // block b's products c[tm] (scales sc[tm]) into the outputs (XS: into the
    // super-block's integer sums, folded at its last group)
    auto fold = [&](int b, const Ops &o, const v16i (&c)[2], const v16f (&sc)[2]) {
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
            if constexpr (XS) {
                // |ls * dot| <= 32 * 32 * 127 * 128, eight of them fit int32
                const int ls = (int)o.sw;
#pragma unroll
                for (int v = 0; v < 16; v++) isb[tm][v] += ls * c[tm][v];
                if ((b & 7) == 7) {
                    const float d = b < nb ? dsb[(int64_t)(b >> 3) * Npad + min(n0 + wr, Npad - 1)] : 0.0f;
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int tl = 32 * tm + crow(v, lane);
                        out[tm][v] = fmaf(d * (float)isb[tm][v], o.da[tm][v], out[tm][v]);
                        if constexpr (SUBSUMS)
                            if (b < nb && m0 + tl < M && n0 + wr < N)
                                sub[((int64_t)(m0 + tl) * N + (n0 + wr)) * (nb >> 3) + (b >> 3)] = isb[tm][v];
                        isb[tm][v] = 0;
                    }
                }
            } else {
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    out[tm][v] = fmaf(sc[tm][v], (float)c[tm][v], out[tm][v]);
                    if constexpr (SUBSUMS) {
                        const int tl = 32 * tm + crow(v, lane);
                        if (b < nb && m0 + tl < M && n0 + wr < N)
                            sub[((int64_t)(m0 + tl) * N + (n0 + wr)) * nb + b] = c[tm][v];
                    }
                }
            }
        }
    };
    // this wavefront's weight pieces: group g's block kb at wpc + (4g + kb) * 1024
    const int8_t *wpc = wc + q8w_piece(n0 + 32 * wave, 0, Kpad) + 16 * lane;
    v4i bq[GB], bqn[GB];  // this group's and the next group's
    auto load_w = [&](int g, v4i (&q)[GB]) {
#pragma unroll
        for (int kb = 0; kb < GB; kb++)
            q[kb] = *reinterpret_cast<const v4i *>(wpc + (int64_t)(g * GB + kb) * 1024);
    };
    load_w(0, bq);
    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const v16i zi = {};
    const v16f zf = {};
    v16i c[2][2];  // block kb's dots in c[kb & 1], scales in sc[kb & 1]
    v16f sc[2][2];
    for (int g = 0; g < ng; g++) {
        const int p = g & 1;
        if (g + 1 < ng) {
            issue(g + 1, p ^ 1);
            load_w(g + 1, bqn);
        }
        // block kb+1's operands are read while block kb multiplies and block
        // kb-1 folds (the previous group's last block folds under this
        // group's first MFMAs; XS folds it at the group's end)
        Ops ops[3];  // block kb in ops[kb % 3]
        load(p, 0, ops[0]);
#pragma unroll
        for (int kb = 0; kb < GB; kb++) {
            const int cb = kb & 1;
            if (kb + 1 < GB) load(p, kb + 1, ops[(kb + 1) % 3]);
            const Ops &o = ops[kb % 3];
#pragma unroll
            for (int tm = 0; tm < 2; tm++) {
                c[cb][tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[tm], bq[kb], zi, 0, 0, 0);
                if constexpr (!XS) sc[cb][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o.sa[tm], o.sb, zf, 0, 0, 0);
            }
            if (kb > 0)
                fold(g * GB + kb - 1, ops[(kb + 2) % 3], c[cb ^ 1], sc[cb ^ 1]);
            else if (!XS && g > 0)
                fold(g * GB - 1, ops[0], c[1], sc[1]);
            if constexpr (!XS && !SUBSUMS) {
                // spread the fold's VALU work between the MFMAs
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x8, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x2, 18, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (XS) fold(g * GB + GB - 1, ops[(GB - 1) % 3], c[(GB - 1) & 1], sc[(GB - 1) & 1]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
#pragma unroll
        for (int kb = 0; kb < GB; kb++) bq[kb] = bqn[kb];
    }
    if (!XS && ng > 0) {
        Ops none = {};  // the non-XS fold reads no operands
        fold(ng * GB - 1, none, c[1], sc[1]);
    }
    const int n = n0 + wr;
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + 32 * tm + crow(v, lane);
            if (m < M && n < N) dst[(int64_t)m * ldd + n] = out[tm][v];
        }
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8(const int8_t *__restrict__ wc, const float *__restrict__ dw, int N, int Npad, int nb, int Kpad,
                 const int8_t *__restrict__ ac, const float *__restrict__ da, int M, int Mpad,
                 float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    gemm_q8_impl<false>(wc, dw, N, Npad, nb, Kpad, ac, da, M, Mpad, dst, ldd, sub);
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8_sub(const int8_t *__restrict__ wc, const float *__restrict__ dw, int N, int Npad, int nb,
                     int Kpad, const int8_t *__restrict__ ac, const float *__restrict__ da, int M, int Mpad,
                     float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub) {
    gemm_q8_impl<true>(wc, dw, N, Npad, nb, Kpad, ac, da, M, Mpad, dst, ldd, sub);
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8_xs(const int8_t *__restrict__ wc, const float *__restrict__ dw, int N, int Npad, int nb, int Kpad,
                    const int8_t *__restrict__ ac, const float *__restrict__ da, int M, int Mpad,
                    float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub, const float *__restrict__ dsb) {
    gemm_q8_impl<false, true>(wc, dw, N, Npad, nb, Kpad, ac, da, M, Mpad, dst, ldd, sub, dsb);
}
extern "C" __global__ void __launch_bounds__(256)
    ghip_gemm_q8_xs_sub(const int8_t *__restrict__ wc, const float *__restrict__ dw, int N, int Npad, int nb,
                        int Kpad, const int8_t *__restrict__ ac, const float *__restrict__ da, int M, int Mpad,
                        float *__restrict__ dst, int64_t ldd, int32_t *__restrict__ sub,
                        const float *__restrict__ dsb) {
    gemm_q8_impl<true, true>(wc, dw, N, Npad, nb, Kpad, ac, da, M, Mpad, dst, ldd, sub, dsb);
}
static_assert(sizeof(g8::Smem) == 22528, "host code launches with this LDS size");
