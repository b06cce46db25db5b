// ghip_moe.hip -- GGML_OP_MUL_MAT_ID with MXFP4 experts (gpt-oss MoE).
//
// Reference (compute.rs:1917-2202, repack.rs:1048-1100): activations are
// quantized to Q8_0 per (token, i11) row; for every (token, slot) pair with
// expert id = ids[token][slot] and every expert row r,
//   dst[token][slot][r] = fold over 32-blocks b of
//       acc = fma(f32(dot_b), e8m0_half(e[r,b]) * d_a[b], acc)
// with dot_b = sum_32 kvalue(nibble) * q8 (exact int32, |dot| <= 48768).
//
// On the GPU the pairs are first sorted by expert (ghip_moe_route), so each
// expert's weights stream once per tile of 64 pairs.  The block dot runs on the
// f16 matrix cores: kvalues and Q8 codes are small integers, exact in f16, and
// every 32-element block gets a fresh fp32 accumulator, so the MFMA result IS
// the integer dot_b (all partial sums < 2^24).  The epilogue then applies the
// reference's own fold -- the same fma, the same block order -- so the output
// is bit-identical to the reference's repack route.
#include "ghip_common.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int MOE_TR = 128;  // expert rows per workgroup (32 per wavefront)
constexpr int MOE_KB = 8;    // 32-blocks staged in LDS at a time

DEV int crowm(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// ---------------------------------------------------------------- routing
// One workgroup: counting sort of the (token, slot) pairs by expert id and
// the tile list of the GEMM (tiles of at most tp pairs of one expert).  route layout (int32):
//   [0] n_tiles, [1] n_bad,
//   [2 .. 2+n_pairs)              pairs sorted by expert,
//   then per tile: expert, first, count (3 ints) for up to max_tiles tiles.
extern "C" __global__ void __launch_bounds__(1024)
ghip_moe_route(const int32_t *__restrict__ ids, int64_t ids_nb1, int n_ids, int n_tokens, int n_as,
               int32_t *__restrict__ route, int max_tiles, int tp, float *__restrict__ dst, int64_t dst_nb1,
               int64_t dst_nb2, int rows) {
    extern __shared__ int cnt[];  // [n_as] counts, then [n_as] cursors
    int *cur = cnt + n_as;
    const int n_pairs = n_ids * n_tokens;
    for (int e = threadIdx.x; e < n_as; e += blockDim.x) cnt[e] = 0;
    __shared__ int bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int t = p / n_ids, s = p - t * n_ids;
        const int e = ids[(int64_t)t * ids_nb1 + s];
        if (e >= 0 && e < n_as) atomicAdd(&cnt[e], 1);
        else atomicAdd(&bad, 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int off = 0, nt = 0;
        int32_t *tiles = route + 2 + n_pairs;
        for (int e = 0; e < n_as; e++) {
            cur[e] = off;
            for (int f = 0; f < cnt[e]; f += tp) {
                if (nt < max_tiles) {
                    tiles[3 * nt + 0] = e;
                    tiles[3 * nt + 1] = off + f;
                    tiles[3 * nt + 2] = min(tp, cnt[e] - f);
                }
                nt++;
            }
            off += cnt[e];
        }
        route[0] = min(nt, max_tiles);
        route[1] = bad;
    }
    __syncthreads();
    // scatter; the order inside one expert does not affect any output value
    for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int t = p / n_ids, s = p - t * n_ids;
        const int e = ids[(int64_t)t * ids_nb1 + s];
        if (e >= 0 && e < n_as) {
            route[2 + atomicAdd(&cur[e], 1)] = p;
        } else {
            // no reference value exists (compute.rs:2117 asserts): NaN row
            float *o = dst + (int64_t)t * dst_nb2 + (int64_t)s * dst_nb1;
            for (int r = 0; r < rows; r++) o[r] = __builtin_nanf("");
        }
    }
}

// byte -> {f16(kvalue(lo nibble)), f16(kvalue(hi nibble))} (KVALUES_MXFP4,
// quants.rs:660; the values are small integers, exact in f16)
DEV uint32_t kv_pair_f16(int byte) {
    const int kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)(float)kv[byte & 15]);
    const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)(float)kv[byte >> 4]);
    return lo | (hi << 16);
}

// ---------------------------------------------------------------- GEMM
// grid (tile, row block); 256 threads = 4 wavefronts x 32 expert rows; a tile
// is NMT x 32 pairs of one expert.  MFMA orientation: C[i = pair][j = row]; a
// lane owns row j = lane%32 of its wavefront and 16 pairs per 32-pair block.
// K-slot e of MFMA half m for lane half h2 is element (e&1)*16 + 8m + 4h2 + e/2
// of the 32-block: byte 8m+4h2+e/2 of the block's qs, low nibble for even e,
// high for odd.  REPACK selects the reference's rows % 8 == 0 fold
// (fma(dot, e*d, acc), repack.rs:1071) over the plain one (acc += (d*e)*dot,
// compute.rs:7140).
template <int NMT, bool REPACK, bool SUBSUMS>
__device__ __forceinline__ void moe_mxfp4_impl(const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2,
                                               const uint8_t *__restrict__ act, int64_t act_row_bytes, int ne11,
                                               const int32_t *__restrict__ route, int n_pairs, int n_ids,
                                               float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows,
                                               int nb, int32_t *__restrict__ sub) {
    constexpr int TP = 32 * NMT;
    __shared__ __attribute__((aligned(16))) _Float16 As[MOE_KB * 2 * 2 * TP * 8];  // [kb][m][h2][pair][8]
    __shared__ __attribute__((aligned(16))) float Ds[MOE_KB * TP];                // [kb][pair]
    __shared__ uint32_t lut[256];
    __shared__ int pairs[TP];
    const int tile = blockIdx.x;
    if (tile >= route[0]) return;
    const int32_t *tinfo = route + 2 + n_pairs + 3 * tile;
    const int e = tinfo[0], first = tinfo[1], np = tinfo[2];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int li = lane & 31, h2 = lane >> 5;
    const int row = blockIdx.y * MOE_TR + w * 32 + li;
    const bool rvalid = row < rows;
    if (threadIdx.x < TP) pairs[threadIdx.x] = threadIdx.x < np ? route[2 + first + threadIdx.x] : -1;
    lut[threadIdx.x] = kv_pair_f16(threadIdx.x);
    const uint8_t *wrow = as + (int64_t)e * as_nb2 + (int64_t)(rvalid ? row : 0) * as_nb1;

    float acc[NMT][16];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[mt][v] = 0.0f;

    for (int kb0 = 0; kb0 < nb; kb0 += MOE_KB) {
        const int nkb = min(MOE_KB, nb - kb0);
        // this lane's weight bytes for the group (clamped to the last block)
        uint32_t we[MOE_KB], wq[MOE_KB][2];
#pragma unroll
        for (int kb = 0; kb < MOE_KB; kb++) {
            const uint8_t *wb = wrow + (int64_t)(kb0 + min(kb, nkb - 1)) * MXFP4_BYTES;
            we[kb] = wb[0];
            wq[kb][0] = ld4(wb + 1 + 4 * h2);
            wq[kb][1] = ld4(wb + 1 + 8 + 4 * h2);
        }
        __syncthreads();  // previous group consumed (and pairs / lut visible)
        // stage the Q8_0 codes of the tile's pairs as f16, in K-slot order
        for (int c = threadIdx.x; c < TP * nkb * 4; c += blockDim.x) {
            const int pi = c / (nkb * 4), rest = c - pi * nkb * 4, kb = rest >> 2, q4 = rest & 3;
            const int m = q4 >> 1, hh = q4 & 1;
            const int p = pairs[pi];
            v8h val;
            float dval = 0.0f;
            if (p >= 0) {
                const int t = p / n_ids, s = p - t * n_ids;
                const uint8_t *blk = act + ((int64_t)t * ne11 + (s % ne11)) * act_row_bytes + (int64_t)(kb0 + kb) * Q8_0_BYTES;
                const uint32_t lo = ld4(blk + 2 + 8 * m + 4 * hh);       // elements 8m+4hh .. +3
                const uint32_t hi = ld4(blk + 2 + 16 + 8 * m + 4 * hh);  // elements 16+8m+4hh .. +3
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    val[2 * q] = (_Float16)(float)(int8_t)((lo >> (8 * q)) & 0xff);
                    val[2 * q + 1] = (_Float16)(float)(int8_t)((hi >> (8 * q)) & 0xff);
                }
                dval = h2f(ld2(blk));
            } else {
#pragma unroll
                for (int q = 0; q < 8; q++) val[q] = (_Float16)0.0f;
            }
            if (q4 == 0) Ds[kb * TP + pi] = dval;
            *reinterpret_cast<v8h *>(&As[(((kb * 2 + m) * 2 + hh) * TP + pi) * 8]) = val;
        }
        __syncthreads();
#pragma unroll
        for (int kb = 0; kb < MOE_KB; kb++) {
            if (kb >= nkb) break;
            const int b = kb0 + kb;
            const float sw = e8m0_half(we[kb]);
            v16f c[NMT];
#pragma unroll
            for (int m = 0; m < 2; m++) {
                v8h bw;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t pr = lut[(wq[kb][m] >> (8 * q)) & 0xff];
                    bw[2 * q] = __builtin_bit_cast(_Float16, (uint16_t)(pr & 0xffff));
                    bw[2 * q + 1] = __builtin_bit_cast(_Float16, (uint16_t)(pr >> 16));
                }
#pragma unroll
                for (int mt = 0; mt < NMT; mt++) {
                    const v8h a = *reinterpret_cast<const v8h *>(&As[(((kb * 2 + m) * 2 + h2) * TP + mt * 32 + li) * 8]);
                    if (m == 0) {
                        v16f z;
#pragma unroll
                        for (int v = 0; v < 16; v++) z[v] = 0.0f;
                        c[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bw, z, 0, 0, 0);
                    } else {
                        c[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bw, c[mt], 0, 0, 0);
                    }
                }
            }
            // c[mt][v] is the exact int32 block dot of pair mt*32 + crowm(v)
#pragma unroll
            for (int mt = 0; mt < NMT; mt++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 d4 = *reinterpret_cast<const float4 *>(&Ds[kb * TP + mt * 32 + 8 * g + 4 * h2]);
                    const float dd[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int v = 4 * g + r;
                        const float dot = c[mt][v];
                        if (REPACK) {
                            acc[mt][v] = fmaf(dot, sw * dd[r], acc[mt][v]);
                        } else {
                            acc[mt][v] = acc[mt][v] + (dd[r] * sw) * dot;
                        }
                        if (SUBSUMS && rvalid) {
                            const int pi = mt * 32 + crowm(v, lane);
                            if (pi < np) sub[((int64_t)pairs[pi] * rows + row) * nb + b] = (int)dot;
                        }
                    }
                }
        }
    }
    if (!rvalid) return;
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int pi = mt * 32 + crowm(v, lane);
            if (pi < np) {
                const int p = pairs[pi];
                const int t = p / n_ids, s = p - t * n_ids;
                dst[(int64_t)t * dst_nb2 + (int64_t)s * dst_nb1 + row] = acc[mt][v];
            }
        }
}

#define MOE_ARGS                                                                                              \
    const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2, const uint8_t *__restrict__ act,          \
        int64_t act_row_bytes, int ne11, const int32_t *__restrict__ route, int n_pairs, int n_ids,            \
        float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows, int nb, int32_t *__restrict__ sub
#define MOE_PASS as, as_nb1, as_nb2, act, act_row_bytes, ne11, route, n_pairs, n_ids, dst, dst_nb1, dst_nb2, rows, nb, sub

#define MOE_KERNEL(name, NMT, REPACK, SUB) \
    extern "C" __global__ void __launch_bounds__(256) name(MOE_ARGS) { moe_mxfp4_impl<NMT, REPACK, SUB>(MOE_PASS); }
MOE_KERNEL(ghip_moe_mxfp4_t32, 1, true, false)
MOE_KERNEL(ghip_moe_mxfp4_t64, 2, true, false)
MOE_KERNEL(ghip_moe_mxfp4_t32_plain, 1, false, false)
MOE_KERNEL(ghip_moe_mxfp4_t64_plain, 2, false, false)
MOE_KERNEL(ghip_moe_mxfp4_t32_sub, 1, true, true)
MOE_KERNEL(ghip_moe_mxfp4_t32_plain_sub, 1, false, true)
