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
#include <type_traits>
#include "ghip_common.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int MOE_TR = 128;  // expert rows per workgroup (32 per wavefront)

DEV int crowm(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// ---------------------------------------------------------------- routing
// One workgroup: counting sort of the (token, slot) pairs by expert id and
// the tile list of the GEMM (tiles of at most tp pairs of one expert), the
// list built by the first wavefront with prefix sums over the experts
// (config 4: 9.5 -> 5.4 us against one thread walking the experts).  route layout (int32):
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
    if (threadIdx.x < 64) {
        // experts in chunks of 64 lanes: an exclusive scan of the pair counts
        // (each expert's first routed slot) and of the tile counts (its first
        // tile), then every lane writes its expert's tiles
        const int lane = threadIdx.x;
        int off = 0, nt = 0;
        int32_t *tiles = route + 2 + n_pairs;
        for (int e0 = 0; e0 < n_as; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < n_as ? cnt[e] : 0;
            const int ntl = (c + tp - 1) / tp;
            int sc = c, st = ntl;  // inclusive scans
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int a = __shfl_up(sc, o, 64), b = __shfl_up(st, o, 64);
                if (lane >= o) {
                    sc += a;
                    st += b;
                }
            }
            const int my_off = off + sc - c, my_t0 = nt + st - ntl;
            if (e < n_as) {
                cur[e] = my_off;
                for (int f = 0, k = my_t0; f < c; f += tp, k++)
                    if (k < max_tiles) {
                        tiles[3 * k + 0] = e;
                        tiles[3 * k + 1] = my_off + f;
                        tiles[3 * k + 2] = min(tp, c - f);
                    }
            }
            off += __shfl(sc, 63, 64);
            nt += __shfl(st, 63, 64);
        }
        if (lane == 0) {
            route[0] = min(nt, max_tiles);
            route[1] = bad;
        }
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

// Eight MXFP4 codes (the nibbles of x) -> their kvalues as f16, slot order
// [lo(b0), hi(b0), lo(b1), hi(b1), ...], with the magnitudes scaled by 2^k:
// the f16 of |kvalue| in {0,1,2,3,4,6,8,12} differ only in the high byte
// (00 3C 40 42 44 46 48 4A), so one v_perm over an 8-byte table gives four of
// them at once; 2^k adds 4k to every non-zero table byte (exact while
// 2^-14 <= 2^k and 12 * 2^k < 2^16), and the sign is bit 3 of the nibble.
DEV uint4 kv_expand(uint32_t x, uint32_t t0, uint32_t t1) {
    const uint32_t hbl = __builtin_amdgcn_perm(t1, t0, x & 0x07070707u) | ((x << 4) & 0x80808080u);
    const uint32_t hbh = __builtin_amdgcn_perm(t1, t0, (x >> 4) & 0x07070707u) | (x & 0x80808080u);
    uint4 r;
    r.x = __builtin_amdgcn_perm(hbh, hbl, 0x040C000Cu);
    r.y = __builtin_amdgcn_perm(hbh, hbl, 0x050C010Cu);
    r.z = __builtin_amdgcn_perm(hbh, hbl, 0x060C020Cu);
    r.w = __builtin_amdgcn_perm(hbh, hbl, 0x070C030Cu);
    return r;
}

// ---------------------------------------------------------------- activations
// Q8_0 activation rows -> f16 codes in MFMA K-slot order (exact: |q| <= 128),
// once per call and per (token, slot) pair, in the routed order (after
// ghip_moe_route), so that a tile's pairs are consecutive rows:
// actf [slot][block][4 pieces][8 f16], piece (m, h2) slot e holding element
// (e&1)*16 + 8m + 4*h2 + e/2; actd [slot][block] = d as f32.  Pair
// p = t * n_ids + s reads activation row t * ne11 + s % ne11.
extern "C" __global__ void __launch_bounds__(256)
ghip_moe_act_f16(const uint8_t *__restrict__ q8, int64_t q8_row_bytes, const int32_t *__restrict__ route,
                 int n_pairs, int n_ids, int ne11, int nb, _Float16 *__restrict__ actf, float *__restrict__ actd) {
    const int64_t task = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (slot, block, piece)
    const int n_valid = n_pairs - route[1];                         // pairs with a valid expert id
    if (task >= (int64_t)n_valid * nb * 4) return;
    const int piece = (int)(task & 3);
    const int64_t rb = task >> 2;
    const int64_t slot = rb / nb;
    const int b = (int)(rb - slot * nb);
    const int m = piece >> 1, hh = piece & 1;
    const int p = route[2 + slot], t = p / n_ids, sl = p - t * n_ids;
    const int64_t row = (int64_t)t * ne11 + sl % ne11;
    const uint8_t *blk = q8 + row * q8_row_bytes + (int64_t)b * Q8_0_BYTES;
    const uint32_t lo = ld4(blk + 2 + 8 * m + 4 * hh);       // elements 8m+4hh .. +3
    const uint32_t hi = ld4(blk + 2 + 16 + 8 * m + 4 * hh);  // elements 16+8m+4hh .. +3
    v8h val;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        val[2 * q] = (_Float16)(float)(int8_t)((lo >> (8 * q)) & 0xff);
        val[2 * q + 1] = (_Float16)(float)(int8_t)((hi >> (8 * q)) & 0xff);
    }
    *reinterpret_cast<v8h *>(actf + (rb * 4 + piece) * 8) = val;
    if (piece == 0) actd[rb] = h2f(ld2(blk));
}

// ---------------------------------------------------------------- GEMM
// grid (tile, row block); 256 threads = 4 wavefronts x 32 expert rows; a tile
// is NMT x 32 pairs of one expert.  MFMA orientation: C[i = pair][j = row]; a
// lane owns row j = lane%32 of its wavefront and 16 pairs per 32-pair block.
// K-slot e of MFMA half m for lane half h2 is element (e&1)*16 + 8m + 4h2 + e/2
// of the 32-block: byte 8m+4h2+e/2 of the block's qs, low nibble for even e,
// high for odd.  Per group of MOE_GB blocks, the expert rows' 68-byte windows,
// the tile's pre-expanded f16 activation codes and their scales are staged in
// LDS by direct global->LDS loads, one group ahead (about 38 KB per
// workgroup, four workgroups per CU).  REPACK selects the reference's rows % 8 == 0 fold
// (fma(dot, e*d, acc), repack.rs:1071) over the plain one (acc += (d*e)*dot,
// compute.rs:7140).
constexpr int MOE_GB = 4;                               // 32-blocks per staging group
constexpr int MOE_WB = 17 * MOE_GB;                     // weight window bytes per row and group
constexpr int MOE_WIN = (MOE_WB + 4 + 15) / 16;         // 16-byte loads per window (+ the dword the last reads touch)
static_assert(MOE_WIN * 16 >= 17 * MOE_GB, "the registered window (qs at 16kb, e bytes after) fits");

template <int NMT, bool REPACK, bool SUBSUMS>
__device__ __forceinline__ void moe_mxfp4_impl(const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2,
                                               const _Float16 *__restrict__ actf, const float *__restrict__ actd,
                                               int ne11, const int32_t *__restrict__ route, int n_pairs, int n_ids,
                                               float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows,
                                               int nb, int32_t *__restrict__ sub) {
    constexpr int TP = 32 * NMT;
    __shared__ __attribute__((aligned(16))) float ds_lds[2][MOE_GB][TP];  // [stage][block][pair] activation scales
    __shared__ __attribute__((aligned(16))) uint4 a_lds[2][MOE_GB][4][TP];  // [stage][block][piece][pair] 8 f16 each
    __shared__ __attribute__((aligned(16))) uint32_t w_lds[2][MOE_TR][MOE_WIN * 4];  // [stage][row][window]
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
    __syncthreads();
    __syncthreads();
    const uint8_t *wrow = as + (int64_t)e * as_nb2 + (int64_t)(rvalid ? row : 0) * as_nb1;
    const int row_bytes = nb * MXFP4_BYTES;

    // Staging of group g (MOE_GB blocks) into LDS stage g&1 with direct global->LDS
    // loads (no registers, no LDS stores): the three layouts are contiguous in
    // the thread index, chunk i = c*256 + tid at byte 16i (weights, A) or 4i
    // (scales), so instruction c of wavefront w writes the 1 KB (256 B) at
    // chunk c*256 + 64w.
    //   A:      chunk i -> pair i % TP, block kb = (i / TP) >> 2, piece (i / TP) & 3
    //   scales: chunk i -> pair i % TP, block kb = i / TP
    //   window: chunk i -> row i / 9, 16-byte piece i % 9
    // Padding pairs and blocks past the row read a valid row (the tile's first
    // pair, the last block): those lanes' MFMA rows and folds are discarded.
    constexpr int ACHUNK = MOE_GB * 4 * TP / 256;        // 16-byte chunks per thread per group
    constexpr int DCH = (MOE_GB * TP + 255) / 256;       // scale chunks per thread per group
    static_assert(256 % TP == 0, "one pair per thread");
    const int my_pi = threadIdx.x % TP;
    const int my_slot = first + (my_pi < np ? my_pi : 0);
    const _Float16 *my_arow = actf + (int64_t)my_slot * nb * 32;
    const float *my_drow = actd + (int64_t)my_slot * nb;
    constexpr int WCHUNK = (MOE_TR * MOE_WIN + 255) / 256;
    const uint8_t *wexp = as + (int64_t)e * as_nb2;
    const uint8_t *wbase[WCHUNK];
    int wl16[WCHUNK];
#pragma unroll
    for (int c = 0; c < WCHUNK; c++) {
        const int idx = c * 256 + threadIdx.x;
        const int r = idx / MOE_WIN, l = idx - r * MOE_WIN;
        wbase[c] = wexp + (int64_t)min((int)blockIdx.y * MOE_TR + r, rows - 1) * as_nb1;
        wl16[c] = 16 * l;
    }
    const int wv = threadIdx.x >> 6;
    auto issue = [&](int g, int stage, bool with_w) {
#pragma unroll
        for (int c = 0; c < ACHUNK; c++) {
            const int rest = (c * 256 + (int)threadIdx.x) / TP;
            const int piece = rest & 3, b = min(MOE_GB * g + (rest >> 2), nb - 1);
            g2lds(my_arow + ((int64_t)b * 4 + piece) * 8,
                  reinterpret_cast<uint8_t *>(&a_lds[stage][0][0][0]) + (c * 256 + 64 * wv) * 16);
        }
#pragma unroll
        for (int c = 0; c < DCH; c++) {
            if (c * 256 + 64 * wv >= MOE_GB * TP) continue;  // whole wavefronts
            const int b = min(MOE_GB * g + (c * 256 + (int)threadIdx.x) / TP, nb - 1);
            __builtin_amdgcn_global_load_lds(my_drow + b,
                                             (lds_void *)(reinterpret_cast<uint8_t *>(&ds_lds[stage][0][0]) +
                                                          (c * 256 + 64 * wv) * 4),
                                             4, 0, 0);
        }
        if (with_w) {
#pragma unroll
            for (int c = 0; c < WCHUNK; c++)
                if (c * 256 + 64 * wv < MOE_TR * MOE_WIN)  // whole wavefronts in or out
                    g2lds(wbase[c] + min(MOE_WB * g + wl16[c], row_bytes - 16),
                          reinterpret_cast<uint8_t *>(&w_lds[stage][0][0]) + (c * 256 + 64 * wv) * 16);
        }
    };
    float acc[NMT][16];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[mt][v] = 0.0f;

    // one block: dots on the f16 matrix cores, then the reference's fold.
    // Fast path (every row of the wavefront has k = e - 128 in [-14, 12]): the
    // block scale 2^k is folded into the weight operand, so the MFMA returns
    // dot * 2^k exactly and the fold is fma(dot * 2^k, d, acc) -- the same
    // real value as the reference's fma(dot, 2^k * d, acc) (2^k * d is exact),
    // hence the same rounding.  Otherwise the exact dot and the reference's
    // own fold.  The sub-sum instantiations always take the exact dot.
    auto dots = [&](uint32_t k4, uint32_t q0, uint32_t q1, const v8h (&a)[NMT][2], v16f (&c)[NMT]) {
        // k4 * 0x01010101 (mod 2^32) by shift-adds (full rate, no v_mul_lo_u32)
        const uint32_t y = k4 + (k4 << 8), z = y + (y << 16);
        const uint32_t t0 = 0x42403C00u + (z << 8), t1 = 0x4A484644u + z;
        const uint32_t qm[2] = {q0, q1};
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const v8h bw = __builtin_bit_cast(v8h, kv_expand(qm[m], t0, t1));
#pragma unroll
            for (int mt = 0; mt < NMT; mt++) {
                const v16f z = {};
                c[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mt][m], bw, m ? c[mt] : z, 0, 0, 0);
            }
        }
    };
    // fast path (FAST): the block scale 2^k is in the weight operand, the MFMA
    // returns dot * 2^k exactly and the fold is fma(dot * 2^k, d, acc), the
    // real value of the reference's fma(dot, 2^k * d, acc) (2^k * d exact).
    // Exact path: the integer dot and the reference's own fold.
    auto fold_block = [&](auto FAST, int b, const float *dsb, uint32_t e8, const v16f (&c)[NMT]) {
        constexpr bool fast = decltype(FAST)::value;
        const float sw = e8m0_half(e8);
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 d4 = *reinterpret_cast<const float4 *>(&dsb[mt * 32 + 8 * g + 4 * h2]);
                const float dd[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int v = 4 * g + r;
                    const float dot = c[mt][v];
                    if (fast) {
                        if (REPACK) acc[mt][v] = fmaf(dot, dd[r], acc[mt][v]);
                        else acc[mt][v] = acc[mt][v] + dd[r] * dot;
                    } else if (REPACK) {
                        acc[mt][v] = fmaf(dot, sw * dd[r], acc[mt][v]);
                    } else {
                        acc[mt][v] = acc[mt][v] + (dd[r] * sw) * dot;
                    }
                    if (!fast && SUBSUMS && rvalid) {
                        const int pi = mt * 32 + crowm(v, lane);
                        if (pi < np) sub[((int64_t)pairs[pi] * rows + row) * nb + b] = (int)dot;
                    }
                }
            }
    };
    auto do_block = [&](auto FAST, int b, const float *dsb, uint32_t e8, uint32_t q0, uint32_t q1,
                        const v8h (&a)[NMT][2]) {
        constexpr bool fast = decltype(FAST)::value;
        v16f c[NMT];
        dots(fast ? 4u * (e8 - 128u) : 0u, q0, q1, a, c);
        fold_block(FAST, b, dsb, e8, c);
    };
    // the 2^k fold holds for k = e - 128 in [-14, 12]
    auto in_range = [](uint32_t e8) { return e8 >= 114u && e8 <= 140u; };

    // full windows that end inside the row; the rest are tail blocks
    int ngroups = nb / MOE_GB;
    while (ngroups > 0 && MOE_WB * (ngroups - 1) + 16 * MOE_WIN > row_bytes) ngroups--;
    const int nga = (nb + MOE_GB - 1) / MOE_GB;  // activation groups (the tail included)
    auto a_of = [&](int stage, int kb, v8h (&a)[NMT][2]) {
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
#pragma unroll
            for (int m = 0; m < 2; m++) a[mt][m] = __builtin_bit_cast(v8h, a_lds[stage][kb][2 * m + h2][mt * 32 + li]);
    };
    // group g+1 lands in LDS stage (g+1)&1 while group g is multiplied
    const int rl = w * 32 + li;  // this lane's row inside the workgroup
    issue(0, 0, ngroups > 0);
    for (int g = 0; g < nga; g++) {
        const int stage = g & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's share of group g is in LDS
        __syncthreads();  // ... every thread's; and stage ^ 1 (group g-1) is no longer read
        if (g + 1 < nga) issue(g + 1, stage ^ 1, g + 1 < ngroups);
        if (g < ngroups) {
            const uint32_t *wl = w_lds[stage][rl];
            // the row's whole window (17-byte blocks from byte 0; 20 dwords)
            uint32_t W[4 * MOE_WIN];
#pragma unroll
            for (int i = 0; i < MOE_WIN; i++) {
                const uint4 t = reinterpret_cast<const uint4 *>(wl)[i];
                W[4 * i] = t.x; W[4 * i + 1] = t.y; W[4 * i + 2] = t.z; W[4 * i + 3] = t.w;
            }
            // block kb: e at byte 17kb (byte kb of dword 4kb), qs at 17kb+1; this
            // lane half needs qs bytes 4h2.. (m = 0) and 8+4h2.. (m = 1)
            auto e_of = [&](int kb) { return (W[(17 * kb) >> 2] >> (8 * ((17 * kb) & 3))) & 0xffu; };
            auto q_of = [&](int kb, int m) {
                const int o = 17 * kb + 1 + 8 * m, d = o >> 2, sh = o & 3;
                const uint32_t lo = h2 ? W[d + 1] : W[d], hi = h2 ? W[d + 2] : W[d + 1];
                return __builtin_amdgcn_alignbyte(hi, lo, sh);
            };
            // software-pipelined: the dots of block kb are issued before the
            // fold of block kb-1, whose MFMA results are ready by then
            auto window = [&](auto FAST) {
                constexpr bool fast = decltype(FAST)::value;
                v16f c[2][NMT];
#pragma unroll
                for (int kb = 0; kb < MOE_GB; kb++) {
                    v8h a[NMT][2];
                    a_of(stage, kb, a);
                    dots(fast ? 4u * (e_of(kb) - 128u) : 0u, q_of(kb, 0), q_of(kb, 1), a, c[kb & 1]);
                    if (kb > 0)
                        fold_block(FAST, MOE_GB * g + kb - 1, ds_lds[stage][kb - 1], e_of(kb - 1), c[(kb - 1) & 1]);
                }
                fold_block(FAST, MOE_GB * g + MOE_GB - 1, ds_lds[stage][MOE_GB - 1], e_of(MOE_GB - 1),
                           c[(MOE_GB - 1) & 1]);
            };
            // one decision per window for the whole wavefront
            bool ok = !SUBSUMS;
#pragma unroll
            for (int kb = 0; kb < MOE_GB; kb++) ok = ok && in_range(e_of(kb));
            if (__ballot(!ok) == 0) window(std::true_type{});
            else window(std::false_type{});
        } else {
            for (int kb = 0; kb < MOE_GB && MOE_GB * g + kb < nb; kb++) {  // tail blocks: exact loads, exact path
                const uint8_t *wb = wrow + (int64_t)(MOE_GB * g + kb) * MXFP4_BYTES;
                v8h a[NMT][2];
                a_of(stage, kb, a);
                do_block(std::false_type{}, MOE_GB * g + kb, ds_lds[stage][kb], wb[0], ld4(wb + 1 + 4 * h2),
                         ld4(wb + 9 + 4 * h2), a);
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
    const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2, const _Float16 *__restrict__ actf,        \
        const float *__restrict__ actd, int ne11, const int32_t *__restrict__ route, int n_pairs, int n_ids,   \
        float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows, int nb, int32_t *__restrict__ sub
#define MOE_PASS as, as_nb1, as_nb2, actf, actd, ne11, route, n_pairs, n_ids, dst, dst_nb1, dst_nb2, rows, nb, sub

#define MOE_KERNEL(name, NMT, REPACK, SUB) \
    extern "C" __global__ void __launch_bounds__(256) name(MOE_ARGS) { moe_mxfp4_impl<NMT, REPACK, SUB>(MOE_PASS); }
MOE_KERNEL(ghip_moe_mxfp4_t32, 1, true, false)
MOE_KERNEL(ghip_moe_mxfp4_t64, 2, true, false)
MOE_KERNEL(ghip_moe_mxfp4_t32_plain, 1, false, false)
MOE_KERNEL(ghip_moe_mxfp4_t64_plain, 2, false, false)
MOE_KERNEL(ghip_moe_mxfp4_t32_sub, 1, true, true)
MOE_KERNEL(ghip_moe_mxfp4_t32_plain_sub, 1, false, true)

// ------------------------------------------------- scaled FP4 matrix cores
// The same MUL_MAT_ID on v_mfma_scale_f32_32x32x64_f8f6f4: the MXFP4 nibbles
// are the FP4 (E2M1) A operand as they lie in memory (E2M1 values are the
// kvalues / 2), and the Q8_0 codes enter as two exact FP8 (E4M3) planes,
// q = ql + 16 * qh with ql = q & 15 and qh = q >> 4, in the two K halves of
// one instruction: A holds the block's 32 weights in both halves, B the ql
// plane (scale 2^0) and the qh plane (scale 2^4), so one MFMA returns
// sum kvalue * q * 2^(e - 128) = dot * e8m0_half(e) exactly per 32-block
// (A's scale is the block's own E8M0 byte; every partial sum is an integer
// times a power of two below 2^24 of it).  The fold is then the reference's
// fma(dot, e8m0_half(e) * d, acc) with the exact product dot * 2^k
// (fma(dot * 2^k, d, acc), the fast path of moe_mxfp4_impl) for k = e - 128
// in [-14, 12]; other windows and the sub-sum kernels take A's scale 2^0
// (dot / 2, exact) and the reference's own fold.
//
// K order inside a lane: FP4 nibble n of the 16 qs bytes is element n / 2
// (n even) or 16 + n / 2 (n odd) of the block (low nibble of qs[j] is element
// j, the high one element j + 16); the FP8 planes use the same order.

// E4M3 bytes of 0..15
DEV uint32_t e4m3_small(uint32_t v) {
    constexpr uint64_t lo = 0x4E4C4A4844403800ull, hi = 0x5756555453525150ull;
    return (uint32_t)(((v < 8 ? lo : hi) >> (8 * (v & 7))) & 0xff);
}

// Q8_0 rows -> the two FP8 planes in MFMA K order, per (routed slot, block):
// four 16-byte pieces (plane h, piece j) = 2h + j, piece j holding K positions
// 16j..16j+15 (elements 8j..8j+7 interleaved with 16+8j..16+8j+7), stored
// actq [block][piece][slot]; actd [block][slot] = d.
extern "C" __global__ void __launch_bounds__(256)
ghip_moe_act_fp8(const uint8_t *__restrict__ q8, int64_t q8_row_bytes, const int32_t *__restrict__ route,
                 int n_pairs, int n_ids, int ne11, int nb, uint8_t *__restrict__ actq, float *__restrict__ actd) {
    const int64_t task = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (slot, block, piece)
    const int n_valid = n_pairs - route[1];
    if (task >= (int64_t)n_valid * nb * 4) return;
    const int piece = (int)(task & 3), hplane = piece >> 1, j = piece & 1;
    const int64_t rb = task >> 2;
    const int64_t slot = rb / nb;
    const int b = (int)(rb - slot * nb);
    const int p = route[2 + slot], t = p / n_ids, sl = p - t * n_ids;
    const int64_t row = (int64_t)t * ne11 + sl % ne11;
    const uint8_t *blk = q8 + row * q8_row_bytes + (int64_t)b * Q8_0_BYTES;
    const uint2 lo = ld8(blk + 2 + 8 * j), hi = ld8(blk + 2 + 16 + 8 * j);
    const uint32_t lw[2] = {lo.x, lo.y}, hw[2] = {hi.x, hi.y};
    uint32_t out[4];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int qa = (int)(int8_t)(lw[i >> 2] >> (8 * (i & 3)));
        const int qb = (int)(int8_t)(hw[i >> 2] >> (8 * (i & 3)));
        uint32_t ba, bb;
        if (hplane == 0) {
            ba = e4m3_small((uint32_t)(qa & 15));
            bb = e4m3_small((uint32_t)(qb & 15));
        } else {
            const int ha = qa >> 4, hb = qb >> 4;  // -8 .. 7
            ba = e4m3_small((uint32_t)(ha < 0 ? -ha : ha)) | (ha < 0 ? 0x80u : 0u);
            bb = e4m3_small((uint32_t)(hb < 0 ? -hb : hb)) | (hb < 0 ? 0x80u : 0u);
        }
        const uint32_t pair = ba | (bb << 8);  // K positions 2i, 2i+1
        if ((i & 1) == 0) out[i >> 1] = pair;
        else out[i >> 1] |= pair << 16;
    }
    // [block][piece][slot]: a tile's consecutive slots are consecutive 16-byte chunks
    *reinterpret_cast<uint4 *>(actq + (((int64_t)b * 4 + piece) * n_pairs + slot) * 16) =
        make_uint4(out[0], out[1], out[2], out[3]);
    if (piece == 0) actd[(int64_t)b * n_pairs + slot] = h2f(ld2(blk));
}

// The same planes straight from the f32 rows of src1: each 4-lane group of
// tasks shares one (slot, block) and quantizes it with ghip_quantize_q8_0's
// arithmetic (quantize_row_q8_0, quants.rs:331-362: amax over the block,
// d = f16(amax / 127), q = rne(x * 127 / amax), NaN or out of range -> -128),
// so the codes and d equal a Q8_0 pass followed by ghip_moe_act_fp8 and the
// separate quantization launch is not needed.  x_nb1 / x_nb2: floats between
// src1 rows / tokens.
extern "C" __global__ void __launch_bounds__(256)
ghip_moe_act_fp8_f(const float *__restrict__ x, int64_t x_nb1, int64_t x_nb2, const int32_t *__restrict__ route,
                   int n_pairs, int n_ids, int ne11, int nb, uint8_t *__restrict__ actq, float *__restrict__ actd) {
    const int64_t task = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (slot, block, piece)
    const int n_valid = n_pairs - route[1];
    if (task >= (int64_t)n_valid * nb * 4) return;  // whole 4-lane groups exit together
    const int piece = (int)(task & 3), hplane = piece >> 1, j = piece & 1;
    const int64_t rb = task >> 2;
    const int64_t slot = rb / nb;
    const int b = (int)(rb - slot * nb);
    const int p = route[2 + slot], t = p / n_ids, sl = p - t * n_ids;
    const float *xb = x + (int64_t)t * x_nb2 + (int64_t)(sl % ne11) * x_nb1 + (int64_t)b * 32;
    float v[16];  // elements 8j .. 8j+7, then 16 + 8j .. 16 + 8j + 7
    __builtin_memcpy(v, xb + 8 * j, 32);
    __builtin_memcpy(v + 8, xb + 16 + 8 * j, 32);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));  // the other half of the block (piece ^ 1)
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    auto code = [&](float xv) {
        const float r = rintf(__fmul_rn(xv, id));
        const int q = (r != r || fabsf(r) >= 2147483648.0f) ? -128 : (int)r;
        return (int)(int8_t)(q & 0xff);
    };
    uint32_t out[4];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int qa = code(v[i]), qb = code(v[8 + i]);
        uint32_t ba, bb;
        if (hplane == 0) {
            ba = e4m3_small((uint32_t)(qa & 15));
            bb = e4m3_small((uint32_t)(qb & 15));
        } else {
            const int ha = qa >> 4, hb = qb >> 4;  // -8 .. 7
            ba = e4m3_small((uint32_t)(ha < 0 ? -ha : ha)) | (ha < 0 ? 0x80u : 0u);
            bb = e4m3_small((uint32_t)(hb < 0 ? -hb : hb)) | (hb < 0 ? 0x80u : 0u);
        }
        const uint32_t pair = ba | (bb << 8);  // K positions 2i, 2i+1
        if ((i & 1) == 0) out[i >> 1] = pair;
        else out[i >> 1] |= pair << 16;
    }
    *reinterpret_cast<uint4 *>(actq + (((int64_t)b * 4 + piece) * n_pairs + slot) * 16) =
        make_uint4(out[0], out[1], out[2], out[3]);
    if (piece == 0) actd[(int64_t)b * n_pairs + slot] = h2f(f2h_rn(d));
}

typedef int v8i __attribute__((ext_vector_type(8)));

// grid (tile, row block of 128); 4 wavefronts x 32 expert rows; a tile is 32
// pairs of one expert.  C[row][pair]: lane l holds pair l % 32 and the rows
// crowm(v, l) of its wavefront's 32.  Staging as moe_mxfp4_impl (weight
// windows of 4 blocks, the tile's planes and scales, one group ahead).
template <int NMT, bool REPACK, bool SUBSUMS, bool REG>
__device__ __forceinline__ void moe_fp4_impl(const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2,
                                             const uint8_t *__restrict__ actq, const float *__restrict__ actd,
                                             int ne11, const int32_t *__restrict__ route, int n_pairs, int n_ids,
                                             float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows,
                                             int nb, int32_t *__restrict__ sub, const uint8_t *__restrict__ wrep,
                                             int ngp, int order) {
    constexpr int TP = 32 * NMT;
    static_assert(256 % TP == 0, "one pair per thread");
    // One LDS variable per pipeline stage, every access naming its stage at
    // compile time: the compiler then knows that the next stage's LDS-DMA
    // writes do not alias this stage's reads, and does not wait for them
    // (one [2][..] array indexed at run time made it wait for the prefetch
    // before every read of the current stage)
    __shared__ __attribute__((aligned(16))) float ds_lds0[MOE_GB][TP], ds_lds1[MOE_GB][TP];
    __shared__ __attribute__((aligned(16))) uint4 a_lds0[MOE_GB][4][TP], a_lds1[MOE_GB][4][TP];  // [block][piece][pair]
    __shared__ __attribute__((aligned(16))) uint32_t w_lds0[MOE_TR][MOE_WIN * 4], w_lds1[MOE_TR][MOE_WIN * 4];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto A_ = [&](auto st) -> decltype(a_lds0) & { if constexpr (decltype(st)::value == 0) return a_lds0; else return a_lds1; };
    auto D_ = [&](auto st) -> decltype(ds_lds0) & { if constexpr (decltype(st)::value == 0) return ds_lds0; else return ds_lds1; };
    auto W_ = [&](auto st) -> decltype(w_lds0) & { if constexpr (decltype(st)::value == 0) return w_lds0; else return w_lds1; };
    __shared__ int pairs[TP];
    // Workgroups go to the 8 XCDs round-robin by linear id.  With a grid whose
    // size is a multiple of 8 (the host pads the tile count), order 1 remaps
    // so each XCD takes a contiguous run of (row block, tile) ids, tiles
    // fastest: the tiles of one expert (an expert with more than TP pairs has
    // several) then read the same rows of weights on one XCD close together.
    // Config 4 gate_up, registered: 147.1 us without the remap, 136.3 us with
    // it (L2 fetch 555 -> 529 MB); order 2 (row blocks fastest, an expert's
    // pair activations kept in L2) fetches 459 MB but takes 145.1 us.
    int tile = blockIdx.x, yb = blockIdx.y;
    {
        const int total = gridDim.x * gridDim.y, lin = blockIdx.y * gridDim.x + blockIdx.x;
        if ((total & 7) == 0 && order != 0) {
            const int l2 = (lin & 7) * (total >> 3) + (lin >> 3);
            if (order == 1) {
                tile = l2 % gridDim.x;
                yb = l2 / gridDim.x;
            } else {
                yb = l2 % gridDim.y;
                tile = l2 / gridDim.y;
            }
        }
    }
    if (tile >= route[0]) return;
    const int32_t *tinfo = route + 2 + n_pairs + 3 * tile;
    const int e = tinfo[0], first = tinfo[1], np = tinfo[2];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int li = lane & 31, h2 = lane >> 5;
    const int row0 = yb * MOE_TR + w * 32;  // this wavefront's first row
    if (threadIdx.x < TP) pairs[threadIdx.x] = threadIdx.x < np ? route[2 + first + threadIdx.x] : -1;
    const int row_bytes = nb * MXFP4_BYTES;

    constexpr int ACHUNK = MOE_GB * 4 * TP / 256;
    constexpr int DCH = (MOE_GB * TP + 255) / 256;
    const int my_pi = threadIdx.x % TP;
    const int my_slot = first + (my_pi < np ? my_pi : 0);
    const uint8_t *my_arow = actq + (int64_t)my_slot * 16;  // + (block * 4 + piece) * n_pairs * 16
    const float *my_drow = actd + my_slot;                   // + block * n_pairs
    constexpr int WCHUNK = (MOE_TR * MOE_WIN + 255) / 256;
    const uint8_t *wexp = as + (int64_t)e * as_nb2;
    const uint8_t *wbase[WCHUNK];
    int wl16[WCHUNK];
#pragma unroll
    for (int c = 0; c < WCHUNK; c++) {
        const int idx = c * 256 + threadIdx.x;
        const int r = idx / MOE_WIN, l = idx - r * MOE_WIN;
        wbase[c] = wexp + (int64_t)min(yb * MOE_TR + r, rows - 1) * as_nb1;
        wl16[c] = 16 * l;
    }
    const int wv = threadIdx.x >> 6;
    auto issue = [&](int g, auto stage, bool with_w) {
#pragma unroll
        for (int c = 0; c < ACHUNK; c++) {
            const int rest = (c * 256 + (int)threadIdx.x) / TP;
            const int piece = rest & 3, b = min(MOE_GB * g + (rest >> 2), nb - 1);
            g2lds(my_arow + ((int64_t)b * 4 + piece) * n_pairs * 16,
                  reinterpret_cast<uint8_t *>(&A_(stage)[0][0][0]) + (c * 256 + 64 * wv) * 16);
        }
#pragma unroll
        for (int c = 0; c < DCH; c++) {
            if (c * 256 + 64 * wv >= MOE_GB * TP) continue;
            const int b = min(MOE_GB * g + (c * 256 + (int)threadIdx.x) / TP, nb - 1);
            __builtin_amdgcn_global_load_lds(my_drow + (int64_t)b * n_pairs,
                                             (lds_void *)(reinterpret_cast<uint8_t *>(&D_(stage)[0][0]) +
                                                          (c * 256 + 64 * wv) * 4),
                                             4, 0, 0);
        }
        if (REG) {  // registered copy: the group's windows are one contiguous run in LDS order
            const uint8_t *src = wrep + (((int64_t)e * gridDim.y + yb) * ngp + g) * (MOE_TR * MOE_WIN * 16);
#pragma unroll
            for (int c = 0; c < WCHUNK; c++)
                if (c * 256 + 64 * wv < MOE_TR * MOE_WIN)
                    g2lds(src + (c * 256 + (int)threadIdx.x) * 16,
                          reinterpret_cast<uint8_t *>(&W_(stage)[0][0]) + (c * 256 + 64 * wv) * 16);
        } else if (with_w) {
#pragma unroll
            for (int c = 0; c < WCHUNK; c++)
                if (c * 256 + 64 * wv < MOE_TR * MOE_WIN)
                    g2lds(wbase[c] + min(MOE_WB * g + wl16[c], row_bytes - 16),
                          reinterpret_cast<uint8_t *>(&W_(stage)[0][0]) + (c * 256 + 64 * wv) * 16);
        }
    };
    float acc[NMT][16];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[mt][v] = 0.0f;
    const v16f zero = {};
    const int scale_b = h2 ? 127 + 4 : 127;  // ql plane x 1, qh plane x 16
    // E8M0 127 (2^0) held in a VGPR: a constant scale operand would be encoded
    // as an f32 inline constant
    int s127;
    asm volatile("v_mov_b32 %0, 127" : "=v"(s127));

    // dots of one block: A = the 16 qs bytes of row li, B = this lane's plane
    auto mfma = [&](const uint32_t (&q)[4], int scale_a, auto stage, int kb, int mt) {
        // B lane half h2: bytes 0..15 = K 16h2.. (ql piece h2), bytes 16..31 =
        // K 32+16h2.. (qh piece h2); A lane half h holds K 32h..32h+31
        const uint4 b0 = A_(stage)[kb][h2][mt * 32 + li], b1 = A_(stage)[kb][2 + h2][mt * 32 + li];
        const v8i A = {(int)q[0], (int)q[1], (int)q[2], (int)q[3], 0, 0, 0, 0};
        const v8i B = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B, zero, 4, 0, 0, scale_a, 0, scale_b);
    };
    // fast fold: c = dot * 2^k, acc = fma(c, d, acc) (REPACK) or acc + d * c
    auto fold_fast = [&](const v16f &c, float d, int mt) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            if (REPACK) acc[mt][v] = fmaf(c[v], d, acc[mt][v]);
            else acc[mt][v] = acc[mt][v] + d * c[v];
        }
    };
    // exact fold: c = dot / 2; the row scales come from the lanes holding the rows
    auto fold_exact = [&](const v16f &c, float d, uint32_t e8, int b, int mt) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = crowm(v, lane);
            const float sw = e8m0_half((uint32_t)__shfl((int)e8, r, 64));
            const float dot = 2.0f * c[v];
            if (REPACK) acc[mt][v] = fmaf(dot, sw * d, acc[mt][v]);
            else acc[mt][v] = acc[mt][v] + (d * sw) * dot;
            if (SUBSUMS && mt * 32 + li < np && row0 + r < rows)
                sub[((int64_t)pairs[mt * 32 + li] * rows + row0 + r) * nb + b] = (int)dot;
        }
    };
    auto in_range = [](uint32_t e8) { return e8 >= 114u && e8 <= 140u; };

    int ngroups = nb / MOE_GB;
    while (ngroups > 0 && MOE_WB * (ngroups - 1) + 16 * MOE_WIN > row_bytes) ngroups--;
    const int nga = (nb + MOE_GB - 1) / MOE_GB;
    if (REG) ngroups = nga;  // every window of the registered copy is whole (zero past the row)
    const int rl = w * 32 + li;
    issue(0, I0{}, ngroups > 0);
    auto group = [&](int g, auto stage) {
        constexpr int other = 1 - decltype(stage)::value;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (g + 1 < nga) issue(g + 1, std::integral_constant<int, other>{}, g + 1 < ngroups);
        if (g < ngroups) {
            const uint32_t *wl = W_(stage)[rl];
            // GGUF windows: 17-byte blocks from byte 0 (the whole window in
            // registers); registered windows: qs of block kb at 16kb, the e
            // bytes at 64 (aligned reads, no byte shifts)
            uint32_t W[REG ? 1 : 4 * MOE_WIN];
            if constexpr (REG) {
                W[0] = wl[16];
            } else {
#pragma unroll
                for (int i = 0; i < MOE_WIN; i++) {
                    const uint4 t = reinterpret_cast<const uint4 *>(wl)[i];
                    W[4 * i] = t.x; W[4 * i + 1] = t.y; W[4 * i + 2] = t.z; W[4 * i + 3] = t.w;
                }
            }
            auto e_of = [&](int kb) {
                if constexpr (REG) return (W[0] >> (8 * kb)) & 0xffu;
                else return (W[(17 * kb) >> 2] >> (8 * ((17 * kb) & 3))) & 0xffu;
            };
            auto q_of = [&](int kb, uint32_t (&q)[4]) {
                if constexpr (REG) {
                    const uint4 t = reinterpret_cast<const uint4 *>(wl)[kb];
                    q[0] = t.x; q[1] = t.y; q[2] = t.z; q[3] = t.w;
                } else {
                    const int o = 17 * kb + 1, d = o >> 2, sh = o & 3;
#pragma unroll
                    for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(W[d + i + 1], W[d + i], sh);
                }
            };
            const int nbl = nb - MOE_GB * g;  // blocks of this group inside the row
            bool ok = !SUBSUMS;
#pragma unroll
            for (int kb = 0; kb < MOE_GB; kb++) ok = ok && (kb >= nbl || in_range(e_of(kb)));
            if (__ballot(!ok) == 0) {
#pragma unroll
                for (int kb = 0; kb < MOE_GB; kb++) {
                    if (kb >= nbl) break;
                    uint32_t q[4];
                    q_of(kb, q);
#pragma unroll
                    for (int mt = 0; mt < NMT; mt++)
                        if (mt == 0 || np > 32 * mt)
                            fold_fast(mfma(q, (int)e_of(kb), stage, kb, mt), D_(stage)[kb][mt * 32 + li], mt);
                }
            } else {
                for (int kb = 0; kb < MOE_GB && kb < nbl; kb++) {
                    uint32_t q[4];
                    q_of(kb, q);
#pragma unroll
                    for (int mt = 0; mt < NMT; mt++)
                        if (mt == 0 || np > 32 * mt)
                            fold_exact(mfma(q, s127, stage, kb, mt), D_(stage)[kb][mt * 32 + li], e_of(kb),
                                       MOE_GB * g + kb, mt);
                }
            }
        } else {
            for (int kb = 0; kb < MOE_GB && MOE_GB * g + kb < nb; kb++) {  // tail blocks: global loads, exact fold
                const int b = MOE_GB * g + kb;
                const uint8_t *wb = as + (int64_t)e * as_nb2 + (int64_t)min(row0 + li, rows - 1) * as_nb1 +
                                    (int64_t)b * MXFP4_BYTES;
                const uint32_t q[4] = {ld4(wb + 1), ld4(wb + 5), ld4(wb + 9), ld4(wb + 13)};
#pragma unroll
                for (int mt = 0; mt < NMT; mt++)
                    if (mt == 0 || np > 32 * mt)
                        fold_exact(mfma(q, s127, stage, kb, mt), D_(stage)[kb][mt * 32 + li], wb[0], b, mt);
            }
        }
    };
    for (int g = 0; g < nga; g++) {
        if (g & 1) group(g, I1{});
        else group(g, I0{});
    }
#pragma unroll
    for (int mt = 0; mt < NMT; mt++) {
        if (mt * 32 + li >= np) continue;
        const int p = pairs[mt * 32 + li];
        const int t = p / n_ids, s = p - t * n_ids;
        float *o = dst + (int64_t)t * dst_nb2 + (int64_t)s * dst_nb1;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = row0 + crowm(v, lane);
            if (r < rows) o[r] = acc[mt][v];
        }
    }
}
// wrep: the registered copy of the experts (ghip_mxfp4_repack; the _reg
// kernels) or unused; ngp its groups per row.  Four workgroups per CU (38 KB
// of LDS each) need at most 128 VGPRs: 4 wavefronts per SIMD measured 184 us
// against 226 us at 2 (config 4 gate_up, registered).
#define MOE_FP4_KERNEL(name, NMT, REPACK, SUB, REG)                                                           \
    extern "C" __global__ void __launch_bounds__(256)                                                         \
        __attribute__((amdgpu_waves_per_eu(NMT == 1 && !SUB ? 4 : 1)))                                        \
        name(MOE_ARGS, const uint8_t *__restrict__ wrep, int ngp, int order) {                                \
        moe_fp4_impl<NMT, REPACK, SUB, REG>(MOE_PASS_FP4);                                                    \
    }
#define MOE_PASS_FP4                                                                                          \
    as, as_nb1, as_nb2, (const uint8_t *)actf, actd, ne11, route, n_pairs, n_ids, dst, dst_nb1, dst_nb2, rows, nb, \
        sub, wrep, ngp, order
MOE_FP4_KERNEL(ghip_moe_fp4, 1, true, false, false)
MOE_FP4_KERNEL(ghip_moe_fp4_plain, 1, false, false, false)
MOE_FP4_KERNEL(ghip_moe_fp4_sub, 1, true, true, false)
MOE_FP4_KERNEL(ghip_moe_fp4_plain_sub, 1, false, true, false)
MOE_FP4_KERNEL(ghip_moe_fp4_t64, 2, true, false, false)
MOE_FP4_KERNEL(ghip_moe_fp4_t64_plain, 2, false, false, false)
MOE_FP4_KERNEL(ghip_moe_fp4_reg, 1, true, false, true)
MOE_FP4_KERNEL(ghip_moe_fp4_plain_reg, 1, false, false, true)
MOE_FP4_KERNEL(ghip_moe_fp4_sub_reg, 1, true, true, true)
MOE_FP4_KERNEL(ghip_moe_fp4_plain_sub_reg, 1, false, true, true)
MOE_FP4_KERNEL(ghip_moe_fp4_t64_reg, 2, true, false, true)
MOE_FP4_KERNEL(ghip_moe_fp4_t64_plain_reg, 2, false, false, true)



// The registered layout of MXFP4 experts for moe_fp4_impl: per (expert, block
// of 128 rows, group of MOE_GB blocks) the 128 rows' windows, 80 bytes each --
// the qs of block kb at 16kb, the four e bytes at 64, zero past the row and
// in the padding -- one contiguous run in the order the kernel stages them in
// LDS.  One thread per 16-byte chunk.
extern "C" __global__ void __launch_bounds__(256)
ghip_mxfp4_repack(const uint8_t *__restrict__ W, int64_t nb1, int64_t nb2, int rows, int nb, int n_as, int nrb,
                  int ngp, uint8_t *__restrict__ out) {
    constexpr int CH = MOE_TR * MOE_WIN;  // chunks per (expert, row block, group)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)n_as * nrb * ngp * CH) return;
    const int c = (int)(i % CH);
    const int64_t rest = i / CH;
    const int g = (int)(rest % ngp);
    const int64_t erb = rest / ngp;
    const int rb = (int)(erb % nrb), e = (int)(erb / nrb);
    const int r = c / MOE_WIN, c16 = c - r * MOE_WIN;
    const int row = rb * MOE_TR + r;
    const int row_bytes = nb * MXFP4_BYTES;
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    if (row < rows) {
        const uint8_t *src = W + (int64_t)e * nb2 + (int64_t)row * nb1;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            int pos = -1;  // byte of the row for byte k of this chunk
            if (c16 < MOE_GB) pos = MXFP4_BYTES * (MOE_GB * g + c16) + 1 + k;        // qs of block c16
            else if (c16 == MOE_GB && k < MOE_GB) pos = MXFP4_BYTES * (MOE_GB * g + k);  // e of block k
            if (pos >= 0 && pos < row_bytes) v[k >> 2] |= (uint32_t)src[pos] << (8 * (k & 3));
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------- K-quant experts
// MUL_MAT_ID with Q4_K, Q5_K or Q6_K experts (forward_mul_mat_id,
// compute.rs:1917-2202): the activation rows quantized once to Q8_K
// (quantize_row_q8_K, the reference's wdata pass), the pairs routed by
// ghip_moe_route, then per (tile, 16 expert rows) one workgroup of four
// wavefronts, 4 rows each held in registers, walking the tile's pairs.  Per
// (pair, row) the value is the decode GEMV's: the integer sums of
// vec_dot_q4_K_q8_K / vec_dot_q5_K_q8_K / vec_dot_q6_K_q8_K per super-block
// (vec_dot.rs:928-1040) and the same fp32 scaling, summed over the
// wavefront.  A wavefront covers 16 super-blocks per pass (4 lanes each);
// wider rows take several passes, their partials added in the lanes first.
constexpr int MMID_RB = 4;  // rows per wavefront

// Lane i's quarter of super-block b: its integer sums (the caller adds the
// four quarters exactly before any rounding) and the block's scales.
template <int TYPE>  // 12 Q4_K, 13 Q5_K, 14 Q6_K
DEV void kq_lane_dot(const uint8_t *__restrict__ wrow, const uint8_t *__restrict__ arow, int b, int i, bool valid,
                     int32_t *sub_ia, int32_t *sub_im, float *d8o, float *dwo, float *dmo) {
    if (!valid) return;
    const uint8_t *ab = arow + (int64_t)b * Q8K_BYTES;
    const float d8 = __uint_as_float(ld4(ab));
    *d8o = d8;
    if constexpr (TYPE == 14) {
        // lane i: half j = i / 2, 16-element column hh = i % 2 of each quarter q
        const int j = i >> 1, hh = i & 1;
        const uint8_t *blk = wrow + (int64_t)b * Q6K_BYTES;
        const uint4 l0 = ld16(blk + 64 * j + 16 * hh), l1 = ld16(blk + 64 * j + 16 * hh + 32);
        const uint4 qh = ld16(blk + 128 + 32 * j + 16 * hh);
        const uint2 scv = ld8(blk + 192 + 8 * j);
        const float dw = h2f(ld2(blk + 208));
        const uint32_t la[4] = {l0.x, l0.y, l0.z, l0.w}, lb[4] = {l1.x, l1.y, l1.z, l1.w};
        const uint32_t hv[4] = {qh.x, qh.y, qh.z, qh.w};
        int is = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 y = ld16(ab + 4 + 128 * j + 16 * hh + 32 * q);
            const uint32_t yv[4] = {y.x, y.y, y.z, y.w};
            int dq = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t src = (q & 1) ? lb[k] : la[k];
                const uint32_t nib = (q & 2) ? ((src >> 4) & 0x0f0f0f0f) : (src & 0x0f0f0f0f);
                dq = dot4(nib | (((hv[k] >> (2 * q)) & 0x03030303) << 4), yv[k], dq);
            }
            const int bs32 = 32 * (int)(int16_t)ld2(ab + 260 + 2 * (8 * j + hh + 2 * q));
            const uint32_t sw = q < 2 ? scv.x : scv.y;
            const int sc = (int)(int8_t)(sw >> (8 * hh + 16 * (q & 1)));
            is += sc * (dq - bs32);
        }
        *sub_ia = is;
        *dwo = dw;
    } else {
        constexpr bool Q5 = TYPE == 13;
        constexpr int BB = Q5 ? 176 : Q4K_BYTES;
        const uint8_t *blk = wrow + (int64_t)b * BB;
        const uint4 hd = ld16(blk);
        const uint4 x0 = ld16(blk + (Q5 ? 48 : 16) + 32 * i), x1 = ld16(blk + (Q5 ? 64 : 32) + 32 * i);
        const float dw = h2f(hd.x), dmin = h2f(hd.x >> 16);
        int sc0, sc1, m0, m1;
        k4_scales(hd.y, hd.z, hd.w, scale_sel(i), sc0, sc1, m0, m1);
        const uint32_t qv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            lo[k] = qv[k] & 0x0f0f0f0f;
            hi[k] = (qv[k] >> 4) & 0x0f0f0f0f;
        }
        if constexpr (Q5) {
            const uint4 g0 = ld16(blk + 16), g1 = ld16(blk + 32);
            const uint32_t hv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t q2 = hv[k] >> (2 * i);
                lo[k] |= (q2 & 0x01010101u) << 4;
                hi[k] |= (q2 << 3) & 0x10101010u;
            }
        }
        const uint4 a0 = ld16(ab + 4 + 64 * i), a1 = ld16(ab + 20 + 64 * i);
        const uint4 a2 = ld16(ab + 36 + 64 * i), a3 = ld16(ab + 52 + 64 * i);
        const uint32_t al[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const uint32_t ah[8] = {a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
        int dl = 0, dh = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dl = dot4(lo[k], al[k], dl);
            dh = dot4(hi[k], ah[k], dh);
        }
        const uint2 bsv = ld8(ab + 260 + 8 * i);  // bsum16 of 16-groups 4i .. 4i+3
        const int bs0 = (int)(int16_t)(bsv.x & 0xffff) + (int)(int16_t)(bsv.x >> 16);
        const int bs1 = (int)(int16_t)(bsv.y & 0xffff) + (int)(int16_t)(bsv.y >> 16);
        const int ia = __mul24(sc0, dl) + __mul24(sc1, dh);
        const int im = __mul24(m0, bs0) + __mul24(m1, bs1);
        *sub_ia = ia;
        *sub_im = im;
        *dwo = dw;
        *dmo = dmin;
    }
}

// grid: (tiles, ceil(rows / 16)); route as written by ghip_moe_route
template <int TYPE, bool SUBSUMS>
__device__ __forceinline__ void mmid_kq_impl(const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2,
                                             const uint8_t *__restrict__ act, int64_t act_rb, int ne11,
                                             const int32_t *__restrict__ route, int n_pairs, int n_ids,
                                             float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows,
                                             int nb, int32_t *__restrict__ sub) {
    const int tile = blockIdx.x;
    if (tile >= route[0]) return;
    const int32_t *tl = route + 2 + n_pairs + 3 * tile;
    const int e = tl[0], first = tl[1], count = tl[2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = (int)blockIdx.y * 16 + wave * MMID_RB;
    const int i = lane & 3;
    const uint8_t *ebase = as + (int64_t)e * as_nb2;
    for (int pi = 0; pi < count; pi++) {
        const int p = route[2 + first + pi];
        const int t = p / n_ids, s = p - t * n_ids;
        const uint8_t *arow = act + ((int64_t)t * ne11 + s % ne11) * act_rb;
        float part[MMID_RB];
#pragma unroll
        for (int rr = 0; rr < MMID_RB; rr++) part[rr] = 0.0f;
        for (int c = 0; c < nb; c += 16) {
            const int b = c + (lane >> 2);
            const bool valid = b < nb;
#pragma unroll
            for (int rr = 0; rr < MMID_RB; rr++) {
                const int r = min(r0 + rr, rows - 1);
                int32_t ia = 0, im = 0;
                float d8 = 0.0f, dw = 0.0f, dm = 0.0f;
                kq_lane_dot<TYPE>(ebase + (int64_t)r * as_nb1, arow, b, i, valid, &ia, &im, &d8, &dw, &dm);
                // whole super-block sums (exact), then the block scale
                // d = d8 * dw applied once per super-block (vec_dot.rs:881-909,
                // vec_dot.rs:998-1028)
                const int iab = quad_sum_dpp(ia), imb = TYPE == 14 ? 0 : quad_sum_dpp(im);
                if (i == 0)
                    part[rr] += TYPE == 14 ? (d8 * dw) * (float)iab
                                           : fmaf(d8 * dw, (float)iab, (-d8 * dm) * (float)imb);
                if (SUBSUMS) {
                    if (i == 0 && valid && r0 + rr < rows) {
                        int32_t *sp = sub + ((int64_t)p * rows + r0 + rr) * nb * (TYPE == 14 ? 1 : 2);
                        if (TYPE == 14) sp[b] = iab;
                        else {
                            sp[2 * b] = iab;
                            sp[2 * b + 1] = imb;
                        }
                    }
                }
            }
        }
        float *o = dst + (int64_t)t * dst_nb2 + (int64_t)s * dst_nb1;
#pragma unroll
        for (int rr = 0; rr < MMID_RB; rr++) {
            const float tot = wave_sum_dpp(part[rr]);
            if (lane == 0 && r0 + rr < rows) o[r0 + rr] = tot;
        }
    }
}
#define MMID_KQ(TN, TYPE)                                                                                           \
    extern "C" __global__ void __launch_bounds__(256)                                                               \
        ghip_mmid_##TN(const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2,                             \
                       const uint8_t *__restrict__ act, int64_t act_rb, int ne11, const int32_t *__restrict__ route, \
                       int n_pairs, int n_ids, float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2, int rows,  \
                       int nb, int32_t *__restrict__ sub) {                                                          \
        mmid_kq_impl<TYPE, false>(as, as_nb1, as_nb2, act, act_rb, ne11, route, n_pairs, n_ids, dst, dst_nb1,      \
                                  dst_nb2, rows, nb, sub);                                                          \
    }                                                                                                               \
    extern "C" __global__ void __launch_bounds__(256)                                                               \
        ghip_mmid_##TN##_sub(const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2,                        \
                             const uint8_t *__restrict__ act, int64_t act_rb, int ne11,                             \
                             const int32_t *__restrict__ route, int n_pairs, int n_ids, float *__restrict__ dst,    \
                             int64_t dst_nb1, int64_t dst_nb2, int rows, int nb, int32_t *__restrict__ sub) {       \
        mmid_kq_impl<TYPE, true>(as, as_nb1, as_nb2, act, act_rb, ne11, route, n_pairs, n_ids, dst, dst_nb1,       \
                                 dst_nb2, rows, nb, sub);                                                           \
    }
MMID_KQ(q4_K, 12)
MMID_KQ(q5_K, 13)
MMID_KQ(q6_K, 14)
