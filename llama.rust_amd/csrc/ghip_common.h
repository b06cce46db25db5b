// ghip_common.h -- device-side helpers shared by the gfx950 kernels.
//
// Block layouts are the GGUF ones, unchanged (crates/ggml/src/blocks.rs:33-168):
//   block_q4_0  18 B  {f16 d; u8 qs[16]}
//   block_q8_0  34 B  {f16 d; i8 qs[32]}
//   block_q4_K 144 B  {f16 d, dmin; u8 scales[12]; u8 qs[128]}
//   block_q6_K 210 B  {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}
//   block_q8_K 292 B  {f32 d; i8 qs[256]; i16 bsums[16]}
//   block_mxfp4 17 B  {u8 e; u8 qs[16]}
// Rows of these blocks are only 2-byte aligned in general; gfx950 runs in
// unaligned-access mode, so a byte-pointer memcpy into a uint4 compiles to one
// global_load_dwordx4.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define DEV static __device__ __forceinline__

constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8K_BYTES = 292;
constexpr int Q4_0_BYTES = 18;
constexpr int Q8_0_BYTES = 34;
constexpr int MXFP4_BYTES = 17;

// Int8 weight codes of the Q8-family prefill GEMM: 32-row tiles, and in a
// tile one 1 KB piece per 32-block in which lane 32h + r of a wavefront finds
// row r's bytes 16h .. 16h+15 at lane * 16 (one coalesced 16-byte load per
// lane gives the MFMA's B operand).  Byte offset of row's block b, half 0;
// half 1 follows at +512.
DEV int64_t q8w_piece(int row, int b, int Kpad) {
    return ((int64_t)(row >> 5) * (Kpad >> 5) + b) * 1024 + (row & 31) * 16;
}

DEV uint4 ld16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
DEV uint2 ld8(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
DEV uint32_t ld4(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
DEV uint16_t ld2(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
// non-temporal streaming load for weights that are read exactly once
DEV uint4 ld16_stream(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// Value barrier: keeps the compiler from folding the producing multiply into a
// later conversion (e.g. v_fma_mix with a +0 addend, which turns -0 into +0).
DEV float opaque(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// fp32 -> fp16 bits, round to nearest even, of exactly this fp32 value
DEV uint16_t f2h_rn(float f) { return __half_as_ushort(__float2half_rn(opaque(f))); }

DEV float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (global_load_lds_dwordx4; lds is wave-uniform). The data is in LDS once the
// issuing wavefront's vmcnt reaches zero.
typedef __attribute__((address_space(3))) void lds_void;
DEV void g2lds(const void *gptr, void *lds) {
    __builtin_amdgcn_global_load_lds(gptr, (lds_void *)lds, 16, 0, 0);
}

DEV int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// Transposed reduction of 8 per-row partials over a wavefront: on return every
// lane of the 8-lane group g = lane>>3 holds the wavefront total of row g.
// 10 cross-lane exchanges instead of 8 x 6.
DEV float reduce8_rows(float v[8], int lane) {
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
    float u[4], w[2], x;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float send = b5 ? v[i] : v[i + 4];
        const float keep = b5 ? v[i + 4] : v[i];
        u[i] = keep + __shfl_xor(send, 32, 64);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float send = b4 ? u[i] : u[i + 2];
        const float keep = b4 ? u[i + 2] : u[i];
        w[i] = keep + __shfl_xor(send, 16, 64);
    }
    {
        const float send = b3 ? w[0] : w[1];
        const float keep = b3 ? w[1] : w[0];
        x = keep + __shfl_xor(send, 8, 64);
    }
    x += __shfl_xor(x, 4, 64);
    x += __shfl_xor(x, 2, 64);
    x += __shfl_xor(x, 1, 64);
    return x;
}
// Transposed reduction of R per-row partials across the wavefront: the rows
// are halved with each of the first log2(R) exchanges (lane bit 5 first), the
// rest of the lanes then sum normally.  Row r's total ends in the lanes whose
// top log2(R) bits equal r (lane / (64 / R) == r).
template <int R>
DEV float reduce_rows(float v[R], int lane) {
    if constexpr (R == 8) {
        return reduce8_rows(v, lane);
    } else if constexpr (R == 4) {
        const bool b5 = lane & 32, b4 = lane & 16;
        float u[2], x;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float send = b5 ? v[i] : v[i + 2];
            const float keep = b5 ? v[i + 2] : v[i];
            u[i] = keep + __shfl_xor(send, 32, 64);
        }
        {
            const float send = b4 ? u[0] : u[1];
            const float keep = b4 ? u[1] : u[0];
            x = keep + __shfl_xor(send, 16, 64);
        }
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
        return x;
    } else if constexpr (R == 2) {
        const bool b5 = lane & 32;
        const float send = b5 ? v[0] : v[1];
        float x = (b5 ? v[1] : v[0]) + __shfl_xor(send, 32, 64);
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
        return x;
    } else {
        float x = v[0];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
        return x;
    }
}

// Wave-wide float sum with DPP row operations (no LDS): quad xor 1 and 2,
// half-row and row mirrors leave every lane of a 16-lane row holding the
// row's sum; the four row sums are read as scalars.  The result is uniform.
#define GHIP_DPP_ADD(v, ctrl) \
    ((v) + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), 0xF, 0xF, false)))
DEV float wave_sum_dpp(float v) {
    v = GHIP_DPP_ADD(v, 0xB1);   // quad_perm [1,0,3,2]
    v = GHIP_DPP_ADD(v, 0x4E);   // quad_perm [2,3,0,1]
    v = GHIP_DPP_ADD(v, 0x141);  // row_half_mirror
    v = GHIP_DPP_ADD(v, 0x140);  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}
// sum over the 4 lanes of each quad (every lane of the quad gets it)
DEV int quad_sum_dpp(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    return v;
}

DEV int group8_sum(int v) {
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    return v;
}

// byte i (0..11) of three little-endian dwords
DEV uint32_t byte_of3(uint32_t a, uint32_t b, uint32_t c, int i) {
    const uint32_t w = i < 4 ? a : (i < 8 ? b : c);
    return (w >> (8 * (i & 3))) & 0xffu;
}

// get_scale_min_k4 (quants_k.rs:1672) on the 12 scale bytes held in s0..s2
DEV void scale_min_k4(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &m) {
    if (j < 4) {
        sc = (int)(byte_of3(s0, s1, s2, j) & 63);
        m = (int)(byte_of3(s0, s1, s2, j + 4) & 63);
    } else {
        sc = (int)((byte_of3(s0, s1, s2, j + 4) & 0xF) | ((byte_of3(s0, s1, s2, j - 4) >> 6) << 4));
        m = (int)((byte_of3(s0, s1, s2, j + 4) >> 4) | ((byte_of3(s0, s1, s2, j) >> 6) << 4));
    }
}

// Scales and mins of sub-blocks 2i and 2i+1 (get_scale_min_k4,
// quants_k.rs:1672) for this lane's fixed i, without lane-divergent branches:
// for sub-block t < 4 the scale is bits 0-5 of byte t and the min bits 0-5
// of byte t+4; for t >= 4 the scale is the low nibble of byte t+4 with the
// top two bits of byte t-4 above it, the min the high nibble of byte t+4 with
// the top two bits of byte t.  The lane's selectors come from ScaleSel.
struct ScaleSel {
    bool hi;     // i >= 2: sub-blocks 4..7
    int o0, o1;  // bit offsets of the two sub-blocks' bytes (8 * (t & 3))
};
DEV ScaleSel scale_sel(int i) { return ScaleSel{i >= 2, 8 * ((2 * i) & 3), 8 * ((2 * i + 1) & 3)}; }
DEV void k4_scales(uint32_t s0, uint32_t s1, uint32_t s2, const ScaleSel &q, int &sc0, int &sc1, int &m0, int &m1) {
    const uint32_t a = q.hi ? s2 : s0;  // scale low bits
    const uint32_t bm = q.hi ? s2 : s1; // min low bits
    const uint32_t ts = q.hi ? s0 : 0u; // scale top bits
    const uint32_t tm = q.hi ? s1 : 0u; // min top bits
    const int ws = q.hi ? 4 : 6, om = q.hi ? 4 : 0;
    sc0 = (int)(__builtin_amdgcn_ubfe(a, q.o0, ws) | (__builtin_amdgcn_ubfe(ts, q.o0 + 6, 2) << 4));
    sc1 = (int)(__builtin_amdgcn_ubfe(a, q.o1, ws) | (__builtin_amdgcn_ubfe(ts, q.o1 + 6, 2) << 4));
    m0 = (int)(__builtin_amdgcn_ubfe(bm, q.o0 + om, ws) | (__builtin_amdgcn_ubfe(tm, q.o0 + 6, 2) << 4));
    m1 = (int)(__builtin_amdgcn_ubfe(bm, q.o1 + om, ws) | (__builtin_amdgcn_ubfe(tm, q.o1 + 6, 2) << 4));
}

// KVALUES_MXFP4 (quants.rs:660)
__device__ static const int8_t kvalues_mxfp4_dev[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

// e8m0_to_fp32_half (quants.rs:682): 2^(x-128) from bits
DEV float e8m0_half(uint32_t x) {
    const uint32_t bits = x < 2 ? (0x00200000u << x) : ((x - 1) << 23);
    return __uint_as_float(bits);
}

// MUL_MAT_ID through a decode kernel: blockIdx.y is the (token, slot) pair
// p = t * n_ids + s (dst row [t][s], compute.rs:1917-2202): its expert's
// weights, its activation row t * ne11 + s % ne11 and its sub-sums.  A pair
// whose expert id is out of range gets NaN rows (the reference asserts on it);
// the workgroup then returns false after writing them.
#define MMID_ARGS                                                                                                   \
    const uint8_t *__restrict__ as, int64_t as_nb1, int64_t as_nb2, int rows, int nb,                               \
        const uint8_t *__restrict__ act, int64_t act_rb, int ne11, const int32_t *__restrict__ ids,                 \
        int64_t ids_nb1, int n_ids, int n_as, float *__restrict__ dst, int64_t dst_nb1, int64_t dst_nb2,            \
        int32_t *__restrict__ sub, int64_t sub_pair, int rpw
struct MmidPair {
    const uint8_t *W, *act;
    float *dst;
    int32_t *sub;
};
DEV bool mmid_pair(const uint8_t *as, int64_t as_nb2, const uint8_t *act, int64_t act_rb, int ne11,
                   const int32_t *ids, int64_t ids_nb1, int n_ids, int n_as, float *dst, int64_t dst_nb1,
                   int64_t dst_nb2, int32_t *sub, int64_t sub_pair, int rows, int rpw, MmidPair &q) {
    const int p = (int)blockIdx.y, t = p / n_ids, s = p - t * n_ids;
    const int e = ids[(int64_t)t * ids_nb1 + s];
    q.dst = dst + (int64_t)t * dst_nb2 + (int64_t)s * dst_nb1;
    if (e < 0 || e >= n_as) {
        const int r = (int)blockIdx.x * rpw + (int)threadIdx.x;
        if ((int)threadIdx.x < rpw && r < rows) q.dst[r] = __builtin_nanf("");
        return false;
    }
    q.W = as + (int64_t)e * as_nb2;
    q.act = act + ((int64_t)t * ne11 + s % ne11) * act_rb;
    q.sub = sub ? sub + (int64_t)p * sub_pair : nullptr;
    return true;
}
#define MMID_PAIR(q)                                                                                                \
    MmidPair q;                                                                                                     \
    if (!mmid_pair(as, as_nb2, act, act_rb, ne11, ids, ids_nb1, n_ids, n_as, dst, dst_nb1, dst_nb2, sub, sub_pair,  \
                   rows, rpw, q))                                                                                   \
        return;
