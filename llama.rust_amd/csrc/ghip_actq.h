// ghip_actq.h -- activation images of the whole-row decode kernels: the
// activation rows quantized to Q8_K (or copied, when src1 is already Q8_K)
// once per workgroup into LDS.  Shared by ghip_gemv.hip and ghip_skinny.hip.
//
// LDS image: codes [NC][K] int8 | d [NC][nb] f32 | 16-element sums
// [NC][nb][16] int32.
#pragma once
#include <type_traits>
#include "ghip_common.h"

// Quantization of the activation rows into the LDS image, bit-identical to
// ghip_quantize_q8_K: 16 lanes per super-block ("task" = one lane's 16
// consecutive elements); the signed max-abs is reduced over the 16 lanes with
// the first occurrence winning ties; rows c < n_mat take the
// quantize_mat_q8_K_4x8 values.  Tasks run in rounds of blockDim lanes; every
// lane of the workgroup takes part in every round (the shuffles need them).
struct XTask {
    float v[16];
};

DEV XTask quant_q8K_load(const float *__restrict__ x, int64_t x_stride, int ncols, int nb, int total, int task) {
    XTask t;
    const int l = task & 15, blk = task >> 4;
    const int c = blk / nb, b = blk - c * nb;
    if (task < total && c < ncols) {
        __builtin_memcpy(t.v, x + (int64_t)c * x_stride + (int64_t)b * QK_K + 16 * l, 64);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) t.v[i] = 0.0f;
    }
    return t;
}

// cstride / bstride: the image's per-token strides of codes (bytes) and
// 16-element sums (ints); -1: nb * 256 and nb * 16 (packed)
DEV void quant_q8K_store(const XTask &t, int nb, int n_mat, int total, int task, int8_t *codes, float *dq, int *bsum,
                         int cstride = -1, int bstride = -1) {
    const float *v = t.v;
    const bool live = task < total;
    const int l = task & 15, blk = task >> 4;
    const int c = live ? blk / nb : 0, b = live ? blk - c * nb : 0;
    float bax = 0.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float a = fabsf(v[i]);
        if (a > bax) { bax = a; bval = v[i]; bidx = 16 * l + i; }
    }
    // all-reduce over the task's 16 lanes (one DPP row; every caller runs
    // whole wavefronts with task % 16 == lane % 16): partners by quad xor 1,
    // quad xor 2, half-row mirror (i <-> 7 - i) and row mirror (i <-> 15 - i),
    // each pairing two disjoint groups that already agree, so every lane ends
    // with the largest |v|, ties to the lowest index
    auto step = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const float oax = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bax), C, 0xF, 0xF, false));
        const float oval = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bval), C, 0xF, 0xF, false));
        const int oidx = __builtin_amdgcn_update_dpp(0, bidx, C, 0xF, 0xF, false);
        if (oax > bax || (oax == bax && oidx < bidx)) { bax = oax; bval = oval; bidx = oidx; }
    };
    step(std::integral_constant<int, 0xB1>{});
    step(std::integral_constant<int, 0x4E>{});
    step(std::integral_constant<int, 0x141>{});
    step(std::integral_constant<int, 0x140>{});
    int q[16];
    float d;
    if (bax == 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = 0;
        d = 0.0f;
    } else if (c >= n_mat) {
        const float iscale = __fdiv_rn(-127.0f, bval);
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = min(127, (int)rintf(__fmul_rn(iscale, v[i])));
        d = __fdiv_rn(1.0f, iscale);
    } else {
        const float iscale = __fdiv_rn(127.0f, bax);
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = (int)fminf(fmaxf(rintf(__fmul_rn(iscale, v[i])), -128.0f), 127.0f);
        d = __fdiv_rn(1.0f, iscale);
    }
    uint32_t pk[4];
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        pk[k] = (uint32_t)(q[4 * k] & 0xff) | ((uint32_t)(q[4 * k + 1] & 0xff) << 8) |
                ((uint32_t)(q[4 * k + 2] & 0xff) << 16) | ((uint32_t)(q[4 * k + 3] & 0xff) << 24);
        sum += q[4 * k] + q[4 * k + 1] + q[4 * k + 2] + q[4 * k + 3];
    }
    if (live) {
        const int cs = cstride < 0 ? nb * QK_K : cstride, bst = bstride < 0 ? nb * 16 : bstride;
        *reinterpret_cast<uint4 *>(codes + (int64_t)c * cs + b * QK_K + 16 * l) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        bsum[c * bst + b * 16 + l] = sum;  // bsums[l] of block_q8_K
        if (l == 0) dq[c * nb + b] = d;
    }
}

// Ready Q8_K rows (pre-quantized src1) copied into the same LDS image, in
// the same task shape (16 codes per lane).
struct Q8KTask {
    uint4 v;
    int sum;
    float d;
};

DEV Q8KTask q8K_load(const uint8_t *__restrict__ act, int64_t act_row_bytes, int ncols, int nb, int total, int task) {
    Q8KTask t{make_uint4(0, 0, 0, 0), 0, 0.0f};
    const int l = task & 15, blk = task >> 4;
    const int c = blk / nb, b = blk - c * nb;
    if (task < total && c < ncols) {
        const uint8_t *A = act + (int64_t)c * act_row_bytes + (int64_t)b * Q8K_BYTES;
        t.v = ld16(A + 4 + 16 * l);
        t.sum = (int)(int16_t)ld2(A + 260 + 2 * l);
        t.d = __uint_as_float(ld4(A));
    }
    return t;
}

DEV void q8K_store(const Q8KTask &t, int nb, int total, int task, int8_t *codes, float *dq, int *bsum) {
    if (task >= total) return;
    const int l = task & 15, blk = task >> 4;
    const int c = blk / nb, b = blk - c * nb;
    *reinterpret_cast<uint4 *>(codes + (int64_t)c * nb * QK_K + b * QK_K + 16 * l) = t.v;
    bsum[(c * nb + b) * 16 + l] = t.sum;
    if (l == 0) dq[c * nb + b] = t.d;
}

