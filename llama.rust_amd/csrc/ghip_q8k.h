// ghip_q8k.h -- Q8_K activation quantization of one 256-element block by one
// wavefront (lane l owns elements 4l .. 4l+3), shared by the standalone
// quantizer (ghip_quant.hip) and the GEMM's fused quantize-and-layout kernel
// (ghip_gemm.hip), so both produce the same bytes:
//   quantize_row_q8_K_ref   quants.rs:615-650   iscale = -127/max (signed max-abs),
//                                               q = min(127, rne(iscale*x)), d = 1/iscale
//   quantize_mat_q8_K_4x8   repack.rs:1561-1620 iscale = 127/amax, q = clamp(rne(iscale*x)),
//                                               d = 1/iscale
// Compiled with -ffp-contract=off: every product is rounded before rne().
#pragma once
#include <type_traits>
#include "ghip_common.h"

// codes q[0..3] of this lane's elements and the block scale d (uniform);
// mat selects the quantize_mat_q8_K_4x8 values
DEV void q8K_block(const float xs[4], int lane, bool mat, int q[4], float &d) {
    // signed max-abs, first occurrence wins (strict '>' scan in element order)
    float bax = 0.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(xs[i]);
        if (a > bax) { bax = a; bval = xs[i]; bidx = lane * 4 + i; }
    }
    // all-reduce within each 16-lane row by DPP: partners by quad xor 1, quad
    // xor 2, half-row mirror (i <-> 7 - i) and row mirror (i <-> 15 - i), each
    // pairing two disjoint groups that already agree (ties: lower index)
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
    // the four rows hold ascending element ranges: combine them in order from
    // their first lanes, a later row winning only with a strictly larger |x|
    {
        float ax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bax), 0));
        float val = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bval), 0));
#pragma unroll
        for (int r = 1; r < 4; r++) {
            const float oax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bax), 16 * r));
            const float oval = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bval), 16 * r));
            if (oax > ax) { ax = oax; val = oval; }
        }
        bax = ax;
        bval = val;
    }
    if (bax == 0.0f) {
        q[0] = q[1] = q[2] = q[3] = 0;
        d = 0.0f;
    } else if (!mat) {
        const float iscale = __fdiv_rn(-127.0f, bval);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int v = (int)rintf(__fmul_rn(iscale, xs[i]));
            q[i] = v < 127 ? v : 127;
        }
        d = __fdiv_rn(1.0f, iscale);
    } else {
        const float iscale = __fdiv_rn(127.0f, bax);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float r = rintf(__fmul_rn(iscale, xs[i]));
            r = fminf(fmaxf(r, -128.0f), 127.0f);
            q[i] = (int)r;
        }
        d = __fdiv_rn(1.0f, iscale);
    }
}
// sum of the 16 codes of this lane's quad (the block_q8_K bsums entry lane/4),
// valid in every lane of the quad
DEV int q8K_bsum16(const int q[4], int lane) {
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    (void)lane;
    return s;
}
