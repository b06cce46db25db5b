// ghip_quant.hip -- activation quantizers for the MUL_MAT path, on the GPU.
//
// Bit-exact with the reference's CPU quantizers (the integer codes, bsums and
// scales are what the dot kernels consume, so they must be identical):
//   quantize_row_q8_K_ref   quants.rs:615-650   iscale = -127/max (signed max-abs),
//                                               q = min(127, rne(iscale*x)), d = 1/iscale
//   quantize_mat_q8_K_4x8   repack.rs:1561-1620 iscale = 127/amax, q = clamp(rne(iscale*x)),
//                                               d = 1/iscale (values; plain block_q8_K layout)
//   quantize_row_q8_0       quants.rs:331-362   d = f16(amax/127), q = rne(x*127/amax)
// Compiled with -ffp-contract=off: every product is rounded before rne().
#include "ghip_common.h"
#include "ghip_q8k.h"

// One wavefront per 256-element super-block; each lane owns 4 consecutive
// elements.  Rows r < n_mat use the quantize_mat_q8_K_4x8 values, the others
// quantize_row_q8_K_ref (the reference's repack route quantizes the leading
// ne11 - ne11 % 4 activation rows with the former, compute.rs:5350-5398).
// wavefront wid of a matrix of nb super-blocks per row
DEV void quantize_q8K_wave(const float *__restrict__ x, int64_t x_stride, int64_t nb, int64_t wid,
                           uint8_t *__restrict__ y, int64_t y_stride, int64_t n_mat, int lane) {
    const int64_t row = wid / nb, b = wid - row * nb;
    float xs[4];
    __builtin_memcpy(xs, x + row * x_stride + b * QK_K + lane * 4, 16);
    int q[4];
    float d;
    q8K_block(xs, lane, row < n_mat, q, d);
    uint8_t *blk = y + row * y_stride + b * Q8K_BYTES;
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    __builtin_memcpy(blk + 4 + lane * 4, &packed, 4);
    const int s = q8K_bsum16(q, lane);
    if ((lane & 3) == 0) {
        const int16_t s16 = (int16_t)s;
        __builtin_memcpy(blk + 260 + 2 * (lane >> 2), &s16, 2);
    }
    if (lane == 0) __builtin_memcpy(blk, &d, 4);
}

extern "C" __global__ void __launch_bounds__(256)
ghip_quantize_q8_K(const float *__restrict__ x, int64_t x_stride, int64_t n, int64_t nrows,
                   uint8_t *__restrict__ y, int64_t y_stride, int64_t n_mat) {
    const int64_t nb = n / QK_K;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= nrows * nb) return;
    quantize_q8K_wave(x, x_stride, nb, wid, y, y_stride, n_mat, threadIdx.x & 63);
}

// Several activation matrices in one launch (ghip_graph_compute quantizes the
// independent inputs of its whole-K decode groups together): segment i takes
// wavefronts [w0[i], w0[i+1]).  Host mirror in ghip.cpp.
struct Q8KSegs {
    const float *x[8];
    int64_t x_stride[8];
    uint8_t *y[8];
    int64_t y_stride[8];
    int64_t nb[8];
    int64_t n_mat[8];
    int64_t w0[9];
    int n;
};

extern "C" __global__ void __launch_bounds__(256) ghip_quantize_q8_K_segs(Q8KSegs g) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= g.w0[g.n]) return;
    int i = 0;
    while (i + 1 < g.n && wid >= g.w0[i + 1]) i++;
    quantize_q8K_wave(g.x[i], g.x_stride[i], g.nb[i], wid - g.w0[i], g.y[i], g.y_stride[i], g.n_mat[i],
                      threadIdx.x & 63);
}

// quantize_row_q8_0 (runtime AVX2 arithmetic, quants.rs:331-362): 8 lanes per
// 32-element block, 8 blocks per wavefront.
extern "C" __global__ void __launch_bounds__(256)
ghip_quantize_q8_0(const float *__restrict__ x, int64_t x_stride, int64_t n, int64_t nrows,
                   uint8_t *__restrict__ y, int64_t y_stride) {
    const int lane = threadIdx.x & 63;
    const int64_t nb = n / 32;
    const int64_t blk_id = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const int sub = lane & 7;
    if (blk_id >= nrows * nb) return;  // whole 8-lane groups exit together
    const int64_t row = blk_id / nb, b = blk_id - row * nb;
    float xs[4];
    __builtin_memcpy(xs, x + row * x_stride + b * 32 + sub * 4, 16);
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
    uint8_t *blk = y + row * y_stride + b * Q8_0_BYTES;
    __builtin_memcpy(blk + 2 + sub * 4, &packed, 4);
    if (sub == 0) {
        const unsigned short dh = f2h_rn(d);
        __builtin_memcpy(blk, &dh, 2);
    }
}

// f32 rows -> Q8_1 blocks (36 B: f16 d, f16 s, int8 qs[32]), quantize_row_q8_1
// (quants.rs:375-397): d = amax / 127, id = 1 / d (0 if d == 0),
// q = round-half-even(x * id) saturated to int8 with NaN -> 0 (a Rust `as i8`),
// s = f16(sum(q) * d).  8 lanes per block, 4 elements each.
extern "C" __global__ void __launch_bounds__(256)
ghip_quantize_q8_1(const float *__restrict__ x, int64_t x_stride, int64_t n, int64_t nrows,
                   uint8_t *__restrict__ y, int64_t y_stride) {
    const int lane = threadIdx.x & 63;
    const int64_t nb = n / 32;
    const int64_t blk_id = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const int sub = lane & 7;
    if (blk_id >= nrows * nb) return;  // whole 8-lane groups exit together
    const int64_t row = blk_id / nb, b = blk_id - row * nb;
    float xs[4];
    __builtin_memcpy(xs, x + row * x_stride + b * 32 + sub * 4, 16);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(xs[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t packed = 0;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float r = rintf(__fmul_rn(xs[i], id));
        const int v = r != r ? 0 : r >= 127.0f ? 127 : r <= -128.0f ? -128 : (int)r;
        sum += v;
        packed |= (uint32_t)(v & 0xff) << (8 * i);
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    uint8_t *blk = y + row * y_stride + b * 36;
    __builtin_memcpy(blk + 4 + sub * 4, &packed, 4);
    if (sub == 0) {
        const uint32_t ds = (uint32_t)f2h_rn(d) | ((uint32_t)f2h_rn(__fmul_rn((float)sum, d)) << 16);
        __builtin_memcpy(blk, &ds, 4);
    }
}
