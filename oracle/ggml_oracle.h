/*
 * ggml_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of llama.rust's CPU arithmetic for the quantized
 * MUL_MAT / MUL_MAT_ID / FLASH_ATTN_EXT path (the crates/ggml/src Rust files of
 * fly88oj/llama.rust).  It is the checker the HIP kernels are compared with and
 * the timed CPU baseline of bench.py.  Nothing in the product library links,
 * loads or calls it; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg do.
 *
 * Every function cites the reference file:line it restates.  Parity status of
 * each function (what pins it) is listed beside its declaration.
 */
#ifndef GGML_ORACLE_H
#define GGML_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (crates/ggml/src/types.rs:15) */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_BF16 = 30, OR_IQ2_XXS = 16, OR_IQ2_XS = 17, OR_IQ3_XXS = 18, OR_IQ1_S = 19,
    OR_IQ3_S = 21, OR_IQ2_S = 22, OR_IQ1_M = 29, OR_Q4_0 = 2, OR_Q4_1 = 3, OR_Q5_0 = 6, OR_Q5_1 = 7, OR_Q8_0 = 8, OR_Q8_1 = 9,
    OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12,
    OR_Q5_K = 13, OR_Q6_K = 14, OR_Q8_K = 15, OR_IQ4_NL = 20, OR_IQ4_XS = 23, OR_MXFP4 = 39, OR_NVFP4 = 40,
    OR_Q1_0 = 41, OR_Q2_0 = 42
};

/* ---- scalar helpers ---- */
uint16_t oracle_fp32_to_fp16(float f);
uint16_t oracle_fp32_to_bf16(float f);            /* half 2.7.1 bf16::from_f32: RNE, NaN kept quiet */
float oracle_bf16_to_fp32(uint16_t h);            /* half 2.7.1 from_f32 (RNE); pinned by every fp16 d in quants_ref.bin */
float    oracle_fp16_to_fp32(uint16_t h);
int32_t  oracle_nearest_int(float f);             /* quants.rs:13 */
float    oracle_e8m0_to_fp32_half(uint8_t e);     /* quants.rs:682; pinned by closed form 2^(e-128) */
float    oracle_ue4m3_to_fp32(uint8_t x);         /* quants.rs:699; pinned by the closed form over all 256 bytes and quants_ref_fp4.bin NVFP4 dequant */

/* ---- weight quantizers (one-time prep) ---- */
void oracle_quantize_row_q4_0_ref(const float *x, void *y, int64_t k);  /* quants.rs:124; quants_ref.bin */
void oracle_quantize_row_q4_K_ref(const float *x, void *y, int64_t k);  /* quants_k.rs:1861; quants_ref.bin */
void oracle_quantize_row_q6_K_ref(const float *x, void *y, int64_t k);  /* quants_k.rs:2058; quants_ref.bin */
void oracle_quantize_row_q5_0_ref(const float *x, void *y, int64_t k);  /* quants.rs:207; quants_ref.bin */
void oracle_quantize_row_q4_1_ref(const float *x, void *y, int64_t k);  /* quants.rs:169; quants_ref.bin type 3 */
void oracle_quantize_row_q5_1_ref(const float *x, void *y, int64_t k);  /* quants.rs:260; quants_ref.bin type 7 */
void oracle_quantize_row_q8_1(const float *x, void *y, int64_t k);      /* quants.rs:375; quants_ref.bin type 9 */
void oracle_quantize_row_q5_K_ref(const float *x, void *y, int64_t k);  /* quants_k.rs:1952; quants_ref.bin */
void oracle_quantize_row_mxfp4_ref(const float *x, void *y, int64_t k); /* absent in the reference; quants_ref_fp4.bin */
void oracle_quantize_row_q8_0_ref(const float *x, void *y, int64_t k);  /* quants.rs:302; quants_ref.bin */
void oracle_quantize_row_q1_0_ref(const float *x, void *y, int64_t k);  /* quants.rs:44; quants_ref_q1q2.bin type 41 */
void oracle_quantize_row_q2_0_ref(const float *x, void *y, int64_t k);  /* quants.rs:82; quants_ref_q1q2.bin type 42 */

/* ---- activation quantizers ---- */
void oracle_quantize_row_q8_0(const float *x, void *y, int64_t k);      /* quants.rs:331; q4_0_repack_ref.bin */
void oracle_quantize_row_q8_K_ref(const float *x, void *y, int64_t k);  /* quants.rs:615; quants_ref.bin, q4k_repack_ref.bin */
/* quantize_mat_q8_K_4x8 values (repack.rs:1561), written as plain block_q8_K rows */
void oracle_quantize_row_q8_K_mat(const float *x, void *y, int64_t k);  /* q4k_repack_ref.bin (values) */

/* ---- dequantizers ---- */
void oracle_dequantize_row(int type, const void *x, float *y, int64_t k);

/* ---- dot kernels in the reference's own fp32 order ---- */
float oracle_vec_dot_q4_0_q8_0(int n, const void *x, const void *y);  /* vec_dot.rs:599 */
float oracle_vec_dot_q4_K_q8_K(int n, const void *x, const void *y);  /* vec_dot.rs:872 */
float oracle_vec_dot_q6_K_q8_K(int n, const void *x, const void *y);  /* vec_dot.rs:990 */
float oracle_vec_dot_q5_0_q8_0(int n, const void *x, const void *y);  /* vec_dot.rs:661; mulmat_ref*.bin type 6 */
float oracle_vec_dot_q4_1_q8_1(int n, const void *x, const void *y);  /* vec_dot.rs:620; parity unpinned by a fixture: brute force */
float oracle_vec_dot_q5_1_q8_1(int n, const void *x, const void *y);  /* vec_dot.rs:687; parity unpinned by a fixture: brute force */
float oracle_vec_dot_q2_K_q8_K(int n, const void *x, const void *y);  /* vec_dot.rs:758; no fixture holds the dot: brute force */
float oracle_vec_dot_q3_K_q8_K(int n, const void *x, const void *y);  /* vec_dot.rs:801; no fixture holds the dot: brute force */
float oracle_vec_dot_q8_0_q8_0(int n, const void *x, const void *y);  /* vec_dot.rs:732; mulmat_ref*.bin type 8 */
float oracle_vec_dot_q5_K_q8_K(int n, const void *x, const void *y);  /* vec_dot.rs:928; mulmat_ref*.bin type 13 */
float oracle_vec_dot_iq4_nl_q8_0(int n, const void *x, const void *y); /* vec_dot.rs:1597; vecdot3_ref.bin type 20 */
float oracle_vec_dot_iq4_xs_q8_K(int n, const void *x, const void *y); /* vec_dot.rs:1655; vecdot3_ref.bin type 23 */
float oracle_vec_dot_nvfp4_q8_0(int n, const void *x, const void *y);  /* vec_dot.rs:1154; vecdot3_ref.bin type 40 */
float oracle_vec_dot_q1_0_q8_0(int n, const void *x, const void *y);   /* vec_dot.rs:1074; vecdot3_ref.bin type 41 */
float oracle_vec_dot_q2_0_q8_0(int n, const void *x, const void *y);   /* vec_dot.rs:1120; vecdot3_ref.bin type 42 */

/*
 * The reference's MUL_MAT routing for a 2-D quantized weight W [rows x n]
 * (row-major GGUF blocks) and f32 activations X [cols x n]
 * (compute.rs:1420-1839):
 *   Q4_0, rows%8==0 -> 8x8 repack gemv/gemm, Q8_0 activations  (compute.rs:5192)
 *   Q4_K, rows%8==0 -> 8x8 repack: 4-row groups quantized by quantize_mat_q8_K_4x8
 *                      and run through the gemm, the cols%4 tail by
 *                      quantize_row_q8_K_ref through the gemv   (compute.rs:5322)
 *   K-quant, not repacked, cols>=8 -> tiled                     (tiled.rs:1656)
 *   otherwise row vec_dot with quantize_row_q8_K_ref / quantize_row_q8_0
 * Q4_0 with rows%8!=0 and cols>=2 would take tinyBLAS, which is out of scope:
 * returns -1 there.  Q5_0 / Q8_0 always take the row vec_dot, whose values
 * tinyBLAS_Q0 reproduces for cols>=2 (tinyblas.rs:55-75); Q5_K (no x86
 * repack) takes tiled for cols>=8, else vec_dot.
 * out is [cols x rows] f32.  subsums (optional) receives the exact integer
 * partials per (col, row, block) -- see ghip.h ghip_mul_mat_subsums for the
 * layout.  route (optional) receives the route id (see ORACLE_ROUTE_*).
 * nthreads<=0 uses every OpenMP thread.
 */
enum { ORACLE_ROUTE_REPACK = 1, ORACLE_ROUTE_TILED = 2, ORACLE_ROUTE_VECDOT = 3 };
int oracle_mul_mat(int type, const void *w, int64_t n, int64_t rows,
                   const float *x, int64_t cols, float *out,
                   int32_t *subsums, int *route, int nthreads);

/* the activation bytes the route above feeds the kernels with (plain rows of
 * block_q8_0 / block_q8_K) */
int oracle_mul_mat_act(int type, int64_t n, int64_t rows, const float *x,
                       int64_t cols, void *act);

/*
 * MUL_MAT_ID with MXFP4 experts (compute.rs:1917-2202): as [n_as][rows][n],
 * b [n_tokens][ne11][n] f32, ids [n_tokens][n_ids] i32, dst
 * [n_tokens][n_ids][rows].  Activations quantize_row_q8_0; per 8-row group the
 * repack gemv_mxfp4_8x8_q8_0 (repack.rs:1086) when rows%8==0, else
 * vec_dot_mxfp4_q8_0 (compute.rs:7123).
 */
int oracle_mul_mat_id_mxfp4(const void *as, int64_t n, int64_t rows, int64_t n_as,
                            const float *b, int64_t ne11, int64_t n_tokens,
                            const int32_t *ids, int64_t n_ids, float *dst,
                            int nthreads);

/*
 * FLASH_ATTN_EXT (compute.rs:4563-4625, flash_attn.rs), dense tensors:
 *   q    element (d, t, h) at q[h*q_nb2 + t*q_nb1 + d]       (f32; strides in floats)
 *   k, v element (d, s, h) at k[h*k_nb2 + s*k_nb1 + d]       (f16 or f32; strides in elements)
 *   mask element (s, t)    at mask[t*mask_nb1 + s]           (f16, may be NULL)
 *   sinks[h] (may be NULL), dst element (d, h, t) at dst[(t*H + h)*DV + d]
 * n_chunks: the split-KV chunk count of the single-row decode path (the
 * reference uses its thread count).  Returns the path taken: 1 split-KV,
 * 2 tiled, 3 one_chunk; < 0 on bad shapes.
 */
typedef struct oracle_fa_args {
    const float *q;
    int64_t q_nb1, q_nb2;
    const void *k, *v;
    int64_t k_nb1, k_nb2, v_nb1, v_nb2;
    int kv_f16;
    const uint16_t *mask;
    int64_t mask_nb1;
    const float *sinks;
    float *dst;
    int DK, DV, T, H, S, H_kv;
    float scale, max_bias, softcap;
    int n_chunks, nthreads;
} oracle_fa_args;
int oracle_flash_attn_ext(const oracle_fa_args *a);

double oracle_wtime(void);

#ifdef __cplusplus
}
#endif

/* MUL_MAT with F32 / F16 / BF16 weights (compute.rs:1700-1745; vec_dot.rs:1700-1727):
 * F16 / BF16: the f32 activations rounded to the weight type (RNE) and the
 * exact products summed in double, rounded once (ggml_vec_dot_f16 / _bf16 scalar
 * twins); F32: x * y rounded to f32, summed in double (ggml_vec_dot_f32 scalar).
 * w: rows x n weights, x: cols x n, out: cols x rows.  Returns 0, or -1 for another type. */
int oracle_mul_mat_dense(int type, const void *w, int64_t n, int64_t rows, const float *x, int64_t cols, float *out,
                         int nthreads);

/* IQ1 / IQ2 / IQ3 (vec_dot.rs:1215-1590): block bytes (0 for other types) and the row dot */
int oracle_iq_block_bytes(int type);
float oracle_vec_dot_iq(int type, int n, const void *vx, const void *vy);

#endif
