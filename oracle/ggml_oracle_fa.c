/* ggml_oracle_fa.c -- TEST INFRASTRUCTURE ONLY: FLASH_ATTN_EXT restatement. */
#include "ggml_oracle.h"
int oracle_flash_attn_ext(const float *q, int64_t q_nb1, int64_t q_nb2,
                          const uint16_t *k, const uint16_t *v, int64_t kv_nb1, int64_t kv_nb2,
                          const uint16_t *mask, int64_t mask_nb1,
                          float *dst, int D, int n_q, int H, int S, int H_kv,
                          float scale, float max_bias, float softcap,
                          int n_chunks, int nthreads) {
    (void)q; (void)q_nb1; (void)q_nb2; (void)k; (void)v; (void)kv_nb1; (void)kv_nb2;
    (void)mask; (void)mask_nb1; (void)dst; (void)D; (void)n_q; (void)H; (void)S; (void)H_kv;
    (void)scale; (void)max_bias; (void)softcap; (void)n_chunks; (void)nthreads;
    return -1;
}
