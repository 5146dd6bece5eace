/* oracle.h -- TEST INFRASTRUCTURE ONLY: CPU restatement of miniTensor's fp32
 * GEMM reference path (see oracle.c for the per-function reference citations). */
#ifndef MT_ORACLE_H
#define MT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ora_mt19937 {
    uint32_t s[624];
    int i;
} ora_mt19937;

void ora_mt19937_seed(ora_mt19937* g, uint32_t seed);
uint32_t ora_mt19937_next(ora_mt19937* g);
void ora_fill_uniform(float* out, size_t n, uint32_t seed, float lo, float hi);
void ora_fill_normal(float* out, size_t n, uint32_t seed, float mean, float std);

void ora_matmul(const float* a, const float* b, float* c, size_t M, size_t K, size_t N);
void ora_matmul_strided(const float* a, size_t a_sm, size_t a_sk, const float* b, size_t b_sk,
                        size_t b_sn, float* c, size_t c_sm, size_t c_sn, size_t M, size_t K,
                        size_t N);
void ora_bmm(const float* a, const float* b, float* c, size_t batch, size_t M, size_t K, size_t N);
void ora_conv2d(const float* in, const float* w, const float* bias, float* out, size_t N,
                size_t C_in, size_t H, size_t W, size_t C_out, size_t kH, size_t kW,
                size_t stride, size_t pad);
void ora_conv2d_bwd_input(const float* go, const float* w, float* gi, size_t N, size_t C_in,
                          size_t H, size_t W, size_t C_out, size_t kH, size_t kW, size_t stride,
                          size_t pad);
void ora_conv2d_bwd_weight(const float* go, const float* in, float* gw, size_t N, size_t C_in,
                           size_t H, size_t W, size_t C_out, size_t kH, size_t kW, size_t stride,
                           size_t pad);
void ora_conv2d_bwd_bias(const float* go, float* gb, size_t N, size_t C_out, size_t Ho, size_t Wo);
void ora_colsum(const float* x, size_t rs, size_t cs, size_t R, size_t Cn, float* out);
void ora_matmul_f64_rows(const float* a, size_t a_sm, size_t a_sk, const float* b, size_t b_sk,
                         size_t b_sn, const int64_t* rows, size_t n_rows, size_t K, size_t N,
                         double* out);

#ifdef __cplusplus
}
#endif

#endif
